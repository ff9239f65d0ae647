"""ctypes layouts and signatures of include/rxmet_lstm.h (the QuantLSTM C ABI)."""
from __future__ import annotations

import ctypes

import numpy as np

import rxmet_lib as _rx

OP_NAMES = ("input", "output", "cell_state", "weight_ih", "weight_hh", "bias_ih", "bias_hh",
            "weight_ih_linear", "weight_hh_linear", "input_gate_input", "forget_gate_input",
            "cell_gate_input", "output_gate_input", "input_gate_output", "forget_gate_output",
            "cell_gate_output", "output_gate_output", "cell_tanh_output")
OP = {n: i for i, n in enumerate(OP_NAMES)}
NOPS = 18
PARAM_OPS = ("weight_ih", "weight_hh", "bias_ih", "bias_hh")
SIGMOID_OUTPUTS = ("input_gate_output", "forget_gate_output", "output_gate_output")
PER_TENSOR, PER_GATE, PER_CHANNEL = 0, 1, 2
GRANULARITY = {"per_tensor": PER_TENSOR, "per_gate": PER_GATE, "per_channel": PER_CHANNEL}
AFFINE, POT2 = 0, 1


class OpConfig(ctypes.Structure):
    _fields_ = [("bits", ctypes.c_int32), ("is_unsigned", ctypes.c_int32),
                ("is_symmetric", ctypes.c_int32), ("granularity", ctypes.c_int32)]


class Config(ctypes.Structure):
    _fields_ = [("scale_mode", ctypes.c_int32), ("op", OpConfig * NOPS)]


class Params(ctypes.Structure):
    _fields_ = [("hidden", ctypes.c_int32), ("bias_enabled", ctypes.c_int32), ("config", Config),
                ("scale", ctypes.c_float * NOPS), ("zero_point", ctypes.c_int32 * NOPS),
                ("chan_scale", ctypes.POINTER(ctypes.c_float) * 4)]


class Rescale(ctypes.Structure):
    _fields_ = [("is_mshift", ctypes.c_int32), ("multiplier", ctypes.c_int32),
                ("shift", ctypes.c_int32)]


class Q31(ctypes.Structure):
    _fields_ = [("multiplier", ctypes.c_int64), ("mantissa", ctypes.c_double),
                ("exponent", ctypes.c_int32), ("uses_fp", ctypes.c_int32)]


_SAVED_F = ("x_q", "w_ih_q", "w_hh_q", "b_ih_q", "b_hh_q", "h0_q", "c0_q")
_SAVED_M = ("x_m", "w_ih_m", "w_hh_m", "b_ih_m", "b_hh_m", "h0_m", "c0_m")
_CKPT_F = ("gate_out", "cell", "cell_tanh", "hidden")
_CKPT_M = ("ih_linear_m", "hh_linear_m", "gate_in_m", "gate_out_m", "cell_m", "cell_tanh_m",
           "hidden_m")
SAVED_FIELDS = _SAVED_F + _SAVED_M + _CKPT_F + _CKPT_M


class Saved(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in SAVED_FIELDS]


class SavedCodes(ctypes.Structure):
    """rxmet_lstm_saved_codes: the saved-codes blocks and the cell codes."""
    _fields_ = [("blocks", ctypes.c_void_p), ("cell_codes", ctypes.c_void_p)]


# bytes of one saved-codes block and u16 codes of one cell-code block (rxmet_lstm_saved_codes)
CODES_BLOCK = 3840
CELL_BLOCK = 256


def default_config() -> Config:
    """The reference's default profile (config/defaults/lstm_quant_default_v1.json): all
    8-bit, affine, sigmoid gate outputs unsigned, everything symmetric, parameters
    per-channel."""
    c = Config()
    c.scale_mode = AFFINE
    for i, n in enumerate(OP_NAMES):
        c.op[i] = OpConfig(8, 1 if n in SIGMOID_OUTPUTS else 0, 1,
                           PER_CHANNEL if n in PARAM_OPS else PER_TENSOR)
    return c


def stats_size(hidden: int) -> int:
    return 2 * NOPS + 8 * 4 * hidden + 1


def empty_stats(hidden: int) -> np.ndarray:
    s = np.empty(stats_size(hidden), np.float32)
    s[:NOPS] = np.inf
    s[NOPS:2 * NOPS] = -np.inf
    C = 4 * hidden
    for k in range(4):
        base = 2 * NOPS + k * 2 * C
        s[base:base + C] = np.inf
        s[base + C:base + 2 * C] = -np.inf
    s[-1] = 0.0
    return s


def new_params(hidden: int) -> Params:
    """Params whose chan_scale points at owned numpy buffers (kept on the object)."""
    p = Params()
    p.hidden = hidden
    bufs = [np.zeros(4 * hidden, np.float32) for _ in range(4)]
    for k in range(4):
        p.chan_scale[k] = bufs[k].ctypes.data_as(ctypes.POINTER(ctypes.c_float))
    p._bufs = bufs  # noqa: SLF001 (keep the arrays alive with the struct)
    return p


def chan_scales(p: Params, k: int) -> np.ndarray:
    return np.ctypeslib.as_array(p.chan_scale[k], shape=(4 * p.hidden,))


_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_SIGS = {
    "rxmet_lstm_stats_size": (ctypes.c_int64, [_i32]),
    "rxmet_lstm_finalize_params": (ctypes.c_int, [_p, ctypes.POINTER(Config), _i32, _i32,
                                                  ctypes.POINTER(Params)]),
    "rxmet_lstm_derive_exec": (ctypes.c_int, [ctypes.POINTER(Params), _i32, _p, _p, _p, _p, _p]),
    "rxmet_lstm_forward_workspace_bytes": (ctypes.c_int64, [_i32] * 4),
    "rxmet_lstm_backward_workspace_bytes": (ctypes.c_int64, [_i32] * 4),
    "rxmet_lstm_calibrate_workspace_bytes": (ctypes.c_int64, [_i32] * 4),
    "rxmet_lstm_forward_quant": (ctypes.c_int, [_i32] * 4 + [_p] * 7 + [ctypes.POINTER(Params)] +
                                 [_p] * 3 + [ctypes.POINTER(Saved), _p, _p]),
    "rxmet_lstm_backward_quant": (ctypes.c_int, [_i32] * 4 + [ctypes.POINTER(Params),
                                                              ctypes.POINTER(Saved)] +
                                  [_p] * 3 + [_p] * 7 + [_p, _p]),
    "rxmet_lstm_forward_quant_codes": (ctypes.c_int, [_i32] * 4 + [_p] * 7 + [ctypes.POINTER(Params)] +
                                       [_p] * 3 + [ctypes.POINTER(Saved), ctypes.POINTER(SavedCodes),
                                                   _p, _p]),
    "rxmet_lstm_backward_quant_codes": (ctypes.c_int, [_i32] * 4 + [ctypes.POINTER(Params),
                                                                    ctypes.POINTER(Saved),
                                                                    ctypes.POINTER(SavedCodes)] +
                                        [_p] * 3 + [_p] * 7 + [_p, _p]),
    "rxmet_lstm_forward_calibrate": (ctypes.c_int, [_i32] * 4 + [_p] * 7 + [_p] * 4 + [_p, _p]),
    "rxmet_lstm_forward_float": (ctypes.c_int, [_i32] * 4 + [_p] * 7 + [_p] * 3 + [_p]),
    "rxmet_lstm_activation_table": (_i32, [ctypes.POINTER(Params), _i32, _i32, _p, _i32]),
    "rxmet_lstm_activation_exceptions": (_i32, [ctypes.POINTER(Params), _p, _p, _i32, _p, _p]),
}
for _name, (_res, _args) in _SIGS.items():
    _rx.register(_name, _res, _args)
