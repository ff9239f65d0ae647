"""ctypes mirror of the structs in ``include/rxmet_gru.h`` and the GRU signatures."""
from __future__ import annotations

import ctypes

import rxmet_lib as _rx

NGRIDS = 13
NCHAN = 4

# scalar grids (order of the RXMET_GRU_* enum)
GRID_NAMES = ("x", "h", "weight_ih_linear", "weight_hh_linear", "update_gate_input",
              "reset_gate_input", "new_gate_input", "update_gate_output", "reset_gate_output",
              "new_gate_output", "mul_reset_hidden", "mul_new_contribution",
              "mul_old_contribution")
GRID = {n: i for i, n in enumerate(GRID_NAMES)}
# per-channel operators (W, R, bw, br)
CHAN_NAMES = ("W", "R", "bw", "br")
CHAN = {n: i for i, n in enumerate(CHAN_NAMES)}

PER_TENSOR, PER_GATE, PER_CHANNEL = 0, 1, 2
POT_ROUND, POT_COVER_RANGE, POT_FLOOR = 0, 1, 2


class BitSpec(ctypes.Structure):
    _fields_ = [("bits", ctypes.c_int32), ("is_unsigned", ctypes.c_int32),
                ("symmetric", ctypes.c_int32), ("granularity", ctypes.c_int32)]


class GruConfig(ctypes.Structure):
    _fields_ = [("op", BitSpec * NGRIDS), ("chan", BitSpec * NCHAN),
                ("use_pot2", ctypes.c_int32), ("pot_method", ctypes.c_int32),
                ("pot_tolerance", ctypes.c_float)]


class GruRanges(ctypes.Structure):
    _fields_ = [("hidden", ctypes.c_int32), ("min", ctypes.c_float * NGRIDS),
                ("max", ctypes.c_float * NGRIDS),
                ("chan_min", ctypes.POINTER(ctypes.c_float) * NCHAN),
                ("chan_max", ctypes.POINTER(ctypes.c_float) * NCHAN)]


class Grid(ctypes.Structure):
    _fields_ = [("scale", ctypes.c_float), ("zero_point", ctypes.c_int32),
                ("bits", ctypes.c_int32), ("is_unsigned", ctypes.c_int32)]


class GruQParams(ctypes.Structure):
    _fields_ = [("hidden", ctypes.c_int32), ("use_pot2", ctypes.c_int32), ("g", Grid * NGRIDS),
                ("chan_bits", ctypes.c_int32 * NCHAN), ("chan_unsigned", ctypes.c_int32 * NCHAN),
                ("chan_scale", ctypes.POINTER(ctypes.c_float) * NCHAN)]


class PwlSegment(ctypes.Structure):
    _fields_ = [("q_b", ctypes.c_int32), ("n", ctypes.c_int32), ("c", ctypes.c_int32),
                ("threshold", ctypes.c_int32)]


class PwlLut(ctypes.Structure):
    _fields_ = [("seg", PwlSegment * 16), ("zp_x", ctypes.c_int32)]


_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64

FWD_DIR_FIELDS = ("W", "R", "bw", "br", "x", "h0", "params", "h", "v", "W_q", "R_q", "bw_q",
                  "br_q", "x_q", "x_mask", "h0_mask", "W_mask", "R_mask", "bw_mask", "br_mask",
                  "ih_mask", "hh_mask", "gate_in_mask", "gate_out_mask", "h_mask", "workspace")
BWD_DIR_FIELDS = ("W_q", "R_q", "bw_q", "br_q", "x_q", "dh_new", "h", "v", "params", "x_mask",
                  "h0_mask", "W_mask", "R_mask", "bw_mask", "br_mask", "ih_mask", "hh_mask",
                  "gate_in_mask", "gate_out_mask", "h_mask", "dx", "dW", "dR", "dbw", "dbr", "dh0",
                  "workspace")


class FwdDir(ctypes.Structure):
    """rxmet_gru_fwd_dir: the arguments of one rxmet_gru_forward_quant call."""
    _fields_ = [(n, _p) for n in FWD_DIR_FIELDS]


INT_DIR_FIELDS = ("W", "R", "bw", "br", "x", "h0", "x_q_in", "h0_q_in", "params", "h", "v", "h_q",
                  "W_q", "R_q", "bw_q", "br_q", "x_q", "x_mask", "h0_mask", "W_mask", "R_mask",
                  "bw_mask", "br_mask", "ih_mask", "hh_mask", "gate_in_mask", "gate_out_mask",
                  "h_mask", "workspace")


class IntDir(ctypes.Structure):
    """rxmet_gru_int_dir: the arguments of one rxmet_gru_forward_quant_int (or int-IO) call."""
    _fields_ = [(n, _p) for n in INT_DIR_FIELDS]


class BwdDir(ctypes.Structure):
    """rxmet_gru_bwd_dir: the arguments of one rxmet_gru_backward_quant call."""
    _fields_ = [(n, _p) for n in BWD_DIR_FIELDS]


class SavedCodes(ctypes.Structure):
    """rxmet_gru_saved_codes: one direction's v codes [T, B, 4H] and mask bits [T, B, H]."""
    _fields_ = [("v_codes", _p), ("mask_bits", _p)]


class GradView(ctypes.Structure):
    """rxmet_gru_grad_view: a direction's dh read in place from the layer's output gradient."""
    _fields_ = [("g", _p), ("st", ctypes.c_int64), ("sb", ctypes.c_int64), ("sk", ctypes.c_int64),
                ("col0", ctypes.c_int32), ("reverse", ctypes.c_int32), ("g_hn", _p)]


_SIGS = {
    "rxmet_gru_make_params": (ctypes.c_int, [ctypes.POINTER(GruRanges), ctypes.POINTER(GruConfig),
                                             ctypes.POINTER(GruQParams)]),
    "rxmet_gru_make_luts": (ctypes.c_int, [ctypes.POINTER(GruQParams), ctypes.POINTER(PwlLut)]),
    "rxmet_gru_effective_scale": (ctypes.c_float, [ctypes.c_float, _i32]),
    "rxmet_gru_forward_workspace_bytes": (ctypes.c_int64, [_i32, _i32, _i32, _i32]),
    "rxmet_gru_backward_workspace_bytes": (ctypes.c_int64, [_i32, _i32, _i32, _i32]),
    "rxmet_gru_calibrate_workspace_bytes": (ctypes.c_int64, [_i32, _i32, _i32, _i32]),
    "rxmet_gru_forward_quant": (ctypes.c_int, [_i32, _i32, _i32, _i32, _i32] + [_p] * 6 +
                                [ctypes.POINTER(GruQParams)] + [_p] * 18 + [_p, _p]),
    "rxmet_gru_backward_quant": (ctypes.c_int, [_i32, _i32, _i32, _i32] + [_p] * 8 +
                                 [ctypes.POINTER(GruQParams)] + [_p] * 11 + [_p] * 6 + [_p, _p]),
    "rxmet_gru_forward_quant_dirs": (ctypes.c_int, [_i32] * 6 + [ctypes.POINTER(FwdDir), _p]),
    "rxmet_gru_backward_quant_dirs": (ctypes.c_int, [_i32] * 5 + [ctypes.POINTER(BwdDir), _p]),
    "rxmet_gru_forward_calibrate": (ctypes.c_int, [_i32, _i32, _i32, _i32] + [_p] * 9 + [_p, _p]),
    "rxmet_gru_forward_fp": (ctypes.c_int, [_i32] * 5 + [_p] * 8 + [_p]),
    "rxmet_gru_forward_quant_dirs_x": (ctypes.c_int, [_i32] * 6 + [ctypes.POINTER(FwdDir), _p, _p]),
    "rxmet_gru_backward_quant_dirs_x": (ctypes.c_int, [_i32] * 5 + [ctypes.POINTER(BwdDir), _i32, _p]),
    "rxmet_gru_bidir_assemble": (ctypes.c_int, [_i32] * 3 + [_p] * 3 + [_i64, _i64, _p, _p]),
    "rxmet_gru_bidir_split_grad": (ctypes.c_int, [_i32] * 3 + [_p, _i64, _i64, _i64] + [_p] * 4),
    "rxmet_gru_bidir_dx": (ctypes.c_int, [_i32] * 3 + [_p] * 3 + [_i64, _i64, _p]),
    "rxmet_gru_forward_int_workspace_bytes": (ctypes.c_int64, [_i32, _i32, _i32, _i32]),
    "rxmet_gru_forward_quant_int": (ctypes.c_int, [_i32, _i32, _i32, _i32, _i32] + [_p] * 6 +
                                    [ctypes.POINTER(GruQParams)] + [_p] * 18 + [_p, _p]),
    "rxmet_gru_forward_int_io": (ctypes.c_int, [_i32] * 4 + [_p] * 6 +
                                 [ctypes.POINTER(GruQParams)] + [_p] * 5 + [_p, _p]),
    "rxmet_gru_forward_quant_int_dirs": (ctypes.c_int, [_i32] * 6 + [ctypes.POINTER(IntDir), _p]),
    "rxmet_gru_forward_quant_dirs_codes": (ctypes.c_int, [_i32] * 6 + [ctypes.POINTER(FwdDir), _p,
                                                                     ctypes.POINTER(SavedCodes), _p]),
    "rxmet_gru_backward_quant_dirs_codes": (ctypes.c_int, [_i32] * 5 + [ctypes.POINTER(BwdDir), _i32,
                                                                      ctypes.POINTER(SavedCodes),
                                                                      ctypes.POINTER(GradView), _p]),
}
for _name, (_res, _args) in _SIGS.items():
    _rx.register(_name, _res, _args)


def fptr(arr):
    """ctypes float* of a contiguous float32 numpy array."""
    return arr.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


# ---------------------------------------------------------------------------------
# OperatorQuantConfig defaults and set_all_bitwidth (quantize_bitwidth_config.h:56-122,
# pytorch/quant_gru.py:1628-1660)
# ---------------------------------------------------------------------------------

_UNSIGNED_DEFAULT = {"update_gate_output", "reset_gate_output"}


def default_config() -> GruConfig:
    """All operators 8-bit symmetric, sigmoid outputs unsigned, weights per-channel."""
    cfg = GruConfig()
    for i, name in enumerate(GRID_NAMES):
        cfg.op[i] = BitSpec(8, 1 if name in _UNSIGNED_DEFAULT else 0, 1, PER_CHANNEL)
    for k in range(NCHAN):
        cfg.chan[k] = BitSpec(8, 0, 1, PER_CHANNEL)
    cfg.use_pot2 = 0
    cfg.pot_method = POT_COVER_RANGE
    cfg.pot_tolerance = 0.02
    return cfg


def set_all_bitwidth(cfg: GruConfig, bits: int, is_symmetric: bool = True) -> GruConfig:
    """Every operator to ``bits``; activations symmetric per the flag, weights always
    symmetric; unsigned flags are kept."""
    for i in range(NGRIDS):
        cfg.op[i].bits = bits
        cfg.op[i].symmetric = 1 if is_symmetric else 0
    for k in range(NCHAN):
        cfg.chan[k].bits = bits
        cfg.chan[k].symmetric = 1
    return cfg


def new_qparams(hidden: int):
    """A GruQParams whose per-channel scale arrays are owned numpy buffers."""
    import numpy as np

    qp = GruQParams()
    qp.hidden = hidden
    bufs = [np.zeros(3 * hidden, np.float32) for _ in range(NCHAN)]
    for k in range(NCHAN):
        qp.chan_scale[k] = fptr(bufs[k])
    qp._bufs = bufs  # keep the arrays alive with the struct
    return qp


def qparams_chan(qp, k):
    return qp._bufs[k]


def make_ranges(stats, hidden: int):
    """GruRanges view over a flat statistics vector (layout of rxmet_gru_forward_calibrate)."""
    import numpy as np

    stats = np.ascontiguousarray(stats, dtype=np.float32)
    C = 3 * hidden
    r = GruRanges()
    r.hidden = hidden
    for i in range(NGRIDS):
        r.min[i] = float(stats[i])
        r.max[i] = float(stats[NGRIDS + i])
    chans = []
    for k in range(NCHAN):
        lo = np.ascontiguousarray(stats[2 * NGRIDS + 2 * k * C: 2 * NGRIDS + 2 * k * C + C])
        hi = np.ascontiguousarray(stats[2 * NGRIDS + 2 * k * C + C: 2 * NGRIDS + 2 * (k + 1) * C])
        chans += [lo, hi]
        r.chan_min[k] = fptr(lo)
        r.chan_max[k] = fptr(hi)
    r._bufs = chans
    return r


def stats_size(hidden: int) -> int:
    return 2 * NGRIDS + 8 * 3 * hidden


def empty_stats(hidden: int):
    import numpy as np

    s = np.empty(stats_size(hidden), np.float32)
    s[:NGRIDS] = np.finfo(np.float32).max
    s[NGRIDS:2 * NGRIDS] = np.finfo(np.float32).min
    C = 3 * hidden
    for k in range(NCHAN):
        base = 2 * NGRIDS + 2 * k * C
        s[base:base + C] = np.finfo(np.float32).max
        s[base + C:base + 2 * C] = np.finfo(np.float32).min
    return s
