"""QuantLSTM for MI355X: a drop-in for single-layer ``nn.LSTM`` with MinMax calibration and
FP32 q-carrier quantisation-aware training.

Mirrors the reference module (``operators/quant-lstm/pytorch/quant_lstm.py:397-1418``) and
its autograd bridge (``lstm_autograd.py:139-325``): the same constructor arguments, parameter
names (``weight_ih_l0``, ``..._reverse``), operator configuration (18 quantisation points,
schema 1, ``config/defaults/lstm_quant_default_v1.json`` defaults), calibration workflow
(``calibrating`` -> ``finalize_calibration``), checkpoint-saving rule and the public v1 quant
params document.  Every compute step runs in librxmet.so on the GPU; there is no CPU path.

Not provided: SQNR / percentile calibration, the float-path backward and ONNX export; each
raises NotImplementedError where it would be used.
"""
from __future__ import annotations

import copy
import json
import math
import struct
import warnings
from pathlib import Path
from typing import Any, Optional

import numpy as np
import torch
from torch import Tensor, nn

import lstm_ops
import rxmet_lstm_abi as L

OPERATORS = L.OP_NAMES
PARAMETER_OPERATORS = set(L.PARAM_OPS)
_CALIBRATION_METHODS = {"minmax", "sqnr", "percentile"}
_MATH_MODES = {"pedantic", "tf32"}
_GRANULARITY = {"per_tensor": L.PER_TENSOR, "per_gate": L.PER_GATE, "per_channel": L.PER_CHANNEL}
_GRANULARITY_NAME = {v: k for k, v in _GRANULARITY.items()}
_EXTERNAL_GRANULARITY = {"per_tensor": "PER_TENSOR", "per_gate": "PER_GATE",
                         "per_channel": "PER_CHANNEL"}
_EXTERNAL_FIELDS = {"dtype", "symmetric", "scale", "zero_point", "enc_type", "real_min", "real_max"}


# ------------------------------------------------------------------------------------------
# operator configuration (quant_config_loader.cc: resolveQuantConfig / validate)
# ------------------------------------------------------------------------------------------

def default_quant_config() -> dict:
    """The resolved default profile: every point 8-bit signed symmetric, the three sigmoid gate
    outputs unsigned, parameters per-channel, affine scales."""
    ops = {}
    for name in OPERATORS:
        if name in PARAMETER_OPERATORS:
            ops[name] = {"bitwidth": 8, "granularity": "per_channel"}
        else:
            ops[name] = {"bitwidth": 8, "is_unsigned": name in L.SIGMOID_OUTPUTS,
                         "is_symmetric": True}
    return {"schema_version": 1, "scale_mode": "affine", "operators": ops}


def _strict_json_loads(text: str) -> dict:
    def no_duplicates(pairs):
        out = {}
        for k, v in pairs:
            if k in out:
                raise ValueError(f"JSON has a duplicate key: {k}")
            out[k] = v
        return out

    value = json.loads(text, object_pairs_hook=no_duplicates)
    if not isinstance(value, dict):
        raise ValueError("JSON root must be an object")
    return value


def _load_json_source(source) -> dict:
    if source is None:
        return {"schema_version": 1}
    if isinstance(source, dict):
        return copy.deepcopy(source)
    if isinstance(source, Path):
        return _strict_json_loads(source.read_text(encoding="utf-8"))
    if isinstance(source, str):
        if source.lstrip().startswith("{"):
            return _strict_json_loads(source)
        return _strict_json_loads(Path(source).read_text(encoding="utf-8"))
    raise TypeError("quant config must be a dict, JSON text or a path")


def _check_bits(value) -> int:
    if isinstance(value, bool) or not isinstance(value, int):
        raise ValueError("bitwidth must be an integer")
    if not 1 <= value <= 32:
        raise ValueError("operator bitwidth must be in [1, 32]")
    return value


def _check_bool(value, field) -> bool:
    if not isinstance(value, bool):
        raise ValueError(f"{field} must be a boolean")
    return value


def _validate_resolved(cfg: dict) -> None:
    if cfg["scale_mode"] not in ("affine", "pot2"):
        raise ValueError(f"unknown scale_mode: {cfg['scale_mode']}")
    for name in OPERATORS:
        op = cfg["operators"][name]
        bits = _check_bits(op["bitwidth"])
        if name in PARAMETER_OPERATORS:
            if op["granularity"] not in _GRANULARITY:
                raise ValueError(f"unknown granularity: {op['granularity']}")
            if bits == 1:
                raise ValueError("signed symmetric INT1 has qmax=0 and is unsupported")
        else:
            if op["is_unsigned"] and bits == 32:
                raise ValueError("UINT32 exceeds the int32 quantization metadata range")
            if not op["is_unsigned"] and op["is_symmetric"] and bits == 1:
                raise ValueError("signed symmetric INT1 has qmax=0 and is unsupported")


def resolve_quant_config(override: Optional[dict] = None, defaults: Optional[dict] = None) -> dict:
    """Apply a sparse override ``{"schema_version": 1, "scale_mode"?, "operators"?: {name:
    {field: value}}}`` to the defaults and validate the result (resolveQuantConfig,
    src/lstm/quant_config_loader.cc:330-353)."""
    cfg = copy.deepcopy(defaults if defaults is not None else default_quant_config())
    ov = {"schema_version": 1} if override is None else override
    unknown = set(ov) - {"schema_version", "scale_mode", "operators"}
    if unknown:
        raise ValueError(f"override root unknown field: {sorted(unknown)[0]}")
    sv = ov.get("schema_version")
    if isinstance(sv, bool) or sv != 1:
        raise ValueError("only schema_version=1 is supported")
    if "scale_mode" in ov:
        if not isinstance(ov["scale_mode"], str):
            raise ValueError("scale_mode must be a string")
        cfg["scale_mode"] = ov["scale_mode"]
    for name, fields in (ov.get("operators") or {}).items():
        if name not in cfg["operators"]:
            raise ValueError(f"unknown quant operator: {name}")
        if not isinstance(fields, dict):
            raise ValueError(f"{name} must be an object")
        allowed = ({"bitwidth", "granularity", "comment"} if name in PARAMETER_OPERATORS
                   else {"bitwidth", "is_unsigned", "is_symmetric", "comment"})
        bad = set(fields) - allowed
        if bad:
            raise ValueError(f"{name} unknown field: {sorted(bad)[0]}")
        if set(fields) <= {"comment"}:
            raise ValueError(f"{name} override must set at least one field")
        tgt = cfg["operators"][name]
        for k, v in fields.items():
            if v is None:
                raise ValueError(f"override field cannot be null: {k}")
            if k == "bitwidth":
                tgt[k] = _check_bits(v)
            elif k in ("is_unsigned", "is_symmetric"):
                tgt[k] = _check_bool(v, k)
            elif k == "granularity":
                if v not in _GRANULARITY:
                    raise ValueError(f"unknown granularity: {v}")
                tgt[k] = v
    _validate_resolved(cfg)
    return cfg


def config_struct(cfg: dict) -> L.Config:
    """Resolved config dict -> the C ``rxmet_lstm_config``."""
    c = L.Config()
    c.scale_mode = L.POT2 if cfg["scale_mode"] == "pot2" else L.AFFINE
    for i, name in enumerate(OPERATORS):
        op = cfg["operators"][name]
        if name in PARAMETER_OPERATORS:
            c.op[i] = L.OpConfig(op["bitwidth"], 0, 1, _GRANULARITY[op["granularity"]])
        else:
            c.op[i] = L.OpConfig(op["bitwidth"], int(op["is_unsigned"]), int(op["is_symmetric"]),
                                 L.PER_TENSOR)
    return c


# ------------------------------------------------------------------------------------------
# public v1 quant params document (quant_lstm.py:145-380 of the reference)
# ------------------------------------------------------------------------------------------

def _f32(v: float) -> float:
    try:
        return struct.unpack("!f", struct.pack("!f", float(v)))[0]
    except (OverflowError, struct.error) as e:
        raise ValueError("scale is outside the FP32 range") from e


def _qrange(bits: int, unsigned: bool):
    if unsigned:
        return 0, (1 << bits) - 1
    return -(1 << (bits - 1)), (1 << (bits - 1)) - 1


def _one_or_list(v: list):
    return v[0] if len(v) == 1 else v


def _compact_scales(p: lstm_ops.LstmQuantParams, name: str, gran: str) -> list:
    s = p.channel_scales(name)
    H = p.hidden
    if gran == "per_tensor":
        return [float(s[0])]
    if gran == "per_gate":
        return [float(s[g * H]) for g in range(4)]
    return [float(v) for v in s]


def export_operators(p: lstm_ops.LstmQuantParams, cfg: dict) -> dict:
    out = {}
    for i, name in enumerate(OPERATORS):
        op = cfg["operators"][name]
        if name in PARAMETER_OPERATORS:
            if name.startswith("bias") and not p.bias_enabled:
                continue
            unsigned, symmetric, gran = False, True, op["granularity"]
            scales = _compact_scales(p, name, gran)
            zps = [0] * len(scales)
        else:
            unsigned, symmetric, gran = op["is_unsigned"], op["is_symmetric"], "per_tensor"
            scales = [p.scale(name)]
            zps = [p.zero_point(name)]
        lo, hi = _qrange(op["bitwidth"], unsigned)
        out[name] = {
            "dtype": f"{'U' if unsigned else ''}INT{op['bitwidth']}",
            "symmetric": symmetric,
            "scale": _one_or_list([_f32(s) for s in scales]),
            "zero_point": _one_or_list(zps),
            "enc_type": _EXTERNAL_GRANULARITY[gran],
            "real_min": _one_or_list([s * (lo - z) for s, z in zip(scales, zps)]),
            "real_max": _one_or_list([s * (hi - z) for s, z in zip(scales, zps)]),
        }
    return out


def _as_list(value, field, integer):
    is_list = isinstance(value, list)
    vals = value if is_list else [value]
    if not vals:
        raise ValueError(f"{field} cannot be empty")
    for v in vals:
        if isinstance(v, bool) or not isinstance(v, int if integer else (int, float)):
            raise ValueError(f"{field} must be a JSON {'integer' if integer else 'number'} "
                             "or an array of them")
        if not integer and not math.isfinite(float(v)):
            raise ValueError(f"{field} must be finite")
    return [int(v) if integer else float(v) for v in vals], is_list


def import_operators(ops: dict, hidden: int, bias: bool, scale_mode: str):
    """Public v1 operators -> (resolved config, LstmQuantParams); validates every field like
    the reference importer (_internal_operator / audit)."""
    expected = [n for n in OPERATORS if bias or not n.startswith("bias")]
    if set(ops) != set(expected):
        raise ValueError("operators must list exactly the module's quantisation points")
    cfg = default_quant_config()
    cfg["scale_mode"] = scale_mode
    p = lstm_ops.LstmQuantParams(hidden)
    s = p.struct
    s.bias_enabled = int(bool(bias))
    C = 4 * hidden
    for name in expected:
        e = ops[name]
        if not isinstance(e, dict) or set(e) != _EXTERNAL_FIELDS:
            raise ValueError(f"operator {name} has missing or unknown fields")
        if not isinstance(e["symmetric"], bool):
            raise ValueError(f"operator {name} symmetric must be a boolean")
        dt = e["dtype"]
        if not isinstance(dt, str) or not (dt.startswith("UINT") or dt.startswith("INT")):
            raise ValueError(f"operator {name} dtype is invalid")
        unsigned = dt.startswith("UINT")
        try:
            bits = int(dt[4:] if unsigned else dt[3:])
        except ValueError as err:
            raise ValueError(f"operator {name} dtype is invalid") from err
        _check_bits(bits)
        if e["enc_type"] not in _EXTERNAL_GRANULARITY.values():
            raise ValueError(f"operator {name} enc_type is invalid")
        gran = {v: k for k, v in _EXTERNAL_GRANULARITY.items()}[e["enc_type"]]
        scales, l1 = _as_list(e["scale"], f"{name}.scale", False)
        zps, l2 = _as_list(e["zero_point"], f"{name}.zero_point", True)
        rmin, l3 = _as_list(e["real_min"], f"{name}.real_min", False)
        rmax, l4 = _as_list(e["real_max"], f"{name}.real_max", False)
        if not (l1 == l2 == l3 == l4) or not (len(scales) == len(zps) == len(rmin) == len(rmax)):
            raise ValueError(f"operator {name} scalar/array forms or lengths disagree")
        lo, hi = _qrange(bits, unsigned)
        for k, (sc, z, a, b) in enumerate(zip(scales, zps, rmin, rmax)):
            if not (math.isclose(a, sc * (lo - z), rel_tol=1e-12)
                    and math.isclose(b, sc * (hi - z), rel_tol=1e-12)):
                raise ValueError(f"operator {name} real_min/real_max[{k}] disagree with scale/zp")
            if not sc > 0.0 or not math.isfinite(_f32(sc)) or _f32(sc) <= 0.0:
                raise ValueError(f"operator {name} scale must be a finite positive FP32")
        i = L.OP[name]
        if name in PARAMETER_OPERATORS:
            if unsigned or not e["symmetric"] or any(zps):
                raise ValueError(f"{name} must be signed symmetric with zero_point 0")
            n = {"per_tensor": 1, "per_gate": 4, "per_channel": C}[gran]
            if len(scales) != n:
                raise ValueError(f"{name} needs {n} scales for {gran}")
            arr = np.asarray(scales, np.float32)
            full = (np.full(C, arr[0], np.float32) if n == 1 else
                    np.repeat(arr, hidden).astype(np.float32) if n == 4 else arr)
            L.chan_scales(s, L.PARAM_OPS.index(name))[:] = full
            cfg["operators"][name] = {"bitwidth": bits, "granularity": gran}
            s.config.op[i] = L.OpConfig(bits, 0, 1, _GRANULARITY[gran])
        else:
            if gran != "per_tensor" or len(scales) != 1:
                raise ValueError(f"{name} must be per-tensor")
            if not lo <= zps[0] <= hi:
                raise ValueError(f"{name} zero_point is outside the quantised range")
            s.scale[i] = _f32(scales[0])
            s.zero_point[i] = zps[0]
            cfg["operators"][name] = {"bitwidth": bits, "is_unsigned": unsigned,
                                      "is_symmetric": e["symmetric"]}
            s.config.op[i] = L.OpConfig(bits, int(unsigned), int(e["symmetric"]), L.PER_TENSOR)
    if not bias:
        for name in ("bias_ih", "bias_hh"):
            s.config.op[L.OP[name]] = config_struct(cfg).op[L.OP[name]]
    _validate_resolved(cfg)
    s.config.scale_mode = L.POT2 if scale_mode == "pot2" else L.AFFINE
    # the derived execution encodings reject inconsistent documents (e.g. POT2 scales that
    # are not powers of two)
    lstm_ops.check_params(p, 1)
    return cfg, p


# ------------------------------------------------------------------------------------------
# autograd bridge (lstm_autograd.py:139-258)
# ------------------------------------------------------------------------------------------

# Training forwards of the module keep the checkpoints other than hidden and the recurrence
# masks as blocked codes (lstm_ops.forward_quant(codes=True), 16-bit codes and mask bits)
# rather than the reference's fp32 / byte format; qat_saved_state() decodes them on request and
# the gradients are the same bit for bit.  False: the reference format throughout.
SAVE_STATE_AS_CODES = True


class _QuantizedLSTMFunction(torch.autograd.Function):
    """One direction, time-major.  Saves the 25 backward tensors (7 masters, 7 master masks,
    4 checkpoints, 7 checkpoint masks) when ``save_checkpoints`` is set, or with the saved
    codes the masters, hidden, the ih-linear mask and the two code arrays."""

    @staticmethod
    def forward(ctx, x, W_ih, W_hh, b_ih, b_hh, h0, c0, params, save_checkpoints, sink):
        codes = bool(save_checkpoints and SAVE_STATE_AS_CODES and W_hh.shape[1] % 16 == 0
                     and lstm_ops.codes_fit(params))
        out, hn, cn, saved = lstm_ops.forward_quant(x, W_ih, W_hh, b_ih, b_hh, h0, c0, params,
                                                    save_checkpoints, codes=codes)
        ctx.has_checkpoints = saved is not None
        ctx.params = params
        ctx.has_bias = b_ih is not None
        ctx.has_state = h0 is not None
        if saved is not None:
            sink["saved"] = saved
            sink["batch"] = x.shape[1]
            ctx.names = [k for k in L.SAVED_FIELDS + lstm_ops.CODE_KEYS if saved.get(k) is not None]
            ctx.save_for_backward(*(saved[k] for k in ctx.names))
        return out, hn, cn

    @staticmethod
    def backward(ctx, grad_out, grad_hn, grad_cn):
        if not ctx.has_checkpoints:
            raise RuntimeError("quantised backward needs the training q-carrier checkpoints "
                               "(run the forward with grad enabled or in training mode)")
        saved = dict(zip(ctx.names, ctx.saved_tensors))
        go = grad_out if grad_out is not None else torch.zeros_like(saved["hidden"])
        dx, dwi, dwh, dbi, dbh, dh0, dc0 = lstm_ops.backward_quant(saved, ctx.params, go, grad_hn,
                                                                   grad_cn)
        return (dx, dwi, dwh, dbi if ctx.has_bias else None, dbh if ctx.has_bias else None,
                dh0 if ctx.has_state else None, dc0 if ctx.has_state else None, None, None, None)


class _FloatLSTMFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, W_ih, W_hh, b_ih, b_hh, h0, c0):
        return lstm_ops.forward_float(x, W_ih, W_hh, b_ih, b_hh, h0, c0)

    @staticmethod
    def backward(ctx, *grads):
        raise NotImplementedError("the float QuantLSTM path has no backward in this build; "
                                  "train with use_quantization=True (QAT) after calibration")


def _qat_state(saved: dict, params=None, batch: int = 0) -> dict:
    """The reference's qat_saved_state layout (masks as bool views of the uint8 masks); saved
    codes are decoded into it first."""
    if "codes_blocks" in saved:
        saved = {**saved, **lstm_ops.decode_saved_codes(saved, params, batch)}
    m = lambda k: None if saved.get(k) is None else saved[k].view(torch.bool)
    master = {"input": "x", "weight_ih": "w_ih", "weight_hh": "w_hh", "bias_ih": "b_ih",
              "bias_hh": "b_hh", "h_0": "h0", "c_0": "c0"}
    return {
        "quantized_master": {k: saved[v + "_q"] for k, v in master.items()
                             if saved.get(v + "_q") is not None},
        "master_clamp_masks": {k: m(v + "_m") for k, v in master.items()
                               if saved.get(v + "_m") is not None},
        "checkpoints": {"gate_outputs": saved["gate_out"], "cell_states": saved["cell"],
                        "cell_tanh_outputs": saved["cell_tanh"],
                        "hidden_outputs": saved["hidden"]},
        "checkpoint_clamp_masks": {
            "weight_ih_linear": m("ih_linear_m"), "weight_hh_linear": m("hh_linear_m"),
            "gate_inputs": m("gate_in_m"), "gate_outputs": m("gate_out_m"),
            "cell_states": m("cell_m"), "cell_tanh_outputs": m("cell_tanh_m"),
            "hidden_outputs": m("hidden_m")},
    }


# ------------------------------------------------------------------------------------------
# the module
# ------------------------------------------------------------------------------------------

class QuantLSTM(nn.Module):
    """Single-layer, uni- or bidirectional LSTM with nn.LSTM's interface.

    ``use_quantization=False`` runs the float path; after calibration (``calibrating=True``
    forwards, then ``finalize_calibration()``) ``use_quantization=True`` runs the FP32
    q-carrier path with STE backward (quant_lstm.py:397-862, 863-1418)."""

    def __init__(self, input_size: int, hidden_size: int, num_layers: int = 1, bias: bool = True,
                 batch_first: bool = False, dropout: float = 0.0, bidirectional: bool = False, *,
                 device=None, dtype=None, use_quantization: bool = False,
                 quant_config: dict | str | Path | None = None,
                 calibration_method: str = "minmax", cublas_math_mode: str = "pedantic",
                 require_exact_accumulation: bool = False) -> None:
        super().__init__()
        if input_size <= 0 or hidden_size <= 0:
            raise ValueError("input_size and hidden_size must be positive")
        if num_layers != 1:
            raise ValueError("only num_layers=1 is supported")
        if dropout != 0.0:
            raise ValueError("only dropout=0 is supported")
        if dtype not in (None, torch.float32):
            raise ValueError("only torch.float32 is supported")
        if calibration_method not in _CALIBRATION_METHODS:
            raise ValueError("calibration_method must be minmax, sqnr or percentile")
        if cublas_math_mode not in _MATH_MODES:
            raise ValueError("cublas_math_mode must be pedantic or tf32")
        self.input_size = input_size
        self.hidden_size = hidden_size
        self.num_layers = num_layers
        self.bias = bias
        self.batch_first = batch_first
        self.dropout = dropout
        self.bidirectional = bool(bidirectional)
        self.use_quantization = bool(use_quantization)
        self.calibrating = False
        self.require_exact_accumulation = bool(require_exact_accumulation)
        self._calibration_method = calibration_method
        self._percentile_value = 99.99
        # the GEMMs here are exact integer products: both math modes give the pedantic result
        self._cublas_math_mode = cublas_math_mode
        fk = {"device": device, "dtype": torch.float32}
        H4 = 4 * hidden_size
        for sfx in self._suffixes():
            setattr(self, f"weight_ih_l0{sfx}", nn.Parameter(torch.empty((H4, input_size), **fk)))
            setattr(self, f"weight_hh_l0{sfx}", nn.Parameter(torch.empty((H4, hidden_size), **fk)))
            if bias:
                setattr(self, f"bias_ih_l0{sfx}", nn.Parameter(torch.empty(H4, **fk)))
                setattr(self, f"bias_hh_l0{sfx}", nn.Parameter(torch.empty(H4, **fk)))
            else:
                self.register_parameter(f"bias_ih_l0{sfx}", None)
                self.register_parameter(f"bias_hh_l0{sfx}", None)
        self.reset_parameters()
        self._config = resolve_quant_config(_load_json_source(quant_config))
        self._invalidate_quant_params()

    # ---- basic properties ----
    def _suffixes(self):
        return ("", "_reverse") if self.bidirectional else ("",)

    @property
    def num_directions(self) -> int:
        return 2 if self.bidirectional else 1

    @property
    def calibration_method(self) -> str:
        return self._calibration_method

    @calibration_method.setter
    def calibration_method(self, value: str) -> None:
        if value not in _CALIBRATION_METHODS:
            raise ValueError("calibration_method must be minmax, sqnr or percentile")
        if value != self._calibration_method:
            self.reset_calibration()
        self._calibration_method = value

    @property
    def cublas_math_mode(self) -> str:
        return self._cublas_math_mode

    @cublas_math_mode.setter
    def cublas_math_mode(self, value: str) -> None:
        if value not in _MATH_MODES:
            raise ValueError("cublas_math_mode must be pedantic or tf32")
        self._cublas_math_mode = value

    @property
    def percentile_value(self) -> float:
        return self._percentile_value

    @percentile_value.setter
    def percentile_value(self, value: float) -> None:
        value = float(value)
        if not math.isfinite(value) or not 0 < value <= 100:
            raise ValueError("percentile_value must be in (0, 100]")
        if value != self._percentile_value:
            self.reset_calibration()
        self._percentile_value = value

    def reset_parameters(self) -> None:
        bound = 1.0 / math.sqrt(self.hidden_size)
        with torch.no_grad():
            for p in self.parameters():
                p.uniform_(-bound, bound)

    def _direction_params(self, reverse: bool):
        sfx = "_reverse" if reverse else ""
        return (getattr(self, f"weight_ih_l0{sfx}"), getattr(self, f"weight_hh_l0{sfx}"),
                getattr(self, f"bias_ih_l0{sfx}"), getattr(self, f"bias_hh_l0{sfx}"))

    # ---- configuration ----
    def _invalidate_quant_params(self) -> None:
        self._quant_params_locked = False
        self._stats: list = [None] * self.num_directions
        self._batch_count = [0] * self.num_directions
        self._params: list = [None] * self.num_directions
        self._qat_saved_state = None

    def __getstate__(self):
        if self.calibrating:
            raise RuntimeError("Cannot copy QuantLSTM during calibration")
        state = super().__getstate__().copy()
        state["_qat_saved_state"] = None
        state["_params"] = [None if p is None else p.to_dict() for p in self._params]
        return state

    def __setstate__(self, state):
        params = state.get("_params", [])
        state["_params"] = [None if d is None else lstm_ops.LstmQuantParams.from_dict(d)
                            for d in params]
        super().__setstate__(state)

    def load_quant_config(self, source) -> None:
        cfg = resolve_quant_config(_load_json_source(source))
        if cfg == self._config:
            return
        if self.is_calibrated():
            raise RuntimeError("Reset QuantLSTM calibration before changing quant_config")
        self._config = cfg
        self._invalidate_quant_params()

    def get_quant_config(self, operator: Optional[str] = None) -> dict:
        if operator is None:
            return copy.deepcopy(self._config)
        if operator not in self._config["operators"]:
            raise ValueError(f"unknown quant operator: {operator}")
        return copy.deepcopy(self._config["operators"][operator])

    def adjust_quant_config(self, operator: str, **changes: Any) -> None:
        allowed = {"bitwidth", "is_unsigned", "is_symmetric", "granularity"}
        unknown = set(changes) - allowed
        if unknown:
            raise ValueError(f"unknown config fields: {sorted(unknown)}")
        if not changes:
            raise ValueError("give at least one config field")
        if operator not in self._config["operators"]:
            raise ValueError(f"unknown quant operator: {operator}")
        self._config = resolve_quant_config({"schema_version": 1,
                                             "operators": {operator: dict(changes)}},
                                            defaults=self._config)
        self._invalidate_quant_params()

    def set_all_bitwidth(self, bitwidth: int = 8) -> None:
        self._config = resolve_quant_config(
            {"schema_version": 1, "operators": {n: {"bitwidth": bitwidth} for n in OPERATORS}},
            defaults=self._config)
        self._invalidate_quant_params()

    # ---- calibration ----
    def quant_params_locked(self) -> bool:
        return self._quant_params_locked

    def set_quant_params_locked(self, locked: bool = True) -> None:
        if locked and not self.is_calibrated():
            raise RuntimeError("Cannot lock uncalibrated QuantLSTM parameters")
        self._quant_params_locked = bool(locked)

    def reset_calibration(self) -> None:
        self._invalidate_quant_params()

    def is_calibrated(self) -> bool:
        return all(p is not None for p in self._params)

    def calibration_state(self):
        def one(d):
            if self._params[d] is not None:
                return "locked"
            return "dirty" if self._stats[d] is not None else "empty"

        if not self.bidirectional:
            return one(0)
        return {"forward": one(0), "reverse": one(1)}

    def finalize_calibration(self) -> dict:
        """MinMax finalisation of every direction (CalibrationSession::finalize)."""
        if any(s is None for s in self._stats):
            raise RuntimeError("no calibration data: set calibrating=True and run forward first")
        if self.bidirectional and self._batch_count[0] != self._batch_count[1]:
            raise RuntimeError("bidirectional calibration batch counts differ")
        cfg = config_struct(self._config)
        self._params = [lstm_ops.finalize_params(s, cfg, self.hidden_size, self.bias)
                        for s in self._stats]
        if self.bidirectional:
            a, b = self._params
            if (a.scale("input"), a.zero_point("input")) != (b.scale("input"),
                                                             b.zero_point("input")):
                raise RuntimeError("both directions must share the same input grid")
        return {"batch_count": self._batch_count[0], "method": self._calibration_method}

    # ---- forward ----
    def _split_state(self, x: Tensor, hx):
        D, H = self.num_directions, self.hidden_size
        if hx is None:
            return [(None, None)] * D
        if len(hx) != 2:
            raise ValueError("hx must be (h_0, c_0)")
        h, c = hx
        if h is None or c is None:
            raise ValueError("h_0 and c_0 must be given together")
        B = x.size(0 if self.batch_first else 1)
        if tuple(h.shape) != (D, B, H) or tuple(c.shape) != (D, B, H):
            raise RuntimeError(f"h_0/c_0 must have shape [{D},{B},{H}]")
        return [(h[d], c[d]) for d in range(D)]

    def _directions(self, x: Tensor, hx, run):
        xt = x.transpose(0, 1) if self.batch_first else x
        outs, hs, cs = [], [], []
        for d, (h0, c0) in enumerate(self._split_state(x, hx)):
            xd = torch.flip(xt, (0,)) if d == 1 else xt
            o, h, c = run(d, xd.contiguous(), h0, c0)
            outs.append(torch.flip(o, (0,)) if d == 1 else o)
            hs.append(h)
            cs.append(c)
        out = outs[0] if len(outs) == 1 else torch.cat(outs, dim=-1)
        if self.batch_first:
            out = out.transpose(0, 1)
        return out, (torch.stack(hs, 0), torch.stack(cs, 0))

    def _collect_calibration(self, x: Tensor, hx):
        if self._calibration_method != "minmax":
            raise NotImplementedError(f"{self._calibration_method} calibration is not provided "
                                      "by this build (MinMax only)")

        def run(d, xd, h0, c0):
            if self._stats[d] is None:
                self._stats[d] = lstm_ops.new_stats(self.hidden_size, xd.device)
            self._params[d] = None
            self._batch_count[d] += 1
            Wi, Wh, bi, bh = (None if p is None else p.detach() for p in self._direction_params(d == 1))
            return lstm_ops.forward_calibrate(xd, Wi, Wh, bi, bh,
                                              None if h0 is None else h0.detach(),
                                              None if c0 is None else c0.detach(), self._stats[d])

        with torch.no_grad():
            return self._directions(x, hx, run)

    def _float_forward(self, x: Tensor, hx):
        def run(d, xd, h0, c0):
            return _FloatLSTMFunction.apply(xd, *self._direction_params(d == 1), h0, c0)

        return self._directions(x, hx, run)

    def qat_saved_state(self):
        st = self._qat_saved_state
        if callable(st):  # saved codes: decoded on the first request
            st = self._qat_saved_state = st()
        return st

    def _quantized_forward(self, x: Tensor, hx):
        if not self.is_calibrated():
            raise RuntimeError("quantised forward needs finalize_calibration() or "
                               "load_quant_params() first")
        save = x.is_cuda and (self.training or torch.is_grad_enabled())
        sinks = []

        def run(d, xd, h0, c0):
            sink = {}
            sinks.append(sink)
            return _QuantizedLSTMFunction.apply(xd, *self._direction_params(d == 1), h0, c0,
                                                self._params[d], save, sink)

        result = self._directions(x, hx, run)
        if self.training and save:
            params = list(self._params)

            def build(sinks=sinks, params=params, bidir=self.bidirectional):
                states = [_qat_state(s["saved"], params[d], s["batch"]) if "saved" in s else None
                          for d, s in enumerate(sinks)]
                return states[0] if not bidir else {"forward": states[0], "reverse": states[1]}

            self._qat_saved_state = build
        else:
            self._qat_saved_state = None
        return result

    def forward(self, input: Tensor, hx: Optional[tuple] = None):
        if not input.is_cuda:
            raise RuntimeError("QuantLSTM on this build runs on the GPU only (MI355X kernels; "
                               "there is no CPU path)")
        if input.dim() != 3 or input.size(-1) != self.input_size:
            raise RuntimeError(f"input must be 3-D with {self.input_size} features")
        if self.calibrating:
            return self._collect_calibration(input, hx)
        if self.use_quantization:
            return self._quantized_forward(input, hx)
        return self._float_forward(input, hx)

    # ---- quant params document ----
    def export_quant_params(self, destination: str | Path | None = None) -> dict:
        if not self.is_calibrated():
            raise RuntimeError("the module is not calibrated; nothing to export")
        doc = {
            "schema_version": 1,
            "model_info": {"input_size": self.input_size, "hidden_size": self.hidden_size,
                           "bias": self.bias, "batch_first": self.batch_first,
                           "bidirectional": self.bidirectional,
                           "use_pot2_scale": self._config["scale_mode"] == "pot2"},
            "execution_metadata": {"carrier": "cuda_fp32_qcarrier",
                                   "activation_mode": "real_sigmoid_tanh",
                                   "cublas_math_mode": self.cublas_math_mode,
                                   "standard_scale_mode": self._config["scale_mode"]},
            "operators": export_operators(self._params[0], self._config),
        }
        if self.bidirectional:
            doc["operators_reverse"] = export_operators(self._params[1], self._config)
        if destination is not None:
            Path(destination).write_text(json.dumps(doc, indent=2, ensure_ascii=False) + "\n",
                                         encoding="utf-8")
        return doc

    def load_quant_params(self, source) -> None:
        doc = _load_json_source(source)
        fields = {"schema_version", "model_info", "execution_metadata", "operators"}
        if self.bidirectional:
            fields.add("operators_reverse")
        if set(doc) != fields:
            raise ValueError("quant params document has missing or unknown fields")
        if isinstance(doc["schema_version"], bool) or doc["schema_version"] != 1:
            raise ValueError("only quant params documents with schema_version=1 are supported")
        mi, md = doc["model_info"], doc["execution_metadata"]
        if not isinstance(mi, dict) or set(mi) != {"input_size", "hidden_size", "bias",
                                                   "batch_first", "bidirectional",
                                                   "use_pot2_scale"}:
            raise ValueError("model_info has missing or unknown fields")
        if (mi["input_size"], mi["hidden_size"], mi["bias"], mi["bidirectional"]) != (
                self.input_size, self.hidden_size, self.bias, self.bidirectional):
            raise ValueError("model_info shape, bias or bidirectional does not match the module")
        if mi["batch_first"] != self.batch_first:
            warnings.warn("the document's batch_first differs from the module; quant params "
                          "do not depend on layout", RuntimeWarning, stacklevel=2)
        if not isinstance(md, dict) or set(md) != {"carrier", "activation_mode",
                                                   "cublas_math_mode", "standard_scale_mode"}:
            raise ValueError("execution_metadata has missing or unknown fields")
        if md["carrier"] != "cuda_fp32_qcarrier":
            raise ValueError("only the cuda_fp32_qcarrier carrier is supported")
        if md["activation_mode"] != "real_sigmoid_tanh":
            raise ValueError("only the real_sigmoid_tanh activation mode is supported")
        if md["cublas_math_mode"] not in _MATH_MODES:
            raise ValueError("cublas_math_mode is invalid")
        if md["standard_scale_mode"] not in ("affine", "pot2"):
            raise ValueError("standard_scale_mode is invalid")
        if mi["use_pot2_scale"] != (md["standard_scale_mode"] == "pot2"):
            raise ValueError("use_pot2_scale disagrees with standard_scale_mode")
        keys = ["operators", "operators_reverse"] if self.bidirectional else ["operators"]
        loaded = [import_operators(doc[k], self.hidden_size, self.bias,
                                   md["standard_scale_mode"]) for k in keys]
        if self.bidirectional and loaded[0][0] != loaded[1][0]:
            raise ValueError("both directions must use the same operator configuration")
        self._config = loaded[0][0]
        self._invalidate_quant_params()
        self._params = [p for _, p in loaded]
        self.cublas_math_mode = md["cublas_math_mode"]

    import_quant_params = load_quant_params

    def extra_repr(self) -> str:
        return (f"{self.input_size}, {self.hidden_size}, bias={self.bias}, "
                f"batch_first={self.batch_first}, bidirectional={self.bidirectional}, "
                f"use_quantization={self.use_quantization}")
