"""MI355X drop-in for the reference's native QuantLSTM module ``_quant_lstm``
(``operators/quant-lstm/pytorch/lib/lstm_interface_binding.cc:917-975``), the module its
autograd bridge imports (``lstm_autograd.py:10``) and its ``quant_lstm.py`` calls.

The functions take the reference's arguments and return its structures:
  lstm_forward_quantized(input, weight_ih, weight_hh, bias_ih, bias_hh, initial_hidden,
      initial_cell, batch_first, bundle_json, math_mode, require_exact_accumulation,
      save_checkpoints) -> (output, h_n, c_n, checkpoints, safety)
  lstm_backward_qat(master_values, batch_first, bundle_json, checkpoint_values, grad_output,
      grad_final_hidden, grad_final_cell, master_masks, checkpoint_masks) -> 7 gradients
  CalibrationSession(resolved_config_json, input_size, hidden_size, bias_enabled, method,
      percentile) with collect / finalize / reset / state / batch_count
  resolve_quant_config, validate_resolved_quant_config, audit_quant_params_bundle, lstm_forward
and run on librxmet.so (``include/rxmet_lstm.h``) through ``lstm_ops`` on PyTorch's current
stream.  The quantisation parameters travel as the reference's params bundle JSON (schema 1:
input_size, hidden_size, bias_enabled, scale_mode, and per operator bitwidth, is_unsigned,
is_symmetric, granularity, scales as shortest round-trip FP32 strings, zero_points; parameter
operators with all 4H values), parsed once per distinct text and cached.

Differences from the reference:
  * the quantised GEMMs are exact integer products, so ``math_mode`` ("pedantic" / "tf32") is
    validated and has no further effect;
  * the FP32 exactness audit of the pointwise q-carrier arithmetic (``auditQuantParamsBundle``,
    src/lstm/lstm_execution_params.cc:211-328) is not part of this build: the returned safety
    summary classifies the two linears, which are exact here for every range, and marks the
    gate, cell and output entries ``not_audited``; ``require_exact_accumulation=True`` raises
    NotImplementedError instead of answering without the audit;
  * a training forward's checkpoints hold the four traces the backward consumes (gate outputs,
    cell states, tanh of the cell, hidden outputs) and all seven clamp-mask families; the three
    trace-only linears / gate-input values are not materialised;
  * SQNR / percentile calibration and the float-path training entry points
    (``lstm_forward_training``, ``lstm_backward_float``) raise NotImplementedError.
"""
from __future__ import annotations

import collections
import json
import math
from typing import Any, Optional

import numpy as np
import torch

import lstm_ops
import quant_lstm as _Q
import rxmet_lstm_abi as L

_F32 = torch.float32
_CHECKPOINT_NAMES = ("weight_ih_linear", "weight_hh_linear", "gate_inputs", "gate_outputs",
                     "cell_states", "cell_tanh_outputs", "hidden_outputs")
_CHECKPOINT_SAVED = ("ih_linear_m", "hh_linear_m", "gate_in_m", "gate_out_m", "cell_m",
                     "cell_tanh_m", "hidden_m")
_VALUE_NAMES = ("gate_outputs", "cell_states", "cell_tanh_outputs", "hidden_outputs")
_VALUE_SAVED = ("gate_out", "cell", "cell_tanh", "hidden")
_MASTER_NAMES = ("input", "weight_ih", "weight_hh", "bias_ih", "bias_hh", "h_0", "c_0")
_MASTER_SAVED = ("x", "w_ih", "w_hh", "b_ih", "b_hh", "h0", "c0")
_MATH_MODES = ("pedantic", "tf32")

cpu_only = False


# ------------------------------------------------------------------------------------------
# FP32 scale text: the shortest decimal that reads back to the same FP32 value, laid out as
# std::to_chars(..., std::chars_format::general) writes it (src/lstm/quant_params_io.cc:66-78):
# plain digits for decimal exponents -4..5, otherwise d[.ddd]e+XX.
# ------------------------------------------------------------------------------------------

def format_float32(value: float) -> str:
    v = np.float32(value)
    if not np.isfinite(v):
        raise ValueError("a standard scale must be a finite FP32 value")
    if v == 0:
        return "-0" if np.signbit(v) else "0"
    sci = np.format_float_scientific(v, unique=True, trim="-")
    sign = "-" if sci.startswith("-") else ""
    mant, exp = sci.lstrip("-").split("e")
    digits = mant.replace(".", "")
    x = int(exp)
    if -4 <= x < 6:
        if x >= 0:
            whole = digits[:x + 1].ljust(x + 1, "0")
            frac = digits[x + 1:]
            return sign + whole + ("." + frac if frac else "")
        return sign + "0." + "0" * (-x - 1) + digits
    m = digits[0] + ("." + digits[1:] if len(digits) > 1 else "")
    return f"{sign}{m}e{'-' if x < 0 else '+'}{abs(x):02d}"


def _parse_scale(text: Any) -> float:
    if not isinstance(text, str):
        raise ValueError("scale must be a canonical FP32 string")
    try:
        value = np.float32(float(text))
    except ValueError as err:
        raise ValueError(f"scale is not a decimal number: {text!r}") from err
    if not np.isfinite(value) or format_float32(value) != text:
        raise ValueError(f"scale is not the shortest round-trip FP32 decimal string: {text!r}")
    return float(value)


# ------------------------------------------------------------------------------------------
# resolved configuration (src/lstm/quant_config_loader.cc:220-390)
# ------------------------------------------------------------------------------------------

def _parse_resolved(text: str) -> dict:
    root = _Q._strict_json_loads(text)
    bad = set(root) - {"schema_version", "scale_mode", "operators"}
    if bad:
        raise ValueError(f"resolved root unknown field: {sorted(bad)[0]}")
    sv = root.get("schema_version")
    if isinstance(sv, bool) or sv != 1:
        raise ValueError("only schema_version=1 is supported")
    if not isinstance(root.get("scale_mode"), str):
        raise ValueError("resolved scale_mode is missing or not a string")
    ops = root.get("operators")
    if not isinstance(ops, dict):
        raise ValueError("resolved operators is missing or not an object")
    unknown = set(ops) - set(_Q.OPERATORS)
    if unknown:
        raise ValueError(f"unknown quant operator: {sorted(unknown)[0]}")
    cfg = {"schema_version": 1, "scale_mode": root["scale_mode"], "operators": {}}
    for name in _Q.OPERATORS:
        if name not in ops:
            raise ValueError(f"resolved operator missing: {name}")
        e = ops[name]
        if not isinstance(e, dict):
            raise ValueError(f"{name} must be an object")
        param = name in _Q.PARAMETER_OPERATORS
        allowed = {"bitwidth", "granularity", "comment"} if param else \
            {"bitwidth", "is_unsigned", "is_symmetric", "comment"}
        extra = set(e) - allowed
        if extra:
            raise ValueError(f"{name} unknown field: {sorted(extra)[0]}")
        if "comment" in e and not isinstance(e["comment"], str):
            raise ValueError("comment must be a string")
        need = ("bitwidth", "granularity") if param else ("bitwidth", "is_unsigned", "is_symmetric")
        for f in need:
            if e.get(f) is None:
                raise ValueError(f"{name} resolved field missing: {f}")
        if param:
            if e["granularity"] not in _Q._GRANULARITY:
                raise ValueError(f"unknown granularity: {e['granularity']}")
            cfg["operators"][name] = {"bitwidth": _Q._check_bits(e["bitwidth"]),
                                      "granularity": e["granularity"]}
        else:
            cfg["operators"][name] = {"bitwidth": _Q._check_bits(e["bitwidth"]),
                                      "is_unsigned": _Q._check_bool(e["is_unsigned"], "is_unsigned"),
                                      "is_symmetric": _Q._check_bool(e["is_symmetric"],
                                                                     "is_symmetric")}
    _Q._validate_resolved(cfg)
    return cfg


def _canonical_config(cfg: dict) -> str:
    """toCanonicalJson (quant_config_loader.cc:365-385): two-space indentation, newline."""
    return json.dumps({"schema_version": 1, "scale_mode": cfg["scale_mode"],
                       "operators": {n: cfg["operators"][n] for n in _Q.OPERATORS}},
                      indent=2, ensure_ascii=False) + "\n"


def resolve_quant_config(defaults_json: str, override_json: str) -> str:
    """The resolved configuration of ``defaults_json`` (a resolved document, comments allowed)
    with the sparse override ``override_json`` applied; canonical JSON text."""
    defaults = _parse_resolved(defaults_json)
    override = _Q._strict_json_loads(override_json) if override_json.strip() else \
        {"schema_version": 1}
    return _canonical_config(_Q.resolve_quant_config(override, defaults))


def validate_resolved_quant_config(resolved_json: str) -> str:
    return _canonical_config(_parse_resolved(resolved_json))


# ------------------------------------------------------------------------------------------
# params bundle (src/lstm/quant_params_io.cc:178-258)
# ------------------------------------------------------------------------------------------

class _Bundle:
    __slots__ = ("input_size", "hidden", "bias", "config", "params")

    def __init__(self, input_size, hidden, bias, config, params):
        self.input_size, self.hidden, self.bias = input_size, hidden, bias
        self.config, self.params = config, params


_CACHE: "collections.OrderedDict[str, _Bundle]" = collections.OrderedDict()
_CACHE_SIZE = 32


def _int_field(root: dict, field: str) -> int:
    v = root.get(field)
    if isinstance(v, bool) or not isinstance(v, int):
        raise ValueError(f"{field} must be a JSON integer")
    return v


def _import_bundle(text: str) -> _Bundle:
    hit = _CACHE.get(text)
    if hit is not None:
        _CACHE.move_to_end(text)
        return hit
    root = _Q._strict_json_loads(text)
    bad = set(root) - {"schema_version", "input_size", "hidden_size", "bias_enabled",
                       "scale_mode", "operators"}
    if bad:
        raise ValueError(f"quant params root unknown field: {sorted(bad)[0]}")
    if _int_field(root, "schema_version") != 1:
        raise ValueError("only quant params bundle schema_version=1 is supported")
    input_size = _int_field(root, "input_size")
    hidden = _int_field(root, "hidden_size")
    if input_size <= 0 or hidden <= 0:
        raise ValueError("input_size and hidden_size must be positive")
    bias = root.get("bias_enabled")
    if not isinstance(bias, bool):
        raise ValueError("bias_enabled must be a boolean")
    mode = root.get("scale_mode")
    if mode not in ("affine", "pot2"):
        raise ValueError(f"unknown scale_mode: {mode}")
    ops = root.get("operators")
    if not isinstance(ops, dict):
        raise ValueError("operators is missing")
    names = [n for n in _Q.OPERATORS if bias or n not in ("bias_ih", "bias_hh")]
    extra = set(ops) - set(names)
    if extra:
        raise ValueError(f"operators holds an invalid or disabled field: {sorted(extra)[0]}")
    cfg = _Q.default_quant_config()
    cfg["scale_mode"] = mode
    p = lstm_ops.LstmQuantParams(hidden)
    s = p.struct
    s.bias_enabled = int(bias)
    C = 4 * hidden
    for name in names:
        if name not in ops:
            raise ValueError(f"operators is missing: {name}")
        e = ops[name]
        if not isinstance(e, dict):
            raise ValueError(f"{name} must be an object")
        extra = set(e) - {"bitwidth", "is_unsigned", "is_symmetric", "granularity", "scales",
                          "zero_points"}
        if extra:
            raise ValueError(f"{name} unknown field: {sorted(extra)[0]}")
        bits = _Q._check_bits(e.get("bitwidth"))
        uns = _Q._check_bool(e.get("is_unsigned"), "is_unsigned")
        sym = _Q._check_bool(e.get("is_symmetric"), "is_symmetric")
        gran = e.get("granularity")
        if gran not in _Q._GRANULARITY:
            raise ValueError(f"unknown granularity: {gran}")
        scales, zps = e.get("scales"), e.get("zero_points")
        if not isinstance(scales, list) or not isinstance(zps, list):
            raise ValueError("scales/zero_points must be arrays")
        param = name in _Q.PARAMETER_OPERATORS
        n = C if param else 1
        if len(scales) != n or len(zps) != n:
            raise ValueError("quant params must use the full 4H or the single-value form")
        for z in zps:
            if isinstance(z, bool) or not isinstance(z, int):
                raise ValueError("zero_point must be a JSON integer")
            if not -(1 << 31) <= z < (1 << 31):
                raise ValueError("zero_point is outside int32")
        vals = [_parse_scale(t) for t in scales]
        if any(not v > 0.0 for v in vals):
            raise ValueError(f"{name} scales must be positive")
        i = L.OP[name]
        if param:
            if uns or not sym or any(zps):
                raise ValueError(f"{name} must be signed symmetric with zero_point 0")
            cfg["operators"][name] = {"bitwidth": bits, "granularity": gran}
            s.config.op[i] = L.OpConfig(bits, 0, 1, _Q._GRANULARITY[gran])
            L.chan_scales(s, L.PARAM_OPS.index(name))[:] = np.asarray(vals, np.float32)
        else:
            if gran != "per_tensor":
                raise ValueError(f"{name} must be per_tensor")
            cfg["operators"][name] = {"bitwidth": bits, "is_unsigned": uns, "is_symmetric": sym}
            s.config.op[i] = L.OpConfig(bits, int(uns), int(sym), L.PER_TENSOR)
            s.scale[i] = vals[0]
            s.zero_point[i] = zps[0]
    if not bias:
        for name in ("bias_ih", "bias_hh"):
            s.config.op[L.OP[name]] = _Q.config_struct(cfg).op[L.OP[name]]
    _Q._validate_resolved(cfg)
    s.config.scale_mode = L.POT2 if mode == "pot2" else L.AFFINE
    # deriving the integer execution encodings rejects inconsistent parameter sets
    lstm_ops.check_params(p, input_size)
    b = _Bundle(input_size, hidden, bias, cfg, p)
    _CACHE[text] = b
    if len(_CACHE) > _CACHE_SIZE:
        _CACHE.popitem(last=False)
    return b


def _export_bundle(input_size: int, cfg: dict, p: lstm_ops.LstmQuantParams) -> str:
    """exportQuantParamsBundle: compact JSON, operators in QuantOperator order."""
    ops = {}
    for name in _Q.OPERATORS:
        if not p.bias_enabled and name in ("bias_ih", "bias_hh"):
            continue
        c = cfg["operators"][name]
        if name in _Q.PARAMETER_OPERATORS:
            scales = [format_float32(v) for v in p.channel_scales(name)]
            ops[name] = {"bitwidth": c["bitwidth"], "is_unsigned": False, "is_symmetric": True,
                         "granularity": c["granularity"], "scales": scales,
                         "zero_points": [0] * len(scales)}
        else:
            ops[name] = {"bitwidth": c["bitwidth"], "is_unsigned": c["is_unsigned"],
                         "is_symmetric": c["is_symmetric"], "granularity": "per_tensor",
                         "scales": [format_float32(p.scale(name))],
                         "zero_points": [p.zero_point(name)]}
    root = {"schema_version": 1, "input_size": int(input_size), "hidden_size": p.hidden,
            "bias_enabled": p.bias_enabled, "scale_mode": cfg["scale_mode"], "operators": ops}
    return json.dumps(root, separators=(",", ":"), ensure_ascii=False)


def _safety_summary(hidden: int) -> dict:
    """The safety summary's layout (lstm_interface_binding.cc:508-552) with what this build
    knows: both linears are exact integer GEMMs for every range; the pointwise arithmetic is
    not audited."""
    entries = [{"name": f"weight_ih_linear[{c}]", "fp32_accumulation": "exact_integer_range",
                "safe": True} for c in range(4 * hidden)]
    entries += [{"name": f"weight_hh_linear[{c}]", "fp32_accumulation": "exact_integer_range",
                 "safe": True} for c in range(4 * hidden)]
    for name in ("input_gate_input", "forget_gate_input", "cell_gate_input", "output_gate_input",
                 "cell_state", "output"):
        entries.append({"name": name, "fp32_accumulation": "not_audited", "safe": None})
    return {"exact_integer_range_count": 8 * hidden, "precision_risk_count": 0,
            "unsafe_non_finite_count": 0, "not_audited_count": 6, "has_precision_risk": False,
            "entries": entries}


def _check_exact_request(require_exact_accumulation: bool) -> None:
    if require_exact_accumulation:
        raise NotImplementedError("require_exact_accumulation needs the FP32 exactness audit of "
                                  "the pointwise arithmetic, which this build does not run")


def audit_quant_params_bundle(bundle_json: str, require_exact_accumulation: bool = False) -> dict:
    _check_exact_request(require_exact_accumulation)
    b = _import_bundle(bundle_json)
    return {"bundle_json": _export_bundle(b.input_size, b.config, b.params),
            "resolved_config_json": _canonical_config(b.config),
            "safety": _safety_summary(b.hidden), "input_size": b.input_size,
            "hidden_size": b.hidden, "bias_enabled": b.bias}


# ------------------------------------------------------------------------------------------
# forward / backward
# ------------------------------------------------------------------------------------------

def _time_major(t: torch.Tensor, batch_first: bool) -> torch.Tensor:
    return t.transpose(0, 1).contiguous() if batch_first else t.contiguous()


def _state(t: Optional[torch.Tensor], B: int, H: int, name: str) -> Optional[torch.Tensor]:
    if t is None or t.numel() == 0:
        return None
    if tuple(t.shape) != (1, B, H):
        raise RuntimeError(f"{name} must have shape [1, {B}, {H}]")
    return t[0].contiguous()


def _check_inputs(input, weight_ih, weight_hh, bias_ih, bias_hh, initial_hidden, initial_cell,
                  batch_first):
    if not input.is_cuda:
        raise RuntimeError("this build runs the LSTM on the GPU only")
    if input.dim() != 3:
        raise RuntimeError("input must be 3-D")
    x = _time_major(input, batch_first)
    T, B, I = x.shape
    H = weight_hh.shape[1]
    if tuple(weight_ih.shape) != (4 * H, I) or tuple(weight_hh.shape) != (4 * H, H):
        raise RuntimeError("weight_ih / weight_hh shapes do not match the input and hidden sizes")
    if (bias_ih is None) != (bias_hh is None):
        raise RuntimeError("bias_ih and bias_hh must be given together")
    if (initial_hidden is None) != (initial_cell is None):
        raise RuntimeError("initial_hidden and initial_cell must be given together")
    h0 = _state(initial_hidden, B, H, "initial_hidden")
    c0 = _state(initial_cell, B, H, "initial_cell")
    return x, T, B, I, H, h0, c0


def lstm_forward(input, weight_ih, weight_hh, bias_ih=None, bias_hh=None, initial_hidden=None,
                 initial_cell=None, batch_first=False):
    """Float forward (lstmForward): (output, h_n [1,B,H], c_n [1,B,H])."""
    x, T, B, I, H, h0, c0 = _check_inputs(input, weight_ih, weight_hh, bias_ih, bias_hh,
                                          initial_hidden, initial_cell, batch_first)
    out, hn, cn = lstm_ops.forward_float(x, weight_ih, weight_hh, bias_ih, bias_hh, h0, c0)
    return (out.transpose(0, 1) if batch_first else out), hn.unsqueeze(0), cn.unsqueeze(0)


def lstm_forward_training(*args, **kwargs):
    raise NotImplementedError("the float-path LSTM training forward and backward are not "
                              "provided by this build (QAT runs through lstm_forward_quantized)")


lstm_backward_float = lstm_forward_training


def lstm_forward_quantized(input, weight_ih, weight_hh, bias_ih=None, bias_hh=None,
                           initial_hidden=None, initial_cell=None, batch_first=False,
                           bundle_json="", math_mode="pedantic",
                           require_exact_accumulation=False, save_checkpoints=False):
    """lstmForwardQuantized (lstm_interface_binding.cc:643-806): (output, h_n [1,B,H],
    c_n [1,B,H], checkpoints, safety).  checkpoints is empty unless save_checkpoints; then it
    holds "values", "clamp_masks" (uint8), "quantized_master" (q-carrier codes; the input in
    the caller's layout, h_0 / c_0 as [1,B,H]) and "master_clamp_masks" (bool)."""
    if math_mode not in _MATH_MODES:
        raise ValueError("cublas_math_mode must be pedantic or tf32")
    _check_exact_request(require_exact_accumulation)
    x, T, B, I, H, h0, c0 = _check_inputs(input, weight_ih, weight_hh, bias_ih, bias_hh,
                                          initial_hidden, initial_cell, batch_first)
    b = _import_bundle(bundle_json)
    if b.input_size != I:
        raise RuntimeError("quant params input_size does not match the module")
    if b.hidden != H:
        raise RuntimeError("quant params hidden_size does not match the module")
    if b.bias != (bias_ih is not None):
        raise RuntimeError("quant params bias_enabled does not match the module")
    out, hn, cn, saved = lstm_ops.forward_quant(x, weight_ih, weight_hh, bias_ih, bias_hh, h0, c0,
                                                b.params, bool(save_checkpoints))
    checkpoints: dict = {}
    if save_checkpoints:
        checkpoints["values"] = {n: saved[k] for n, k in zip(_VALUE_NAMES, _VALUE_SAVED)}
        checkpoints["clamp_masks"] = {n: saved[k] for n, k in zip(_CHECKPOINT_NAMES,
                                                                   _CHECKPOINT_SAVED)}
        master, masks = {}, {}
        for n, k in zip(_MASTER_NAMES, _MASTER_SAVED):
            if k + "_q" not in saved:
                continue
            v, m = saved[k + "_q"], saved[k + "_m"].view(torch.bool)
            if n == "input" and batch_first:
                v, m = v.transpose(0, 1), m.transpose(0, 1)
            if n in ("h_0", "c_0"):
                v, m = v.unsqueeze(0), m.unsqueeze(0)
            master[n], masks[n] = v, m
        checkpoints["quantized_master"] = master
        checkpoints["master_clamp_masks"] = masks
    if batch_first:
        out = out.transpose(0, 1)
    return out, hn.unsqueeze(0), cn.unsqueeze(0), checkpoints, _safety_summary(H)


def _as_u8(t: torch.Tensor) -> torch.Tensor:
    t = t.contiguous()
    return t.view(torch.uint8) if t.dtype == torch.bool else t.to(torch.uint8)


def lstm_backward_qat(master_values, batch_first, bundle_json, checkpoint_values, grad_output,
                      grad_final_hidden, grad_final_cell, master_masks, checkpoint_masks):
    """lstmBackwardQat (lstm_interface_binding.cc:437-480): the STE backward from a training
    forward's masters (7: input in the caller's layout, weight_ih, weight_hh, bias_ih, bias_hh
    (empty without bias), h_0, c_0 [1,B,H]), checkpoint values (4), the time-major output
    gradient and the final-state gradients [B,H], and the clamp masks (7 + 7).  Returns
    (dx in the caller's layout, dW_ih, dW_hh, db_ih, db_hh, dh0 [B,H], dc0 [B,H]); the bias
    gradients are empty tensors without bias."""
    if len(master_values) != 7:
        raise RuntimeError("QAT master_values must hold 7 tensors")
    if len(checkpoint_values) != 4:
        raise RuntimeError("QAT checkpoint_values must hold the 4 minimum trace tensors")
    if len(master_masks) != 7 or len(checkpoint_masks) != 7:
        raise RuntimeError("QAT masks must hold 7 master and 7 checkpoint masks")
    b = _import_bundle(bundle_json)
    if not b.bias and (master_values[3].numel() or master_values[4].numel()):
        raise RuntimeError("with bias disabled the QAT bias masters must be empty")
    saved = {}
    for i, k in enumerate(_MASTER_SAVED):
        v, m = master_values[i], master_masks[i]
        if k in ("b_ih", "b_hh") and not b.bias:
            continue
        if k == "x":
            v, m = _time_major(v, batch_first), _time_major(m, batch_first)
        if k in ("h0", "c0"):
            v, m = v.reshape(v.shape[-2:]), m.reshape(m.shape[-2:])
        saved[k + "_q"] = v.contiguous()
        saved[k + "_m"] = _as_u8(m)
    for k, v in zip(_VALUE_SAVED, checkpoint_values):
        saved[k] = v.contiguous()
    for k, m in zip(_CHECKPOINT_SAVED, checkpoint_masks):
        saved[k] = _as_u8(m)
    dx, dwi, dwh, dbi, dbh, dh0, dc0 = lstm_ops.backward_quant(
        saved, b.params, grad_output, grad_final_hidden, grad_final_cell)
    empty = dx.new_empty(0)
    return ((dx.transpose(0, 1) if batch_first else dx), dwi, dwh,
            dbi if dbi is not None else empty, dbh if dbh is not None else empty, dh0, dc0)


# ------------------------------------------------------------------------------------------
# calibration (CalibrationSessionBinding, lstm_interface_binding.cc:808-900)
# ------------------------------------------------------------------------------------------

def _min_scale(lo: int, hi: int) -> np.float32:
    return np.float32(min(2.0 ** -23, 0.01 / (float(hi) - float(lo))))


def _adjusted_range(rmin: float, rmax: float, bits: int, unsigned: bool, symmetric: bool):
    """The range calibrateMinMax represents with its FP32 scale (src/quantization/
    scale_encoding.cc:47-101), reported as the activation ranges of finalize()."""
    lo, hi = _Q._qrange(bits, unsigned)
    steps = float(hi) - float(lo)
    rmin, rmax = np.float32(rmin), np.float32(rmax)
    if symmetric and not unsigned:
        cand = max(abs(float(rmin)), abs(float(rmax))) / hi
    elif symmetric:
        cand = float(max(rmax, np.float32(0))) / hi
    else:
        cand = (float(max(rmax, np.float32(0))) - float(min(rmin, np.float32(0)))) / steps
    floor = _min_scale(lo, hi)
    scale = floor if cand < float(floor) else np.float32(cand)
    if symmetric and not unsigned:
        ext = np.float32(np.float32(hi) * scale)
        return float(-ext), float(ext)
    if symmetric:
        return 0.0, float(np.float32(np.float32(hi) * scale))
    amin = min(rmin, np.float32(0))
    return float(amin), float(np.float32(amin + np.float32(np.float32(steps) * scale)))


class CalibrationSession:
    """MinMax calibration of one direction: collect() runs the float forward on the GPU and
    merges the statistics; finalize() derives the parameters once and locks the session."""

    def __init__(self, resolved_config_json: str, input_size: int, hidden_size: int,
                 bias_enabled: bool, method: str = "minmax", percentile: float = 99.99):
        self._config = _parse_resolved(resolved_config_json)
        if method not in ("minmax", "sqnr", "percentile"):
            raise ValueError("calibration_method must be minmax, sqnr or percentile")
        if not (math.isfinite(percentile) and 0.0 < percentile <= 100.0):
            raise ValueError("percentile must be in (0, 100]")
        if method != "minmax":
            raise NotImplementedError(f"{method} calibration is not provided by this build "
                                      "(MinMax only)")
        if input_size <= 0 or hidden_size <= 0:
            raise ValueError("input_size and hidden_size must be positive")
        self._input_size, self._hidden = int(input_size), int(hidden_size)
        self._bias = bool(bias_enabled)
        self._method = method
        self.reset()

    def reset(self) -> None:
        self._stats = None
        self._batches = 0
        self._state = "empty"
        self._finalized = None

    @property
    def state(self) -> str:
        return self._state

    @property
    def batch_count(self) -> int:
        return self._batches

    def collect(self, input, weight_ih, weight_hh, bias_ih=None, bias_hh=None,
                initial_hidden=None, initial_cell=None, batch_first=False):
        if self._state == "locked":
            raise RuntimeError("a locked calibration session refuses more data")
        x, T, B, I, H, h0, c0 = _check_inputs(input, weight_ih, weight_hh, bias_ih, bias_hh,
                                              initial_hidden, initial_cell, batch_first)
        if I != self._input_size or H != self._hidden:
            raise RuntimeError("calibration tensor shapes do not match the session")
        if (bias_ih is not None) != self._bias:
            raise RuntimeError("calibration bias state does not match the session")
        if self._stats is None:
            self._stats = lstm_ops.new_stats(self._hidden, x.device)
        with torch.no_grad():
            out, hn, cn = lstm_ops.forward_calibrate(
                x, weight_ih.detach(), weight_hh.detach(),
                None if bias_ih is None else bias_ih.detach(),
                None if bias_hh is None else bias_hh.detach(), h0, c0, self._stats)
        self._batches += 1
        self._state = "dirty"
        return (out.transpose(0, 1) if batch_first else out), hn.unsqueeze(0), cn.unsqueeze(0)

    def finalize(self, require_exact_accumulation: bool = False) -> dict:
        _check_exact_request(require_exact_accumulation)
        if self._state == "locked":
            return dict(self._finalized)
        if self._state == "empty":
            raise RuntimeError("an empty calibration session cannot be finalized")
        p = lstm_ops.finalize_params(self._stats, _Q.config_struct(self._config), self._hidden,
                                     self._bias)
        host = self._stats.detach().cpu().numpy()
        ranges = {}
        for name in _Q.OPERATORS:
            if name in _Q.PARAMETER_OPERATORS:
                continue
            i = L.OP[name]
            c = self._config["operators"][name]
            ranges[name] = _adjusted_range(host[i], host[L.NOPS + i], c["bitwidth"],
                                           c["is_unsigned"], c["is_symmetric"])
        self._finalized = {
            "bundle_json": _export_bundle(self._input_size, self._config, p),
            "resolved_config_json": _canonical_config(self._config),
            "safety": _safety_summary(self._hidden),
            "batch_count": self._batches,
            "method": self._method,
            "activation_ranges": ranges,
        }
        self._state = "locked"
        return dict(self._finalized)
