"""QuantGRU for MI355X: an ``nn.GRU``-compatible module whose QAT forward/backward and
MinMax calibration run in librxmet.so.

Mirrors the public surface of the reference module
(``operators/quant-gru/pytorch/quant_gru.py``): ``QuantGRU`` (:1120-2306), ``GRUFunction``
(:807-1102), the weight-format helpers (:664-806) and the operator map (:181-262), with
the reference's names, argument meanings and error behaviour, so a user can swap the
import.  Every numerical step goes through ``gru_ops`` (the replacement of the
reference's pybind module), which calls the HIP kernels; nothing here computes on the CPU.

Not provided (raise ``NotImplementedError`` with the reason): ``num_layers > 1`` and
dropout (as in the reference), histogram calibration ('sqnr', 'percentile'), the int32
quantised-value storage and the backward of the float (``use_quantization=False``) path;
its forward runs on the GPU.
"""
from __future__ import annotations

import copy
import json
import math
import re
from contextlib import contextmanager
from typing import Optional, Tuple

import numpy as np

import torch
import torch.nn as nn

import gru_ops
import rxmet_gru_abi as A

# ------------------------------------------------------------------------------------
# Operator map (quant_gru.py:181-262): public operator name -> config attribute names.
# ------------------------------------------------------------------------------------


def _op_info(base: str, per_channel: bool = False, default_unsigned: bool = False) -> dict:
    return {"bw_attr": base, "sym_attr": f"{base}symmetric_", "unsigned_attr": f"{base}unsigned_",
            "scale_attr": f"scale_{base}", "zp_attr": None if per_channel else f"zp_{base}",
            "is_per_channel": per_channel, "default_unsigned": default_unsigned}


_OPERATOR_MAP = {
    "input": _op_info("x_"),
    "output": _op_info("h_"),
    "weight_ih": _op_info("W_", per_channel=True),
    "weight_hh": _op_info("R_", per_channel=True),
    "bias_ih": _op_info("bw_", per_channel=True),
    "bias_hh": _op_info("br_", per_channel=True),
    "weight_ih_linear": _op_info("weight_ih_linear_"),
    "weight_hh_linear": _op_info("weight_hh_linear_"),
    "update_gate_input": _op_info("update_gate_input_"),
    "update_gate_output": _op_info("update_gate_output_", default_unsigned=True),
    "reset_gate_input": _op_info("reset_gate_input_"),
    "reset_gate_output": _op_info("reset_gate_output_", default_unsigned=True),
    "new_gate_input": _op_info("new_gate_input_"),
    "new_gate_output": _op_info("new_gate_output_"),
    "mul_reset_hidden": _op_info("mul_reset_hidden_"),
    "mul_old_contribution": _op_info("mul_old_contribution_"),
    "mul_new_contribution": _op_info("mul_new_contribution_"),
}
_VALID_BITWIDTH_ATTRS = {i["bw_attr"] for i in _OPERATOR_MAP.values()}
_VALID_SYMMETRIC_ATTRS = {i["sym_attr"] for i in _OPERATOR_MAP.values()}
_VALID_UNSIGNED_ATTRS = {i["unsigned_attr"] for i in _OPERATOR_MAP.values()}
_WEIGHT_SYMMETRIC_ATTRS = {"W_symmetric_", "R_symmetric_", "bw_symmetric_", "br_symmetric_"}
_ACTIVATION_SYMMETRIC_ATTRS = _VALID_SYMMETRIC_ATTRS - _WEIGHT_SYMMETRIC_ATTRS


def _validate_operator_map() -> None:
    """Import-time check that every mapped attribute exists on the config object
    (quant_gru.py:264-296)."""
    cfg = gru_ops.OperatorQuantConfig()
    missing = [f"{op} -> {a}" for op, info in _OPERATOR_MAP.items()
               for a in (info["bw_attr"], info["sym_attr"]) if not hasattr(cfg, a)]
    if missing:
        raise RuntimeError(f"_OPERATOR_MAP does not match OperatorQuantConfig: {missing}")


_validate_operator_map()

# ------------------------------------------------------------------------------------
# Weight-format helpers (quant_gru.py:664-759).  PyTorch stores gates as (r, z, n) rows;
# the kernels take (z, r, n) columns, i.e. W [I, 3H] and R [H, 3H].
# ------------------------------------------------------------------------------------

_GATE_PERM = {}


def _gate_perm(n3: int, device) -> torch.Tensor:
    key = (n3, str(device))
    perm = _GATE_PERM.get(key)
    if perm is None:
        h = n3 // 3
        perm = torch.cat([torch.arange(h, 2 * h), torch.arange(0, h),
                          torch.arange(2 * h, 3 * h)]).to(device)
        _GATE_PERM[key] = perm
    return perm


def reorder_weights_pytorch_to_haste(w: torch.Tensor) -> torch.Tensor:
    """(r, z, n) -> (z, r, n) along dim 0 (quant_gru.py:664-686); an involution."""
    w = w.contiguous()
    return w.index_select(0, _gate_perm(w.shape[0], w.device)).contiguous()


def reorder_weights_haste_to_pytorch(w: torch.Tensor) -> torch.Tensor:
    """(z, r, n) -> (r, z, n) along dim 0 (quant_gru.py:689-702)."""
    return reorder_weights_pytorch_to_haste(w)


_ZEROS = {}


def _zeros(n: int, device) -> torch.Tensor:
    """A cached read-only zero vector (the bias of a layer without biases)."""
    key = (n, str(device))
    z = _ZEROS.get(key)
    if z is None:
        z = _ZEROS[key] = torch.zeros(n, device=device, dtype=torch.float32)
    return z


def ensure_cuda_float32(tensor: torch.Tensor, device: torch.device) -> torch.Tensor:
    """quant_gru.py:705-711."""
    if tensor.device != device:
        tensor = tensor.to(device)
    if tensor.dtype != torch.float32:
        tensor = tensor.float()
    return tensor


def convert_weights_to_haste_format(weight_ih, weight_hh, bias_ih, bias_hh, hidden_size: int,
                                    device) -> Tuple[torch.Tensor, ...]:
    """(W [I,3H], R [H,3H], bw [3H], br [3H]) in kernel layout (quant_gru.py:714-759).
    Missing biases become zeros."""
    W = reorder_weights_pytorch_to_haste(ensure_cuda_float32(weight_ih, device)).t().contiguous()
    R = reorder_weights_pytorch_to_haste(ensure_cuda_float32(weight_hh, device)).t().contiguous()
    if bias_ih is not None and bias_hh is not None:
        bw = reorder_weights_pytorch_to_haste(ensure_cuda_float32(bias_ih, device))
        br = reorder_weights_pytorch_to_haste(ensure_cuda_float32(bias_hh, device))
    else:
        bw = torch.zeros(3 * hidden_size, device=device, dtype=torch.float32)
        br = torch.zeros(3 * hidden_size, device=device, dtype=torch.float32)
    return W, R, bw, br


def get_quant_range(bitwidth: int, is_unsigned: bool = False) -> Tuple[int, int]:
    """Integer grid of a bit width (quant_gru.py:766-797)."""
    if not 1 <= bitwidth <= 32:
        raise ValueError(f"bitwidth must be in range [1, 32], got {bitwidth}")
    if is_unsigned:
        return 0, (1 << bitwidth) - 1
    return -(1 << (bitwidth - 1)), (1 << (bitwidth - 1)) - 1


def _require_device(t: torch.Tensor) -> torch.device:
    if not t.is_cuda:
        raise RuntimeError("QuantGRU runs on the GPU: move the module and its inputs to a "
                           "CUDA (ROCm) device")
    return t.device


# ------------------------------------------------------------------------------------
# Quant-params JSON document (quant_gru.py:2548-2592, 3961-4230, 4353-4526): per operator
# dtype, symmetric, scale, zero_point, enc_type, real_min, real_max; per-tensor operators
# first, the per-channel weights last; "operators_reverse" for a bidirectional layer.
# ------------------------------------------------------------------------------------

# JSON operator name -> grid of the rxmet_gru_qparams struct
_JSON_GRID = {"input": "x", "output": "h", "weight_ih_linear": "weight_ih_linear",
              "weight_hh_linear": "weight_hh_linear", "update_gate_input": "update_gate_input",
              "update_gate_output": "update_gate_output", "reset_gate_input": "reset_gate_input",
              "reset_gate_output": "reset_gate_output", "new_gate_input": "new_gate_input",
              "new_gate_output": "new_gate_output", "mul_reset_hidden": "mul_reset_hidden",
              "mul_old_contribution": "mul_old_contribution",
              "mul_new_contribution": "mul_new_contribution"}
_JSON_CHAN = {"weight_ih": "W", "weight_hh": "R", "bias_ih": "bw", "bias_hh": "br"}
_ENC_TYPES = ("PER_TENSOR", "PER_GATE", "PER_CHANNEL")


def _one_or_list(values):
    """quant_gru.py:4032-4036: one value as a scalar, several as a list."""
    return values[0] if len(values) == 1 else values


def _operators_to_json(cfg, qp: "gru_ops.GRUQuantParams") -> dict:
    """One direction's operators dict (quant_gru.py:4111-4198)."""
    per_tensor, per_channel = {}, {}
    for name, info in _OPERATOR_MAP.items():
        bits = int(getattr(cfg, info["bw_attr"]))
        unsigned = bool(getattr(cfg, info["unsigned_attr"]))
        qmin, qmax = get_quant_range(bits, unsigned)
        if name in _JSON_CHAN:
            scales = [float(v) for v in qp.channel_scales(_JSON_CHAN[name])]
            enc = _ENC_TYPES[int(getattr(cfg, info["bw_attr"] + "granularity_"))]
            zps = [0] * len(scales)
        else:
            scales = [float(qp.scale(_JSON_GRID[name]))]
            enc = "PER_TENSOR"
            zps = [int(qp.zero_point(_JSON_GRID[name]))]
        op = {"dtype": f"{'UINT' if unsigned else 'INT'}{bits}",
              "symmetric": bool(getattr(cfg, info["sym_attr"])),
              "scale": _one_or_list(scales), "zero_point": _one_or_list(zps), "enc_type": enc,
              "real_min": _one_or_list([sc * (qmin - z) for sc, z in zip(scales, zps)]),
              "real_max": _one_or_list([sc * (qmax - z) for sc, z in zip(scales, zps)])}
        (per_channel if enc != "PER_TENSOR" else per_tensor)[name] = op
    per_tensor.update(per_channel)
    return per_tensor


def _operators_from_json(ops: dict, cfg, hidden: int) -> "gru_ops.GRUQuantParams":
    """Parse one direction's operators dict into cfg and new grids (quant_gru.py:4230-4434).
    Per-channel scales may be given per channel (3H values), per gate (3) or per tensor (1)."""
    qp = gru_ops.GRUQuantParams(hidden)
    C = 3 * hidden
    for name, op in ops.items():
        if name not in _OPERATOR_MAP:
            raise ValueError(f"unknown operator {name!r} in the quant params document")
        info = _OPERATOR_MAP[name]
        if "dtype" in op:
            dtype = str(op["dtype"]).upper()
            digits = "".join(ch for ch in dtype if ch.isdigit())
            setattr(cfg, info["bw_attr"], int(digits) if digits else 8)
            setattr(cfg, info["unsigned_attr"], dtype.startswith("UINT"))
        if "symmetric" in op:
            setattr(cfg, info["sym_attr"], bool(op["symmetric"]))
        if "scale" not in op:
            raise ValueError(f"operator {name!r} has no scale")
        scales = op["scale"] if isinstance(op["scale"], list) else [op["scale"]]
        scales = [float(v) for v in scales]
        if not scales or any(not (v > 0.0) or not math.isfinite(v) for v in scales):
            raise ValueError(f"operator {name!r}: scales must be positive and finite")
        bits = int(getattr(cfg, info["bw_attr"]))
        unsigned = bool(getattr(cfg, info["unsigned_attr"]))
        if name in _JSON_CHAN:
            enc = op.get("enc_type", "PER_CHANNEL")
            if enc not in _ENC_TYPES:
                raise ValueError(f"operator {name!r}: unknown enc_type {enc!r}")
            setattr(cfg, info["bw_attr"] + "granularity_", _ENC_TYPES.index(enc))
            if len(scales) == 1:
                full = scales * C
            elif len(scales) == 3:
                full = [scales[c // hidden] for c in range(C)]
            elif len(scales) == C:
                full = scales
            else:
                raise ValueError(f"operator {name!r}: {len(scales)} scales for {C} channels")
            k = A.CHAN[_JSON_CHAN[name]]
            qp.struct.chan_bits[k] = bits
            qp.struct.chan_unsigned[k] = int(unsigned)
            A.qparams_chan(qp.struct, k)[:] = np.asarray(full, dtype=np.float32)
        else:
            zp = op.get("zero_point", 0)
            zp = zp[0] if isinstance(zp, list) else zp
            g = qp.struct.g[A.GRID[_JSON_GRID[name]]]
            g.scale, g.zero_point, g.bits, g.is_unsigned = scales[0], int(zp), bits, int(unsigned)
    qp.struct.use_pot2 = int(bool(cfg.usePOT2_))
    qp.bitwidth_config_ = cfg
    return qp


# ------------------------------------------------------------------------------------
# AIMET encodings (quant_gru.py:2593-3592): the operators dict above rewritten into an
# AIMET encodings dictionary — activation_encodings[module] {input, output, internal_ops
# (+ internal_ops_reverse)}, param_encodings[module.weight_ih.weight / .weight_hh.weight /
# .bias] (the reverse direction appended to every list; the bias as [bias_ih, bias_hh] per
# direction) — and back.
# ------------------------------------------------------------------------------------

# the 13 internal-op slots of the skeleton, in its key order
_AIMET_SLOTS = ("add_final_hidden", "mul_new_contribution", "mul_old_contribution",
                "mul_reset_hidden", "new_gate_input", "new_gate_output", "reset_gate_input",
                "reset_gate_output", "sub_one_minus_update", "update_gate_input",
                "update_gate_output", "weight_ih_linear", "weight_hh_linear")
# the 11 operators stored under their own name, in export order
_AIMET_OWN = ("weight_ih_linear", "weight_hh_linear", "update_gate_input", "update_gate_output",
              "reset_gate_input", "reset_gate_output", "new_gate_input", "new_gate_output",
              "mul_reset_hidden", "mul_old_contribution", "mul_new_contribution")
# slots that carry another operator's encoding
_AIMET_ALIAS = {"add_final_hidden": "output", "sub_one_minus_update": "update_gate_output"}
_AIMET_LIST_FIELDS = ("scale", "zero_point", "real_min", "real_max")
_AIMET_DROP = ("multiplier", "shift", "scale_encoding", "n", "exp2_inv")


def _encoding_n(scale):
    """round(-log2(scale)) per scale (quant_gru.py:4039-4046)."""
    if isinstance(scale, list):
        if not scale:
            raise ValueError("Encoding scale cannot be empty")
        return [_encoding_n(v) for v in scale]
    if isinstance(scale, bool) or not isinstance(scale, (int, float)) or \
            not math.isfinite(scale) or scale <= 0:
        raise ValueError("Encoding scale must be positive and finite")
    return int(round(-math.log2(scale)))


def _validate_encoding_n(value) -> None:
    """Every encoding that states n must state the n of its scale (quant_gru.py:4049-4065)."""
    if isinstance(value, list):
        for v in value:
            _validate_encoding_n(v)
        return
    if not isinstance(value, dict):
        return
    if "scale" not in value:
        for v in value.values():
            _validate_encoding_n(v)
        return
    if "n" not in value:
        return

    def same(a, e):
        if isinstance(e, list):
            return isinstance(a, list) and len(a) == len(e) and all(map(same, a, e))
        return type(a) is int and a == e

    if not same(value["n"], _encoding_n(value["scale"])):
        raise ValueError("Encoding n does not match scale")


def _aimet_zero_points(op: dict) -> dict:
    """A list of scales gets a zero point per scale (quant_gru.py:2593-2626)."""
    if not isinstance(op, dict) or not isinstance(op.get("scale"), list):
        return op
    n = len(op["scale"])
    zp = op.get("zero_point", 0)
    if not isinstance(zp, list):
        op["zero_point"] = [zp] * n
    elif len(zp) == 1:
        op["zero_point"] = zp * n
    elif not zp:
        op["zero_point"] = [0] * n
    elif len(zp) != n:
        raise ValueError(f"zero_point length mismatch: expected {n}, got {len(zp)}")
    return op


def _aimet_encoding(op: dict) -> dict:
    """One operator as an AIMET encoding (quant_gru.py:2628-2672): bitwidth from dtype,
    is_symmetric as "True"/"False", execution fields dropped, n derived from the scale."""
    if not isinstance(op, dict):
        return op
    enc = copy.deepcopy(op)
    m = re.fullmatch(r"U?INT([1-9][0-9]*)", str(enc.get("dtype", "")))
    if m:
        enc["bitwidth"] = int(m.group(1))
    if "symmetric" in enc:
        enc["is_symmetric"] = "True" if enc.pop("symmetric") else "False"
    if isinstance(enc.get("is_symmetric"), bool):
        enc["is_symmetric"] = "True" if enc["is_symmetric"] else "False"
    for key in _AIMET_DROP:
        enc.pop(key, None)
    if "scale" in enc:
        enc["n"] = _encoding_n(enc["scale"])
    return enc


def _append_fields(dst: Optional[dict], src: Optional[dict], fields=_AIMET_LIST_FIELDS):
    """dst's list fields followed by src's (scalars become lists)."""
    if dst is None:
        return copy.deepcopy(src)
    if src is None:
        return dst
    for f in fields:
        if f not in src:
            continue
        if f not in dst:
            dst[f] = copy.deepcopy(src[f])
            continue
        a, b = dst[f], src[f]
        dst[f] = (a if isinstance(a, list) else [a]) + (list(b) if isinstance(b, list) else [b])
    return dst


def _aimet_skeleton() -> dict:
    return {slot: {"output": []} for slot in _AIMET_SLOTS}


def _aimet_fill_internal(slots: dict, ops: dict) -> None:
    for name in _AIMET_OWN + tuple(_AIMET_ALIAS):
        src = ops.get(_AIMET_ALIAS.get(name, name))
        if src is None:
            continue
        enc = _aimet_encoding(_aimet_zero_points(copy.deepcopy(src)))
        if isinstance(slots.get(name), dict) and "output" in slots[name]:
            slots[name]["output"] = [enc]
        else:
            slots[name] = enc


def _aimet_first(entry):
    """An encoding stored as {"0": enc}, [enc, ...], {"output": [enc]} or enc itself."""
    if isinstance(entry, dict) and "output" in entry:
        out = entry["output"]
        return out[0] if isinstance(out, list) and out else (out if isinstance(out, dict) else None)
    if isinstance(entry, dict) and "0" in entry:
        return entry["0"]
    if isinstance(entry, list):
        return entry[0] if entry else None
    return entry if isinstance(entry, dict) else None


def _aimet_split(op: dict, parts: int) -> list:
    """Cut every list field of an encoding into `parts` equal pieces (scalars repeated)."""
    out = [copy.deepcopy(op) for _ in range(parts)]
    for f in ("scale", "multiplier", "shift", "real_min", "real_max", "zero_point"):
        v = op.get(f)
        if isinstance(v, list):
            n = len(v) // parts
            for k in range(parts):
                out[k][f] = v[k * n:(k + 1) * n] if k < parts - 1 else v[k * n:]
    return out


# ------------------------------------------------------------------------------------
# GRUFunction (quant_gru.py:807-1102)
# ------------------------------------------------------------------------------------


# Training forwards of the module keep their saved state as codes (gru_ops.
# forward_quant_codes_dirs: v as 16-bit codes, the 13 per-step masks as bits) rather than in
# the reference's float / byte format, which only the gru_ops entry points hand out; the
# gradients are the same bit for bit.  False: the reference format throughout.
SAVE_STATE_AS_CODES = True


def _codes_fit(quant_params) -> bool:
    """The saved codes hold grids of at most 16 bits (gate outputs and weight_hh_linear)."""
    g = quant_params.struct.g
    return all(int(g[A.GRID[n]].bits) <= 16 for n in ("update_gate_output", "reset_gate_output",
                                                       "new_gate_output", "weight_hh_linear"))


class GRUFunction(torch.autograd.Function):
    """One direction of a quantised GRU.  forward: weight reorder -> forward_quant_float_storage
    (or forward_quant_int_storage for quant_storage_dtype='int32'; inference on the FP32
    carrier and training with the state saved as codes read PyTorch's weight layout in the
    library instead); backward: dh_new [T+1,B,H]
    (dh_new[0]=0, dh_new[1:]=grad_output, grad_h_n added to the last step) ->
    backward_quant_float_storage (backward_quant_int_storage) -> gradients reordered back to
    (r, z, n)."""

    @staticmethod
    def forward(ctx, input, weight_ih, weight_hh, bias_ih, bias_hh, h0, is_training,
                use_quantization=False, quant_params=None, quant_storage_dtype="float32"):
        T, B, I = input.shape
        H = weight_hh.shape[1]
        ctx.dims = (T, B, I, H)
        ctx.use_quantization = bool(use_quantization)
        if not use_quantization:
            device = _require_device(input)
            W, R, bw, br = convert_weights_to_haste_format(weight_ih, weight_hh, bias_ih, bias_hh,
                                                           H, device)
            h0_t = ensure_cuda_float32(h0, device).contiguous() if h0 is not None else None
            h_full, _ = gru_ops.forward_fp(False, T, B, I, H, W, R, bw, br,
                                           ensure_cuda_float32(input, device).contiguous(), h0_t)
            return h_full[1:], h_full[-1:]
        if quant_params is None:
            raise RuntimeError("quant_params is required when use_quantization=True")
        if quant_storage_dtype not in ("float32", "int32"):
            raise ValueError(f"quant_storage_dtype must be 'float32' or 'int32', got "
                             f"{quant_storage_dtype}")
        device = _require_device(input)
        # inference on the FP32 carrier reads the weights as they are too (no reorder kernels),
        # and x in place when its feature stride is 1 (a batch-first caller's transposed view)
        eval_torch_w = (not is_training and quant_storage_dtype == "float32"
                        and H % 16 == 0)
        input = ensure_cuda_float32(input, device)
        if not (eval_torch_w and input.stride(2) == 1):
            input = input.contiguous()
        h0_t = (ensure_cuda_float32(h0, device).contiguous() if h0 is not None
                else torch.empty(0, device=device, dtype=torch.float32))
        ctx.codes = bool(is_training and quant_storage_dtype == "float32" and H % 16 == 0
                         and SAVE_STATE_AS_CODES and _codes_fit(quant_params))
        if ctx.codes or eval_torch_w:
            # weights read in PyTorch's layout by the library; in training the state saved as codes
            W = ensure_cuda_float32(weight_ih, device).contiguous()
            R = ensure_cuda_float32(weight_hh, device).contiguous()
            if bias_ih is not None and bias_hh is not None:
                bw = ensure_cuda_float32(bias_ih, device).contiguous()
                br = ensure_cuda_float32(bias_hh, device).contiguous()
            else:
                bw = br = _zeros(3 * H, device)
            fwd = (gru_ops.forward_quant_codes_dirs if ctx.codes
                   else gru_ops.forward_quant_float_storage_dirs_x)
            outs = fwd(bool(is_training), T, B, I, H, [(W, R, bw, br, input, h0_t, quant_params)],
                       [(input.stride(0), input.stride(1), 0, 1)])[0]
        else:
            W, R, bw, br = convert_weights_to_haste_format(weight_ih, weight_hh, bias_ih, bias_hh,
                                                           H, device)
            # float32: codes stored as fp32 (FP32 carrier); int32: the int32 carrier
            forward_fn = (gru_ops.forward_quant_int_storage if quant_storage_dtype == "int32"
                          else gru_ops.forward_quant_float_storage)
            outs = forward_fn(
                is_training=is_training, time_steps=T, batch_size=B, input_size=I, hidden_size=H,
                W=W, R=R, bw=bw, br=br, x=input, h0=h0_t, quant_params=quant_params)
        h_full = outs[0]
        ctx.quant_storage_dtype = quant_storage_dtype
        ctx.bias_none = (bias_ih is None, bias_hh is None)
        ctx.h0_is_none = h0 is None
        ctx.quant_params = quant_params
        ctx.saved_state = bool(is_training)
        if is_training:
            # (W_q, R_q, bw_q, br_q, x_q, h, v, 11 masks) as the backward consumes them, or
            # (.., h, v_codes, 6 masks, mask_bits)
            ctx.save_for_backward(outs[2], outs[3], outs[4], outs[5], outs[6], h_full, outs[1],
                                  *outs[7:])
        return h_full[1:], h_full[-1:]

    @staticmethod
    def backward(ctx, grad_output, grad_h_n):
        if not ctx.use_quantization:
            raise NotImplementedError("the float GRU backward (use_quantization=False training) "
                                      "is not provided by the MI355X build")
        if not ctx.saved_state:
            raise RuntimeError("QuantGRU forward ran without saving backward state (no_grad "
                               "eval); rerun it with gradients enabled")
        T, B, I, H = ctx.dims
        saved = ctx.saved_tensors
        W_q, R_q, bw_q, br_q, x_q, h, v = saved[:7]
        masks = saved[7:]
        if ctx.codes:
            # dh read in place from grad_output / grad_h_n (no dh_new buffer)
            views, _keep = gru_ops.grad_views(grad_output, grad_h_n, T, B, H, False, 1)
            dx, dW, dR, dbw, dbr, dh = gru_ops.backward_quant_codes_dirs(
                T, B, I, H, [(W_q, R_q, bw_q, br_q, x_q, None, h, v, ctx.quant_params,
                              masks)], views=views)[0]
            return (dx, dW, dR, None if ctx.bias_none[0] else dbw,
                    None if ctx.bias_none[1] else dbr, None if ctx.h0_is_none else dh,
                    None, None, None, None)
        dh_new = torch.zeros((T + 1, B, H), device=h.device, dtype=torch.float32)
        if grad_output is not None:
            dh_new[1:] = grad_output
        if grad_h_n is not None and grad_h_n.numel() > 0:
            dh_new[-1] += grad_h_n[0]
        backward_fn = (gru_ops.backward_quant_int_storage if ctx.quant_storage_dtype == "int32"
                       else gru_ops.backward_quant_float_storage)
        dx, dW, dR, dbw, dbr, dh = backward_fn(
            time_steps=T, batch_size=B, input_size=I, hidden_size=H, W_q=W_q, R_q=R_q,
            bw_q=bw_q, br_q=br_q, x_q=x_q, dh_new=dh_new, h=h, v=v,
            quant_params=ctx.quant_params, **dict(zip(gru_ops.MASK_NAMES, masks)))
        dW_pt = reorder_weights_haste_to_pytorch(dW.t())
        dR_pt = reorder_weights_haste_to_pytorch(dR.t())
        dbw_pt = None if ctx.bias_none[0] else reorder_weights_haste_to_pytorch(dbw)
        dbr_pt = None if ctx.bias_none[1] else reorder_weights_haste_to_pytorch(dbr)
        dh0 = None if ctx.h0_is_none else dh
        return dx, dW_pt, dR_pt, dbw_pt, dbr_pt, dh0, None, None, None, None


class GRUBidirectionalFunction(torch.autograd.Function):
    """Both directions of a quantised bidirectional GRU, equal to two GRUFunction applications
    on (input, input.flip(0)) followed by the output concatenation (quant_gru.py:2270-2288,
    1402-1432), with the layout work done by the library instead of tensor copies: each
    direction reads its x in place from the caller's input (batch-first or not, the reverse
    direction time-reversed), one kernel assembles output and h_n in the caller's layout, and
    the backward splits the output gradient and assembles dx the same way.  Each direction
    pair of recurrences is one launch (forward_quant_float_storage_dirs_x /
    backward_quant_float_storage_dirs), so the two directions' sequential steps overlap.
    Returns (output, h_n)."""

    @staticmethod
    def forward(ctx, input, wi_f, wh_f, bi_f, bh_f, h0_f, wi_r, wh_r, bi_r, bh_r, h0_r, is_training,
                qp_f, qp_r, batch_first):
        device = _require_device(input)
        x = ensure_cuda_float32(input, device)
        if x.stride(2) != 1:
            x = x.contiguous()
        if batch_first:
            B, T, I = x.shape
            st, sb = x.stride(1), x.stride(0)
        else:
            T, B, I = x.shape
            st, sb = x.stride(0), x.stride(1)
        H = wh_f.shape[1]
        ctx.dims = (T, B, I, H)
        ctx.batch_first = bool(batch_first)
        dirs = []
        for (wi, wh, bi, bh, h0, qp) in ((wi_f, wh_f, bi_f, bh_f, h0_f, qp_f),
                                         (wi_r, wh_r, bi_r, bh_r, h0_r, qp_r)):
            # weights in PyTorch's layout and gate order: the library reads them as they are
            W = ensure_cuda_float32(wi, device).contiguous()
            R = ensure_cuda_float32(wh, device).contiguous()
            if bi is not None and bh is not None:
                bw = ensure_cuda_float32(bi, device).contiguous()
                br = ensure_cuda_float32(bh, device).contiguous()
            else:
                bw = br = _zeros(3 * H, device)
            h0_t = (ensure_cuda_float32(h0, device).contiguous() if h0 is not None
                    else torch.empty(0, device=device, dtype=torch.float32))
            dirs.append((W, R, bw, br, x, h0_t, qp))
        ctx.codes = bool(is_training and SAVE_STATE_AS_CODES and _codes_fit(qp_f)
                         and _codes_fit(qp_r))
        fwd = (gru_ops.forward_quant_codes_dirs if ctx.codes
               else gru_ops.forward_quant_float_storage_dirs_x)
        outs = fwd(is_training, T, B, I, H, dirs, [(st, sb, 0, 1), (st, sb, 1, 1)])
        ctx.bias_none = (bi_f is None, bh_f is None)
        ctx.h0_none = (h0_f is None, h0_r is None)
        ctx.quant_params = (qp_f, qp_r)
        ctx.saved_state = bool(is_training)
        if is_training:
            saved = []
            for o in outs:
                saved += [o[2], o[3], o[4], o[5], o[6], o[0], o[1], *o[7:]]
            ctx.save_for_backward(*saved)
        return gru_ops.bidir_assemble(outs[0][0], outs[1][0], ctx.batch_first)

    @staticmethod
    def backward(ctx, g_out, g_hn):
        if not ctx.saved_state:
            raise RuntimeError("QuantGRU forward ran without saving backward state (no_grad "
                               "eval); rerun it with gradients enabled")
        T, B, I, H = ctx.dims
        saved = ctx.saved_tensors
        n = len(saved) // 2
        if ctx.codes:
            # each direction reads its dh in place from g_out / g_hn (no split copies)
            views, _keep = gru_ops.grad_views(g_out, g_hn, T, B, H, ctx.batch_first, 2)
            dhs = (None, None)
        else:
            views = None
            dh_f, dh_r, _ = gru_ops.bidir_split_grad(g_out, g_hn, T, B, H, ctx.batch_first,
                                                     saved[5].device)
            dhs = (dh_f, dh_r)
        dirs = []
        for k, dh_new in enumerate(dhs):
            W_q, R_q, bw_q, br_q, x_q, h, v = saved[k * n:k * n + 7]
            masks = saved[k * n + 7:(k + 1) * n]
            dirs.append((W_q, R_q, bw_q, br_q, x_q, dh_new, h, v, ctx.quant_params[k], masks))
        # weight gradients come back in PyTorch's layout and gate order
        res = (gru_ops.backward_quant_codes_dirs(T, B, I, H, dirs, views=views) if ctx.codes
               else gru_ops.backward_quant_float_storage_dirs_x(T, B, I, H, dirs))
        grads = []
        for k, (dx, dW, dR, dbw, dbr, dh) in enumerate(res):
            grads.append((dW, dR, None if ctx.bias_none[0] else dbw,
                          None if ctx.bias_none[1] else dbr, None if ctx.h0_none[k] else dh))
        dx = gru_ops.bidir_dx(res[0][0], res[1][0], ctx.batch_first)
        return (dx, *grads[0], *grads[1], None, None, None, None)


# ------------------------------------------------------------------------------------
# QuantGRU (quant_gru.py:1120-2306)
# ------------------------------------------------------------------------------------


class QuantGRU(nn.Module):
    """nn.GRU-compatible quantisation-aware GRU (single layer, optional bidirectional).

    Workflow as in the reference: ``calibrating=True`` + forward collects MinMax ranges
    (on the GPU), ``use_quantization=True`` turns on fake-quantised execution; grids are
    derived lazily (dirty flag) on the next quantised forward or by ``finalize_calibration``.
    """

    owns_quantization = True

    def __init__(self, input_size: int, hidden_size: int, num_layers: int = 1, bias: bool = True,
                 batch_first: bool = False, dropout: float = 0.0, bidirectional: bool = False,
                 use_quantization: bool = False, use_po2_scale: Optional[bool] = None,
                 quant_storage_dtype: str = "float32", *, use_pot2_scale: Optional[bool] = None):
        super().__init__()
        if num_layers != 1:
            raise NotImplementedError("only num_layers=1 is supported")
        if dropout > 0:
            raise NotImplementedError("dropout is not supported")
        if quant_storage_dtype not in ("float32", "int32"):
            raise ValueError("quant_storage_dtype must be 'float32' or 'int32', got "
                             f"{quant_storage_dtype}")
        if (use_po2_scale is not None and use_pot2_scale is not None
                and bool(use_po2_scale) != bool(use_pot2_scale)):
            raise ValueError("use_po2_scale and use_pot2_scale conflict")
        self.input_size = input_size
        self.hidden_size = hidden_size
        self.num_layers = num_layers
        self.bias = bias
        self.batch_first = batch_first
        self.dropout = dropout
        self.bidirectional = bidirectional
        self.use_quantization = use_quantization
        self.num_directions = 2 if bidirectional else 1
        self.quant_storage_dtype = quant_storage_dtype
        self.export_mode = False
        self._use_pot2_scale = bool(use_po2_scale if use_po2_scale is not None
                                    else use_pot2_scale)

        g3 = 3 * hidden_size
        for sfx in ("", "_reverse") if bidirectional else ("",):
            setattr(self, "weight_ih_l0" + sfx, nn.Parameter(torch.empty(g3, input_size)))
            setattr(self, "weight_hh_l0" + sfx, nn.Parameter(torch.empty(g3, hidden_size)))
            if bias:
                setattr(self, "bias_ih_l0" + sfx, nn.Parameter(torch.empty(g3)))
                setattr(self, "bias_hh_l0" + sfx, nn.Parameter(torch.empty(g3)))
            else:
                self.register_parameter("bias_ih_l0" + sfx, None)
                self.register_parameter("bias_hh_l0" + sfx, None)
        self.reset_parameters()

        self.quant_ranges = None
        self.quant_params = None
        if bidirectional:
            self.quant_ranges_reverse = None
            self.quant_params_reverse = None
        self._quant_params_dirty = False
        self._quant_params_locked = False
        self._bitwidth_config = gru_ops.OperatorQuantConfig()
        self._bitwidth_config.usePOT2_ = self._use_pot2_scale
        self._module_name = None
        self.calibration_method = "minmax"
        self.percentile_value = 100.0
        self.hist_collectors = None
        if bidirectional:
            self.hist_collectors_reverse = None
        self.calibrating = False

    # -- pickling (quant_gru.py:1277-1350): bit-width config kept, calibration dropped ----

    def __getstate__(self):
        state = self.__dict__.copy()
        cfg = {}
        for info in _OPERATOR_MAP.values():
            for a in (info["bw_attr"], info["sym_attr"], info["unsigned_attr"]):
                cfg[a] = getattr(self._bitwidth_config, a)
        for a in ("W_granularity_", "R_granularity_", "bw_granularity_", "br_granularity_",
                  "usePOT2_", "pot_scale_method_", "pot_scale_tolerance_"):
            cfg[a] = getattr(self._bitwidth_config, a)
        state["_bitwidth_config"] = cfg
        for k in ("quant_ranges", "quant_params", "hist_collectors"):
            state[k] = None
            if self.bidirectional:
                state[k + "_reverse"] = None
        state["_quant_params_dirty"] = False
        return state

    def __setstate__(self, state):
        cfg = state.get("_bitwidth_config")
        obj = gru_ops.OperatorQuantConfig()
        if isinstance(cfg, dict):
            for a, v in cfg.items():
                setattr(obj, a, v)
        state["_bitwidth_config"] = obj
        state.setdefault("_quant_params_locked", False)
        state.setdefault("quant_storage_dtype", "float32")
        self.__dict__.update(state)
        self._use_pot2_scale = bool(obj.usePOT2_)

    def reset_parameters(self):
        """U(-1/sqrt(H), 1/sqrt(H)) for every parameter, as nn.GRU (quant_gru.py:1352-1356)."""
        stdv = 1.0 / (self.hidden_size ** 0.5)
        for p in self.parameters():
            nn.init.uniform_(p, -stdv, stdv)

    # -- configuration ---------------------------------------------------------------

    def set_all_bitwidth(self, bitwidth: int = 8, is_symmetric: bool = True,
                         verbose: bool = False):
        """One bit width for every operator; weights/biases stay symmetric, activations
        follow ``is_symmetric`` (quant_gru.py:1628-1658)."""
        if not 1 <= bitwidth <= 32:
            raise ValueError(f"bitwidth must be in range [1, 32], got {bitwidth}")
        for a in _VALID_BITWIDTH_ATTRS:
            setattr(self._bitwidth_config, a, bitwidth)
        for a in _WEIGHT_SYMMETRIC_ATTRS:
            setattr(self._bitwidth_config, a, True)
        for a in _ACTIVATION_SYMMETRIC_ATTRS:
            setattr(self._bitwidth_config, a, is_symmetric)
        self._quant_params_dirty = True
        if verbose:
            print(f"[QuantGRU] all operators {bitwidth}-bit, activations "
                  f"{'symmetric' if is_symmetric else 'asymmetric'}, weights symmetric")

    def _get_config_attr(self, op_name: str, suffix: str, valid: set, default):
        attr = f"{op_name}{suffix}"
        if attr not in valid:
            import warnings
            warnings.warn(f"unknown config attribute '{attr}', returning {default}", UserWarning)
            return default
        return getattr(self._bitwidth_config, attr, default)

    def _get_bitwidth(self, op_name: str) -> int:
        return self._get_config_attr(op_name, "_", _VALID_BITWIDTH_ATTRS, 8)

    def _get_symmetric(self, op_name: str) -> bool:
        return self._get_config_attr(op_name, "_symmetric_", _VALID_SYMMETRIC_ATTRS, True)

    def _get_unsigned(self, op_name: str) -> bool:
        return self._get_config_attr(op_name, "_unsigned_", _VALID_UNSIGNED_ATTRS, False)

    @property
    def use_po2_scale(self) -> bool:
        return bool(self._bitwidth_config.usePOT2_)

    @use_po2_scale.setter
    def use_po2_scale(self, value: bool):
        self._use_pot2_scale = bool(value)
        self._bitwidth_config.usePOT2_ = self._use_pot2_scale
        if self.quant_params is not None:
            self.quant_params.bitwidth_config_ = self._bitwidth_config
        self._quant_params_dirty = True

    use_pot2_scale = use_po2_scale

    def enable_po2(self, method="cover_range", tolerance=0.02):
        """quant_gru.py:1679-1685."""
        if self.use_po2_scale:
            return
        if self._quant_params_locked:
            raise RuntimeError("QuantGRU encodings are locked; cannot change scale mode")
        self.use_po2_scale = True

    def enable_pot2(self, method="cover_range", tolerance=0.02):
        return self.enable_po2(method=method, tolerance=tolerance)

    def set_module_name(self, module_name: str) -> None:
        self._module_name = module_name

    # -- quant-params document (quant_gru.py:2548-2592, 4475-4526, 4581-4680) ----------

    def export_quant_params(self, export_path: str, include_weights: bool = False,
                            verbose: bool = False) -> None:
        """Write the grids of each direction as the reference's JSON document."""
        if not self.is_calibrated() and not (self._quant_params_dirty and
                                             self.quant_ranges is not None):
            raise RuntimeError("calibrate first: gru.calibrating = True; gru(data); "
                               "gru.calibrating = False; gru.finalize_calibration()")
        self._ensure_quant_params_fresh()
        doc = {"model_info": {"input_size": self.input_size, "hidden_size": self.hidden_size,
                              "bias": self.bias, "batch_first": self.batch_first,
                              "bidirectional": self.bidirectional,
                              "use_pot2_scale": bool(self.use_po2_scale)},
               "operators": _operators_to_json(self._bitwidth_config, self.quant_params)}
        if self.bidirectional and self.quant_params_reverse is not None:
            doc["operators_reverse"] = _operators_to_json(self._bitwidth_config,
                                                          self.quant_params_reverse)
        if include_weights:
            doc["quantized_weights"] = self._quantized_weights_json()
        with open(export_path, "w", encoding="utf-8") as f:
            json.dump(doc, f, indent=2, ensure_ascii=False)
        if verbose:
            print(f"[QuantGRU] quant params written to {export_path}")

    def _quantized_weights_json(self) -> dict:
        """Integer weight codes in kernel layout (quant_gru.py:4527-4580)."""
        qp = self.quant_params
        W, R, bw, br = convert_weights_to_haste_format(
            self.weight_ih_l0, self.weight_hh_l0, self.bias_ih_l0 if self.bias else None,
            self.bias_hh_l0 if self.bias else None, self.hidden_size, self.weight_ih_l0.device)
        cfg = self._bitwidth_config

        def codes(t, name, bits):
            s = torch.from_numpy(np.array(qp.channel_scales(name), dtype=np.float32)).to(t.device)
            lo, hi = get_quant_range(bits)
            return torch.clamp(torch.round(t.detach() / s), lo, hi).to(torch.int32).tolist()

        out = {"W": codes(W, "W", cfg.W_), "R": codes(R, "R", cfg.R_)}
        if self.bias:
            out["bw"] = codes(bw, "bw", cfg.bw_)
            out["br"] = codes(br, "br", cfg.br_)
        return out

    def load_quant_params(self, import_path: str, verbose: bool = False) -> None:
        """Read a quant-params document; the module is calibrated afterwards."""
        with open(import_path, "r", encoding="utf-8") as f:
            doc = json.load(f)
        info = doc.get("model_info", {})
        for key, mine in (("input_size", self.input_size), ("hidden_size", self.hidden_size),
                          ("bidirectional", self.bidirectional)):
            if info.get(key, False if key == "bidirectional" else None) != mine:
                raise ValueError(f"{key} mismatch: document has {info.get(key)}, module has {mine}")
        if "operators" not in doc:
            raise ValueError(f"not a quant params document (no 'operators'; keys {list(doc)})")
        if self.bidirectional and "operators_reverse" not in doc:
            raise ValueError("bidirectional=True needs 'operators_reverse' in the document")
        cfg = gru_ops.OperatorQuantConfig()
        cfg.usePOT2_ = bool(info.get("use_pot2_scale", False))
        qp = _operators_from_json(doc["operators"], cfg, self.hidden_size)
        qpr = None
        if self.bidirectional:
            qpr = _operators_from_json(doc["operators_reverse"], cfg, self.hidden_size)
            fin, rin = doc["operators"].get("input", {}), doc["operators_reverse"].get("input", {})
            if fin.get("zero_point") != rin.get("zero_point"):
                raise ValueError("operators.input and operators_reverse.input disagree")
        self._bitwidth_config = cfg
        self._use_pot2_scale = bool(cfg.usePOT2_)
        self.quant_params = qp
        if self.bidirectional:
            self.quant_params_reverse = qpr
        self._quant_params_dirty = False
        if verbose:
            print(f"[QuantGRU] quant params loaded from {import_path}")

    # -- AIMET encodings (quant_gru.py:2674-3592) --------------------------------------

    def export_quant_params_to_aimet_format(self, encodings_dict: dict, module_name: str = None,
                                            verbose: bool = False, *,
                                            for_onnx: bool = True) -> dict:
        """Merge this layer's grids into an AIMET encodings dictionary and return it.  An
        uncalibrated layer is skipped (the dictionary comes back unchanged); a
        "tensor_encodings" entry is removed, as the reference does for older loaders."""
        if not self.is_calibrated():
            if verbose:
                print(f"[QuantGRU] {module_name or 'unknown'} is not calibrated; not exported")
            return encodings_dict
        self._ensure_quant_params_fresh()
        name = module_name or self._module_name or "gru"
        ops = _operators_to_json(self._bitwidth_config, self.quant_params)
        rev = None
        if self.bidirectional and self.quant_params_reverse is not None:
            rev = _operators_to_json(self._bitwidth_config, self.quant_params_reverse)
        encodings_dict.setdefault("schema_version", 3)
        acts = encodings_dict.setdefault("activation_encodings", {})
        if name not in acts:
            acts[name] = {"is_GRU": True, "input": {}, "output": {},
                          "internal_ops": _aimet_skeleton()}
            if self.bidirectional:
                acts[name]["internal_ops_reverse"] = _aimet_skeleton()
        params = encodings_dict.setdefault("param_encodings", {})
        encodings_dict.setdefault("tensor_encodings", {})
        layer = acts[name]
        if self.bidirectional and "internal_ops_reverse" not in layer:
            layer["internal_ops_reverse"] = _aimet_skeleton()

        def enc(op):
            return _aimet_encoding(_aimet_zero_points(copy.deepcopy(op)))

        layer["input"] = {"0": enc(ops["input"])}
        layer["output"] = {"0": enc(ops["output"])}
        for key, op in (("weight_ih.weight", "weight_ih"), ("weight_hh.weight", "weight_hh")):
            data = _aimet_zero_points(copy.deepcopy(ops[op]))
            if rev is not None:
                data = _append_fields(data, _aimet_zero_points(copy.deepcopy(rev[op])))
            params[f"{name}.{key}"] = _aimet_encoding(data)
        for op in ("bias_ih", "bias_hh"):
            if op not in ops:
                raise ValueError(f"{name}.bias needs both bias_ih and bias_hh (missing {op})")
        bias = _aimet_zero_points(copy.deepcopy(ops["bias_ih"]))
        bias = _append_fields(bias, _aimet_zero_points(copy.deepcopy(ops["bias_hh"])))
        if rev is not None:
            for op in ("bias_ih", "bias_hh"):
                bias = _append_fields(bias, _aimet_zero_points(copy.deepcopy(rev[op])))
        params[f"{name}.bias"] = _aimet_encoding(bias)
        _aimet_fill_internal(layer["internal_ops"], ops)
        if rev is not None and "internal_ops_reverse" in layer:
            _aimet_fill_internal(layer["internal_ops_reverse"], rev)
        encodings_dict.pop("tensor_encodings", None)
        if verbose:
            print(f"[QuantGRU] {name} exported to AIMET encodings")
        return encodings_dict

    def load_quant_params_from_aimet_format(self, encodings_dict: dict, module_name: str = None,
                                            verbose: bool = False) -> bool:
        """Read this layer's grids from an AIMET encodings dictionary.  Returns False when the
        layer's entries are missing or do not parse; an n that contradicts its scale raises
        ValueError.  Scales that are all powers of two select the POT2 execution mode."""
        name = module_name or self._module_name or "gru"
        self._module_name = name

        def fail(msg):
            if verbose:
                print(f"[QuantGRU] {name}: {msg}")
            return False

        acts = encodings_dict.get("activation_encodings")
        if not isinstance(acts, dict):
            return fail("no activation_encodings")
        if name not in acts:
            return fail("no activation_encodings entry for this module")
        layer = acts[name]
        _validate_encoding_n(layer)
        params = encodings_dict.get("param_encodings", {})
        for suffix in ("weight_ih.weight", "weight_hh.weight", "bias"):
            _validate_encoding_n(params.get(f"{name}.{suffix}"))
        if layer.get("is_GRU") is not True and verbose:
            print(f"[QuantGRU] {name}: is_GRU is not True")
        bidir = self.bidirectional
        ops, rev = {}, ({} if bidir else None)
        for key in ("input", "output"):
            if key not in layer or _aimet_first(layer[key]) is None:
                return fail(f"no {key!r} encoding")
            ops[key] = copy.deepcopy(_aimet_first(layer[key]))
        if bidir:
            rev["input"] = copy.deepcopy(ops["input"])  # both directions read one x
        if "param_encodings" in encodings_dict:
            for key, op in (("weight_ih.weight", "weight_ih"), ("weight_hh.weight", "weight_hh")):
                data = params.get(f"{name}.{key}")
                if data is None:
                    return fail(f"no param encoding {name}.{key}")
                if bidir:
                    ops[op], rev[op] = _aimet_split(data, 2)
                else:
                    ops[op] = copy.deepcopy(data)
            data = params.get(f"{name}.bias")
            if data is None:
                return fail(f"no param encoding {name}.bias")
            if bidir:
                n = next((len(data[f]) for f in _AIMET_LIST_FIELDS
                          if isinstance(data.get(f), list)), None)
                if n is None or n % 4:
                    return fail("cannot split the bias into two directions")
                ops["bias_ih"], ops["bias_hh"], rev["bias_ih"], rev["bias_hh"] = \
                    _aimet_split(data, 4)
            else:
                ops["bias_ih"], ops["bias_hh"] = _aimet_split(data, 2)
        elif verbose:
            print(f"[QuantGRU] {name}: no param_encodings")
        for slots_key, dst in (("internal_ops", ops), ("internal_ops_reverse", rev)):
            slots = layer.get(slots_key)
            if dst is None or not isinstance(slots, dict):
                continue
            for op in _AIMET_OWN:
                if op in slots and _aimet_first(slots[op]) is not None:
                    dst[op] = copy.deepcopy(_aimet_first(slots[op]))
            if dst is rev and "add_final_hidden" in slots:
                first = _aimet_first(slots["add_final_hidden"])
                if first is not None:
                    rev["output"] = copy.deepcopy(first)
        for d in (ops, rev):
            for op in (d or {}).values():
                if isinstance(op, dict) and "is_symmetric" in op:
                    v = op.pop("is_symmetric")
                    op["symmetric"] = v.lower() == "true" if isinstance(v, str) else bool(v)
        try:
            scales = []
            for d in (ops, rev):
                for op in (d or {}).values():
                    sc = op.get("scale", [])
                    scales.extend(sc if isinstance(sc, list) else [sc])
            pot2 = bool(scales) and all(
                isinstance(v, (int, float)) and v > 0 and math.isfinite(v)
                and math.frexp(v)[0] == 0.5 for v in scales)
            cfg = gru_ops.OperatorQuantConfig()
            cfg.usePOT2_ = pot2
            qp = _operators_from_json(ops, cfg, self.hidden_size)
            qpr = _operators_from_json(rev, cfg, self.hidden_size) if bidir and rev else None
        except (ValueError, KeyError, TypeError) as e:
            return fail(f"could not load the encodings: {e}")
        self._bitwidth_config = cfg
        self._use_pot2_scale = pot2
        self.quant_params = qp
        if bidir:
            self.quant_params_reverse = qpr
        self._quant_params_dirty = False
        if verbose:
            print(f"[QuantGRU] {name} loaded from AIMET encodings")
        return True

    # -- calibration state -------------------------------------------------------------

    def is_calibrated(self) -> bool:
        if self.bidirectional:
            return self.quant_params is not None and self.quant_params_reverse is not None
        return self.quant_params is not None

    def _use_histogram_collection(self) -> bool:
        return self.calibration_method in ("sqnr", "percentile")

    def _check_calibration_method(self):
        if self.calibration_method not in ("minmax", "sqnr", "percentile"):
            raise ValueError(f"unknown calibration_method {self.calibration_method!r}")
        if self._use_histogram_collection():
            raise NotImplementedError("histogram calibration ('sqnr', 'percentile') is not "
                                      "provided by the MI355X build; use 'minmax'")

    def _ensure_quant_params_fresh(self):
        """Resolve a pending dirty flag before locking (quant_gru.py:4436-4472)."""
        if not self._quant_params_dirty:
            return
        if self._quant_params_locked and self.quant_params is not None:
            self._quant_params_dirty = False
            return
        if self.quant_ranges is None:
            raise RuntimeError("quantisation parameters are stale and the calibration data is "
                               "gone: recalibrate or call finalize_calibration() first")
        self.finalize_calibration()

    def set_quant_params_locked(self, locked: bool) -> None:
        """quant_gru.py:1709-1721."""
        if locked and not self._quant_params_locked:
            self._ensure_quant_params_fresh()
        self._quant_params_locked = bool(locked)

    @contextmanager
    def calibration_context(self):
        """One PTQ pass: reset, collect, finalize, restore flags (quant_gru.py:1662-1677)."""
        if self._quant_params_locked or self.calibrating:
            yield
            return
        previous = self.calibrating
        self.reset_calibration()
        self.calibrating = True
        try:
            yield
            if self.quant_ranges is not None:
                self.finalize_calibration(verbose=False)
        finally:
            self.calibrating = previous

    def finalize_calibration(self, verbose: bool = False):
        """Ranges -> grids for each direction (quant_gru.py:1724-1800)."""
        if self._quant_params_locked and self.is_calibrated():
            self._quant_params_dirty = False
            return
        self._check_calibration_method()
        if self.quant_ranges is None:
            raise RuntimeError("no calibration data: set calibrating=True and call forward() first")
        cfg = self._bitwidth_config
        self.quant_params = gru_ops.calculate_gru_quantitative_parameters(
            quant_ranges=self.quant_ranges, bitwidth_config=cfg)
        if self.bidirectional:
            if self.quant_ranges_reverse is None:
                raise RuntimeError("bidirectional GRU: reverse-direction calibration data missing")
            self.quant_params_reverse = gru_ops.calculate_gru_quantitative_parameters(
                quant_ranges=self.quant_ranges_reverse, bitwidth_config=cfg)
        self._quant_params_dirty = False
        if verbose:
            print(f"[QuantGRU] MINMAX grids: x scale {self.quant_params.scale('x'):.6g}, "
                  f"h scale {self.quant_params.scale('h'):.6g}")

    def reset_calibration(self):
        """quant_gru.py:1802-1813."""
        self.quant_ranges = None
        self.quant_params = None
        self.hist_collectors = None
        self._quant_params_dirty = False
        if self.bidirectional:
            self.quant_ranges_reverse = None
            self.quant_params_reverse = None
            self.hist_collectors_reverse = None

    # -- forward -------------------------------------------------------------------------

    def _direction_weights(self, reverse: bool, device):
        sfx = "_reverse" if reverse else ""
        return convert_weights_to_haste_format(
            getattr(self, "weight_ih_l0" + sfx), getattr(self, "weight_hh_l0" + sfx),
            getattr(self, "bias_ih_l0" + sfx) if self.bias else None,
            getattr(self, "bias_hh_l0" + sfx) if self.bias else None, self.hidden_size, device)

    def _parse_initial_state(self, hx, batch_size: int):
        """hx [D, B, H] -> (h0_forward, h0_reverse) (quant_gru.py:1372-1400)."""
        if hx is None:
            return None, None
        expected = (self.num_layers * self.num_directions, batch_size, self.hidden_size)
        if tuple(hx.shape) != expected:
            raise ValueError(f"hx must have shape {expected}, got {tuple(hx.shape)}")
        return hx[0], (hx[1] if self.bidirectional else None)

    def _combine_bidirectional_outputs(self, out_f, hn_f, out_r=None, hn_r=None):
        """quant_gru.py:1402-1432."""
        if self.bidirectional and out_r is not None:
            return torch.cat([out_f, out_r], dim=-1), torch.cat([hn_f, hn_r], dim=0)
        return out_f, hn_f

    def _forward_with_calibration(self, input, hx=None):
        """Float GRU on the GPU + MinMax ranges merged per direction
        (quant_gru.py:2054-2149)."""
        self._check_calibration_method()
        T, B, I = input.shape
        H = self.hidden_size
        device = _require_device(input)
        input = ensure_cuda_float32(input, device).contiguous()
        h0f, h0r = self._parse_initial_state(hx, B)
        empty = torch.empty(0, device=device)
        if self.quant_ranges is None:
            self.quant_ranges = gru_ops.GRUQuantizationRanges(H, device=device)
        W, R, bw, br = self._direction_weights(False, device)
        with torch.no_grad():
            # the gate values (v) are not needed for the ranges: not materialised
            h, _ = gru_ops.forward_calibrate(
                is_training=False, time_steps=T, batch_size=B, input_size=I, hidden_size=H,
                W=W, R=R, bw=bw, br=br, x=input,
                h0=ensure_cuda_float32(h0f, device).contiguous() if h0f is not None else empty,
                calib_method=self.calibration_method, bitwidth_config=self._bitwidth_config,
                quant_ranges=self.quant_ranges)
        out_f, hn_f = h[1:], h[-1:]
        out_r = hn_r = None
        if self.bidirectional:
            if self.quant_ranges_reverse is None:
                self.quant_ranges_reverse = gru_ops.GRUQuantizationRanges(H, device=device)
            W, R, bw, br = self._direction_weights(True, device)
            with torch.no_grad():
                h_r, _ = gru_ops.forward_calibrate(
                    is_training=False, time_steps=T, batch_size=B, input_size=I, hidden_size=H,
                    W=W, R=R, bw=bw, br=br, x=input.flip(0).contiguous(),
                    h0=ensure_cuda_float32(h0r, device).contiguous() if h0r is not None else empty,
                    calib_method=self.calibration_method, bitwidth_config=self._bitwidth_config,
                    quant_ranges=self.quant_ranges_reverse)
            out_r, hn_r = h_r[1:].flip(0), h_r[-1:]
        if (not self._quant_params_locked) or self.quant_params is None:
            self._quant_params_dirty = True
        return self._combine_bidirectional_outputs(out_f, hn_f, out_r, hn_r)

    def _resolve_quant_params(self):
        """Dirty / lock handling before a quantised forward (quant_gru.py:2218-2242)."""
        if self._quant_params_locked and not self.is_calibrated():
            raise RuntimeError("quant_params are locked but incomplete: calibrate or load them "
                               "before locking, or call set_quant_params_locked(False)")
        if self._quant_params_dirty:
            if self._quant_params_locked and self.quant_params is not None:
                self._quant_params_dirty = False
            else:
                self.finalize_calibration()
        elif not self.is_calibrated():
            if self.quant_ranges is not None or self.hist_collectors is not None:
                self.finalize_calibration()
            else:
                raise RuntimeError(
                    "quantisation is enabled but the module is not calibrated:\n"
                    "  1. gru.calibrating = True\n  2. gru(calibration_data)\n"
                    "  3. gru.calibrating = False\n"
                    "(calibration data does not survive pickle/deepcopy)")

    def _forward_cuda(self, input, hx=None):
        """Quantised forward through GRUFunction per direction (quant_gru.py:2207-2288)."""
        if self.use_quantization:
            self._resolve_quant_params()
        T, B, I = input.shape
        device = _require_device(input)
        input = ensure_cuda_float32(input, device)
        h0f, h0r = self._parse_initial_state(hx, B)
        save_state = self._save_state(input, hx)
        if (self.bidirectional and self.use_quantization and not save_state
                and self.quant_storage_dtype == "int32" and self.hidden_size % 4 == 0):
            return self._forward_int_bidir(input, h0f, h0r, device)
        b = self.bias
        out_f, hn_f = GRUFunction.apply(
            input, self.weight_ih_l0, self.weight_hh_l0, self.bias_ih_l0 if b else None,
            self.bias_hh_l0 if b else None, h0f, save_state, self.use_quantization,
            self.quant_params, self.quant_storage_dtype)
        out_r = hn_r = None
        if self.bidirectional:
            out_r, hn_r = GRUFunction.apply(
                input.flip(0), self.weight_ih_l0_reverse, self.weight_hh_l0_reverse,
                self.bias_ih_l0_reverse if b else None, self.bias_hh_l0_reverse if b else None,
                h0r, save_state, self.use_quantization, self.quant_params_reverse,
                self.quant_storage_dtype)
            out_r = out_r.flip(0)
        return self._combine_bidirectional_outputs(out_f, hn_f, out_r, hn_r)

    def _forward_int_bidir(self, input, h0f, h0r, device, int_io=False):
        """Inference of both directions on the int32 carrier in one library call (one clustered
        recurrence launch for the two directions) and the output assembled in the library; the
        reverse direction reads a time-flipped copy of the input.  Replaces the per-direction
        calls with flip / cat of the reference (quant_gru.py:2207-2288, 2482-2537)."""
        T, B, I = input.shape
        H = self.hidden_size
        dirs = []
        for reverse, h0 in ((False, h0f), (True, h0r)):
            if h0 is not None and not int_io:
                h0 = ensure_cuda_float32(h0, device).contiguous()
            W, R, bw, br = self._direction_weights(reverse, device)
            qp = self.quant_params_reverse if reverse else self.quant_params
            dirs.append((W, R, bw, br, input.flip(0) if reverse else input, h0, qp))
        h_f, h_r = gru_ops.forward_int_bidir(T, B, I, H, dirs, int_io=int_io)
        return gru_ops.bidir_assemble(h_f, h_r, False)

    def _save_state(self, input, hx) -> bool:
        """Gate values and masks are kept whenever a backward may follow
        (quant_gru.py:2258-2263)."""
        return self.training or (torch.is_grad_enabled() and (
            input.requires_grad or (hx is not None and hx.requires_grad)
            or any(p.requires_grad for p in self.parameters())))

    def _forward_bidirectional(self, input, hx=None):
        """Quantised bidirectional forward on the caller's layout (GRUBidirectionalFunction):
        no transposes, flips or concatenations outside the library."""
        self._resolve_quant_params()
        device = _require_device(input)
        B = input.shape[0] if self.batch_first else input.shape[1]
        h0f, h0r = self._parse_initial_state(hx, B)
        b = self.bias
        return GRUBidirectionalFunction.apply(
            ensure_cuda_float32(input, device), self.weight_ih_l0, self.weight_hh_l0,
            self.bias_ih_l0 if b else None, self.bias_hh_l0 if b else None, h0f,
            self.weight_ih_l0_reverse, self.weight_hh_l0_reverse,
            self.bias_ih_l0_reverse if b else None, self.bias_hh_l0_reverse if b else None, h0r,
            self._save_state(input, hx), self.quant_params, self.quant_params_reverse,
            self.batch_first)

    def forward(self, input: torch.Tensor, hx: Optional[torch.Tensor] = None
                ) -> Tuple[torch.Tensor, torch.Tensor]:
        """input [T,B,I] or [B,T,I] (batch_first); hx [D,B,H].  Returns (output [.., D*H],
        h_n [D,B,H]) (quant_gru.py:2151-2205)."""
        if self.export_mode:
            raise NotImplementedError("ONNX export mode is not provided by the MI355X build")
        if (not self.calibrating and self.bidirectional and self.use_quantization
                and self.quant_storage_dtype == "float32" and self.hidden_size % 16 == 0):
            return self._forward_bidirectional(input, hx)
        if self.batch_first:
            input = input.transpose(0, 1)
            if (self.calibrating or self.bidirectional or not self.use_quantization
                    or self.quant_storage_dtype != "float32" or self._save_state(input, hx)):
                input = input.contiguous()  # else GRUFunction reads the [B, T, I] rows in place
        if self.calibrating:
            output, h_n = self._forward_with_calibration(input, hx)
        else:
            output, h_n = self._forward_cuda(input, hx)
        if self.batch_first:
            output = output.transpose(0, 1).contiguous()
        return output, h_n


    # -- AIMET fixed-point contract (quant_gru.py:2290-2537) -------------------------------

    _AIMET_SUPPORTED_MODES = ("fp32", "fp32_qdq", "fp16_qdq", "int16_fixed_eval",
                              "int16_fixed_qat_sim", "calibrating")

    def aimet_capabilities(self) -> dict:
        """The adapter capability report (quant_gru.py:2336-2353)."""
        return {
            "adapter_version": "1.1",
            "supported_modes": list(self._AIMET_SUPPORTED_MODES),
            "forward_io_dtype": "float32",
            "forward_io_device": "cuda",
            "requires_calibration_for": ["int16_fixed_eval", "int16_fixed_qat_sim"],
            "supports_forward_quantized": True,
            "forward_quantized_input_dtypes": ["int32"],
        }

    def aimet_configure(self, mode: str) -> None:
        """Map an AIMET execution mode onto the module flags (quant_gru.py:2355-2378)."""
        normalized = str(mode).lower()
        if normalized not in self._AIMET_SUPPORTED_MODES:
            raise ValueError(f"Unsupported aimet_configure mode: {mode!r}. "
                             f"Expected one of: {', '.join(self._AIMET_SUPPORTED_MODES)}.")
        self.export_mode = False
        if normalized == "calibrating":
            self.calibrating = True
            self.use_quantization = False
            return
        self.calibrating = False
        self.use_quantization = normalized in ("int16_fixed_eval", "int16_fixed_qat_sim")

    def get_io_quant_meta(self) -> dict:
        """Grids of the input, output and hidden state as forward_quantized reads and writes
        them (quant_gru.py:2380-2429): the effective (encoded) scale, zero point, bit width and
        signedness of the x and h operators."""
        if not self.is_calibrated() or self.quant_params is None:
            raise RuntimeError("QuantGRU not calibrated")
        qp = self.quant_params
        cfg = self._bitwidth_config
        use_pot2 = bool(self.use_pot2_scale)

        def entry(prefix: str) -> dict:
            scale = float(gru_ops.decode_effective_scale(float(getattr(qp, f"scale_{prefix}")),
                                                         use_pot2))
            is_symmetric = bool(getattr(cfg, f"{prefix}symmetric_"))
            is_unsigned = bool(getattr(cfg, f"{prefix}unsigned_", False))
            if is_unsigned and is_symmetric:
                is_symmetric = False
            return {"scale": scale, "zp": int(getattr(qp, f"zp_{prefix}")),
                    "bitwidth": int(getattr(cfg, prefix)), "is_symmetric": is_symmetric,
                    "is_unsigned": is_unsigned}

        return {"input": entry("x_"), "output": entry("h_"), "hidden": entry("h_")}

    def _forward_quantized_dir(self, x_q, h0_q, reverse: bool, device):
        T, B, I = x_q.shape
        W, R, bw, br = self._direction_weights(reverse, device)
        qp = self.quant_params_reverse if reverse else self.quant_params
        h0 = h0_q if h0_q is not None else torch.empty(0, dtype=torch.int32, device=device)
        return gru_ops.forward_quantized_int_io(T, B, I, self.hidden_size, W, R, bw, br, x_q, h0,
                                                qp)

    def forward_quantized(self, input: torch.Tensor, hx: Optional[torch.Tensor] = None
                          ) -> Tuple[torch.Tensor, torch.Tensor]:
        """Integer-in, integer-out inference (quant_gru.py:2482-2537): input holds int32 codes
        on the x grid ([T,B,I], or [B,T,I] with batch_first), hx int32 codes on the h grid (or
        None); only the weights are quantised.  Returns int32 (output_q, h_n_q) shaped like
        forward's outputs, with (output_q - zp) * scale equal to the quantised forward's
        output (scale and zp from get_io_quant_meta)."""
        if not self.is_calibrated() or self.quant_params is None:
            raise RuntimeError("QuantGRU not calibrated")
        if self.export_mode:
            raise RuntimeError("forward_quantized does not support export_mode")
        if input.is_floating_point():
            raise TypeError("forward_quantized takes integer codes on the input grid (int in, "
                            f"int out); got dtype={input.dtype}")
        if self.batch_first:
            input = input.transpose(0, 1)
        T, B, I = input.shape
        device = _require_device(input)
        input = input.to(device=device, dtype=torch.int32).contiguous()
        h0f = h0r = None
        if hx is not None:
            expected = (self.num_layers * self.num_directions, B, self.hidden_size)
            if tuple(hx.shape) != expected:
                raise ValueError(f"hx must have shape {expected}, got {tuple(hx.shape)}")
            hx = hx.to(device=device, dtype=torch.int32)
            h0f = hx[0].contiguous()
            h0r = hx[1].contiguous() if self.bidirectional else None
        if self.bidirectional and self.hidden_size % 4 == 0:
            output_q, h_n_q = self._forward_int_bidir(input, h0f, h0r, device, int_io=True)
            if self.batch_first:
                output_q = output_q.transpose(0, 1).contiguous()
            return output_q, h_n_q
        out_f, hn_f = self._forward_quantized_dir(input, h0f, False, device)
        out_r = hn_r = None
        if self.bidirectional:
            out_r, hn_r = self._forward_quantized_dir(input.flip(0).contiguous(), h0r, True,
                                                      device)
            out_r = out_r.flip(0)
        output_q, h_n_q = self._combine_bidirectional_outputs(out_f, hn_f, out_r, hn_r)
        if self.batch_first:
            output_q = output_q.transpose(0, 1).contiguous()
        return output_q, h_n_q


def set_quant_gru_module_names(model: nn.Module, prefix: str = "") -> None:
    """Give every QuantGRU in ``model`` its dotted module path (quant_gru.py:4875-4893)."""
    for name, mod in model.named_modules(prefix=prefix):
        if isinstance(mod, QuantGRU):
            mod.set_module_name(name)
