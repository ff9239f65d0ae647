"""MI355X quantization backend for aimet_torch's affine quantizers.

This module implements aimet_torch's backend protocol
(``src/aimet_torch/v2/quantization/affine/backends/utils.py:45-74``):
``quantize``, ``dequantize`` and ``quantize_dequantize`` with the same signatures,
argument checks and numerics as the default ``torch_builtins`` backend
(``backends/torch_builtins.py``), but each call is one hand-written HIP kernel per
direction (``librxmet.so``, ``include/rxmet_qdq.h``) instead of a chain of aten ops.

Drop-in use with aimet_torch::

    from aimet_torch.v2.quantization.affine.backends import add_backend, set_backend
    import mi355x_qdq
    add_backend("mi355x", mi355x_qdq)
    with set_backend("mi355x"):
        ...

Numerics (torch_builtins.py:199-279): when encodings are frozen (scale/offset need no
gradient, or autograd is off), no block size and no zero-point shift are given, and
the encoding is per-tensor or single-axis per-channel, the reference calls
``torch.fake_quantize_per_{tensor,channel}_affine`` (``rint(x * fl(1/s)) + zp``) and then
restores NaN; otherwise it runs ``QuantDequantFunc`` (``rint(x / s) - offset``).  This
backend makes the same choice and runs the matching kernel mode, so results are
bit-identical to the path the reference would have taken.
"""
from __future__ import annotations

import functools
import math
from typing import List, Optional, Tuple

import torch

import rxmet_lib as _rx

LEARNABLE = 0
FROZEN = 1

# ---------------------------------------------------------------------------------
# Argument checks (torch_builtins.py:58-148)
# ---------------------------------------------------------------------------------


def _is_expandable(src_shape, target_shape) -> bool:
    """``aimet_torch.v2.utils._is_expandable`` (utils.py:48-59)."""
    if len(src_shape) > len(target_shape):
        return False
    for s, d in zip(tuple(src_shape)[::-1], tuple(target_shape)[::-1]):
        if s not in (1, d):
            return False
    return True


def _is_value_representable(dtype: torch.dtype, value: int) -> bool:
    r = torch.tensor(value, dtype=dtype)
    return bool(r.isfinite()) and int(r.long()) == value


@functools.lru_cache(None)
def _is_grid_representable(dtype: torch.dtype, qmin: int, qmax: int) -> bool:
    return (_is_value_representable(dtype, qmax) and _is_value_representable(dtype, qmax - 1)
            and _is_value_representable(dtype, qmin + 1) and _is_value_representable(dtype, qmin))


def _is_numerically_stable(dtype: torch.dtype, qmin: int, qmax: int) -> bool:
    if not _is_grid_representable(dtype, qmin, qmax):
        return False
    if qmin == qmax:
        return True
    return not torch.finfo(dtype).eps > 1e-1 / (qmax - qmin)


def _validate_arguments(tensor, scale, qmin=None, qmax=None, block_size=None):
    """Same checks and messages as torch_builtins._validate_arguments (:104-148)."""
    if block_size is not None:
        if len(scale.shape) != len(block_size):
            raise RuntimeError(
                f"Length of scale shape {scale.shape} must equal length of block size {block_size}")
        for i in range(1, len(block_size) + 1):
            if block_size[-i] == -1:
                if tensor.shape[-i] % scale.shape[-i] != 0:
                    raise RuntimeError(
                        f"Each tensor dimension size for tensor shape {tensor.shape} must divide "
                        f"evenly with corresponding scale dimension value for scale shape {scale.shape}")
            elif block_size[-i] * scale.shape[-i] != tensor.shape[-i]:
                raise RuntimeError(
                    f"Each tensor dimension size for tensor shape {tensor.shape} must equal the "
                    f"corresponding scale dimension size * block size for scale shape {scale.shape} "
                    f"and block size {block_size}")
    elif not _is_expandable(scale.shape, tensor.shape):
        raise RuntimeError(
            f"Scale of shape {scale.shape} cannot be expanded like input tensor of shape "
            f"{tensor.shape}. ")
    if qmin is not None and qmax is not None and qmin > qmax:
        raise RuntimeError(f"qmin ({qmin}) must be smaller than or equal to qmax ({qmax})")


def get_encoding_shape_with_blocks(original_encoding_shape, block_size):
    """torch_builtins.get_encoding_shape_with_blocks (:694-714)."""
    if block_size is None:
        return original_encoding_shape
    new_shape = []
    for size in original_encoding_shape:
        new_shape.append(size)
        new_shape.append(1)
    return new_shape


def reshape_tensor_for_blocks(tensor, encoding_shape, block_size):
    """torch_builtins.reshape_tensor_for_blocks (:717-754)."""
    if block_size is None:
        return tensor
    input_reshape = []
    for i in range(1, len(block_size) + 1):
        if block_size[-i] == -1:
            input_reshape.insert(0, tensor.shape[-i] // encoding_shape[-i])
            input_reshape.insert(0, encoding_shape[-i])
        else:
            input_reshape.insert(0, block_size[-i])
            input_reshape.insert(0, encoding_shape[-i])
    input_reshape = list(tensor.shape[: -len(block_size)]) + input_reshape
    return tensor.view(input_reshape)


# ---------------------------------------------------------------------------------
# Layout: map (tensor shape, encoding shape) onto the kernels' [outer, C0, mid, C1, inner]
# view (encoding c0 * C1 + c1 of row-major element (o, c0, m, c1, k)).
# ---------------------------------------------------------------------------------

_IO_CODE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2, torch.float64: 3}
_INTERNAL_CODE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2, torch.float64: 3}


def _groups(tensor_shape, enc_shape):
    """Maximal runs of adjacent axes that all carry encodings ("E") or none ("N"), as
    (kind, size, axes); axes of size 1 join no group."""
    tensor_shape = tuple(int(d) for d in tensor_shape)
    nd = len(tensor_shape)
    enc = (1,) * (nd - len(enc_shape)) + tuple(int(d) for d in enc_shape)
    out = []
    for a, (t, e) in enumerate(zip(tensor_shape, enc)):
        if e not in (1, t):
            raise ValueError(f"encoding shape {tuple(enc_shape)} does not match tensor shape "
                             f"{tensor_shape}")
        if t == 1:
            continue
        kind = "E" if e != 1 else "N"
        if out and out[-1][0] == kind:
            out[-1] = (kind, out[-1][1] * t, out[-1][2] + (a,))
        else:
            out.append((kind, t, (a,)))
    return out


def kernel_layout(tensor_shape, enc_shape) -> Optional[Tuple[int, int, int, int, int]]:
    """(outer, C0, mid, C1, inner) for encodings on at most two separated groups of axes,
    or None (three or more groups)."""
    numel = math.prod(int(d) for d in tensor_shape)
    groups = _groups(tensor_shape, enc_shape)
    n_enc = sum(1 for g in groups if g[0] == "E")
    if n_enc == 0:
        return 1, 1, 1, 1, numel
    if n_enc > 2:
        return None
    sizes = [g[1] for g in groups]
    outer = 1
    if groups[0][0] == "N":
        outer, sizes = sizes[0], sizes[1:]
    sizes = sizes + [1] * (4 - len(sizes))  # E [N [E [N]]]
    if n_enc == 1:
        return 1, 1, outer, sizes[0], sizes[1]
    return outer, sizes[0], sizes[1], sizes[2], sizes[3]


class _Plan:
    """How a tensor reaches the kernels: its layout, and (for encodings on three or more
    separated axis groups) the permutation that gathers the encoding axes in front."""

    __slots__ = ("layout", "perm", "inv", "C")

    def __init__(self, tensor_shape, enc_shape):
        tensor_shape = tuple(int(d) for d in tensor_shape)
        nd = len(tensor_shape)
        enc = (1,) * (nd - len(enc_shape)) + tuple(int(d) for d in enc_shape)
        self.C = math.prod(enc)
        self.perm = self.inv = None
        if math.prod(tensor_shape) == 0:
            self.layout = (1, 1, 0, max(self.C, 1), 1)
            return
        lay = kernel_layout(tensor_shape, enc)
        if lay is None:
            e_axes = [a for a in range(nd) if enc[a] != 1 and tensor_shape[a] != 1]
            self.perm = tuple(e_axes + [a for a in range(nd) if a not in e_axes])
            self.inv = tuple(sorted(range(nd), key=self.perm.__getitem__))
            lay = (1, 1, 1, self.C, math.prod(tensor_shape) // self.C)
        self.layout = lay

    def to_kernel(self, t: torch.Tensor) -> torch.Tensor:
        return (t.permute(self.perm) if self.perm else t).contiguous()

    def from_kernel(self, t: torch.Tensor) -> torch.Tensor:
        return t.permute(self.inv).contiguous() if self.perm else t

    def cstruct(self):
        return _rx.QdqLayout(*self.layout)


def _require(tensor: torch.Tensor, what: str):
    if not tensor.is_cuda:
        raise RuntimeError(f"mi355x backend: {what} must be a GPU tensor")
    if tensor.dtype not in _IO_CODE:
        raise NotImplementedError(
            f"mi355x backend: {what} must be float32, float16, bfloat16 or float64 "
            f"(got {tensor.dtype})")


def _numerics(io: torch.dtype, internal: torch.dtype, shift: float = 0.0,
              scalar_scale: bool = False):
    return _rx.QdqNumerics(_IO_CODE[io], _INTERNAL_CODE[internal], float(shift),
                           int(bool(scalar_scale)), 0)


def _internal_dtype(dtype: torch.dtype, qmin: int, qmax: int) -> torch.dtype:
    """The reference's widening rule (torch_builtins.py:171-174, 255-262)."""
    internal = dtype
    if not _is_numerically_stable(internal, qmin, qmax):
        internal = torch.float32
        if not _is_numerically_stable(internal, qmin, qmax):
            internal = torch.float64
    return internal


def _enc_vectors(scale, offset, internal: torch.dtype, enc_shape):
    """scale.to(internal) / offset.to(internal) of the reference, broadcast to the encoding
    shape and flattened in the kernels' encoding order, carried as float32 (exact: the
    internal type is fp16/bf16/fp32, or fp64 holding fp32/fp16/bf16 values).  Autograd flows
    through these conversions back to the caller's parameters."""
    if internal == torch.float64 and torch.float64 in (scale.dtype, offset.dtype):
        raise NotImplementedError(
            "mi355x backend: float64 encodings with float64 arithmetic are not supported")

    def vec(t):
        return t.to(internal).expand(enc_shape).reshape(-1).to(torch.float32).contiguous()

    return vec(scale), vec(offset)


def _enc_shape(scale, offset, nd: int):
    shape = torch.broadcast_shapes(tuple(scale.shape), tuple(offset.shape))
    return (1,) * (nd - len(shape)) + tuple(shape)


def _workspace(plan: _Plan, io: torch.dtype, device) -> torch.Tensor:
    lay = plan.cstruct()
    nbytes = int(_rx.load().rxmet_qdq_workspace_bytes_ex(lay, _IO_CODE[io]))
    return torch.empty(max(nbytes, 16), dtype=torch.uint8, device=device)


def _enc_grad(need: bool, C: int, device):
    return torch.empty(C, dtype=torch.float32, device=device) if need else None


# ---------------------------------------------------------------------------------
# Autograd functions — each direction is one kernel launch (+ a tiny fold kernel).
# The encoding arguments are the flat float32 vectors of _enc_vectors.
# ---------------------------------------------------------------------------------


class _QuantDequant(torch.autograd.Function):
    """QuantDequantFunc (torch_builtins.py:618-691) with the zero_point_shift around it
    (:276-284), or the fake_quantize fast path (:221-249)."""

    @staticmethod
    def forward(ctx, x, s, o, qmin: int, qmax: int, mode: int, plan: _Plan, numerics):
        xk = plan.to_kernel(x)
        y = torch.empty_like(xk)
        if s.numel() > 0:
            _rx.call("rxmet_qdq_forward_ex", _rx.ptr(xk), _rx.ptr(y), plan.cstruct(), numerics,
                     _rx.ptr(s), _rx.ptr(o), int(qmin), int(qmax), int(mode),
                     _rx.stream_of(xk.device))
        ctx.args = (int(qmin), int(qmax), int(mode), plan, numerics)
        ctx.save_for_backward(xk, s, o)
        return plan.from_kernel(y)

    @staticmethod
    def backward(ctx, g):
        xk, s, o = ctx.saved_tensors
        qmin, qmax, mode, plan, numerics = ctx.args
        need_x, need_s, need_o = ctx.needs_input_grad[:3]
        learn = mode == LEARNABLE
        gk = plan.to_kernel(g.to(xk.dtype))
        dx = torch.empty_like(xk)
        ds = _enc_grad(need_s and learn, s.numel(), xk.device)
        do = _enc_grad(need_o and learn, s.numel(), xk.device)
        ws = _workspace(plan, xk.dtype, xk.device) if (ds is not None or do is not None) else None
        if s.numel() > 0:
            _rx.call("rxmet_qdq_backward_ex", _rx.ptr(xk), _rx.ptr(gk), _rx.ptr(dx), _rx.ptr(ds),
                     _rx.ptr(do), plan.cstruct(), numerics, _rx.ptr(s), _rx.ptr(o), qmin, qmax,
                     mode, _rx.ptr(ws), _rx.stream_of(xk.device))
        return (plan.from_kernel(dx) if need_x else None), ds, do, None, None, None, None, None


class _QuantDequantMinMax(torch.autograd.Function):
    """QuantizeDequantize.forward with learnable min / max (quantizer.py:1048-1082): the
    encodings of get_encodings() (:466-483) and the learnable QuantDequantFunc path in one
    launch each way (rxmet_qdq_forward_minmax / _backward_minmax).  The kernels derive scale and
    offset from min and max themselves, and the backward's fold takes the encoding gradients on
    to min and max; the results equal minmax_encodings() followed by quantize_dequantize() bit
    for bit."""

    @staticmethod
    def forward(ctx, x, mn, mx, qmin: int, qmax: int, enc: tuple, plan: _Plan, numerics):
        xk = plan.to_kernel(x)
        y = torch.empty_like(xk)
        mnv, mxv = mn.detach().reshape(-1), mx.detach().reshape(-1)
        _rx.call("rxmet_qdq_forward_minmax", _rx.ptr(xk), _rx.ptr(y), plan.cstruct(), numerics,
                 _minmax_struct(mnv, mxv, enc), int(qmin), int(qmax), _rx.stream_of(xk.device))
        ctx.args = (int(qmin), int(qmax), enc, plan, numerics)
        ctx.min_shape = mn.shape
        ctx.save_for_backward(xk, mnv, mxv)
        return plan.from_kernel(y)

    @staticmethod
    def backward(ctx, g):
        xk, mnv, mxv = ctx.saved_tensors
        qmin, qmax, enc, plan, numerics = ctx.args
        need_x, need_mn, need_mx = ctx.needs_input_grad[:3]
        gk = plan.to_kernel(g.to(xk.dtype))
        dx = torch.empty_like(xk)
        need_enc = need_mn or need_mx
        d_min = torch.empty_like(mnv) if need_enc else None
        d_max = torch.empty_like(mxv) if need_enc else None
        ws = _workspace(plan, xk.dtype, xk.device) if need_enc else None
        _rx.call("rxmet_qdq_backward_minmax", _rx.ptr(xk), _rx.ptr(gk), _rx.ptr(dx),
                 _rx.ptr(d_min), _rx.ptr(d_max), plan.cstruct(), numerics,
                 _minmax_struct(mnv, mxv, enc), qmin, qmax, _rx.ptr(ws),
                 _rx.stream_of(xk.device))
        shape = ctx.min_shape
        return ((plan.from_kernel(dx) if need_x else None),
                d_min.view(shape) if need_mn else None, d_max.view(shape) if need_mx else None,
                None, None, None, None, None)


def _minmax_struct(mnv, mxv, enc):
    symmetric, sym_offset, min_scale = enc
    return _rx.QdqMinMaxEnc(mnv.data_ptr(), mxv.data_ptr(), int(bool(symmetric)),
                            float(sym_offset), float(min_scale), 0)


class _Quantize(torch.autograd.Function):
    """QuantizeFunc (torch_builtins.py:505-571)."""

    @staticmethod
    def forward(ctx, x, s, o, qmin: int, qmax: int, plan: _Plan, numerics):
        xk = plan.to_kernel(x)
        q = torch.empty_like(xk)
        if s.numel() > 0:
            _rx.call("rxmet_quantize_forward_ex", _rx.ptr(xk), _rx.ptr(q), plan.cstruct(),
                     numerics, _rx.ptr(s), _rx.ptr(o), int(qmin), int(qmax),
                     _rx.stream_of(xk.device))
        ctx.args = (int(qmin), int(qmax), plan, numerics)
        ctx.save_for_backward(xk, s, o)
        return plan.from_kernel(q)

    @staticmethod
    def backward(ctx, g):
        xk, s, o = ctx.saved_tensors
        qmin, qmax, plan, numerics = ctx.args
        need_x, need_s, need_o = ctx.needs_input_grad[:3]
        gk = plan.to_kernel(g.to(xk.dtype))
        dx = torch.empty_like(xk)
        ds = _enc_grad(need_s, s.numel(), xk.device)
        do = _enc_grad(need_o, s.numel(), xk.device)
        ws = _workspace(plan, xk.dtype, xk.device) if (need_s or need_o) else None
        if s.numel() > 0:
            _rx.call("rxmet_quantize_backward_ex", _rx.ptr(xk), _rx.ptr(gk), _rx.ptr(dx),
                     _rx.ptr(ds), _rx.ptr(do), plan.cstruct(), numerics, _rx.ptr(s),
                     _rx.ptr(o), qmin, qmax, _rx.ptr(ws), _rx.stream_of(xk.device))
        return (plan.from_kernel(dx) if need_x else None), ds, do, None, None, None, None


class _Dequantize(torch.autograd.Function):
    """DequantizeFunc (torch_builtins.py:574-615)."""

    @staticmethod
    def forward(ctx, q, s, o, plan: _Plan, numerics):
        qk = plan.to_kernel(q)
        y = torch.empty_like(qk)
        if s.numel() > 0:
            _rx.call("rxmet_dequantize_forward_ex", _rx.ptr(qk), _rx.ptr(y), plan.cstruct(),
                     numerics, _rx.ptr(s), _rx.ptr(o), _rx.stream_of(qk.device))
        ctx.args = (plan, numerics)
        ctx.save_for_backward(qk, s, o)
        return plan.from_kernel(y)

    @staticmethod
    def backward(ctx, g):
        qk, s, o = ctx.saved_tensors
        plan, numerics = ctx.args
        need_q, need_s, need_o = ctx.needs_input_grad[:3]
        gk = plan.to_kernel(g.to(qk.dtype))
        dq = torch.empty_like(qk)
        ds = _enc_grad(need_s, s.numel(), qk.device)
        do = _enc_grad(need_o, s.numel(), qk.device)
        ws = _workspace(plan, qk.dtype, qk.device) if (need_s or need_o) else None
        if s.numel() > 0:
            _rx.call("rxmet_dequantize_backward_ex", _rx.ptr(qk), _rx.ptr(gk), _rx.ptr(dq),
                     _rx.ptr(ds), _rx.ptr(do), plan.cstruct(), numerics, _rx.ptr(s),
                     _rx.ptr(o), _rx.ptr(ws), _rx.stream_of(qk.device))
        return (plan.from_kernel(dq) if need_q else None), ds, do, None, None


# ---------------------------------------------------------------------------------
# Backend protocol
# ---------------------------------------------------------------------------------


def _fast_path_layout(scale, offset, tensor, qmin: int, qmax: int) -> bool:
    """Would torch_builtins._torch_fake_quantize (:287-361) accept these encodings?"""
    if scale.numel() == offset.numel() == 1:
        return True
    nd = tensor.dim()
    s_shape = (1,) * (nd - scale.dim()) + tuple(scale.shape)
    o_shape = (1,) * (nd - offset.dim()) + tuple(offset.shape)
    if s_shape != o_shape:
        return False
    if not all(sd in (1, td) for sd, td in zip(s_shape, tensor.shape)):
        return False
    axes = [a for a, sd in enumerate(s_shape) if sd != 1]
    if len(axes) != 1:
        return False
    # aten's per-channel kernel rejects zero points outside [qmin, qmax]; the reference
    # then falls back to QuantDequantFunc (torch_builtins.py:350-356).
    zp = -offset.detach().to(torch.int32)
    return not bool(((zp < qmin) | (zp > qmax)).any())


def _blocked(tensor, scale, offset, block_size):
    """The reference's block reshape (torch_builtins.py:178-181, 266-271)."""
    t = reshape_tensor_for_blocks(tensor, scale.shape, block_size)
    s = scale.view(get_encoding_shape_with_blocks(scale.shape, block_size))
    o = offset.view(get_encoding_shape_with_blocks(offset.shape, block_size))
    return t, s, o


def quantize(tensor: torch.Tensor, scale: torch.Tensor, offset: torch.Tensor, qmin: int, qmax: int,
             block_size: Optional[List] = None) -> torch.Tensor:
    """Differentiable quantization (torch_builtins.quantize, :151-194)."""
    _validate_arguments(tensor, scale, qmin, qmax, block_size)
    _require(tensor, "tensor")
    if not _is_grid_representable(tensor.dtype, qmin, qmax):
        raise RuntimeError(
            f"{tensor.dtype} is unable to represent quantized output of range [{qmin}, {qmax}].")
    internal = _internal_dtype(tensor.dtype, qmin, qmax)
    orig_shape = tensor.shape
    t, s, o = _blocked(tensor, scale, offset, block_size)
    enc_shape = _enc_shape(s, o, t.dim())
    sv, ov = _enc_vectors(s, o, internal, enc_shape)
    scalar = s.dim() == 0 and t.dim() > 0 and internal != t.dtype
    return _Quantize.apply(t, sv, ov, int(qmin), int(qmax), _Plan(t.shape, enc_shape),
                           _numerics(t.dtype, internal, 0.0, scalar)).view(orig_shape)


def dequantize(tensor: torch.Tensor, scale: torch.Tensor, offset: torch.Tensor,
               block_size: Optional[List] = None) -> torch.Tensor:
    """Differentiable dequantization (torch_builtins.dequantize, :459-488)."""
    _validate_arguments(tensor, scale, block_size=block_size)
    _require(tensor, "tensor")
    orig_shape = tensor.shape
    t, s, o = _blocked(tensor, scale, offset, block_size)
    enc_shape = _enc_shape(s, o, t.dim())
    sv, ov = _enc_vectors(s, o, t.dtype, enc_shape)
    return _Dequantize.apply(t, sv, ov, _Plan(t.shape, enc_shape),
                             _numerics(t.dtype, t.dtype)).view(orig_shape)


def quantize_dequantize(tensor: torch.Tensor, scale: torch.Tensor, offset: torch.Tensor, qmin: int,
                        qmax: int, block_size: Optional[List] = None,
                        zero_point_shift: float = 0.0) -> torch.Tensor:
    """Differentiable fake quantization (torch_builtins.quantize_dequantize, :199-284)."""
    _validate_arguments(tensor, scale, qmin, qmax, block_size)
    _require(tensor, "tensor")
    fast = block_size is None and not torch.jit.is_tracing() and zero_point_shift == 0.0
    fast &= ((not scale.requires_grad and not getattr(offset, "requires_grad", False))
             or not torch.is_grad_enabled())
    # grids beyond 2^24 steps leave the fp32 fast path (its codes and zero points would round)
    # for the general kernels, which compute in float64 for such grids
    fast &= max(abs(int(qmin)), abs(int(qmax))) <= 1 << 24
    if fast and _fast_path_layout(scale, offset, tensor, qmin, qmax):
        enc_shape = _enc_shape(scale, offset, tensor.dim())
        sv = scale.detach().to(torch.float32).expand(enc_shape).reshape(-1).contiguous()
        ov = offset.detach().to(torch.float32).expand(enc_shape).reshape(-1).contiguous()
        return _QuantDequant.apply(tensor, sv, ov, int(qmin), int(qmax), FROZEN,
                                   _Plan(tensor.shape, enc_shape),
                                   _numerics(tensor.dtype, torch.float32))
    internal = _internal_dtype(tensor.dtype, qmin, qmax)
    if not _is_grid_representable(internal, qmin, qmax):
        raise RuntimeError(
            f"{internal} is unable to represent quantized output of range [{qmin}, {qmax}].")
    orig_shape = tensor.shape
    t, s, o = _blocked(tensor, scale, offset, block_size)
    enc_shape = _enc_shape(s, o, t.dim())
    sv, ov = _enc_vectors(s, o, internal, enc_shape)
    scalar = s.dim() == 0 and t.dim() > 0 and internal != t.dtype
    return _QuantDequant.apply(t, sv, ov, int(qmin), int(qmax), LEARNABLE,
                               _Plan(t.shape, enc_shape),
                               _numerics(t.dtype, internal, zero_point_shift, scalar)
                               ).view(orig_shape)


def quantize_dequantize_minmax(tensor: torch.Tensor, mn: torch.Tensor, mx: torch.Tensor,
                               qmin: int, qmax: int, symmetric: bool, min_scale: float,
                               sym_offset: float, block_size: Optional[List] = None,
                               zero_point_shift: float = 0.0) -> Optional[torch.Tensor]:
    """QuantizeDequantize.forward of learnable fp32 min / max parameters (their shape is the
    encoding shape) through the fused kernels, or None where this form does not apply (the
    caller then takes get_encodings() and quantize_dequantize): it needs CUDA fp32 contiguous
    min / max with one value per encoding, and a tensor on the same device.  Encodings without
    gradient (frozen min / max, or autograd off) take the reference's fake_quantize fast path
    (torch_builtins.py:221-249), so they are left to quantize_dequantize."""
    if not (torch.is_grad_enabled() and (mn.requires_grad or mx.requires_grad)):
        return None
    if not (mn.is_cuda and mx.is_cuda and tensor.is_cuda and mn.dtype == torch.float32
            and mx.dtype == torch.float32 and mn.is_contiguous() and mx.is_contiguous()
            and mn.shape == mx.shape and tensor.dtype in _IO_CODE and qmax > qmin):
        return None
    _validate_arguments(tensor, mn, qmin, qmax, block_size)
    internal = _internal_dtype(tensor.dtype, qmin, qmax)
    if not _is_grid_representable(internal, qmin, qmax):
        raise RuntimeError(
            f"{internal} is unable to represent quantized output of range [{qmin}, {qmax}].")
    if max(abs(int(qmin)), abs(int(qmax))) > 1 << 24:
        return None
    orig_shape = tensor.shape
    t = reshape_tensor_for_blocks(tensor, mn.shape, block_size)
    enc_view = get_encoding_shape_with_blocks(mn.shape, block_size)
    enc_shape = (1,) * (t.dim() - len(enc_view)) + tuple(enc_view)
    plan = _Plan(t.shape, enc_shape)
    if plan.C != mn.numel() or t.numel() == 0:
        return None
    scalar = mn.dim() == 0 and t.dim() > 0 and internal != t.dtype
    fn = _QuantDequantMinMax
    y = fn.apply(t, mn, mx, int(qmin), int(qmax),
                 (bool(symmetric), float(sym_offset), float(min_scale)), plan,
                 _numerics(t.dtype, internal, zero_point_shift, scalar))
    return y.view(orig_shape)


def minmax(tensor: torch.Tensor, enc_shape) -> Tuple[torch.Tensor, torch.Tensor]:
    """Min and max of ``tensor`` reduced to ``enc_shape`` (NaN propagates), in the tensor's
    dtype.  Kernel of ``_MinMaxObserver.collect_stats`` (encoding_analyzer.py:101-105)."""
    _require(tensor, "tensor")
    nd = tensor.dim()
    enc = (1,) * (nd - len(enc_shape)) + tuple(int(d) for d in enc_shape)
    plan = _Plan(tensor.shape, enc)
    x = plan.to_kernel(tensor)
    if x.numel() == 0:
        raise RuntimeError("mi355x backend: min/max of an empty tensor")
    C = plan.C
    mn = torch.empty(C, dtype=torch.float32, device=x.device)
    mx = torch.empty(C, dtype=torch.float32, device=x.device)
    ws = _workspace(plan, x.dtype, x.device)
    _rx.call("rxmet_qdq_minmax_ex", _rx.ptr(x), _IO_CODE[x.dtype], plan.cstruct(), _rx.ptr(mn),
             _rx.ptr(mx), _rx.ptr(ws), _rx.stream_of(x.device))
    shape = tuple(enc_shape)
    return mn.to(x.dtype).view(shape), mx.to(x.dtype).view(shape)


class _MinMaxEncodings(torch.autograd.Function):
    """(scale, offset) of learnable min/max in one launch each way
    (rxmet_qdq_encoding_forward / _backward): the values of QuantizeDequantize.get_scale and
    _get_offset (quantizer.py:345-464) bit for bit, and their gradients by the same autograd
    rules, without the chain of one-element tensor operations."""

    @staticmethod
    def forward(ctx, mn, mx, qmin: int, qmax: int, symmetric: bool, min_scale: float,
                sym_offset: float):
        scale = torch.empty_like(mn)
        offset = torch.empty_like(mn)
        _rx.call("rxmet_qdq_encoding_forward", _rx.ptr(mn), _rx.ptr(mx), mn.numel(), int(qmin),
                 int(qmax), int(bool(symmetric)), float(sym_offset), float(min_scale),
                 _rx.ptr(scale), _rx.ptr(offset), _rx.stream_of(mn.device))
        ctx.save_for_backward(mn, mx)
        ctx.args = (int(qmin), int(qmax), bool(symmetric), float(min_scale))
        if symmetric:
            ctx.mark_non_differentiable(offset)
        return scale, offset

    @staticmethod
    def backward(ctx, g_scale, g_offset):
        mn, mx = ctx.saved_tensors
        qmin, qmax, symmetric, min_scale = ctx.args
        gs = g_scale.contiguous() if g_scale is not None else None
        go = g_offset.contiguous() if (g_offset is not None and not symmetric) else None
        d_min, d_max = torch.empty_like(mn), torch.empty_like(mx)
        _rx.call("rxmet_qdq_encoding_backward", _rx.ptr(mn), _rx.ptr(mx), _rx.ptr(gs), _rx.ptr(go),
                 mn.numel(), qmin, qmax, int(symmetric), min_scale, _rx.ptr(d_min), _rx.ptr(d_max),
                 _rx.stream_of(mn.device))
        return d_min, d_max, None, None, None, None, None


def minmax_encodings(mn: torch.Tensor, mx: torch.Tensor, qmin: int, qmax: int, symmetric: bool,
                     min_scale: float, sym_offset: float):
    """Fused (scale, offset) of contiguous CUDA float32 min/max tensors."""
    return _MinMaxEncodings.apply(mn, mx, qmin, qmax, symmetric, min_scale, sym_offset)
