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
# Layout: map (tensor shape, encoding shape) onto the kernels' [outer, C, inner] view.
# ---------------------------------------------------------------------------------


def kernel_layout(tensor_shape, enc_shape) -> Optional[Tuple[int, int, int]]:
    """Return (outer, C, inner) with encoding index (i // inner) % C for row-major
    element i, or None when the encoding axes are not one contiguous span."""
    tensor_shape = tuple(int(d) for d in tensor_shape)
    nd = len(tensor_shape)
    enc = (1,) * (nd - len(enc_shape)) + tuple(int(d) for d in enc_shape)
    numel = math.prod(tensor_shape)
    axes = [a for a in range(nd) if enc[a] != 1]
    if not axes:
        return 1, 1, numel
    a0, a1 = axes[0], axes[-1]
    for a in range(a0, a1 + 1):
        if enc[a] == 1 and tensor_shape[a] != 1:
            return None
        if enc[a] != 1 and enc[a] != tensor_shape[a]:
            return None
    outer = math.prod(tensor_shape[:a0])
    C = math.prod(tensor_shape[a0:a1 + 1])
    inner = math.prod(tensor_shape[a1 + 1:])
    return outer, C, inner


def _require(tensor: torch.Tensor, what: str):
    if not tensor.is_cuda:
        raise RuntimeError(f"mi355x backend: {what} must be a GPU tensor")
    if tensor.dtype != torch.float32:
        raise NotImplementedError(
            f"mi355x backend: {what} must be float32 (got {tensor.dtype})")


def _enc_vector(t: Optional[torch.Tensor], like: torch.Tensor, C: int) -> Optional[torch.Tensor]:
    if t is None:
        return None
    v = t.detach().to(device=like.device, dtype=torch.float32).reshape(-1)
    if v.numel() == 1 and C != 1:
        v = v.expand(C)
    return v.contiguous()


def _workspace(outer: int, C: int, inner: int, device) -> torch.Tensor:
    nbytes = int(_rx.load().rxmet_qdq_workspace_bytes(outer, C, inner))
    return torch.empty(max(nbytes, 16), dtype=torch.uint8, device=device)


def _plan(tensor: torch.Tensor, scale: torch.Tensor):
    layout = kernel_layout(tensor.shape, scale.shape)
    if layout is None:
        raise NotImplementedError(
            f"mi355x backend: encodings of shape {tuple(scale.shape)} over a tensor of shape "
            f"{tuple(tensor.shape)} span non-adjacent axes")
    return layout


# ---------------------------------------------------------------------------------
# Autograd functions — each direction is one kernel launch (+ a tiny fold kernel).
# ---------------------------------------------------------------------------------


class _QuantDequant(torch.autograd.Function):
    """QuantDequantFunc (torch_builtins.py:618-691) or the fake_quantize fast path."""

    @staticmethod
    def forward(ctx, x, scale, offset, qmin: int, qmax: int, mode: int):
        _require(x, "tensor")
        x_c = x.contiguous()
        outer, C, inner = _plan(x_c, scale)
        s = _enc_vector(scale, x_c, C)
        o = _enc_vector(offset, x_c, C)
        y = torch.empty_like(x_c)
        _rx.call("rxmet_qdq_forward", _rx.ptr(x_c), _rx.ptr(y), outer, C, inner, _rx.ptr(s),
                 _rx.ptr(o), int(qmin), int(qmax), int(mode), _rx.stream_of(x_c.device))
        ctx.layout = (outer, C, inner)
        ctx.qmin, ctx.qmax, ctx.mode = int(qmin), int(qmax), int(mode)
        ctx.scale_shape = scale.shape
        ctx.offset_shape = None if offset is None else offset.shape
        ctx.save_for_backward(x_c, s, o)
        return y

    @staticmethod
    def backward(ctx, g):
        x, s, o = ctx.saved_tensors
        outer, C, inner = ctx.layout
        need_x, need_s, need_o = ctx.needs_input_grad[:3]
        g = g.contiguous()
        dx = torch.empty_like(x)
        learn = ctx.mode == LEARNABLE
        ds = torch.empty(C, dtype=torch.float32, device=x.device) if (need_s and learn) else None
        do = torch.empty(C, dtype=torch.float32, device=x.device) if (need_o and learn) else None
        ws = _workspace(outer, C, inner, x.device) if (ds is not None or do is not None) else None
        _rx.call("rxmet_qdq_backward", _rx.ptr(x), _rx.ptr(g), _rx.ptr(dx), _rx.ptr(ds), _rx.ptr(do),
                 outer, C, inner, _rx.ptr(s), _rx.ptr(o), ctx.qmin, ctx.qmax, ctx.mode,
                 _rx.ptr(ws), _rx.stream_of(x.device))
        ds = None if ds is None else ds.view(ctx.scale_shape)
        do = None if do is None else do.view(ctx.offset_shape)
        return (dx if need_x else None), ds, do, None, None, None


class _Quantize(torch.autograd.Function):
    """QuantizeFunc (torch_builtins.py:505-571)."""

    @staticmethod
    def forward(ctx, x, scale, offset, qmin: int, qmax: int):
        _require(x, "tensor")
        x_c = x.contiguous()
        outer, C, inner = _plan(x_c, scale)
        s = _enc_vector(scale, x_c, C)
        o = _enc_vector(offset, x_c, C)
        q = torch.empty_like(x_c)
        _rx.call("rxmet_quantize_forward", _rx.ptr(x_c), _rx.ptr(q), outer, C, inner, _rx.ptr(s),
                 _rx.ptr(o), int(qmin), int(qmax), _rx.stream_of(x_c.device))
        ctx.layout = (outer, C, inner)
        ctx.qmin, ctx.qmax = int(qmin), int(qmax)
        ctx.scale_shape = scale.shape
        ctx.offset_shape = None if offset is None else offset.shape
        ctx.save_for_backward(x_c, s, o)
        return q

    @staticmethod
    def backward(ctx, g):
        x, s, o = ctx.saved_tensors
        outer, C, inner = ctx.layout
        need_x, need_s, need_o = ctx.needs_input_grad[:3]
        g = g.contiguous()
        dx = torch.empty_like(x)
        ds = torch.empty(C, dtype=torch.float32, device=x.device) if need_s else None
        do = torch.empty(C, dtype=torch.float32, device=x.device) if need_o else None
        ws = _workspace(outer, C, inner, x.device) if (need_s or need_o) else None
        _rx.call("rxmet_quantize_backward", _rx.ptr(x), _rx.ptr(g), _rx.ptr(dx), _rx.ptr(ds),
                 _rx.ptr(do), outer, C, inner, _rx.ptr(s), _rx.ptr(o), ctx.qmin, ctx.qmax,
                 _rx.ptr(ws), _rx.stream_of(x.device))
        ds = None if ds is None else ds.view(ctx.scale_shape)
        do = None if do is None else do.view(ctx.offset_shape)
        return (dx if need_x else None), ds, do, None, None


class _Dequantize(torch.autograd.Function):
    """DequantizeFunc (torch_builtins.py:574-615)."""

    @staticmethod
    def forward(ctx, q, scale, offset):
        _require(q, "tensor")
        q_c = q.contiguous()
        outer, C, inner = _plan(q_c, scale)
        s = _enc_vector(scale, q_c, C)
        o = _enc_vector(offset, q_c, C)
        y = torch.empty_like(q_c)
        _rx.call("rxmet_dequantize_forward", _rx.ptr(q_c), _rx.ptr(y), outer, C, inner,
                 _rx.ptr(s), _rx.ptr(o), _rx.stream_of(q_c.device))
        ctx.layout = (outer, C, inner)
        ctx.scale_shape = scale.shape
        ctx.offset_shape = None if offset is None else offset.shape
        ctx.save_for_backward(q_c, s, o)
        return y

    @staticmethod
    def backward(ctx, g):
        q, s, o = ctx.saved_tensors
        outer, C, inner = ctx.layout
        need_q, need_s, need_o = ctx.needs_input_grad[:3]
        g = g.contiguous()
        dq = torch.empty_like(q)
        ds = torch.empty(C, dtype=torch.float32, device=q.device) if need_s else None
        do = torch.empty(C, dtype=torch.float32, device=q.device) if need_o else None
        ws = _workspace(outer, C, inner, q.device) if (need_s or need_o) else None
        _rx.call("rxmet_dequantize_backward", _rx.ptr(q), _rx.ptr(g), _rx.ptr(dq), _rx.ptr(ds),
                 _rx.ptr(do), outer, C, inner, _rx.ptr(s), _rx.ptr(o), _rx.ptr(ws),
                 _rx.stream_of(q.device))
        ds = None if ds is None else ds.view(ctx.scale_shape)
        do = None if do is None else do.view(ctx.offset_shape)
        return (dq if need_q else None), ds, do


# ---------------------------------------------------------------------------------
# Backend protocol
# ---------------------------------------------------------------------------------


def _check_fp32_grid(dtype, qmin, qmax):
    if not _is_numerically_stable(dtype, qmin, qmax):
        raise NotImplementedError(
            f"mi355x backend: grid [{qmin}, {qmax}] needs float64 internals (fp32 kernels only)")
    if not _is_grid_representable(dtype, qmin, qmax):
        raise RuntimeError(f"{dtype} is unable to represent quantized output of range [{qmin}, {qmax}].")


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


def quantize(tensor: torch.Tensor, scale: torch.Tensor, offset: torch.Tensor, qmin: int, qmax: int,
             block_size: Optional[List] = None) -> torch.Tensor:
    """Differentiable quantization (torch_builtins.quantize, :151-194)."""
    _validate_arguments(tensor, scale, qmin, qmax, block_size)
    _require(tensor, "tensor")
    if not _is_grid_representable(tensor.dtype, qmin, qmax):
        raise RuntimeError(
            f"{tensor.dtype} is unable to represent quantized output of range [{qmin}, {qmax}].")
    _check_fp32_grid(tensor.dtype, qmin, qmax)
    orig_shape = tensor.shape
    t = reshape_tensor_for_blocks(tensor, scale.shape, block_size)
    s = scale.view(get_encoding_shape_with_blocks(scale.shape, block_size))
    o = offset.view(get_encoding_shape_with_blocks(offset.shape, block_size))
    return _Quantize.apply(t, s.to(torch.float32), o.to(torch.float32), qmin, qmax).view(orig_shape)


def dequantize(tensor: torch.Tensor, scale: torch.Tensor, offset: torch.Tensor,
               block_size: Optional[List] = None) -> torch.Tensor:
    """Differentiable dequantization (torch_builtins.dequantize, :459-488)."""
    _validate_arguments(tensor, scale, block_size=block_size)
    _require(tensor, "tensor")
    orig_shape = tensor.shape
    t = reshape_tensor_for_blocks(tensor, scale.shape, block_size)
    s = scale.view(get_encoding_shape_with_blocks(scale.shape, block_size))
    o = offset.view(get_encoding_shape_with_blocks(offset.shape, block_size))
    return _Dequantize.apply(t, s.to(torch.float32), o.to(torch.float32)).view(orig_shape)


def quantize_dequantize(tensor: torch.Tensor, scale: torch.Tensor, offset: torch.Tensor, qmin: int,
                        qmax: int, block_size: Optional[List] = None,
                        zero_point_shift: float = 0.0) -> torch.Tensor:
    """Differentiable fake quantization (torch_builtins.quantize_dequantize, :199-284)."""
    _validate_arguments(tensor, scale, qmin, qmax, block_size)
    _require(tensor, "tensor")
    if zero_point_shift != 0.0:
        raise NotImplementedError("mi355x backend: zero_point_shift is not supported yet")
    fast = block_size is None and not torch.jit.is_tracing()
    fast &= ((not scale.requires_grad and not getattr(offset, "requires_grad", False))
             or not torch.is_grad_enabled())
    if fast and _fast_path_layout(scale, offset, tensor, qmin, qmax):
        if scale.dtype != torch.float32:
            scale = scale.to(torch.float32)
        return _QuantDequant.apply(tensor, scale, offset.to(torch.float32), int(qmin), int(qmax),
                                   FROZEN)
    _check_fp32_grid(tensor.dtype, qmin, qmax)
    orig_shape = tensor.shape
    t = reshape_tensor_for_blocks(tensor, scale.shape, block_size)
    s = scale.view(get_encoding_shape_with_blocks(scale.shape, block_size)).to(torch.float32)
    o = offset.view(get_encoding_shape_with_blocks(offset.shape, block_size)).to(torch.float32)
    return _QuantDequant.apply(t, s, o, int(qmin), int(qmax), LEARNABLE).view(orig_shape)


def minmax(tensor: torch.Tensor, enc_shape) -> Tuple[torch.Tensor, torch.Tensor]:
    """Min and max of ``tensor`` reduced to ``enc_shape`` (NaN propagates).

    Kernel of ``_MinMaxObserver.collect_stats`` (encoding_analyzer.py:101-105)."""
    _require(tensor, "tensor")
    x = tensor.contiguous()
    layout = kernel_layout(x.shape, enc_shape)
    if layout is None:
        raise NotImplementedError(
            f"mi355x backend: cannot reduce shape {tuple(x.shape)} to {tuple(enc_shape)}")
    outer, C, inner = layout
    mn = torch.empty(C, dtype=torch.float32, device=x.device)
    mx = torch.empty(C, dtype=torch.float32, device=x.device)
    ws = _workspace(outer, C, inner, x.device)
    _rx.call("rxmet_qdq_minmax", _rx.ptr(x), outer, C, inner, _rx.ptr(mn), _rx.ptr(mx), _rx.ptr(ws),
             _rx.stream_of(x.device))
    return mn.view(tuple(enc_shape)), mx.view(tuple(enc_shape))


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
