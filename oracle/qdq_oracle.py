"""CPU oracle for the fake-quantization (QuantizeDequantize) path — TEST INFRASTRUCTURE.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg use
this module, and only as the checker / CPU baseline.  The product path never imports it.

numpy restatement of aimet_torch's fake-quantization numerics, fp32 arithmetic with
IEEE round-half-to-even (``np.rint``) and fp64 accumulation of encoding gradients:

* ``qdq_frozen``      — torch.fake_quantize_per_{tensor,channel}_affine as called by the
  frozen-encoding fast path (torch_builtins.py:287-361): ``q = rint(x * fl(1/s)) + zp``,
  ``y = (clamp(q) - zp) * s``, NaN restored (:249), +-inf saturated (the grid contract of
  tests/integration/test_native_qdq_alignment.py:139-147).
* ``qdq_learnable``   — QuantDequantFunc.forward (torch_builtins.py:640-672).
* ``qdq_learnable_backward`` — QuantDequantFunc.backward (:675-691) followed by the
  reduction of the broadcast scale/offset gradients to the encoding shape.
* ``quantize`` / ``quantize_backward`` — QuantizeFunc (:505-571).
* ``dequantize`` / ``dequantize_backward`` — DequantizeFunc (:574-615).
* ``minmax``          — _MinMaxObserver.collect_stats (encoding_analyzer.py:101-105).
* ``compute_encodings_from_stats`` — MinMaxEncodingAnalyzer (encoding_analyzer.py:217-272).
* ``scale_offset``    — get_scale / _get_offset (quantizer.py:345-403).
* ``native_qdq``      — the native libpymo form, DlQuantization::stableQuantizeDequantize
  (native/common/src/quantize_dequantize.hpp:35-46): clip in value space, multiply by the
  correctly rounded reciprocal of the scale, round half to even, times the scale.

Pinned by tests/test_qdq_oracle.py against: torch's own fake_quantize kernels (the
reference's frozen path, third-party, exact); the reference's docstring tables
(backends/__init__.py:169-187, 336-354); the ties-to-even, reciprocal and saturation
tables of test_native_qdq_alignment.py:94-147; and an independent autograd derivation
of the STE gradients (torch autograd through a straight-through surrogate).
"""
from __future__ import annotations

import math

import numpy as np

f32 = np.float32


def layout_view(x: np.ndarray, outer: int, C: int, inner: int) -> np.ndarray:
    """View x as [outer, C, inner]."""
    return x.reshape(outer, C, inner)


def _bcast(v, C):
    v = np.asarray(v, dtype=f32).reshape(-1)
    if v.size == 1 and C != 1:
        v = np.full(C, v[0], dtype=f32)
    return v.reshape(1, C, 1)


def _clamp_keep_nan(v, lo, hi):
    out = np.where(v < lo, lo, np.where(v > hi, hi, v))
    return out.astype(f32)


def qdq_frozen(x, scale, offset, qmin, qmax, layout):
    outer, C, inner = layout
    xv = layout_view(np.asarray(x, dtype=f32), outer, C, inner)
    s = _bcast(scale, C)
    inv_s = (f32(1.0) / s).astype(f32)
    zp = -np.trunc(_bcast(offset, C)).astype(f32)
    with np.errstate(invalid="ignore", over="ignore"):
        r = (np.rint((xv * inv_s).astype(f32)) + zp).astype(f32)
        q = _clamp_keep_nan(r, f32(qmin), f32(qmax))
        y = ((q - zp).astype(f32) * s).astype(f32)
        mask = (r >= qmin) & (r <= qmax)
    return y.reshape(np.shape(x)), mask.reshape(np.shape(x))


def qdq_learnable(x, scale, offset, qmin, qmax, layout):
    outer, C, inner = layout
    xv = layout_view(np.asarray(x, dtype=f32), outer, C, inner)
    s = _bcast(scale, C)
    o = _bcast(offset, C)
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        r = (np.rint((xv / s).astype(f32)) - o).astype(f32)
        mask = (r >= qmin) & (r <= qmax)
        q = _clamp_keep_nan(r, f32(qmin), f32(qmax))
        y = ((q + o).astype(f32) * s).astype(f32)
    return y.reshape(np.shape(x)), mask.reshape(np.shape(x))


def qdq_learnable_backward(x, g, scale, offset, qmin, qmax, layout):
    """Return (dx, dscale[C], doffset[C]); sums accumulated in fp64."""
    outer, C, inner = layout
    xv = layout_view(np.asarray(x, dtype=f32), outer, C, inner)
    gv = layout_view(np.asarray(g, dtype=f32), outer, C, inner)
    s = _bcast(scale, C)
    o = _bcast(offset, C)
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        xs = (xv / s).astype(f32)
        rr = np.rint(xs).astype(f32)
        r = (rr - o).astype(f32)
        m = ((r >= qmin) & (r <= qmax)).astype(f32)
        dx = (gv * m).astype(f32)
        lo = (o + f32(qmin)).astype(f32)
        hi = (o + f32(qmax)).astype(f32)
        ds_el = (gv * (_clamp_keep_nan(rr, lo, hi) - (xs * m).astype(f32)).astype(f32)).astype(f32)
        do_el = (gv * ((f32(1.0) - m) * s).astype(f32)).astype(f32)
    ds = ds_el.astype(np.float64).sum(axis=(0, 2))
    do = do_el.astype(np.float64).sum(axis=(0, 2))
    return dx.reshape(np.shape(x)), ds.astype(f32), do.astype(f32)


def native_qdq(x, minimum, maximum, scale, dtype=np.float32, noise=None):
    """stableQuantizeDequantize (quantize_dequantize.hpp:35-46) in `dtype` (float or double):
    NaN is returned as is; the value is clipped to [minimum, maximum]
    (``fmax(fmin(v, max), min)``), multiplied by ``qdqReciprocal(scale)`` = the correctly
    rounded 1 / scale (:15-29), rounded half to even (``nearbyint``) — or ``floor(scaled +
    noise)`` when a stochastic noise array is given — and multiplied by the scale.  minimum,
    maximum and scale broadcast against x (per-channel encodings)."""
    dt = np.dtype(dtype)
    v = np.asarray(x, dtype=dt)
    lo, hi, sc = (np.asarray(a, dtype=dt) for a in (minimum, maximum, scale))
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        clipped = np.fmax(np.fmin(v, hi), lo)  # fmin/fmax return the other operand for NaN
        scaled = (clipped * (dt.type(1) / sc).astype(dt)).astype(dt)
        if noise is None:
            rounded = np.rint(scaled)
        else:
            rounded = np.floor((scaled + np.asarray(noise, dtype=dt)).astype(dt))
        out = (rounded * sc).astype(dt)
    return np.where(np.isnan(v), v, out).astype(dt)


def qdq_frozen_backward(x, g, scale, offset, qmin, qmax, layout):
    _, mask = qdq_frozen(x, scale, offset, qmin, qmax, layout)
    return (np.asarray(g, dtype=f32) * mask.astype(f32)).astype(f32)


def quantize(x, scale, offset, qmin, qmax, layout):
    outer, C, inner = layout
    xv = layout_view(np.asarray(x, dtype=f32), outer, C, inner)
    s, o = _bcast(scale, C), _bcast(offset, C)
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        r = (np.rint((xv / s).astype(f32)) - o).astype(f32)
        q = _clamp_keep_nan(r, f32(qmin), f32(qmax))
    return q.reshape(np.shape(x))


def quantize_backward(x, g, scale, offset, qmin, qmax, layout):
    outer, C, inner = layout
    xv = layout_view(np.asarray(x, dtype=f32), outer, C, inner)
    gv = layout_view(np.asarray(g, dtype=f32), outer, C, inner)
    s, o = _bcast(scale, C), _bcast(offset, C)
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        r = (np.rint((xv / s).astype(f32)) - o).astype(f32)
        m = ((r >= qmin) & (r <= qmax)).astype(f32)
        mg = (gv * m).astype(f32)
        gs = (mg / s).astype(f32)
        ds_el = (-gs * (xv / s).astype(f32)).astype(f32)
    ds = ds_el.astype(np.float64).sum(axis=(0, 2))
    do = (-mg).astype(np.float64).sum(axis=(0, 2))
    return gs.reshape(np.shape(x)), ds.astype(f32), do.astype(f32)


def dequantize(q, scale, offset, layout):
    outer, C, inner = layout
    qv = layout_view(np.asarray(q, dtype=f32), outer, C, inner)
    s, o = _bcast(scale, C), _bcast(offset, C)
    return ((qv + o).astype(f32) * s).astype(f32).reshape(np.shape(q))


def dequantize_backward(q, g, scale, offset, layout):
    outer, C, inner = layout
    qv = layout_view(np.asarray(q, dtype=f32), outer, C, inner)
    gv = layout_view(np.asarray(g, dtype=f32), outer, C, inner)
    s, o = _bcast(scale, C), _bcast(offset, C)
    gs = (gv * s).astype(f32)
    ds = (gv * (qv + o).astype(f32)).astype(f32).astype(np.float64).sum(axis=(0, 2))
    do = gs.astype(np.float64).sum(axis=(0, 2))
    return gs.reshape(np.shape(q)), ds.astype(f32), do.astype(f32)


def minmax(x, layout):
    outer, C, inner = layout
    xv = layout_view(np.asarray(x, dtype=f32), outer, C, inner)
    # np.min/np.max propagate NaN like torch.min/torch.max.
    return xv.min(axis=(0, 2)).astype(f32), xv.max(axis=(0, 2)).astype(f32)


# ---------------------------------------------------------------------------------
# Encoding math (fp32, same operation order as the reference)
# ---------------------------------------------------------------------------------


def minimum_scale(num_steps: int) -> float:
    """aimet_common/quantsim.py:447-480."""
    raw = min(float(np.finfo(np.float32).eps), 0.01 / num_steps)
    return float(2.0 ** math.ceil(math.log2(raw)))


def sdiv(a, b, gpu_scalar_div: bool):
    """``tensor / python_scalar`` as PyTorch evaluates it: a true fp32 division on the
    CPU, but a multiplication by the fp32 reciprocal fl(1/b) on the GPU (aten's
    div_true kernel for a CPU-scalar divisor).  The reference's encoding math therefore
    depends on the device its quantizer lives on; pass the device it ran on."""
    a = np.asarray(a, dtype=f32)
    if gpu_scalar_div:
        return (a * f32(f32(1.0) / f32(b))).astype(f32)
    return (a / f32(b)).astype(f32)


def compute_encodings_from_stats(mn, mx, num_steps: int, is_symmetric: bool,
                                 gpu_scalar_div: bool = False):
    """MinMaxEncodingAnalyzer.compute_encodings_from_stats (encoding_analyzer.py:217-272)."""
    mn = np.asarray(mn, dtype=f32)
    mx = np.asarray(mx, dtype=f32)
    ms = f32(minimum_scale(num_steps))
    mn0 = np.minimum(mn, f32(0))
    mx0 = np.maximum(mx, f32(0))
    diff = sdiv(mx0 - mn0, num_steps, gpu_scalar_div)
    adj = (ms * (diff < ms).astype(f32)).astype(f32)
    if is_symmetric:
        npos, nneg = num_steps // 2, -(-num_steps // 2)
        umax = (mx0 + f32(npos) * adj).astype(f32)
        umin = (mn0 - f32(nneg) * adj).astype(f32)
        extra = 1 if num_steps == 3 else 0
        delta = np.maximum(sdiv(umax, npos + extra, gpu_scalar_div),
                           sdiv(-umin, nneg, gpu_scalar_div))
        umin = (f32(-nneg) * delta).astype(f32)
        umax = (f32(npos) * delta).astype(f32)
    else:
        umax = (mx0 + f32(num_steps) * adj).astype(f32)
        umin = mn0
    fmax = np.finfo(np.float32).max
    return np.maximum(umin, -fmax).astype(f32), np.minimum(umax, fmax).astype(f32)


def scale_offset(mn, mx, qmin: int, qmax: int, symmetric: bool, gpu_scalar_div: bool = False):
    """get_scale / _get_offset of a min/max-parametrised quantizer (quantizer.py:345-403)."""
    mn = np.asarray(mn, dtype=f32)
    mx = np.asarray(mx, dtype=f32)
    num_steps = qmax - qmin
    s = np.abs(sdiv(mx - mn, num_steps, gpu_scalar_div))
    s = np.maximum(s, f32(minimum_scale(num_steps))).astype(f32)
    if symmetric:
        o = np.full_like(s, f32(0 if qmin >= 0 else -round((qmin + qmax) / 2)))
    else:
        o = np.clip(np.rint((mn / s).astype(f32)) - f32(qmin), -qmax, -qmin).astype(f32)
    return s, o


# ---------------------------------------------------------------------------------
# torch-on-CPU forms, for the CPU baseline (all intra-op threads)
# ---------------------------------------------------------------------------------


def torch_learnable_step(torch, x, g, scale, offset, qmin: int, qmax: int):
    """QuantDequantFunc forward + backward (torch_builtins.py:640-691) as aten operations on
    CPU tensors, the encoding gradients summed to the scale's shape as autograd does.
    Returns (y, dx, dscale, doffset).  The same arithmetic as ``qdq_learnable`` and
    ``qdq_learnable_backward`` (fp32 elementwise); the sums use aten's reduction order."""
    xs = x / scale
    rr = torch.round(xs)
    r = rr - offset
    mask = (r >= qmin) & (r <= qmax)
    y = (r.clamp(qmin, qmax) + offset) * scale
    mf = mask.to(x.dtype)
    dx = g * mf
    lo, hi = offset + qmin, offset + qmax
    ds = (g * (torch.maximum(torch.minimum(rr, hi), lo) - xs * mf)).sum_to_size(scale.shape)
    do = (g * ((1.0 - mf) * scale)).sum_to_size(offset.shape)
    return y, dx, ds, do


def torch_frozen_step(torch, x, g, scale: float, zero_point: int, qmin: int, qmax: int):
    """The frozen-encoding path (torch_builtins.py:287-361): aten's
    fake_quantize_per_tensor_affine forward and its STE backward, on CPU tensors."""
    xg = x.detach().requires_grad_(True)
    y = torch.fake_quantize_per_tensor_affine(xg, scale, zero_point, qmin, qmax)
    y.backward(g)
    return y.detach(), xg.grad


# ---------------------------------------------------------------------------------
# General numerics: fp16 / bf16 tensors, the reference's internal arithmetic type, the
# zero-point shift, and encodings of any broadcastable shape.
#
# torch_builtins.quantize_dequantize (:199-284) computes in an internal type R (the tensor's
# type, widened to fp32 or fp64 while the grid is not numerically stable in it, :255-262)
# and returns the result in the tensor's type T.  PyTorch evaluates each elementwise
# operation on 16-bit tensors in fp32 and rounds the result to the storage type; these
# functions do the same with numpy: every operation in fp32 (fp64 when R is fp64), its
# result rounded to R.  Shapes follow torch broadcasting: x of any shape, scale/offset
# broadcastable to it, encoding gradients summed back to the broadcast encoding shape in
# fp64 (the reference sums in R; the sums here are then rounded to R).
#
# On the GPU a 0-dim scale tensor next to a T tensor makes PyTorch evaluate the operation
# in T with the scale rounded to T (``scalar_scale``): the shift's subtraction (:277) and
# QuantizeFunc.backward's tensor / scale (:567).  The CPU tensor iterator instead reads a
# 0-dim operand at its original precision, so the CPU cannot stand in for this case; the
# GPU tests check it against torch on the GPU.
# ---------------------------------------------------------------------------------

f64 = np.float64
TYPES = ("f32", "f16", "bf16", "f64")


def round_to(v, dt: str):
    """Values rounded to type ``dt``, returned as float32 (float64 for "f64")."""
    if dt == "f64":
        return np.asarray(v, dtype=f64)
    v = np.asarray(v, dtype=f32)
    if dt == "f32":
        return v
    if dt == "f16":
        return v.astype(np.float16).astype(f32)
    if dt == "bf16":
        u = v.view(np.uint32).astype(np.uint64)
        r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
        out = r.astype(np.uint32).view(f32)
        return np.where(np.isnan(v), f32(np.nan), out).astype(f32)
    raise ValueError(dt)


def to_io(v, io: str):
    """The final ``.to(T)``: fp64 results pass through fp32 on their way to 16-bit types,
    as PyTorch's conversions do."""
    v = np.asarray(v)
    if v.dtype == f64:
        v = v.astype(f32)
    return round_to(v, io)


def _ctype(internal: str):
    return f64 if internal == "f64" else f32


def _sum_to(el, shape):
    """Sum fp64 terms over the axes broadcast from ``shape`` (torch's sum_to_size)."""
    el = np.asarray(el, dtype=f64)
    nd = el.ndim
    shape = (1,) * (nd - len(shape)) + tuple(shape)
    axes = tuple(a for a in range(nd) if shape[a] == 1 and el.shape[a] != 1)
    return el.sum(axis=axes, keepdims=True).reshape(shape)


def _check_shift(shift):
    # x - shift * s and y + shift * s are evaluated as fused multiply-adds on the GPU; a
    # power-of-two shift (the quantizers allow 0.5) makes the product exact, so one rounding
    # of the sum is the result either way
    if shift != 0.0:
        m, _ = math.frexp(abs(shift))
        assert m == 0.5, "power-of-two zero_point_shift only"


def _shifted(x, s, shift, io, internal, scalar_scale):
    A = _ctype(internal)
    if shift == 0.0:
        return np.asarray(x, dtype=A)
    if scalar_scale:
        s_io = round_to(np.asarray(s, dtype=f32), io)
        return round_to((np.asarray(x, f32) - (f32(shift) * s_io).astype(f32)).astype(f32),
                        io).astype(A)
    return round_to((np.asarray(x, A) - (A(shift) * np.asarray(s, A)).astype(A)).astype(A),
                    internal)


def qdq_general(x, scale, offset, qmin, qmax, io="f32", internal="f32", shift=0.0,
                scalar_scale=False):
    """quantize_dequantize forward, learnable path (QuantDequantFunc :640-672, with the
    shift of :276-284).  ``x`` holds values of type ``io``; scale/offset hold the values of
    scale.to(R) / offset.to(R).  Returns (y as ``io`` values, mask)."""
    _check_shift(shift)
    A = _ctype(internal)

    def r(v):
        return round_to(np.asarray(v, A), internal)

    s, o = np.asarray(scale, A), np.asarray(offset, A)
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        v = _shifted(x, scale, shift, io, internal, scalar_scale)
        t = r(v / s)
        q = r(np.rint(t) - o)
        mask = (q >= qmin) & (q <= qmax)
        c = np.where(q < qmin, A(qmin), np.where(q > qmax, A(qmax), q)).astype(A)
        y = r(r(c + o) * s)
        if shift != 0.0:
            y = r(y + (A(shift) * s).astype(A))
    return to_io(y, io), mask


def qdq_general_backward(x, g, scale, offset, qmin, qmax, io="f32", internal="f32", shift=0.0,
                         scalar_scale=False):
    """QuantDequantFunc.backward (:675-691) plus the shift's scale terms; returns
    (dx as ``io`` values, dscale, doffset) with the encoding gradients in the broadcast
    encoding shape, summed in fp64 and rounded to R."""
    _check_shift(shift)
    A = _ctype(internal)

    def r(v):
        return round_to(np.asarray(v, A), internal)

    s, o = np.asarray(scale, A), np.asarray(offset, A)
    enc_shape = np.broadcast_shapes(np.shape(scale), np.shape(offset))
    ga = np.asarray(g, A)
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        v = _shifted(x, scale, shift, io, internal, scalar_scale)
        t = r(v / s)
        rr = np.rint(t)
        q = r(rr - o)
        m = ((q >= qmin) & (q <= qmax)).astype(A)
        lo, hi = r(o + A(qmin)), r(o + A(qmax))
        cl = np.where(rr < lo, lo, np.where(rr > hi, hi, rr)).astype(A)
        ds_el = r(ga * r(cl - (t * m).astype(A))).astype(f64)
        if shift != 0.0:
            ds_el = ds_el + f64(shift) * (ga * (A(1) - m)).astype(f64)
        do_el = r(ga * r((A(1) - m) * s)).astype(f64)
        dx = (ga * m).astype(A)
    ds = round_to(_sum_to(ds_el, enc_shape).astype(f32), internal)
    do = round_to(_sum_to(do_el, enc_shape).astype(f32), internal)
    return to_io(dx, io), np.asarray(ds, f32), np.asarray(do, f32)


def qdq_frozen_general(x, scale, offset, qmin, qmax, io="f32"):
    """The fast path for any io type: torch.fake_quantize computes in fp32 and stores the
    result in the tensor's type (torch_builtins.py:287-361)."""
    xs = np.asarray(x, f32)
    s = np.asarray(scale, f32)
    inv_s = (f32(1.0) / s).astype(f32)
    zp = -np.trunc(np.asarray(offset, f32)).astype(f32)
    with np.errstate(invalid="ignore", over="ignore"):
        q = (np.rint((xs * inv_s).astype(f32)) + zp).astype(f32)
        mask = (q >= qmin) & (q <= qmax)
        c = np.where(q < qmin, f32(qmin), np.where(q > qmax, f32(qmax), q)).astype(f32)
        y = ((c - zp).astype(f32) * s).astype(f32)
    return round_to(y, io), mask


def quantize_general(x, scale, offset, qmin, qmax, io="f32", internal="f32"):
    """QuantizeFunc.forward (:527-552) in R, stored in T."""
    A = _ctype(internal)

    def r(v):
        return round_to(np.asarray(v, A), internal)

    s, o = np.asarray(scale, A), np.asarray(offset, A)
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        q = r(np.rint(r(np.asarray(x, A) / s)) - o)
        c = np.where(q < qmin, A(qmin), np.where(q > qmax, A(qmax), q)).astype(A)
    return to_io(c, io)


def quantize_general_backward(x, g, scale, offset, qmin, qmax, io="f32", internal="f32",
                              scalar_scale=False):
    """QuantizeFunc.backward (:555-571): dx = fl(g*mask/s), dscale = sum -(g*mask/s)*(x/s),
    doffset = sum -g*mask, each operation rounded to R (x/s in T when the scale is 0-dim)."""
    A = _ctype(internal)

    def r(v):
        return round_to(np.asarray(v, A), internal)

    s, o = np.asarray(scale, A), np.asarray(offset, A)
    enc_shape = np.broadcast_shapes(np.shape(scale), np.shape(offset))
    ga = np.asarray(g, A)
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        t = r(np.asarray(x, A) / s)
        q = r(np.rint(t) - o)
        m = ((q >= qmin) & (q <= qmax)).astype(A)
        mg = (ga * m).astype(A)
        gs = r(mg / s)
        if scalar_scale:
            s_io = round_to(np.asarray(scale, f32), io)
            xs = round_to((np.asarray(x, f32) / s_io).astype(f32), io).astype(A)
        else:
            xs = t
        ds_el = r(-gs * xs).astype(f64)
        do_el = (-mg).astype(f64)
    ds = round_to(_sum_to(ds_el, enc_shape).astype(f32), internal)
    do = round_to(_sum_to(do_el, enc_shape).astype(f32), internal)
    return to_io(gs, io), np.asarray(ds, f32), np.asarray(do, f32)


def dequantize_general(q, scale, offset, io="f32"):
    """DequantizeFunc.forward (:589-603) in the tensor's type."""
    def r(v):
        return round_to(np.asarray(v, f32), io)

    return r(r(np.asarray(q, f32) + np.asarray(offset, f32)) * np.asarray(scale, f32))


def dequantize_general_backward(q, g, scale, offset, io="f32"):
    """DequantizeFunc.backward (:607-615) in the tensor's type."""
    def r(v):
        return round_to(np.asarray(v, f32), io)

    s, o = np.asarray(scale, f32), np.asarray(offset, f32)
    enc_shape = np.broadcast_shapes(np.shape(scale), np.shape(offset))
    ga = np.asarray(g, f32)
    gs = r(ga * s)
    ds = round_to(_sum_to(r(ga * r(np.asarray(q, f32) + o)), enc_shape).astype(f32), io)
    do = round_to(_sum_to(gs, enc_shape).astype(f32), io)
    return gs, np.asarray(ds, f32), np.asarray(do, f32)


def minmax_general(x, enc_shape):
    """Min / max of x reduced to ``enc_shape`` (NaN propagates)."""
    x = np.asarray(x, f32)
    nd = x.ndim
    shape = (1,) * (nd - len(enc_shape)) + tuple(enc_shape)
    axes = tuple(a for a in range(nd) if shape[a] == 1)
    return (x.min(axis=axes, keepdims=True).reshape(tuple(enc_shape)),
            x.max(axis=axes, keepdims=True).reshape(tuple(enc_shape)))
