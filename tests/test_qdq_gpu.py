"""GPU parity of the QDQ kernels (librxmet.so) against the pinned oracle.

Bar: outputs, masks and dx bit-exact; encoding gradients (fp64-accumulated sums) within
1e-6 relative of the oracle's fp64 sums; min/max exact.
"""
import numpy as np
import pytest
import torch

import aimet_affine as A
import mi355x_qdq as Q
import qdq_oracle as O
import rxmet_lib

pytestmark = pytest.mark.gpu
f32 = np.float32

LAYOUTS = [
    (1, 1, 100003),      # per-tensor, odd length (scalar tail path)
    (1, 64, 1000),       # per-channel on dim 0, runs path, inner % 4 == 0
    (1, 7, 1027),        # per-channel, runs path with unaligned runs
    (40, 16, 1),         # per-channel on the last dim: column path
    (3, 8, 50),          # per-channel on a middle dim: column path
    (2, 5, 2048),        # outer > 1 with long runs
    (1, 3, 20000),       # runs split into several chunks
]


def _data(n, seed):
    g = np.random.default_rng(seed)
    x = g.standard_normal(n).astype(f32)
    m = g.random(n) < 0.01
    x[m] = (g.standard_normal(int(m.sum())) * 10).astype(f32)
    return x


def _enc(C, seed, qmin, qmax, symmetric):
    g = np.random.default_rng(seed)
    mn = -(g.random(C) * 2 + 0.5).astype(f32)
    mx = (g.random(C) * 2 + 0.5).astype(f32)
    return O.scale_offset(mn, mx, qmin, qmax, symmetric)


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _ws(layout, dev):
    return torch.empty(max(16, rxmet_lib.load().rxmet_qdq_workspace_bytes(*layout)),
                       dtype=torch.uint8, device=dev)


def _stream(dev):
    return torch.cuda.current_stream(dev).cuda_stream


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("grid", [(-128, 127, True), (0, 255, False), (-8, 7, True),
                                  (0, 65535, False)])
@pytest.mark.parametrize("mode", [Q.LEARNABLE, Q.FROZEN])
def test_forward_backward_match_oracle(cuda, layout, grid, mode):
    qmin, qmax, sym = grid
    outer, C, inner = layout
    n = outer * C * inner
    print(f"[qdq] layout={layout} grid={grid} mode={mode}", flush=True)
    x = _data(n, 1)
    x[:5] = [np.nan, np.inf, -np.inf, 0.0, -0.0] if n > 5 else x[:5]
    g = np.random.default_rng(2).standard_normal(n).astype(f32)
    s, o = _enc(C, 3, qmin, qmax, sym)
    xd, gd, sd, od = _t(x, cuda), _t(g, cuda), _t(s, cuda), _t(o, cuda)
    y = torch.empty_like(xd)
    rxmet_lib.call("rxmet_qdq_forward", xd.data_ptr(), y.data_ptr(), outer, C, inner, sd.data_ptr(),
                   od.data_ptr(), qmin, qmax, mode, _stream(cuda))
    dx = torch.empty_like(xd)
    learn = mode == Q.LEARNABLE
    ds = torch.empty(C, device=cuda) if learn else None
    do = torch.empty(C, device=cuda) if learn else None
    rxmet_lib.call("rxmet_qdq_backward", xd.data_ptr(), gd.data_ptr(), dx.data_ptr(),
                   rxmet_lib.ptr(ds), rxmet_lib.ptr(do), outer, C, inner, sd.data_ptr(),
                   od.data_ptr(), qmin, qmax, mode, _ws(layout, cuda).data_ptr(), _stream(cuda))
    torch.cuda.synchronize()
    if learn:
        ey, _ = O.qdq_learnable(x, s, o, qmin, qmax, layout)
        edx, eds, edo = O.qdq_learnable_backward(x, g, s, o, qmin, qmax, layout)
    else:
        ey, _ = O.qdq_frozen(x, s, o, qmin, qmax, layout)
        edx = O.qdq_frozen_backward(x, g, s, o, qmin, qmax, layout)
    np.testing.assert_array_equal(y.cpu().numpy(), ey)
    np.testing.assert_array_equal(dx.cpu().numpy(), edx)
    if learn:
        # NaN/inf inputs make the reference's scale gradient NaN for their encoding
        np.testing.assert_allclose(ds.cpu().numpy(), eds, rtol=1e-6, atol=1e-6, equal_nan=True)
        np.testing.assert_allclose(do.cpu().numpy(), edo, rtol=1e-6, atol=1e-6, equal_nan=True)


def _backward(cuda, x, g, s, o, layout, qmin, qmax):
    xd, gd, sd, od = _t(x, cuda), _t(g, cuda), _t(s, cuda), _t(o, cuda)
    C = layout[1]
    dx, ds, do = torch.empty_like(xd), torch.empty(C, device=cuda), torch.empty(C, device=cuda)
    rxmet_lib.call("rxmet_qdq_backward", xd.data_ptr(), gd.data_ptr(), dx.data_ptr(),
                   ds.data_ptr(), do.data_ptr(), *layout, sd.data_ptr(), od.data_ptr(), qmin,
                   qmax, Q.LEARNABLE, _ws(layout, cuda).data_ptr(), _stream(cuda))
    torch.cuda.synchronize()
    return dx, ds, do


# Plans of the c2 shapes: per-channel rows of 2, 3 and 4 chunks held whole by one workgroup
# (1024+ rows; the workgroup writes its encoding gradients, no fold), and single runs of 2048+
# chunks taken two interleaved chunks per workgroup (the last chunk partial: 16-byte vector
# path, and the element path of an odd length)
FOLD_LAYOUTS = [(1, 1024, 8192), (1, 1030, 12284), (1, 1024, 16384), (1, 1, 4096 * 2051 + 8),
                (1, 1, 4096 * 2049 + 7)]


@pytest.mark.parametrize("layout", FOLD_LAYOUTS)
def test_whole_run_and_two_chunk_plans_match_oracle(cuda, layout):
    qmin, qmax = -128, 127
    n = int(np.prod(layout))
    print(f"[qdq] plan layout={layout}", flush=True)
    x, g = _data(n, 41), np.random.default_rng(42).standard_normal(n).astype(f32)
    s, o = _enc(layout[1], 43, qmin, qmax, False)
    xd, sd, od = _t(x, cuda), _t(s, cuda), _t(o, cuda)
    y = torch.empty_like(xd)
    rxmet_lib.call("rxmet_qdq_forward", xd.data_ptr(), y.data_ptr(), *layout, sd.data_ptr(),
                   od.data_ptr(), qmin, qmax, Q.LEARNABLE, _stream(cuda))
    dx, ds, do = _backward(cuda, x, g, s, o, layout, qmin, qmax)
    ey, _ = O.qdq_learnable(x, s, o, qmin, qmax, layout)
    edx, eds, edo = O.qdq_learnable_backward(x, g, s, o, qmin, qmax, layout)
    np.testing.assert_array_equal(y.cpu().numpy(), ey)
    np.testing.assert_array_equal(dx.cpu().numpy(), edx)
    np.testing.assert_allclose(ds.cpu().numpy(), eds, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(do.cpu().numpy(), edo, rtol=1e-6, atol=1e-6)


def test_per_tensor_encoding_gradients_at_scale(cuda):
    """Per-tensor over 20000 chunks (10000 workgroups of two interleaved chunks, folded by the
    1024-thread fold): the tensor repeats one 16384-element block 5000 times, so its encoding
    gradients are 5000 times the oracle's over the block, and dx is the block's dx repeated."""
    qmin, qmax = -128, 127
    blk, reps = 16384, 5000
    xb, gb = _data(blk, 51), np.random.default_rng(52).standard_normal(blk).astype(f32)
    s, o = _enc(1, 53, qmin, qmax, False)
    edx, eds, edo = O.qdq_learnable_backward(xb, gb, s, o, qmin, qmax, (1, 1, blk))
    dx, ds, do = _backward(cuda, np.tile(xb, reps), np.tile(gb, reps), s, o,
                           (1, 1, blk * reps), qmin, qmax)
    assert torch.equal(dx.view(reps, blk), _t(edx, cuda).expand(reps, blk))
    np.testing.assert_allclose(ds.cpu().numpy(), eds.astype(np.float64) * reps, rtol=1e-6)
    np.testing.assert_allclose(do.cpu().numpy(), edo.astype(np.float64) * reps, rtol=1e-6)


@pytest.mark.parametrize("layout", LAYOUTS)
def test_minmax_matches_oracle(cuda, layout):
    outer, C, inner = layout
    x = _data(outer * C * inner, 4)
    mn = torch.empty(C, device=cuda)
    mx = torch.empty(C, device=cuda)
    xd = _t(x, cuda)
    rxmet_lib.call("rxmet_qdq_minmax", xd.data_ptr(), outer, C, inner, mn.data_ptr(), mx.data_ptr(),
                   _ws(layout, cuda).data_ptr(), _stream(cuda))
    emn, emx = O.minmax(x, layout)
    np.testing.assert_array_equal(mn.cpu().numpy(), emn)
    np.testing.assert_array_equal(mx.cpu().numpy(), emx)
    x[len(x) // 2] = np.nan
    xd = _t(x, cuda)
    rxmet_lib.call("rxmet_qdq_minmax", xd.data_ptr(), outer, C, inner, mn.data_ptr(), mx.data_ptr(),
                   _ws(layout, cuda).data_ptr(), _stream(cuda))
    emn, emx = O.minmax(x, layout)
    np.testing.assert_array_equal(mn.cpu().numpy(), emn)
    np.testing.assert_array_equal(mx.cpu().numpy(), emx)


def _bits_equal(a, e, msg):
    """Bit-for-bit equality (signed zeros told apart), NaN matching NaN."""
    a, e = np.asarray(a, f32), np.asarray(e, f32)
    na, ne = np.isnan(a), np.isnan(e)
    np.testing.assert_array_equal(na, ne, err_msg=msg)
    np.testing.assert_array_equal(a[~na].view(np.uint32), e[~ne].view(np.uint32), err_msg=msg)


def test_quotients_are_correctly_rounded(cuda):
    """x / s as the kernels evaluate it (a product by the rounded reciprocal with one fma
    correction inside [2^-100, 2^100], the division elsewhere) against IEEE division: the
    quantized codes of values within two ulps of every rounding tie (k + 1/2) s, and
    dx = g m / s of QuantizeFunc's backward, which is the quotient itself, for scales with
    all-ones and minimal significands, powers of two, tiny and huge scales, and operands at
    and beyond the fast range (zeros, denormals, 2^-110 .. 2^110, inf, NaN)."""
    fb = lambda u: np.array([u], np.uint32).view(f32)[0]
    scales = np.array([0.0173, 0.1, 3.0, 1.0, 0.5, fb(0x3fffffff), fb(0x3f7fffff), fb(0x3f800001),
                       fb(0x3fc00001), 1e-30, 1e30, 2.0 ** -120, 2.0 ** -126, 2.0 ** 120], f32)
    C, n = len(scales), 6000
    rng = np.random.default_rng(71)
    x = np.empty((C, n), f32)
    g = np.empty((C, n), f32)
    edge = np.array([0.0, -0.0, 1e-40, -1e-40, 2.0 ** -110, -(2.0 ** -110), 2.0 ** -100,
                     2.0 ** 100, 2.0 ** 110, 3e38, -3e38, np.inf, -np.inf, np.nan], f32)
    for c, s in enumerate(scales):
        k = rng.integers(-(1 << 20), 1 << 20, n // 5)
        tie = ((k + 0.5) * np.float64(s)).astype(f32)
        row = [tie, np.nextafter(tie, np.inf, dtype=f32), np.nextafter(tie, -np.inf, dtype=f32),
               np.nextafter(np.nextafter(tie, np.inf, dtype=f32), np.inf, dtype=f32),
               np.nextafter(np.nextafter(tie, -np.inf, dtype=f32), -np.inf, dtype=f32)]
        x[c] = np.concatenate(row)[:n]
        x[c, :len(edge)] = edge
        gr = rng.standard_normal(n).astype(f32) * (10.0 ** rng.integers(-38, 38, n)).astype(f32)
        gr[:len(edge)] = edge
        g[c] = gr
    o = np.zeros(C, f32)
    qmin, qmax = -(1 << 23), (1 << 23) - 1
    layout = (1, C, n)
    xd, gd, sd, od = (_t(a, cuda) for a in (x.reshape(-1), g.reshape(-1), scales, o))
    q, dx = torch.empty_like(xd), torch.empty_like(xd)
    ds, do = torch.empty(C, device=cuda), torch.empty(C, device=cuda)
    rxmet_lib.call("rxmet_quantize_forward", xd.data_ptr(), q.data_ptr(), *layout, sd.data_ptr(),
                   od.data_ptr(), qmin, qmax, _stream(cuda))
    rxmet_lib.call("rxmet_quantize_backward", xd.data_ptr(), gd.data_ptr(), dx.data_ptr(),
                   ds.data_ptr(), do.data_ptr(), *layout, sd.data_ptr(), od.data_ptr(), qmin, qmax,
                   _ws(layout, cuda).data_ptr(), _stream(cuda))
    torch.cuda.synchronize()
    eq = O.quantize(x.reshape(-1), scales, o, qmin, qmax, layout)
    edx, _, _ = O.quantize_backward(x.reshape(-1), g.reshape(-1), scales, o, qmin, qmax, layout)
    _bits_equal(q.cpu().numpy(), eq, "codes")
    _bits_equal(dx.cpu().numpy(), edx, "dx = g m / s")


@pytest.mark.parametrize("layout", [(1, 1, 5001), (1, 4, 3000), (30, 6, 1)])
def test_quantize_dequantize_kernels(cuda, layout):
    outer, C, inner = layout
    n = outer * C * inner
    x = _data(n, 5)
    g = np.random.default_rng(6).standard_normal(n).astype(f32)
    s, o = _enc(C, 7, 0, 255, False)
    xd, gd, sd, od = (_t(a, cuda) for a in (x, g, s, o))
    q = torch.empty_like(xd)
    rxmet_lib.call("rxmet_quantize_forward", xd.data_ptr(), q.data_ptr(), outer, C, inner,
                   sd.data_ptr(), od.data_ptr(), 0, 255, _stream(cuda))
    dx = torch.empty_like(xd)
    ds, do = torch.empty(C, device=cuda), torch.empty(C, device=cuda)
    rxmet_lib.call("rxmet_quantize_backward", xd.data_ptr(), gd.data_ptr(), dx.data_ptr(),
                   ds.data_ptr(), do.data_ptr(), outer, C, inner, sd.data_ptr(), od.data_ptr(), 0,
                   255, _ws(layout, cuda).data_ptr(), _stream(cuda))
    eq = O.quantize(x, s, o, 0, 255, layout)
    edx, eds, edo = O.quantize_backward(x, g, s, o, 0, 255, layout)
    np.testing.assert_array_equal(q.cpu().numpy(), eq)
    np.testing.assert_array_equal(dx.cpu().numpy(), edx)
    np.testing.assert_allclose(ds.cpu().numpy(), eds, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(do.cpu().numpy(), edo, rtol=1e-6, atol=1e-6)
    y = torch.empty_like(xd)
    rxmet_lib.call("rxmet_dequantize_forward", q.data_ptr(), y.data_ptr(), outer, C, inner,
                   sd.data_ptr(), od.data_ptr(), _stream(cuda))
    rxmet_lib.call("rxmet_dequantize_backward", q.data_ptr(), gd.data_ptr(), dx.data_ptr(),
                   ds.data_ptr(), do.data_ptr(), outer, C, inner, sd.data_ptr(), od.data_ptr(),
                   _ws(layout, cuda).data_ptr(), _stream(cuda))
    ey = O.dequantize(eq, s, o, layout)
    edq, eds, edo = O.dequantize_backward(eq, g, s, o, layout)
    np.testing.assert_array_equal(y.cpu().numpy(), ey)
    np.testing.assert_array_equal(dx.cpu().numpy(), edq)
    np.testing.assert_allclose(ds.cpu().numpy(), eds, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(do.cpu().numpy(), edo, rtol=1e-6, atol=1e-6)


def test_empty_tensor(cuda):
    x = torch.empty(0, device=cuda)
    s = torch.ones(1, device=cuda)
    y = Q.quantize_dequantize(x, s, torch.zeros(1, device=cuda), -128, 127)
    assert y.numel() == 0


def test_errors_are_raised(cuda):
    x = torch.randn(10, device=cuda)
    with pytest.raises(RuntimeError):
        Q.quantize_dequantize(x, torch.ones(3, device=cuda), torch.zeros(3, device=cuda), 0, 255)
    with pytest.raises(RuntimeError):
        Q.quantize_dequantize(x, torch.ones(1, device=cuda), torch.zeros(1, device=cuda), 5, 1)


def _module_case(cuda, shape, enc_shape, bits, symmetric, seed, learn=True):
    """QuantizeDequantize through the aimet mirror vs the oracle pipeline."""
    x = _data(int(np.prod(shape)), seed).reshape(shape)
    g = np.random.default_rng(seed + 1).standard_normal(x.shape).astype(f32)
    q = A.QuantizeDequantize(enc_shape, bits, symmetric).to(cuda)
    xd = _t(x, cuda)
    with q.compute_encodings():
        q(xd)
    if not learn:
        q.requires_grad_(False)
    xg = xd.clone().requires_grad_()
    y = q(xg)
    y.backward(_t(g, cuda))
    lay5 = Q.kernel_layout(shape, enc_shape)
    assert lay5[0] == lay5[1] == 1  # one encoding group
    layout = lay5[2:]
    C = layout[1]
    mn, mx = O.minmax(x, layout)
    qmin, qmax = q.qmin, q.qmax
    lo, hi = O.compute_encodings_from_stats(mn, mx, qmax - qmin, symmetric and qmin < 0,
                                            gpu_scalar_div=True)
    np.testing.assert_array_equal(q.min.detach().cpu().numpy().reshape(-1), lo)
    np.testing.assert_array_equal(q.max.detach().cpu().numpy().reshape(-1), hi)
    s, o = O.scale_offset(lo, hi, qmin, qmax, symmetric, gpu_scalar_div=True)
    es, eo = q.get_encodings()
    np.testing.assert_array_equal(es.detach().cpu().numpy().reshape(-1), s)
    np.testing.assert_array_equal(eo.detach().cpu().numpy().reshape(-1), o)
    if learn:
        ey, _ = O.qdq_learnable(x, s, o, qmin, qmax, layout)
        edx, eds, edo = O.qdq_learnable_backward(x, g, s, o, qmin, qmax, layout)
    else:
        ey, _ = O.qdq_frozen(x, s, o, qmin, qmax, layout)
        edx = O.qdq_frozen_backward(x, g, s, o, qmin, qmax, layout)
    np.testing.assert_array_equal(y.detach().cpu().numpy(), ey)
    np.testing.assert_array_equal(xg.grad.cpu().numpy(), edx)
    if learn:
        # chain the oracle's encoding gradients through the same min/max -> (s, o) graph
        pmn = torch.from_numpy(lo.reshape(enc_shape)).requires_grad_()
        pmx = torch.from_numpy(hi.reshape(enc_shape)).requires_grad_()
        ref = A.QuantizeDequantize(enc_shape, bits, symmetric)
        ref.set_range(pmn.detach(), pmx.detach())
        st = ref.get_scale()
        ot = ref._get_offset(scale=st)
        outs = [st] + ([ot] if ot.requires_grad else [])
        grads = [torch.from_numpy(eds.reshape(st.shape))] + (
            [torch.from_numpy(edo.reshape(ot.shape))] if ot.requires_grad else [])
        torch.autograd.backward(outs, grads)
        np.testing.assert_allclose(q.min.grad.cpu().numpy(), ref.min.grad.numpy(), rtol=1e-5,
                                   atol=1e-3)
        np.testing.assert_allclose(q.max.grad.cpu().numpy(), ref.max.grad.numpy(), rtol=1e-5,
                                   atol=1e-3)
    return C


@pytest.mark.parametrize("learn", [True, False])
def test_module_per_tensor_8bit_asym(cuda, learn):
    _module_case(cuda, (512, 768), (), 8, False, 21, learn)


@pytest.mark.parametrize("learn", [True, False])
def test_module_per_channel_4bit_sym(cuda, learn):
    _module_case(cuda, (512, 768), (512, 1), 4, True, 22, learn)


def test_full_size_c2(cuda):
    """c2 at its full shape [8192, 8192]: both modes against the oracle, plus frozen QDQ
    against torch's own fake_quantize on the GPU."""
    shape = (8192, 8192)
    for enc_shape, bits, sym in (((), 8, False), ((8192, 1), 4, True)):
        print(f"[qdq] full size enc={enc_shape} bits={bits}", flush=True)
        _module_case(cuda, shape, enc_shape, bits, sym, 31, learn=True)
    x = torch.from_numpy(_data(8192 * 8192, 33).reshape(shape)).to(cuda)
    s = torch.tensor(0.0173, device=cuda)
    y = Q.quantize_dequantize(x, s, torch.tensor(-3.0, device=cuda), -128, 127)
    ref = torch.fake_quantize_per_tensor_affine(x, s, torch.tensor(3, dtype=torch.int32,
                                                                   device=cuda), -128, 127)
    assert torch.equal(y, ref)
