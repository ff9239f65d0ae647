"""Pin the fake-quantization oracle (oracle/qdq_oracle.py) before trusting it.

Checks, each chosen so a plausible mistake (wrong rounding mode, 1/s vs /s, sign of
the offset, a dropped term of a gradient) fails:
* frozen-encoding mode == torch.fake_quantize_per_{tensor,channel}_affine, the
  third-party kernels the reference's fast path calls (torch_builtins.py:287-361);
* the reference's docstring tables (backends/__init__.py:169-187, 336-354);
* ties-to-even, decimal-reciprocal and NaN/inf tables of
  tests/integration/test_native_qdq_alignment.py:94-147;
* learnable-mode gradients == torch autograd through a straight-through surrogate of
  QuantDequantFunc's forward (an independent derivation of torch_builtins.py:675-691);
* the encoding analyzer's closed forms (encoding_analyzer.py:217-272, quantsim.py:463-470).
"""
import numpy as np
import pytest
import torch

import qdq_oracle as O

f32 = np.float32


def _data(n, seed, outliers=True):
    g = np.random.default_rng(seed)
    x = g.standard_normal(n).astype(f32)
    if outliers:
        m = g.random(n) < 0.01
        x[m] = (g.standard_normal(int(m.sum())) * 10).astype(f32)
    return x


@pytest.mark.parametrize("bits,signed", [(8, True), (8, False), (4, True), (16, True)])
@pytest.mark.parametrize("scale", [0.0173, 1 / 15, 2.0 ** -5, 0.027019, 1 / 32767])
def test_frozen_matches_torch_fake_quantize_per_tensor(bits, signed, scale):
    qmin, qmax = (-(1 << (bits - 1)), (1 << (bits - 1)) - 1) if signed else (0, (1 << bits) - 1)
    x = _data(20000, 1)
    for offset in (0.0, float(-qmin - 3) if not signed else 0.0, -5.0 if not signed else 3.0):
        zp = -int(offset)
        if not (qmin <= zp <= qmax):
            continue
        y, mask = O.qdq_frozen(x, [scale], [offset], qmin, qmax, (1, 1, x.size))
        xt = torch.from_numpy(x.copy()).requires_grad_()
        ref = torch.fake_quantize_per_tensor_affine(
            xt, torch.tensor(scale, dtype=torch.float32), torch.tensor(zp, dtype=torch.int32),
            qmin, qmax)
        np.testing.assert_array_equal(y, ref.detach().numpy())
        ref.backward(torch.ones_like(ref))
        np.testing.assert_array_equal(mask.astype(f32), xt.grad.numpy())


def test_frozen_matches_torch_fake_quantize_per_channel():
    x = _data(64 * 300, 2).reshape(64, 300)
    g = np.random.default_rng(3)
    scale = (g.random(64) * 0.05 + 0.001).astype(f32)
    for qmin, qmax, offset in ((-8, 7, np.zeros(64, f32)), (0, 255, -np.full(64, 100, f32))):
        y, mask = O.qdq_frozen(x, scale, offset, qmin, qmax, (1, 64, 300))
        xt = torch.from_numpy(x.copy()).requires_grad_()
        ref = torch.fake_quantize_per_channel_affine(
            xt, torch.from_numpy(scale), torch.from_numpy(-offset).to(torch.int32), 0, qmin, qmax)
        np.testing.assert_array_equal(y, ref.detach().numpy())
        ref.backward(torch.ones_like(ref))
        np.testing.assert_array_equal(mask.astype(f32), xt.grad.numpy())


def test_docstring_tables():
    # backends/__init__.py:169-187 and :336-354 (4-bit unsigned, scale 1/15, offset 0)
    x = torch.arange(start=-0.3, end=1.3, step=0.05).numpy()
    s = np.float32(torch.tensor(1 / 15).item())
    q = O.quantize(x, [s], [0.0], 0, 15, (1, 1, x.size))
    expect_q = [0, 0, 0, 0, 0, 0, -0, 1, 2, 2, 3, 4, 4, 5, 6, 7, 7, 8, 9, 10, 10, 11, 12, 13,
                13, 14, 15, 15, 15, 15, 15, 15]
    np.testing.assert_array_equal(q, np.array(expect_q, f32))
    y, _ = O.qdq_learnable(x, [s], [0.0], 0, 15, (1, 1, x.size))
    expect_y = [0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0667, 0.1333, 0.1333, 0.2000, 0.2667, 0.2667,
                0.3333, 0.4000, 0.4667, 0.4667, 0.5333, 0.6000, 0.6667, 0.6667, 0.7333, 0.8000,
                0.8667, 0.8667, 0.9333, 1.0000, 1.0000, 1.0000, 1.0000, 1.0000, 1.0000]
    np.testing.assert_allclose(y, expect_y, atol=5e-5, rtol=0)


@pytest.mark.parametrize("bits", [8, 16])
@pytest.mark.parametrize("symmetric", [True, False])
def test_ties_to_even_table(bits, symmetric):
    # test_native_qdq_alignment.py:111-118
    codes = np.array([-7.5, -3.5, -2.5, -1.5, -.5, .5, 1.5, 2.5, 3.5, 7.5], dtype=f32)
    s = f32(2.0 ** -7 if bits == 8 else 2.0 ** -15)
    x = (codes * s).astype(f32)
    if symmetric:
        qmin, qmax, off = -(1 << (bits - 1)), (1 << (bits - 1)) - 1, 0.0
    else:
        qmin, qmax, off = 0, (1 << bits) - 1, -13.0
    expect = (np.rint(codes) * s).astype(f32)
    for fn in (O.qdq_frozen, O.qdq_learnable):
        y, _ = fn(x, [s], [off], qmin, qmax, (1, 1, x.size))
        np.testing.assert_array_equal(y, expect)
    assert list(np.rint(codes)) == [-8, -4, -2, -2, -0, 0, 2, 2, 4, 8]


@pytest.mark.parametrize("scale", [1.0 / 32767, .013007, .027019])
def test_decimal_scale_uses_float32_reciprocal(scale):
    # test_native_qdq_alignment.py:120-124: frozen QDQ multiplies by fl(1/scale)
    codes = np.arange(-63, 64, dtype=f32) + f32(.5)
    x = (codes * f32(scale)).astype(f32)
    y, _ = O.qdq_frozen(x, [scale], [0.0], -32768, 32767, (1, 1, x.size))
    ref = torch.fake_quantize_per_tensor_affine(torch.from_numpy(x), torch.tensor(scale),
                                                torch.tensor(0, dtype=torch.int32), -32768, 32767)
    np.testing.assert_array_equal(y, ref.numpy())


def test_nan_kept_and_infinity_saturates():
    # test_native_qdq_alignment.py:126-137
    for bits in (8, 16):
        s = f32(2.0 ** -7 if bits == 8 else 2.0 ** -15)
        qmin, qmax = -(1 << (bits - 1)), (1 << (bits - 1)) - 1
        x = np.array([np.nan, -np.inf, -s, 0, s, np.inf], dtype=f32)
        expect = np.array([np.nan, qmin * s, -s, 0, s, qmax * s], dtype=f32)
        for fn in (O.qdq_frozen, O.qdq_learnable):
            y, mask = fn(x, [s], [0.0], qmin, qmax, (1, 1, x.size))
            np.testing.assert_array_equal(y, expect)
            assert list(mask) == [False, False, True, True, True, False]


def _tf_grid(bits, scale, offset=None):
    """TfEncoding min / max of test_native_qdq_alignment.py:18-25."""
    off = -(1 << (bits - 1)) if offset is None else offset
    return off * scale, (off + (1 << bits) - 1) * scale


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_native_qdq_alignment_tables(dtype):
    # quantize_dequantize.hpp:35-46 on the cases of test_native_qdq_alignment.py:88-137
    t = np.dtype(dtype).type
    # exact integer codes with an int32 offset (:88-90) and per channel (:107-110)
    codes = np.array([-257, -65, -7, -3, -1, 0, 1, 3, 7, 65, 257], dtype=dtype)
    s = 2.0 ** -21
    lo, hi = _tf_grid(32, s)
    np.testing.assert_array_equal(O.native_qdq(codes * t(s), lo, hi, s, dtype), codes * t(s))
    codes = np.array([-7, -3, -1, 0, 1, 3, 7], dtype=dtype)
    scales = np.array([[2.0 ** -21], [2.0 ** -20]])
    x = np.stack([codes * t(sc) for sc in scales[:, 0]])
    lo, hi = _tf_grid(32, scales)
    np.testing.assert_array_equal(O.native_qdq(x, lo, hi, scales, dtype), x)
    # ties to even (:111-118), also on asymmetric grids (offset -13)
    codes = np.array([-7.5, -3.5, -2.5, -1.5, -.5, .5, 1.5, 2.5, 3.5, 7.5], dtype=dtype)
    for bits in (8, 16, 32):
        s = 2.0 ** -7 if bits == 8 else 2.0 ** -15 if bits == 16 else 2.0 ** -21
        for off in (None, -13):
            lo, hi = _tf_grid(bits, s, off)
            y = O.native_qdq(codes * t(s), lo, hi, s, dtype)
            np.testing.assert_array_equal(y, np.array([-8, -4, -2, -2, 0, 0, 2, 2, 4, 8]) * t(s))
    # NaN kept, infinity clipped to the grid ends (:126-137)
    for bits in (8, 16, 32):
        s = 2.0 ** -7 if bits == 8 else 2.0 ** -15 if bits == 16 else 2.0 ** -21
        lo, hi = _tf_grid(bits, s)
        x = np.array([np.nan, -np.inf, -s, 0, s, np.inf], dtype=dtype)
        y = O.native_qdq(x, lo, hi, s, dtype)
        np.testing.assert_array_equal(y, np.array([np.nan, lo, -s, 0, s, hi], dtype=dtype))


@pytest.mark.parametrize("scale", [.013007, .027019])
def test_native_qdq_multiplies_by_the_rounded_reciprocal(scale):
    # :120-124.  On these half-code values x / s and x * fl(1 / s) round apart: a division
    # in place of qdqReciprocal would fail here.
    s = f32(scale)
    x = ((np.arange(-63, 64, dtype=f32) + f32(.5)) * s).astype(f32)
    lo, hi = _tf_grid(16, float(s))
    y = O.native_qdq(x, lo, hi, s)
    by_rcp = (np.rint((x * (f32(1) / s)).astype(f32)) * s).astype(f32)
    by_div = (np.rint((x / s).astype(f32)) * s).astype(f32)
    np.testing.assert_array_equal(y, by_rcp)
    assert (y != by_div).any()
    # and it is the value the Torch path gives (the alignment the reference test asserts)
    ref = torch.fake_quantize_per_tensor_affine(torch.from_numpy(x), float(s), 0, -32768, 32767)
    np.testing.assert_array_equal(y, ref.numpy())


@pytest.mark.parametrize("bits,scale,off", [(8, 2.0 ** -5, None), (8, 0.0173, -40), (16, 0.00031, None),
                                            (4, 0.25, -3)])
def test_native_qdq_equals_frozen_qdq_on_random_values(bits, scale, off):
    # on grid-aligned minimum / maximum the two forms agree value for value
    g = np.random.default_rng(bits)
    s = f32(scale)
    lo, hi = _tf_grid(bits, float(s), off)
    x = (g.standard_normal(4096) * (hi - lo) / 3).astype(f32)
    x[:4] = [np.nan, np.inf, -np.inf, 0.0]
    if off is None:  # symmetric: signed codes, offset 0
        qmin, qmax, aoff = -(1 << (bits - 1)), (1 << (bits - 1)) - 1, 0.0
    else:  # asymmetric: unsigned codes shifted by the offset
        qmin, qmax, aoff = 0, (1 << bits) - 1, float(off)
    yf, _ = O.qdq_frozen(x, [s], [aoff], qmin, qmax, (1, 1, x.size))
    yn = O.native_qdq(x, f32(lo), f32(hi), s)
    np.testing.assert_array_equal(yn, yf)


def test_native_qdq_stochastic_rounding():
    # floor(scaled + noise): noise 0 truncates down, noise just below 1 rounds every
    # non-integer up, and the mean over uniform noise is the value itself
    s = 2.0 ** -4
    lo, hi = _tf_grid(8, s)
    x = np.array([-1.3, -0.55, 0.2, 0.7, 0.95], dtype=f32) * f32(8 * s)  # no whole codes
    scaled = x / f32(s)
    np.testing.assert_array_equal(O.native_qdq(x, lo, hi, s, noise=np.zeros(5)), np.floor(scaled) * f32(s))
    near1 = np.full(5, np.nextafter(f32(1), f32(0)))
    np.testing.assert_array_equal(O.native_qdq(x, lo, hi, s, noise=near1), np.ceil(scaled) * f32(s))
    g = np.random.default_rng(1)
    noise = g.random((20000, 5)).astype(f32)
    mean = O.native_qdq(np.broadcast_to(x, noise.shape), lo, hi, s, noise=noise).mean(axis=0)
    np.testing.assert_allclose(mean, x, atol=4 * float(s) / np.sqrt(20000) * 3)


def _surrogate_grads(x, g, s, o, qmin, qmax, layout):
    """Autograd of y = (clamp(ste_round(x/s) - o) + o) * s, fp64 arithmetic with the
    fp32 rounding decisions of the forward; independent of the oracle's formulas."""
    outer, C, inner = layout
    xt = torch.from_numpy(x.astype(np.float64)).view(outer, C, inner)
    st = torch.from_numpy(np.asarray(s, np.float64)).view(1, C, 1).requires_grad_()
    ot = torch.from_numpy(np.asarray(o, np.float64)).view(1, C, 1).requires_grad_()
    xt = xt.requires_grad_()
    xs32 = (x.reshape(outer, C, inner) / np.asarray(s, f32).reshape(1, C, 1)).astype(f32)
    rounded = torch.from_numpy(np.rint(xs32).astype(np.float64))
    xs = xt / st
    r = xs + (rounded - xs).detach() - ot
    q = torch.clamp(r, qmin, qmax)
    y = (q + ot) * st
    y.backward(torch.from_numpy(g.astype(np.float64)).view(outer, C, inner))
    return xt.grad.numpy().reshape(x.shape), st.grad.numpy().reshape(-1), ot.grad.numpy().reshape(-1)


@pytest.mark.parametrize("layout,qmin,qmax,asym", [((1, 1, 6000), -128, 127, False),
                                                   ((1, 1, 6000), 0, 255, True),
                                                   ((1, 16, 400), -8, 7, False),
                                                   ((3, 8, 50), 0, 255, True)])
def test_learnable_gradients_match_autograd_surrogate(layout, qmin, qmax, asym):
    outer, C, inner = layout
    n = outer * C * inner
    x = _data(n, 7)
    g = np.random.default_rng(8).standard_normal(n).astype(f32)
    mn = np.full(C, -2.0, f32)
    mx = np.full(C, 2.5, f32) * (1 + np.arange(C, dtype=f32) / C)
    s, o = O.scale_offset(mn, mx, qmin, qmax, symmetric=not asym)
    dx, ds, do = O.qdq_learnable_backward(x, g, s, o, qmin, qmax, layout)
    sdx, sds, sdo = _surrogate_grads(x, g, s, o, qmin, qmax, layout)
    np.testing.assert_array_equal(dx, sdx.astype(f32))
    scale_ref = np.abs(g).reshape(outer, C, inner).sum(axis=(0, 2)) * 8
    np.testing.assert_allclose(ds, sds, rtol=0, atol=1e-5 * scale_ref.max())
    np.testing.assert_allclose(do, sdo, rtol=1e-5, atol=1e-5 * (s * np.abs(g).sum()).max())


def test_quantize_dequantize_gradients_match_autograd():
    layout = (1, 4, 500)
    x = _data(2000, 11)
    g = np.random.default_rng(12).standard_normal(2000).astype(f32)
    s = np.array([0.01, 0.02, 0.03, 0.05], f32)
    o = np.array([-100, -128, -10, -200], f32)
    q = O.quantize(x, s, o, 0, 255, layout)
    dq, dsd, dod = O.dequantize_backward(q, g, s, o, layout)
    qt = torch.from_numpy(q.astype(np.float64)).view(1, 4, 500).requires_grad_()
    st = torch.from_numpy(s.astype(np.float64)).view(1, 4, 1).requires_grad_()
    ot = torch.from_numpy(o.astype(np.float64)).view(1, 4, 1).requires_grad_()
    ((qt + ot) * st).backward(torch.from_numpy(g.astype(np.float64)).view(1, 4, 500))
    np.testing.assert_allclose(dq, qt.grad.numpy().reshape(-1), rtol=1e-6)
    np.testing.assert_allclose(dsd, st.grad.numpy().reshape(-1), rtol=1e-5)
    np.testing.assert_allclose(dod, ot.grad.numpy().reshape(-1), rtol=1e-5)
    y = O.dequantize(q, s, o, layout)
    np.testing.assert_array_equal(y, ((q.reshape(1, 4, 500) + o.reshape(1, 4, 1)) *
                                      s.reshape(1, 4, 1)).astype(f32).reshape(-1))


@pytest.mark.parametrize("qmin,qmax", [(0, 255), (-128, 127), (-8, 7)])
def test_quantize_gradients_match_autograd_surrogate(qmin, qmax):
    """QuantizeFunc's backward (torch_builtins.py:554-571) against torch autograd through
    q = clamp(ste_round(x/s) - o): float64 arithmetic, the forward's fp32 rounding decisions,
    clamp's inclusive pass-through at the grid ends as the reference's mask."""
    layout = (1, 4, 500)
    x = _data(2000, 13)
    g = np.random.default_rng(14).standard_normal(2000).astype(f32)
    s = np.array([0.01, 0.02, 0.03, 0.05], f32)
    o = np.array([-100, -128, -10, -200], f32) if qmin == 0 else np.zeros(4, f32)
    gq, ds, do = O.quantize_backward(x, g, s, o, qmin, qmax, layout)
    xt = torch.from_numpy(x.astype(np.float64)).view(1, 4, 500).requires_grad_()
    st = torch.from_numpy(s.astype(np.float64)).view(1, 4, 1).requires_grad_()
    ot = torch.from_numpy(o.astype(np.float64)).view(1, 4, 1).requires_grad_()
    xs32 = (x.reshape(1, 4, 500) / s.reshape(1, 4, 1)).astype(f32)
    rounded = torch.from_numpy(np.rint(xs32).astype(np.float64))
    xs = xt / st
    r = xs + (rounded - xs).detach() - ot
    q = torch.clamp(r, qmin, qmax)
    q.backward(torch.from_numpy(g.astype(np.float64)).view(1, 4, 500))
    assert 0 < (gq == 0).mean() < 1, "case must clamp some elements and keep others"
    np.testing.assert_allclose(gq, xt.grad.numpy().reshape(-1), rtol=1e-6)
    sref = (np.abs(g) * np.abs(x)).reshape(1, 4, 500).sum(axis=(0, 2)) / s.astype(np.float64) ** 2
    np.testing.assert_allclose(ds, st.grad.numpy().reshape(-1), rtol=0, atol=1e-6 * sref.max())
    np.testing.assert_allclose(do, ot.grad.numpy().reshape(-1), rtol=1e-6, atol=1e-6)
    np.testing.assert_array_equal(
        O.quantize(x, s, o, qmin, qmax, layout),
        np.clip(np.rint(xs32) - o.reshape(1, 4, 1), qmin, qmax).astype(f32).reshape(-1))


@pytest.mark.parametrize("shape,bits", [((), 8), ((64, 1), 4)])
def test_torch_cpu_step_matches_numpy_oracle(shape, bits):
    """The torch-on-CPU form used as the QDQ CPU baseline computes what the oracle does:
    y and dx bit for bit, the encoding gradients within summation-order noise."""
    R, Cc = 64, 1000
    rng = np.random.default_rng(21)
    x = rng.standard_normal((R, Cc)).astype(f32)
    g = rng.standard_normal((R, Cc)).astype(f32)
    qmin, qmax = (-128, 127) if bits == 8 else (-8, 7)
    n = 1 if shape == () else R
    s = (rng.random(n) * 0.05 + 0.01).astype(f32)
    o = (np.round(rng.random(n) * 10) - 5).astype(f32) if bits == 8 else np.zeros(n, f32)
    layout = (1, 1, R * Cc) if shape == () else (1, R, Cc)
    ey, _ = O.qdq_learnable(x, s, o, qmin, qmax, layout)
    edx, eds, edo = O.qdq_learnable_backward(x, g, s, o, qmin, qmax, layout)
    st = torch.from_numpy(s).reshape(shape)
    ot = torch.from_numpy(o).reshape(shape)
    y, dx, ds, do = O.torch_learnable_step(torch, torch.from_numpy(x), torch.from_numpy(g), st, ot,
                                           qmin, qmax)
    np.testing.assert_array_equal(y.numpy(), ey)
    np.testing.assert_array_equal(dx.numpy(), edx)
    np.testing.assert_allclose(ds.numpy().reshape(-1), eds, rtol=1e-4, atol=1e-3)
    np.testing.assert_allclose(do.numpy().reshape(-1), edo, rtol=1e-4, atol=1e-3)


def test_minimum_scale_table():
    # quantsim.py:463-470
    assert O.minimum_scale(15) == 2.0 ** -23
    assert O.minimum_scale(255) == 2.0 ** -23
    assert O.minimum_scale(65535) == 2.0 ** -23
    assert O.minimum_scale(2 ** 32 - 1) == 2.0 ** -38


def test_encoding_closed_forms():
    mn = np.array([-1.0, 0.5, -3.0], f32)
    mx = np.array([2.0, 4.0, -1.0], f32)
    lo, hi = O.compute_encodings_from_stats(mn, mx, 255, False)
    np.testing.assert_array_equal(lo, [-1.0, 0.0, -3.0])     # zero always inside
    np.testing.assert_array_equal(hi, [2.0, 4.0, 0.0])
    lo, hi = O.compute_encodings_from_stats(mn, mx, 255, True)
    delta = np.maximum(np.maximum(mx, 0) / f32(127), -np.minimum(mn, 0) / f32(128)).astype(f32)
    np.testing.assert_array_equal(lo, (-128 * delta).astype(f32))
    np.testing.assert_array_equal(hi, (127 * delta).astype(f32))
    # degenerate range gets the minimum-scale adjustment
    lo, hi = O.compute_encodings_from_stats(np.zeros(1, f32), np.zeros(1, f32), 255, False)
    assert hi[0] == f32(255 * 2.0 ** -23) and lo[0] == 0
    s, o = O.scale_offset(np.array([-1.0], f32), np.array([2.0], f32), -128, 127, False)
    assert s[0] == f32(3.0 / 255) and o[0] == f32(np.rint(-1.0 / s[0]) + 128)


def test_encoding_math_matches_torch_on_cpu():
    """The oracle's encoding math (CPU division) equals the torch expressions of
    encoding_analyzer.py:226-268 / quantizer.py:359-368 evaluated on the CPU."""
    g = np.random.default_rng(5)
    mn = -(g.random(300) * 3).astype(f32)
    mx = (g.random(300) * 3).astype(f32)
    for n, sym in ((255, False), (255, True), (15, True), (65535, False), (3, True)):
        lo, hi = O.compute_encodings_from_stats(mn, mx, n, sym)
        tmn, tmx = torch.from_numpy(mn), torch.from_numpy(mx)
        ms = O.minimum_scale(n)
        m0, x0 = torch.clamp(tmn, max=0), torch.clamp(tmx, min=0)
        adj = ms * ((x0 - m0) / n < ms)
        if sym:
            umax = x0 + (n // 2) * adj
            umin = m0 - (-(-n // 2)) * adj
            d = torch.maximum(umax / (n // 2 + (1 if n == 3 else 0)), -umin / (-(-n // 2)))
            umin, umax = -1 * (-(-n // 2)) * d, (n // 2) * d
        else:
            umax, umin = x0 + n * adj, m0
        np.testing.assert_array_equal(lo, umin.numpy())
        np.testing.assert_array_equal(hi, umax.numpy())
        s, o = O.scale_offset(lo, hi, 0, n, sym)
        ts = ((torch.from_numpy(hi) - torch.from_numpy(lo)) / n).abs().clamp_min_(ms)
        np.testing.assert_array_equal(s, ts.numpy())


def test_gpu_scalar_division_is_reciprocal_multiply():
    a = np.array([1.0, 3.0, 0.7, 1e-3], f32)
    np.testing.assert_array_equal(O.sdiv(a, 255, True), (a * f32(f32(1) / f32(255))).astype(f32))
    np.testing.assert_array_equal(O.sdiv(a, 255, False), (a / f32(255)).astype(f32))


# ---------------------------------------------------------------------------------
# General numerics (fp16 / bf16 tensors, internal types, zero_point_shift, any encoding
# shape).  The reference's operation sequence run by torch on CPU tensors of the real
# dtypes pins the oracle's per-operation rounding; torch's own casts pin round_to.
# ---------------------------------------------------------------------------------

TDT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16, "f64": torch.float64}


def _internal(io, qmin, qmax):
    """torch_builtins' widening rule (:85-101, 255-262) on the io type's eps."""
    for dt in (io, "f32", "f64"):
        eps = torch.finfo(TDT[dt]).eps
        if qmin == qmax or not eps > 1e-1 / (qmax - qmin):
            return dt
    return "f64"


def _edge_values():
    v = [0.0, -0.0, 1.0, 1.5, 2.5, -2.5, 65504.0, 65520.0, 65519.99, 1e-8, 6e-8, 2.0 ** -24,
         2.0 ** -25, 3.0 * 2.0 ** -26, 1 + 2.0 ** -8, 1 + 3 * 2.0 ** -9, 1 + 2.0 ** -9,
         3.3895314e38, np.inf, -np.inf, np.nan, 1e-40, -1e-40]
    return np.concatenate([np.array(v, f32), _data(5000, 40) * f32(3.7)])


@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_round_to_matches_torch_casts(dt):
    v = _edge_values()
    exp = torch.from_numpy(v).to(TDT[dt]).float().numpy()
    with np.errstate(over="ignore"):
        got = O.round_to(v, dt)
    np.testing.assert_array_equal(got, exp)
    # fp64 values reach 16-bit types through fp32, as torch's .to() does
    d = np.array([1 + 2.0 ** -11 + 2.0 ** -40, 1 + 2.0 ** -8 + 2.0 ** -30], np.float64)
    exp = torch.from_numpy(d).to(TDT[dt]).float().numpy()
    np.testing.assert_array_equal(O.to_io(d, dt), exp)


def _torch_qdq(x, scale, offset, qmin, qmax, io, internal, shift):
    """quantize_dequantize's learnable path (torch_builtins.py:255-284 + :640-672) as torch
    operations on CPU tensors of the real dtypes (dimensioned encodings)."""
    R = TDT[internal]
    xt = torch.from_numpy(x).to(TDT[io])
    s = torch.from_numpy(scale).to(R)
    o = torch.from_numpy(offset).to(R)
    sh = torch.sub(xt, s, alpha=shift) if shift else xt
    x_round = torch.round(sh.to(R) / s).sub_(o)
    mask = (qmin <= x_round) & (x_round <= qmax)
    y = x_round.clamp_(qmin, qmax).add_(o).mul_(s)
    if shift:
        y = torch.add(y, s, alpha=shift)
    return y.to(TDT[io]).float().numpy(), mask.numpy()


def _torch_qdq_backward(x, g, scale, offset, qmin, qmax, io, internal, shift):
    """QuantDequantFunc.backward (:675-691) and the shift's add/sub gradients, elementwise in
    the real dtypes, summed to the encoding shape in fp64."""
    R = TDT[internal]
    xt = torch.from_numpy(x).to(TDT[io])
    gt = torch.from_numpy(g).to(TDT[io]).to(R)
    s = torch.from_numpy(scale).to(R)
    o = torch.from_numpy(offset).to(R)
    sh = torch.sub(xt, s, alpha=shift) if shift else xt
    t = sh.to(R) / s
    x_round = torch.round(t) - o
    mask = (qmin <= x_round) & (x_round <= qmax)
    ds = gt * (torch.round(t).clamp(o + qmin, o + qmax) - (t * mask))
    do = gt * (~mask * s)
    dx = gt * mask
    ds64 = ds.double()
    if shift:
        ds64 = ds64 + (gt * shift).double() + (-(dx * shift)).double()
    enc = tuple(np.broadcast_shapes(scale.shape, offset.shape))
    return (dx.to(TDT[io]).float().numpy(), O._sum_to(ds64.numpy(), enc),
            O._sum_to(do.double().numpy(), enc))


CASES = [  # io, (qmin, qmax)
    ("f16", (-8, 7)), ("f16", (0, 63)), ("f16", (-128, 127)), ("bf16", (-4, 3)),
    ("bf16", (0, 255)), ("f32", (-128, 127)), ("f32", (0, (1 << 22) - 1)),
]


@pytest.mark.parametrize("io,grid", CASES, ids=[f"{c[0]}-{c[1][1]}" for c in CASES])
@pytest.mark.parametrize("shift", [0.0, 0.5])
@pytest.mark.parametrize("enc", ["per_tensor", "per_channel", "two_axes"])
def test_general_oracle_matches_torch_on_cpu(io, grid, shift, enc):
    qmin, qmax = grid
    internal = _internal(io, qmin, qmax)
    g = np.random.default_rng(qmax + int(shift * 10))
    shape = (6, 5, 40)
    enc_shape = {"per_tensor": (1,), "per_channel": (5, 1), "two_axes": (6, 1, 40)}[enc]
    x = O.round_to(_data(int(np.prod(shape)), qmax).reshape(shape) * f32(0.8), io)
    x.reshape(-1)[:6] = [np.nan, np.inf, -np.inf, 0.0, -0.0, 1e-3]
    gr = O.round_to(g.standard_normal(shape).astype(f32), io)
    steps = qmax - qmin
    scale = O.round_to((g.random(enc_shape) * 2 + 0.5).astype(f32) / f32(steps), internal)
    offset = np.full(enc_shape, f32(-round((qmin + qmax) / 2) if qmin < 0 else -(steps // 3)))
    scale, offset = scale.astype(f32), offset.astype(f32)
    y, mask = O.qdq_general(x, scale, offset, qmin, qmax, io, internal, shift)
    ey, emask = _torch_qdq(x, scale, offset, qmin, qmax, io, internal, shift)
    np.testing.assert_array_equal(y, ey)
    np.testing.assert_array_equal(mask, emask)
    dx, ds, do = O.qdq_general_backward(x, gr, scale, offset, qmin, qmax, io, internal, shift)
    edx, eds, edo = _torch_qdq_backward(x, gr, scale, offset, qmin, qmax, io, internal, shift)
    np.testing.assert_array_equal(dx, edx)
    # the oracle's sums are rounded to the internal type; the reference rounds its sum too
    ulp = 2.0 ** -10 if internal == "f16" else 2.0 ** -7 if internal == "bf16" else 1e-6
    for a, e in ((ds, eds), (do, edo)):
        fin = np.isfinite(e)
        if fin.any():
            np.testing.assert_allclose(a[fin], e[fin], rtol=ulp,
                                       atol=ulp * np.abs(e[fin]).max())
        assert np.array_equal(np.isnan(a), np.isnan(e))


@pytest.mark.parametrize("io", ["f16", "bf16", "f32"])
def test_shift_grid_invariant(io):
    """With a power-of-two scale every step is exact: y = (k + offset + shift) * scale for an
    integer k in [qmin, qmax], inputs beyond the grid land on its ends, and a NaN stays NaN."""
    qmin, qmax, s, o = -8, 7, 2.0 ** -3, 0.0
    internal = _internal(io, qmin, qmax)
    x = O.round_to(np.linspace(-3, 3, 401).astype(f32), io)
    y, _ = O.qdq_general(x, f32(s), f32(o), qmin, qmax, io, internal, 0.5)
    k = y / s - 0.5 - o
    np.testing.assert_array_equal(k, np.rint(k))
    assert k.min() == qmin and k.max() == qmax
    # the nearest grid point: |x - y| <= s / 2 inside the grid
    inside = (x >= (qmin + 0.5) * s) & (x <= (qmax + 0.5) * s)
    assert np.all(np.abs(x[inside] - y[inside]) <= s / 2)
    assert np.isnan(O.qdq_general(np.array([np.nan], f32), f32(s), f32(o), qmin, qmax, io,
                                  internal, 0.5)[0][0])


def test_general_oracle_equals_fp32_oracle():
    """io = internal = fp32 without a shift reduces to the [outer, C, inner] oracle."""
    x = _data(3 * 7 * 50, 41).reshape(3, 7, 50)
    g = _data(x.size, 42).reshape(x.shape)
    s = (np.random.default_rng(43).random(7) * 0.05 + 0.01).astype(f32)
    o = np.full(7, f32(-3))
    y, m = O.qdq_general(x, s.reshape(7, 1), o.reshape(7, 1), -8, 7)
    ey, em = O.qdq_learnable(x, s, o, -8, 7, (3, 7, 50))
    np.testing.assert_array_equal(y, ey)
    dx, ds, do = O.qdq_general_backward(x, g, s.reshape(7, 1), o.reshape(7, 1), -8, 7)
    edx, eds, edo = O.qdq_learnable_backward(x, g, s, o, -8, 7, (3, 7, 50))
    np.testing.assert_array_equal(dx, edx)
    np.testing.assert_array_equal(ds.reshape(-1), eds)
    np.testing.assert_array_equal(do.reshape(-1), edo)
    q = O.quantize_general(x, s.reshape(7, 1), o.reshape(7, 1), 0, 15)
    np.testing.assert_array_equal(q, O.quantize(x, s, o, 0, 15, (3, 7, 50)))
    qd = O.quantize_general_backward(x, g, s.reshape(7, 1), o.reshape(7, 1), 0, 15)
    eq = O.quantize_backward(x, g, s, o, 0, 15, (3, 7, 50))
    np.testing.assert_array_equal(qd[0], eq[0])
    np.testing.assert_array_equal(qd[1].reshape(-1), eq[1])
    np.testing.assert_array_equal(qd[2].reshape(-1), eq[2])
    dq = O.dequantize_general(q, s.reshape(7, 1), o.reshape(7, 1))
    np.testing.assert_array_equal(dq, O.dequantize(q, s, o, (3, 7, 50)))


@pytest.mark.parametrize("io,grid", [("f16", (-8, 7)), ("bf16", (0, 255)), ("f16", (0, 255))])
def test_quantize_and_dequantize_general_match_torch(io, grid):
    qmin, qmax = grid
    internal = _internal(io, qmin, qmax)
    x = O.round_to(_data(4 * 300, 44).reshape(4, 300), io)
    g = O.round_to(_data(x.size, 45).reshape(x.shape), io)
    scale = O.round_to(np.array([[0.05], [0.11], [0.013], [0.3]], f32), internal)
    offset = np.array([[0.0], [-2.0], [3.0], [-1.0]], f32)
    R, T = TDT[internal], TDT[io]
    xt, gt = torch.from_numpy(x).to(T), torch.from_numpy(g).to(T)
    s, o = torch.from_numpy(scale).to(R), torch.from_numpy(offset).to(R)
    # QuantizeFunc.forward / backward (:527-571) in R, result .to(T)
    x_round = torch.round(xt.to(R) / s).sub_(o)
    mask = (x_round >= qmin) * (x_round <= qmax)
    q_ref = x_round.clamp_(qmin, qmax).to(T).float().numpy()
    np.testing.assert_array_equal(O.quantize_general(x, scale, offset, qmin, qmax, io, internal),
                                  q_ref)
    mg = gt.to(R) * mask
    dx_ref = (mg / s).to(T).float().numpy()
    ds_ref = O._sum_to((-(mg / s) * (xt / s)).double().numpy(), scale.shape)
    dx, ds, do = O.quantize_general_backward(x, g, scale, offset, qmin, qmax, io, internal)
    np.testing.assert_array_equal(dx, dx_ref)
    ulp = 2.0 ** -10 if internal == "f16" else 2.0 ** -7 if internal == "bf16" else 1e-6
    np.testing.assert_allclose(ds, ds_ref, rtol=ulp, atol=ulp * np.abs(ds_ref).max())
    np.testing.assert_allclose(do, O._sum_to((-mg).double().numpy(), scale.shape), rtol=ulp)
    # DequantizeFunc (:589-615) in the tensor's type
    qt = torch.from_numpy(q_ref).to(T)
    sT, oT = s.to(T), o.to(T)
    y_ref = (qt + oT).mul_(sT).float().numpy()
    sv, ov = O.round_to(scale, io), O.round_to(offset, io)
    np.testing.assert_array_equal(O.dequantize_general(q_ref, sv, ov, io), y_ref)
    gq, dsq, doq = O.dequantize_general_backward(q_ref, g, sv, ov, io)
    np.testing.assert_array_equal(gq, (gt * sT).float().numpy())
    ulp_io = 2.0 ** -10 if io == "f16" else 2.0 ** -7
    eds = O._sum_to((gt * (qt + oT)).double().numpy(), scale.shape)
    np.testing.assert_allclose(dsq, eds, rtol=ulp_io, atol=ulp_io * np.abs(eds).max())
    edo = O._sum_to((gt * sT).double().numpy(), scale.shape)
    np.testing.assert_allclose(doq, edo, rtol=ulp_io, atol=ulp_io * np.abs(edo).max())
