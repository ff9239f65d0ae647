"""GPU parity of the general fake-quantization entry points (rxmet_qdq.h, *_ex): fp16 / bf16
tensors, the reference's internal arithmetic type (the tensor's type, fp32 or fp64),
zero_point_shift, 0-dim scales, and encodings on two separated axis groups, against the
oracle's general restatement (oracle/qdq_oracle.py, pinned against torch's CPU arithmetic by
tests/test_qdq_oracle.py) and against torch running the reference's operations on the GPU
(for the 0-dim scale promotion, which only the GPU shows).

Bars: outputs, masks and dx bit-exact; encoding gradients within one unit in the last place
of the internal type (sums in a different order, each rounded to that type)."""
import ctypes

import numpy as np
import pytest
import torch

import mi355x_qdq as Q
import qdq_oracle as O
import rxmet_lib as L

pytestmark = pytest.mark.gpu
f32 = np.float32
TDT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16, "f64": torch.float64}
CODE = {"f32": 0, "f16": 1, "bf16": 2, "f64": 3}
ULP = {"f16": 2.0 ** -10, "bf16": 2.0 ** -7, "f32": 2e-6, "f64": 2e-6}


def _internal(io, qmin, qmax):
    for dt in (io, "f32", "f64"):
        if qmin == qmax or not torch.finfo(TDT[dt]).eps > 1e-1 / (qmax - qmin):
            return dt
    return "f64"


def _dev(a, io, cuda):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=f32)).to(cuda).to(TDT[io])


def _host(t):
    return t.float().cpu().numpy()


def _close(a, e, dt, what):
    fin = np.isfinite(e)
    assert np.array_equal(np.isnan(a), np.isnan(e)), what
    if fin.any():
        tol = ULP[dt]
        np.testing.assert_allclose(a[fin], e[fin], rtol=tol, atol=tol * np.abs(e[fin]).max(),
                                   err_msg=what)


# [outer, C0, mid, C1, inner] layouts: per-tensor, long runs, medium runs (aligned and not),
# short runs (narrow and wide matrices), and two encoding groups in each decomposition
LAYOUTS = [
    (1, 1, 1, 1, 70001),
    (1, 1, 2, 6, 3000),
    (1, 1, 5, 24, 64),
    (1, 1, 3, 8, 50),
    (1, 1, 300, 16, 1),
    (1, 1, 40, 700, 2),
    (2, 3, 4, 5, 64),
    (2, 3, 7, 5, 1),
    (1, 4, 3, 2, 2048),
]
GRIDS = [("f16", -8, 7), ("f16", -128, 127), ("bf16", -4, 3), ("bf16", 0, 255),
         ("f32", -128, 127), ("f32", 0, (1 << 21) - 1)]


def _case(layout, io, qmin, qmax, seed):
    g = np.random.default_rng(seed)
    shape = tuple(layout)
    n = int(np.prod(shape))
    x = g.standard_normal(n).astype(f32)
    m = g.random(n) < 0.01
    x[m] *= 10
    if n > 6:
        x[:6] = [np.nan, np.inf, -np.inf, 0.0, -0.0, 1e-3]
    x = O.round_to(x.reshape(shape), io)
    gr = O.round_to(g.standard_normal(shape).astype(f32), io)
    enc_shape = (1, layout[1], 1, layout[3], 1)
    steps = qmax - qmin
    scale = ((g.random(enc_shape) * 2 + 0.5) / steps).astype(f32)
    off = -np.round((qmin + qmax) / 2) if qmin < 0 else -(steps // 3)
    offset = np.full(enc_shape, f32(off))
    return x, gr, scale, offset


def _lay(layout):
    return L.QdqLayout(*layout)


def _num(io, internal, shift=0.0, scalar=False):
    return L.QdqNumerics(CODE[io], CODE[internal], shift, int(scalar), 0)


def _ws(layout, io, cuda):
    n = L.load().rxmet_qdq_workspace_bytes_ex(_lay(layout), CODE[io])
    return torch.empty(max(16, n), dtype=torch.uint8, device=cuda)


def _stream(cuda):
    return torch.cuda.current_stream(cuda).cuda_stream


@pytest.mark.parametrize("layout", LAYOUTS, ids=[str(l) for l in LAYOUTS])
@pytest.mark.parametrize("io,qmin,qmax", GRIDS, ids=[f"{g[0]}{g[2]}" for g in GRIDS])
@pytest.mark.parametrize("shift", [0.0, 0.5])
def test_learnable_qdq_matches_oracle(cuda, layout, io, qmin, qmax, shift):
    internal = _internal(io, qmin, qmax)
    print(f"[qdq ex] layout={layout} io={io} internal={internal} grid=({qmin},{qmax}) "
          f"shift={shift}", flush=True)
    x, gr, scale, offset = _case(layout, io, qmin, qmax, sum(layout) + qmax)
    scale = O.round_to(scale, internal).astype(f32)
    xd, gd = _dev(x, io, cuda), _dev(gr, io, cuda)
    sd = torch.from_numpy(scale.reshape(-1)).to(cuda)
    od = torch.from_numpy(offset.reshape(-1)).to(cuda)
    y = torch.empty_like(xd)
    num = _num(io, internal, shift)
    L.call("rxmet_qdq_forward_ex", xd.data_ptr(), y.data_ptr(), _lay(layout), num, sd.data_ptr(),
           od.data_ptr(), qmin, qmax, Q.LEARNABLE, _stream(cuda))
    dx = torch.empty_like(xd)
    C = sd.numel()
    ds, do = torch.empty(C, device=cuda), torch.empty(C, device=cuda)
    L.call("rxmet_qdq_backward_ex", xd.data_ptr(), gd.data_ptr(), dx.data_ptr(), ds.data_ptr(),
           do.data_ptr(), _lay(layout), num, sd.data_ptr(), od.data_ptr(), qmin, qmax,
           Q.LEARNABLE, _ws(layout, io, cuda).data_ptr(), _stream(cuda))
    torch.cuda.synchronize()
    ey, _ = O.qdq_general(x, scale, offset, qmin, qmax, io, internal, shift)
    edx, eds, edo = O.qdq_general_backward(x, gr, scale, offset, qmin, qmax, io, internal,
                                           shift)
    np.testing.assert_array_equal(_host(y), ey)
    np.testing.assert_array_equal(_host(dx), edx)
    _close(ds.cpu().numpy(), eds.reshape(-1), internal, "dscale")
    _close(do.cpu().numpy(), edo.reshape(-1), internal, "doffset")


@pytest.mark.parametrize("layout", LAYOUTS[:3] + LAYOUTS[4:7], ids=str)
@pytest.mark.parametrize("io,qmin,qmax", [("f16", -8, 7), ("bf16", 0, 255), ("f16", 0, 255),
                                          ("f32", -8, 7)], ids=str)
def test_quantize_dequantize_match_oracle(cuda, layout, io, qmin, qmax):
    internal = _internal(io, qmin, qmax)
    print(f"[q/dq ex] layout={layout} io={io} internal={internal}", flush=True)
    x, gr, scale, offset = _case(layout, io, qmin, qmax, 7 + qmax)
    scale = O.round_to(scale, internal).astype(f32)
    xd, gd = _dev(x, io, cuda), _dev(gr, io, cuda)
    sd = torch.from_numpy(scale.reshape(-1)).to(cuda)
    od = torch.from_numpy(offset.reshape(-1)).to(cuda)
    C = sd.numel()
    num = _num(io, internal)
    q = torch.empty_like(xd)
    L.call("rxmet_quantize_forward_ex", xd.data_ptr(), q.data_ptr(), _lay(layout), num,
           sd.data_ptr(), od.data_ptr(), qmin, qmax, _stream(cuda))
    dx, ds, do = torch.empty_like(xd), torch.empty(C, device=cuda), torch.empty(C, device=cuda)
    L.call("rxmet_quantize_backward_ex", xd.data_ptr(), gd.data_ptr(), dx.data_ptr(),
           ds.data_ptr(), do.data_ptr(), _lay(layout), num, sd.data_ptr(), od.data_ptr(), qmin,
           qmax, _ws(layout, io, cuda).data_ptr(), _stream(cuda))
    torch.cuda.synchronize()
    eq = O.quantize_general(x, scale, offset, qmin, qmax, io, internal)
    edx, eds, edo = O.quantize_general_backward(x, gr, scale, offset, qmin, qmax, io, internal)
    np.testing.assert_array_equal(_host(q), eq)
    np.testing.assert_array_equal(_host(dx), edx)
    _close(ds.cpu().numpy(), eds.reshape(-1), internal, "dscale")
    _close(do.cpu().numpy(), edo.reshape(-1), internal, "doffset")
    # dequantize in the tensor's own type
    sv, ov = O.round_to(scale, io).astype(f32), O.round_to(offset, io).astype(f32)
    svd, ovd = torch.from_numpy(sv.reshape(-1)).to(cuda), torch.from_numpy(ov.reshape(-1)).to(cuda)
    numd = _num(io, io)
    y = torch.empty_like(q)
    L.call("rxmet_dequantize_forward_ex", q.data_ptr(), y.data_ptr(), _lay(layout), numd,
           svd.data_ptr(), ovd.data_ptr(), _stream(cuda))
    L.call("rxmet_dequantize_backward_ex", q.data_ptr(), gd.data_ptr(), dx.data_ptr(),
           ds.data_ptr(), do.data_ptr(), _lay(layout), numd, svd.data_ptr(), ovd.data_ptr(),
           _ws(layout, io, cuda).data_ptr(), _stream(cuda))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_host(y), O.dequantize_general(eq, sv, ov, io))
    egq, edsq, edoq = O.dequantize_general_backward(eq, gr, sv, ov, io)
    np.testing.assert_array_equal(_host(dx), egq)
    _close(ds.cpu().numpy(), edsq.reshape(-1), io, "dequantize dscale")
    _close(do.cpu().numpy(), edoq.reshape(-1), io, "dequantize doffset")


@pytest.mark.parametrize("layout", [LAYOUTS[0], LAYOUTS[2], LAYOUTS[4], LAYOUTS[6]], ids=str)
@pytest.mark.parametrize("io", ["f16", "bf16", "f32"])
def test_minmax_any_type_and_layout(cuda, layout, io):
    x, _, _, _ = _case(layout, io, -8, 7, 11)
    x = x.copy()
    x.reshape(-1)[:6] = np.arange(6, dtype=f32)  # finite: exact min / max
    xd = _dev(x, io, cuda)
    C = layout[1] * layout[3]
    mn, mx = torch.empty(C, device=cuda), torch.empty(C, device=cuda)
    L.call("rxmet_qdq_minmax_ex", xd.data_ptr(), CODE[io], _lay(layout), mn.data_ptr(),
           mx.data_ptr(), _ws(layout, io, cuda).data_ptr(), _stream(cuda))
    torch.cuda.synchronize()
    emn, emx = O.minmax_general(x, (1, layout[1], 1, layout[3], 1))
    np.testing.assert_array_equal(mn.cpu().numpy(), emn.reshape(-1))
    np.testing.assert_array_equal(mx.cpu().numpy(), emx.reshape(-1))


# ---------------------------------------------------------------------------------
# Through the backend (mi355x_qdq), against torch running the reference's operations on the
# GPU: the reference's semantics including type promotion of 0-dim scales.
# ---------------------------------------------------------------------------------


def _torch_reference(x, scale, offset, qmin, qmax, shift, block_size=None):
    """torch_builtins.quantize_dequantize's learnable path (:255-284, QuantDequantFunc
    :640-691) as torch operations on the GPU, with autograd through a surrogate whose
    backward is QuantDequantFunc.backward."""

    class QDQ(torch.autograd.Function):
        @staticmethod
        def forward(ctx, t, s, o):
            x_round = torch.round(t.to(s.dtype) / s).sub_(o)
            mask = (qmin <= x_round) & (x_round <= qmax)
            ctx.save_for_backward(t, s, o, mask)
            return x_round.clamp_(qmin, qmax).add_(o).mul_(s)

        @staticmethod
        def backward(ctx, grad):
            t, s, o, mask = ctx.saved_tensors
            tt = t.to(s.dtype) / s
            sg = grad * (torch.round(tt).clamp(o + qmin, o + qmax) - (tt * mask))
            return grad * mask, sg, grad * (~mask * s)

    internal = x.dtype
    if not Q._is_numerically_stable(internal, qmin, qmax):
        internal = torch.float32
        if not Q._is_numerically_stable(internal, qmin, qmax):
            internal = torch.float64
    orig = x.shape
    t = Q.reshape_tensor_for_blocks(x, scale.shape, block_size)
    s = scale.view(Q.get_encoding_shape_with_blocks(scale.shape, block_size)).to(internal)
    o = offset.view(Q.get_encoding_shape_with_blocks(offset.shape, block_size))
    sh = torch.sub(t, s, alpha=shift) if shift else t
    y = QDQ.apply(sh, s, o.to(internal))
    if shift:
        y = torch.add(y, s, alpha=shift)
    return y.to(x.dtype).view(orig)


def _run_both(x, scale, offset, qmin, qmax, shift, g, block_size=None):
    outs = []
    for fn in (Q.quantize_dequantize, None):
        xs = x.clone().requires_grad_(True)
        ss = scale.clone().requires_grad_(True)
        os_ = offset.clone().requires_grad_(True)
        if fn is None:
            y = _torch_reference(xs, ss, os_, qmin, qmax, shift, block_size)
        else:
            y = fn(xs, ss, os_, qmin, qmax, block_size=block_size, zero_point_shift=shift)
        y.backward(g)
        outs.append((y.detach(), xs.grad, ss.grad, os_.grad))
    return outs


BACKEND_CASES = [  # tensor dtype, grid, scale shape, tensor shape
    (torch.float16, (-8, 7), (), (64, 257)),
    (torch.float16, (-128, 127), (), (64, 257)),
    (torch.bfloat16, (-128, 127), (), (64, 257)),
    (torch.float16, (-128, 127), (64, 1), (64, 257)),
    (torch.bfloat16, (-2, 1), (1, 257), (64, 257)),
    (torch.float32, (-128, 127), (), (64, 257)),
    (torch.float32, (-(1 << 22), (1 << 22) - 1), (), (64, 257)),
    (torch.float16, (-8, 7), (4, 1, 8), (4, 33, 8)),
    (torch.float64, (-128, 127), (), (64, 257)),
    (torch.float64, (-8, 7), (64, 1), (64, 257)),
    (torch.float64, (-(1 << 22), (1 << 22) - 1), (1, 257), (64, 257)),
]


@pytest.mark.parametrize("dtype,grid,sshape,shape", BACKEND_CASES, ids=[
    f"{c[0]}-{c[1][1]}-{c[2]}" for c in BACKEND_CASES])
@pytest.mark.parametrize("shift", [0.0, 0.5])
def test_backend_matches_torch_reference_on_gpu(cuda, dtype, grid, sshape, shape, shift):
    qmin, qmax = grid
    print(f"[qdq backend] {dtype} grid={grid} scale{sshape} x{shape} shift={shift}", flush=True)
    gen = torch.Generator().manual_seed(qmax + len(sshape))
    x = (torch.randn(shape, generator=gen) * 1.5).to(dtype).to(cuda)
    x.view(-1)[:3] = torch.tensor([float("nan"), float("inf"), -2.0], dtype=dtype)
    g = torch.randn(shape, generator=gen).to(dtype).to(cuda)
    steps = qmax - qmin
    scale = ((torch.rand(sshape, generator=gen) + 0.5) * 3.0 / steps).to(cuda)
    offset = torch.full(sshape, -float(round((qmin + qmax) / 2))).to(cuda)
    (y, dx, ds, do), (ey, edx, eds, edo) = _run_both(x, scale, offset, qmin, qmax, shift, g)
    assert y.dtype == dtype and dx.dtype == dtype
    assert torch.equal(torch.isnan(y), torch.isnan(ey))
    assert torch.equal(y[~torch.isnan(y)], ey[~torch.isnan(ey)])
    assert torch.equal(dx, edx)
    internal = Q._internal_dtype(dtype, qmin, qmax)
    tol = {torch.float16: 2.0 ** -10, torch.bfloat16: 2.0 ** -7}.get(internal, 2e-6)
    for a, e, what in ((ds, eds, "scale"), (do, edo, "offset")):
        a, e = a.double().cpu().numpy(), e.double().cpu().numpy()
        fin = np.isfinite(e)
        assert np.array_equal(np.isnan(a), np.isnan(e)), what
        if fin.any():
            np.testing.assert_allclose(a[fin], e[fin], rtol=tol, atol=tol * np.abs(e[fin]).max(),
                                       err_msg=what)


@pytest.mark.parametrize("sshape", [(), (64, 1)])
def test_shift_not_exact_in_fp32_on_a_double_grid(cuda, sshape):
    """A grid of more than 838,860 steps computes in fp64 (the reference's stability rule),
    where torch.sub / torch.add(..., alpha=shift) use the shift at double precision: a shift
    of 0.1, which fp32 cannot hold, must enter the double arithmetic unrounded."""
    qmin, qmax = -(1 << 22), (1 << 22) - 1
    shift = 0.1
    print(f"[qdq backend] f64 internal shift={shift} scale{sshape}", flush=True)
    gen = torch.Generator().manual_seed(77)
    shape = (64, 257)
    x = (torch.randn(shape, generator=gen) * 1.5).to(cuda)
    g = torch.randn(shape, generator=gen).to(cuda)
    scale = ((torch.rand(sshape, generator=gen) + 0.5) * 3.0 / (qmax - qmin)).to(cuda)
    offset = torch.zeros(sshape).to(cuda)
    assert Q._internal_dtype(torch.float32, qmin, qmax) == torch.float64
    (y, dx, ds, do), (ey, edx, eds, edo) = _run_both(x, scale, offset, qmin, qmax, shift, g)
    assert torch.equal(y, ey)
    assert torch.equal(dx, edx)
    for a, e, what in ((ds, eds, "scale"), (do, edo, "offset")):
        a, e = a.double().cpu().numpy(), e.double().cpu().numpy()
        np.testing.assert_allclose(a, e, rtol=2e-6, atol=2e-6 * np.abs(e).max(), err_msg=what)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("block_size,sshape,shape", [
    ((16, 32), (4, 8), (64, 256)),      # two-dimensional blocks: two encoding groups
    ((1, 64), (32, 4), (32, 256)),      # blocks along the last axis: one group
    ((2, 4, 8), (3, 5, 4), (6, 20, 32)),  # three groups: the permuted path
])
def test_block_quantization_matches_torch_reference(cuda, dtype, block_size, sshape, shape):
    qmin, qmax = -8, 7
    print(f"[qdq blocks] {dtype} block={block_size} x{shape}", flush=True)
    gen = torch.Generator().manual_seed(len(shape) + shape[-1])
    x = torch.randn(shape, generator=gen).to(dtype).to(cuda)
    g = torch.randn(shape, generator=gen).to(dtype).to(cuda)
    scale = ((torch.rand(sshape, generator=gen) + 0.5) / 5).to(cuda)
    offset = torch.zeros(sshape, device=cuda)
    (y, dx, ds, do), (ey, edx, eds, edo) = _run_both(x, scale, offset, qmin, qmax, 0.0, g,
                                                     block_size=list(block_size))
    assert torch.equal(y, ey) and torch.equal(dx, edx)
    internal = Q._internal_dtype(dtype, qmin, qmax)
    tol = {torch.float16: 2.0 ** -10, torch.bfloat16: 2.0 ** -7}.get(internal, 2e-6)
    for a, e in ((ds, eds), (do, edo)):
        a, e = a.double().cpu().numpy(), e.double().cpu().numpy()
        np.testing.assert_allclose(a, e, rtol=tol, atol=tol * np.abs(e).max())


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("per_channel", [False, True])
def test_frozen_fast_path_matches_torch_fake_quantize(cuda, dtype, per_channel):
    """Frozen encodings on a 16-bit tensor: torch.fake_quantize is the reference's own path
    (torch_builtins.py:287-361), NaN restored (:249).  It computes the result in fp32 and
    rounds that to the tensor's type; the checker is torch's CPU kernel, because the ROCm build
    of torch's GPU kernel lets the compiler fold the last multiply into the fp16 conversion
    (v_fma_mixlo_f16: one rounding of the exact product), which differs on fp16 ties — seed 3
    has three such elements in the per-channel case."""
    gen = torch.Generator().manual_seed(3)
    x = (torch.randn(96, 1000, generator=gen) * 2).to(dtype).to(cuda)
    x[0, :3] = torch.tensor([float("nan"), float("inf"), -float("inf")], dtype=dtype)
    xc = x.cpu()
    if per_channel:
        scale = (torch.rand(96, 1, generator=gen) * 0.05 + 0.01).to(cuda)
        offset = torch.zeros(96, 1, device=cuda)
        ref = torch.fake_quantize_per_channel_affine(
            xc, scale.flatten().cpu(), torch.zeros(96, dtype=torch.int32), 0, -128, 127)
    else:
        scale = torch.tensor(0.0173, device=cuda)
        offset = torch.tensor(-3.0, device=cuda)
        ref = torch.fake_quantize_per_tensor_affine(xc, scale.cpu(), torch.tensor(3, dtype=torch.int32),
                                                    -128, 127)
    ref = ref.masked_fill_(torch.isnan(xc), float("nan")).to(cuda)
    y = Q.quantize_dequantize(x, scale, offset, -128, 127)
    assert y.dtype == dtype
    fin = torch.isfinite(x)
    assert torch.equal(torch.isnan(y), torch.isnan(x))
    assert torch.equal(y[fin], ref[fin])
    # +-inf: the grid's saturation contract of the reference's own test
    # (tests/integration/test_native_qdq_alignment.py:139-148); aten's fake_quantize converts
    # +-inf to int64 (undefined) and on fp16 wraps +inf to the bottom of the grid
    s0 = scale.flatten()[0].item()
    zp = 3 if not per_channel else 0
    assert y[0, 1].item() == torch.tensor((127 - zp) * s0).to(dtype).item()
    assert y[0, 2].item() == torch.tensor((-128 - zp) * s0).to(dtype).item()


@pytest.mark.parametrize("per_channel", [False, True])
def test_frozen_fast_path_on_fp64_matches_torch_fake_quantize(cuda, per_channel):
    """Frozen encodings on an fp64 tensor: the reference's torch.fake_quantize on the GPU
    (aten's kernel: x times the fp32 1 / scale and its rounding in fp64, the clamp, zero point
    and scale in fp32), NaN restored.  Checked against that very kernel."""
    gen = torch.Generator().manual_seed(5)
    x = (torch.randn(96, 1000, generator=gen, dtype=torch.float64) * 2).to(cuda)
    x[0, :1] = float("nan")
    if per_channel:
        scale = (torch.rand(96, 1, generator=gen) * 0.05 + 0.01).to(cuda)
        offset = torch.zeros(96, 1, device=cuda)
        ref = torch.fake_quantize_per_channel_affine(
            x, scale.flatten(), torch.zeros(96, dtype=torch.int32, device=cuda), 0, -128, 127)
    else:
        scale = torch.tensor(0.0173, device=cuda)
        offset = torch.tensor(-3.0, device=cuda)
        ref = torch.fake_quantize_per_tensor_affine(
            x, scale, torch.tensor(3, dtype=torch.int32, device=cuda), -128, 127)
    ref = ref.masked_fill_(torch.isnan(x), float("nan"))
    y = Q.quantize_dequantize(x, scale, offset, -128, 127)
    assert y.dtype == torch.float64
    assert torch.equal(torch.isnan(y), torch.isnan(x))
    fin = torch.isfinite(x)
    assert torch.equal(y[fin], ref[fin])
    # the gradient is the fake_quantize mask
    xs = x.clone().requires_grad_(True)
    g = torch.randn(x.shape, generator=gen, dtype=torch.float64).to(cuda)
    Q.quantize_dequantize(xs, scale, offset, -128, 127).backward(g)
    xr = x.clone().requires_grad_(True)
    if per_channel:
        torch.fake_quantize_per_channel_affine(
            xr, scale.flatten(), torch.zeros(96, dtype=torch.int32, device=cuda), 0, -128,
            127).backward(g)
    else:
        torch.fake_quantize_per_tensor_affine(
            xr, scale, torch.tensor(3, dtype=torch.int32, device=cuda), -128, 127).backward(g)
    assert torch.equal(xs.grad[fin], xr.grad[fin])


def test_fp64_module_forward_backward_matches_torch_reference(cuda):
    """aimet's QuantizeDequantize on an fp64 input (fp32 learnable min / max): the tensor
    computes in fp64, as the reference's backend does; checked against the reference's
    operations run by torch on the GPU with the module's own encodings."""
    import aimet_affine as A

    gen = torch.Generator().manual_seed(9)
    x = (torch.randn(64, 300, generator=gen, dtype=torch.float64) * 1.3).to(cuda)
    g = torch.randn(64, 300, generator=gen, dtype=torch.float64).to(cuda)
    for shape, bits, sym in (((), 8, False), ((64, 1), 4, True)):
        q = A.QuantizeDequantize(shape, bits, sym).to(cuda)
        with q.compute_encodings():
            q(x)
        xs = x.clone().requires_grad_(True)
        y = q(xs)
        y.backward(g)
        assert y.dtype == torch.float64 and xs.grad.dtype == torch.float64
        scale, offset = q.get_scale().detach(), q.get_offset().detach()
        xr = x.clone().requires_grad_(True)
        yr = _torch_reference(xr, scale, offset, q.qmin, q.qmax, 0.0)
        yr.backward(g)
        assert torch.equal(torch.isnan(y), torch.isnan(yr))
        assert torch.equal(y.detach(), yr.detach()), (shape, bits)
        assert torch.equal(xs.grad, xr.grad), (shape, bits)


def test_backend_quantize_dequantize_16bit(cuda):
    """quantize / dequantize of a bf16 tensor against the reference's operations on the GPU
    (QuantizeFunc in fp32 for an 8-bit grid, DequantizeFunc in bf16)."""
    gen = torch.Generator().manual_seed(9)
    x = torch.randn(40, 300, generator=gen).to(torch.bfloat16).to(cuda)
    scale = (torch.rand(40, 1, generator=gen) * 0.05 + 0.01).to(cuda)
    offset = torch.full((40, 1), -3.0, device=cuda)
    q = Q.quantize(x, scale, offset, 0, 255)
    ref = torch.round(x.to(torch.float32) / scale).sub_(offset).clamp_(0, 255).to(torch.bfloat16)
    assert q.dtype == torch.bfloat16 and torch.equal(q, ref)
    y = Q.dequantize(q, scale, offset)
    ref_y = (q + offset.to(torch.bfloat16)).mul_(scale.to(torch.bfloat16))
    assert y.dtype == torch.bfloat16 and torch.equal(y, ref_y)
    lo, hi = Q.minmax(x, (40, 1))
    assert lo.dtype == torch.bfloat16
    assert torch.equal(lo, x.amin(dim=1, keepdim=True)) and torch.equal(hi, x.amax(dim=1,
                                                                                keepdim=True))


def _tf_grid(bits, scale, offset=None):
    off = -(1 << (bits - 1)) if offset is None else offset
    return off * scale, (off + (1 << bits) - 1) * scale


def _frozen_qdq(x, scales, bits, offset, cuda):
    """The backend's frozen-encoding QDQ with the aimet grid of a TfEncoding (symmetric:
    signed codes and offset 0; otherwise unsigned codes and the given offset)."""
    shape = (len(scales), 1) if len(scales) > 1 else ()
    scale = torch.tensor(scales, dtype=torch.float32).reshape(shape).to(cuda)
    if offset is None:
        qmin, qmax, off = -(1 << (bits - 1)), (1 << (bits - 1)) - 1, 0.0
    else:
        qmin, qmax, off = 0, (1 << bits) - 1, float(offset)
    offs = torch.full(shape, off, dtype=torch.float32, device=cuda)
    return Q.quantize_dequantize(torch.from_numpy(x).to(cuda), scale, offs, qmin, qmax).cpu().numpy()


def test_native_libpymo_qdq_alignment_on_gpu(cuda):
    """The cases of the reference's native-vs-Torch alignment test
    (tests/integration/test_native_qdq_alignment.py:88-137) through this backend's frozen QDQ
    equal the native form stableQuantizeDequantize (quantize_dequantize.hpp:35-46): exact
    codes with int32 offsets, per-channel 32-bit grids, ties to even at 8/16/32 bits on
    symmetric and asymmetric grids, the float32 reciprocal of decimal scales, NaN kept and
    infinity clipped."""
    cases = []
    codes = np.array([-257, -65, -7, -3, -1, 0, 1, 3, 7, 65, 257], dtype=f32)
    cases.append(((codes * f32(2.0 ** -21)).reshape(1, -1), 32, [2.0 ** -21], None))
    codes = np.array([-7, -3, -1, 0, 1, 3, 7], dtype=f32)
    sc = [2.0 ** -21, 2.0 ** -20]
    cases.append((np.stack([codes * f32(s) for s in sc]), 32, sc, None))
    codes = np.array([-7.5, -3.5, -2.5, -1.5, -.5, .5, 1.5, 2.5, 3.5, 7.5], dtype=f32)
    for bits in (8, 16, 32):
        s = 2.0 ** -7 if bits == 8 else 2.0 ** -15 if bits == 16 else 2.0 ** -21
        for off in (None, -13):
            cases.append(((codes * f32(s)).reshape(1, -1), bits, [s], off))
    for s in (1.0 / 32767, .013007, .027019):
        cases.append((((np.arange(-63, 64, dtype=f32) + f32(.5)) * f32(s)).reshape(1, -1), 16, [s], None))
    for bits in (8, 16, 32):
        s = 2.0 ** -7 if bits == 8 else 2.0 ** -15 if bits == 16 else 2.0 ** -21
        cases.append((np.array([[np.nan, -np.inf, -s, 0, s, np.inf]], dtype=f32), bits, [s], None))
    for x, bits, scales, off in cases:
        print(f"[native alignment] bits={bits} scales={scales} offset={off}", flush=True)
        s = np.array(scales, dtype=f32).reshape(-1, 1) if len(scales) > 1 else f32(scales[0])
        lo, hi = _tf_grid(bits, np.asarray(scales, dtype=np.float64).reshape(np.shape(s)), off)
        expect = O.native_qdq(x, f32(lo) if np.ndim(lo) == 0 else lo.astype(f32),
                              f32(hi) if np.ndim(hi) == 0 else hi.astype(f32), s)
        np.testing.assert_array_equal(_frozen_qdq(x, scales, bits, off, cuda), expect)
