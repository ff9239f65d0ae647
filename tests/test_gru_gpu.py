"""GPU parity of the QuantGRU kernels against the pinned oracle (oracle/gru_oracle.c).

Bar: every forward output (codes, masks, dequantised h and v) bit-exact; backward
gradients within 1e-4 relative of the oracle (fp32 GEMM summation order differs from the
oracle's fp64 sums).
"""
import numpy as np
import pytest
import torch

import gru_ops
import gru_oracle as GO
import rxmet_gru_abi as A
import rxmet_lib

pytestmark = pytest.mark.gpu
f32 = np.float32


def test_mfma_layout_selftest(cuda):
    g = np.random.default_rng(0)
    a = g.integers(-128, 128, (16, 64), dtype=np.int8)
    b = g.integers(-128, 128, (64, 16), dtype=np.int8)
    d = torch.zeros((16, 16), dtype=torch.int32, device=cuda)
    at, bt = torch.from_numpy(a).to(cuda), torch.from_numpy(b).to(cuda)
    rxmet_lib.call("rxmet_selftest_mfma", 0, at.data_ptr(), bt.data_ptr(), d.data_ptr(),
                   torch.cuda.current_stream().cuda_stream)
    np.testing.assert_array_equal(d.cpu().numpy(), a.astype(np.int64) @ b.astype(np.int64))
    a = g.integers(-100, 100, (16, 32)).astype(f32)
    b = (g.integers(-100, 100, (32, 16)) / 64.0).astype(f32)
    d = torch.zeros((16, 16), dtype=torch.float32, device=cuda)
    at, bt = torch.from_numpy(a).to(cuda), torch.from_numpy(b).to(cuda)
    rxmet_lib.call("rxmet_selftest_mfma", 1, at.data_ptr(), bt.data_ptr(), d.data_ptr(),
                   torch.cuda.current_stream().cuda_stream)
    np.testing.assert_array_equal(d.cpu().numpy(), (a.astype(np.float64) @ b).astype(f32))
    a = g.integers(-100, 100, (16, 4)).astype(f32)
    b = (g.integers(-100, 100, (4, 16)) / 64.0).astype(f32)
    d = torch.zeros((16, 16), dtype=torch.float32, device=cuda)
    at, bt = torch.from_numpy(a).to(cuda), torch.from_numpy(b).to(cuda)
    rxmet_lib.call("rxmet_selftest_mfma", 2, at.data_ptr(), bt.data_ptr(), d.data_ptr(),
                   torch.cuda.current_stream().cuda_stream)
    np.testing.assert_array_equal(d.cpu().numpy(), (a.astype(np.float64) @ b).astype(f32))


def _weights(I, H, seed, amp=None):
    g = np.random.default_rng(seed)
    k = amp if amp is not None else 1.0 / np.sqrt(H)
    W = ((g.random((I, 3 * H)) * 2 - 1) * k).astype(f32)
    R = ((g.random((H, 3 * H)) * 2 - 1) * k).astype(f32)
    bw = ((g.random(3 * H) * 2 - 1) * k).astype(f32)
    br = ((g.random(3 * H) * 2 - 1) * k).astype(f32)
    return W, R, bw, br


def _config(name):
    if name == "8b-sym":
        return A.default_config()
    if name == "8b-asym":
        return A.set_all_bitwidth(A.default_config(), 8, False)
    if name == "c3":  # 8-bit per-channel weights, 8-bit activations, 16-bit hidden state
        c = A.set_all_bitwidth(A.default_config(), 8, False)
        c.op[A.GRID["h"]].bits = 16
        return c
    if name == "16b-act-pot2":
        c = A.set_all_bitwidth(A.default_config(), 16, False)
        c.chan[0].bits = c.chan[1].bits = 8
        c.use_pot2 = 1
        return c
    if name == "h-unsigned":
        c = A.set_all_bitwidth(A.default_config(), 8, False)
        c.op[A.GRID["h"]].is_unsigned = 1
        c.op[A.GRID["h"]].bits = 12
        return c
    if name == "c5":  # 4-bit symmetric per-channel W and R, 16-bit activations and h, pot2 scales
        c = A.set_all_bitwidth(A.default_config(), 16, False)
        c.chan[0].bits = c.chan[1].bits = 4
        c.use_pot2 = 1
        return c
    if name == "16b-all":  # every grid 16-bit, recurrent weights included (stepped recurrence)
        return A.set_all_bitwidth(A.default_config(), 16, False)
    if name == "r12-pot2":  # 12-bit recurrent weights, 16-bit activations, power-of-two scales
        c = A.set_all_bitwidth(A.default_config(), 16, False)
        c.chan[0].bits = 8
        c.chan[1].bits = 12
        c.use_pot2 = 1
        return c
    if name == "16b-r8":  # 16-bit x and W: the input projection needs int64 accumulation
        c = A.set_all_bitwidth(A.default_config(), 16, False)
        c.chan[1].bits = 8
        return c
    raise KeyError(name)


def _case(T, B, I, H, cfg_name, seed, with_h0):
    W, R, bw, br = _weights(I, H, seed)
    g = np.random.default_rng(seed + 100)
    x = g.standard_normal((T, B, I)).astype(f32)
    h0 = (g.standard_normal((B, H)) * 0.4).astype(f32) if with_h0 else None
    _, _, stats = GO.forward_calibrate(W, R, bw, br, x, h0)
    qp, _ = GO.make_params(A.make_ranges(stats, H), _config(cfg_name))
    return W, R, bw, br, x, h0, qp


def _gpu_forward(dev, W, R, bw, br, x, h0, qp, training):
    T, B, I = x.shape
    H = R.shape[0]
    t = lambda a: None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    out = gru_ops.forward_quant_float_storage(
        training, T, B, I, H, t(W), t(R), t(bw), t(br), t(x),
        t(h0) if h0 is not None else torch.empty(0, device=dev), gru_ops.GRUQuantParams.from_struct(qp))
    torch.cuda.synchronize()
    return out


NAMES = ("h", "v", "W_q", "R_q", "bw_q", "br_q", "x_q") + GO.MASKS


@pytest.mark.parametrize("shape", [(5, 20, 7, 32), (4, 16, 80, 256), (3, 33, 40, 64),
                                   (2, 5, 3, 16), (6, 48, 9, 48)])
@pytest.mark.parametrize("cfg_name", ["8b-sym", "8b-asym", "c3", "16b-act-pot2", "h-unsigned",
                                      "16b-r8"])
@pytest.mark.parametrize("with_h0", [False, True])
def test_forward_bit_exact(cuda, shape, cfg_name, with_h0):
    T, B, I, H = shape
    print(f"[gru fwd] shape={shape} cfg={cfg_name} h0={with_h0}", flush=True)
    W, R, bw, br, x, h0, qp = _case(T, B, I, H, cfg_name, 1, with_h0)
    exp = GO.forward_quant(W, R, bw, br, x, qp, h0=h0, training=True)
    got = _gpu_forward(cuda, W, R, bw, br, x, h0, qp, True)
    for name, tensor in zip(NAMES, got):
        e = exp[name]
        if e is None:
            assert tensor.numel() == 0, name
            continue
        np.testing.assert_array_equal(tensor.cpu().numpy(), e, err_msg=name)


@pytest.mark.parametrize("shape,cfg_name", [((2, 4800, 8, 256), "c3"), ((3, 200, 16, 128), "c3"),
                                            ((3, 40, 8, 96), "16b-act-pot2")])
def test_clustered_forward_matches_oracle_and_single_tile_path(cuda, shape, cfg_name,
                                                               monkeypatch):
    """The clustered recurrence (units of a batch tile split over several workgroups, several
    batch tiles per cluster when B is large) equals the oracle and the one-workgroup-per-tile
    recurrence bit for bit."""
    T, B, I, H = shape
    print(f"[gru fwd cluster] shape={shape} cfg={cfg_name}", flush=True)
    W, R, bw, br, x, h0, qp = _case(T, B, I, H, cfg_name, 4, True)
    exp = GO.forward_quant(W, R, bw, br, x, qp, h0=h0, training=True)
    got = _gpu_forward(cuda, W, R, bw, br, x, h0, qp, True)
    for name, tensor in zip(NAMES, got):
        np.testing.assert_array_equal(tensor.cpu().numpy(), exp[name], err_msg=name)
    monkeypatch.setenv("RXMET_NO_CLUSTER", "1")
    ref = _gpu_forward(cuda, W, R, bw, br, x, h0, qp, True)
    for name, a, b in zip(NAMES, got, ref):
        assert torch.equal(a, b), name


@pytest.mark.parametrize("H", [512, 1024])
def test_forward_recurrent_sums_beyond_int32_are_exact(cuda, H):
    """A 16-bit unsigned h grid with 8-bit R: all-positive R columns (codes near 127) against
    h0 saturated at the top code make |R_q h| about 65535 * 120 * H, beyond 2^31.  The
    recurrent sums must still be the oracle's exact int64 sums rounded once to fp32."""
    T, B, I = 3, 16, 8
    print(f"[gru fwd wide sums] H={H}", flush=True)
    g = np.random.default_rng(31)
    W = ((g.random((I, 3 * H)) * 2 - 1) * 0.1).astype(f32)
    R = (0.05 + 0.01 * g.random((H, 3 * H))).astype(f32)
    bw = ((g.random(3 * H) * 2 - 1) * 0.1).astype(f32)
    br = ((g.random(3 * H) * 2 - 1) * 0.1).astype(f32)
    x = g.standard_normal((T, B, I)).astype(f32)
    h0 = np.full((B, H), 50.0, f32)
    _, _, stats = GO.forward_calibrate(W, R, bw, br, x, h0)
    c = A.set_all_bitwidth(A.default_config(), 8, False)
    c.op[A.GRID["h"]].bits = 16
    c.op[A.GRID["h"]].is_unsigned = 1
    qp, _ = GO.make_params(A.make_ranges(stats, H), c)
    exp = GO.forward_quant(W, R, bw, br, x, qp, h0=h0, training=True)
    hq = exp["h"][0] / GO.effective_scale(float(qp.g[A.GRID["h"]].scale), False) \
        + qp.g[A.GRID["h"]].zero_point
    rmax = np.abs(exp["R_q"]).sum(axis=0).max()
    assert float(np.abs(hq).max()) * rmax >= 2 ** 31, "case does not exceed int32"
    got = _gpu_forward(cuda, W, R, bw, br, x, h0, qp, True)
    for name, tensor in zip(NAMES, got):
        np.testing.assert_array_equal(tensor.cpu().numpy(), exp[name], err_msg=name)


def test_forward_eval_matches_training_h(cuda):
    W, R, bw, br, x, h0, qp = _case(4, 16, 8, 32, "c3", 2, True)
    tr = _gpu_forward(cuda, W, R, bw, br, x, h0, qp, True)
    ev = _gpu_forward(cuda, W, R, bw, br, x, h0, qp, False)
    assert torch.equal(tr[0], ev[0])
    assert all(m.numel() == 0 for m in ev[7:])


@pytest.mark.parametrize("H", [1, 2, 5, 20, 33])
@pytest.mark.parametrize("cfg_name", ["c3", "16b-act-pot2"])
def test_any_hidden_size_forward_backward_match_oracle(cuda, H, cfg_name):
    """Hidden sizes that are not a multiple of 16 (the reference's own fixtures use 1 and 2)
    run with inert padded units inside the boundary: every forward output bit-exact, every
    gradient within 1e-4 of the oracle at the real size."""
    T, B, I = 4, 6, 3
    print(f"[gru any H] H={H} cfg={cfg_name}", flush=True)
    W, R, bw, br, x, h0, qp = _case(T, B, I, H, cfg_name, 17, True)
    exp_f = GO.forward_quant(W, R, bw, br, x, qp, h0=h0, training=True)
    fwd = _gpu_forward(cuda, W, R, bw, br, x, h0, qp, True)
    for name, tensor in zip(NAMES, fwd):
        np.testing.assert_array_equal(tensor.cpu().numpy(), exp_f[name], err_msg=name)
    g = np.random.default_rng(18)
    dh_new = (g.standard_normal((T + 1, B, H)) * 1e-2).astype(f32)
    exp = GO.backward_quant(exp_f, dh_new, qp)
    got = _gpu_backward(cuda, fwd, dh_new, qp, T, B, I, H)
    for name, a in zip(("dx", "dW", "dR", "dbw", "dbr", "dh0"), got):
        e = exp[name]
        scale = max(float(np.abs(e).max()), 1e-30)
        np.testing.assert_allclose(a, e, rtol=1e-4, atol=1e-5 * scale, err_msg=name)


def test_two_direction_entry_points_refuse_unaligned_hidden_size(cuda):
    W, R, bw, br, x, h0, qp = _case(2, 4, 3, 20, "8b-sym", 3, False)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(cuda)
    d = (t(W), t(R), t(bw), t(br), t(x), torch.empty(0, device=cuda),
         gru_ops.GRUQuantParams.from_struct(qp))
    with pytest.raises(RuntimeError, match="hidden_size % 16"):
        gru_ops.forward_quant_float_storage_dirs(True, 2, 4, 3, 20, [d, d])


def _gpu_backward(dev, fwd, dh_new, qp, T, B, I, H):
    (h, v, W_q, R_q, bw_q, br_q, x_q, *masks) = fwd
    dh = torch.from_numpy(np.ascontiguousarray(dh_new)).to(dev)
    out = gru_ops.backward_quant_float_storage(T, B, I, H, W_q, R_q, bw_q, br_q, x_q, dh, h, v,
                                               gru_ops.GRUQuantParams.from_struct(qp), *masks)
    torch.cuda.synchronize()
    return [t.cpu().numpy() for t in out]


@pytest.mark.parametrize("shape", [(5, 20, 7, 32), (4, 16, 80, 256), (3, 33, 40, 64),
                                   (6, 48, 9, 48), (12, 64, 16, 128)])
@pytest.mark.parametrize("cfg_name", ["8b-sym", "8b-asym", "c3", "16b-act-pot2"])
@pytest.mark.parametrize("with_h0", [False, True])
def test_backward_matches_oracle(cuda, shape, cfg_name, with_h0):
    T, B, I, H = shape
    print(f"[gru bwd] shape={shape} cfg={cfg_name} h0={with_h0}", flush=True)
    W, R, bw, br, x, h0, qp = _case(T, B, I, H, cfg_name, 4, with_h0)
    exp_f = GO.forward_quant(W, R, bw, br, x, qp, h0=h0, training=True)
    fwd = _gpu_forward(cuda, W, R, bw, br, x, h0, qp, True)
    g = np.random.default_rng(5)
    dh_new = np.zeros((T + 1, B, H), f32)
    dh_new[1:] = (g.standard_normal((T, B, H)) * 1e-3).astype(f32)
    dh_new[-1] += (g.standard_normal((B, H)) * 1e-3).astype(f32)
    exp = GO.backward_quant(exp_f, dh_new, qp)
    got = _gpu_backward(cuda, fwd, dh_new, qp, T, B, I, H)
    for name, a in zip(("dx", "dW", "dR", "dbw", "dbr", "dh0"), got):
        e = exp[name]
        scale = max(float(np.abs(e).max()), 1e-30)
        np.testing.assert_allclose(a, e, rtol=1e-4, atol=1e-5 * scale, err_msg=name)


@pytest.mark.parametrize("shape,cfg_name", [((2, 4800, 8, 256), "c3"), ((3, 200, 16, 128), "c3"),
                                            ((4, 40, 8, 96), "16b-act-pot2"), ((3, 20, 5, 16), "8b-sym")])
def test_clustered_backward_matches_oracle_and_single_tile_path(cuda, shape, cfg_name,
                                                                monkeypatch):
    """The clustered backward (split-bf16 MFMA dh, dq exchanged between the workgroups of a batch
    tile) against the oracle, and against the one-workgroup-per-tile path within 1e-4."""
    T, B, I, H = shape
    print(f"[gru bwd cluster] shape={shape} cfg={cfg_name}", flush=True)
    W, R, bw, br, x, h0, qp = _case(T, B, I, H, cfg_name, 5, True)
    exp_f = GO.forward_quant(W, R, bw, br, x, qp, h0=h0, training=True)
    fwd = _gpu_forward(cuda, W, R, bw, br, x, h0, qp, True)
    g = np.random.default_rng(6)
    dh_new = (g.standard_normal((T + 1, B, H)) * 1e-2).astype(f32)
    exp = GO.backward_quant(exp_f, dh_new, qp)
    got = _gpu_backward(cuda, fwd, dh_new, qp, T, B, I, H)
    names = ("dx", "dW", "dR", "dbw", "dbr", "dh0")
    for name, a in zip(names, got):
        e = exp[name]
        scale = max(float(np.abs(e).max()), 1e-30)
        np.testing.assert_allclose(a, e, rtol=1e-4, atol=1e-5 * scale, err_msg=name)
    monkeypatch.setenv("RXMET_NO_CLUSTER", "1")
    ref = _gpu_backward(cuda, fwd, dh_new, qp, T, B, I, H)
    for name, a, b in zip(names, got, ref):
        scale = max(float(np.abs(b).max()), 1e-30)
        np.testing.assert_allclose(a, b, rtol=1e-4, atol=1e-5 * scale, err_msg=name)


def test_backward_without_masks_and_nan_propagation(cuda):
    T, B, I, H = 3, 16, 5, 32
    W, R, bw, br, x, h0, qp = _case(T, B, I, H, "8b-asym", 6, False)
    fwd = _gpu_forward(cuda, W, R, bw, br, x, None, qp, True)
    dh_new = np.zeros((T + 1, B, H), f32)
    dh_new[1:] = 1e-3
    dh_new[2, 3, 7] = np.nan
    got = _gpu_backward(cuda, fwd, dh_new, qp, T, B, I, H)
    assert np.isnan(got[5][3]).any(), "NaN upstream gradient must reach dh0 of its sequence"
    assert np.isfinite(np.delete(got[5], 3, axis=0)).all(), "NaN leaked into other sequences"


@pytest.mark.parametrize("shape", [(4, 48, 9, 64), (3, 300, 16, 256)])
def test_two_direction_entry_points_equal_single_calls(cuda, shape):
    """rxmet_gru_forward_quant_dirs / backward_quant_dirs (both directions, one clustered
    launch each way) equal one call per direction: forward bit for bit, backward within the
    GEMM summation-order tolerance."""
    T, B, I, H = shape
    args = []
    for d in range(2):
        W, R, bw, br, x, h0, qp = _case(T, B, I, H, "c3", 7 + d, True)
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(cuda)
        args.append((t(W), t(R), t(bw), t(br), t(x), t(h0), gru_ops.GRUQuantParams.from_struct(qp)))
    both = gru_ops.forward_quant_float_storage_dirs(True, T, B, I, H, args)
    torch.cuda.synchronize()
    single = [gru_ops.forward_quant_float_storage(True, T, B, I, H, *a) for a in args]
    torch.cuda.synchronize()
    for d in range(2):
        for name, a, b in zip(NAMES, both[d], single[d]):
            assert torch.equal(a, b), (d, name)
    g = np.random.default_rng(9)
    bargs = []
    for d in range(2):
        (h, v, W_q, R_q, bw_q, br_q, x_q, *masks) = both[d]
        dh = torch.from_numpy((g.standard_normal((T + 1, B, H)) * 1e-2).astype(f32)).to(cuda)
        bargs.append((W_q, R_q, bw_q, br_q, x_q, dh, h, v, args[d][6], masks))
    gb = gru_ops.backward_quant_float_storage_dirs(T, B, I, H, bargs)
    torch.cuda.synchronize()
    for d in range(2):
        W_q, R_q, bw_q, br_q, x_q, dh, h, v, qp, masks = bargs[d]
        gs = gru_ops.backward_quant_float_storage(T, B, I, H, W_q, R_q, bw_q, br_q, x_q, dh, h, v,
                                                  qp, *masks)
        torch.cuda.synchronize()
        for name, a, b in zip(("dx", "dW", "dR", "dbw", "dbr", "dh0"), gb[d], gs):
            a, b = a.cpu().numpy(), b.cpu().numpy()
            scale = max(float(np.abs(b).max()), 1e-30)
            np.testing.assert_allclose(a, b, rtol=1e-5, atol=1e-6 * scale, err_msg=f"{d} {name}")


@pytest.mark.parametrize("shape", [(3, 20, 24, 1024), (4, 35, 16, 512), (2, 18, 8, 272),
                                   (2, 18, 8, 544)])
def test_large_hidden_forward_backward_match_oracle(cuda, shape):
    """H above 256 (the c5 hidden size 1024 with its quantisation): the clustered forward
    (K split over four waves, several batch tiles per cluster) bit for bit, and the stepped
    backward (pointwise + dh GEMM per step) within 1e-4 of the oracle."""
    T, B, I, H = shape
    print(f"[gru large H] shape={shape}", flush=True)
    W, R, bw, br, x, h0, qp = _case(T, B, I, H, "c5", 11, True)
    exp_f = GO.forward_quant(W, R, bw, br, x, qp, h0=h0, training=True)
    fwd = _gpu_forward(cuda, W, R, bw, br, x, h0, qp, True)
    for name, tensor in zip(NAMES, fwd):
        np.testing.assert_array_equal(tensor.cpu().numpy(), exp_f[name], err_msg=name)
    g = np.random.default_rng(12)
    dh_new = (g.standard_normal((T + 1, B, H)) * 1e-2).astype(f32)
    exp = GO.backward_quant(exp_f, dh_new, qp)
    got = _gpu_backward(cuda, fwd, dh_new, qp, T, B, I, H)
    for name, a in zip(("dx", "dW", "dR", "dbw", "dbr", "dh0"), got):
        e = exp[name]
        scale = max(float(np.abs(e).max()), 1e-30)
        np.testing.assert_allclose(a, e, rtol=1e-4, atol=1e-5 * scale, err_msg=name)


@pytest.mark.parametrize("shape,cfg_name", [((3, 40, 8, 96), "c3"), ((4, 33, 5, 48), "16b-act-pot2")])
def test_stepped_backward_matches_clustered(cuda, shape, cfg_name, monkeypatch):
    """The stepped backward (forced with RXMET_BWD_STEPPED) against the oracle and the
    clustered backward within 1e-4, masks and h0 included."""
    T, B, I, H = shape
    print(f"[gru bwd stepped] shape={shape} cfg={cfg_name}", flush=True)
    W, R, bw, br, x, h0, qp = _case(T, B, I, H, cfg_name, 13, True)
    exp_f = GO.forward_quant(W, R, bw, br, x, qp, h0=h0, training=True)
    fwd = _gpu_forward(cuda, W, R, bw, br, x, h0, qp, True)
    g = np.random.default_rng(14)
    dh_new = (g.standard_normal((T + 1, B, H)) * 1e-2).astype(f32)
    exp = GO.backward_quant(exp_f, dh_new, qp)
    clustered = _gpu_backward(cuda, fwd, dh_new, qp, T, B, I, H)
    monkeypatch.setenv("RXMET_BWD_STEPPED", "1")
    got = _gpu_backward(cuda, fwd, dh_new, qp, T, B, I, H)
    for name, a, c in zip(("dx", "dW", "dR", "dbw", "dbr", "dh0"), got, clustered):
        e = exp[name]
        scale = max(float(np.abs(e).max()), 1e-30)
        np.testing.assert_allclose(a, e, rtol=1e-4, atol=1e-5 * scale, err_msg=name)
        np.testing.assert_allclose(a, c, rtol=1e-4, atol=1e-5 * scale, err_msg=name)


def test_c5_full_size_rows_match_oracle(cuda):
    """c5 at its full size (T=50, B=1024, I=256, H=1024, 4-bit W and R, 16-bit activations and
    h, pot2): sequences are independent, so the GPU's rows of a sample of sequences equal the
    oracle run on those sequences alone — forward outputs and masks bit for bit.  The output
    gradient is set on the sampled sequences only (zero elsewhere), so every weight and bias
    gradient is a sum over those sequences: dx, dh0, dW, dR, dbw and dbr within 1e-4."""
    T, B, I, H = 50, 1024, 256, 1024
    rows = [0, 1, 517, 1023]
    print(f"[gru c5 full] T={T} B={B} I={I} H={H} rows={rows}", flush=True)
    W, R, bw, br = _weights(I, H, 21)
    g = np.random.default_rng(22)
    x = g.standard_normal((T, B, I)).astype(f32)
    h0 = (g.standard_normal((B, H)) * 0.4).astype(f32)
    _, _, stats = GO.forward_calibrate(W, R, bw, br, x[:, rows], h0[rows])
    qp, _ = GO.make_params(A.make_ranges(stats, H), _config("c5"))
    fwd = _gpu_forward(cuda, W, R, bw, br, x, h0, qp, True)
    exp_f = GO.forward_quant(W, R, bw, br, np.ascontiguousarray(x[:, rows]), qp,
                             h0=np.ascontiguousarray(h0[rows]), training=True)
    per_seq = {"h": 1, "v": 1, "x_q": 1, "x_mask": 1, "h0_mask": 0}
    for name, tensor in zip(NAMES, fwd):
        e = exp_f[name]
        if e is None:
            continue
        axis = per_seq.get(name, 1 if tensor.dim() >= 3 else None)
        if name in ("W_q", "R_q", "bw_q", "br_q", "W_mask", "R_mask", "bw_mask", "br_mask"):
            np.testing.assert_array_equal(tensor.cpu().numpy(), e, err_msg=name)
            continue
        idx = torch.tensor(rows, device=tensor.device)
        np.testing.assert_array_equal(tensor.index_select(axis, idx).cpu().numpy(), e, err_msg=name)
    dh_new = np.zeros((T + 1, B, H), f32)
    dh_new[1:, rows] = (g.standard_normal((T, len(rows), H)) * 1e-2).astype(f32)
    got = _gpu_backward(cuda, fwd, dh_new, qp, T, B, I, H)
    exp = GO.backward_quant(exp_f, np.ascontiguousarray(dh_new[:, rows]), qp)
    for name, a, axis in (("dx", got[0], 1), ("dW", got[1], None), ("dR", got[2], None),
                          ("dbw", got[3], None), ("dbr", got[4], None), ("dh0", got[5], 0)):
        e = exp[name]
        scale = max(float(np.abs(e).max()), 1e-30)
        assert np.isfinite(a).all(), name
        np.testing.assert_allclose(a if axis is None else a.take(rows, axis=axis), e, rtol=1e-4,
                                   atol=1e-5 * scale, err_msg=name)


@pytest.mark.parametrize("shape", [(4, 20, 7, 32), (3, 33, 40, 64), (2, 5, 3, 256), (3, 40, 8, 512),
                                   (3, 6, 2, 1), (3, 6, 2, 33)])
@pytest.mark.parametrize("cfg_name", ["16b-all", "r12-pot2"])
def test_wide_recurrent_weights_forward_backward_match_oracle(cuda, shape, cfg_name):
    """Recurrent weights of 16 bits (the reference's set_all_bitwidth(16)): the stepped
    recurrence (an exact two-plane GEMM and a pointwise launch per step) bit-exact in every
    forward output, and the backward within 1e-4 of the oracle."""
    T, B, I, H = shape
    print(f"[gru wide R] shape={shape} cfg={cfg_name}", flush=True)
    W, R, bw, br, x, h0, qp = _case(T, B, I, H, cfg_name, 23, True)
    exp_f = GO.forward_quant(W, R, bw, br, x, qp, h0=h0, training=True)
    fwd = _gpu_forward(cuda, W, R, bw, br, x, h0, qp, True)
    for name, tensor in zip(NAMES, fwd):
        np.testing.assert_array_equal(tensor.cpu().numpy(), exp_f[name], err_msg=name)
    g = np.random.default_rng(24)
    dh_new = (g.standard_normal((T + 1, B, H)) * 1e-2).astype(f32)
    exp = GO.backward_quant(exp_f, dh_new, qp)
    got = _gpu_backward(cuda, fwd, dh_new, qp, T, B, I, H)
    for name, a in zip(("dx", "dW", "dR", "dbw", "dbr", "dh0"), got):
        e = exp[name]
        scale = max(float(np.abs(e).max()), 1e-30)
        np.testing.assert_allclose(a, e, rtol=1e-4, atol=1e-5 * scale, err_msg=name)


@pytest.mark.parametrize("shape,cfg_name", [((4, 40, 9, 64), "c3"), ((3, 20, 5, 256), "8b-asym")])
def test_stepped_forward_equals_clustered(cuda, shape, cfg_name, monkeypatch):
    """The stepped recurrence forced on 8-bit recurrent weights equals the clustered one bit
    for bit."""
    T, B, I, H = shape
    print(f"[gru fwd stepped] shape={shape} cfg={cfg_name}", flush=True)
    W, R, bw, br, x, h0, qp = _case(T, B, I, H, cfg_name, 25, True)
    ref = _gpu_forward(cuda, W, R, bw, br, x, h0, qp, True)
    monkeypatch.setenv("RXMET_FWD_STEPPED", "1")
    got = _gpu_forward(cuda, W, R, bw, br, x, h0, qp, True)
    for name, a, b in zip(NAMES, got, ref):
        assert torch.equal(a, b), name


@pytest.mark.parametrize("cfg_name", ["c3", "16b-all"])
@pytest.mark.parametrize("H", [48, 33])
def test_workspace_contents_never_leak_into_results(cuda, monkeypatch, cfg_name, H):
    """Forward and backward (FP32 and int32 carriers) read no workspace byte they did not write:
    with every workspace filled with NaN bytes first the results equal those of zero-filled
    workspaces.  3H = 144 / 99 is not a multiple of 32, where the GEMMs' last K chunk and the
    packed operand tiles run past the data."""
    T, B, I = 4, 10, 6
    print(f"[gru workspace] H={H} cfg={cfg_name}", flush=True)
    W, R, bw, br, x, h0, qp = _case(T, B, I, H, cfg_name, 9, True)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(cuda)
    g = np.random.default_rng(10)
    dh_new = g.standard_normal((T + 1, B, H)).astype(f32)

    def run(fill):
        monkeypatch.setattr(gru_ops, "_ws", lambda n, dev: torch.full(
            (max(int(n), 256),), fill, dtype=torch.uint8, device=dev))
        P = gru_ops.GRUQuantParams.from_struct(qp)
        res = []
        for fwd_fn, bwd_fn in ((gru_ops.forward_quant_float_storage,
                                gru_ops.backward_quant_float_storage),
                               (gru_ops.forward_quant_int_storage,
                                gru_ops.backward_quant_int_storage)):
            outs = fwd_fn(True, T, B, I, H, t(W), t(R), t(bw), t(br), t(x), t(h0), P)
            grads = bwd_fn(T, B, I, H, outs[2], outs[3], outs[4], outs[5], outs[6], t(dh_new),
                           outs[0], outs[1], P, *outs[7:])
            res += [o.cpu().numpy() for o in (*outs, *grads) if o.numel()]
        torch.cuda.synchronize()
        return res

    clean, dirty = run(0), run(255)
    for k, (a, b) in enumerate(zip(clean, dirty)):
        assert np.isfinite(b).all() if b.dtype.kind == "f" else True, k
        np.testing.assert_array_equal(a, b, err_msg=f"output {k}")
