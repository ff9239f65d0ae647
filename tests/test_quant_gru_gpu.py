"""GPU parity of the GRU calibration pass and of the QuantGRU module (calibrate -> QAT
forward -> backward, both directions) against the pinned oracle.

Bars: calibration h/v and ranges within 2e-6 absolute + 1e-5 relative of the oracle (the
oracle sums in the same order; device tanhf/exp may differ from glibc in the last ulp);
module forward outputs bit-exact against the oracle given the module's own grids; module
gradients within 1e-4 relative.
"""
import numpy as np
import pytest
import torch

import gru_ops
import gru_oracle as GO
import quant_gru as Q
import rxmet_gru_abi as A

pytestmark = pytest.mark.gpu
f32 = np.float32


def _haste(w_ih, w_hh, b_ih, b_hh):
    def swap(t):
        r, z, n = np.split(t, 3, axis=0)
        return np.concatenate([z, r, n], 0)
    return (np.ascontiguousarray(swap(w_ih).T), np.ascontiguousarray(swap(w_hh).T), swap(b_ih),
            swap(b_hh))


def _weights(I, H, seed, amp=None):
    g = np.random.default_rng(seed)
    k = amp if amp is not None else 1.0 / np.sqrt(H)
    return tuple(((g.random(s) * 2 - 1) * k).astype(f32)
                 for s in ((3 * H, I), (3 * H, H), (3 * H,), (3 * H,)))


def _gpu_calibrate(dev, W, R, bw, br, x, h0, ranges=None):
    T, B, I = x.shape
    H = R.shape[0]
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    ranges = ranges or gru_ops.GRUQuantizationRanges(H, device=dev)
    h, v = gru_ops.forward_calibrate(True, T, B, I, H, t(W), t(R), t(bw), t(br), t(x),
                                     t(h0) if h0 is not None else torch.empty(0, device=dev),
                                     quant_ranges=ranges)
    torch.cuda.synchronize()
    return h.cpu().numpy(), v.cpu().numpy(), ranges


def _close(a, e, name, atol=2e-6, rtol=1e-5):
    np.testing.assert_allclose(a, e, rtol=rtol, atol=atol, err_msg=name)


# H = 336 .. 1024 take the 8-wave recurrence (3 .. 6 items per wave); B = 300 at H = 528 and
# B = 200 at H = 1024 give clusters several batch tiles (the multi-tile recurrence)
@pytest.mark.parametrize("shape", [(5, 20, 7, 32), (4, 16, 80, 256), (3, 9, 40, 48),
                                   (2, 3, 1, 5), (3, 4, 6, 300), (3, 40, 16, 336),
                                   (2, 300, 8, 528), (2, 48, 8, 704), (2, 200, 8, 1024)])
@pytest.mark.parametrize("with_h0", [False, True])
def test_calibration_matches_oracle(cuda, shape, with_h0):
    T, B, I, H = shape
    print(f"[gru calib] shape={shape} h0={with_h0}", flush=True)
    W, R, bw, br = _haste(*_weights(I, H, 11))
    g = np.random.default_rng(12)
    x = g.standard_normal((T, B, I)).astype(f32)
    h0 = (g.standard_normal((B, H)) * 0.5).astype(f32) if with_h0 else None
    he, ve, se = GO.forward_calibrate(W, R, bw, br, x, h0)
    h, v, ranges = _gpu_calibrate(cuda, W, R, bw, br, x, h0)
    _close(h, he, "h")
    _close(v, ve, "v")
    _close(ranges.stats.cpu().numpy(), se, "stats")


def test_calibration_merges_batches_and_ignores_non_finite(cuda):
    T, B, I, H = 4, 6, 5, 32
    W, R, bw, br = _haste(*_weights(I, H, 13))
    g = np.random.default_rng(14)
    x1 = g.standard_normal((T, B, I)).astype(f32)
    x2 = (g.standard_normal((T, B, I)) * 3).astype(f32)
    x2[1, 2, 3] = np.inf  # poisons one sequence; its non-finite values must be skipped
    _, _, s = GO.forward_calibrate(W, R, bw, br, x1)
    _, _, s = GO.forward_calibrate(W, R, bw, br, x2, stats=s)
    _, _, ranges = _gpu_calibrate(cuda, W, R, bw, br, x1, None)
    _, _, ranges = _gpu_calibrate(cuda, W, R, bw, br, x2, None, ranges)
    got = ranges.stats.cpu().numpy()
    assert np.isfinite(got).all()
    _close(got, s, "merged stats")


@pytest.mark.parametrize("shape", [(2, 8, 40, 64), (2, 4, 300, 128)])
def test_parameter_ranges_skip_non_finite_weights(cuda, shape):
    """Per-channel ranges of W, R, bw, br (the stats after the 2 x 13 activation grids): W and R
    taken in 64-row slabs (I + H = 104 and 428 rows), non-finite entries skipped, a channel with
    no finite entry contributing 0; merged into ranges from an earlier batch."""
    T, B, I, H = shape
    W, R, bw, br = _haste(*_weights(I, H, 15))
    W[3, 5], W[I - 1, 7], R[H - 1, 2] = np.nan, np.inf, -np.inf
    R[:, 9] = np.inf          # one recurrent channel with no finite value
    bw[4], br[11] = np.nan, -np.inf
    x = np.random.default_rng(16).standard_normal((T, B, I)).astype(f32)
    W1, R1, bw1, br1 = _haste(*_weights(I, H, 17, amp=3.0))
    _, _, s = GO.forward_calibrate(W1, R1, bw1, br1, x)
    _, _, s = GO.forward_calibrate(W, R, bw, br, x, stats=s)
    _, _, ranges = _gpu_calibrate(cuda, W1, R1, bw1, br1, x, None)
    _, _, ranges = _gpu_calibrate(cuda, W, R, bw, br, x, None, ranges)
    n = 2 * A.NGRIDS
    got = ranges.stats.cpu().numpy()[n:]
    assert np.isfinite(got).all()
    np.testing.assert_array_equal(got, s[n:])


def _module_case(bidirectional, batch_first, with_hx, cfg, seed, shape=(6, 24, 10, 32)):
    T, B, I, H = shape
    torch.manual_seed(seed)
    m = Q.QuantGRU(I, H, batch_first=batch_first, bidirectional=bidirectional)
    if cfg == "c3":
        m.set_all_bitwidth(8, is_symmetric=False)
        m._bitwidth_config.h_ = 16
        m._bitwidth_config.W_granularity_ = A.PER_CHANNEL
        m._bitwidth_config.R_granularity_ = A.PER_CHANNEL
        m._bitwidth_config.bw_granularity_ = A.PER_CHANNEL
        m._bitwidth_config.br_granularity_ = A.PER_CHANNEL
    elif cfg == "po2-16b":
        m.set_all_bitwidth(16, is_symmetric=False)
        m._bitwidth_config.W_ = m._bitwidth_config.R_ = 8
        m.use_po2_scale = True
    D = 2 if bidirectional else 1
    g = torch.Generator().manual_seed(seed + 1)
    x = torch.randn(T, B, I, generator=g)
    hx = torch.randn(D, B, H, generator=g) * 0.3 if with_hx else None
    return m, x, hx


def _oracle_direction(m, reverse, x_tbi, h0, qp_struct, gout_tbh, ghn_bh):
    sfx = "_reverse" if reverse else ""
    p = lambda n: getattr(m, n + sfx).detach().cpu().numpy()
    W, R, bw, br = _haste(p("weight_ih_l0"), p("weight_hh_l0"), p("bias_ih_l0"), p("bias_hh_l0"))
    xs = x_tbi[::-1].copy() if reverse else x_tbi
    fwd = GO.forward_quant(W, R, bw, br, xs, qp_struct, h0=h0, training=True)
    T, B, H = gout_tbh.shape
    dh_new = np.zeros((T + 1, B, H), f32)
    dh_new[1:] = gout_tbh[::-1] if reverse else gout_tbh
    dh_new[-1] += ghn_bh
    bwd = GO.backward_quant(fwd, dh_new, qp_struct)
    out = fwd["h"][1:]
    return (out[::-1] if reverse else out), fwd["h"][-1], bwd, (W, R, bw, br, xs, h0)


@pytest.mark.parametrize("bidirectional", [False, True])
@pytest.mark.parametrize("batch_first", [False, True])
@pytest.mark.parametrize("with_hx", [False, True])
@pytest.mark.parametrize("cfg", ["c3", "po2-16b"])
@pytest.mark.parametrize("shape", [(6, 24, 10, 32), (5, 12, 6, 33)])
def test_module_calibrate_qat_matches_oracle(cuda, bidirectional, batch_first, with_hx, cfg,
                                             shape):
    print(f"[quantgru module] bi={bidirectional} bf={batch_first} hx={with_hx} cfg={cfg} "
          f"shape={shape}", flush=True)
    m, x_tbi, hx = _module_case(bidirectional, batch_first, with_hx, cfg, 21, shape=shape)
    m = m.to(cuda)
    T, B, I = x_tbi.shape
    H = m.hidden_size
    D = 2 if bidirectional else 1
    x_in = (x_tbi.transpose(0, 1).contiguous() if batch_first else x_tbi).to(cuda)
    hx_d = hx.to(cuda) if hx is not None else None
    # calibration pass: ranges of each direction vs the oracle's
    with m.calibration_context():
        m(x_in, hx_d)
    assert m.is_calibrated() and not m.calibrating
    xn = x_tbi.numpy()
    for d in range(D):
        sfx = "_reverse" if d else ""
        pn = lambda n: getattr(m, n + sfx).detach().cpu().numpy()
        W, R, bw, br = _haste(pn("weight_ih_l0"), pn("weight_hh_l0"), pn("bias_ih_l0"),
                              pn("bias_hh_l0"))
        h0 = hx[d].numpy() if hx is not None else None
        _, _, se = GO.forward_calibrate(W, R, bw, br, xn[::-1].copy() if d else xn, h0)
        ranges = m.quant_ranges_reverse if d else m.quant_ranges
        _close(ranges.stats.cpu().numpy(), se, f"stats dir{d}")
    # QAT step
    m.use_quantization = True
    m.train()
    x_leaf = x_in.clone().requires_grad_(True)
    hx_leaf = hx_d.clone().requires_grad_(True) if hx_d is not None else None
    out, hn = m(x_leaf, hx_leaf)
    g = torch.Generator().manual_seed(5)
    gout = torch.randn(out.shape, generator=g) * 1e-2
    ghn = torch.randn(hn.shape, generator=g) * 1e-2
    ((out * gout.to(cuda)).sum() + (hn * ghn.to(cuda)).sum()).backward()
    torch.cuda.synchronize()
    gout_tb = (gout.transpose(0, 1) if batch_first else gout).numpy()
    out_tb = (out.transpose(0, 1) if batch_first else out).detach().cpu().numpy()
    dx_tot = np.zeros((T, B, I), np.float64)
    for d in range(D):
        qp = (m.quant_params_reverse if d else m.quant_params).struct
        h0 = hx[d].numpy() if hx is not None else None
        o, hlast, bwd, _ = _oracle_direction(m, bool(d), xn, h0, qp,
                                             np.ascontiguousarray(gout_tb[..., d * H:(d + 1) * H]),
                                             ghn[d].numpy())
        np.testing.assert_array_equal(out_tb[..., d * H:(d + 1) * H], o, err_msg=f"out dir{d}")
        np.testing.assert_array_equal(hn[d].detach().cpu().numpy(), hlast, err_msg=f"h_n dir{d}")
        sfx = "_reverse" if d else ""

        def check(name, got, exp):
            scale = max(float(np.abs(exp).max()), 1e-30)
            np.testing.assert_allclose(got, exp, rtol=1e-4, atol=1e-5 * scale,
                                       err_msg=f"{name} dir{d}")

        swap = lambda a: np.concatenate([a[H:2 * H], a[:H], a[2 * H:]], 0)
        check("dW_ih", getattr(m, "weight_ih_l0" + sfx).grad.cpu().numpy(), swap(bwd["dW"].T))
        check("dW_hh", getattr(m, "weight_hh_l0" + sfx).grad.cpu().numpy(), swap(bwd["dR"].T))
        check("db_ih", getattr(m, "bias_ih_l0" + sfx).grad.cpu().numpy(), swap(bwd["dbw"]))
        check("db_hh", getattr(m, "bias_hh_l0" + sfx).grad.cpu().numpy(), swap(bwd["dbr"]))
        if hx is not None:
            check("dhx", hx_leaf.grad[d].cpu().numpy(), bwd["dh0"])
        dx_tot += bwd["dx"][::-1] if d else bwd["dx"]
    dx = x_leaf.grad
    dx = (dx.transpose(0, 1) if batch_first else dx).cpu().numpy()
    scale = float(np.abs(dx_tot).max())
    np.testing.assert_allclose(dx, dx_tot, rtol=1e-4, atol=1e-5 * scale, err_msg="dx")


def test_module_tracks_nn_gru_at_16_bits(cuda):
    T, B, I, H = 8, 16, 12, 64
    torch.manual_seed(3)
    ref = torch.nn.GRU(I, H, bidirectional=True, batch_first=True)
    m = Q.QuantGRU(I, H, bidirectional=True, batch_first=True)
    m.load_state_dict(ref.state_dict())
    m.set_all_bitwidth(16, is_symmetric=False)
    m = m.to(cuda)
    x = torch.randn(B, T, I)
    with m.calibration_context():
        yc, hc = m(x.to(cuda))
    with torch.no_grad():
        y, hn = ref(x)
    # calibration runs the float GRU: close to torch's within fp32 summation noise
    np.testing.assert_allclose(yc.cpu().numpy(), y.numpy(), atol=1e-5)
    np.testing.assert_allclose(hc.cpu().numpy(), hn.numpy(), atol=1e-5)
    m.use_quantization = True
    m.eval()
    with torch.no_grad():
        yq, _ = m(x.to(cuda))
    err = np.abs(yq.cpu().numpy() - y.numpy())
    # 16-segment PWL sigmoid/tanh approximations bound the deviation (a few 1e-3)
    assert err.max() < 3e-2 and err.mean() < 5e-3, (err.max(), err.mean())


def test_module_no_grad_eval_saves_nothing_and_matches_training(cuda):
    m, x, hx = _module_case(True, False, True, "c3", 31)
    m = m.to(cuda)
    x, hx = x.to(cuda), hx.to(cuda)
    with m.calibration_context():
        m(x, hx)
    m.use_quantization = True
    m.train()
    y_tr, h_tr = m(x, hx)
    m.eval()
    with torch.no_grad():
        y_ev, h_ev = m(x, hx)
    assert torch.equal(y_tr.detach(), y_ev) and torch.equal(h_tr.detach(), h_ev)


@pytest.mark.parametrize("shape", [(6, 24, 10, 32), (5, 12, 6, 48), (4, 9, 7, 33)])
@pytest.mark.parametrize("with_hx", [False, True])
def test_batch_first_eval_reads_x_in_place_and_matches_training(cuda, shape, with_hx):
    """Unidirectional batch-first inference reads the [B, T, I] input through its strides and
    PyTorch-layout weights (H % 16 == 0; H = 33 takes the reordering path): the output equals
    the training forward's on the same grids bit for bit."""
    print(f"[quantgru bf eval] shape={shape} hx={with_hx}", flush=True)
    m, x_tbi, hx = _module_case(False, True, with_hx, "c3", 41, shape=shape)
    m = m.to(cuda)
    x = x_tbi.transpose(0, 1).contiguous().to(cuda)
    hx = hx.to(cuda) if with_hx else None
    with m.calibration_context():
        m(x, hx)
    m.use_quantization = True
    m.train()
    y_tr, h_tr = m(x, hx)
    m.eval()
    with torch.no_grad():
        y_ev, h_ev = m(x, hx)
    assert y_ev.is_contiguous() and y_ev.shape == y_tr.shape
    assert torch.equal(y_tr.detach(), y_ev) and torch.equal(h_tr.detach(), h_ev)


def test_lock_keeps_grids_across_recalibration(cuda):
    m, x, _ = _module_case(False, False, False, "c3", 41)
    m = m.to(cuda)
    x = x.to(cuda)
    with m.calibration_context():
        m(x)
    scale = m.quant_params.scale("x")
    m.use_quantization = True
    m.set_quant_params_locked(True)
    with m.calibration_context():  # locked: no reset, no recalibration
        m(x * 10)
    assert m.quant_params.scale("x") == scale
    m.set_quant_params_locked(False)
    with m.calibration_context():
        m(x * 10)
    assert m.quant_params.scale("x") > scale


def test_float_forward_matches_nn_gru_and_refuses_backward(cuda):
    T, B, I, H = 7, 10, 6, 40
    torch.manual_seed(8)
    ref = torch.nn.GRU(I, H, bidirectional=True)
    m = Q.QuantGRU(I, H, bidirectional=True)
    m.load_state_dict(ref.state_dict())
    m = m.to(cuda)
    x = torch.randn(T, B, I)
    hx = torch.randn(2, B, H) * 0.2
    with torch.no_grad():
        y, hn = m(x.to(cuda), hx.to(cuda))
        ye, hne = ref(x, hx)
    np.testing.assert_allclose(y.cpu().numpy(), ye.numpy(), atol=1e-5)
    np.testing.assert_allclose(hn.cpu().numpy(), hne.numpy(), atol=1e-5)
    y, _ = m(x.to(cuda))
    with pytest.raises(NotImplementedError, match="float GRU backward"):
        y.sum().backward()


@pytest.mark.parametrize("batch_first", [False, True])
def test_bidirectional_layout_in_library_equals_per_direction_path(cuda, batch_first):
    """The bidirectional QAT path (each direction reads x in place, output / h_n assembled,
    the output gradient split and dx assembled by the library) equals the per-direction
    GRUFunction path with PyTorch's flips, concatenations and transposes: outputs and h_n bit
    for bit, gradients within 1e-5.  The input is a view with padded rows and the loss a mean
    (a stride-0 output gradient) plus a term on h_n."""
    T, B, I, H = 7, 20, 12, 48
    m, x_tbi, hx = _module_case(True, batch_first, True, "c3", 31, shape=(T, B, I, H))
    m = m.to(cuda)
    x_in = (x_tbi.transpose(0, 1).contiguous() if batch_first else x_tbi).to(cuda)
    hx = hx.to(cuda)
    with m.calibration_context():
        m(x_in, hx)
    m.use_quantization = True
    m.train()
    wide = torch.zeros(*x_in.shape[:2], I + 5, device=cuda)
    wide[..., :I] = x_in
    results = []
    for fused in (True, False):
        m.zero_grad(set_to_none=True)
        leaf = wide.clone().requires_grad_(True)
        hxl = hx.clone().requires_grad_(True)
        xv = leaf[..., :I]
        if fused:
            out, hn = m(xv, hxl)
        else:
            x_tb = xv.transpose(0, 1) if batch_first else xv
            out, hn = m._forward_cuda(x_tb.contiguous(), hxl)
            if batch_first:
                out = out.transpose(0, 1).contiguous()
        (out.mean() + 0.5 * hn.sum()).backward()
        torch.cuda.synchronize()
        grads = [leaf.grad, hxl.grad] + [p.grad for p in m.parameters()]
        results.append((out.detach(), hn.detach(), [g.clone() for g in grads]))
    (o1, h1, g1), (o2, h2, g2) = results
    assert torch.equal(o1, o2) and torch.equal(h1, h2)
    for k, (a, b) in enumerate(zip(g1, g2)):
        a, b = a.cpu().numpy(), b.cpu().numpy()
        scale = max(float(np.abs(b).max()), 1e-30)
        np.testing.assert_allclose(a, b, rtol=1e-5, atol=1e-6 * scale, err_msg=f"grad {k}")


@pytest.mark.parametrize("bidirectional", [False, True])
def test_quant_params_document_reproduces_qat_forward(cuda, tmp_path, bidirectional):
    """Grids calibrated on the GPU, written with export_quant_params and read into a fresh
    module with the same weights: the quantised forward is bit for bit the same."""
    T, B, I, H = 5, 24, 10, 32
    m, x_tbi, hx = _module_case(bidirectional, False, True, "po2-16b", 41, shape=(T, B, I, H))
    m = m.to(cuda)
    x, hx = x_tbi.to(cuda), hx.to(cuda)
    with m.calibration_context():
        m(x, hx)
    m.use_quantization = True
    path = tmp_path / "gru_qp.json"
    m.export_quant_params(str(path))
    n = Q.QuantGRU(I, H, bidirectional=bidirectional).to(cuda)
    n.load_state_dict(m.state_dict())
    n.load_quant_params(str(path))
    n.use_quantization = True
    with torch.no_grad():
        o1, h1 = m(x, hx)
        o2, h2 = n(x, hx)
    assert torch.equal(o1, o2) and torch.equal(h1, h2)


@pytest.mark.parametrize("bidirectional", [False, True])
def test_aimet_encodings_reproduce_qat_forward(cuda, bidirectional):
    """Grids calibrated on the GPU, exported with export_quant_params_to_aimet_format, passed
    through JSON and loaded into a fresh module with the same weights
    (load_quant_params_from_aimet_format): the quantised forward is bit for bit the same."""
    import json
    T, B, I, H = 5, 24, 10, 32
    print(f"[quantgru aimet] bidirectional={bidirectional}", flush=True)
    m, x_tbi, hx = _module_case(bidirectional, False, True, "c3", 43, shape=(T, B, I, H))
    m = m.to(cuda)
    x, hx = x_tbi.to(cuda), hx.to(cuda)
    with m.calibration_context():
        m(x, hx)
    m.use_quantization = True
    enc = json.loads(json.dumps(m.export_quant_params_to_aimet_format({}, "model.gru")))
    n = Q.QuantGRU(I, H, bidirectional=bidirectional).to(cuda)
    n.load_state_dict(m.state_dict())
    assert n.load_quant_params_from_aimet_format(enc, "model.gru")
    n.use_quantization = True
    with torch.no_grad():
        o1, h1 = m(x, hx)
        o2, h2 = n(x, hx)
    assert torch.equal(o1, o2) and torch.equal(h1, h2)


@pytest.mark.parametrize("bits,mse,mae,cos", [(8, 1e-3, 0.05, 0.999), (16, 1e-4, 0.015, 0.999)])
def test_quantized_module_tracks_nn_gru_with_reference_thresholds(cuda, bits, mse, mae, cos):
    """operators/quant-gru/tests/test_quant_gru.py:400-526: QuantGRU with nn.GRU's weights,
    set_all_bitwidth(bits), calibrated on one U(-0.7, 0.8) batch (I=128, H=256, B=64, T=50),
    then evaluated on a fresh batch; MSE, MAE and cosine similarity against nn.GRU within the
    reference's thresholds.  At 16 bits every grid is 16-bit, the recurrent weights included."""
    I, H, B, T = 128, 256, 64, 50
    print(f"[quantgru vs nn.GRU] bits={bits}", flush=True)
    torch.manual_seed(0)
    ref = torch.nn.GRU(I, H).to(cuda)
    m = Q.QuantGRU(I, H).to(cuda)
    m.load_state_dict(ref.state_dict())
    m.set_all_bitwidth(bits)
    calib = torch.rand(T, B, I, device=cuda) * 1.5 - 0.7
    m.calibrating = True
    with torch.no_grad():
        m(calib)
    m.calibrating = False
    m.finalize_calibration()
    m.use_quantization = True
    x = torch.rand(T, B, I, device=cuda) * 1.5 - 0.7
    ref.eval()
    m.eval()
    with torch.no_grad():
        y_ref, _ = ref(x)
        y, _ = m(x)
    d = (y - y_ref).double()
    got_mse = float((d ** 2).mean())
    got_mae = float(d.abs().mean())
    got_cos = float(torch.nn.functional.cosine_similarity(y.double().flatten(),
                                                          y_ref.double().flatten(), dim=0))
    assert got_mse < mse and got_mae < mae and got_cos > cos, (got_mse, got_mae, got_cos)
