"""Pin the GRU oracle (oracle/gru_oracle.c) and the product's host parameter code.

* Quantisation parameters and activation LUTs: oracle == the reference's own C++
  (compiled from /root/reference into oracle/_ref) == librxmet host code, bit for bit,
  over random ranges and every configuration axis the reference exposes.
* Calibration forward: oracle == reference forwardWithCalibrationCPU.
* Quantised forward: with 16-bit grids the FP32-carrier GRU tracks torch.nn.GRU (gate
  order, transposes, update rule); train and eval forwards agree exactly; codes are
  integral and masks binary (tests/recurrent/test_gru_storage.py:31-64).
* Backward: equals torch autograd through the reference's surrogate construction
  (tests/recurrent/test_gru_autograd.py:21-48) built on the oracle's saved tensors.
"""
import ctypes

import numpy as np
import pytest
import torch

import gru_oracle as GO
import rxmet_gru_abi as A
import rxmet_lib

f32 = np.float32

needs_ref = pytest.mark.skipif(not GO.has_ref(), reason="oracle/_ref not built (no reference checkout)")


def _random_stats(H, seed, scale=1.0):
    g = np.random.default_rng(seed)
    s = A.empty_stats(H)
    n = A.NGRIDS
    lo = -(g.random(n) * 3 * scale).astype(f32)
    hi = (g.random(n) * 3 * scale).astype(f32)
    # gate outputs live in (0, 1) / (-1, 1)
    for i, (a, b) in {7: (0.02, 0.97), 8: (0.1, 0.9), 9: (-0.95, 0.99)}.items():
        lo[i], hi[i] = a * g.random(), b
    lo[7] = 0.49  # narrow range -> ensureMinRange kicks in
    hi[7] = 0.51
    s[:n], s[n:2 * n] = lo, hi
    C = 3 * H
    for k in range(A.NCHAN):
        b0 = 2 * n + 2 * k * C
        amp = (g.random(C) * 0.4 + 0.01).astype(f32)
        s[b0:b0 + C] = -amp * g.random(C).astype(f32)
        s[b0 + C:b0 + 2 * C] = amp
    return s


def _configs():
    out = []
    c = A.default_config()
    out.append(("default-8b-sym", c))
    c = A.set_all_bitwidth(A.default_config(), 8, False)
    out.append(("8b-asym", c))
    c = A.set_all_bitwidth(A.default_config(), 16, False)
    out.append(("16b-asym", c))
    c = A.set_all_bitwidth(A.default_config(), 8, False)
    c.op[A.GRID["h"]].bits = 16
    for k in range(4):
        c.chan[k].granularity = A.PER_TENSOR
    out.append(("c3-like-per-tensor-w", c))
    c = A.set_all_bitwidth(A.default_config(), 16, False)
    c.chan[0].bits = c.chan[1].bits = 4
    for k in range(4):
        c.chan[k].granularity = A.PER_GATE
    c.use_pot2 = 1
    out.append(("c5-like-pot2-cover", c))
    for m in (A.POT_ROUND, A.POT_FLOOR):
        c = A.set_all_bitwidth(A.default_config(), 8, False)
        c.use_pot2 = 1
        c.pot_method = m
        out.append((f"pot2-method{m}", c))
    c = A.set_all_bitwidth(A.default_config(), 4, True)
    out.append(("4b-sym", c))
    return out


def _product_params(ranges, cfg):
    qp = A.new_qparams(ranges.hidden)
    rxmet_lib.call("rxmet_gru_make_params", ctypes.byref(ranges), ctypes.byref(cfg), ctypes.byref(qp))
    luts = (A.PwlLut * 3)()
    rxmet_lib.call("rxmet_gru_make_luts", ctypes.byref(qp), luts)
    return qp, luts


def _params_equal(a, b, H):
    for i in range(A.NGRIDS):
        assert np.float32(a.g[i].scale).tobytes() == np.float32(b.g[i].scale).tobytes(), \
            (A.GRID_NAMES[i], a.g[i].scale, b.g[i].scale)
        assert a.g[i].zero_point == b.g[i].zero_point, (A.GRID_NAMES[i], a.g[i].zero_point,
                                                        b.g[i].zero_point)
    for k in range(A.NCHAN):
        np.testing.assert_array_equal(A.qparams_chan(a, k), A.qparams_chan(b, k))


def _luts_equal(a, b):
    for i in range(3):
        for s in range(16):
            x, y = a[i].seg[s], b[i].seg[s]
            assert (x.q_b, x.n, x.c, x.threshold) == (y.q_b, y.n, y.c, y.threshold), (i, s)
        assert a[i].zp_x == b[i].zp_x


@needs_ref
@pytest.mark.parametrize("name,cfg", _configs(), ids=[n for n, _ in _configs()])
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_params_and_luts_match_reference(name, cfg, seed):
    H = 8
    stats = _random_stats(H, seed)
    ranges = A.make_ranges(stats, H)
    ref_qp, ref_luts = GO.make_params(ranges, cfg, ref=True)
    or_qp, or_luts = GO.make_params(ranges, cfg)
    pr_qp, pr_luts = _product_params(ranges, cfg)
    _params_equal(or_qp, ref_qp, H)
    _params_equal(pr_qp, ref_qp, H)
    _luts_equal(or_luts, ref_luts)
    _luts_equal(pr_luts, ref_luts)


def test_asymmetric_weights_are_rejected():
    # gru_calibration_helpers.h:7-13
    cfg = A.default_config()
    cfg.chan[0].symmetric = 0
    ranges = A.make_ranges(_random_stats(4, 0), 4)
    qp = A.new_qparams(4)
    with pytest.raises(rxmet_lib.RxmetError, match="symmetric"):
        rxmet_lib.call("rxmet_gru_make_params", ctypes.byref(ranges), ctypes.byref(cfg),
                       ctypes.byref(qp))


def test_effective_scale_known_values():
    lib = rxmet_lib.load()
    for s in (0.0173, 1 / 15, 2.0 ** -7, 3.3e-5, 0.9):
        e = GO.effective_scale(s, False)
        assert e == lib.rxmet_gru_effective_scale(s, 0)
        assert abs(e - s) / s < 2 ** -16          # 16-bit mantissa
        m, ex = np.frexp(np.float64(e))
        assert float(m * 65536).is_integer()
    assert GO.effective_scale(2.0 ** -9, True) == 2.0 ** -9
    assert GO.effective_scale(0.003, True) == 2.0 ** -8   # round(-log2 .003) = 8


def _gru_weights(I, H, seed, amp=None):
    g = torch.Generator().manual_seed(seed)
    k = amp if amp is not None else 1.0 / H ** 0.5
    w_ih = (torch.rand(3 * H, I, generator=g) * 2 - 1) * k
    w_hh = (torch.rand(3 * H, H, generator=g) * 2 - 1) * k
    b_ih = (torch.rand(3 * H, generator=g) * 2 - 1) * k
    b_hh = (torch.rand(3 * H, generator=g) * 2 - 1) * k
    return w_ih, w_hh, b_ih, b_hh


def to_haste(w_ih, w_hh, b_ih, b_hh):
    """PyTorch (r, z, n) -> (z, r, n) and transpose (quant_gru.py:664-759)."""
    def swap(t):
        r, z, n = t.chunk(3, 0)
        return torch.cat([z, r, n], 0)
    return (swap(w_ih).t().contiguous().numpy(), swap(w_hh).t().contiguous().numpy(),
            swap(b_ih).numpy(), swap(b_hh).numpy())


@needs_ref
def test_calibration_forward_matches_reference():
    T, B, I, H = 5, 3, 6, 8
    W, R, bw, br = to_haste(*_gru_weights(I, H, 0))
    x = np.random.default_rng(1).standard_normal((T, B, I)).astype(f32)
    h0 = (np.random.default_rng(2).standard_normal((B, H)) * 0.3).astype(f32)
    h_r, v_r, s_r = GO.forward_calibrate(W, R, bw, br, x, h0, ref=True)
    h_o, v_o, s_o = GO.forward_calibrate(W, R, bw, br, x, h0)
    np.testing.assert_array_equal(h_o, h_r)
    np.testing.assert_array_equal(v_o, v_r)
    np.testing.assert_array_equal(s_o, s_r)


def test_calibration_forward_matches_torch_gru():
    T, B, I, H = 7, 4, 5, 6
    w = _gru_weights(I, H, 3)
    x = np.random.default_rng(4).standard_normal((T, B, I)).astype(f32)
    ref = torch.nn.GRU(I, H)
    with torch.no_grad():
        ref.weight_ih_l0.copy_(w[0]); ref.weight_hh_l0.copy_(w[1])
        ref.bias_ih_l0.copy_(w[2]); ref.bias_hh_l0.copy_(w[3])
        y, _ = ref(torch.from_numpy(x))
    h, _, _ = GO.forward_calibrate(*to_haste(*w), x)
    np.testing.assert_allclose(h[1:], y.numpy(), rtol=0, atol=2e-6)


def calibrated_params(W, R, bw, br, x, cfg, h0=None):
    _, _, stats = GO.forward_calibrate(W, R, bw, br, x, h0)
    ranges = A.make_ranges(stats, R.shape[0])
    qp, _ = GO.make_params(ranges, cfg)
    return qp, ranges


def test_quant_forward_tracks_float_gru_at_16_bits():
    T, B, I, H = 6, 4, 5, 8
    w = _gru_weights(I, H, 5)
    W, R, bw, br = to_haste(*w)
    x = np.random.default_rng(6).standard_normal((T, B, I)).astype(f32)
    cfg = A.set_all_bitwidth(A.default_config(), 16, False)
    qp, _ = calibrated_params(W, R, bw, br, x, cfg)
    out = GO.forward_quant(W, R, bw, br, x, qp)
    ref = torch.nn.GRU(I, H)
    with torch.no_grad():
        ref.weight_ih_l0.copy_(w[0]); ref.weight_hh_l0.copy_(w[1])
        ref.bias_ih_l0.copy_(w[2]); ref.bias_hh_l0.copy_(w[3])
        y, _ = ref(torch.from_numpy(x))
    # 16-segment PWL sigmoid/tanh approximations bound the deviation (a few 1e-3)
    err = np.abs(out["h"][1:] - y.numpy())
    assert err.max() < 3e-2 and err.mean() < 5e-3, (err.max(), err.mean())


def test_train_eval_forward_equal_codes_integral_masks_binary():
    T, B, I, H = 4, 3, 5, 6
    W, R, bw, br = to_haste(*_gru_weights(I, H, 7))
    x = np.random.default_rng(8).standard_normal((T, B, I)).astype(f32)
    h0 = (np.random.default_rng(9).standard_normal((B, H)) * 0.5).astype(f32)
    cfg = A.set_all_bitwidth(A.default_config(), 8, False)
    cfg.op[A.GRID["h"]].bits = 16
    qp, _ = calibrated_params(W, R, bw, br, x, cfg)
    tr = GO.forward_quant(W, R, bw, br, x, qp, h0=h0, training=True)
    ev = GO.forward_quant(W, R, bw, br, x, qp, h0=h0, training=False)
    np.testing.assert_array_equal(tr["h"], ev["h"])
    np.testing.assert_array_equal(tr["v"], ev["v"])
    for k in ("W_q", "R_q", "bw_q", "br_q", "x_q"):
        assert np.all(tr[k] == np.round(tr[k])), k
    for k in GO.MASKS:
        assert set(np.unique(tr[k])) <= {0, 1}, k


def _surrogate_grads(fwd, qp, dh_out, dh_last):
    """Restatement of the reference's surrogate (test_gru_autograd.py:21-48) on the
    oracle's saved tensors: every clamp masks its input, gates use dequantised outputs."""
    T, B, I = fwd["x_q"].shape
    H = fwd["R_q"].shape[0]
    pot = bool(qp.use_pot2)
    es = lambda s: GO.effective_scale(float(s), pot)
    sW = torch.tensor([es(s) for s in A.qparams_chan(qp, 0)])
    sR = torch.tensor([es(s) for s in A.qparams_chan(qp, 1)])
    sbw = torch.tensor([es(s) for s in A.qparams_chan(qp, 2)])
    sbr = torch.tensor([es(s) for s in A.qparams_chan(qp, 3)])
    gx = qp.g[A.GRID["x"]]
    t = lambda a: torch.from_numpy(np.asarray(a, np.float64))
    w = (t(fwd["W_q"]) * sW.double()).requires_grad_()
    r = (t(fwd["R_q"]) * sR.double()).requires_grad_()
    bw_ = (t(fwd["bw_q"]) * sbw.double()).requires_grad_()
    br_ = (t(fwd["br_q"]) * sbr.double()).requires_grad_()
    x = ((t(fwd["x_q"]) - gx.zero_point) * es(gx.scale)).requires_grad_()
    h = t(fwd["h"])
    v = t(fwd["v"])
    m = {k: t(fwd[k]) for k in GO.MASKS if fwd[k] is not None}
    h0 = h[0].clone().requires_grad_()

    def masked(val, mask):
        return val.detach() + (val - val.detach()) * mask

    def anchor(val, actual):
        return actual.detach() + (val - val.detach())

    mw, mr = masked(w, m["W_mask"]), masked(r, m["R_mask"])
    mbw, mbr = masked(bw_, m["bw_mask"]), masked(br_, m["br_mask"])
    mx = masked(x, m["x_mask"])
    prev = masked(h0, m["h0_mask"]) if "h0_mask" in m else h0
    ys = []
    for s in range(T):
        p = masked(mx[s] @ mw + mbw, m["ih_mask"][s])
        q = masked(prev @ mr + mbr, m["hh_mask"][s])
        z0, r0, n0, qg = v[s].chunk(4, dim=-1)
        iz, ir, ig = m["gate_in_mask"][s].chunk(3, dim=-1)
        oz, orr, og = m["gate_out_mask"][s].chunk(3, dim=-1)
        pz, pr, pg = p.chunk(3, dim=-1)
        qz, qr, qn = q.chunk(3, dim=-1)

        def act(pre, out, mask, der):
            return out.detach() + (pre - pre.detach()) * mask * der.detach()

        z = act(pz + qz, z0, iz * oz, z0 * (1 - z0))
        rr = act(pr + qr, r0, ir * orr, r0 * (1 - r0))
        cand = act(pg + rr * anchor(qn, qg), n0, ig * og, 1 - n0 * n0)
        prev = anchor(masked(z * prev + (1 - z) * cand, m["h_mask"][s]), h[s + 1])
        ys.append(prev)
    y = torch.stack(ys)
    loss = (y * t(dh_out)).sum() + (prev * t(dh_last)).sum()
    loss.backward()
    return {"dW": w.grad, "dR": r.grad, "dbw": bw_.grad, "dbr": br_.grad, "dx": x.grad,
            "dh0": h0.grad}


@pytest.mark.parametrize("bits,h_bits,seed", [(8, 8, 10), (8, 16, 11), (16, 16, 12)])
def test_backward_matches_autograd_surrogate(bits, h_bits, seed):
    T, B, I, H = 5, 3, 4, 6
    W, R, bw, br = to_haste(*_gru_weights(I, H, seed, amp=0.9))
    x = np.random.default_rng(seed).standard_normal((T, B, I)).astype(f32)
    h0 = (np.random.default_rng(seed + 1).standard_normal((B, H)) * 0.5).astype(f32)
    cfg = A.set_all_bitwidth(A.default_config(), bits, False)
    cfg.op[A.GRID["h"]].bits = h_bits
    # narrow the calibrated ranges a little so that every clamp family actually fires
    _, _, stats = GO.forward_calibrate(W, R, bw, br, x, h0)
    stats[:A.NGRIDS] *= 0.8
    stats[A.NGRIDS:2 * A.NGRIDS] *= 0.8
    qp, _ = GO.make_params(A.make_ranges(stats, H), cfg)
    fwd = GO.forward_quant(W, R, bw, br, x, qp, h0=h0)
    for k in ("ih_mask", "gate_in_mask", "h_mask"):
        assert fwd[k].min() == 0, f"{k} never clamps; the test would not cover it"
    g = np.random.default_rng(seed + 2)
    dh_out = g.standard_normal((T, B, H)).astype(f32)
    dh_last = g.standard_normal((B, H)).astype(f32)
    dh_new = np.zeros((T + 1, B, H), f32)
    dh_new[1:] = dh_out
    dh_new[-1] += dh_last
    got = GO.backward_quant(fwd, dh_new, qp)
    exp = _surrogate_grads(fwd, qp, dh_out, dh_last)
    for k in ("dW", "dR", "dbw", "dbr", "dx", "dh0"):
        e = exp[k].numpy()
        np.testing.assert_allclose(got[k], e, rtol=1e-5, atol=1e-6 * max(1.0, np.abs(e).max()),
                                   err_msg=k)


@needs_ref
@pytest.mark.parametrize("seed", [5, 9])
def test_reference_int_carrier_agrees_with_fp_carrier(seed):
    """Pins the compiled reference CPU int carrier (``quantGRUForwardCPU``,
    gru_host.cc:161-252 / gru_forward_cpu_quant.cc:109-343), the checker for an int-IO forward.
    Both carriers share the grids and LUTs and differ only in how the rescales round, so
    at 8-bit grids they give the same h codes, and at 16-bit grids they stay within a few steps
    of the h grid.  Both track the float GRU."""
    T, B, I, H = 6, 4, 5, 8
    w = _gru_weights(I, H, seed)
    W, R, bw, br = to_haste(*w)
    x = np.random.default_rng(seed + 1).standard_normal((T, B, I)).astype(f32)
    ref = torch.nn.GRU(I, H)
    with torch.no_grad():
        ref.weight_ih_l0.copy_(w[0]); ref.weight_hh_l0.copy_(w[1])
        ref.bias_ih_l0.copy_(w[2]); ref.bias_hh_l0.copy_(w[3])
        y, _ = ref(torch.from_numpy(x))
    for bits in (8, 16):
        cfg = A.set_all_bitwidth(A.default_config(), bits, False)
        qp, ranges = calibrated_params(W, R, bw, br, x, cfg)
        fp = GO.forward_quant(W, R, bw, br, x, qp)["h"]
        h, _ = GO.ref_forward_ptq(W, R, bw, br, x, ranges, cfg)
        steps = np.abs(h - fp) / qp.g[A.GRID["h"]].scale
        if bits == 8:
            np.testing.assert_array_equal(h, fp)
        else:
            assert steps.max() <= 3.0 and steps.mean() <= 0.5, (steps.max(), steps.mean())
        assert np.abs(h[1:] - y.numpy()).max() < 3e-2
