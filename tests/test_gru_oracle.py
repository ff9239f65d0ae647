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
    gru_host.cc:161-252 / gru_forward_cpu_quant.cc:109-343), the checker for an int-IO forward,
    and the FP carrier's v against it.  Both carriers share the grids and LUTs and differ only
    in how the rescales round: on these short 8-bit cases they give the same h codes and the
    same v (z, r, n, hh_n, dequantised with the same grids); at 16-bit grids h stays within 2
    steps of the h grid with at least 3/4 of the codes equal.  Both track the float GRU."""
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
        fwd = GO.forward_quant(W, R, bw, br, x, qp)
        fp = fwd["h"]
        h, v = GO.ref_forward_ptq(W, R, bw, br, x, ranges, cfg)
        steps = np.abs(h - fp) / GO.effective_scale(qp.g[A.GRID["h"]].scale, False)
        if bits == 8:
            np.testing.assert_array_equal(h, fp)
            np.testing.assert_array_equal(v, fwd["v"])
        else:
            assert steps.max() <= 2.01 and (steps < 0.5).mean() >= 0.75, \
                (steps.max(), (steps < 0.5).mean())
        assert np.abs(h[1:] - y.numpy()).max() < 3e-2


def _torch_fp_carrier(W, R, bw, br, x, h0, qp, luts, gran):
    """An independent restatement of the reference's FP-carrier forward, written from its CUDA
    source and vectorised in torch fp32: boundary quantisation (quantize_ops.cu:109-142,
    quantize_ops_helper.h:132-140: rint(v / s_eff) then + zp), host rescale ratios
    (gru_forward_gpu_quant_fp.cu:853-1044, raw scales), weight sums (:474-486), bias rescale
    (:138-163), gates (:174-314), PWL (:90-109), hidden update (:335-393) and clamp_f
    (quantize_ops_helper.h:332-354).  Every mask is taken at its own clamp, 1 = kept."""
    fl = torch.float32
    T, B, I = x.shape
    H = R.shape[0]
    C = 3 * H
    pot = bool(qp.use_pot2)
    g = lambda n: qp.g[A.GRID[n]]
    eff = lambda s: GO.effective_scale(float(s), pot)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a, f32))

    def clampk(v, bits, uns):
        lo, hi = (0.0, 2.0 ** bits - 1) if uns else (-2.0 ** (bits - 1), 2.0 ** (bits - 1) - 1)
        return v.clamp(lo, hi), ((v >= lo) & (v <= hi)).to(torch.uint8)

    def gclamp(v, name):
        return clampk(v, g(name).bits, g(name).is_unsigned)

    def qweight(M, k):
        sc = A.qparams_chan(qp, k)
        cols = np.arange(C)
        idx = {A.PER_TENSOR: np.zeros(C, int), A.PER_GATE: (cols // H) * H,
               A.PER_CHANNEL: cols}[gran[k]]
        s_eff = torch.tensor([eff(sc[i]) for i in idx], dtype=fl)
        return clampk(torch.round(t(M) / s_eff), qp.chan_bits[k], qp.chan_unsigned[k])

    Wq, Wm = qweight(W, 0)
    Rq, Rm = qweight(R, 1)
    bwq, bwm = qweight(bw[None], 2)
    brq, brm = qweight(br[None], 3)
    gx, gh = g("x"), g("h")
    xq, xm = gclamp(torch.round(t(x) / eff(gx.scale)) + float(gx.zero_point), "x")
    if h0 is None:
        hq, h0m = torch.full((B, H), float(gh.zero_point)), None
    else:
        hq, h0m = gclamp(torch.round(t(h0) / eff(gh.scale)) + float(gh.zero_point), "h")

    S = lambda n: f32(g(n).scale)
    zp = lambda n: float(g(n).zero_point)
    sW, sR, sbw, sbr = (A.qparams_chan(qp, k).astype(f32) for k in range(4))
    sx, sh = S("x"), S("h")
    tv = lambda vals: torch.tensor(np.array(vals, f32))
    inv_gemm_x = tv([f32(sW[c] * sx) / S("weight_ih_linear") for c in range(C)])
    inv_bw = tv([sbw[c] / f32(sW[c] * sx) for c in range(C)])
    inv_gemm_h = tv([f32(sR[c] * sh) / S("weight_hh_linear") for c in range(C)])
    inv_br = tv([sbr[c] / f32(sR[c] * sh) for c in range(C)])

    def colsum(Mq):  # sequential fp32 sum over rows
        s = torch.zeros(C, dtype=fl)
        for row in Mq:
            s = s + row
        return s

    wsum_zp = colsum(Wq) * zp("x")
    rsum_zp = colsum(Rq) * zp("h")
    ratio = lambda a, b: float(f32(a) / f32(b))
    r_ih = {gt: ratio(S("weight_ih_linear"), S(gt + "_gate_input")) for gt in ("update", "reset", "new")}
    r_hh = {gt: ratio(S("weight_hh_linear"), S(gt + "_gate_input")) for gt in ("update", "reset")}
    r_rmul = ratio(f32(S("reset_gate_output") * S("weight_hh_linear")), S("new_gate_input"))
    q1 = float(f32(np.rint(f32(1.0) / S("update_gate_output"))) + f32(zp("update_gate_output")))
    inv_upd = ratio(f32(S("update_gate_output") * sh), sh)
    inv_n_h = ratio(S("new_gate_output"), sh)

    def pwl(q, lut, out):
        thr = torch.tensor([float(lut.seg[i].threshold) for i in range(16)], dtype=fl)
        lt = q[..., None] < thr
        seg = torch.where(lt.any(-1), lt.to(torch.int64).argmax(-1), torch.full_like(q, 15, dtype=torch.int64))
        qb = torch.tensor([float(lut.seg[i].q_b) for i in range(16)], dtype=fl)[seg]
        n = torch.tensor([lut.seg[i].n for i in range(16)])[seg]
        c = torch.tensor([float(lut.seg[i].c) for i in range(16)], dtype=fl)[seg]
        val = torch.round(torch.ldexp(qb * (q - float(lut.zp_x)), -n).to(fl)) + c
        return gclamp(val, out)

    gih_all = (xq.double() @ Wq.double()).to(fl)  # exact integer sums, rounded once
    bias_x = torch.round(bwq[0] * inv_bw)
    bias_h = torch.round(brq[0] * inv_br)
    hs, vs, mk = [hq], [], {k: [] for k in ("ih", "hh", "gin", "gout", "h")}
    for s in range(T):
        ghh = (hq.double() @ Rq.double()).to(fl)
        wih, mih = gclamp(torch.round(((gih_all[s] - wsum_zp) + bias_x) * inv_gemm_x)
                          + zp("weight_ih_linear"), "weight_ih_linear")
        whh, mhh = gclamp(torch.round(((ghh - rsum_zp) + bias_h) * inv_gemm_h)
                          + zp("weight_hh_linear"), "weight_hh_linear")
        ci = lambda a, k: a[:, k * H:(k + 1) * H]
        wi = lambda k: ci(wih, k) - zp("weight_ih_linear")
        wh = lambda k: ci(whh, k) - zp("weight_hh_linear")
        zin, mz = gclamp((torch.round(wi(0) * r_ih["update"]) + torch.round(wh(0) * r_hh["update"]))
                         + zp("update_gate_input"), "update_gate_input")
        z, oz = pwl(zin, luts[0], "update_gate_output")
        rin, mr = gclamp((torch.round(wi(1) * r_ih["reset"]) + torch.round(wh(1) * r_hh["reset"]))
                         + zp("reset_gate_input"), "reset_gate_input")
        r, orr = pwl(rin, luts[1], "reset_gate_output")
        rh = torch.round(((r - zp("reset_gate_output")) * wh(2)) * r_rmul)
        nin, mn = gclamp((torch.round(wi(2) * r_ih["new"]) + rh) + zp("new_gate_input"),
                         "new_gate_input")
        n, on = pwl(nin, luts[2], "new_gate_output")
        n_al = torch.round((n - zp("new_gate_output")) * inv_n_h) + zp("h")
        old = (z - zp("update_gate_output")) * (hq - zp("h"))
        new = (q1 - z) * (n_al - zp("h"))
        hq, mh = gclamp(torch.round((old + new) * inv_upd) + zp("h"), "h")
        hs.append(hq)
        deq = lambda q, name: (q - zp(name)) * eff(S(name))
        vs.append(torch.cat([deq(z, "update_gate_output"), deq(r, "reset_gate_output"),
                             deq(n, "new_gate_output"), deq(ci(whh, 2), "weight_hh_linear")], -1))
        for k, m in (("ih", mih), ("hh", mhh), ("gin", torch.cat([mz, mr, mn], -1)),
                     ("gout", torch.cat([oz, orr, on], -1)), ("h", mh)):
            mk[k].append(m)
    h = (torch.stack(hs) - zp("h")) * eff(sh)
    out = {"h": h, "v": torch.stack(vs), "W_q": Wq, "R_q": Rq, "bw_q": bwq[0], "br_q": brq[0],
           "x_q": xq, "x_mask": xm, "h0_mask": h0m, "W_mask": Wm, "R_mask": Rm,
           "bw_mask": bwm[0], "br_mask": brm[0], "ih_mask": torch.stack(mk["ih"]),
           "hh_mask": torch.stack(mk["hh"]), "gate_in_mask": torch.stack(mk["gin"]),
           "gate_out_mask": torch.stack(mk["gout"]), "h_mask": torch.stack(mk["h"])}
    return {k: (None if v is None else v.numpy()) for k, v in out.items()}


def _narrowed_case(I, H, T, B, cfg, seed, shrink=0.7, h_shrink=1.0):
    W, R, bw, br = to_haste(*_gru_weights(I, H, seed, amp=0.9))
    x = np.random.default_rng(seed).standard_normal((T, B, I)).astype(f32)
    h0 = (np.random.default_rng(seed + 1).standard_normal((B, H)) * 0.8).astype(f32)
    _, _, stats = GO.forward_calibrate(W, R, bw, br, x, h0)
    # narrow every range so that each clamp family fires somewhere
    n = A.NGRIDS
    stats[:n] *= shrink
    stats[n:2 * n] *= shrink
    stats[A.GRID["h"]] *= h_shrink
    stats[n + A.GRID["h"]] *= h_shrink
    for k in range(A.NCHAN):
        b0 = 2 * n + 2 * k * 3 * H
        stats[b0:b0 + 6 * H] *= shrink
    qp, luts = GO.make_params(A.make_ranges(stats, H), cfg)
    return W, R, bw, br, x, h0, qp, luts


_RESTATEMENT_CASES = [  # name, bits, h bits, pot2, weight granularity, unsigned h, shrink, h shrink
    ("8b-asym-per-channel", 8, 8, False, A.PER_CHANNEL, False, 0.7, 1.0),
    ("c3-16b-h", 8, 16, False, A.PER_CHANNEL, False, 0.7, 1.0),
    ("16b-pot2-per-gate", 16, 16, True, A.PER_GATE, False, 0.4, 1.0),
    ("8b-per-tensor-h-unsigned", 8, 12, False, A.PER_TENSOR, True, 0.7, 1.0),
    ("4b-weights-tight", 4, 8, False, A.PER_CHANNEL, False, 0.3, 1.0),
    ("h-grid-clamps", 8, 8, False, A.PER_CHANNEL, False, 0.7, 0.1),
]


def _restatement_case(bits, h_bits, pot2, gran, h_unsigned, shrink, h_shrink, with_h0):
    T, B, I, H = 5, 6, 4, 8
    cfg = A.set_all_bitwidth(A.default_config(), bits, False)
    cfg.op[A.GRID["h"]].bits = h_bits
    cfg.op[A.GRID["h"]].is_unsigned = int(h_unsigned)
    cfg.use_pot2 = int(pot2)
    for k in range(4):
        cfg.chan[k].granularity = gran
    W, R, bw, br, x, h0, qp, luts = _narrowed_case(I, H, T, B, cfg, 31, shrink, h_shrink)
    h0 = h0 if with_h0 else None
    exp = GO.forward_quant(W, R, bw, br, x, qp, h0=h0, training=True)
    got = _torch_fp_carrier(W, R, bw, br, x, h0, qp, luts, [gran] * 4)
    return exp, got


@pytest.mark.parametrize("name,bits,h_bits,pot2,gran,h_unsigned,shrink,h_shrink",
                         _RESTATEMENT_CASES)
@pytest.mark.parametrize("with_h0", [False, True])
def test_fp_carrier_equals_independent_torch_restatement(name, bits, h_bits, pot2, gran,
                                                         h_unsigned, shrink, h_shrink, with_h0):
    """Every output of the oracle's forward — h, v (z, r, n, hh_n), the codes and all eleven
    mask families — equals a second implementation written from the reference's CUDA source
    in torch, which takes each mask at its own clamp."""
    exp, got = _restatement_case(bits, h_bits, pot2, gran, h_unsigned, shrink, h_shrink, with_h0)
    for k in ("h", "v", "W_q", "R_q", "bw_q", "br_q", "x_q") + GO.MASKS:
        if exp[k] is None:
            assert got[k] is None, k
            continue
        np.testing.assert_array_equal(got[k], exp[k], err_msg=k)


def test_restatement_cases_fire_every_clamp_family():
    """The cases above clamp somewhere in every mask family, so the equality covers both
    values of every mask."""
    fired = set()
    for _, bits, h_bits, pot2, gran, h_unsigned, shrink, h_shrink in _RESTATEMENT_CASES:
        _, got = _restatement_case(bits, h_bits, pot2, gran, h_unsigned, shrink, h_shrink, True)
        fired |= {k for k in GO.MASKS if got[k] is not None and got[k].min() == 0}
    assert fired == set(GO.MASKS), sorted(set(GO.MASKS) - fired)
