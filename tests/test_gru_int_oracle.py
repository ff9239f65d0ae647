"""Pin the oracle's int32-carrier GRU forward (oracle_gru_forward_int, oracle/gru_oracle.c).

* Codes: equal, code for code, to the reference's own CPU int32 carrier compiled from
  /root/reference into oracle/_ref (quantitativeWeightCPU + ForwardPassQuantCPU::Run,
  src/gru_host.cc:127-216, src/gru_forward_cpu_quant.cc:109-343): h, v (z, r, n, weight_hh_linear
  of n), W/R/bias and x codes, over every configuration axis, with and without h0, the int-IO
  form (codes in) included.  The reference's CUDA carrier (src/gru_forward_gpu_quant.cu) runs the
  same templates (quantize_ops_helper.h:683-1023), so this is also its arithmetic.
* Masks: the reference's CPU carrier keeps none, so the eleven mask families are pinned against
  an independent vectorised numpy restatement written from the CUDA source
  (quantizedGemmBiasFused :112-176, PointwiseOperationsQuant :230-373, the gate templates and
  clamp_by_bitwidth<true>), which takes every mask at its own clamp; configurations are chosen
  so that every family fires.
* Identities: the int-IO forward on the float forward's codes reproduces it; training and
  inference give the same codes.
"""
import numpy as np
import pytest

import gru_oracle as GO
import rxmet_gru_abi as A
from test_gru_oracle import (_RESTATEMENT_CASES, _configs, _gru_weights, _narrowed_case,
                             calibrated_params, to_haste)

f32, i64 = np.float32, np.int64
needs_ref = pytest.mark.skipif(not GO.has_ref(), reason="oracle/_ref not built (no reference checkout)")
KEYS = ("h_q", "v_q", "W_q", "R_q", "bw_q", "br_q", "x_q")


def _case(T, B, I, H, cfg, seed, with_h0=True):
    W, R, bw, br = to_haste(*_gru_weights(I, H, seed))
    g = np.random.default_rng(seed + 10)
    x = g.standard_normal((T, B, I)).astype(f32)
    h0 = (g.standard_normal((B, H)) * 0.5).astype(f32) if with_h0 else None
    qp, _ = calibrated_params(W, R, bw, br, x, cfg)
    return W, R, bw, br, x, h0, qp


@needs_ref
@pytest.mark.parametrize("name,cfg", _configs(), ids=[n for n, _ in _configs()])
@pytest.mark.parametrize("seed", [0, 1, 2])
@pytest.mark.parametrize("shape", [(7, 3, 5, 8), (12, 5, 9, 20), (4, 2, 3, 1)], ids=str)
def test_int_carrier_matches_reference_cpu_carrier(name, cfg, seed, shape):
    T, B, I, H = shape
    W, R, bw, br, x, h0, qp = _case(T, B, I, H, cfg, seed, with_h0=seed != 1)
    o = GO.forward_int(W, R, bw, br, x, qp, h0=h0)
    r = GO.ref_forward_int_codes(W, R, bw, br, x, qp, h0=h0)
    for k in KEYS:
        np.testing.assert_array_equal(o[k], r[k], err_msg=k)
    # the int-IO form, codes in: the reference carrier on the same codes
    ro = GO.ref_forward_int_codes(W, R, bw, br, None, qp, x_q=o["x_q"], h0_q=o["h_q"][0])
    oo = GO.forward_int(W, R, bw, br, None, qp, x_q=o["x_q"], h0_q=o["h_q"][0])
    for k in ("h_q", "v_q"):
        np.testing.assert_array_equal(oo[k], ro[k], err_msg=k)
        np.testing.assert_array_equal(oo[k], o[k], err_msg=k)


@needs_ref
@pytest.mark.parametrize("bits,pot2", [(8, False), (8, True), (16, False), (16, True)])
def test_int_carrier_matches_reference_on_arbitrary_codes(bits, pot2):
    """Int-IO codes anywhere on the x / h grids (not only codes a quantiser produces),
    grid ends included."""
    T, B, I, H = 6, 4, 7, 12
    cfg = A.set_all_bitwidth(A.default_config(), bits, False)
    cfg.use_pot2 = int(pot2)
    W, R, bw, br, x, h0, qp = _case(T, B, I, H, cfg, 7)
    g = np.random.default_rng(8)
    gx, gh = qp.g[A.GRID["x"]], qp.g[A.GRID["h"]]
    lo_x, hi_x = _lims(gx.bits, gx.is_unsigned)
    lo_h, hi_h = _lims(gh.bits, gh.is_unsigned)
    x_q = g.integers(lo_x, hi_x + 1, (T, B, I)).astype(np.int32)
    x_q[0, 0, :2] = (lo_x, hi_x)
    h0_q = g.integers(lo_h, hi_h + 1, (B, H)).astype(np.int32)
    h0_q[0, :2] = (lo_h, hi_h)
    o = GO.forward_int(W, R, bw, br, None, qp, x_q=x_q, h0_q=h0_q)
    r = GO.ref_forward_int_codes(W, R, bw, br, None, qp, x_q=x_q, h0_q=h0_q)
    for k in ("h_q", "v_q", "W_q", "R_q", "bw_q", "br_q"):
        np.testing.assert_array_equal(o[k], r[k], err_msg=k)


# ------------------------------------------------------------------------------------------
# An independent restatement of the reference's CUDA int32 carrier, vectorised in numpy int64.
# ------------------------------------------------------------------------------------------

def _lims(bits, uns):
    """QuantBitWidth::qmin / qmax (quantize_bitwidth_config.h:15-23)."""
    if bits >= 32:
        return -(1 << 31), (1 << 31) - 1
    return (0, (1 << bits) - 1) if uns else (-(1 << (bits - 1)), (1 << (bits - 1)) - 1)


def _rshift_round(x, n):
    """rshift_round (quantize_ops_helper.h:201-224), elementwise over int64 x and shifts n."""
    x = np.asarray(x, i64)
    n = np.broadcast_to(np.asarray(n, i64), x.shape)
    left = x << np.maximum(-n, 0)
    m = np.maximum(n, 1)
    ax = np.abs(x)
    q, r, half = ax >> m, ax & ((i64(1) << m) - 1), i64(1) << (m - 1)
    res = np.where(r > half, q + 1, np.where(r < half, q, q + (q & 1)))
    return np.where(n <= 0, left, np.where(x < 0, -res, res))


def _mshift(ratio):
    """encodeMShift (scale_encoding.h:87-106) of an fp32 ratio."""
    mant, e = np.frexp(np.float64(np.float32(ratio)))
    m = int(np.floor(mant * 65536.0 + 0.5))  # llround of a positive value
    if m == 65536:
        m, e = 32768, e + 1
    return max(m, 32768), 16 - int(e)


def _pot(scale):
    return int(np.round(-np.log2(np.float64(scale))))


def _rescale(x, pot, ratio, pshift):
    if pot:
        return _rshift_round(x, pshift)
    m, s = _mshift(ratio)
    return _rshift_round(np.asarray(x, i64) * m, s)


def _clamp(v, bits, uns):
    lo, hi = _lims(bits, uns)
    keep = ((v >= lo) & (v <= hi)).astype(np.uint8)
    return np.clip(v, lo, hi), keep


def _i32(v):
    return np.asarray(v, i64).astype(np.int32).astype(i64)


def _np_int_forward(W, R, bw, br, x, h0, qp):
    q = qp.g
    pot = bool(qp.use_pot2)
    G = lambda n: q[A.GRID[n]]
    T, B, I = x.shape
    H = R.shape[0]
    C = 3 * H
    out = {}

    def quant(v, scale, zp, bits, uns):
        eff = f32(GO.effective_scale(scale, pot))
        code = np.rint(np.asarray(v, f32) / eff).astype(np.float64) + zp
        lo, hi = _lims(bits, uns)
        keep = ((code >= lo) & (code <= hi)).astype(np.uint8)
        return np.clip(code, lo, hi).astype(i64), keep

    cs = [np.array(A.qparams_chan(qp, k), f32) for k in range(4)]
    for k, (name, src) in enumerate((("W", W), ("R", R), ("bw", bw), ("br", br))):
        codes = np.empty(src.shape, i64)
        keep = np.empty(src.shape, np.uint8)
        for c in range(C):
            codes[..., c], keep[..., c] = quant(src[..., c], cs[k][c], 0, qp.chan_bits[k],
                                                qp.chan_unsigned[k])
        out[name + "_q"], out[name + "_mask"] = codes, keep
    gx, gh = G("x"), G("h")
    out["x_q"], out["x_mask"] = quant(x, gx.scale, gx.zero_point, gx.bits, gx.is_unsigned)
    if h0 is not None:
        hq, out["h0_mask"] = quant(h0, gh.scale, gh.zero_point, gh.bits, gh.is_unsigned)
    else:
        hq = np.full((B, H), gh.zero_point, i64)
    s = lambda n: f32(G(n).scale)
    zp = lambda n: i64(G(n).zero_point)

    def lin(acc, bias_q, ksrc, kmat, sin, dst):
        # bias into the accumulator scale S_mat S_in, then GEMM + bias to the linear grid
        res = np.empty(acc.shape, i64)
        for c in range(C):
            sm, sb = cs[kmat][c], cs[ksrc][c]
            b = _rescale(bias_q[c], pot, f32(sb / f32(sm * sin)),
                         _pot(sb) - (_pot(sm) + _pot(sin)))
            res[..., c] = _rescale(acc[..., c] + b, pot, f32(f32(sm * sin) / s(dst)),
                                   _pot(sm) + _pot(sin) - _pot(s(dst)))
        return _clamp(_i32(_i32(res) + zp(dst)), G(dst).bits, G(dst).is_unsigned)

    xc = out["x_q"] - zp("x")
    wx, out["ih_mask"] = lin(np.einsum("tbi,ic->tbc", xc, out["W_q"]), out["bw_q"], 2, 0, s("x"),
                             "weight_ih_linear")
    luts = GO.make_luts(qp)

    def pwl(v, lut):
        thr = np.array([lut.seg[i].threshold for i in range(16)], i64)
        below = v[..., None] < thr
        seg = np.where(below.any(-1), below.argmax(-1), 15)
        qb = np.array([lut.seg[i].q_b for i in range(16)], i64)[seg]
        n = np.array([lut.seg[i].n for i in range(16)], i64)[seg]
        c = np.array([lut.seg[i].c for i in range(16)], i64)[seg]
        return _i32(_i32(_rshift_round(qb * _i32(v - lut.zp_x), n)) + c)

    def single(v, src, dst):
        return _i32(_rescale(v, pot, f32(s(src) / s(dst)), _pot(s(src)) - _pot(s(dst))))

    def prod(v, a, b, dst):
        return _i32(_rescale(v, pot, f32(f32(s(a) * s(b)) / s(dst)),
                             _pot(s(a)) + _pot(s(b)) - _pot(s(dst))))

    hs, vs = [hq], []
    for k in ("hh_mask", "gate_in_mask", "gate_out_mask", "h_mask"):
        out[k] = []
    for t in range(T):
        hc = hs[-1] - zp("h")
        rh, km = lin(hc @ out["R_q"], out["br_q"], 3, 1, s("h"), "weight_hh_linear")
        out["hh_mask"].append(km)
        gin, gout = np.empty((B, C), np.uint8), np.empty((B, C), np.uint8)
        w = wx[t] - zp("weight_ih_linear")
        r_ = rh - zp("weight_hh_linear")
        gates = []
        for gi, (gin_n, gout_n, lut) in enumerate((("update_gate_input", "update_gate_output", luts[0]),
                                                   ("reset_gate_input", "reset_gate_output", luts[1]))):
            sl = slice(gi * H, (gi + 1) * H)
            v = _i32(single(w[:, sl], "weight_ih_linear", gin_n) +
                     single(r_[:, sl], "weight_hh_linear", gin_n) + zp(gin_n))
            v, gin[:, sl] = _clamp(v, G(gin_n).bits, G(gin_n).is_unsigned)
            o, gout[:, sl] = _clamp(pwl(v, lut), G(gout_n).bits, G(gout_n).is_unsigned)
            gates.append(o)
        z, r = gates
        sl = slice(2 * H, 3 * H)
        rm = (r - zp("reset_gate_output")) * r_[:, sl]
        v = _i32(single(w[:, sl], "weight_ih_linear", "new_gate_input") +
                 prod(rm, "reset_gate_output", "weight_hh_linear", "new_gate_input") +
                 zp("new_gate_input"))
        v, gin[:, sl] = _clamp(v, G("new_gate_input").bits, G("new_gate_input").is_unsigned)
        n, gout[:, sl] = _clamp(pwl(v, luts[2]), G("new_gate_output").bits,
                                G("new_gate_output").is_unsigned)
        n_h = _i32(single(n - zp("new_gate_output"), "new_gate_output", "h") + zp("h"))
        one = _i32(i64(np.rint(f32(1) / s("update_gate_output"))) + zp("update_gate_output"))
        comb = (z - zp("update_gate_output")) * hc + (one - z) * (n_h - zp("h"))
        hn, hk = _clamp(_i32(prod(comb, "update_gate_output", "h", "h") + zp("h")),
                        G("h").bits, G("h").is_unsigned)
        hs.append(hn)
        vs.append(np.concatenate([z, r, n, rh[:, sl]], axis=1))
        out["gate_in_mask"].append(gin)
        out["gate_out_mask"].append(gout)
        out["h_mask"].append(hk)
    for k in ("hh_mask", "gate_in_mask", "gate_out_mask", "h_mask"):
        out[k] = np.stack(out[k])
    out["h_q"], out["v_q"] = np.stack(hs), np.stack(vs)
    return out


def _restated(case, with_h0):
    _, bits, h_bits, pot2, gran, h_unsigned, shrink, h_shrink = case
    T, B, I, H = 5, 6, 4, 8
    cfg = A.set_all_bitwidth(A.default_config(), bits, False)
    cfg.op[A.GRID["h"]].bits = h_bits
    cfg.op[A.GRID["h"]].is_unsigned = int(h_unsigned)
    cfg.use_pot2 = int(pot2)
    for k in range(4):
        cfg.chan[k].granularity = gran
    W, R, bw, br, x, h0, qp, _ = _narrowed_case(I, H, T, B, cfg, 31, shrink, h_shrink)
    h0 = h0 if with_h0 else None
    return GO.forward_int(W, R, bw, br, x, qp, h0=h0), _np_int_forward(W, R, bw, br, x, h0, qp)


@pytest.mark.parametrize("case", _RESTATEMENT_CASES, ids=[c[0] for c in _RESTATEMENT_CASES])
@pytest.mark.parametrize("with_h0", [False, True])
def test_int_carrier_matches_numpy_restatement(case, with_h0):
    """Every code and all eleven mask families of the oracle's int32 carrier equal a second
    implementation, on ranges narrowed so that the clamps fire."""
    o, e = _restated(case, with_h0)
    for k in KEYS:
        np.testing.assert_array_equal(o[k], e[k], err_msg=k)
    for k in GO.MASKS:
        if o[k] is None:
            assert k == "h0_mask" and not with_h0
            continue
        np.testing.assert_array_equal(o[k], e[k], err_msg=k)


def test_restatement_cases_fire_every_mask_family():
    fired = set()
    for case in _RESTATEMENT_CASES:
        o, _ = _restated(case, True)
        fired |= {k for k in GO.MASKS if o[k].min() == 0}
    assert fired == set(GO.MASKS), sorted(set(GO.MASKS) - fired)


def test_train_and_eval_codes_agree():
    T, B, I, H = 6, 4, 5, 16
    cfg = A.set_all_bitwidth(A.default_config(), 8, False)
    W, R, bw, br, x, h0, qp = _case(T, B, I, H, cfg, 4)
    a = GO.forward_int(W, R, bw, br, x, qp, h0=h0, training=True)
    b = GO.forward_int(W, R, bw, br, x, qp, h0=h0, training=False)
    for k in KEYS:
        np.testing.assert_array_equal(a[k], b[k], err_msg=k)
    assert all(b[k] is None for k in GO.MASKS)
