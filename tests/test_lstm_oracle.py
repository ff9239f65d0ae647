"""Pins of the QuantLSTM CPU oracle (oracle/lstm_oracle.c), CPU only.

* Golden vectors of the reference's own tests (tests/golden/lstm/*.json, copied data from
  operators/quant-lstm/tests/golden/spec): rounding, integer grids, quantise/dequantise
  boundaries, M+shift encodings, POT2 CoverRange, real-activation boundaries, one cell
  step and a 3-step recurrence of the CPU FP32 q-carrier reference.
* The reference compiled into oracle/_ref (skipped where the reference is absent):
  parameter finalisation, execution encodings, the q-carrier forward (codes and traces),
  the float forward and the calibration statistics — all bit-exact.
* Mathematics: the float forward against torch.nn.LSTM, the STE backward against torch
  autograd through a surrogate with gradient stoppers at every clamped point, and the
  oracle backward (masks off) against the reference's float CPU backward.
"""
import ctypes
import json
from pathlib import Path

import numpy as np
import pytest
import torch

import lstm_oracle as O
import rxmet_lstm_abi as L

GOLD = Path(__file__).resolve().parent / "golden" / "lstm"
f32 = np.float32
needs_ref = pytest.mark.skipif(not O.has_ref(), reason="reference checkout not present")


def _load(name):
    return json.loads((GOLD / name).read_text())


def _arr(entry):
    dt = entry["dtype"]
    data = entry["data"]
    if dt.startswith("float"):
        return np.array([float(v) for v in data], dtype=np.float64 if dt == "float64" else f32)
    if dt == "bool":
        return np.array(data, dtype=bool)
    if dt == "string":
        return list(data)
    return np.array(data, dtype=np.int64)


def _opcfg(bits, uns, sym, gran=L.PER_TENSOR):
    return L.OpConfig(int(bits), int(bool(uns)), int(bool(sym)), gran)


# --------------------------------------------------------------------------------------
# primitive golden vectors
# --------------------------------------------------------------------------------------


def test_golden_round_half_ties():
    d = _load("round_half_ties.json")
    vals = _arr(d["inputs"]["values"])
    exp = _arr(d["expected"]["checkpoints"]["rounded"])
    assert [O.prim.olstm_prim_rne(float(v)) for v in vals] == list(exp)


def test_golden_quantized_ranges():
    d = _load("quantized_ranges.json")
    i = d["inputs"]
    for b, u, s, lo, hi in zip(_arr(i["bitwidth"]), _arr(i["is_unsigned"]), _arr(i["is_symmetric"]),
                               _arr(d["expected"]["checkpoints"]["minimum"]),
                               _arr(d["expected"]["checkpoints"]["maximum"])):
        a, c = ctypes.c_int32(), ctypes.c_int32()
        O.prim.olstm_prim_range(ctypes.byref(_opcfg(b, u, s)), ctypes.byref(a), ctypes.byref(c))
        assert (a.value, c.value) == (lo, hi)


def test_golden_quantize_and_dequantize_boundaries():
    d = _load("quant_dequant_boundaries.json")
    i = d["inputs"]
    for v, s, z, b, u, sym, e in zip(_arr(i["value"]), _arr(i["scale"]), _arr(i["zero_point"]),
                                     _arr(i["bitwidth"]), _arr(i["is_unsigned"]),
                                     _arr(i["is_symmetric"]),
                                     _arr(d["expected"]["checkpoints"]["quantized"])):
        assert O.prim.olstm_prim_quantize(float(v), float(s), int(z),
                                          ctypes.byref(_opcfg(b, u, sym))) == e
    d = _load("dequantize_boundaries.json")
    i = d["inputs"]
    for q, s, z, e in zip(_arr(i["value"]), _arr(i["scale"]), _arr(i["zero_point"]),
                          _arr(d["expected"]["checkpoints"]["real"])):
        assert O.prim.olstm_prim_dequantize(float(q), float(s), int(z)) == e


def test_golden_m_shift_known_vectors():
    d = _load("m_shift_known_vectors.json")
    i, e = d["inputs"], d["expected"]["checkpoints"]
    for ratio, v, m, s, fp in zip(_arr(i["ratio"]), _arr(i["value"]), _arr(e["multiplier"]),
                                  _arr(e["shift"]), _arr(e["fp_apply"])):
        r = L.Rescale()
        assert O.prim.olstm_prim_mshift(float(ratio), ctypes.byref(r)) == 0
        assert (r.multiplier, r.shift) == (m, s)
        assert O.prim.olstm_prim_apply(float(v), ctypes.byref(r)) == fp


def test_golden_pot2_cover_range():
    d = _load("pot2_cover_range.json")
    i, e = d["inputs"], d["expected"]["checkpoints"]
    for mn, mx, b, u, s, es, ez in zip(_arr(i["range_minimum"]), _arr(i["range_maximum"]),
                                       _arr(i["bitwidth"]), _arr(i["is_unsigned"]),
                                       _arr(i["is_symmetric"]), _arr(e["scale"]),
                                       _arr(e["zero_point"])):
        sc, zp = ctypes.c_float(), ctypes.c_int32()
        assert O.prim.olstm_prim_calibrate(float(mn), float(mx), ctypes.byref(_opcfg(b, u, s)), 1,
                                           0, ctypes.byref(sc), ctypes.byref(zp)) == 0
        assert (f32(sc.value), zp.value) == (es, ez)


@pytest.mark.parametrize("name", ["real_activation_boundaries.json",
                                  "real_activation_boundaries_cpu_fp32.json"])
@pytest.mark.parametrize("mode", [O.ACT_LIBM, O.ACT_CR])
def test_golden_real_activation(name, mode):
    d = _load(name)
    i = d["inputs"]
    exp = _arr(d["expected"]["checkpoints"]["quantized"])
    for k, (kind, q, si, zi, so, zo) in enumerate(zip(
            _arr(i["kind"]), _arr(i["quantized"]), _arr(i["input_scale"]),
            _arr(i["input_zero_point"]), _arr(i["output_scale"]), _arr(i["output_zero_point"]))):
        out_cfg = _opcfg(8, kind == "sigmoid", True)
        v, _ = O.real_activation(q, si, zi, so, zo, out_cfg, kind == "tanh", mode)
        assert v == exp[k], (kind, q)


# --------------------------------------------------------------------------------------
# cell and recurrent golden cases (execution_model cpu_fp32)
# --------------------------------------------------------------------------------------


def _golden_case(name):
    d = _load(name)
    i = d["inputs"]
    T, B, I, H = (int(v) for v in _arr(i["shape"]))
    C = 4 * H
    cfg = L.Config()
    cfg.scale_mode = L.POT2 if i["scale_mode"]["data"][0] == "pot2" else L.AFFINE
    for k, (b, u, s, g) in enumerate(zip(_arr(i["operator_bitwidth"]), _arr(i["operator_is_unsigned"]),
                                         _arr(i["operator_is_symmetric"]),
                                         _arr(i["operator_granularity"]))):
        cfg.op[k] = _opcfg(b, u, s, L.GRANULARITY[g])
    bias = bool(_arr(i["bias_enabled"])[0])
    p = L.new_params(H)
    p.bias_enabled = int(bias)
    p.config = cfg
    scales = _arr(i["quant_param_scales"])
    zps = _arr(i["quant_param_zero_points"])
    off = _arr(i["quant_param_value_offsets"])
    for k, name_ in enumerate(L.OP_NAMES):
        vs, zs = scales[off[k]:off[k + 1]], zps[off[k]:off[k + 1]]
        if name_ in L.PARAM_OPS:
            if len(vs):
                L.chan_scales(p, L.PARAM_OPS.index(name_))[:] = np.repeat(vs, C // len(vs))
        else:
            p.scale[k] = float(vs[0])
            p.zero_point[k] = int(zs[0])

    def deq(key, op, per_channel=False):
        q = _arr(i[key]).reshape(i[key]["shape"]).astype(np.float64)
        if per_channel:
            s = L.chan_scales(p, L.PARAM_OPS.index(op)).astype(np.float64)
            return (q * s.reshape(-1, *([1] * (q.ndim - 1)))).astype(f32)
        return ((q - p.zero_point[L.OP[op]]) * float(p.scale[L.OP[op]])).astype(f32)

    x = deq("input", "input")
    Wi = deq("weight_ih", "weight_ih", True)
    Wh = deq("weight_hh", "weight_hh", True)
    bi = deq("bias_ih", "bias_ih", True) if bias else None
    bh = deq("bias_hh", "bias_hh", True) if bias else None
    h0 = deq("initial_hidden", "output")
    c0 = deq("initial_cell", "cell_state")
    return d, (T, B, I, H), p, (Wi, Wh, bi, bh, x, h0, c0)


@pytest.mark.parametrize("name", ["reference_cell_t1_b1_i2_h2_cpu_fp32.json",
                                  "reference_recurrent_t3_b1_i2_h2_cpu_fp32.json"])
def test_golden_cell_and_recurrence(name):
    d, (T, B, I, H), p, (Wi, Wh, bi, bh, x, h0, c0) = _golden_case(name)
    o = O.forward_quant(Wi, Wh, bi, bh, x, p, h0, c0, mode=O.ACT_LIBM, traces=True)
    exp = d["expected"]["checkpoints"]

    def ex(key):
        return _arr(exp[key]).reshape(exp[key]["shape"])

    assert np.array_equal(o["hidden"], ex("output").astype(f32))
    assert np.array_equal(o["cell"], ex("cell").astype(f32))
    assert np.array_equal(o["cell_tanh"], ex("cell_tanh").astype(f32))
    C = 4 * H
    for g, gname in enumerate(("input", "forget", "cell", "output")):
        sl = slice(g * H, (g + 1) * H)
        assert np.array_equal(o["gate_in"][..., sl], ex(f"{gname}_gate_input").astype(f32)), gname
        assert np.array_equal(o["gate_out"][..., sl], ex(f"{gname}_gate_output").astype(f32)), gname
    assert np.array_equal(o["ih_linear"].reshape(T, B, 4, H), ex("weight_ih_linear").astype(f32))
    assert np.array_equal(o["hh_linear"].reshape(T, B, 4, H), ex("weight_hh_linear").astype(f32))
    zh, sh = p.zero_point[L.OP["output"]], p.scale[L.OP["output"]]
    zc, sc = p.zero_point[L.OP["cell_state"]], p.scale[L.OP["cell_state"]]
    assert np.array_equal(o["h_n"], ((ex("h_n") - zh) * np.float64(sh)).astype(f32))
    assert np.array_equal(o["c_n"], ((ex("c_n") - zc) * np.float64(sc)).astype(f32))
    assert C == o["gate_out"].shape[-1]


# --------------------------------------------------------------------------------------
# random cases against the compiled reference
# --------------------------------------------------------------------------------------


def _weights(I, H, seed, bias=True, amp=None):
    g = np.random.default_rng(seed)
    k = amp if amp is not None else 1.0 / np.sqrt(H)
    u = lambda *s: ((g.random(s) * 2 - 1) * k).astype(f32)
    return u(4 * H, I), u(4 * H, H), (u(4 * H) if bias else None), (u(4 * H) if bias else None)


def _config(name):
    c = L.default_config()
    if name == "default":
        return c
    if name == "c4":  # 8-bit weights per channel, 8-bit gates, 16-bit cell, 8-bit h, affine
        for k in range(L.NOPS):
            if L.OP_NAMES[k] not in L.PARAM_OPS:
                c.op[k].is_symmetric = 0
        c.op[L.OP["cell_state"]].bits = 16
        return c
    if name == "pot2-gate":
        c.scale_mode = L.POT2
        for n in L.PARAM_OPS:
            c.op[L.OP[n]].granularity = L.PER_GATE
        c.op[L.OP["output"]].is_symmetric = 0
        return c
    if name == "16b-tensor":
        for k in range(L.NOPS):
            c.op[k].bits = 16
            if L.OP_NAMES[k] in L.PARAM_OPS:
                c.op[k].granularity = L.PER_TENSOR
        return c
    raise KeyError(name)


CONFIGS = ["default", "c4", "pot2-gate", "16b-tensor"]


def _calibrated(T, B, I, H, cfg_name, seed, bias=True, with_state=False):
    Wi, Wh, bi, bh = _weights(I, H, seed, bias)
    g = np.random.default_rng(seed + 1)
    x = (g.random((T, B, I)) * 2 - 1).astype(f32)
    h0 = c0 = None
    if with_state:
        h0 = (g.standard_normal((B, H)) * 0.3).astype(f32)
        c0 = (g.standard_normal((B, H)) * 0.5).astype(f32)
    stats = O.calibrate(Wi, Wh, bi, bh, x, h0, c0)
    cfg = _config(cfg_name)
    p = O.finalize(stats, cfg, H, bias)
    return (Wi, Wh, bi, bh, x, h0, c0), stats, cfg, p


@needs_ref
@pytest.mark.parametrize("cfg_name", CONFIGS)
@pytest.mark.parametrize("bias", [True, False])
def test_finalize_and_exec_match_reference(cfg_name, bias):
    (Wi, Wh, bi, bh, x, h0, c0), stats, cfg, p = _calibrated(4, 3, 5, 6, cfg_name, 3, bias, True)
    r = O.finalize(stats, cfg, 6, bias, ref=True)
    assert list(p.scale) == list(r.scale) and list(p.zero_point) == list(r.zero_point)
    for k in range(4):
        if k >= 2 and not bias:
            continue
        assert np.array_equal(L.chan_scales(p, k), L.chan_scales(r, k)), k
    assert O.derive_exec(p, 5) == O.derive_exec(r, 5, ref=True)


@needs_ref
def test_calibration_stats_match_reference():
    Wi, Wh, bi, bh = _weights(7, 8, 5)
    g = np.random.default_rng(9)
    s1 = O.calibrate(Wi, Wh, bi, bh, (g.random((5, 4, 7)) * 2 - 1).astype(f32))
    r1 = O.calibrate(Wi, Wh, bi, bh, (np.random.default_rng(9).random((5, 4, 7)) * 2 - 1).astype(f32),
                     ref=True)
    assert np.array_equal(s1, r1)
    h0 = (g.standard_normal((4, 8)) * 0.4).astype(f32)
    c0 = (g.standard_normal((4, 8))).astype(f32)
    x2 = (g.standard_normal((3, 4, 7)) * 2).astype(f32)
    s2 = O.calibrate(Wi, Wh, bi, bh, x2, h0, c0, stats=s1.copy())
    r2 = O.calibrate(Wi, Wh, bi, bh, x2, h0, c0, stats=r1.copy(), ref=True)
    assert np.array_equal(s2, r2)


@needs_ref
@pytest.mark.parametrize("cfg_name", CONFIGS)
@pytest.mark.parametrize("with_state", [False, True])
def test_quantized_forward_matches_reference(cfg_name, with_state):
    T, B, I, H = 6, 3, 5, 8
    (Wi, Wh, bi, bh, x, h0, c0), _, _, p = _calibrated(T, B, I, H, cfg_name, 11, True, with_state)
    o = O.forward_quant(Wi, Wh, bi, bh, x, p, h0, c0, mode=O.ACT_LIBM, traces=True)
    r = O.ref_forward_fp(Wi, Wh, bi, bh, x, p, h0, c0)
    assert np.array_equal(o["hidden"], r["output"])
    for k in ("ih_linear", "hh_linear", "gate_in"):
        assert np.array_equal(o[k], r[k]), k
    for k in ("gate_out", "cell", "cell_tanh"):
        assert np.array_equal(o[k], r[k]), k
    zh, sh = p.zero_point[L.OP["output"]], np.float64(p.scale[L.OP["output"]])
    assert np.array_equal(o["h_n"], ((r["h_n"].astype(np.float64) - zh) * sh).astype(f32))


@needs_ref
def test_float_forward_matches_reference():
    Wi, Wh, bi, bh = _weights(6, 10, 13)
    g = np.random.default_rng(14)
    x = g.standard_normal((7, 4, 6)).astype(f32)
    h0 = (g.standard_normal((4, 10)) * 0.3).astype(f32)
    c0 = g.standard_normal((4, 10)).astype(f32)
    for args in ((None, None), (h0, c0)):
        a = O.forward_float(Wi, Wh, bi, bh, x, *args)
        b = O.forward_float(Wi, Wh, bi, bh, x, *args, ref=True)
        for u, v in zip(a, b):
            assert np.array_equal(u, v)


def test_float_forward_matches_torch_lstm():
    I, H = 5, 7
    Wi, Wh, bi, bh = _weights(I, H, 17)
    x = np.random.default_rng(18).standard_normal((6, 3, I)).astype(f32)
    ref = torch.nn.LSTM(I, H)
    with torch.no_grad():
        for n, v in (("weight_ih_l0", Wi), ("weight_hh_l0", Wh), ("bias_ih_l0", bi),
                     ("bias_hh_l0", bh)):
            getattr(ref, n).copy_(torch.from_numpy(v))
        y, (hn, cn) = ref(torch.from_numpy(x))
    for mode in (O.ACT_LIBM, O.ACT_CR):
        out, h, c = O.forward_float(Wi, Wh, bi, bh, x, mode=mode)
        np.testing.assert_allclose(out, y.numpy(), atol=2e-6)
        np.testing.assert_allclose(c, cn[0].numpy(), atol=2e-6)


@pytest.mark.parametrize("cfg_name", ["default", "c4"])
def test_cr_activation_rarely_differs_from_libm(cfg_name):
    # The GPU implements ACT_CR; the reference CPU uses the C library's expf/tanhf.  Step by
    # step the two differ only where an activation lands within an ulp of a rounding
    # boundary of its output grid.
    T, B, I, H = 1, 64, 8, 32
    (Wi, Wh, bi, bh, x, h0, c0), _, _, p = _calibrated(T, B, I, H, cfg_name, 21, True, True)
    a = O.forward_quant(Wi, Wh, bi, bh, x, p, h0, c0, mode=O.ACT_LIBM)
    b = O.forward_quant(Wi, Wh, bi, bh, x, p, h0, c0, mode=O.ACT_CR)
    for k in ("gate_out", "cell_tanh", "hidden"):
        d = np.abs(a[k] - b[k])
        assert d.max() <= 1 and (d > 0).mean() <= 1e-3, (k, d.max(), (d > 0).mean())


def test_codes_integral_and_masks_binary():
    (Wi, Wh, bi, bh, x, h0, c0), _, _, p = _calibrated(5, 4, 6, 8, "c4", 23, True, True)
    o = O.forward_quant(Wi, Wh, bi, bh, x * 3, p, h0, c0)
    for k in ("x_q", "w_ih_q", "w_hh_q", "b_ih_q", "gate_out", "cell", "cell_tanh", "hidden"):
        assert np.array_equal(o[k], np.rint(o[k])), k
    for k in L.SAVED_FIELDS:
        if k.endswith("_m"):
            assert set(np.unique(o[k])) <= {0, 1}, k
    assert o["x_m"].any(), "inputs scaled x3 beyond the calibrated range must clamp"


# --------------------------------------------------------------------------------------
# backward
# --------------------------------------------------------------------------------------


@needs_ref
def test_backward_without_masks_matches_reference_float_backward():
    T, B, I, H = 5, 3, 4, 6
    (Wi, Wh, bi, bh, x, h0, c0), _, _, p = _calibrated(T, B, I, H, "c4", 31, True, True)
    f = O.forward_quant(Wi, Wh, bi, bh, x, p, h0, c0)
    for k in L.SAVED_FIELDS:
        if k.endswith("_m") and f.get(k) is not None:
            f[k][...] = 0
    g = np.random.default_rng(32)
    go = (g.standard_normal((T, B, H)) * 0.1).astype(f32)
    gh = (g.standard_normal((B, H)) * 0.1).astype(f32)
    gc = (g.standard_normal((B, H)) * 0.1).astype(f32)
    ours = O.backward_quant(f, p, go, gh, gc)

    def deq(q, op):
        return ((q.astype(np.float64) - p.zero_point[L.OP[op]]) * np.float64(p.scale[L.OP[op]])).astype(f32)

    C = 4 * H
    gates = np.concatenate([deq(f["gate_out"][..., k * H:(k + 1) * H], n) for k, n in enumerate(
        ("input_gate_output", "forget_gate_output", "cell_gate_output", "output_gate_output"))], -1)
    wi = (f["w_ih_q"] * L.chan_scales(p, 0)[:, None]).astype(f32)
    wh = (f["w_hh_q"] * L.chan_scales(p, 1)[:, None]).astype(f32)
    ref = O.ref_backward_float(wi, wh, deq(f["x_q"], "input"), deq(f["h0_q"], "output"),
                               deq(f["c0_q"], "cell_state"), gates, deq(f["cell"], "cell_state"),
                               deq(f["cell_tanh"], "cell_tanh_output"), deq(f["hidden"], "output"),
                               go, gh, gc)
    for k in ("dx", "dW_ih", "dW_hh", "db_ih", "db_hh", "dh0", "dc0"):
        scale = max(float(np.abs(ref[k]).max()), 1e-30)
        np.testing.assert_allclose(ours[k], ref[k], rtol=1e-4, atol=1e-5 * scale, err_msg=k)
    assert C == f["gate_out"].shape[-1]


def _surrogate_grads(f, p, T, B, I, H, go, gh, gc):
    """torch autograd through the float LSTM step built from the saved dequantised values,
    with every clamped point turned into a gradient stopper (STE, mask 1 = clamped)."""
    dt = torch.float64

    def deq(q, op):
        return torch.tensor((q.astype(np.float64) - p.zero_point[L.OP[op]]) * np.float64(p.scale[L.OP[op]]), dtype=dt)

    def keep(m):
        return torch.tensor(1.0 - m.astype(np.float64), dtype=dt)

    def ste(v, m):  # value unchanged, gradient zero where m == 1
        k = keep(m)
        return v * k + (v * (1 - k)).detach()

    wi = torch.tensor(f["w_ih_q"] * L.chan_scales(p, 0)[:, None].astype(np.float64), dtype=dt, requires_grad=True)
    wh = torch.tensor(f["w_hh_q"] * L.chan_scales(p, 1)[:, None].astype(np.float64), dtype=dt, requires_grad=True)
    bi = torch.zeros(4 * H, dtype=dt, requires_grad=True)
    bh = torch.zeros(4 * H, dtype=dt, requires_grad=True)
    x = deq(f["x_q"], "input").requires_grad_()
    h0 = deq(f["h0_q"], "output").requires_grad_()
    c0 = deq(f["c0_q"], "cell_state").requires_grad_()
    gate_ops = ("input_gate_output", "forget_gate_output", "cell_gate_output", "output_gate_output")
    h, c = ste(h0, f["h0_m"]), ste(c0, f["c0_m"])
    xs = ste(x, f["x_m"])
    wis, whs = ste(wi, f["w_ih_m"]), ste(wh, f["w_hh_m"])
    loss = 0
    for t in range(T):
        li = ste(xs[t] @ wis.T + bi, f["ih_linear_m"][t])
        lh = ste(h @ whs.T + bh, f["hh_linear_m"][t])
        pre = ste(li + lh, f["gate_in_m"][t])
        # the saved (quantised) activations stand in for the exact ones; gradients flow
        # through the analytic derivative evaluated at them
        outs = []
        for g in range(4):
            sl = slice(g * H, (g + 1) * H)
            a = deq(f["gate_out"][t][..., sl], gate_ops[g])
            der = (1 - a * a) if g == 2 else a * (1 - a)
            z = pre[..., sl]
            outs.append(ste(a + der * (z - z.detach()), f["gate_out_m"][t][..., sl]))
        i_, f_, g_, o_ = outs
        cq = deq(f["cell"][t], "cell_state")
        cn = f_ * c + i_ * g_
        cn = ste(cq + (cn - cn.detach()), f["cell_m"][t])
        tq = deq(f["cell_tanh"][t], "cell_tanh_output")
        ct = ste(tq + (1 - tq * tq) * (cn - cn.detach()), f["cell_tanh_m"][t])
        hq = deq(f["hidden"][t], "output")
        hv = o_ * ct
        h = ste(hq + (hv - hv.detach()), f["hidden_m"][t])
        c = cn
        loss = loss + (h * torch.tensor(go[t], dtype=dt)).sum()
    loss = loss + (h * torch.tensor(gh, dtype=dt)).sum() + (c * torch.tensor(gc, dtype=dt)).sum()
    loss.backward()
    return {"dx": x.grad, "dW_ih": wi.grad, "dW_hh": wh.grad, "db_ih": bi.grad, "db_hh": bh.grad,
            "dh0": h0.grad, "dc0": c0.grad}


@pytest.mark.parametrize("cfg_name", ["default", "c4"])
@pytest.mark.parametrize("seed", [41, 42])
def test_backward_matches_autograd_surrogate(cfg_name, seed):
    T, B, I, H = 4, 3, 5, 6
    (Wi, Wh, bi, bh, x, h0, c0), _, _, p = _calibrated(T, B, I, H, cfg_name, seed, True, True)
    # scaled inputs and weights push values past the calibrated ranges so masks are active
    f = O.forward_quant(Wi * 1.5, Wh * 1.5, bi, bh, x * 2.5, p, h0 * 2, c0 * 2)
    assert f["x_m"].any() and f["hidden_m"].any() + f["gate_in_m"].any() + f["cell_m"].any()
    g = np.random.default_rng(seed + 100)
    go = (g.standard_normal((T, B, H)) * 0.1).astype(f32)
    gh = (g.standard_normal((B, H)) * 0.1).astype(f32)
    gc = (g.standard_normal((B, H)) * 0.1).astype(f32)
    ours = O.backward_quant(f, p, go, gh, gc)
    exp = _surrogate_grads(f, p, T, B, I, H, go, gh, gc)
    for k in ("dx", "dW_ih", "dW_hh", "db_ih", "db_hh", "dh0", "dc0"):
        e = exp[k].numpy()
        if k in ("dW_ih", "dW_hh"):
            e = e * (1 - f["w_ih_m" if k == "dW_ih" else "w_hh_m"])
        if k in ("db_ih", "db_hh"):
            e = e * (1 - f["b_ih_m" if k == "db_ih" else "b_hh_m"])
        scale = max(float(np.abs(e).max()), 1e-30)
        np.testing.assert_allclose(ours[k], e, rtol=1e-4, atol=1e-5 * scale, err_msg=k)


def test_cr_mode_sums_are_order_free():
    """ACT_CR sums each linear exactly, so relabelling the hidden units (a permutation of the
    recurrent sum's order) only permutes the outputs, even where float partial sums would
    pass 2^24 (16-bit h and weights)."""
    T, B, I, H = 4, 3, 5, 32
    (Wi, Wh, bi, bh, x, h0, c0), _, _, p = _calibrated(T, B, I, H, "16b-tensor", 51, True, True)
    perm = np.random.default_rng(52).permutation(H)
    rows = np.concatenate([g * H + perm for g in range(4)])
    o = O.forward_quant(Wi, Wh, bi, bh, x, p, h0, c0, mode=O.ACT_CR)
    q = O.forward_quant(Wi[rows], Wh[rows][:, perm], bi[rows], bh[rows], x, p, h0[:, perm],
                        c0[:, perm], mode=O.ACT_CR)
    assert np.array_equal(q["output"], o["output"][..., perm])
    assert np.array_equal(q["c_n"], o["c_n"][:, perm])
    assert np.array_equal(q["gate_out"], o["gate_out"][..., rows])
    # the float-order (reference CPU) sum really does pass 2^24 here
    hc = o["hidden"] - p.zero_point[L.OP["output"]]
    wq = o["w_hh_q"]
    assert np.abs(hc[0] @ wq.T.astype(np.float64)).max() > 2 ** 24 or \
        np.abs(np.cumsum(hc[0][:, None, :] * wq[None], axis=-1)).max() > 2 ** 24


# --------------------------------------------------------------------------------------
# masks: an independent restatement of the q-carrier forward that takes each mask at its
# own clamp
# --------------------------------------------------------------------------------------


def _np_qcarrier(Wi, Wh, bi, bh, x, h0, c0, p, ex, mode):
    """The reference's FP32 q-carrier forward restated in numpy from its CPU source:
    masters (quantizeFp: RNE(double(v) / double(s)) + zp, clamped), linearValue
    (forward_quantized_fp_cpu.cc:18-44, exact centred sums as the GPU-semantics mode),
    gate inputs (:116-129), the cell and hidden cores (quantized_cell_fp.h:74-141) and the
    rescale cores (float_carrier_ops.h:81-90); the activation is the oracle's single-value
    realActivation (pinned by the reference's golden boundary vectors).  Each mask is taken
    where its value is clamped: 1 = clamped (the CUDA kernels' convention)."""
    T, B, I = x.shape
    H = Wh.shape[1]
    C = 4 * H
    cfg = p.config
    op = lambda n: cfg.op[L.OP[n]]

    def grid(n):
        o = op(n)
        if o.is_unsigned:
            return 0.0, float(2 ** o.bits - 1)
        return float(-2 ** (o.bits - 1)), float(2 ** (o.bits - 1) - 1)

    def clampm(v, n):
        lo, hi = grid(n)
        v = np.asarray(v, np.float64)
        return np.clip(v, lo, hi).astype(f32), ((v < lo) | (v > hi)).astype(np.uint8)

    S = lambda n: p.scale[L.OP[n]]
    Z = lambda n: p.zero_point[L.OP[n]]

    def master(v, s, zp, n):
        return clampm(np.rint(np.asarray(v, np.float64) / np.float64(s)) + zp, n)

    def R(v, enc):
        is_m, mult, sh = enc
        v = np.asarray(v, f32)
        if is_m:
            v = (v * f32(mult)).astype(f32)
        return np.rint(np.ldexp(v, -sh).astype(f32)).astype(f32)

    cs = lambda k: L.chan_scales(p, k)
    xq, xm = master(x, S("input"), Z("input"), "input")
    wiq, wim = master(Wi, cs(0)[:, None], 0, "weight_ih")
    whq, whm = master(Wh, cs(1)[:, None], 0, "weight_hh")
    biq = bim = bhq = bhm = None
    if bi is not None:
        biq, bim = master(bi, cs(2), 0, "bias_ih")
        bhq, bhm = master(bh, cs(3), 0, "bias_hh")
    hq, h0m = master(np.zeros((B, H), f32) if h0 is None else h0, S("output"), Z("output"), "output")
    cq, c0m = master(np.zeros((B, H), f32) if c0 is None else c0, S("cell_state"), Z("cell_state"),
                     "cell_state")
    acc_enc = [ex["acc_to_linear"][:C], ex["acc_to_linear"][C:]]
    bias_enc = None if bi is None else [ex["bias_to_acc"][:C], ex["bias_to_acc"][C:]]

    def linear(v, vzp, w, b, l, out):
        acc = ((v.astype(np.float64) - vzp) @ w.astype(np.float64).T).astype(f32)
        if b is not None:
            acc = (acc + np.array([R(b[c], bias_enc[l][c]) for c in range(C)], f32)).astype(f32)
        r = np.stack([R(acc[:, c], acc_enc[l][c]) for c in range(C)], -1)
        return clampm(r.astype(np.float64) + Z(out), out)

    act_cache = {}

    def act(q, inp, out, tanh):
        key = (inp, out)
        tab = act_cache.setdefault(key, {})
        vals = np.empty(q.shape, f32)
        msk = np.empty(q.shape, np.uint8)
        for i, v in np.ndenumerate(q):
            if v not in tab:
                tab[v] = O.real_activation(v, S(inp), Z(inp), S(out), Z(out), op(out), tanh, mode)
            vals[i], msk[i] = tab[v][0], tab[v][1]
        return vals, msk

    def q31(v, enc):
        mult, mant, expo, uses_fp = enc
        if uses_fp:
            return np.ldexp(v.astype(np.float64) * mant, expo).astype(f32)
        return (v * np.ldexp(f32(mult), -31).astype(f32)).astype(f32)

    gates = ("input_gate", "forget_gate", "cell_gate", "output_gate")
    rec = {k: [] for k in ("ih_linear_m", "hh_linear_m", "gate_in_m", "gate_out_m", "cell_m",
                           "cell_tanh_m", "hidden_m", "gate_out", "cell", "cell_tanh", "hidden")}
    for t in range(T):
        li, mli = linear(xq[t], Z("input"), wiq, biq, 0, "weight_ih_linear")
        lh, mlh = linear(hq, Z("output"), whq, bhq, 1, "weight_hh_linear")
        gin, gout, mgi, mgo = [], [], [], []
        for gi, gname in enumerate(gates):
            sl = slice(gi * H, (gi + 1) * H)
            lhs = R(li[:, sl] - f32(Z("weight_ih_linear")), ex["linear_to_gate"][gi])
            rhs = R(lh[:, sl] - f32(Z("weight_hh_linear")), ex["linear_to_gate"][4 + gi])
            q, m = clampm((lhs + rhs).astype(f32).astype(np.float64) + Z(gname + "_input"),
                          gname + "_input")
            a, am = act(q, gname + "_input", gname + "_output", gi == 2)
            gin.append(q); mgi.append(m); gout.append(a); mgo.append(am)
        cen = lambda v, n: (np.asarray(v, np.float64) - Z(n)).astype(f32)
        pf = (cen(gout[1], "forget_gate_output") * cen(cq, "cell_state")).astype(f32)
        pi = (cen(gout[0], "input_gate_output") * cen(gout[2], "cell_gate_output")).astype(f32)
        pre = (q31(pf, ex["cell"][0]) + q31(pi, ex["cell"][1])).astype(f32)
        cq, mc = clampm(np.rint(pre).astype(np.float64) + Z("cell_state"), "cell_state")
        tq, mt = act(cq, "cell_state", "cell_tanh_output", True)
        raw = (cen(gout[3], "output_gate_output") * cen(tq, "cell_tanh_output")).astype(f32)
        hq, mh = clampm(R(raw, ex["hidden"][0]).astype(np.float64) + Z("output"), "output")
        for k, v in (("ih_linear_m", mli), ("hh_linear_m", mlh),
                     ("gate_in_m", np.concatenate(mgi, -1)), ("gate_out_m", np.concatenate(mgo, -1)),
                     ("cell_m", mc), ("cell_tanh_m", mt), ("hidden_m", mh),
                     ("gate_out", np.concatenate(gout, -1)), ("cell", cq), ("cell_tanh", tq),
                     ("hidden", hq)):
            rec[k].append(v)
    out = {k: np.stack(v) for k, v in rec.items()}
    out.update({"x_q": xq, "x_m": xm, "w_ih_q": wiq, "w_ih_m": wim, "w_hh_q": whq, "w_hh_m": whm,
                "b_ih_q": biq, "b_ih_m": bim, "b_hh_q": bhq, "b_hh_m": bhm, "h0_m": h0m,
                "c0_m": c0m})
    return out


_LSTM_MASKS = ("x_m", "w_ih_m", "w_hh_m", "b_ih_m", "b_hh_m", "h0_m", "c0_m", "ih_linear_m",
               "hh_linear_m", "gate_in_m", "gate_out_m", "cell_m", "cell_tanh_m", "hidden_m")


def _narrow_lstm(T, B, I, H, cfg_name, seed, shrink, cell_shrink=1.0):
    (Wi, Wh, bi, bh, x, h0, c0), stats, cfg, _ = _calibrated(T, B, I, H, cfg_name, seed, True, True)
    n = L.NOPS
    stats[:n] *= shrink
    stats[n:2 * n] *= shrink
    stats[L.OP["cell_state"]] *= cell_shrink
    stats[n + L.OP["cell_state"]] *= cell_shrink
    stats[2 * n:2 * n + 8 * 4 * H] *= shrink
    return (Wi, Wh, bi, bh, x, h0 * 2, c0 * 2), O.finalize(stats, cfg, H, True)


@pytest.mark.parametrize("cfg_name", CONFIGS)
@pytest.mark.parametrize("mode", [O.ACT_LIBM, O.ACT_CR])
@pytest.mark.parametrize("cell_shrink", [1.0, 0.05])
def test_masks_equal_independent_restatement(cfg_name, mode, cell_shrink):
    """The oracle's codes and all fourteen mask families (masters, linear, gate input/output,
    cell, cell tanh, hidden) equal an independent restatement that takes each mask at its own
    clamp; ranges are narrowed so that clamps fire."""
    T, B, I, H = 4, 3, 5, 8
    (Wi, Wh, bi, bh, x, h0, c0), p = _narrow_lstm(T, B, I, H, cfg_name, 17, 0.6, cell_shrink)
    exp = O.forward_quant(Wi, Wh, bi, bh, x, p, h0, c0, mode=mode)
    got = _np_qcarrier(Wi, Wh, bi, bh, x, h0, c0, p, O.derive_exec(p, I), mode)
    for k in ("gate_out", "cell", "cell_tanh", "hidden", "x_q", "w_ih_q", "w_hh_q", "b_ih_q",
              "b_hh_q") + _LSTM_MASKS:
        np.testing.assert_array_equal(got[k], exp[k], err_msg=k)


def test_mask_restatement_cases_fire_every_family():
    fired = set()
    for cfg_name in CONFIGS:
        for shrink, cell_shrink in ((0.6, 1.0), (0.3, 1.0), (0.6, 0.05)):
            (Wi, Wh, bi, bh, x, h0, c0), p = _narrow_lstm(4, 3, 5, 8, cfg_name, 17, shrink,
                                                          cell_shrink)
            got = _np_qcarrier(Wi, Wh, bi, bh, x, h0, c0, p, O.derive_exec(p, 5), O.ACT_CR)
            fired |= {k for k in _LSTM_MASKS if got[k].max() == 1}
    assert fired == set(_LSTM_MASKS), sorted(set(_LSTM_MASKS) - fired)
