"""GPU parity of the QuantLSTM kernels against the pinned oracle (oracle/lstm_oracle.c).

Bar: the quantised forward (dequantised outputs, saved masters, checkpoints and clamp masks)
is bit-exact with the oracle run in its reference activation mode (ACT_LIBM: the C library's
expf / tanhf, as the reference CPU core compiled into oracle/_ref; the kernels evaluate in double
and take the reference's result at the few codes where the output code differs); backward
gradients within 1e-4 relative of the oracle's fp64 sums; calibration statistics (a float
forward, activations in double on the GPU) within float rounding of the oracle's.
"""
import numpy as np
import pytest
import torch

import lstm_ops
import lstm_oracle as O
import rxmet_lib
import rxmet_lstm_abi as L

pytestmark = pytest.mark.gpu
f32 = np.float32


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
    if name == "16b-whh":  # every operator 16-bit, W_hh included
        for k in range(L.NOPS):
            c.op[k].bits = 16
        return c
    if name == "mixed-8-16":  # the strict matrix's mixed profile: 16-bit W_ih, input branch
        for n in ("output", "weight_ih", "bias_ih", "weight_ih_linear", "input_gate_input",
                  "cell_gate_input", "input_gate_output", "cell_gate_output", "cell_tanh_output",
                  "weight_hh"):
            c.op[L.OP[n]].bits = 16
        return c
    if name == "whh16-h8":  # 16-bit W_hh, everything else 8-bit (one h plane)
        c.op[L.OP["weight_hh"]].bits = 16
        return c
    if name == "16b-act":  # 16-bit activations and state, 8-bit per-tensor parameters
        for k in range(L.NOPS):
            if L.OP_NAMES[k] in L.PARAM_OPS:
                c.op[k].granularity = L.PER_TENSOR
            else:
                c.op[k].bits = 16
        c.op[L.OP["output"]].is_unsigned = 1
        c.op[L.OP["output"]].is_symmetric = 0
        return c
    raise KeyError(name)


def _case(T, B, I, H, cfg_name, seed, bias=True, with_state=False):
    Wi, Wh, bi, bh = _weights(I, H, seed, bias)
    g = np.random.default_rng(seed + 1)
    x = (g.random((T, B, I)) * 2 - 1).astype(f32)
    h0 = c0 = None
    if with_state:
        h0 = (g.standard_normal((B, H)) * 0.3).astype(f32)
        c0 = (g.standard_normal((B, H)) * 0.5).astype(f32)
    stats = O.calibrate(Wi, Wh, bi, bh, x, h0, c0, mode=O.ACT_CR)
    p = O.finalize(stats, _config(cfg_name), H, bias)
    return (Wi, Wh, bi, bh, x, h0, c0), stats, p


def _wrap(p) -> lstm_ops.LstmQuantParams:
    w = lstm_ops.LstmQuantParams(p.hidden)
    w._p = p  # noqa: SLF001 (share the oracle-finalised struct)
    return w


def _dev(a, cuda):
    return None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(cuda)


def _np(t):
    return None if t is None else t.cpu().numpy()


def _gpu_forward(cuda, args, p, train):
    Wi, Wh, bi, bh, x, h0, c0 = (_dev(a, cuda) for a in args)
    out, hn, cn, saved = lstm_ops.forward_quant(x, Wi, Wh, bi, bh, h0, c0, _wrap(p), train)
    torch.cuda.synchronize()
    return out, hn, cn, saved


CASES = [  # T, B, I, H
    (5, 16, 7, 16),
    (4, 19, 12, 48),
    (3, 33, 40, 64),
    (2, 5, 3, 80),
]


@pytest.mark.parametrize("shape", CASES)
@pytest.mark.parametrize("with_state", [False, True])
def test_calibration_stats_match_oracle(cuda, shape, with_state):
    T, B, I, H = shape
    (Wi, Wh, bi, bh, x, h0, c0), exp, _ = _case(T, B, I, H, "default", 3, True, with_state)
    st = lstm_ops.new_stats(H, cuda)
    args = [_dev(a, cuda) for a in (x, Wi, Wh, bi, bh, h0, c0)]
    out, hn, cn = lstm_ops.forward_calibrate(*args, st)
    got = st.cpu().numpy()
    n = 2 * L.NOPS
    np.testing.assert_allclose(got[:n], exp[:n], rtol=2e-6, atol=2e-6)
    # parameter channel ranges are pure min/max over the weights: exact
    np.testing.assert_array_equal(got[n:], exp[n:])
    ro, rh, rc = O.forward_float(Wi, Wh, bi, bh, x, h0, c0, mode=O.ACT_CR)
    np.testing.assert_allclose(_np(out), ro, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(_np(hn), rh, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(_np(cn), rc, rtol=1e-5, atol=1e-6)


def test_calibration_merges_batches_and_counts_non_finite(cuda):
    T, B, I, H = 3, 8, 5, 16
    (Wi, Wh, bi, bh, x, h0, c0), _, _ = _case(T, B, I, H, "default", 4)
    st = lstm_ops.new_stats(H, cuda)
    lstm_ops.forward_calibrate(*[_dev(a, cuda) for a in (x, Wi, Wh, bi, bh, None, None)], st)
    x2 = (x * 3).astype(f32)
    lstm_ops.forward_calibrate(*[_dev(a, cuda) for a in (x2, Wi, Wh, bi, bh, None, None)], st)
    exp = O.calibrate(Wi, Wh, bi, bh, x, mode=O.ACT_CR)
    exp = O.calibrate(Wi, Wh, bi, bh, x2, stats=exp, mode=O.ACT_CR)
    np.testing.assert_allclose(st.cpu().numpy(), exp, rtol=2e-6, atol=2e-6)
    bad = Wh.copy()
    bad[3, 2] = np.nan
    st2 = lstm_ops.new_stats(H, cuda)
    lstm_ops.forward_calibrate(*[_dev(a, cuda) for a in (x, Wi, bad, bi, bh, None, None)], st2)
    assert st2.cpu().numpy()[-1] > 0
    with pytest.raises(rxmet_lib.RxmetError):
        lstm_ops.finalize_params(st2, _config("default"), H, True)


CFGS = ["default", "c4", "pot2-gate", "16b-act"]


def _compare_forward(o, out, hn, cn, saved, bias):
    np.testing.assert_array_equal(_np(out), o["output"], err_msg="output")
    np.testing.assert_array_equal(_np(hn), o["h_n"], err_msg="h_n")
    np.testing.assert_array_equal(_np(cn), o["c_n"], err_msg="c_n")
    if saved is None:
        return
    for k in L.SAVED_FIELDS:
        if k.startswith("b_") and not bias:
            continue
        np.testing.assert_array_equal(_np(saved[k]), o[k], err_msg=k)


@pytest.mark.parametrize("cfg_name", CFGS)
@pytest.mark.parametrize("shape", CASES)
@pytest.mark.parametrize("with_state", [False, True])
def test_forward_quant_bit_exact(cuda, cfg_name, shape, with_state):
    T, B, I, H = shape
    args, _, p = _case(T, B, I, H, cfg_name, 11, True, with_state)
    Wi, Wh, bi, bh, x, h0, c0 = args
    o = O.forward_quant(Wi, Wh, bi, bh, x, p, h0, c0, mode=O.ACT_LIBM_EXACT)
    out, hn, cn, saved = _gpu_forward(cuda, args, p, True)
    _compare_forward(o, out, hn, cn, saved, True)
    # inference (no checkpoints) gives the same outputs
    out2, hn2, cn2, s2 = _gpu_forward(cuda, args, p, False)
    assert s2 is None
    assert torch.equal(out, out2) and torch.equal(hn, hn2) and torch.equal(cn, cn2)


@pytest.mark.parametrize("cfg_name", ["default", "c4"])
def test_forward_quant_without_bias(cuda, cfg_name):
    T, B, I, H = 4, 17, 9, 32
    args, _, p = _case(T, B, I, H, cfg_name, 13, False, True)
    Wi, Wh, bi, bh, x, h0, c0 = args
    o = O.forward_quant(Wi, Wh, bi, bh, x, p, h0, c0, mode=O.ACT_LIBM_EXACT)
    out, hn, cn, saved = _gpu_forward(cuda, args, p, True)
    _compare_forward(o, out, hn, cn, saved, False)


def test_forward_quant_c4_hidden_512(cuda):
    # the c4 benchmark's hidden and input sizes on a short, narrow batch
    T, B, I, H = 3, 20, 64, 512
    args, _, p = _case(T, B, I, H, "c4", 17, True, False)
    Wi, Wh, bi, bh, x, h0, c0 = args
    o = O.forward_quant(Wi, Wh, bi, bh, x, p, h0, c0, mode=O.ACT_LIBM_EXACT)
    out, hn, cn, saved = _gpu_forward(cuda, args, p, True)
    _compare_forward(o, out, hn, cn, saved, True)


def test_forward_saturating_inputs_set_masks(cuda):
    T, B, I, H = 3, 16, 6, 16
    args, _, p = _case(T, B, I, H, "c4", 19, True, True)
    Wi, Wh, bi, bh, x, h0, c0 = args
    x = (x * 4).astype(f32)  # beyond the calibrated range: input clamps
    h0 = (h0 * 10).astype(f32)
    o = O.forward_quant(Wi, Wh, bi, bh, x, p, h0, c0, mode=O.ACT_LIBM_EXACT)
    assert o["x_m"].any() and o["h0_m"].any()
    out, hn, cn, saved = _gpu_forward(cuda, (Wi, Wh, bi, bh, x, h0, c0), p, True)
    _compare_forward(o, out, hn, cn, saved, True)


def _grads(T, B, H, seed):
    g = np.random.default_rng(seed)
    go = (g.standard_normal((T, B, H)) * 0.1).astype(f32)
    gh = (g.standard_normal((B, H)) * 0.1).astype(f32)
    gc = (g.standard_normal((B, H)) * 0.1).astype(f32)
    return go, gh, gc


def _assert_grads(got, exp):
    for name, a in got.items():
        e = exp[name]
        if e is None:
            assert a is None, name
            continue
        scale = max(float(np.abs(e).max()), 1e-30)
        np.testing.assert_allclose(a, e, rtol=1e-4, atol=1e-5 * scale, err_msg=name)


def _gpu_backward(cuda, saved, p, go, gh, gc):
    r = lstm_ops.backward_quant(saved, _wrap(p), _dev(go, cuda), _dev(gh, cuda), _dev(gc, cuda))
    torch.cuda.synchronize()
    names = ("dx", "dW_ih", "dW_hh", "db_ih", "db_hh", "dh0", "dc0")
    return {n: _np(t) for n, t in zip(names, r)}


@pytest.mark.parametrize("cfg_name", CFGS)
@pytest.mark.parametrize("shape", CASES)
@pytest.mark.parametrize("with_state", [False, True])
def test_backward_matches_oracle(cuda, cfg_name, shape, with_state):
    T, B, I, H = shape
    args, _, p = _case(T, B, I, H, cfg_name, 21, True, with_state)
    Wi, Wh, bi, bh, x, h0, c0 = args
    o = O.forward_quant(Wi, Wh, bi, bh, x, p, h0, c0, mode=O.ACT_LIBM_EXACT)
    _, _, _, saved = _gpu_forward(cuda, args, p, True)
    go, gh, gc = _grads(T, B, H, 22)
    exp = O.backward_quant(o, p, go, gh, gc)
    got = _gpu_backward(cuda, saved, p, go, gh, gc)
    _assert_grads(got, exp)


def test_backward_without_bias_and_final_state_grads(cuda):
    T, B, I, H = 4, 18, 10, 32
    args, _, p = _case(T, B, I, H, "c4", 23, False, True)
    Wi, Wh, bi, bh, x, h0, c0 = args
    o = O.forward_quant(Wi, Wh, bi, bh, x, p, h0, c0, mode=O.ACT_LIBM_EXACT)
    _, _, _, saved = _gpu_forward(cuda, args, p, True)
    go, _, _ = _grads(T, B, H, 24)
    exp = O.backward_quant(o, p, go)
    got = _gpu_backward(cuda, saved, p, go, None, None)
    _assert_grads(got, exp)


def test_backward_c4_hidden_512(cuda):
    T, B, I, H = 3, 20, 64, 512
    args, _, p = _case(T, B, I, H, "c4", 25, True, True)
    Wi, Wh, bi, bh, x, h0, c0 = args
    o = O.forward_quant(Wi, Wh, bi, bh, x, p, h0, c0, mode=O.ACT_LIBM_EXACT)
    _, _, _, saved = _gpu_forward(cuda, args, p, True)
    go, gh, gc = _grads(T, B, H, 26)
    exp = O.backward_quant(o, p, go, gh, gc)
    got = _gpu_backward(cuda, saved, p, go, gh, gc)
    _assert_grads(got, exp)


def test_backward_nan_stays_in_its_sequence(cuda):
    T, B, I, H = 3, 16, 5, 32
    args, _, p = _case(T, B, I, H, "default", 27, True, False)
    _, _, _, saved = _gpu_forward(cuda, args, p, True)
    go = np.full((T, B, H), 1e-2, f32)
    go[2, 3, 7] = np.nan
    got = _gpu_backward(cuda, saved, p, go, None, None)
    assert np.isnan(got["dh0"][3]).any() or np.isnan(got["dc0"][3]).any()
    assert np.isfinite(np.delete(got["dh0"], 3, axis=0)).all()
    assert np.isfinite(np.delete(got["dc0"], 3, axis=0)).all()


def test_float_forward_matches_torch_lstm(cuda):
    T, B, I, H = 6, 9, 11, 48
    Wi, Wh, bi, bh = _weights(I, H, 31)
    g = np.random.default_rng(32)
    x = (g.random((T, B, I)) * 2 - 1).astype(f32)
    h0 = (g.standard_normal((B, H)) * 0.3).astype(f32)
    c0 = (g.standard_normal((B, H)) * 0.5).astype(f32)
    out, hn, cn = lstm_ops.forward_float(*[_dev(a, cuda) for a in (x, Wi, Wh, bi, bh, h0, c0)])
    m = torch.nn.LSTM(I, H).double()
    with torch.no_grad():
        for name, a in (("weight_ih_l0", Wi), ("weight_hh_l0", Wh), ("bias_ih_l0", bi),
                        ("bias_hh_l0", bh)):
            getattr(m, name).copy_(torch.from_numpy(a).double())
        ro, (rh, rc) = m(torch.from_numpy(x).double(),
                         (torch.from_numpy(h0)[None].double(), torch.from_numpy(c0)[None].double()))
    np.testing.assert_allclose(_np(out), ro.numpy(), rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(_np(hn), rh[0].numpy(), rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(_np(cn), rc[0].numpy(), rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("H", [1, 2, 5, 24, 33])
@pytest.mark.parametrize("cfg_name", ["default", "c4", "16b-act"])
def test_any_hidden_size_forward_backward_match_oracle(cuda, H, cfg_name):
    """Hidden sizes that are not a multiple of 16 (the reference's strict matrix uses 1, 2 and
    33) run with inert padded units inside the boundary: the forward and every saved tensor
    bit-exact, gradients within 1e-4 of the oracle at the real size."""
    T, B, I = 4, 5, 3
    print(f"[lstm any H] H={H} cfg={cfg_name}", flush=True)
    args, _, p = _case(T, B, I, H, cfg_name, 41, True, True)
    Wi, Wh, bi, bh, x, h0, c0 = args
    o = O.forward_quant(Wi, Wh, bi, bh, x, p, h0, c0, mode=O.ACT_LIBM_EXACT)
    out, hn, cn, saved = _gpu_forward(cuda, args, p, True)
    _compare_forward(o, out, hn, cn, saved, True)
    go, gh, gc = _grads(T, B, H, 42)
    exp = O.backward_quant(o, p, go, gh, gc)
    got = _gpu_backward(cuda, saved, p, go, gh, gc)
    _assert_grads(got, exp)


def test_unsupported_shapes_raise(cuda):
    c = _config("default")
    c.op[L.OP["weight_hh"]].bits = 24
    args, stats, _ = _case(2, 4, 3, 16, "default", 34)
    p24 = O.finalize(stats, c, 16, True)
    with pytest.raises(rxmet_lib.RxmetError, match="16 bits"):
        _gpu_forward(cuda, args, p24, False)


@pytest.mark.parametrize("shape", [(4, 20, 7, 32), (3, 33, 40, 64), (3, 6, 2, 33), (2, 40, 8, 640)])
@pytest.mark.parametrize("cfg_name", ["16b-whh", "mixed-8-16"])
def test_wide_recurrent_weights_forward_backward_match_oracle(cuda, shape, cfg_name):
    """W_hh of 16 bits (the reference's int16 and mixed profiles) and H above 512 run on the
    stepped recurrence (an exact two-plane GEMM and a pointwise launch per step; a bf16-plane
    dh GEMM per step backward): forward and saved tensors bit-exact, gradients within 1e-4."""
    T, B, I, H = shape
    print(f"[lstm wide W_hh] shape={shape} cfg={cfg_name}", flush=True)
    args, _, p = _case(T, B, I, H, cfg_name, 51, True, True)
    Wi, Wh, bi, bh, x, h0, c0 = args
    o = O.forward_quant(Wi, Wh, bi, bh, x, p, h0, c0, mode=O.ACT_LIBM_EXACT)
    out, hn, cn, saved = _gpu_forward(cuda, args, p, True)
    _compare_forward(o, out, hn, cn, saved, True)
    go, gh, gc = _grads(T, B, H, 52)
    exp = O.backward_quant(o, p, go, gh, gc)
    got = _gpu_backward(cuda, saved, p, go, gh, gc)
    _assert_grads(got, exp)


@pytest.mark.parametrize("shape,cfg_name", [((3, 40, 8, 128), "c4"), ((4, 20, 5, 64), "16b-act"),
                                            ((3, 17, 6, 1024), "c4")])
def test_hidden_above_512_and_forced_stepped_match_oracle(cuda, shape, cfg_name, monkeypatch):
    """H above 512 steps by itself; below it the stepped path forced with RXMET_LSTM_STEPPED
    gives the same results as the MFMA recurrences (forward bit for bit, gradients within 1e-4
    of the oracle)."""
    T, B, I, H = shape
    print(f"[lstm stepped] shape={shape} cfg={cfg_name}", flush=True)
    args, _, p = _case(T, B, I, H, cfg_name, 53, True, True)
    Wi, Wh, bi, bh, x, h0, c0 = args
    o = O.forward_quant(Wi, Wh, bi, bh, x, p, h0, c0, mode=O.ACT_LIBM_EXACT)
    go, gh, gc = _grads(T, B, H, 54)
    exp = O.backward_quant(o, p, go, gh, gc)
    monkeypatch.setenv("RXMET_LSTM_STEPPED", "1")
    out, hn, cn, saved = _gpu_forward(cuda, args, p, True)
    _compare_forward(o, out, hn, cn, saved, True)
    _assert_grads(_gpu_backward(cuda, saved, p, go, gh, gc), exp)


@pytest.mark.parametrize("shape,cfg_name", [((3, 2560, 16, 128), "c4"), ((2, 100, 24, 256), "c4"),
                                            ((2, 48, 8, 64), "c4"), ((3, 40, 8, 128), "16b-act")])
def test_clustered_recurrence_matches_oracle_and_single_tile_path(cuda, shape, cfg_name,
                                                                   monkeypatch):
    """H a multiple of 64 takes the clustered recurrence (H / 64 workgroups per batch tile,
    several batch tiles per cluster when B is large); it must equal the oracle and the
    one-workgroup-per-tile recurrence bit for bit."""
    T, B, I, H = shape
    args, _, p = _case(T, B, I, H, cfg_name, 41, True, True)
    Wi, Wh, bi, bh, x, h0, c0 = args
    out, hn, cn, saved = _gpu_forward(cuda, args, p, True)
    o = O.forward_quant(Wi, Wh, bi, bh, x, p, h0, c0, mode=O.ACT_LIBM_EXACT)
    _compare_forward(o, out, hn, cn, saved, True)
    monkeypatch.setenv("RXMET_NO_CLUSTER", "1")
    out2, hn2, cn2, saved2 = _gpu_forward(cuda, args, p, True)
    assert torch.equal(out, out2) and torch.equal(hn, hn2) and torch.equal(cn, cn2)
    for k in saved:
        assert torch.equal(saved[k], saved2[k]), k


@pytest.mark.parametrize("shape,cfg_name", [((4, 36, 9, 128), "16b-whh"), ((3, 70, 8, 256), "16b-whh"),
                                            ((3, 40, 8, 64), "mixed-8-16"),
                                            ((3, 50, 12, 192), "whh16-h8"),
                                            ((3, 300, 8, 128), "whh16-h8")])
def test_clustered_recurrence_with_16bit_recurrent_weights(cuda, shape, cfg_name, monkeypatch):
    """W_hh of 9-16 bits in the clustered recurrence (two int8 planes resident in LDS, H a
    multiple of 64 up to 256, sums recombined in int64): forward and saved tensors bit-exact
    against the oracle and against the stepped recurrence, inference equal to training."""
    T, B, I, H = shape
    print(f"[lstm cl 16-bit W_hh] shape={shape} cfg={cfg_name}", flush=True)
    args, _, p = _case(T, B, I, H, cfg_name, 47, True, True)
    Wi, Wh, bi, bh, x, h0, c0 = args
    out, hn, cn, saved = _gpu_forward(cuda, args, p, True)
    o = O.forward_quant(Wi, Wh, bi, bh, x, p, h0, c0, mode=O.ACT_LIBM_EXACT)
    _compare_forward(o, out, hn, cn, saved, True)
    oi, hi, ci, _ = _gpu_forward(cuda, args, p, False)
    assert torch.equal(out, oi) and torch.equal(hn, hi) and torch.equal(cn, ci)
    monkeypatch.setenv("RXMET_LSTM_STEPPED", "1")
    out2, hn2, cn2, saved2 = _gpu_forward(cuda, args, p, True)
    assert torch.equal(out, out2) and torch.equal(hn, hn2) and torch.equal(cn, cn2)
    for k in saved:
        assert torch.equal(saved[k], saved2[k]), k


@pytest.mark.parametrize("shape,cfg_name", [((3, 2560, 16, 128), "c4"), ((2, 100, 24, 256), "c4"),
                                            ((3, 40, 8, 128), "16b-act"),
                                            ((3, 20, 64, 512), "pot2-gate"),
                                            ((3, 40, 8, 384), "c4")])
def test_clustered_backward_matches_oracle_and_single_tile_path(cuda, shape, cfg_name,
                                                                monkeypatch):
    """H a multiple of 128 takes the clustered backward (members exchange block-fixed-point
    gate gradients, one exponent per sequence and member); it must match the oracle within
    1e-4 and the one-workgroup-per-tile backward.  H = 384 (six members, three K-steps per
    wave) has waves whose K-steps span two members, each with its own exponent."""
    T, B, I, H = shape
    args, _, p = _case(T, B, I, H, cfg_name, 43, True, True)
    Wi, Wh, bi, bh, x, h0, c0 = args
    o = O.forward_quant(Wi, Wh, bi, bh, x, p, h0, c0, mode=O.ACT_LIBM_EXACT)
    _, _, _, saved = _gpu_forward(cuda, args, p, True)
    go, gh, gc = _grads(T, B, H, 44)
    exp = O.backward_quant(o, p, go, gh, gc)
    got = _gpu_backward(cuda, saved, p, go, gh, gc)
    _assert_grads(got, exp)
    monkeypatch.setenv("RXMET_NO_CLUSTER", "1")
    ref = _gpu_backward(cuda, saved, p, go, gh, gc)
    _assert_grads(got, ref)


def test_clustered_backward_nan_stays_in_its_sequence(cuda):
    T, B, I, H = 3, 32, 5, 128
    args, _, p = _case(T, B, I, H, "default", 45, True, False)
    _, _, _, saved = _gpu_forward(cuda, args, p, True)
    go = np.full((T, B, H), 1e-2, f32)
    go[2, 3, 7] = np.nan
    got = _gpu_backward(cuda, saved, p, go, None, None)
    assert np.isnan(got["dh0"][3]).any() or np.isnan(got["dc0"][3]).any()
    assert np.isfinite(np.delete(got["dh0"], 3, axis=0)).all()
    assert np.isfinite(np.delete(got["dc0"], 3, axis=0)).all()
