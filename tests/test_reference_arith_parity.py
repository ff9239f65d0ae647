"""Parity against the reference's own arithmetic over whole sequences (CPU only).

QuantLSTM.  The reference's CPU core evaluates its real activations with the C library's
expf / tanhf (realSigmoid / realTanh, operators/quant-lstm/src/lstm/cuda/quantized_fp_math.cuh:
21-30) and accumulates each linear's products in fp32 in index order (linearValue,
forward_quantized_fp_cpu.cc:20-45); the oracle's ACT_LIBM mode does both and is bit-exact against
the core compiled into oracle/_ref (tests/test_lstm_oracle.py).  The kernels sum exactly and
evaluate exp / tanh in double, taking the reference's result at the input codes where the two
evaluations give different output codes; the library lists those codes on the host
(rxmet_lstm_activation_exceptions).  The oracle's ACT_LIBM_EXACT mode (the C library's
activations, exact sums) is what the GPU parity tests compare against bit for bit.
Checked here on every code of every activation grid of at most 2^16 codes:
  * the library's host tables equal the oracle's ACT_LIBM and ACT_CR tables entry for entry,
    and its exception lists are exactly the codes where those two differ;
  * at c4 (8-bit gates, 16-bit cell, 8-bit h) there are none, and every linear sum stays below
    2^24: the kernels' arithmetic equals the reference CPU core's at every reachable code, and
    whole c4-length sequences agree code for code in all three oracle modes;
  * the reference's 8-bit strict-matrix profiles likewise.  The 16-bit profiles have 18-64
    exception codes per tanh grid (applied by the kernels), and their linear sums (16-bit h x
    16-bit W_hh) pass 2^24, where fp32 accumulation depends on the order: the reference CPU
    core's index order and the exact sum then drift apart over whole sequences (measured: up to
    4 LSB on up to 6 % of the codes of the int16 profiles; the reference's CUDA path uses cuBLAS,
    whose order is a third one).  There the kernels are bit-exact against ACT_LIBM_EXACT only.

QuantGRU.  The kernels sum the GEMMs of integer codes exactly; the reference sums them with
cuBLAS SGEMM in fp32 (ComputeLinearX / ComputeLinearH, gru_forward_gpu_quant_fp.cu:1111-1155),
which rounds once partial sums pass 2^24 (c3: 16-bit h x 8-bit R over K = 256; c5: 16-bit x
4-bit over K = 1024).  cuBLAS's order is not reproducible here; the oracle's SUM_SEQ_F32 mode
(fp32 products added in K order) is the plain SGEMM model.  Over whole c3 / c5 sequences the h
codes of the two stay within one LSB on at most 0.1 % of the elements, and so do the gate codes.
"""
import ctypes
import json
from pathlib import Path

import numpy as np
import pytest
import torch

import gru_oracle as GO
import lstm_oracle as O
import quant_lstm as Q
import rxmet_gru_abi as A
import rxmet_lib
import rxmet_lstm_abi as L
from test_gru_oracle import to_haste
from test_lstm_oracle import _calibrated

f32 = np.float32
DOC = json.loads((Path(__file__).resolve().parent / "golden" / "lstm" /
                  "strict_matrix_cuda_cases.json").read_text())
# (input op, output op, tanh) of activation k = 0..4 (gates i, f, g, o; tanh of the cell)
ACTS = [("input_gate_input", "input_gate_output", 0), ("forget_gate_input", "forget_gate_output", 0),
        ("cell_gate_input", "cell_gate_output", 1), ("output_gate_input", "output_gate_output", 0),
        ("cell_state", "cell_tanh_output", 1)]
MAXC = 1 << 16


def _grid(op):
    return (0, (1 << op.bits) - 1) if op.is_unsigned else (-(1 << (op.bits - 1)), (1 << (op.bits - 1)) - 1)


def _oracle_table(p, k, mode):
    src, dst, tanh = ACTS[k]
    lo, hi = _grid(p.config.op[L.OP[src]])
    out, m = O.real_activation_table(lo, hi, p.scale[L.OP[src]], p.zero_point[L.OP[src]],
                                     p.scale[L.OP[dst]], p.zero_point[L.OP[dst]],
                                     p.config.op[L.OP[dst]], tanh, mode)
    olo, _ = _grid(p.config.op[L.OP[dst]])
    return ((out.astype(np.int64) - olo).astype(np.uint32) << 1) | m.astype(np.uint32), lo


def _lib_table(p, k, reference):
    buf = np.zeros(MAXC, np.uint32)
    n = rxmet_lib.load().rxmet_lstm_activation_table(ctypes.byref(p), k, int(reference),
                                                     buf.ctypes.data_as(ctypes.c_void_p), MAXC)
    assert n > 0, rxmet_lib.last_error()
    return buf[:n]


def _lib_exceptions(p):
    keys = np.zeros(5 * MAXC, np.int32)
    vals = np.zeros(5 * MAXC, np.uint32)
    off = np.zeros(5, np.int32)
    cnt = np.zeros(5, np.int32)
    vp = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    tot = rxmet_lib.load().rxmet_lstm_activation_exceptions(ctypes.byref(p), vp(keys), vp(vals),
                                                            5 * MAXC, vp(off), vp(cnt))
    assert tot >= 0, rxmet_lib.last_error()
    return [(keys[off[k]:off[k] + cnt[k]], vals[off[k]:off[k] + cnt[k]]) for k in range(5)]


def _check_tables(p):
    """Library host tables == oracle tables on every code; exceptions == where they differ.
    Returns the number of exceptions per activation."""
    exc = _lib_exceptions(p)
    counts = []
    for k in range(5):
        src = ACTS[k][0]
        lo, hi = _grid(p.config.op[L.OP[src]])
        if hi - lo + 1 > MAXC:
            assert len(exc[k][0]) == 0
            counts.append(None)
            continue
        ref, _ = _oracle_table(p, k, O.ACT_LIBM)
        dbl, _ = _oracle_table(p, k, O.ACT_CR)
        np.testing.assert_array_equal(_lib_table(p, k, True), ref, err_msg=f"reference table {k}")
        np.testing.assert_array_equal(_lib_table(p, k, False), dbl, err_msg=f"double table {k}")
        diff = np.nonzero(ref != dbl)[0]
        np.testing.assert_array_equal(exc[k][0], diff + lo, err_msg=f"exception codes {k}")
        np.testing.assert_array_equal(exc[k][1], ref[diff], err_msg=f"exception entries {k}")
        counts.append(len(diff))
    return counts


def _case_params(case, nseq=8):
    T, B, I, H = case["shape"]
    torch.manual_seed(DOC["parameter_seeds"][case["shape_profile"]])
    m = Q.QuantLSTM(I, H, bias=case["bias_profile"] != "disabled")
    Wi, Wh, bi, bh = (None if t is None else t.detach().numpy() for t in m._direction_params(False))
    g = torch.Generator().manual_seed(1001)
    x = (torch.rand((T, B, I), generator=g) * 2 - 1).numpy()[:, :nseq].copy()
    stats = O.calibrate(Wi, Wh, bi, bh, x)
    p = O.finalize(stats, Q.config_struct(case["resolved_quant_config"]), H, bi is not None)
    return p, (Wi, Wh, bi, bh, x)


def test_lstm_c4_double_evaluation_equals_reference_on_every_code():
    (_, _, _, _, _, _, _), _, _, p = _calibrated(100, 8, 64, 512, "c4", 7, True, False)
    counts = _check_tables(p)
    assert counts == [0, 0, 0, 0, 0], counts


def test_lstm_c4_length_sequences_agree_code_for_code():
    (Wi, Wh, bi, bh, x, _, _), _, _, p = _calibrated(100, 4, 64, 512, "c4", 7, True, False)
    a = O.forward_quant(Wi, Wh, bi, bh, x, p, mode=O.ACT_LIBM)
    for mode in (O.ACT_LIBM_EXACT, O.ACT_CR):
        b = O.forward_quant(Wi, Wh, bi, bh, x, p, mode=mode)
        for k in ("gate_out", "cell", "cell_tanh", "hidden", "output"):
            np.testing.assert_array_equal(a[k], b[k], err_msg=k)


PROFILES = {}
for _c in DOC["cases"]:
    PROFILES.setdefault((_c["bitwidth_profile"], _c["shape_profile"]), _c)


@pytest.mark.parametrize("case", list(PROFILES.values()), ids=[c["case_id"] for c in PROFILES.values()])
def test_lstm_strict_matrix_tables_and_sequences(case):
    p, (Wi, Wh, bi, bh, x) = _case_params(case)
    counts = _check_tables(p)
    if case["bitwidth_profile"] != "all_int8":
        return
    assert counts == [0, 0, 0, 0, 0], counts
    a = O.forward_quant(Wi, Wh, bi, bh, x, p, mode=O.ACT_LIBM)
    for mode in (O.ACT_LIBM_EXACT, O.ACT_CR):
        b = O.forward_quant(Wi, Wh, bi, bh, x, p, mode=mode)
        for k in ("gate_out", "cell", "cell_tanh", "hidden"):
            np.testing.assert_array_equal(a[k], b[k], err_msg=k)


def _gru_weights(I, H, seed):
    g = torch.Generator().manual_seed(seed)
    k = 1.0 / H ** 0.5
    u = lambda *s: (torch.rand(*s, generator=g) * 2 - 1) * k
    return to_haste(u(3 * H, I), u(3 * H, H), u(3 * H), u(3 * H))


def _gru_sum_divergence(T, I, H, nseq, cfg, seed, reverse):
    W, R, bw, br = _gru_weights(I, H, seed)
    x = np.random.default_rng(seed).standard_normal((T, nseq, I)).astype(f32)
    if reverse:
        x = np.ascontiguousarray(x[::-1])
    _, _, stats = GO.forward_calibrate(W, R, bw, br, x)
    qp, _ = GO.make_params(A.make_ranges(stats, H), cfg)
    try:
        GO.set_sum_mode(GO.SUM_SEQ_F32)
        b = GO.forward_quant(W, R, bw, br, x, qp, training=False)
    finally:
        GO.set_sum_mode(GO.SUM_EXACT)
    a = GO.forward_quant(W, R, bw, br, x, qp, training=False)
    eh = GO.effective_scale(qp.g[A.GRID["h"]].scale, bool(cfg.use_pot2))
    dh = np.abs(np.rint(a["h"][1:].astype(np.float64) / eh) - np.rint(b["h"][1:].astype(np.float64) / eh))
    assert dh.max() <= 1 and (dh > 0).mean() <= 1e-3, (dh.max(), (dh > 0).mean())
    for k, nm in enumerate(("z", "r", "n", "hh_n")):
        va, vb = a["v"][..., k * H:(k + 1) * H], b["v"][..., k * H:(k + 1) * H]
        assert (va != vb).mean() <= 1e-3, nm
    # the configuration does reach sums beyond 2^24 (where fp32 summation rounds)
    hz = qp.g[A.GRID["h"]].zero_point
    hc = np.rint(a["h"][T // 2].astype(np.float64) / eh) + hz
    return np.abs(hc @ a["R_q"].astype(np.float64)).max()


@pytest.mark.parametrize("reverse", [False, True])
def test_gru_c3_exact_sums_track_sequential_fp32(reverse):
    cfg = A.set_all_bitwidth(A.default_config(), 8, False)
    cfg.op[A.GRID["h"]].bits = 16
    big = _gru_sum_divergence(200, 80, 256, 4, cfg, 10 + int(reverse), reverse)
    assert big > 2 ** 24


def test_gru_c5_exact_sums_track_sequential_fp32():
    cfg = A.set_all_bitwidth(A.default_config(), 16, False)
    cfg.chan[0].bits = cfg.chan[1].bits = 4
    cfg.use_pot2 = 1
    _gru_sum_divergence(50, 256, 1024, 2, cfg, 12, False)
