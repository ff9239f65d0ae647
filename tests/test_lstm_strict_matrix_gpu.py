"""The reference's strict precision matrix for the CUDA FP32 q-carrier
(operators/quant-lstm/tests/precision/config/strict_matrix_v2.json, its 41 cuda_fp32 cases,
kept as data in tests/golden/lstm/strict_matrix_cuda_cases.json) run through QuantLSTM on the
GPU: each case's resolved operator config (all-int8, all-int16 and mixed 8/16 profiles, W_hh of
16 bits included), shape (1x1x1x1, 3x1x2x2, 7x3x31x33, 256x1x64x128, 50x64x128x256,
16x128x64x128), bias, layout and initial-state profile; calibrated on the GPU, then one QAT
forward and backward.

Bars: output, h_n and c_n bit-exact against the oracle in its reference activation mode (the C
library's expf / tanhf of the reference CPU core) with the module's own grids; every gradient within 1e-4 relative.  The reference gates these cases
against a float LSTM with MSE / MAE / cosine thresholds; the oracle comparison is stricter."""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

import lstm_oracle as O
import quant_lstm as Q

pytestmark = pytest.mark.gpu
DOC = json.loads((Path(__file__).resolve().parent / "golden" / "lstm" /
                  "strict_matrix_cuda_cases.json").read_text())
CASES = DOC["cases"]


def _np(t):
    return t.detach().cpu().numpy()


def _states(profile, B, H, g):
    if profile == "omitted":
        return None
    if profile == "explicit_zero":
        return torch.zeros(1, B, H), torch.zeros(1, B, H)
    h0 = torch.randn(1, B, H, generator=g) * 0.3
    c0 = torch.randn(1, B, H, generator=g) * 0.5
    if profile == "near_quant_boundary":  # beyond the calibrated ranges: both clamp
        return h0 * 8, c0 * 8
    if profile == "mixed_h_random_c_boundary":
        return h0, c0 * 8
    return h0, c0


@pytest.mark.parametrize("case", CASES, ids=[c["case_id"] for c in CASES])
def test_strict_matrix_case_matches_oracle(cuda, case):
    T, B, I, H = case["shape"]
    bias = case["bias_profile"] != "disabled"
    bf = bool(case["batch_first"])
    print(f"[lstm strict] {case['case_id']} shape={case['shape']} bits={case['bitwidth_profile']} "
          f"state={case['state_profile']} bias={bias} bf={bf}", flush=True)
    torch.manual_seed(DOC["parameter_seeds"][case["shape_profile"]])
    m = Q.QuantLSTM(I, H, bias=bias, batch_first=bf,
                    quant_config=case["resolved_quant_config"]).to(cuda)
    g = torch.Generator().manual_seed(1001)
    xt = torch.rand((T, B, I), generator=g) * 2 - 1
    st = _states(case["state_profile"], B, H, g)
    x = (xt.transpose(0, 1).contiguous() if bf else xt).to(cuda)
    hx = None if st is None else tuple(s.to(cuda) for s in st)
    m.calibrating = True
    with torch.no_grad():
        m(x, hx)
    m.calibrating = False
    m.finalize_calibration()
    m.use_quantization = True
    m.train()
    xl = x.clone().requires_grad_(True)
    hxl = None if hx is None else tuple(s.clone().requires_grad_(True) for s in hx)
    out, (hn, cn) = m(xl, hxl)
    go = torch.randn(out.shape, generator=g) * 0.1
    (out * go.to(cuda)).sum().backward()
    torch.cuda.synchronize()
    Wi, Wh, bi, bh = (None if p is None else _np(p) for p in m._direction_params(False))
    p = m._params[0].struct
    h0 = None if st is None else st[0][0].numpy()
    c0 = None if st is None else st[1][0].numpy()
    o = O.forward_quant(Wi, Wh, bi, bh, xt.numpy(), p, h0, c0, mode=O.ACT_LIBM_EXACT)
    out_tm = _np(out.transpose(0, 1) if bf else out)
    np.testing.assert_array_equal(out_tm, o["output"], err_msg="output")
    np.testing.assert_array_equal(_np(hn[0]), o["h_n"], err_msg="h_n")
    np.testing.assert_array_equal(_np(cn[0]), o["c_n"], err_msg="c_n")
    go_tm = (go.transpose(0, 1) if bf else go).contiguous().numpy()
    gr = O.backward_quant(o, p, go_tm)

    def close(got, exp, name):
        assert np.isfinite(got).all(), name
        np.testing.assert_allclose(got, exp, rtol=1e-4, atol=1e-5 * max(np.abs(exp).max(), 1e-30),
                                   err_msg=name)

    gx = _np(xl.grad.transpose(0, 1) if bf else xl.grad)
    close(gx, gr["dx"], "dx")
    close(_np(m.weight_ih_l0.grad), gr["dW_ih"], "dW_ih")
    close(_np(m.weight_hh_l0.grad), gr["dW_hh"], "dW_hh")
    if bias:
        close(_np(m.bias_ih_l0.grad), gr["db_ih"], "db_ih")
        close(_np(m.bias_hh_l0.grad), gr["db_hh"], "db_hh")
    if hxl is not None:
        close(_np(hxl[0].grad[0]), gr["dh0"], "dh0")
        close(_np(hxl[1].grad[0]), gr["dc0"], "dc0")
