"""The benchmark configurations at their full size on the GPU, against the oracle.

Sequences are independent, so the GPU's rows of a sample of sequences must equal the oracle
run on those sequences alone.  The output gradient is set on the sampled sequences only
(zero elsewhere): every weight and bias gradient is then a sum over the sampled sequences and
is checked against the oracle as well.

- c3: QuantGRU bidirectional QAT, B=256, T=200, I=80, H=256, batch_first, 8-bit per-channel
  weights, 8-bit asymmetric activations, 16-bit h; calibrated on the GPU over the whole batch.
- c4: QuantLSTM QAT, B=512, T=100, I=64, H=512, 8-bit weights and gates, 16-bit cell state.
- c1: QuantGRU PTQ calibration pass, B=32, T=98, I=40, H=64, per-tensor symmetric 8-bit
  weights, asymmetric 8-bit activations, then the PTQ forward on the FP32 carrier and on the
  int32 carrier (and int codes in and out); every sequence checked.

Bars: forward outputs bit-exact; gradients within 1e-4 relative of the oracle; calibration
ranges within the device-tanhf tolerance of the calibration tests.
"""
import numpy as np
import pytest
import torch

import gru_oracle as GO
import lstm_oracle as LO
import quant_gru as QG
import quant_lstm as QL
import rxmet_gru_abi as A

pytestmark = pytest.mark.gpu
f32 = np.float32


def _swap(t):
    r, z, n = np.split(t, 3, axis=0)
    return np.concatenate([z, r, n], 0)


def _haste(m, sfx):
    p = lambda n: getattr(m, n + sfx).detach().cpu().numpy()
    return (np.ascontiguousarray(_swap(p("weight_ih_l0")).T),
            np.ascontiguousarray(_swap(p("weight_hh_l0")).T),
            _swap(p("bias_ih_l0")), _swap(p("bias_hh_l0")))


def _close(got, exp, name, rtol=1e-4):
    scale = max(float(np.abs(exp).max()), 1e-30)
    assert np.isfinite(got).all(), f"{name}: non-finite values"
    np.testing.assert_allclose(got, exp, rtol=rtol, atol=1e-5 * scale, err_msg=name)


def test_c3_full_size_quantgru_matches_oracle_on_sampled_sequences(cuda):
    B, T, I, H = 256, 200, 80, 256
    rows = [0, 1, 63, 128, 129, 200, 254, 255]
    print(f"[c3 full] B={B} T={T} I={I} H={H} bidirectional rows={rows}", flush=True)
    torch.manual_seed(6)
    x = torch.randn(B, T, I)
    m = QG.QuantGRU(I, H, batch_first=True, bidirectional=True)
    m.set_all_bitwidth(8, is_symmetric=False)
    m._bitwidth_config.h_ = 16
    m = m.to(cuda)
    xd = x.to(cuda)
    with m.calibration_context():
        m(xd)
    m.use_quantization = True
    m.train()

    # the benchmark's own step (loss = mean of the output): finite, and dx of the sampled
    # sequences as the oracle's
    xl = xd.clone().requires_grad_(True)
    out, hn = m(xl)
    out.mean().backward()
    torch.cuda.synchronize()
    dx_mean = xl.grad[rows].cpu().numpy()
    assert torch.isfinite(out).all() and torch.isfinite(xl.grad).all()
    for p in m.parameters():
        assert torch.isfinite(p.grad).all()
    out_rows = out[rows].detach().cpu().numpy()
    hn_rows = hn[:, rows].detach().cpu().numpy()

    # a random output gradient on the sampled sequences only
    m.zero_grad(set_to_none=True)
    g = torch.Generator().manual_seed(61)
    gout = torch.zeros(B, T, 2 * H)
    gout[rows] = torch.randn(len(rows), T, 2 * H, generator=g) * 1e-3
    xl2 = xd.clone().requires_grad_(True)
    out2, _ = m(xl2)
    (out2 * gout.to(cuda)).sum().backward()
    torch.cuda.synchronize()
    assert torch.equal(out2.detach(), out.detach()), "QAT forward is not deterministic"

    xs = x[rows].transpose(0, 1).contiguous().numpy()  # [T, rows, I]
    gs = gout[rows].transpose(0, 1).contiguous().numpy()  # [T, rows, 2H]
    gmean = np.float32(1.0 / (B * T * 2 * H))
    dx_exp = np.zeros_like(xs, dtype=np.float64)
    dxm_exp = np.zeros_like(xs, dtype=np.float64)
    for d, qp in enumerate((m.quant_params, m.quant_params_reverse)):
        sfx = "_reverse" if d else ""
        W, R, bw, br = _haste(m, sfx)
        xdir = np.ascontiguousarray(xs[::-1]) if d else xs
        fwd = GO.forward_quant(W, R, bw, br, xdir, qp.struct, training=True)
        o = fwd["h"][1:][::-1] if d else fwd["h"][1:]
        np.testing.assert_array_equal(out_rows[..., d * H:(d + 1) * H], o.transpose(1, 0, 2),
                                      err_msg=f"output dir{d}")
        np.testing.assert_array_equal(hn_rows[d], fwd["h"][-1], err_msg=f"h_n dir{d}")
        gdir = np.ascontiguousarray(gs[..., d * H:(d + 1) * H])
        dh = np.zeros((T + 1, len(rows), H), f32)
        dh[1:] = gdir[::-1] if d else gdir
        bwd = GO.backward_quant(fwd, dh, qp.struct)
        dx_exp += bwd["dx"][::-1] if d else bwd["dx"]
        dhm = np.zeros((T + 1, len(rows), H), f32)
        dhm[1:] = gmean
        bwm = GO.backward_quant(fwd, dhm, qp.struct)
        dxm_exp += bwm["dx"][::-1] if d else bwm["dx"]
        _close(getattr(m, "weight_ih_l0" + sfx).grad.cpu().numpy(), _swap(bwd["dW"].T),
               f"dW_ih dir{d}")
        _close(getattr(m, "weight_hh_l0" + sfx).grad.cpu().numpy(), _swap(bwd["dR"].T),
               f"dW_hh dir{d}")
        _close(getattr(m, "bias_ih_l0" + sfx).grad.cpu().numpy(), _swap(bwd["dbw"]),
               f"db_ih dir{d}")
        _close(getattr(m, "bias_hh_l0" + sfx).grad.cpu().numpy(), _swap(bwd["dbr"]),
               f"db_hh dir{d}")
    _close(xl2.grad[rows].cpu().numpy(), dx_exp.transpose(1, 0, 2), "dx (sampled gradient)")
    _close(dx_mean, dxm_exp.transpose(1, 0, 2), "dx (mean loss)")


def test_c4_full_size_quantlstm_matches_oracle_on_sampled_sequences(cuda):
    B, T, I, H = 512, 100, 64, 512
    rows = [0, 5, 255, 256, 511]
    print(f"[c4 full] B={B} T={T} I={I} H={H} rows={rows}", flush=True)
    torch.manual_seed(7)
    x = torch.rand(T, B, I) * 2 - 1
    torch.manual_seed(8)
    gfull = torch.randn(T, B, H) * 0.1
    m = QL.QuantLSTM(I, H, quant_config={"schema_version": 1,
                                         "operators": {"cell_state": {"bitwidth": 16}}}).to(cuda)
    xd = x.to(cuda)
    m.calibrating = True
    with torch.no_grad():
        m(xd)
    m.calibrating = False
    m.finalize_calibration()
    m.use_quantization = True
    m.train()

    # the benchmark's step: finite everywhere, dx of the sampled sequences as the oracle's
    xl = xd.clone().requires_grad_(True)
    out, (hn, cn) = m(xl)
    out.backward(gfull.to(cuda))
    torch.cuda.synchronize()
    assert torch.isfinite(out).all() and torch.isfinite(xl.grad).all()
    for p in m.parameters():
        assert torch.isfinite(p.grad).all()
    dx_bench = xl.grad[:, rows].cpu().numpy()

    m.zero_grad(set_to_none=True)
    gs = torch.zeros(T, B, H)
    gs[:, rows] = gfull[:, rows]
    xl2 = xd.clone().requires_grad_(True)
    out2, (hn2, cn2) = m(xl2)
    out2.backward(gs.to(cuda))
    torch.cuda.synchronize()
    assert torch.equal(out2.detach(), out.detach())

    Wi, Wh, bi, bh = (p.detach().cpu().numpy() for p in m._direction_params(False))
    p = m._params[0].struct
    xs = np.ascontiguousarray(x[:, rows].numpy())
    o = LO.forward_quant(Wi, Wh, bi, bh, xs, p, mode=LO.ACT_LIBM_EXACT)
    np.testing.assert_array_equal(out[:, rows].detach().cpu().numpy(), o["output"], err_msg="output")
    np.testing.assert_array_equal(hn[0, rows].detach().cpu().numpy(), o["h_n"], err_msg="h_n")
    np.testing.assert_array_equal(cn[0, rows].detach().cpu().numpy(), o["c_n"], err_msg="c_n")
    gr = LO.backward_quant(o, p, np.ascontiguousarray(gfull[:, rows].numpy()))
    _close(dx_bench, gr["dx"], "dx (benchmark gradient)")
    _close(xl2.grad[:, rows].cpu().numpy(), gr["dx"], "dx (sampled gradient)")
    for name, key in (("weight_ih_l0", "dW_ih"), ("weight_hh_l0", "dW_hh"),
                      ("bias_ih_l0", "db_ih"), ("bias_hh_l0", "db_hh")):
        _close(getattr(m, name).grad.cpu().numpy(), gr[key], name)


def test_c1_full_size_calibration_and_ptq_forward_match_oracle(cuda):
    B, T, I, H = 32, 98, 40, 64
    print(f"[c1 full] B={B} T={T} I={I} H={H}", flush=True)
    torch.manual_seed(1)
    x = torch.randn(B, T, I)
    m = QG.QuantGRU(I, H, batch_first=True)
    torch.nn.init.xavier_uniform_(m.weight_ih_l0)
    torch.nn.init.xavier_uniform_(m.weight_hh_l0)
    m.set_all_bitwidth(8, is_symmetric=False)
    for k in ("W_granularity_", "R_granularity_", "bw_granularity_", "br_granularity_"):
        setattr(m._bitwidth_config, k, A.PER_TENSOR)
    m = m.to(cuda)
    xd = x.to(cuda)
    with m.calibration_context():
        yc, hc = m(xd)
    torch.cuda.synchronize()
    W, R, bw, br = _haste(m, "")
    xs = np.ascontiguousarray(x.transpose(0, 1).numpy())
    he, _, se = GO.forward_calibrate(W, R, bw, br, xs)
    np.testing.assert_allclose(yc.transpose(0, 1).cpu().numpy(), he[1:], rtol=1e-5, atol=2e-6,
                               err_msg="calibration h")
    np.testing.assert_allclose(m.quant_ranges.stats.cpu().numpy(), se, rtol=1e-5, atol=2e-6,
                               err_msg="calibration ranges")
    if GO.has_ref():
        # the reference's own forwardWithCalibrationCPU, compiled from its sources
        hr, _, sr = GO.forward_calibrate(W, R, bw, br, xs, ref=True)
        np.testing.assert_array_equal(he, hr, err_msg="oracle vs reference calibration h")
        np.testing.assert_array_equal(se, sr, err_msg="oracle vs reference ranges")
    # grids derived from the GPU's ranges equal the oracle's derivation from the same ranges
    qp_exp, _ = GO.make_params(m.quant_ranges.to_struct(), m._bitwidth_config.to_struct())
    qp = m.quant_params.struct
    for i in range(A.NGRIDS):
        assert (qp.g[i].scale, qp.g[i].zero_point, qp.g[i].bits, qp.g[i].is_unsigned) == \
            (qp_exp.g[i].scale, qp_exp.g[i].zero_point, qp_exp.g[i].bits,
             qp_exp.g[i].is_unsigned), f"grid {i}"
    for k in range(A.NCHAN):
        np.testing.assert_array_equal(A.qparams_chan(qp, k), A.qparams_chan(qp_exp, k),
                                      err_msg=f"channel scales {k}")
    m.use_quantization = True
    m.eval()
    with torch.no_grad():
        y, hn = m(xd)
    torch.cuda.synchronize()
    fwd = GO.forward_quant(W, R, bw, br, xs, qp, training=False)
    np.testing.assert_array_equal(y.transpose(0, 1).cpu().numpy(), fwd["h"][1:], err_msg="PTQ h")
    np.testing.assert_array_equal(hn[0].cpu().numpy(), fwd["h"][-1], err_msg="PTQ h_n")
    # the same PTQ forward on the int32 carrier: every code equals the oracle's int32 carrier
    # (pinned code for code against the reference's compiled CPU carrier) and, where oracle/_ref
    # is present, the reference's own quantGRUForwardCPU run on the GPU's grids
    m.quant_storage_dtype = "int32"
    with torch.no_grad():
        yi, hni = m(xd)
    torch.cuda.synchronize()
    fi = GO.forward_int(W, R, bw, br, xs, qp, training=False)
    hi = GO.dequant_int(fi["h_q"], qp.g[A.GRID["h"]], False)
    np.testing.assert_array_equal(yi.transpose(0, 1).cpu().numpy(), hi[1:], err_msg="int32 h")
    np.testing.assert_array_equal(hni[0].cpu().numpy(), hi[-1], err_msg="int32 h_n")
    if GO.has_ref():
        ref = GO.ref_forward_int_codes(W, R, bw, br, xs, qp, with_v=False)
        np.testing.assert_array_equal(fi["h_q"], ref["h_q"], err_msg="oracle vs reference codes")
    # int codes in and out: forward_quantized on the input codes gives the same h codes
    meta = m.get_io_quant_meta()
    out_q, hn_q = m.forward_quantized(torch.from_numpy(fi["x_q"]).transpose(0, 1).to(cuda))
    np.testing.assert_array_equal(out_q.transpose(0, 1).cpu().numpy(), fi["h_q"][1:])
    np.testing.assert_array_equal(hn_q[0].cpu().numpy(), fi["h_q"][-1])
    assert meta["input"]["zp"] == qp.g[A.GRID["x"]].zero_point
    # the two carriers round their rescales differently; they stay within a few h steps
    steps = np.abs(yi.cpu().numpy() - y.cpu().numpy()) / meta["output"]["scale"]
    assert steps.max() <= 8, steps.max()
