"""QuantGRU on the int32 carrier on the GPU: quant_storage_dtype='int32' (calibrate -> QAT
forward -> backward, both directions, batch_first, hx) against the oracle's int32 carrier, and
forward_quantized (int codes in and out) against the int32-storage forward, as the reference's
test_cpu_ptq_integer_carrier_and_encoding_roundtrip (operators/quant-gru/tests/
test_cpu_ptq.py:35-77) checks it: the input quantised with get_io_quant_meta's grid, the
output codes dequantised with it, equal to the forward's output bit for bit.

Bars: forward outputs bit-exact; gradients within 1e-4 relative of the oracle's backward on
the int32 forward's saved tensors."""
import numpy as np
import pytest
import torch

import gru_oracle as GO
import gru_ops
import rxmet_gru_abi as A
from test_quant_gru_gpu import _haste, _module_case

pytestmark = pytest.mark.gpu
f32 = np.float32
CODES = ("W_q", "R_q", "bw_q", "br_q", "x_q")


def _fp_view(fwd, qp, H):
    """The int32 forward's saved tensors as the float-storage backward consumes them."""
    pot = bool(qp.use_pot2)
    out = {k: fwd[k].astype(f32) for k in CODES}
    out["h"] = GO.dequant_int(fwd["h_q"], qp.g[A.GRID["h"]], pot)
    v = np.empty(fwd["v_q"].shape, f32)
    for k, grid in enumerate(("update_gate_output", "reset_gate_output", "new_gate_output",
                              "weight_hh_linear")):
        v[..., k * H:(k + 1) * H] = GO.dequant_int(fwd["v_q"][..., k * H:(k + 1) * H],
                                                   qp.g[A.GRID[grid]], pot)
    out["v"] = v
    for k in GO.MASKS:
        out[k] = fwd[k]
    return out


def _set_cfg(m, cfg):
    if cfg == "16b-all":
        m.set_all_bitwidth(16, is_symmetric=False)


@pytest.mark.parametrize("bidirectional", [False, True])
@pytest.mark.parametrize("batch_first", [False, True])
@pytest.mark.parametrize("with_hx", [False, True])
@pytest.mark.parametrize("cfg", ["c3", "po2-16b", "16b-all"])
@pytest.mark.parametrize("shape", [(6, 24, 10, 32), (5, 12, 6, 33)], ids=str)
def test_module_int32_storage_matches_oracle(cuda, bidirectional, batch_first, with_hx, cfg,
                                             shape):
    print(f"[quantgru int32] bi={bidirectional} bf={batch_first} hx={with_hx} cfg={cfg} "
          f"shape={shape}", flush=True)
    m, x_tbi, hx = _module_case(bidirectional, batch_first, with_hx,
                                cfg if cfg != "16b-all" else "none", 23, shape=shape)
    _set_cfg(m, cfg)
    m.quant_storage_dtype = "int32"
    m = m.to(cuda)
    T, B, I = x_tbi.shape
    H = m.hidden_size
    D = 2 if bidirectional else 1
    x_in = (x_tbi.transpose(0, 1).contiguous() if batch_first else x_tbi).to(cuda)
    hx_d = hx.to(cuda) if hx is not None else None
    with m.calibration_context():
        m(x_in, hx_d)
    m.use_quantization = True
    m.train()
    x_leaf = x_in.clone().requires_grad_(True)
    hx_leaf = hx_d.clone().requires_grad_(True) if hx_d is not None else None
    out, hn = m(x_leaf, hx_leaf)
    g = torch.Generator().manual_seed(7)
    gout = torch.randn(out.shape, generator=g) * 1e-2
    ghn = torch.randn(hn.shape, generator=g) * 1e-2
    ((out * gout.to(cuda)).sum() + (hn * ghn.to(cuda)).sum()).backward()
    torch.cuda.synchronize()
    gout_tb = (gout.transpose(0, 1) if batch_first else gout).numpy()
    out_tb = (out.transpose(0, 1) if batch_first else out).detach().cpu().numpy()
    xn = x_tbi.numpy()
    dx_tot = np.zeros((T, B, I), np.float64)
    for d in range(D):
        sfx = "_reverse" if d else ""
        qp = (m.quant_params_reverse if d else m.quant_params).struct
        pn = lambda n: getattr(m, n + sfx).detach().cpu().numpy()
        W, R, bw, br = _haste(pn("weight_ih_l0"), pn("weight_hh_l0"), pn("bias_ih_l0"),
                              pn("bias_hh_l0"))
        xs = xn[::-1].copy() if d else xn
        h0 = hx[d].numpy() if hx is not None else None
        fwd = GO.forward_int(W, R, bw, br, xs, qp, h0=h0, training=True)
        fv = _fp_view(fwd, qp, H)
        o = fv["h"][1:][::-1] if d else fv["h"][1:]
        np.testing.assert_array_equal(out_tb[..., d * H:(d + 1) * H], o, err_msg=f"out dir{d}")
        np.testing.assert_array_equal(hn[d].detach().cpu().numpy(), fv["h"][-1],
                                      err_msg=f"h_n dir{d}")
        dh_new = np.zeros((T + 1, B, H), f32)
        gd = np.ascontiguousarray(gout_tb[..., d * H:(d + 1) * H])
        dh_new[1:] = gd[::-1] if d else gd
        dh_new[-1] += ghn[d].numpy()
        bwd = GO.backward_quant(fv, dh_new, qp)

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
    np.testing.assert_allclose(dx, dx_tot, rtol=1e-4, atol=1e-5 * float(np.abs(dx_tot).max()),
                               err_msg="dx")


def _codes(v, meta):
    lo = 0 if meta["is_unsigned"] else -(1 << (meta["bitwidth"] - 1))
    hi = (1 << meta["bitwidth"]) - 1 if meta["is_unsigned"] else (1 << (meta["bitwidth"] - 1)) - 1
    s = torch.tensor(meta["scale"], dtype=torch.float32)
    return (torch.round(v.float().cpu() / s) + meta["zp"]).clamp(lo, hi).to(torch.int32)


@pytest.mark.parametrize("bidirectional", [False, True])
@pytest.mark.parametrize("batch_first", [False, True])
@pytest.mark.parametrize("bits,pot2", [(8, False), (8, True), (16, False), (16, True)])
def test_forward_quantized_equals_int32_storage_forward(cuda, bidirectional, batch_first, bits,
                                                        pot2):
    print(f"[quantgru int io] bi={bidirectional} bf={batch_first} bits={bits} pot2={pot2}",
          flush=True)
    torch.manual_seed(39)
    from quant_gru import QuantGRU
    m = QuantGRU(3, 20, bidirectional=bidirectional, batch_first=batch_first).eval()
    m.set_all_bitwidth(bits, is_symmetric=False)
    if pot2:
        m.enable_pot2()
    m = m.to(cuda)
    D = 2 if bidirectional else 1
    x = torch.randn((2, 9, 3) if batch_first else (9, 2, 3)) * 0.3 + 0.15
    hx = torch.randn(D, 2, 20) * 0.2
    with m.calibration_context(), torch.no_grad():
        m(x.to(cuda), hx.to(cuda))
        m((x * 1.1).to(cuda), hx.to(cuda))
    m.use_quantization = True
    m.quant_storage_dtype = "int32"
    meta = m.get_io_quant_meta()
    assert set(meta) == {"input", "output", "hidden"} and meta["output"] == meta["hidden"]
    assert meta["input"]["bitwidth"] == bits

    def grid(d, name):
        # get_io_quant_meta describes the forward direction; a reverse direction has its own
        # h grid (calibrated on its own states), read the same way from quant_params_reverse
        if d == 0:
            return meta["input" if name == "x" else "hidden"]
        qp = m.quant_params_reverse
        e = dict(meta["input" if name == "x" else "hidden"])
        e["scale"] = float(gru_ops.decode_effective_scale(float(getattr(qp, f"scale_{name}_")),
                                                          bool(m.use_pot2_scale)))
        e["zp"] = int(getattr(qp, f"zp_{name}_"))
        return e

    assert all(grid(d, "x") == meta["input"] for d in range(D))  # both directions see x
    with torch.no_grad():
        y, hn = m(x.to(cuda), hx.to(cuda))
    hx_q = torch.stack([_codes(hx[d], grid(d, "h")) for d in range(D)])
    out_q, hn_q = m.forward_quantized(_codes(x, meta["input"]).to(cuda), hx_q.to(cuda))
    assert out_q.dtype == torch.int32 and out_q.shape == y.shape and hn_q.shape == hn.shape
    H = m.hidden_size
    for d in range(D):
        g = grid(d, "h")
        s = torch.tensor(g["scale"], dtype=torch.float32)
        for q, ref in ((out_q[..., d * H:(d + 1) * H], y[..., d * H:(d + 1) * H]),
                       (hn_q[d], hn[d])):
            deq = (q.float() - g["zp"]) * s
            np.testing.assert_array_equal(deq.cpu().numpy(), ref.cpu().numpy(), err_msg=f"dir{d}")
    with pytest.raises(TypeError, match="integer codes"):
        m.forward_quantized(x.to(cuda))


@pytest.mark.parametrize("with_hx", [False, True])
@pytest.mark.parametrize("cfg", ["c3", "po2-16b"])
@pytest.mark.parametrize("shape", [(7, 160, 12, 64), (6, 24, 10, 36), (5, 40, 8, 256)], ids=str)
def test_int32_inference_both_directions_in_one_call(cuda, with_hx, cfg, shape):
    """Bidirectional PTQ inference on the int32 carrier (eval, no autograd) runs both directions
    through rxmet_gru_forward_quant_int_dirs — one clustered recurrence launch for the two
    (H = 64: ten batch tiles, several per cluster; H = 256; H = 36, not a multiple of 16, steps
    each direction) — and assembles the output in the library: output and h_n equal the oracle's
    int32 carrier of each direction bit for bit, and the int-IO form equals it too."""
    print(f"[quantgru int32 bidir inference] hx={with_hx} cfg={cfg} shape={shape}", flush=True)
    m, x_tbi, hx = _module_case(True, False, with_hx, cfg, 29, shape=shape)
    m.quant_storage_dtype = "int32"
    m = m.to(cuda)
    x_in = x_tbi.to(cuda)
    hx_d = hx.to(cuda) if hx is not None else None
    with m.calibration_context():
        m(x_in, hx_d)
    m.use_quantization = True
    m.eval()
    with torch.no_grad():
        out, hn = m(x_in, hx_d)
    torch.cuda.synchronize()
    H = m.hidden_size
    xn = x_tbi.numpy()
    outn = out.cpu().numpy()
    for d in range(2):
        sfx = "_reverse" if d else ""
        qp = (m.quant_params_reverse if d else m.quant_params).struct
        pn = lambda n: getattr(m, n + sfx).detach().cpu().numpy()
        W, R, bw, br = _haste(pn("weight_ih_l0"), pn("weight_hh_l0"), pn("bias_ih_l0"),
                              pn("bias_hh_l0"))
        xs = xn[::-1].copy() if d else xn
        h0 = hx[d].numpy() if hx is not None else None
        fwd = GO.forward_int(W, R, bw, br, xs, qp, h0=h0, training=False)
        h = GO.dequant_int(fwd["h_q"], qp.g[A.GRID["h"]], bool(qp.use_pot2))
        o = h[1:][::-1] if d else h[1:]
        np.testing.assert_array_equal(outn[..., d * H:(d + 1) * H], o, err_msg=f"out dir{d}")
        np.testing.assert_array_equal(hn[d].cpu().numpy(), h[-1], err_msg=f"h_n dir{d}")
