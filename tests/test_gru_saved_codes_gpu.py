"""Saved state as codes (rxmet_gru_forward_quant_dirs_codes / rxmet_gru_backward_quant_dirs_codes,
the module path's format): the saved codes decode to the reference-format v and masks exactly,
and every output and gradient equals the reference-format entry points' bit for bit, on the
clustered, stepped and per-tile recurrences."""
import numpy as np
import pytest
import torch

import gru_ops
import quant_gru as QG
import rxmet_gru_abi as A
import rxmet_lib
from test_gru_gpu import _case

pytestmark = pytest.mark.gpu
f32 = np.float32

# (T, B, I, H, config): clustered both ways; 16-bit h; H > 256 (stepped backward); 12-bit R
# (stepped forward and backward); a batch that is not a multiple of the 16-row tile
CASES = [(5, 40, 9, 64, "c3"), (4, 37, 16, 48, "16b-act-pot2"), (3, 20, 8, 320, "c3"),
         (4, 33, 5, 64, "r12-pot2"), (3, 300, 16, 256, "8b-asym")]


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _decode(vc, mb, qp, B, H):
    """Reference-format v [T, B, 4H] and the five per-step masks from the blocked saved codes."""
    st = qp.struct
    pot = int(st.use_pot2)
    vc = np.ascontiguousarray(gru_ops.unblock_codes(vc, B, H, 4))
    mb = np.ascontiguousarray(gru_ops.unblock_codes(mb, B, H, 1))
    v = np.empty(vc.shape, f32)
    raw = vc.view(np.uint16).astype(f32)
    for q, name in enumerate(("update_gate_output", "reset_gate_output", "new_gate_output",
                              "weight_hh_linear")):
        g = st.g[A.GRID[name]]
        lo = 0 if g.is_unsigned else -(1 << (int(g.bits) - 1))
        eff = f32(rxmet_lib.load().rxmet_gru_effective_scale(g.scale, pot))
        v[..., q * H:(q + 1) * H] = (raw[..., q * H:(q + 1) * H] - f32(g.zero_point - lo)) * eff
    bits = mb.view(np.uint16).astype(np.uint32)
    bit = lambda k: ((bits >> k) & 1).astype(np.uint8)
    fam = lambda k0: np.concatenate([bit(k0 + g) for g in range(3)], axis=-1)  # [T, B, 3H]
    return v, {"ih": fam(0), "hh": fam(3), "gin": fam(6), "gout": fam(9), "h": bit(12)}


@pytest.mark.parametrize("case", CASES)
def test_saved_codes_decode_to_reference_format_and_gradients_equal(cuda, case):
    T, B, I, H, cfg = case
    args = []
    for d in range(2):
        W, R, bw, br, x, h0, qp = _case(T, B, I, H, cfg, 21 + d, d == 1)
        args.append((_t(W, cuda), _t(R, cuda), _t(bw, cuda), _t(br, cuda), _t(x, cuda),
                     _t(h0, cuda) if h0 is not None else torch.empty(0, device=cuda),
                     gru_ops.GRUQuantParams.from_struct(qp)))
    ref = gru_ops.forward_quant_float_storage_dirs(True, T, B, I, H, args)
    cod = gru_ops.forward_quant_codes_dirs(True, T, B, I, H, args)
    torch.cuda.synchronize()
    g = np.random.default_rng(5)
    bref, bcod = [], []
    for d in range(2):
        (h, v, W_q, R_q, bw_q, br_q, x_q, *masks) = ref[d]
        (hc, vc, W_qc, R_qc, bw_qc, br_qc, x_qc, *cm) = cod[d]
        assert len(cm) == 7 and vc.dtype == torch.int16 and cm[6].dtype == torch.int16
        for name, a, b in (("h", h, hc), ("W_q", W_q, W_qc), ("R_q", R_q, R_qc), ("bw_q", bw_q, bw_qc),
                           ("br_q", br_q, br_qc), ("x_q", x_q, x_qc)):
            assert torch.equal(a, b), (d, name)
        for k in range(6):  # x, h0, W, R, bw, br masks
            assert torch.equal(masks[k], cm[k]), (d, k)
        vd, md = _decode(vc.cpu().numpy(), cm[6].cpu().numpy(), args[d][6], B, H)
        np.testing.assert_array_equal(vd.view(np.uint32), v.cpu().numpy().view(np.uint32),
                                      err_msg=f"direction {d}: v")
        for k, name in zip(range(6, 11), ("ih", "hh", "gin", "gout", "h")):
            np.testing.assert_array_equal(md[name], masks[k].cpu().numpy(),
                                          err_msg=f"direction {d}: {name} mask")
        dh = _t((g.standard_normal((T + 1, B, H)) * 1e-2).astype(f32), cuda)
        bref.append((W_q, R_q, bw_q, br_q, x_q, dh, h, v, args[d][6], masks))
        bcod.append((W_qc, R_qc, bw_qc, br_qc, x_qc, dh, hc, vc, args[d][6], cm))
    gr = gru_ops.backward_quant_float_storage_dirs(T, B, I, H, bref)
    gc = gru_ops.backward_quant_codes_dirs(T, B, I, H, bcod, torch_layout=False)
    torch.cuda.synchronize()
    for d in range(2):
        for name, a, b in zip(("dx", "dW", "dR", "dbw", "dbr", "dh0"), gr[d], gc[d]):
            assert torch.equal(a, b), (d, name, float((a - b).abs().max()))


@pytest.mark.parametrize("bidirectional", [False, True])
@pytest.mark.parametrize("loss", ["square_mean", "sum"])
def test_module_gradients_equal_with_and_without_saved_codes(cuda, monkeypatch, bidirectional,
                                                             loss):
    """QuantGRU training step (c3 grids) with the saved state as codes (dh read in place from the
    output gradient: a dense one, and the zero-stride one of a sum) and in the reference format
    (dh_new built by copies): output and every parameter and input gradient bit for bit."""
    torch.manual_seed(3)
    T, B, I, H = 6, 37, 12, 64
    m = QG.QuantGRU(I, H, batch_first=True, bidirectional=bidirectional)
    m.set_all_bitwidth(8, is_symmetric=False)
    m._bitwidth_config.h_ = 16
    m = m.to(cuda)
    x = torch.randn(B, T, I, device=cuda)
    h0 = torch.randn(2 if bidirectional else 1, B, H, device=cuda) * 0.3
    with m.calibration_context():
        m(x)
    m.use_quantization = True
    m.train()
    res = []
    for codes in (True, False):
        monkeypatch.setattr(QG, "SAVE_STATE_AS_CODES", codes)
        m.zero_grad(set_to_none=True)
        xl = x.clone().requires_grad_(True)
        hl = h0.clone().requires_grad_(True)
        out, hn = m(xl, hl)
        if loss == "sum":
            (out.sum() + 0.5 * hn.sum()).backward()
        else:
            (out.square().mean() + hn.sum()).backward()
        torch.cuda.synchronize()
        res.append([out.detach(), hn.detach(), xl.grad, hl.grad] +
                   [p.grad.clone() for p in m.parameters()])
    for k, (a, b) in enumerate(zip(*res)):
        assert torch.equal(a, b), (k, float((a - b).abs().max()))


def test_saved_codes_refuse_wide_grids(cuda):
    """Gate output grids over 16 bits cannot be saved as 16-bit codes: the entry point refuses
    (the module keeps the reference format for them)."""
    T, B, I, H = 2, 16, 4, 16
    W, R, bw, br, x, h0, qp = _case(T, B, I, H, "c3", 3, False)
    qp.g[A.GRID["update_gate_output"]].bits = 20
    args = [(_t(W, cuda), _t(R, cuda), _t(bw, cuda), _t(br, cuda), _t(x, cuda),
             torch.empty(0, device=cuda), gru_ops.GRUQuantParams.from_struct(qp))]
    with pytest.raises(rxmet_lib.RxmetError, match="at most 16 bits"):
        gru_ops.forward_quant_codes_dirs(True, T, B, I, H, args)
    assert not QG._codes_fit(args[0][6])
