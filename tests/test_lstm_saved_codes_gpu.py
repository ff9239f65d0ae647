"""Saved state as codes for QuantLSTM (rxmet_lstm_forward_quant_codes /
rxmet_lstm_backward_quant_codes, the module path's format): the saved codes decode to the
reference-format checkpoints and masks exactly, and every output and gradient equals the
reference-format entry points' bit for bit, on the clustered, per-tile and stepped recurrences."""
import numpy as np
import pytest
import torch

import lstm_ops
import quant_lstm as QL
import rxmet_lib
import rxmet_lstm_abi as L
from test_lstm_gpu import _case, _dev, _wrap

pytestmark = pytest.mark.gpu

# (T, B, I, H, config, bias, state): clustered forward and backward (H % 128 == 0), a batch
# off the 16-row tile, the c4 grids (16-bit cell), H = 48 (per-tile forward, stepped-free
# backward), 16-bit W_hh (stepped recurrences), 16-bit activations with an unsigned h
CASES = [(5, 40, 9, 128, "default", True, False), (4, 37, 16, 256, "c4", True, True),
         (3, 20, 8, 48, "default", False, True), (4, 33, 5, 64, "16b-whh", True, False),
         (3, 18, 6, 128, "16b-act", True, True)]


@pytest.mark.parametrize("case", CASES)
def test_saved_codes_decode_to_reference_format_and_gradients_equal(cuda, case):
    T, B, I, H, cfg, bias, state = case
    args, _, p = _case(T, B, I, H, cfg, 31, bias, state)
    Wi, Wh, bi, bh, x, h0, c0 = (_dev(a, cuda) for a in args)
    prm = _wrap(p)
    ref = lstm_ops.forward_quant(x, Wi, Wh, bi, bh, h0, c0, prm, True)
    cod = lstm_ops.forward_quant(x, Wi, Wh, bi, bh, h0, c0, prm, True, codes=True)
    torch.cuda.synchronize()
    for k in range(3):  # output, h_n, c_n
        assert torch.equal(ref[k], cod[k]), k
    sr, sc = ref[3], cod[3]
    assert "codes_blocks" in sc and "gate_out" not in sc
    for k in sr:
        if k in sc:
            assert torch.equal(sr[k], sc[k]), k
    dec = lstm_ops.decode_saved_codes(sc, prm, B)
    for k in lstm_ops.CODED_FIELDS:
        a, b = sr[k].cpu().numpy(), dec[k].cpu().numpy()
        np.testing.assert_array_equal(a.view(np.uint8) if a.dtype == np.uint8 else a.view(np.uint32),
                                      b.view(np.uint8) if b.dtype == np.uint8 else b.view(np.uint32),
                                      err_msg=k)
    g = torch.from_numpy(np.random.default_rng(3).standard_normal((T, B, H)).astype(np.float32) * 0.1)
    ghn = torch.from_numpy(np.random.default_rng(4).standard_normal((B, H)).astype(np.float32) * 0.1)
    g, ghn = g.to(cuda), ghn.to(cuda)
    gr = lstm_ops.backward_quant(sr, prm, g, ghn, ghn * 0.5)
    gc = lstm_ops.backward_quant(sc, prm, g, ghn, ghn * 0.5)
    torch.cuda.synchronize()
    for name, a, b in zip(("dx", "dW_ih", "dW_hh", "db_ih", "db_hh", "dh0", "dc0"), gr, gc):
        if a is None:
            assert b is None
            continue
        assert torch.equal(a, b), (name, float((a - b).abs().max()))


@pytest.mark.parametrize("bidirectional", [False, True])
def test_module_gradients_and_qat_state_equal_with_and_without_saved_codes(cuda, monkeypatch,
                                                                          bidirectional):
    torch.manual_seed(5)
    T, B, I, H = 6, 35, 12, 128
    m = QL.QuantLSTM(I, H, bidirectional=bidirectional,
                     quant_config={"schema_version": 1,
                                   "operators": {"cell_state": {"bitwidth": 16}}}).to(cuda)
    x = torch.rand(T, B, I, device=cuda) * 2 - 1
    m.calibrating = True
    with torch.no_grad():
        m(x)
    m.calibrating = False
    m.finalize_calibration()
    m.use_quantization = True
    m.train()
    res, states = [], []
    for codes in (True, False):
        monkeypatch.setattr(QL, "SAVE_STATE_AS_CODES", codes)
        m.zero_grad(set_to_none=True)
        xl = x.clone().requires_grad_(True)
        out, (hn, cn) = m(xl)
        (out.square().mean() + hn.sum() + 0.5 * cn.sum()).backward()
        torch.cuda.synchronize()
        res.append([out.detach(), hn.detach(), cn.detach(), xl.grad] +
                   [q.grad.clone() for q in m.parameters()])
        states.append(m.qat_saved_state())
    for k, (a, b) in enumerate(zip(*res)):
        assert torch.equal(a, b), (k, float((a - b).abs().max()))

    def flat(d, pre=""):
        for k, v in d.items():
            if isinstance(v, dict):
                yield from flat(v, pre + k + ".")
            elif v is not None:
                yield pre + k, v
    a, b = dict(flat(states[0])), dict(flat(states[1]))
    assert a.keys() == b.keys()
    for k in a:
        assert torch.equal(a[k], b[k]), k


def test_saved_codes_refuse_wide_grids(cuda):
    T, B, I, H = 2, 16, 4, 16
    args, _, p = _case(T, B, I, H, "default", 3, True, False)
    p.config.op[L.OP["cell_state"]].bits = 20
    prm = _wrap(p)
    assert not lstm_ops.codes_fit(prm)
    Wi, Wh, bi, bh, x, h0, c0 = (_dev(a, cuda) for a in args)
    with pytest.raises(rxmet_lib.RxmetError):
        lstm_ops.forward_quant(x, Wi, Wh, bi, bh, h0, c0, prm, True, codes=True)
