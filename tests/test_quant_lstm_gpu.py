"""QuantLSTM module on the GPU against the oracle: calibrate, then QAT forward (bit-exact) and
backward (1e-4 relative) per direction, for uni/bidirectional, batch_first and given state;
plus the float path against torch.nn.LSTM and the training / inference equivalence."""
import numpy as np
import pytest
import torch

import lstm_oracle as O
import quant_lstm as Q

pytestmark = pytest.mark.gpu
f32 = np.float32

C4 = {"schema_version": 1,
      "operators": {**{n: {"is_symmetric": False} for n in Q.OPERATORS
                       if n not in Q.PARAMETER_OPERATORS},
                    "cell_state": {"bitwidth": 16, "is_symmetric": False}}}


def _module(cuda, I, H, bidirectional, batch_first, bias=True, cfg=None, seed=0):
    torch.manual_seed(seed)
    m = Q.QuantLSTM(I, H, bias=bias, batch_first=batch_first, bidirectional=bidirectional,
                    quant_config=cfg).to(cuda)
    return m


def _calibrate(m, x, hx=None):
    m.calibrating = True
    with torch.no_grad():
        m(x, hx)
    m.calibrating = False
    m.finalize_calibration()
    m.use_quantization = True


def _np(t):
    return t.detach().cpu().numpy()


@pytest.mark.parametrize("bidirectional", [False, True])
@pytest.mark.parametrize("batch_first", [False, True])
@pytest.mark.parametrize("with_state", [False, True])
@pytest.mark.parametrize("cfg", [None, C4])
@pytest.mark.parametrize("H", [32, 33])
def test_module_qat_matches_oracle(cuda, bidirectional, batch_first, with_state, cfg, H):
    T, B, I = 5, 18, 7
    print(f"[quantlstm module] bi={bidirectional} bf={batch_first} state={with_state} "
          f"cfg={cfg is not None} H={H}", flush=True)
    D = 2 if bidirectional else 1
    m = _module(cuda, I, H, bidirectional, batch_first, cfg=cfg)
    g = torch.Generator().manual_seed(3)
    xt = torch.rand((T, B, I), generator=g) * 2 - 1
    x = (xt.transpose(0, 1).contiguous() if batch_first else xt).to(cuda)
    hx = None
    if with_state:
        hx = ((torch.randn((D, B, H), generator=g) * 0.3).to(cuda),
              (torch.randn((D, B, H), generator=g) * 0.5).to(cuda))
    _calibrate(m, x, hx)
    m.train()
    x.requires_grad_(True)
    if hx is not None:
        hx = tuple(t.clone().requires_grad_(True) for t in hx)
    out, (hn, cn) = m(x, hx)
    assert out.shape == ((B, T, D * H) if batch_first else (T, B, D * H))
    go = torch.randn(out.shape, generator=g) * 0.1
    gh = torch.randn(hn.shape, generator=g) * 0.1
    gc = torch.randn(cn.shape, generator=g) * 0.1
    loss = (out * go.to(cuda)).sum() + (hn * gh.to(cuda)).sum() + (cn * gc.to(cuda)).sum()
    loss.backward()
    out_tm = _np(out.transpose(0, 1) if batch_first else out)
    go_tm = (go.transpose(0, 1) if batch_first else go).numpy()
    gx_tm = _np(x.grad.transpose(0, 1) if batch_first else x.grad)
    gx_exp = np.zeros_like(gx_tm)
    for d in range(D):
        Wi, Wh, bi, bh = (_np(p) for p in m._direction_params(d == 1))
        xd = xt.numpy()[::-1].copy() if d == 1 else xt.numpy()
        h0 = _np(hx[0][d]) if hx is not None else None
        c0 = _np(hx[1][d]) if hx is not None else None
        p = m._params[d].struct
        o = O.forward_quant(Wi, Wh, bi, bh, xd, p, h0, c0, mode=O.ACT_LIBM_EXACT)
        od = out_tm[..., d * H:(d + 1) * H]
        np.testing.assert_array_equal(od[::-1] if d == 1 else od, o["output"])
        np.testing.assert_array_equal(_np(hn[d]), o["h_n"])
        np.testing.assert_array_equal(_np(cn[d]), o["c_n"])
        god = go_tm[..., d * H:(d + 1) * H]
        god = god[::-1].copy() if d == 1 else god
        gr = O.backward_quant(o, p, god, gh[d].numpy(), gc[d].numpy())
        gx_exp += gr["dx"][::-1] if d == 1 else gr["dx"]
        sfx = "_reverse" if d == 1 else ""
        for name, key in (("weight_ih_l0", "dW_ih"), ("weight_hh_l0", "dW_hh"),
                          ("bias_ih_l0", "db_ih"), ("bias_hh_l0", "db_hh")):
            got = _np(getattr(m, name + sfx).grad)
            e = gr[key]
            np.testing.assert_allclose(got, e, rtol=1e-4, atol=1e-5 * max(np.abs(e).max(), 1e-30),
                                       err_msg=name + sfx)
        if hx is not None:
            for t, key in ((hx[0], "dh0"), (hx[1], "dc0")):
                e = gr[key]
                np.testing.assert_allclose(_np(t.grad[d]), e, rtol=1e-4,
                                           atol=1e-5 * max(np.abs(e).max(), 1e-30), err_msg=key)
    np.testing.assert_allclose(gx_tm, gx_exp, rtol=1e-4, atol=1e-5 * np.abs(gx_exp).max())
    st = m.qat_saved_state()
    st = st["forward"] if bidirectional else st
    assert set(st) == {"quantized_master", "master_clamp_masks", "checkpoints",
                       "checkpoint_clamp_masks"}
    assert st["checkpoint_clamp_masks"]["gate_inputs"].dtype == torch.bool


def test_eval_no_grad_matches_training_forward(cuda):
    T, B, I, H = 4, 16, 8, 48
    m = _module(cuda, I, H, True, True)
    x = (torch.rand((B, T, I)) * 2 - 1).to(cuda)
    _calibrate(m, x)
    m.train()
    out, (hn, cn) = m(x)
    assert m.qat_saved_state() is not None
    m.eval()
    with torch.no_grad():
        out2, (hn2, cn2) = m(x)
    assert m.qat_saved_state() is None
    assert torch.equal(out, out2) and torch.equal(hn, hn2) and torch.equal(cn, cn2)


def test_export_import_reproduces_outputs(cuda, tmp_path):
    T, B, I, H = 4, 16, 8, 32
    m = _module(cuda, I, H, True, False, cfg=C4)
    x = (torch.rand((T, B, I)) * 2 - 1).to(cuda)
    _calibrate(m, x)
    m.eval()
    with torch.no_grad():
        ref = m(x)[0]
    m.export_quant_params(tmp_path / "qp.json")
    m2 = _module(cuda, I, H, True, False, cfg=C4)
    m2.load_state_dict(m.state_dict())
    m2.load_quant_params(tmp_path / "qp.json")
    m2.use_quantization = True
    m2.eval()
    with torch.no_grad():
        got = m2(x)[0]
    assert torch.equal(ref, got)


def test_float_path_matches_torch_lstm(cuda):
    T, B, I, H = 6, 5, 9, 32
    m = _module(cuda, I, H, True, True)
    ref = torch.nn.LSTM(I, H, batch_first=True, bidirectional=True).double()
    with torch.no_grad():
        for name, p in m.named_parameters():
            getattr(ref, name).copy_(p.detach().cpu().double())
    x = torch.rand((B, T, I)) * 2 - 1
    h0 = torch.randn((2, B, H)) * 0.3
    c0 = torch.randn((2, B, H)) * 0.3
    with torch.no_grad():
        out, (hn, cn) = m(x.to(cuda), (h0.to(cuda), c0.to(cuda)))
        ro, (rh, rc) = ref(x.double(), (h0.double(), c0.double()))
    np.testing.assert_allclose(_np(out), ro.numpy(), rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(_np(hn), rh.numpy(), rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(_np(cn), rc.numpy(), rtol=1e-4, atol=1e-5)
    out = m(x.to(cuda))[0]
    with pytest.raises(NotImplementedError):
        out.sum().backward()


def test_calibration_accumulates_batches_and_locks(cuda):
    T, B, I, H = 3, 16, 4, 16
    m = _module(cuda, I, H, False, False)
    x1 = (torch.rand((T, B, I)) * 2 - 1).to(cuda)
    x2 = x1 * 2
    m.calibrating = True
    with torch.no_grad():
        m(x1)
        m(x2)
    m.calibrating = False
    assert m.calibration_state() == "dirty"
    rep = m.finalize_calibration()
    assert rep["batch_count"] == 2
    assert m.calibration_state() == "locked"
    assert m._params[0].scale("input") > 0
    # x2 doubled the input range: the input scale covers it
    assert m._params[0].scale("input") * 127 >= float(x2.abs().max()) * (1 - 1e-6)
    m.set_quant_params_locked(True)
    assert m.quant_params_locked()
    m.reset_calibration()
    assert not m.is_calibrated() and not m.quant_params_locked()
