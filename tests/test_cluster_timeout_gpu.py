"""Failure handling of the clustered recurrences: a cluster barrier wait that gives up.

The condition is forced from the host: RXMET_TEST_SPIN_LIMIT=0 makes every wait that has to
poll give up at once (the bounded wait of rx-met_amd/csrc/cluster.h), so the launch takes the
path of a real timeout — the flag is raised, the members stop stepping and every wave still
reaches the end of its kernel.  Nothing hangs and nothing faults.  Then:

* forward: every output of the launch is NaN (output and h_n; LSTM output, h_n, c_n);
* backward (forward run normally, the limit forced for the backward only): every gradient of
  the poison list is NaN — dx, dW_ih, dW_hh, db_ih, db_hh of every direction;
* with the normal limit again the next step reproduces the first step bit for bit, so a
  timeout leaves nothing behind (counters and flags are reset by every launch).

Shapes are small but clustered: H = 256 gives clusters of several members (a cluster of one
member never waits for another)."""
import numpy as np
import pytest
import torch

import quant_gru as QG
import quant_lstm as QL

pytestmark = pytest.mark.gpu


def _step(m, x, limit_fwd, limit_bwd, monkeypatch):
    def limit(v):
        if v is None:
            monkeypatch.delenv("RXMET_TEST_SPIN_LIMIT", raising=False)
        else:
            monkeypatch.setenv("RXMET_TEST_SPIN_LIMIT", str(v))
    m.zero_grad(set_to_none=True)
    xl = x.clone().requires_grad_(True)
    limit(limit_fwd)
    out = m(xl)
    torch.cuda.synchronize()
    limit(limit_bwd)
    out[0].sum().backward()
    torch.cuda.synchronize()
    limit(None)
    grads = {"dx": xl.grad.detach().clone()}
    for n, p in m.named_parameters():
        grads[n] = p.grad.detach().clone()
    outs = [out[0].detach().clone()] + [t.detach().clone() for t in
                                       (out[1] if isinstance(out[1], tuple) else (out[1],))]
    return outs, grads


def _gru(cuda):
    T, B, I, H = 16, 32, 16, 256
    torch.manual_seed(3)
    x = torch.randn(T, B, I).to(cuda)
    m = QG.QuantGRU(I, H, bidirectional=True)
    m.set_all_bitwidth(8, is_symmetric=False)
    m = m.to(cuda)
    with m.calibration_context():
        m(x)
    m.use_quantization = True
    m.train()
    return m, x


def _lstm(cuda):
    T, B, I, H = 12, 32, 16, 256
    torch.manual_seed(4)
    x = (torch.rand(T, B, I) * 2 - 1).to(cuda)
    m = QL.QuantLSTM(I, H).to(cuda)
    m.calibrating = True
    with torch.no_grad():
        m(x)
    m.calibrating = False
    m.finalize_calibration()
    m.use_quantization = True
    m.train()
    return m, x


@pytest.mark.parametrize("model", ["gru", "lstm"])
def test_forced_cluster_timeout_poisons_and_recovers(cuda, model, monkeypatch):
    print(f"[cluster timeout] {model}", flush=True)
    m, x = (_gru if model == "gru" else _lstm)(cuda)
    outs0, grads0 = _step(m, x, None, None, monkeypatch)
    for t in outs0 + list(grads0.values()):
        assert torch.isfinite(t).all()

    # forward timed out: every output NaN
    outs1, _ = _step(m, x, 0, None, monkeypatch)
    for k, t in enumerate(outs1):
        assert torch.isnan(t).all(), f"forward output {k} not poisoned"

    # forward normal, backward timed out: every gradient NaN
    outs2, grads2 = _step(m, x, None, 0, monkeypatch)
    for a, b in zip(outs2, outs0):
        assert torch.equal(a, b)
    for k, g in grads2.items():
        assert torch.isnan(g).all(), f"gradient {k} not poisoned"

    # the normal limit again: the first step bit for bit
    outs3, grads3 = _step(m, x, None, None, monkeypatch)
    for a, b in zip(outs3, outs0):
        assert torch.equal(a, b)
    for k in grads0:
        assert torch.equal(grads3[k], grads0[k]), k


def test_forced_timeout_int32_carrier_forward(cuda, monkeypatch):
    print("[cluster timeout] gru int32 carrier", flush=True)
    m, x = _gru(cuda)
    m.quant_storage_dtype = "int32"
    m.eval()
    with torch.no_grad():
        ref = m(x)
        monkeypatch.setenv("RXMET_TEST_SPIN_LIMIT", "0")
        bad = m(x)
        torch.cuda.synchronize()
        monkeypatch.delenv("RXMET_TEST_SPIN_LIMIT")
        again = m(x)
    assert torch.isfinite(ref[0]).all()
    assert torch.isnan(bad[0]).all() and torch.isnan(bad[1]).all()
    assert torch.equal(again[0], ref[0]) and torch.equal(again[1], ref[1])
    assert np.isfinite(again[0].cpu().numpy()).all()
