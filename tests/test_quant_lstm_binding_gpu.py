"""The ``_quant_lstm`` drop-in driven the way the reference's autograd bridge drives its native
module (operators/quant-lstm/pytorch/lstm_autograd.py:139-258: the same positional argument
lists for lstm_forward_quantized and lstm_backward_qat, the 25 saved tensors in its order) and
the way its quant_lstm.py calibrates (CalibrationSession.collect / finalize -> bundle_json).

Bars: the bundle finalised by the session equals the QuantLSTM module's parameters; the
bridge's outputs equal the module's bit for bit and its gradients equal the module's (the
same kernels on the same inputs)."""
import json

import numpy as np
import pytest
import torch

import _quant_lstm as QL
import quant_lstm as Q

pytestmark = pytest.mark.gpu
_NAMES = ("weight_ih_linear", "weight_hh_linear", "gate_inputs", "gate_outputs", "cell_states",
          "cell_tanh_outputs", "hidden_outputs")


class _Bridge(torch.autograd.Function):
    """The reference bridge's call pattern over the drop-in module."""

    @staticmethod
    def forward(ctx, input, w_ih, w_hh, b_ih, b_hh, h0, c0, batch_first, bundle_json):
        out, hn, cn, ck, safety = QL.lstm_forward_quantized(
            input, w_ih, w_hh, b_ih, b_hh, h0, c0, batch_first, bundle_json, "pedantic", False,
            True)
        assert safety["has_precision_risk"] is False
        m, mm, vals, cm = (ck["quantized_master"], ck["master_clamp_masks"], ck["values"],
                           ck["clamp_masks"])
        empty = input.new_empty(0)
        empty_mask = torch.empty(0, dtype=torch.bool, device=input.device)
        ctx.save_for_backward(
            m["input"], m["weight_ih"], m["weight_hh"], m.get("bias_ih", empty),
            m.get("bias_hh", empty), m["h_0"], m["c_0"], mm["input"], mm["weight_ih"],
            mm["weight_hh"], mm.get("bias_ih", empty_mask), mm.get("bias_hh", empty_mask),
            mm["h_0"], mm["c_0"], vals["gate_outputs"], vals["cell_states"],
            vals["cell_tanh_outputs"], vals["hidden_outputs"], *(cm[n] for n in _NAMES))
        ctx.bundle_json, ctx.batch_first = bundle_json, batch_first
        ctx.has_bias, ctx.has_state = b_ih is not None, h0 is not None
        return out, hn, cn

    @staticmethod
    def backward(ctx, g_out, g_h, g_c):
        s = ctx.saved_tensors
        hid = s[17]
        g_tm = torch.zeros_like(hid) if g_out is None else \
            (g_out.transpose(0, 1) if ctx.batch_first else g_out).contiguous()
        g_h = torch.zeros_like(s[5])[0] if g_h is None else g_h[0]
        g_c = torch.zeros_like(s[6])[0] if g_c is None else g_c[0]
        g = QL.lstm_backward_qat(list(s[:7]), ctx.batch_first, ctx.bundle_json, list(s[14:18]),
                                 g_tm, g_h, g_c, list(s[7:14]), list(s[18:25]))
        return (g[0], g[1], g[2], g[3] if ctx.has_bias else None, g[4] if ctx.has_bias else None,
                g[5].unsqueeze(0) if ctx.has_state else None,
                g[6].unsqueeze(0) if ctx.has_state else None, None, None)


@pytest.mark.parametrize("batch_first", [False, True])
@pytest.mark.parametrize("with_state", [False, True])
@pytest.mark.parametrize("bias", [True, False])
@pytest.mark.parametrize("H,cfg", [(32, None), (33, {"schema_version": 1, "operators": {
    "cell_state": {"bitwidth": 16}, "weight_hh": {"bitwidth": 16}}})], ids=["h32", "h33-16b"])
def test_bridge_pattern_matches_quantlstm(cuda, batch_first, with_state, bias, H, cfg):
    print(f"[lstm bridge] bf={batch_first} state={with_state} bias={bias} H={H}", flush=True)
    T, B, I = 6, 9, 7
    torch.manual_seed(5)
    m = Q.QuantLSTM(I, H, bias=bias, batch_first=batch_first, quant_config=cfg).to(cuda)
    g = torch.Generator().manual_seed(6)
    shape = (B, T, I) if batch_first else (T, B, I)
    xs = [(torch.randn(shape, generator=g) * s).to(cuda) for s in (1.0, 1.3)]
    st = None
    if with_state:
        st = tuple((torch.randn(1, B, H, generator=g) * 0.4).to(cuda) for _ in range(2))
    # calibration: the session of the reference's quant_lstm.py vs the module
    resolved = QL._canonical_config(m._config)
    sess = QL.CalibrationSession(resolved, I, H, bias, "minmax", 99.99)
    w = (m.weight_ih_l0, m.weight_hh_l0, m.bias_ih_l0 if bias else None,
         m.bias_hh_l0 if bias else None)
    m.calibrating = True
    for x in xs:
        with torch.no_grad():
            y_cal, (h_cal, c_cal) = m(x, st)
        y_s, h_s, c_s = sess.collect(x, *w, st[0] if st else None, st[1] if st else None,
                                     batch_first)
        assert torch.equal(y_s, y_cal) and torch.equal(h_s, h_cal) and torch.equal(c_s, c_cal)
    m.calibrating = False
    m.finalize_calibration()
    assert sess.state == "dirty" and sess.batch_count == 2
    fin = sess.finalize()
    assert sess.state == "locked" and fin["method"] == "minmax" and fin["batch_count"] == 2
    assert fin["resolved_config_json"] == resolved
    assert set(fin["activation_ranges"]) == set(Q.OPERATORS) - Q.PARAMETER_OPERATORS
    bundle = fin["bundle_json"]
    b = QL._import_bundle(bundle)
    p = m._params[0]
    for name in Q.OPERATORS:
        if name in Q.PARAMETER_OPERATORS:
            if bias or not name.startswith("bias"):
                np.testing.assert_array_equal(b.params.channel_scales(name),
                                              p.channel_scales(name), err_msg=name)
        else:
            assert (b.params.scale(name), b.params.zero_point(name)) == \
                (p.scale(name), p.zero_point(name)), name
    assert json.loads(bundle)["hidden_size"] == H
    # QAT step through the bridge and through the module
    m.use_quantization = True
    m.train()
    go = torch.randn(xs[0].shape[:-1] + (H,), generator=g).to(cuda)
    gh = torch.randn(1, B, H, generator=g).to(cuda)

    def run(use_bridge):
        m.zero_grad(set_to_none=True)
        x = xs[0].clone().requires_grad_(True)
        s = tuple(t.clone().requires_grad_(True) for t in st) if st else None
        if use_bridge:
            out, hn, cn = _Bridge.apply(x, *w, s[0] if s else None, s[1] if s else None,
                                        batch_first, bundle)
        else:
            out, (hn, cn) = m(x, s)
        ((out * go).sum() + (hn * gh).sum() + cn.sum()).backward()
        grads = [x.grad] + [t.grad for t in w if t is not None] + ([t.grad for t in s] if s else [])
        return [out.detach(), hn.detach(), cn.detach()] + grads

    ref = run(False)
    got = run(True)
    for k, (a, e) in enumerate(zip(got, ref)):
        assert torch.equal(a, e), f"tensor {k}: max diff {(a - e).abs().max().item()}"
