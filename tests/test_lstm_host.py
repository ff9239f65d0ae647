"""Host-side QuantLSTM logic of librxmet.so (parameter finalisation and the derived integer
execution encodings, rx-met_amd/csrc/lstm_params.cpp) against the pinned oracle.  These calls
need no GPU."""
import ctypes

import numpy as np
import pytest
import torch

import lstm_ops
import lstm_oracle as O
import rxmet_lib
import rxmet_lstm_abi as L

f32 = np.float32


def _stats(I, H, seed, bias=True, state=False):
    g = np.random.default_rng(seed)
    k = 1.0 / np.sqrt(H)
    u = lambda *s: ((g.random(s) * 2 - 1) * k).astype(f32)
    Wi, Wh = u(4 * H, I), u(4 * H, H)
    bi, bh = (u(4 * H), u(4 * H)) if bias else (None, None)
    x = (g.random((4, 3, I)) * 2 - 1).astype(f32)
    h0 = (g.standard_normal((3, H)) * 0.3).astype(f32) if state else None
    c0 = (g.standard_normal((3, H)) * 0.5).astype(f32) if state else None
    return O.calibrate(Wi, Wh, bi, bh, x, h0, c0)


def _config(name):
    c = L.default_config()
    if name == "c4":
        for k in range(L.NOPS):
            if L.OP_NAMES[k] not in L.PARAM_OPS:
                c.op[k].is_symmetric = 0
        c.op[L.OP["cell_state"]].bits = 16
    elif name == "pot2-gate":
        c.scale_mode = L.POT2
        for n in L.PARAM_OPS:
            c.op[L.OP[n]].granularity = L.PER_GATE
        c.op[L.OP["output"]].is_symmetric = 0
    elif name == "16b-tensor":
        for k in range(L.NOPS):
            c.op[k].bits = 16
            if L.OP_NAMES[k] in L.PARAM_OPS:
                c.op[k].granularity = L.PER_TENSOR
    elif name == "4b-pot2":
        c.scale_mode = L.POT2
        for k in range(L.NOPS):
            c.op[k].bits = 4 if L.OP_NAMES[k] in L.PARAM_OPS else 8
    return c


def _product_exec(p, I):
    C = 4 * p.hidden
    acc = (L.Rescale * (2 * C))()
    bias = (L.Rescale * (2 * C))()
    gate = (L.Rescale * 8)()
    cell = (L.Q31 * 2)()
    hid = (L.Rescale * 1)()
    rxmet_lib.call("rxmet_lstm_derive_exec", ctypes.byref(p), I, ctypes.addressof(acc),
                   ctypes.addressof(bias), ctypes.addressof(gate), ctypes.addressof(cell),
                   ctypes.addressof(hid))

    def rs(arr):
        return [(r.is_mshift, r.multiplier, r.shift) for r in arr]

    return {"acc_to_linear": rs(acc), "bias_to_acc": rs(bias) if p.bias_enabled else None,
            "linear_to_gate": rs(gate),
            "cell": [(q.multiplier, q.mantissa, q.exponent, q.uses_fp) for q in cell],
            "hidden": rs(hid)}


@pytest.mark.parametrize("cfg_name", ["default", "c4", "pot2-gate", "16b-tensor", "4b-pot2"])
@pytest.mark.parametrize("bias", [True, False])
def test_product_finalize_and_exec_match_oracle(cfg_name, bias):
    H, I = 8, 5
    stats = _stats(I, H, 3, bias, True)
    cfg = _config(cfg_name)
    exp = O.finalize(stats, cfg, H, bias)
    got = lstm_ops.finalize_params(torch.from_numpy(stats), cfg, H, bias)
    assert list(got.struct.scale) == list(exp.scale)
    assert list(got.struct.zero_point) == list(exp.zero_point)
    for k in range(4):
        if k >= 2 and not bias:
            continue
        assert np.array_equal(L.chan_scales(got.struct, k), L.chan_scales(exp, k)), k
    assert _product_exec(got.struct, I) == O.derive_exec(exp, I)


def test_finalize_rejects_non_finite_statistics():
    stats = _stats(5, 8, 4)
    stats[-1] = 1.0  # one non-finite parameter value was seen
    with pytest.raises(rxmet_lib.RxmetError):
        lstm_ops.finalize_params(torch.from_numpy(stats), L.default_config(), 8, True)


def test_finalize_rejects_invalid_config():
    stats = _stats(5, 8, 5)
    c = L.default_config()
    c.op[L.OP["input"]].bits = 1
    with pytest.raises(rxmet_lib.RxmetError):
        lstm_ops.finalize_params(torch.from_numpy(stats), c, 8, True)


def test_params_dict_round_trip():
    stats = _stats(5, 8, 6)
    p = lstm_ops.finalize_params(torch.from_numpy(stats), _config("c4"), 8, True)
    q = lstm_ops.LstmQuantParams.from_dict(p.to_dict())
    assert list(q.struct.scale) == list(p.struct.scale)
    assert list(q.struct.zero_point) == list(p.struct.zero_point)
    for k in range(4):
        assert np.array_equal(L.chan_scales(q.struct, k), L.chan_scales(p.struct, k))
    assert _product_exec(q.struct, 5) == _product_exec(p.struct, 5)
