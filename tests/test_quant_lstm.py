"""Host-side QuantLSTM module logic: operator-config resolution and validation, the public v1
quant params document, constructor checks and the GPU-only guard.  No GPU needed."""
import json

import numpy as np
import pytest
import torch

import lstm_oracle as O
import quant_lstm as Q
import rxmet_lstm_abi as L

f32 = np.float32


def test_default_config_matches_reference_profile():
    cfg = Q.default_quant_config()
    assert cfg["scale_mode"] == "affine" and len(cfg["operators"]) == 18
    for name in ("input_gate_output", "forget_gate_output", "output_gate_output"):
        assert cfg["operators"][name]["is_unsigned"] is True
    assert cfg["operators"]["cell_gate_output"]["is_unsigned"] is False
    assert cfg["operators"]["weight_hh"] == {"bitwidth": 8, "granularity": "per_channel"}
    a, b = Q.config_struct(cfg), L.default_config()
    assert a.scale_mode == b.scale_mode
    for i in range(L.NOPS):
        x, y = a.op[i], b.op[i]
        assert (x.bits, x.is_unsigned, x.is_symmetric, x.granularity) == \
               (y.bits, y.is_unsigned, y.is_symmetric, y.granularity), L.OP_NAMES[i]


def test_override_applies_sparse_fields_and_validates():
    cfg = Q.resolve_quant_config({"schema_version": 1, "scale_mode": "pot2",
                                  "operators": {"cell_state": {"bitwidth": 16},
                                                "weight_ih": {"granularity": "per_gate"},
                                                "output": {"is_symmetric": False,
                                                           "comment": "h"}}})
    assert cfg["scale_mode"] == "pot2"
    assert cfg["operators"]["cell_state"]["bitwidth"] == 16
    assert cfg["operators"]["weight_ih"]["granularity"] == "per_gate"
    assert cfg["operators"]["output"]["is_symmetric"] is False
    bad = [
        {"schema_version": 2},
        {"schema_version": 1, "extra": 1},
        {"schema_version": 1, "operators": {"nope": {"bitwidth": 8}}},
        {"schema_version": 1, "operators": {"weight_ih": {"is_unsigned": True}}},
        {"schema_version": 1, "operators": {"input": {"granularity": "per_channel"}}},
        {"schema_version": 1, "operators": {"input": {"comment": "only"}}},
        {"schema_version": 1, "operators": {"input": {"bitwidth": 33}}},
        {"schema_version": 1, "operators": {"input": {"bitwidth": True}}},
        {"schema_version": 1, "operators": {"input": {"bitwidth": None}}},
        {"schema_version": 1, "operators": {"output": {"is_unsigned": True, "bitwidth": 32}}},
        {"schema_version": 1, "operators": {"weight_hh": {"bitwidth": 1}}},
        {"schema_version": 1, "scale_mode": "log"},
    ]
    for ov in bad:
        with pytest.raises(ValueError):
            Q.resolve_quant_config(ov)


def test_json_sources_and_duplicate_keys(tmp_path):
    text = '{"schema_version": 1, "operators": {"output": {"bitwidth": 16}}}'
    p = tmp_path / "cfg.json"
    p.write_text(text)
    for src in (text, str(p), p, json.loads(text)):
        m = Q.QuantLSTM(4, 16, quant_config=src)
        assert m.get_quant_config("output")["bitwidth"] == 16
    with pytest.raises(ValueError, match="duplicate"):
        Q.QuantLSTM(4, 16, quant_config='{"schema_version": 1, "schema_version": 1}')


def test_module_config_api():
    m = Q.QuantLSTM(5, 16, bidirectional=True)
    names = [n for n, _ in m.named_parameters()]
    assert names == ["weight_ih_l0", "weight_hh_l0", "bias_ih_l0", "bias_hh_l0",
                     "weight_ih_l0_reverse", "weight_hh_l0_reverse", "bias_ih_l0_reverse",
                     "bias_hh_l0_reverse"]
    bound = 1.0 / 4.0
    assert all(float(p.detach().abs().max()) <= bound for p in m.parameters())
    m.adjust_quant_config("cell_state", bitwidth=16)
    assert m.get_quant_config("cell_state")["bitwidth"] == 16
    m.set_all_bitwidth(4)
    assert all(v["bitwidth"] == 4 for v in m.get_quant_config()["operators"].values())
    with pytest.raises(ValueError):
        m.adjust_quant_config("cell_state", granularity="per_channel")
    with pytest.raises(ValueError):
        m.adjust_quant_config("nope", bitwidth=8)
    with pytest.raises(ValueError):
        m.adjust_quant_config("input")
    assert m.calibration_state() == {"forward": "empty", "reverse": "empty"}
    assert not m.is_calibrated()
    with pytest.raises(RuntimeError):
        m.set_quant_params_locked(True)
    with pytest.raises(RuntimeError):
        m.finalize_calibration()


@pytest.mark.parametrize("kw", [dict(num_layers=2), dict(dropout=0.1), dict(dtype=torch.float64),
                                dict(calibration_method="kl"), dict(cublas_math_mode="fast")])
def test_constructor_rejects_unsupported_arguments(kw):
    with pytest.raises(ValueError):
        Q.QuantLSTM(4, 16, **kw)


def test_cpu_input_is_rejected():
    m = Q.QuantLSTM(4, 16)
    with pytest.raises(RuntimeError, match="GPU"):
        m(torch.zeros(3, 2, 4))


def _calibrated_module(bidirectional, bias, cfg_override=None, seed=0):
    I, H = 6, 16
    m = Q.QuantLSTM(I, H, bias=bias, bidirectional=bidirectional, quant_config=cfg_override)
    g = np.random.default_rng(seed)
    x = (g.random((5, 3, I)) * 2 - 1).astype(f32)
    cfg = Q.config_struct(m.get_quant_config())
    params = []
    for d in range(m.num_directions):
        Wi, Wh, bi, bh = (None if p is None else p.detach().numpy() for p in
                          m._direction_params(d == 1))
        xd = x[::-1].copy() if d == 1 else x
        st = O.calibrate(Wi, Wh, bi, bh, xd)
        wrap = Q.lstm_ops.LstmQuantParams(H)
        wrap._p = O.finalize(st, cfg, H, bias)  # noqa: SLF001
        params.append(wrap)
    m._params = params  # noqa: SLF001 (oracle-finalised params stand in for a GPU calibration)
    return m


@pytest.mark.parametrize("bidirectional", [False, True])
@pytest.mark.parametrize("bias", [True, False])
@pytest.mark.parametrize("override", [None, {"schema_version": 1, "scale_mode": "pot2",
                                             "operators": {"weight_hh": {"granularity": "per_gate"},
                                                           "weight_ih": {"granularity": "per_tensor"},
                                                           "cell_state": {"bitwidth": 16}}}])
def test_quant_params_document_round_trip(tmp_path, bidirectional, bias, override):
    m = _calibrated_module(bidirectional, bias, override)
    dest = tmp_path / "qp.json"
    doc = m.export_quant_params(dest)
    assert json.loads(dest.read_text()) == json.loads(json.dumps(doc))
    assert set(doc) == {"schema_version", "model_info", "execution_metadata", "operators"} | (
        {"operators_reverse"} if bidirectional else set())
    assert ("bias_ih" in doc["operators"]) == bias
    gran = (override or {}).get("operators", {}).get("weight_hh", {}).get("granularity",
                                                                           "per_channel")
    n = {"per_channel": 64, "per_gate": 4}[gran]
    assert len(doc["operators"]["weight_hh"]["scale"]) == n
    m2 = Q.QuantLSTM(6, 16, bias=bias, bidirectional=bidirectional)
    m2.load_quant_params(dest)
    assert m2.get_quant_config() == m.get_quant_config()
    for a, b in zip(m._params, m2._params):  # noqa: SLF001
        assert list(a.struct.scale) == list(b.struct.scale)
        assert list(a.struct.zero_point) == list(b.struct.zero_point)
        for k in range(4 if bias else 2):
            assert np.array_equal(L.chan_scales(a.struct, k), L.chan_scales(b.struct, k))
        assert Q.lstm_ops.LstmQuantParams.to_dict(a) == Q.lstm_ops.LstmQuantParams.to_dict(b)
    assert m2.is_calibrated()
    assert m2.export_quant_params() == doc


def test_quant_params_document_rejects_inconsistent_input():
    m = _calibrated_module(False, True)
    doc = m.export_quant_params()
    m2 = Q.QuantLSTM(6, 16)
    bad = json.loads(json.dumps(doc))
    bad["model_info"]["hidden_size"] = 32
    with pytest.raises(ValueError):
        m2.load_quant_params(bad)
    bad = json.loads(json.dumps(doc))
    bad["operators"]["output"]["real_max"] = 123.0
    with pytest.raises(ValueError):
        m2.load_quant_params(bad)
    bad = json.loads(json.dumps(doc))
    bad["operators"]["weight_ih"]["zero_point"] = [1] * 64
    with pytest.raises(ValueError):
        m2.load_quant_params(bad)
    bad = json.loads(json.dumps(doc))
    bad["execution_metadata"]["carrier"] = "int"
    with pytest.raises(ValueError):
        m2.load_quant_params(bad)
    bad = json.loads(json.dumps(doc))
    del bad["operators"]["cell_state"]
    with pytest.raises(ValueError):
        m2.load_quant_params(bad)
    with pytest.warns(RuntimeWarning):
        Q.QuantLSTM(6, 16, batch_first=True).load_quant_params(doc)
    assert not m2.is_calibrated()


def test_pickle_keeps_quant_params():
    import pickle

    m = _calibrated_module(True, True)
    m2 = pickle.loads(pickle.dumps(m))
    assert m2.is_calibrated()
    assert m2.export_quant_params() == m.export_quant_params()
