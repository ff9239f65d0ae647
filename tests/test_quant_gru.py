"""Host-side behaviour of the QuantGRU mirror (no GPU): operator map, weight-format
helpers, configuration state, lock/dirty rules and error paths, following the reference's
quant_gru.py and its tests (tests/recurrent/test_gru_storage.py, test_gru_autograd.py)."""
import pickle

import pytest
import torch

import quant_gru as Q


def test_operator_map_matches_config_attributes():
    cfg = Q.gru_ops.OperatorQuantConfig()
    for op, info in Q._OPERATOR_MAP.items():
        assert hasattr(cfg, info["bw_attr"]), op
        assert hasattr(cfg, info["sym_attr"]), op
        assert hasattr(cfg, info["unsigned_attr"]), op
    assert len(Q._OPERATOR_MAP) == 17
    # sigmoid outputs default to unsigned grids (quant_gru.py:244-247)
    assert cfg.update_gate_output_unsigned_ and cfg.reset_gate_output_unsigned_
    assert not cfg.new_gate_output_unsigned_


def test_gate_reorder_is_an_involution_and_swaps_r_z():
    H, I = 4, 3
    w = torch.arange(3 * H * I, dtype=torch.float32).reshape(3 * H, I)
    r, z, n = w.chunk(3, 0)
    out = Q.reorder_weights_pytorch_to_haste(w)
    assert torch.equal(out, torch.cat([z, r, n], 0))
    assert torch.equal(Q.reorder_weights_haste_to_pytorch(out), w)


def test_convert_weights_layout_and_missing_bias():
    H, I = 5, 2
    wi, wh = torch.randn(3 * H, I), torch.randn(3 * H, H)
    W, R, bw, br = Q.convert_weights_to_haste_format(wi, wh, None, None, H, torch.device("cpu"))
    assert W.shape == (I, 3 * H) and R.shape == (H, 3 * H)
    assert torch.equal(W[:, :H], wi[H:2 * H].t()) and torch.equal(R[:, 2 * H:], wh[2 * H:].t())
    assert torch.count_nonzero(bw) == 0 and torch.count_nonzero(br) == 0


def test_get_quant_range():
    assert Q.get_quant_range(8) == (-128, 127)
    assert Q.get_quant_range(8, True) == (0, 255)
    assert Q.get_quant_range(4) == (-8, 7)
    assert Q.get_quant_range(16, True) == (0, 65535)
    with pytest.raises(ValueError):
        Q.get_quant_range(0)


def test_constructor_limits():
    with pytest.raises(NotImplementedError):
        Q.QuantGRU(4, 8, num_layers=2)
    with pytest.raises(NotImplementedError):
        Q.QuantGRU(4, 8, dropout=0.1)
    with pytest.raises(ValueError):
        Q.QuantGRU(4, 8, quant_storage_dtype="int8")
    with pytest.raises(ValueError):
        Q.QuantGRU(4, 8, use_po2_scale=True, use_pot2_scale=False)


def test_parameters_like_nn_gru():
    m = Q.QuantGRU(6, 8, bidirectional=True)
    ref = torch.nn.GRU(6, 8, bidirectional=True)
    assert {n: p.shape for n, p in m.named_parameters()} == \
        {n: p.shape for n, p in ref.named_parameters()}
    bound = 1 / 8 ** 0.5
    assert all(float(p.detach().abs().max()) <= bound for p in m.parameters())
    m2 = Q.QuantGRU(6, 8, bias=False)
    assert m2.bias_ih_l0 is None and len(list(m2.parameters())) == 2


def test_set_all_bitwidth_keeps_weights_symmetric():
    m = Q.QuantGRU(4, 16)
    m.set_all_bitwidth(6, is_symmetric=False)
    cfg = m._bitwidth_config
    for a in Q._VALID_BITWIDTH_ATTRS:
        assert getattr(cfg, a) == 6, a
    for a in Q._WEIGHT_SYMMETRIC_ATTRS:
        assert getattr(cfg, a) is True, a
    for a in Q._ACTIVATION_SYMMETRIC_ATTRS:
        assert getattr(cfg, a) is False, a
    assert m._quant_params_dirty
    with pytest.raises(ValueError):
        m.set_all_bitwidth(33)
    assert m._get_bitwidth("x") == 6 and m._get_symmetric("h") is False
    with pytest.warns(UserWarning):
        assert m._get_bitwidth("nope") == 8


def test_po2_switch_marks_dirty_and_respects_lock():
    m = Q.QuantGRU(4, 16, use_pot2_scale=True)
    assert m.use_po2_scale and m._bitwidth_config.usePOT2_
    m = Q.QuantGRU(4, 16)
    m.enable_po2()
    assert m.use_po2_scale and m._quant_params_dirty
    m = Q.QuantGRU(4, 16)
    m._quant_params_locked = True
    with pytest.raises(RuntimeError, match="locked"):
        m.enable_pot2()


def test_pickle_keeps_bitwidths_drops_calibration():
    m = Q.QuantGRU(4, 16, bidirectional=True)
    m.set_all_bitwidth(5, False)
    m.use_po2_scale = True
    m.quant_ranges = object()
    m2 = pickle.loads(pickle.dumps(m))
    assert m2._bitwidth_config.x_ == 5 and m2._bitwidth_config.usePOT2_
    assert m2._bitwidth_config.x_symmetric_ is False
    assert m2.quant_ranges is None and m2.quant_params_reverse is None
    assert not m2._quant_params_dirty
    for (n, a), (_, b) in zip(m.named_parameters(), m2.named_parameters()):
        assert torch.equal(a, b), n


def test_quantised_forward_requires_calibration():
    m = Q.QuantGRU(4, 16, use_quantization=True)
    with pytest.raises(RuntimeError, match="not calibrated"):
        m(torch.randn(3, 2, 4))


def test_locked_but_uncalibrated_is_an_error():
    m = Q.QuantGRU(4, 16, use_quantization=True)
    m.set_quant_params_locked(True)
    with pytest.raises(RuntimeError, match="locked"):
        m(torch.randn(3, 2, 4))


def test_cpu_input_is_rejected_loudly():
    m = Q.QuantGRU(4, 16)
    m.calibrating = True
    with pytest.raises(RuntimeError, match="GPU"):
        m(torch.randn(3, 2, 4))


def test_histogram_calibration_not_provided():
    m = Q.QuantGRU(4, 16)
    m.calibrating = True
    m.calibration_method = "sqnr"
    with pytest.raises(NotImplementedError):
        m(torch.randn(3, 2, 4))


def test_calibration_context_restores_flag_when_nothing_collected():
    m = Q.QuantGRU(4, 16)
    with m.calibration_context():
        assert m.calibrating
    assert not m.calibrating and m.quant_params is None


def test_finalize_without_data_raises():
    m = Q.QuantGRU(4, 16)
    with pytest.raises(RuntimeError, match="no calibration data"):
        m.finalize_calibration()


def test_hx_shape_checked():
    m = Q.QuantGRU(4, 16, bidirectional=True)
    with pytest.raises(ValueError):
        m._parse_initial_state(torch.zeros(1, 2, 16), 2)


def test_module_names():
    net = torch.nn.Sequential(torch.nn.Linear(2, 4), Q.QuantGRU(4, 16))
    Q.set_quant_gru_module_names(net)
    assert net[1]._module_name == "1"


def _calibrated_on_host(m, seed):
    """Grids from synthetic MinMax ranges through the host parameter derivation (no GPU)."""
    import numpy as np
    import gru_ops
    H = m.hidden_size
    g = np.random.default_rng(seed)
    params = []
    for _ in range(2 if m.bidirectional else 1):
        r = gru_ops.GRUQuantizationRanges(H)
        st = r.stats.numpy()
        # 13 operator minima, 13 maxima, then per-channel min / max blocks of 3H for W, R, bw, br
        mins = -np.abs(g.standard_normal(13)).astype(np.float32) - 0.1
        mins[0] = -1.7  # both directions read the same x: one x grid
        st[:13], st[13:26] = mins, -mins * 1.3
        for k in range(4):
            base = 26 + 2 * k * 3 * H
            cm = -np.abs(g.standard_normal(3 * H)).astype(np.float32) * 0.2 - 0.01
            st[base:base + 3 * H], st[base + 3 * H:base + 6 * H] = cm, -cm * 1.1
        params.append(gru_ops.calculate_gru_quantitative_parameters(r, m._bitwidth_config))
    m.quant_params = params[0]
    if m.bidirectional:
        m.quant_params_reverse = params[1]
    m._quant_params_dirty = False


@pytest.mark.parametrize("bidirectional", [False, True])
@pytest.mark.parametrize("pot2", [False, True])
def test_quant_params_json_round_trip(tmp_path, bidirectional, pot2):
    """export_quant_params -> load_quant_params into a fresh module gives the same grids,
    per-channel scales, bit widths and flags (quant_gru.py:2548-2592)."""
    import json
    import numpy as np
    import rxmet_gru_abi as A
    m = Q.QuantGRU(6, 16, bidirectional=bidirectional)
    m.set_all_bitwidth(8, is_symmetric=False)
    m._bitwidth_config.h_ = 16
    m._bitwidth_config.W_granularity_ = A.PER_GATE
    m.use_po2_scale = pot2
    _calibrated_on_host(m, 3)
    path = tmp_path / "qp.json"
    m.export_quant_params(str(path), include_weights=True)
    doc = json.loads(path.read_text())
    assert list(doc["operators"])[-4:] == ["weight_ih", "weight_hh", "bias_ih", "bias_hh"]
    op = doc["operators"]["output"]
    assert op["dtype"] == "INT16" and op["symmetric"] is False
    assert op["real_min"] == pytest.approx(op["scale"] * (-32768 - op["zero_point"]))
    assert doc["operators"]["weight_ih"]["enc_type"] == "PER_GATE"
    assert doc["operators"]["update_gate_output"]["dtype"] == "UINT8"
    assert ("operators_reverse" in doc) == bidirectional
    assert len(doc["quantized_weights"]["W"]) == 6 and len(doc["quantized_weights"]["W"][0]) == 48
    n = Q.QuantGRU(6, 16, bidirectional=bidirectional)
    n.load_quant_params(str(path))
    assert n.is_calibrated() and n.use_po2_scale == pot2
    for a, b in ((m.quant_params, n.quant_params),) + (
            ((m.quant_params_reverse, n.quant_params_reverse),) if bidirectional else ()):
        for name in A.GRID_NAMES:
            assert a.scale(name) == b.scale(name), name
            assert a.zero_point(name) == b.zero_point(name), name
            ga, gb = a.struct.g[A.GRID[name]], b.struct.g[A.GRID[name]]
            assert (ga.bits, bool(ga.is_unsigned)) == (gb.bits, bool(gb.is_unsigned)), name
        for k, name in enumerate(A.CHAN_NAMES):
            np.testing.assert_array_equal(a.channel_scales(name), b.channel_scales(name))
            assert a.struct.chan_bits[k] == b.struct.chan_bits[k]
        assert a.struct.use_pot2 == b.struct.use_pot2
    for attr in ("x_", "h_", "W_", "R_", "h_symmetric_", "update_gate_output_unsigned_",
                 "W_granularity_", "usePOT2_"):
        assert getattr(m._bitwidth_config, attr) == getattr(n._bitwidth_config, attr), attr


def test_quant_params_json_checks(tmp_path):
    m = Q.QuantGRU(6, 16)
    with pytest.raises(RuntimeError, match="calibrate"):
        m.export_quant_params(str(tmp_path / "x.json"))
    _calibrated_on_host(m, 4)
    m.export_quant_params(str(tmp_path / "a.json"))
    with pytest.raises(ValueError, match="hidden_size"):
        Q.QuantGRU(6, 32).load_quant_params(str(tmp_path / "a.json"))
    with pytest.raises(ValueError, match="bidirectional"):
        Q.QuantGRU(6, 16, bidirectional=True).load_quant_params(str(tmp_path / "a.json"))


def test_aimet_capabilities_and_configure():
    """The AIMET adapter contract (quant_gru.py:2290-2378): capability report and the
    mode -> flag mapping."""
    m = Q.QuantGRU(3, 4)
    caps = m.aimet_capabilities()
    assert caps["supports_forward_quantized"] and caps["forward_quantized_input_dtypes"] == ["int32"]
    assert set(caps["supported_modes"]) == set(Q.QuantGRU._AIMET_SUPPORTED_MODES)
    m.aimet_configure("calibrating")
    assert m.calibrating and not m.use_quantization
    m.aimet_configure("INT16_FIXED_EVAL")
    assert not m.calibrating and m.use_quantization
    m.aimet_configure("fp32_qdq")
    assert not m.use_quantization
    with pytest.raises(ValueError, match="Unsupported aimet_configure mode"):
        m.aimet_configure("int4")


def test_int_io_entry_points_check_their_arguments():
    m = Q.QuantGRU(3, 4, quant_storage_dtype="int32")
    assert m.quant_storage_dtype == "int32"
    with pytest.raises(RuntimeError, match="not calibrated"):
        m.get_io_quant_meta()
    with pytest.raises(RuntimeError, match="not calibrated"):
        m.forward_quantized(torch.zeros(2, 1, 3, dtype=torch.int32))
    with pytest.raises(ValueError, match="quant_storage_dtype"):
        Q.QuantGRU(3, 4, quant_storage_dtype="int16")


def _same_grids(m, n):
    import numpy as np
    import rxmet_gru_abi as A
    pairs = [(m.quant_params, n.quant_params)]
    if m.bidirectional:
        pairs.append((m.quant_params_reverse, n.quant_params_reverse))
    for a, b in pairs:
        for name in A.GRID_NAMES:
            assert a.scale(name) == b.scale(name), name
            assert a.zero_point(name) == b.zero_point(name), name
            ga, gb = a.struct.g[A.GRID[name]], b.struct.g[A.GRID[name]]
            assert (ga.bits, bool(ga.is_unsigned)) == (gb.bits, bool(gb.is_unsigned)), name
        for k, name in enumerate(A.CHAN_NAMES):
            np.testing.assert_array_equal(a.channel_scales(name), b.channel_scales(name))
            assert a.struct.chan_bits[k] == b.struct.chan_bits[k]
        assert a.struct.use_pot2 == b.struct.use_pot2


@pytest.mark.parametrize("bidirectional", [False, True])
@pytest.mark.parametrize("pot2", [False, True])
def test_aimet_encodings_round_trip(bidirectional, pot2):
    """export_quant_params_to_aimet_format -> load_quant_params_from_aimet_format into a fresh
    module gives the same grids (quant_gru.py:2674-3592), through a JSON round trip."""
    import json
    import math
    import numpy as np
    import rxmet_gru_abi as A
    H = 16
    m = Q.QuantGRU(6, H, bidirectional=bidirectional)
    m.set_all_bitwidth(8, is_symmetric=False)
    m._bitwidth_config.h_ = 16
    m._bitwidth_config.W_granularity_ = A.PER_CHANNEL
    m.use_po2_scale = pot2
    _calibrated_on_host(m, 5)
    enc = json.loads(json.dumps(m.export_quant_params_to_aimet_format(
        {"tensor_encodings": {"old": 1}}, "enc.gru")))
    assert enc["schema_version"] == 3 and "tensor_encodings" not in enc
    layer = enc["activation_encodings"]["enc.gru"]
    assert layer["is_GRU"] is True and set(layer["input"]) == {"0"}
    assert list(layer["internal_ops"]) == list(Q._AIMET_SLOTS)
    assert ("internal_ops_reverse" in layer) == bidirectional
    out = layer["output"]["0"]
    assert out["bitwidth"] == 16 and out["is_symmetric"] == "False" and "symmetric" not in out
    assert out["n"] == int(round(-math.log2(out["scale"])))
    assert layer["internal_ops"]["add_final_hidden"]["output"] == [out]
    assert layer["internal_ops"]["sub_one_minus_update"]["output"] == \
        layer["internal_ops"]["update_gate_output"]["output"]
    dirs = [m.quant_params] + ([m.quant_params_reverse] if bidirectional else [])
    w = enc["param_encodings"]["enc.gru.weight_ih.weight"]
    np.testing.assert_array_equal(np.float32(w["scale"]),
                                  np.concatenate([q.channel_scales("W") for q in dirs]))
    assert w["zero_point"] == [0] * len(w["scale"]) and w["n"] == Q._encoding_n(w["scale"])
    b = enc["param_encodings"]["enc.gru.bias"]
    parts = []
    for q in dirs:
        parts += [q.channel_scales("bw"), q.channel_scales("br")]
    np.testing.assert_array_equal(np.float32(b["scale"]), np.concatenate(parts))
    n = Q.QuantGRU(6, H, bidirectional=bidirectional)
    assert n.load_quant_params_from_aimet_format(enc, "enc.gru")
    assert n.is_calibrated() and n._module_name == "enc.gru"
    _same_grids(m, n)
    for attr in ("x_", "h_", "W_", "R_", "h_symmetric_", "update_gate_output_unsigned_",
                 "W_granularity_"):
        assert getattr(m._bitwidth_config, attr) == getattr(n._bitwidth_config, attr), attr
    # the same dictionary comes out again
    again = n.export_quant_params_to_aimet_format({}, "enc.gru")
    assert json.loads(json.dumps(again)) == enc


def test_aimet_encodings_checks():
    m = Q.QuantGRU(6, 16)
    assert m.export_quant_params_to_aimet_format({"a": 1}) == {"a": 1}  # not calibrated
    _calibrated_on_host(m, 6)
    enc = m.export_quant_params_to_aimet_format({})
    assert "gru" in enc["activation_encodings"]  # default module name
    n = Q.QuantGRU(6, 16)
    assert n.load_quant_params_from_aimet_format(enc, "other") is False
    assert n.load_quant_params_from_aimet_format({}, "gru") is False
    bad = json_copy(enc)
    bad["activation_encodings"]["gru"]["output"]["0"]["n"] += 1
    with pytest.raises(ValueError, match="n does not match"):
        n.load_quant_params_from_aimet_format(bad, "gru")
    bad = json_copy(enc)
    del bad["param_encodings"]["gru.bias"]
    assert n.load_quant_params_from_aimet_format(bad, "gru") is False
    assert not n.is_calibrated()


def json_copy(d):
    import json
    return json.loads(json.dumps(d))
