"""Pin the QcQuantizeOp oracle (oracle/qc_quantize_oracle.py) before trusting it, and check the
host-side pieces of the ONNX Runtime op that need no GPU.

* getComputedEncodings' closed forms (quantization_utils.cpp:59-119): asymmetric, symmetric,
  strict symmetric, the 2-bit extra bin, unsigned symmetric, the fp32 clamp of the range and C
  round (half away from zero) — each chosen so that a plausible slip (banker's rounding, the
  wrong count of positive / negative steps, a missing clamp) fails;
* the reference's own C++ (oracle/_ref/libqc_ref.so: quantization_utils.cpp,
  MinMaxEncodingAnalyzer.cpp, ContiguousEncodingAnalyzer.cpp, trim_functions.cpp, ... compiled
  where they lie) on random statistics, tensors, encoding shapes and NaN: encodings and
  quantize-dequantize outputs bit for bit;
* the op-mode machine of QcQuantizeOp::computeImpl (QcQuantizeOp.cpp:101-170);
* the broadcast layout the GPU path addresses (rxmet_qc_broadcast_layout, host code) against
  the oracle's grouping of getBroadcastableShapes;
* the ONNX Runtime plugin library exports RegisterCustomOps.
"""
import ctypes
from pathlib import Path

import numpy as np
import pytest

import qc_quantize_oracle as O
import rxmet_lib
import rxmet_qc_abi as abi

ROOT = Path(__file__).resolve().parents[1]
REF = ROOT / "oracle" / "_ref" / "libqc_ref.so"
f32, f64 = np.float32, np.float64


def _ref():
    if not REF.exists():
        pytest.skip("oracle/_ref/libqc_ref.so not built (reference checkout absent)")
    lib = ctypes.CDLL(str(REF))
    P = ctypes.c_void_p
    lib.qcref_computed_encodings.argtypes = [ctypes.c_int, ctypes.c_double, ctypes.c_double,
                                             ctypes.c_int, ctypes.c_int, ctypes.c_int, P]
    lib.qcref_computed_encodings.restype = None
    lib.qcref_analyzer.argtypes = [P, P, ctypes.c_int, P, ctypes.c_int, ctypes.c_int,
                                   ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, P]
    lib.qcref_qdq.argtypes = [P, P, P, ctypes.c_int, P, ctypes.c_int, P, ctypes.c_int]
    return lib


def _enc1(bw, mn, mx, sym, strict=False, uns=False):
    return tuple(float(v[0]) for v in O.computed_encodings(bw, mn, mx, sym, strict, uns))


def test_computed_encodings_closed_forms():
    # asymmetric 8 bit: delta = range / 255, offset = round(min / delta)
    d = 3.0 / 255
    assert _enc1(8, -1.0, 2.0, False) == (d * -85.0, d * 170.0, d, -85.0)
    # symmetric 8 bit: 127 positive and 128 negative steps, offset -128
    d = max(2.0 / 127, 1.0 / 128)
    assert _enc1(8, -1.0, 2.0, True) == (d * -128.0, d * 127.0, d, -128.0)
    # strict symmetric: 254 steps, 127 each side
    d = 2.0 / 127
    assert _enc1(8, -1.0, 2.0, True, strict=True) == (d * -127.0, d * 127.0, d, -127.0)
    # 2-bit symmetric: 3 steps, 1 positive step plus the extra bin, 2 negative
    d = max(1.0 / 2, 0.6 / 2)
    assert _enc1(2, -0.6, 1.0, True) == (d * -2.0, d * 1.0, d, -2.0)
    # unsigned symmetric with min >= 0 takes the asymmetric grid
    d = 2.0 / 255
    assert _enc1(8, 0.0, 2.0, True, uns=True) == (0.0, d * 255.0, d, 0.0)
    # ... and is ignored when min < 0
    assert _enc1(8, -1.0, 2.0, True, uns=True) == _enc1(8, -1.0, 2.0, True)
    # C round is half away from zero: min / delta = -2.5 -> -3 (banker's rounding gives -2)
    assert _enc1(2, -1.25, 0.25, False)[3] == -3.0
    # min above 0 / max below 0 clamp to 0; the range to 0.99 of fp32's
    assert _enc1(8, 0.5, 2.0, False)[3] == 0.0
    big = float(np.finfo(f32).max) * 0.99
    e = _enc1(8, -1e39, 1e39, False)
    assert e[0] >= -big and e[1] <= big


def test_minmax_encodings_min_range_and_zero():
    # all-zero statistics: max nudged to min + float(0.01) in double
    e = O.minmax_encodings(np.array([0.0], f32), np.array([0.0], f32), 8, False)
    assert e[2][0] == float(f32(0.01)) / 255
    # statistics that exclude zero are widened to include it
    e = O.minmax_encodings(np.array([1.0], f32), np.array([3.0], f32), 8, False)
    assert e[3][0] == 0.0 and e[2][0] == 3.0 / 255


def test_computed_encodings_match_reference_cpp():
    lib = _ref()
    g = np.random.default_rng(7)
    out = np.zeros(4, f64)
    n = 0
    for bw in (1, 2, 3, 4, 8, 12, 16, 31, 32):
        for sym in (False, True):
            for strict in (False, True):
                for uns in (False, True):
                    if sym and strict and uns:
                        continue
                    for _ in range(40):
                        scale = 10.0 ** g.uniform(-8, 38)
                        mn = -abs(g.standard_normal()) * scale * (g.random() < 0.8)
                        mx = abs(g.standard_normal()) * scale * (g.random() < 0.9)
                        lib.qcref_computed_encodings(bw, mn, mx, int(sym), int(strict), int(uns),
                                                     out.ctypes.data)
                        got = np.array(_enc1(bw, mn, mx, sym, strict, uns))
                        np.testing.assert_array_equal(got, out, err_msg=f"{bw} {sym} {strict} "
                                                      f"{uns} {mn!r} {mx!r}")
                        n += 1
    assert n > 1000


CASES = [  # tensor shape, encoding shape
    ((7, 33), ()),
    ((7, 33), (7, 1)),
    ((7, 33), (33,)),
    ((4, 6, 5), (4, 1, 1)),
    ((4, 6, 5), (1, 6, 1)),
    ((4, 6, 5), (5,)),
    ((8, 12), (8, 3)),          # channel + block (blocks of 4 along axis 1)
    ((12, 8), (3, 8)),          # blocks of 4 along axis 0, channel on axis 1
    ((6, 4, 3, 3), (6, 2, 1, 1)),  # conv weight: output channel + input-channel blocks
    ((2, 3, 10), (2, 1, 5)),    # two separated groups
]


def _dims(s):
    a = np.array(s if len(s) else [0], np.int64)
    return a, len(s)


@pytest.mark.parametrize("tshape,eshape", CASES)
def test_analyzer_and_qdq_match_reference_cpp(tshape, eshape):
    lib = _ref()
    g = np.random.default_rng(len(tshape) * 31 + int(np.prod(eshape) if eshape else 1))
    ncalls = 3
    x = (g.standard_normal((ncalls,) + tshape) * g.uniform(0.1, 10)).astype(f32)
    x[0].reshape(-1)[3] = np.nan
    x[1].reshape(-1)[0] = np.nan
    ta, tn = _dims(tshape)
    ea, en = _dims(eshape)
    nenc = int(np.prod(eshape)) if eshape else 1
    for bw, sym, strict in ((8, False, False), (8, True, False), (4, True, True), (16, False, False)):
        ref = np.zeros(4 * nenc, f64)
        assert lib.qcref_analyzer(x.ctypes.data, ta.ctypes.data, tn, ea.ctypes.data, en, ncalls,
                                  bw, int(sym), int(strict), 0, ref.ctypes.data) == 0
        q = O.BlockTensorQuantizerOracle(eshape, bw)
        q.strict = strict
        for k in range(ncalls):
            q.update_stats(x[k])
        enc = q.compute_encodings(sym)
        got = np.stack(enc[:4], axis=1).reshape(-1)
        np.testing.assert_array_equal(got, ref)
        # quantize-dequantize of a fresh tensor with NaN, +-inf and outliers
        y_in = (g.standard_normal(tshape) * 4).astype(f32)
        y_in.reshape(-1)[:3] = [np.nan, np.inf, -np.inf]
        yr = np.zeros_like(y_in)
        assert lib.qcref_qdq(y_in.ctypes.data, yr.ctypes.data, ta.ctypes.data, tn,
                             ea.ctypes.data, en, ref.ctypes.data, bw) == 0
        q.set_encodings(enc)
        yo = q.quantize_dequantize(y_in)
        np.testing.assert_array_equal(yo, yr)


def test_op_mode_machine():
    x = np.linspace(-2, 3, 40, dtype=f32).reshape(4, 10)
    # oneShot: computes encodings, quantizes, then switches to quantizeDequantize
    op = O.QcQuantizeOpOracle(O.BlockTensorQuantizerOracle((), 8), O.ONE_SHOT_QDQ)
    y = op.compute(x)
    assert op.op_mode == O.QDQ and op.q.encoding_valid
    assert not np.array_equal(y, x) and np.abs(y - x).max() <= 5.0 / 255
    # updateStats copies and accumulates
    op2 = O.QcQuantizeOpOracle(O.BlockTensorQuantizerOracle((), 8), O.UPDATE_STATS)
    np.testing.assert_array_equal(op2.compute(x), x)
    np.testing.assert_array_equal(op2.compute(x * 2), x * 2)
    assert op2.q.st_min[0] == -4.0 and op2.q.st_max[0] == 6.0
    # quantizeDequantize before encodings: the reference's error
    op3 = O.QcQuantizeOpOracle(O.BlockTensorQuantizerOracle((), 8), O.QDQ)
    with pytest.raises(RuntimeError, match="before computing encodings"):
        op3.compute(x)
    # disabled: pass through, a oneShot node keeps its mode
    op4 = O.QcQuantizeOpOracle(O.BlockTensorQuantizerOracle((), 8), O.ONE_SHOT_QDQ,
                               enabled=False)
    np.testing.assert_array_equal(op4.compute(x), x)
    assert op4.op_mode == O.ONE_SHOT_QDQ and not op4.q.valid_stats
    # float quantizer: fp16 round trip in the quantizing modes, copy otherwise
    op5 = O.QcQuantizeOpOracle(None, O.QDQ, is_int=False)
    v = np.array([1.0 + 2.0 ** -12, 65519.0, 65520.0, 2.0 ** -25, 2.0 ** -24 * 1.5], f32)
    np.testing.assert_array_equal(op5.compute(v), [1.0, 65504.0, np.inf, 0.0, 2.0 ** -23])
    op6 = O.QcQuantizeOpOracle(None, O.UPDATE_STATS, is_int=False)
    np.testing.assert_array_equal(op6.compute(v), v)


LAYOUT_CASES = [
    ((7, 33), ()), ((7, 33), (7, 1)), ((7, 33), (33,)), ((4, 6, 5), (1, 6, 1)),
    ((8, 12), (8, 3)), ((12, 8), (3, 8)), ((6, 4, 3, 3), (6, 2, 1, 1)), ((2, 3, 10), (2, 1, 5)),
    ((1, 5, 1, 7), (5, 1, 7)), ((3, 1, 4), (1, 1, 4)),
]


@pytest.mark.parametrize("tshape,eshape", LAYOUT_CASES)
def test_broadcast_layout_host_function(tshape, eshape):
    lib = rxmet_lib.load()
    ta, tn = abi.dims(tshape)
    ea, en = abi.dims(eshape)
    out = rxmet_lib.QdqLayout()
    assert lib.rxmet_qc_broadcast_layout(ta, tn, ea, en, ctypes.byref(out)) == 0, \
        lib.rxmet_last_error()
    got = [out.outer, out.C0, out.mid, out.C1, out.inner]
    assert got == O.layout_groups(tshape, eshape)
    assert int(np.prod(got)) == int(np.prod(tshape))


@pytest.mark.parametrize("tshape,eshape,msg", [
    ((4, 6, 5), (4, 6, 5, 2), "more dimensions"),
    ((7, 33), (7, 2), "broadcastable"),
    ((0, 5), (1, 5), "broadcastable"),  # as getBroadcastableShapes: 0 < 1
    ((2, 3, 4, 5), (2, 1, 4, 1), None),
    ((2, 3, 4, 5, 6), (2, 1, 4, 1, 6), "two groups"),
])
def test_broadcast_layout_errors(tshape, eshape, msg):
    lib = rxmet_lib.load()
    ta, tn = abi.dims(tshape)
    ea, en = abi.dims(eshape)
    out = rxmet_lib.QdqLayout()
    rc = lib.rxmet_qc_broadcast_layout(ta, tn, ea, en, ctypes.byref(out))
    if msg is None:
        assert rc == 0
        assert [out.outer, out.C0, out.mid, out.C1, out.inner] == [1, 2, 3, 4, 5]
    else:
        assert rc == -22 and msg in lib.rxmet_last_error().decode()


def test_ort_plugin_exports_register_custom_ops():
    import build as B  # rx-met_amd/build.py

    if not B.ORT_LIB.exists():
        pytest.skip("librxmet_ort_ops.so not built (ONNX Runtime headers absent)")
    lib = ctypes.CDLL(str(B.ORT_LIB))
    assert hasattr(lib, "RegisterCustomOps")
