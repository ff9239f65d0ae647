"""The ONNX Runtime custom op QcQuantizeOp on the GPU (include/rxmet_qc.h) against the oracle
(oracle/qc_quantize_oracle.py, itself pinned bit for bit to the reference's C++ in
tests/test_qc_oracle.py).

Bar: bit-exact — statistics (fp32, compared with ==, so the sign of a zero minimum does not
count), TfEncodings (every double), outputs (NaN in the same places), op mode after the call —
for every op mode of QcQuantizeOp::computeImpl (QcQuantizeOp.cpp:101-170), enabled and
disabled, int and float quantizers, float32 and float16 tensors, per-tensor, per-channel,
block and channel + block encodings, strict / unsigned symmetric grids, NaN and +-inf.  At the
full [8192, 8192] size: sampled rows against the oracle and idempotence of the
quantize-dequantize.  ONNX Runtime's session registration is not exercised (no runtime in
this image); the plugin's compute is exactly rxmet_qc_quantize_compute, which these tests call.
"""
import numpy as np
import pytest
import torch

import qc_quantize_oracle as O
import qdq_oracle as QO
import rxmet_lib
from qc_quantize_op import (BlockTensorQuantizer, OpMode, QcQuantizeInfo, TfEncoding,
                            qc_quantize_op)

pytestmark = pytest.mark.gpu
f32 = np.float32

CASES = [  # tensor shape, encoding shape
    ((7, 33), ()),
    ((64, 1000), ()),
    ((7, 33), (7, 1)),
    ((7, 33), (33,)),
    ((4, 6, 5), (1, 6, 1)),
    ((8, 12), (8, 3)),
    ((12, 8), (3, 8)),
    ((6, 4, 3, 3), (6, 2, 1, 1)),
    ((2, 3, 10), (2, 1, 5)),
    ((96, 4096), (96, 1)),
]
DTYPES = [np.float32, np.float16]


def _ids(c):
    return f"{c[0]}-enc{c[1]}"


def _data(shape, seed, dtype, inf=True):
    """Scaled normal data with two NaN and (inf=True) +-inf elements."""
    g = np.random.default_rng(seed)
    x = (g.standard_normal(shape) * g.uniform(0.5, 8)).astype(f32)
    if x.size > 8:
        x.reshape(-1)[[1, 5]] = np.nan
        if inf:
            x.reshape(-1)[2] = np.inf
            x.reshape(-1)[3] = -np.inf
    return x.astype(dtype)


def _to_dev(x, cuda):
    return torch.from_numpy(np.ascontiguousarray(x)).to(cuda)


def _eq(got, exp, what):
    got = np.asarray(got)
    exp = np.asarray(exp)
    assert got.shape == exp.shape and got.dtype == exp.dtype, what
    assert np.array_equal(np.isnan(got), np.isnan(exp)), what
    assert np.array_equal(np.nan_to_num(got), np.nan_to_num(exp)), what


def _enc_eq(q: BlockTensorQuantizer, oq: O.BlockTensorQuantizerOracle, what):
    enc = q.getEncodings()
    exp = oq.enc
    for k, name in enumerate(("min", "max", "delta", "offset")):
        got = np.array([getattr(e, name) for e in enc])
        assert np.array_equal(got, np.asarray(exp[k]).reshape(-1)), (what, name)
    assert all(e.bw == exp[4] for e in enc), what


def _stats_eq(q, oq, what):
    mn, mx = q.getStats()
    assert np.array_equal(mn, oq.st_min) and np.array_equal(mx, oq.st_max), what


@pytest.mark.parametrize("dtype", DTYPES, ids=["f32", "f16"])
@pytest.mark.parametrize("case", CASES, ids=[_ids(c) for c in CASES])
def test_update_stats_compute_encodings_and_qdq(cuda, case, dtype):
    tshape, eshape = case
    print(f"[qc] stats/encodings/qdq {_ids(case)} {np.dtype(dtype).name}", flush=True)
    for bw, sym, strict, uns in ((8, False, False, False), (8, True, False, False),
                                 (4, True, True, False), (16, False, False, False),
                                 (8, True, False, True)):
        q = BlockTensorQuantizer(eshape, bw)
        oq = O.BlockTensorQuantizerOracle(eshape, bw)
        q.setStrictSymmetric(strict)
        q.setUnsignedSymmetric(uns)
        oq.strict, oq.unsigned_sym = strict, uns
        info = QcQuantizeInfo()
        info.tensorQuantizerRef = q
        info.opMode = OpMode.updateStats
        info.useSymmetricEncoding = sym
        op = O.QcQuantizeOpOracle(oq, O.UPDATE_STATS, symmetric=sym)
        for k in range(3):
            x = _data(tshape, 100 * bw + k, dtype, inf=False)  # NaN is skipped
            if uns:
                x = np.abs(x)  # unsigned symmetric applies to non-negative statistics
            y = qc_quantize_op(info, _to_dev(x, cuda)).cpu().numpy()
            _eq(y, op.compute(x), "updateStats output (a copy)")
            assert info.opMode == OpMode.updateStats
        _stats_eq(q, oq, "statistics")
        q.computeEncodings(sym)
        oq.set_encodings(oq.compute_encodings(sym))
        _enc_eq(q, oq, (bw, sym, strict, uns))
        info.opMode = OpMode.quantizeDequantize
        op.op_mode = O.QDQ
        x = _data(tshape, 7 * bw, dtype)
        _eq(qc_quantize_op(info, _to_dev(x, cuda)).cpu().numpy(), op.compute(x),
            ("quantizeDequantize", bw, sym, strict, uns))
        # the quantizer's own call gives the same
        _eq(q.quantizeDequantize(_to_dev(x, cuda)).cpu().numpy(), op.compute(x),
            "BlockTensorQuantizer.quantizeDequantize")


@pytest.mark.parametrize("dtype", DTYPES, ids=["f32", "f16"])
@pytest.mark.parametrize("case", CASES, ids=[_ids(c) for c in CASES])
def test_one_shot_then_quantize_dequantize(cuda, case, dtype):
    tshape, eshape = case
    print(f"[qc] oneShot {_ids(case)} {np.dtype(dtype).name}", flush=True)
    q = BlockTensorQuantizer(eshape, 8)
    oq = O.BlockTensorQuantizerOracle(eshape, 8)
    info = QcQuantizeInfo()
    info.tensorQuantizerRef = q
    info.opMode = OpMode.oneShotQuantizeDequantize
    op = O.QcQuantizeOpOracle(oq, O.ONE_SHOT_QDQ)
    # statistics from an earlier calibration are discarded by the one-shot reset
    q.updateStats(_to_dev(_data(tshape, 1, dtype) * 100, cuda))
    oq.update_stats(_data(tshape, 1, dtype) * 100)
    x = _data(tshape, 2, dtype, inf=False)
    _eq(qc_quantize_op(info, _to_dev(x, cuda)).cpu().numpy(), op.compute(x), "oneShot")
    assert info.opMode == OpMode.quantizeDequantize and op.op_mode == O.QDQ
    _enc_eq(q, oq, "oneShot encodings")
    _stats_eq(q, oq, "oneShot statistics")
    x2 = _data(tshape, 3, dtype) * 3
    _eq(qc_quantize_op(info, _to_dev(x2, cuda)).cpu().numpy(), op.compute(x2),
        "quantizeDequantize after oneShot")


@pytest.mark.parametrize("dtype", DTYPES, ids=["f32", "f16"])
def test_pass_through_and_disabled(cuda, dtype):
    x = _data((33, 65), 11, dtype)
    q = BlockTensorQuantizer((), 8)
    info = QcQuantizeInfo()
    info.tensorQuantizerRef = q
    info.opMode = OpMode.passThrough
    y = qc_quantize_op(info, _to_dev(x, cuda)).cpu().numpy()
    assert y.tobytes() == x.tobytes()
    # a disabled node passes through in every mode; one-shot stays one-shot, no statistics
    info.opMode = OpMode.oneShotQuantizeDequantize
    info.enabled = False
    y = qc_quantize_op(info, _to_dev(x, cuda)).cpu().numpy()
    assert y.tobytes() == x.tobytes()
    assert info.opMode == OpMode.oneShotQuantizeDequantize and not q.isEncodingValid
    info.opMode = OpMode.updateStats
    qc_quantize_op(info, _to_dev(x, cuda))
    mn, mx = q.getStats()
    assert mn[0] == np.finfo(f32).max and mx[0] == -np.finfo(f32).max  # untouched


@pytest.mark.parametrize("dtype", DTYPES, ids=["f32", "f16"])
def test_float_quantizer_fp16_round_trip(cuda, dtype):
    edge = np.array([1.0 + 2.0 ** -12, 1.0 + 3 * 2.0 ** -11, 65504.0, 65519.0, 65520.0, -65520.0,
                     2.0 ** -25, 2.0 ** -24 * 1.5, -2.0 ** -24 * 0.75, 6.1e-5, np.nan, np.inf,
                     -np.inf, 0.0, -0.0], dtype=f32)
    g = np.random.default_rng(5)
    with np.errstate(over="ignore"):  # values beyond fp16's range become +-inf
        x = np.concatenate([edge, (g.standard_normal(4093) * 10.0 ** g.uniform(-8, 6, 4093))
                            .astype(f32)]).astype(dtype)
    for mode in OpMode:
        info = QcQuantizeInfo()
        info.isIntDataType = False  # no tensor quantizer
        info.opMode = mode
        op = O.QcQuantizeOpOracle(None, int(mode), is_int=False)
        y = qc_quantize_op(info, _to_dev(x, cuda)).cpu().numpy()
        exp = op.compute(x)
        _eq(y, exp, mode)
        assert np.array_equal(np.signbit(y), np.signbit(exp)), mode
        assert int(info.opMode) == op.op_mode


def test_errors_follow_the_reference(cuda):
    q = BlockTensorQuantizer((4, 1), 8)
    info = QcQuantizeInfo()
    info.tensorQuantizerRef = q
    info.opMode = OpMode.quantizeDequantize
    x = torch.randn(4, 16, device=cuda)
    with pytest.raises(rxmet_lib.RxmetError, match="before computing encodings"):
        qc_quantize_op(info, x)
    with pytest.raises(rxmet_lib.RxmetError, match="before updating stats"):
        q.computeEncodings(False)
    with pytest.raises(rxmet_lib.RxmetError, match="broadcastable"):
        q.updateStats(torch.randn(5, 16, device=cuda))
    with pytest.raises(rxmet_lib.RxmetError, match="did not match"):
        q.setEncodings([TfEncoding(-1, 1, 2 / 255, -128, 8)])
    with pytest.raises(TypeError):
        qc_quantize_op(info, x.to(torch.bfloat16))


def test_host_set_encodings_native_alignment_tables(cuda):
    """Encodings set from the host (setEncodings) with the TfEncoding grids of the reference's
    alignment test (tests/integration/test_native_qdq_alignment.py:18-25, 88-147): exact codes,
    ties to even at 8 / 16 / 32 bits on symmetric and asymmetric grids, NaN kept, infinity
    clipped — equal to native_qdq, the form those tables pin."""
    codes = np.array([-7.5, -3.5, -2.5, -1.5, -.5, .5, 1.5, 2.5, 3.5, 7.5, np.nan, np.inf,
                      -np.inf, 0.0], dtype=f32)
    for bits in (8, 16, 32):
        s = 2.0 ** -7 if bits == 8 else 2.0 ** -15 if bits == 16 else 2.0 ** -21
        for off in (-(1 << (bits - 1)), -13):
            q = BlockTensorQuantizer((), bits)
            lo, hi = off * s, (off + (1 << bits) - 1) * s
            q.setEncodings([TfEncoding(lo, hi, s, off, bits)])
            x = codes * f32(s)
            y = q.quantizeDequantize(_to_dev(x, cuda)).cpu().numpy()
            _eq(y, QO.native_qdq(x, f32(lo), f32(hi), f32(s)), (bits, off))
            assert q.getEncodings()[0] == TfEncoding(lo, hi, s, off, bits)


def test_full_size_one_shot_per_channel(cuda):
    """[8192, 8192] float32 with per-row encodings (the c2 tensor): oneShot on the GPU; 64
    sampled rows against the oracle (statistics, encodings, outputs) and the quantize-dequantize
    idempotent on the whole tensor."""
    R = C = 8192
    print("[qc] full size oneShot [8192, 8192] per row", flush=True)
    g = torch.Generator(device=cuda).manual_seed(9)
    x = torch.randn(R, C, device=cuda, generator=g) * 3
    q = BlockTensorQuantizer((R, 1), 8)
    info = QcQuantizeInfo()
    info.tensorQuantizerRef = q
    info.opMode = OpMode.oneShotQuantizeDequantize
    info.useSymmetricEncoding = True
    y = qc_quantize_op(info, x)
    torch.cuda.synchronize()
    assert info.opMode == OpMode.quantizeDequantize
    rows = np.sort(np.random.default_rng(1).choice(R, 64, replace=False))
    xs = x[rows].cpu().numpy()
    oq = O.BlockTensorQuantizerOracle((64, 1), 8)
    oq.update_stats(xs)
    oq.set_encodings(oq.compute_encodings(True))
    mn, mx = q.getStats()
    assert np.array_equal(mn[rows], oq.st_min) and np.array_equal(mx[rows], oq.st_max)
    enc = q.getEncodings()
    assert np.array_equal([enc[r].delta for r in rows], oq.enc[2])
    assert np.array_equal([enc[r].min for r in rows], oq.enc[0])
    _eq(y[rows].cpu().numpy(), oq.quantize_dequantize(xs), "sampled rows")
    y2 = qc_quantize_op(info, y)
    assert torch.equal(y2, y)
