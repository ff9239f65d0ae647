"""ctypes wrapper of the GRU CPU oracle (libgru_oracle.so) and of the reference checker
(_ref/libgru_ref.so, the reference's own CPU code).  TEST INFRASTRUCTURE: imported only by
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg."""
from __future__ import annotations

import ctypes
import subprocess
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent / "rx-met_amd"))
import rxmet_gru_abi as A  # noqa: E402  (struct layouts of include/rxmet_gru.h)

f32 = np.float32
_P = ctypes.c_void_p
_i = ctypes.c_int


def _lib(path: Path, build_target: str):
    if not path.exists():
        subprocess.run(["make", "-C", str(HERE), build_target], check=True,
                       stdout=subprocess.DEVNULL)
    return ctypes.CDLL(str(path))


_o = _lib(HERE / "libgru_oracle.so", "all")
_o.oracle_gru_make_params.argtypes = [ctypes.POINTER(A.GruRanges), ctypes.POINTER(A.GruConfig),
                                      ctypes.POINTER(A.GruQParams)]
_o.oracle_gru_make_luts.argtypes = [ctypes.POINTER(A.GruQParams), ctypes.POINTER(A.PwlLut)]
_o.oracle_effective_scale.restype = ctypes.c_float
_o.oracle_effective_scale.argtypes = [ctypes.c_float, ctypes.c_int32]
_o.oracle_pwl_eval.restype = ctypes.c_float
_o.oracle_pwl_eval.argtypes = [ctypes.c_float, ctypes.POINTER(A.PwlLut), ctypes.c_int32,
                               ctypes.c_int32]
_o.oracle_gru_forward_calibrate.argtypes = [_i] * 4 + [_P] * 9
_o.oracle_gru_forward_quant.argtypes = [_i] * 5 + [_P] * 6 + [ctypes.POINTER(A.GruQParams)] + [_P] * 18
_o.oracle_gru_backward_quant.argtypes = [_i] * 4 + [_P] * 8 + [ctypes.POINTER(A.GruQParams)] + \
    [_P] * 11 + [_P] * 6
_o.oracle_gru_forward_int.argtypes = [_i] * 5 + [_P] * 8 + [ctypes.POINTER(A.GruQParams)] + \
    [_P] * 7 + [_P] * 11

_o.oracle_gru_set_sum_mode.argtypes = [_i]
SUM_EXACT, SUM_SEQ_F32 = 0, 1


def set_sum_mode(mode: int) -> None:
    """GEMM-sum model of the FP32-carrier forward: SUM_EXACT (the kernels' exact integer
    sums, the default) or SUM_SEQ_F32 (fp32 products added in K order, an SGEMM model)."""
    _o.oracle_gru_set_sum_mode(int(mode))


_REF_PATH = HERE / "_ref" / "libgru_ref.so"
_ref = ctypes.CDLL(str(_REF_PATH)) if _REF_PATH.exists() else None
if _ref is not None:
    _ref.ref_gru_make_params.argtypes = [ctypes.POINTER(A.GruRanges), ctypes.POINTER(A.GruConfig),
                                         ctypes.POINTER(A.GruQParams), ctypes.POINTER(A.PwlLut)]
    _ref.ref_gru_forward_calibrate.argtypes = [_i] * 4 + [_P] * 9
    _ref.ref_gru_forward_ptq.argtypes = [_i] * 4 + [_P] * 6 + [ctypes.POINTER(A.GruRanges),
                                                                ctypes.POINTER(A.GruConfig), _P, _P]
    _ref.ref_gru_forward_int_codes.argtypes = [_i] * 4 + [_P] * 8 + \
        [ctypes.POINTER(A.GruQParams)] + [_P] * 7


def has_ref() -> bool:
    return _ref is not None


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a):
    return None if a is None else np.ascontiguousarray(a, dtype=f32)


def make_params(ranges, cfg, ref: bool = False):
    qp = A.new_qparams(ranges.hidden)
    luts = (A.PwlLut * 3)()
    if ref:
        rc = _ref.ref_gru_make_params(ctypes.byref(ranges), ctypes.byref(cfg), ctypes.byref(qp), luts)
    else:
        rc = _o.oracle_gru_make_params(ctypes.byref(ranges), ctypes.byref(cfg), ctypes.byref(qp))
        _o.oracle_gru_make_luts(ctypes.byref(qp), luts)
    if rc != 0:
        raise RuntimeError(f"make_params failed ({rc})")
    return qp, luts


def make_luts(qp):
    luts = (A.PwlLut * 3)()
    _o.oracle_gru_make_luts(ctypes.byref(qp), luts)
    return luts


def effective_scale(scale: float, use_pot2: bool) -> float:
    return float(_o.oracle_effective_scale(scale, int(use_pot2)))


def pwl_eval(q: float, lut, bits: int, uns: int) -> float:
    return float(_o.oracle_pwl_eval(q, ctypes.byref(lut), bits, uns))


def forward_calibrate(W, R, bw, br, x, h0=None, ref: bool = False, stats=None):
    T, B, I = x.shape
    H = R.shape[0]
    W, R, bw, br, x, h0 = (_c(a) for a in (W, R, bw, br, x, h0))
    h = np.zeros((T + 1, B, H), f32)
    v = np.zeros((T, B, 4 * H), f32)
    s = A.empty_stats(H) if stats is None else stats
    fn = _ref.ref_gru_forward_calibrate if ref else _o.oracle_gru_forward_calibrate
    if ref:
        tmp = np.empty_like(s)
        rc = fn(T, B, I, H, _p(W), _p(R), _p(bw), _p(br), _p(x), _p(h0), _p(h), _p(v), _p(tmp))
        C = 3 * H
        n = A.NGRIDS
        s[:n] = np.minimum(s[:n], tmp[:n])
        s[n:2 * n] = np.maximum(s[n:2 * n], tmp[n:2 * n])
        for k in range(A.NCHAN):
            b0 = 2 * n + 2 * k * C
            s[b0:b0 + C] = np.minimum(s[b0:b0 + C], tmp[b0:b0 + C])
            s[b0 + C:b0 + 2 * C] = np.maximum(s[b0 + C:b0 + 2 * C], tmp[b0 + C:b0 + 2 * C])
    else:
        rc = fn(T, B, I, H, _p(W), _p(R), _p(bw), _p(br), _p(x), _p(h0), _p(h), _p(v), _p(s))
    if rc != 0:
        raise RuntimeError("forward_calibrate failed")
    return h, v, s


def forward_quant(W, R, bw, br, x, qp, h0=None, training=True):
    """Returns a dict with the 18 outputs of forward_quant_float_storage."""
    T, B, I = x.shape
    H = R.shape[0]
    C = 3 * H
    W, R, bw, br, x, h0 = (_c(a) for a in (W, R, bw, br, x, h0))
    o = {
        "h": np.zeros((T + 1, B, H), f32), "v": np.zeros((T, B, 4 * H), f32),
        "W_q": np.zeros((I, C), f32), "R_q": np.zeros((H, C), f32), "bw_q": np.zeros(C, f32),
        "br_q": np.zeros(C, f32), "x_q": np.zeros((T, B, I), f32),
    }
    mk = {
        "x_mask": (T, B, I), "h0_mask": (B, H), "W_mask": (I, C), "R_mask": (H, C), "bw_mask": (C,),
        "br_mask": (C,), "ih_mask": (T, B, C), "hh_mask": (T, B, C), "gate_in_mask": (T, B, C),
        "gate_out_mask": (T, B, C), "h_mask": (T, B, H),
    }
    for k, shp in mk.items():
        o[k] = np.zeros(shp, np.uint8) if (training and (k != "h0_mask" or h0 is not None)) else None
    rc = _o.oracle_gru_forward_quant(
        int(training), T, B, I, H, _p(W), _p(R), _p(bw), _p(br), _p(x), _p(h0), ctypes.byref(qp),
        *(_p(o[k]) for k in ("h", "v", "W_q", "R_q", "bw_q", "br_q", "x_q")),
        *(_p(o[k]) for k in mk))
    if rc != 0:
        raise RuntimeError("forward_quant failed")
    return o


MASKS = ("x_mask", "h0_mask", "W_mask", "R_mask", "bw_mask", "br_mask", "ih_mask", "hh_mask",
         "gate_in_mask", "gate_out_mask", "h_mask")


def backward_quant(fwd, dh_new, qp):
    T, B, I = fwd["x_q"].shape
    H = fwd["R_q"].shape[0]
    C = 3 * H
    out = {"dx": np.zeros((T, B, I), f32), "dW": np.zeros((I, C), f32), "dR": np.zeros((H, C), f32),
           "dbw": np.zeros(C, f32), "dbr": np.zeros(C, f32), "dh0": np.zeros((B, H), f32)}
    dh_new = _c(dh_new)
    rc = _o.oracle_gru_backward_quant(
        T, B, I, H, *(_p(fwd[k]) for k in ("W_q", "R_q", "bw_q", "br_q", "x_q")), _p(dh_new),
        _p(fwd["h"]), _p(fwd["v"]), ctypes.byref(qp), *(_p(fwd[k]) for k in MASKS),
        *(_p(out[k]) for k in ("dx", "dW", "dR", "dbw", "dbr", "dh0")))
    if rc != 0:
        raise RuntimeError("backward_quant failed")
    return out


def ref_forward_ptq(W, R, bw, br, x, ranges, cfg, h0=None):
    """Reference CPU PTQ forward (integer carrier), h [T+1,B,H] dequantised."""
    T, B, I = x.shape
    H = R.shape[0]
    W, R, bw, br, x, h0 = (_c(a) for a in (W, R, bw, br, x, h0))
    h = np.zeros((T + 1, B, H), f32)
    v = np.zeros((T, B, 4 * H), f32)
    rc = _ref.ref_gru_forward_ptq(T, B, I, H, _p(W), _p(R), _p(bw), _p(br), _p(x), _p(h0),
                                  ctypes.byref(ranges), ctypes.byref(cfg), _p(h), _p(v))
    if rc != 0:
        raise RuntimeError("ref forward_ptq failed")
    return h, v


I32 = np.int32


def _ci(a):
    return None if a is None else np.ascontiguousarray(a, dtype=I32)


def forward_int(W, R, bw, br, x, qp, h0=None, training=True, x_q=None, h0_q=None):
    """int32 carrier (forward_quant_int_storage / forward_quantized_int_io semantics).

    With x_q (int32 [T,B,I]) given, x is ignored and the codes are used as they are, and
    h0_q (int32 [B,H]) likewise replaces h0.  Returns int32 codes h_q [T+1,B,H],
    v_q [T,B,4H], W_q, R_q, bw_q, br_q, x_q and, in training, the eleven uint8 masks."""
    T, B, I = (x_q if x_q is not None else x).shape
    H = R.shape[0]
    C = 3 * H
    W, R, bw, br, x, h0 = (_c(a) for a in (W, R, bw, br, x, h0))
    x_q, h0_q = _ci(x_q), _ci(h0_q)
    o = {
        "h_q": np.zeros((T + 1, B, H), I32), "v_q": np.zeros((T, B, 4 * H), I32),
        "W_q": np.zeros((I, C), I32), "R_q": np.zeros((H, C), I32), "bw_q": np.zeros(C, I32),
        "br_q": np.zeros(C, I32),
        "x_q": x_q.copy() if x_q is not None else np.zeros((T, B, I), I32),
    }
    mk = {
        "x_mask": (T, B, I), "h0_mask": (B, H), "W_mask": (I, C), "R_mask": (H, C), "bw_mask": (C,),
        "br_mask": (C,), "ih_mask": (T, B, C), "hh_mask": (T, B, C), "gate_in_mask": (T, B, C),
        "gate_out_mask": (T, B, C), "h_mask": (T, B, H),
    }
    skip = set()
    if x_q is not None:
        skip.add("x_mask")
    if h0 is None or h0_q is not None:
        skip.add("h0_mask")
    for k, shp in mk.items():
        o[k] = np.zeros(shp, np.uint8) if (training and k not in skip) else None
    rc = _o.oracle_gru_forward_int(
        int(training), T, B, I, H, _p(W), _p(R), _p(bw), _p(br), _p(x), _p(x_q), _p(h0),
        _p(h0_q), ctypes.byref(qp),
        *(_p(o[k]) for k in ("h_q", "v_q", "W_q", "R_q", "bw_q", "br_q")),
        None if x_q is not None else _p(o["x_q"]), *(_p(o[k]) for k in mk))
    if rc != 0:
        raise RuntimeError("forward_int failed")
    return o


def dequant_int(codes, grid, use_pot2: bool):
    """dequantize(q, FixedPointScale, zp): (q - zp) in int32, converted, times the effective
    scale (quantize_ops_helper.h:450-454)."""
    d = (np.asarray(codes, I32) - I32(grid.zero_point)).astype(f32)
    return d * f32(effective_scale(grid.scale, use_pot2))


def ref_forward_int_codes(W, R, bw, br, x, qp, h0=None, x_q=None, h0_q=None, with_v=True):
    """The reference's CPU int32 carrier on codes (oracle/_ref ref_gru_forward_int_codes)."""
    T, B, I = (x_q if x_q is not None else x).shape
    H = R.shape[0]
    C = 3 * H
    W, R, bw, br, x, h0 = (_c(a) for a in (W, R, bw, br, x, h0))
    x_q, h0_q = _ci(x_q), _ci(h0_q)
    o = {"h_q": np.zeros((T + 1, B, H), I32),
         "v_q": np.zeros((T, B, 4 * H), I32) if with_v else None,
         "W_q": np.zeros((I, C), I32), "R_q": np.zeros((H, C), I32), "bw_q": np.zeros(C, I32),
         "br_q": np.zeros(C, I32), "x_q": np.zeros((T, B, I), I32)}
    rc = _ref.ref_gru_forward_int_codes(
        T, B, I, H, _p(W), _p(R), _p(bw), _p(br), _p(x), _p(x_q), _p(h0), _p(h0_q),
        ctypes.byref(qp), *(_p(o[k]) for k in ("h_q", "v_q", "W_q", "R_q", "bw_q", "br_q", "x_q")))
    if rc != 0:
        raise RuntimeError("ref forward_int_codes failed")
    return o
