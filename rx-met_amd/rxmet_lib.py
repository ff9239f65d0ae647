"""ctypes binding of ``librxmet.so`` (the MI355X C ABI declared in ``include/*.h``).

The library is the only compute path of this package: if it is missing, every entry
point raises instead of falling back to anything else.  Calls pass raw device pointers
(``tensor.data_ptr()``) and PyTorch's current HIP stream, so kernels are ordered with
the caller's other work exactly like aten ops.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path
from typing import Optional

_PKG = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("RXMET_LIB", _PKG / "librxmet.so"))

_lib: Optional[ctypes.CDLL] = None

c_i64 = ctypes.c_int64
c_int = ctypes.c_int
c_ptr = ctypes.c_void_p
c_float = ctypes.c_float



class QdqLayout(ctypes.Structure):
    """rxmet_qdq_layout: [outer, C0, mid, C1, inner], encoding c0 * C1 + c1."""
    _fields_ = [("outer", c_i64), ("C0", c_i64), ("mid", c_i64), ("C1", c_i64), ("inner", c_i64)]


class QdqNumerics(ctypes.Structure):
    """rxmet_qdq_numerics: io / internal element types, zero_point_shift, 0-dim scale."""
    _fields_ = [("io_dtype", ctypes.c_int32), ("internal_dtype", ctypes.c_int32),
                ("zero_point_shift", ctypes.c_double), ("scalar_scale", ctypes.c_int32),
                ("reserved", ctypes.c_int32)]


class QdqMinMaxEnc(ctypes.Structure):
    """rxmet_qdq_minmax_enc: learnable min / max encodings derived inside the kernels."""
    _fields_ = [("min", c_ptr), ("max", c_ptr), ("symmetric", ctypes.c_int32),
                ("sym_offset", ctypes.c_float), ("min_scale", ctypes.c_float),
                ("reserved", ctypes.c_int32)]


_LAY = ctypes.POINTER(QdqLayout)
_MME = ctypes.POINTER(QdqMinMaxEnc)
_NUM = ctypes.POINTER(QdqNumerics)

# name -> (restype, argtypes); mirrors include/rxmet_qdq.h and include/rxmet_gru.h
_SIGNATURES = {
    "rxmet_last_error": (ctypes.c_char_p, []),
    "rxmet_abi_version": (c_int, []),
    "rxmet_qdq_workspace_bytes": (c_i64, [c_i64, c_i64, c_i64]),
    "rxmet_qdq_minmax": (c_int, [c_ptr, c_i64, c_i64, c_i64, c_ptr, c_ptr, c_ptr, c_ptr]),
    "rxmet_qdq_forward": (c_int, [c_ptr, c_ptr, c_i64, c_i64, c_i64, c_ptr, c_ptr, c_i64, c_i64,
                                  c_int, c_ptr]),
    "rxmet_qdq_backward": (c_int, [c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_ptr,
                                   c_ptr, c_i64, c_i64, c_int, c_ptr, c_ptr]),
    "rxmet_qdq_backward_noalloc": (c_int, [c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64,
                                           c_ptr, c_ptr, c_i64, c_i64, c_int, c_ptr]),
    "rxmet_quantize_forward": (c_int, [c_ptr, c_ptr, c_i64, c_i64, c_i64, c_ptr, c_ptr, c_i64,
                                       c_i64, c_ptr]),
    "rxmet_quantize_backward": (c_int, [c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64,
                                        c_ptr, c_ptr, c_i64, c_i64, c_ptr, c_ptr]),
    "rxmet_dequantize_forward": (c_int, [c_ptr, c_ptr, c_i64, c_i64, c_i64, c_ptr, c_ptr, c_ptr]),
    "rxmet_dequantize_backward": (c_int, [c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64,
                                          c_ptr, c_ptr, c_ptr, c_ptr]),
    "rxmet_qdq_workspace_bytes_ex": (c_i64, [_LAY, ctypes.c_int32]),
    "rxmet_qdq_minmax_ex": (c_int, [c_ptr, ctypes.c_int32, _LAY, c_ptr, c_ptr, c_ptr, c_ptr]),
    "rxmet_qdq_forward_ex": (c_int, [c_ptr, c_ptr, _LAY, _NUM, c_ptr, c_ptr, c_i64, c_i64, c_int,
                                     c_ptr]),
    "rxmet_qdq_backward_ex": (c_int, [c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, _LAY, _NUM, c_ptr, c_ptr,
                                      c_i64, c_i64, c_int, c_ptr, c_ptr]),
    "rxmet_qdq_forward_minmax": (c_int, [c_ptr, c_ptr, _LAY, _NUM, _MME, c_i64, c_i64, c_ptr]),
    "rxmet_qdq_backward_minmax": (c_int, [c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, _LAY, _NUM, _MME,
                                          c_i64, c_i64, c_ptr, c_ptr]),
    "rxmet_quantize_forward_ex": (c_int, [c_ptr, c_ptr, _LAY, _NUM, c_ptr, c_ptr, c_i64, c_i64,
                                          c_ptr]),
    "rxmet_quantize_backward_ex": (c_int, [c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, _LAY, _NUM, c_ptr,
                                           c_ptr, c_i64, c_i64, c_ptr, c_ptr]),
    "rxmet_dequantize_forward_ex": (c_int, [c_ptr, c_ptr, _LAY, _NUM, c_ptr, c_ptr, c_ptr]),
    "rxmet_dequantize_backward_ex": (c_int, [c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, _LAY, _NUM, c_ptr,
                                             c_ptr, c_ptr, c_ptr]),
    "rxmet_selftest_mfma": (c_int, [c_int, c_ptr, c_ptr, c_ptr, c_ptr]),
    "rxmet_qdq_encoding_forward": (c_int, [c_ptr, c_ptr, c_i64, c_i64, c_i64, ctypes.c_int32,
                                           ctypes.c_float, ctypes.c_float, c_ptr, c_ptr, c_ptr]),
    "rxmet_qdq_encoding_backward": (c_int, [c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64,
                                            ctypes.c_int32, ctypes.c_float, c_ptr, c_ptr, c_ptr]),
    "rxmet_prof_enable": (c_int, [ctypes.c_int32]),
    "rxmet_prof_filter": (c_int, [ctypes.c_char_p]),
    "rxmet_prof_reset": (c_int, []),
    "rxmet_prof_query": (c_int, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_double),
                                 ctypes.POINTER(c_i64)]),
    "rxmet_prof_names": (c_i64, [ctypes.c_char_p, c_i64]),
}



def exported() -> tuple:
    """Names of every typed entry point (tests check the library exports them all)."""
    return tuple(_SIGNATURES)


class RxmetError(RuntimeError):
    """Raised when a C-ABI call reports a failure (argument or HIP error)."""


def load() -> ctypes.CDLL:
    """Load and type the library once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RxmetError(
            f"{LIB_PATH} is missing: build it with `python rx-met_amd/build.py` "
            "(the MI355X kernels have no fallback)")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in _SIGNATURES.items():
        try:
            fn = getattr(lib, name)
        except AttributeError as e:
            raise RxmetError(f"{LIB_PATH} does not export {name}") from e
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def register(name: str, restype, argtypes) -> None:
    """Add a signature (used by modules that extend the ABI)."""
    _SIGNATURES[name] = (restype, argtypes)
    if _lib is not None:
        fn = getattr(_lib, name)
        fn.restype = restype
        fn.argtypes = argtypes


def call(name: str, *args) -> int:
    """Call ``name`` and raise RxmetError with the library's message on failure."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if isinstance(rc, int) and rc != 0:
        msg = lib.rxmet_last_error().decode(errors="replace")
        raise RxmetError(f"{name} failed ({rc}): {msg}")
    return rc


def ptr(t) -> Optional[int]:
    """Device pointer of a tensor, or None for a missing optional argument."""
    return None if t is None else t.data_ptr()


def stream_of(device) -> int:
    """Handle of PyTorch's current HIP stream on ``device``."""
    import torch

    return torch.cuda.current_stream(device).cuda_stream


def prof_enable(on: bool = True) -> None:
    """Turn the library's per-launch event timing on or off (include/rxmet_prof.h)."""
    load().rxmet_prof_enable(1 if on else 0)


def prof_filter(names=None) -> None:
    """Time only the named launches (an iterable of names; None: all)."""
    load().rxmet_prof_filter(None if names is None else ",".join(names).encode())


def prof_reset() -> None:
    load().rxmet_prof_reset()


def prof_query(name: str) -> tuple:
    """(total milliseconds, launches) recorded for an instrumented kernel name."""
    ms = ctypes.c_double(0.0)
    n = ctypes.c_int64(0)
    load().rxmet_prof_query(name.encode(), ctypes.byref(ms), ctypes.byref(n))
    return ms.value, n.value


def prof_names() -> list:
    lib = load()
    need = lib.rxmet_prof_names(None, 0)
    buf = ctypes.create_string_buffer(int(need) + 1)
    lib.rxmet_prof_names(buf, need + 1)
    return [n for n in buf.value.decode().split(",") if n]
