"""ctypes layouts and signatures of include/rxmet_qc.h (the ONNX Runtime QcQuantizeOp C ABI)."""
from __future__ import annotations

import ctypes

import rxmet_lib as _rx

c_i32, c_i64, c_ptr = ctypes.c_int32, ctypes.c_int64, ctypes.c_void_p


class TfEncodingC(ctypes.Structure):
    """rxmet_tf_encoding = TfEncoding (Quantization.hpp:114-121)."""
    _fields_ = [("min", ctypes.c_double), ("max", ctypes.c_double), ("delta", ctypes.c_double),
                ("offset", ctypes.c_double), ("bw", c_i32), ("reserved", c_i32)]


class QuantizerState(ctypes.Structure):
    _fields_ = [("num_encodings", c_i64), ("bitwidth", c_i32), ("use_strict_symmetric", c_i32),
                ("use_unsigned_symmetric", c_i32), ("valid_stats", c_i32),
                ("is_encoding_valid", c_i32), ("reserved", c_i32)]


class QcQuantizeInfoC(ctypes.Structure):
    """rxmet_qc_quantize_info = QcQuantizeInfo (QcQuantizeInfo.h:40-75)."""
    _fields_ = [("tensor_quantizer", c_ptr), ("op_mode", c_i32),
                ("use_symmetric_encoding", c_i32), ("enabled", c_i32),
                ("is_int_data_type", c_i32), ("use_per_channel_mode", c_i32),
                ("channel_axis", c_i32), ("block_axis", c_i32), ("reserved", c_i32),
                ("block_size", c_i64), ("name", ctypes.c_char_p)]


_I64P = ctypes.POINTER(c_i64)
_ENC = ctypes.POINTER(TfEncodingC)
_INFO = ctypes.POINTER(QcQuantizeInfoC)

_SIGS = {
    "rxmet_block_tensor_quantizer_create": (c_ptr, [_I64P, c_i32, c_i32]),
    "rxmet_block_tensor_quantizer_destroy": (None, [c_ptr]),
    "rxmet_block_tensor_quantizer_get_state": (ctypes.c_int,
                                               [c_ptr, ctypes.POINTER(QuantizerState)]),
    "rxmet_block_tensor_quantizer_set_strict_symmetric": (ctypes.c_int, [c_ptr, c_i32]),
    "rxmet_block_tensor_quantizer_set_unsigned_symmetric": (ctypes.c_int, [c_ptr, c_i32]),
    "rxmet_block_tensor_quantizer_set_bitwidth": (ctypes.c_int, [c_ptr, c_i32]),
    "rxmet_block_tensor_quantizer_workspace_bytes": (c_i64, [c_ptr, _I64P, c_i32, c_i32]),
    "rxmet_block_tensor_quantizer_reset_encoding_stats": (ctypes.c_int, [c_ptr, c_ptr]),
    "rxmet_block_tensor_quantizer_update_stats": (ctypes.c_int, [c_ptr, c_ptr, c_i32, _I64P,
                                                                 c_i32, c_ptr, c_ptr]),
    "rxmet_block_tensor_quantizer_compute_encodings": (ctypes.c_int, [c_ptr, c_i32, c_ptr]),
    "rxmet_block_tensor_quantizer_set_encodings": (ctypes.c_int, [c_ptr, _ENC, c_i64, c_ptr]),
    "rxmet_block_tensor_quantizer_get_encodings": (ctypes.c_int, [c_ptr, _ENC, c_i64, c_ptr]),
    "rxmet_block_tensor_quantizer_get_stats": (ctypes.c_int, [c_ptr, c_ptr, c_ptr, c_i64,
                                                              c_ptr]),
    "rxmet_block_tensor_quantizer_quantize_dequantize": (ctypes.c_int, [c_ptr, c_ptr, c_ptr,
                                                                        c_i32, _I64P, c_i32,
                                                                        c_ptr]),
    "rxmet_qc_quantize_compute": (ctypes.c_int, [_INFO, c_ptr, c_ptr, c_i32, _I64P, c_i32,
                                                 c_ptr, c_ptr]),
    "rxmet_qc_quantize_workspace_bytes": (c_i64, [_INFO, _I64P, c_i32, c_i32]),
    "rxmet_qc_broadcast_layout": (ctypes.c_int, [_I64P, c_i32, _I64P, c_i32,
                                                 ctypes.POINTER(_rx.QdqLayout)]),
}
for _name, (_res, _args) in _SIGS.items():
    _rx.register(_name, _res, _args)


def dims(shape) -> tuple:
    """(int64 array, ndim) of a shape for the C calls."""
    shape = tuple(int(d) for d in shape)
    arr = (c_i64 * max(1, len(shape)))(*shape)
    return arr, len(shape)
