"""MI355X host side of the ONNX Runtime custom op QcQuantizeOp: the objects the reference's
Python front end drives through pybind11 — ``libquant_info.QcQuantizeInfo``
(native/onnx/src/QcQuantizeInfo.cpp:45-60), ``libpymo.BlockTensorQuantizer`` /
``libpymo.TfEncoding`` / ``TensorQuantizerOpMode`` (native/common/bindings/python) — and the op
call itself (QcQuantizeOp.cpp:101-170), all over include/rxmet_qc.h.

The statistics and encodings live on the GPU; tensors are CUDA (HIP) tensors of float32 or
float16 and every call runs on PyTorch's current stream.  numpy arrays are accepted where the
reference's bindings take them (copied to the GPU; results come back as numpy).  There is no
CPU path: without librxmet.so every call raises.
"""
from __future__ import annotations

import ctypes
import enum
from dataclasses import dataclass
from typing import List, Optional, Sequence

import numpy as np
import torch

import rxmet_lib as _rx
import rxmet_qc_abi as _abi

__all__ = ["TensorQuantizerOpMode", "OpMode", "TfEncoding", "BlockTensorQuantizer",
           "QcQuantizeInfo", "qc_quantize_op"]


class TensorQuantizerOpMode(enum.IntEnum):
    """TensorQuantizerOpFacade.h:48-54."""
    updateStats = 0
    oneShotQuantizeDequantize = 1
    quantizeDequantize = 2
    passThrough = 3


OpMode = TensorQuantizerOpMode


@dataclass
class TfEncoding:
    """libpymo.TfEncoding (Quantization.hpp:114-121)."""
    min: float = 0.0
    max: float = 0.0
    delta: float = 0.0
    offset: float = 0.0
    bw: int = 0


def _io(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return 0  # RXMET_QDQ_F32
    if t.dtype == torch.float16:
        return 1  # RXMET_QDQ_F16
    raise TypeError(f"QcQuantizeOp takes float32 or float16 tensors, not {t.dtype}")


def _device_tensor(x, device=None):
    """(contiguous CUDA tensor, was_numpy)."""
    if isinstance(x, np.ndarray):
        if device is None:
            device = torch.device("cuda", torch.cuda.current_device())
        return torch.from_numpy(np.ascontiguousarray(x)).to(device), True
    if not isinstance(x, torch.Tensor) or not x.is_cuda:
        raise TypeError("QcQuantizeOp runs on the GPU: pass a CUDA tensor or a numpy array")
    return x.contiguous(), False


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


class BlockTensorQuantizer:
    """libpymo.BlockTensorQuantizer(shape, bitwidth, QUANTIZATION_TF) on the current GPU
    (TensorQuantizer.h:265-345)."""

    def __init__(self, shape: Sequence[int], bitwidth: int, quant_scheme: str = "tf"):
        if str(quant_scheme).lower() not in ("tf", "quantization_tf", "post_training_tf",
                                             "quantscheme.post_training_tf"):
            raise ValueError(f"only the TF (min / max) scheme is implemented, not {quant_scheme}")
        self.shape = tuple(int(d) for d in shape)
        arr, nd = _abi.dims(self.shape)
        _rx.load()
        self._h = _rx.load().rxmet_block_tensor_quantizer_create(arr, nd, int(bitwidth))
        if not self._h:
            raise _rx.RxmetError(_rx.load().rxmet_last_error().decode())
        self._device = torch.device("cuda", torch.cuda.current_device())

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            _rx.load().rxmet_block_tensor_quantizer_destroy(h)
            self._h = None

    @property
    def handle(self) -> int:
        return self._h

    def _state(self) -> _abi.QuantizerState:
        st = _abi.QuantizerState()
        _rx.call("rxmet_block_tensor_quantizer_get_state", self._h, ctypes.byref(st))
        return st

    @property
    def num_encodings(self) -> int:
        return int(self._state().num_encodings)

    @property
    def bitwidth(self) -> int:
        return int(self._state().bitwidth)

    @bitwidth.setter
    def bitwidth(self, bw: int) -> None:
        _rx.call("rxmet_block_tensor_quantizer_set_bitwidth", self._h, int(bw))

    @property
    def isEncodingValid(self) -> bool:  # noqa: N802 (the reference's name)
        return bool(self._state().is_encoding_valid)

    def getStrictSymmetric(self) -> bool:  # noqa: N802
        return bool(self._state().use_strict_symmetric)

    def setStrictSymmetric(self, on: bool) -> None:  # noqa: N802
        _rx.call("rxmet_block_tensor_quantizer_set_strict_symmetric", self._h, int(bool(on)))

    def getUnsignedSymmetric(self) -> bool:  # noqa: N802
        return bool(self._state().use_unsigned_symmetric)

    def setUnsignedSymmetric(self, on: bool) -> None:  # noqa: N802
        _rx.call("rxmet_block_tensor_quantizer_set_unsigned_symmetric", self._h, int(bool(on)))

    def resetEncodingStats(self) -> None:  # noqa: N802
        s = torch.cuda.current_stream(self._device).cuda_stream
        _rx.call("rxmet_block_tensor_quantizer_reset_encoding_stats", self._h, s)

    def updateStats(self, tensor) -> None:  # noqa: N802
        t, _ = _device_tensor(tensor, self._device)
        arr, nd = _abi.dims(t.shape)
        _rx.call("rxmet_block_tensor_quantizer_update_stats", self._h, t.data_ptr(), _io(t), arr,
                 nd, None, _stream(t))

    def computeEncodings(self, useSymmetricEncodings: bool) -> List[TfEncoding]:  # noqa: N802,N803
        """Computes the encodings from the statistics and installs them (the reference's
        callers follow computeEncodings with setEncodings of the result)."""
        s = torch.cuda.current_stream(self._device).cuda_stream
        _rx.call("rxmet_block_tensor_quantizer_compute_encodings", self._h,
                 int(bool(useSymmetricEncodings)), s)
        return self.getEncodings()

    def setEncodings(self, encodings: Sequence[TfEncoding]) -> None:  # noqa: N802
        n = len(encodings)
        arr = (_abi.TfEncodingC * max(1, n))()
        for i, e in enumerate(encodings):
            arr[i] = _abi.TfEncodingC(float(e.min), float(e.max), float(e.delta),
                                      float(e.offset), int(e.bw), 0)
        s = torch.cuda.current_stream(self._device).cuda_stream
        _rx.call("rxmet_block_tensor_quantizer_set_encodings", self._h, arr, n, s)

    def getEncodings(self) -> List[TfEncoding]:  # noqa: N802
        n = self.num_encodings
        arr = (_abi.TfEncodingC * n)()
        s = torch.cuda.current_stream(self._device).cuda_stream
        _rx.call("rxmet_block_tensor_quantizer_get_encodings", self._h, arr, n, s)
        return [TfEncoding(e.min, e.max, e.delta, e.offset, e.bw) for e in arr]

    def getStats(self):  # noqa: N802
        """(min, max) running statistics as float32 numpy arrays."""
        n = self.num_encodings
        mn = np.empty(n, np.float32)
        mx = np.empty(n, np.float32)
        s = torch.cuda.current_stream(self._device).cuda_stream
        _rx.call("rxmet_block_tensor_quantizer_get_stats", self._h, mn.ctypes.data,
                 mx.ctypes.data, n, s)
        return mn, mx

    def quantizeDequantize(self, tensor):  # noqa: N802
        t, was_np = _device_tensor(tensor, self._device)
        y = torch.empty_like(t)
        arr, nd = _abi.dims(t.shape)
        _rx.call("rxmet_block_tensor_quantizer_quantize_dequantize", self._h, t.data_ptr(),
                 y.data_ptr(), _io(t), arr, nd, _stream(t))
        return y.cpu().numpy() if was_np else y


class QcQuantizeInfo:
    """libquant_info.QcQuantizeInfo (QcQuantizeInfo.cpp:45-60): the per-node state an ONNX
    graph's QcQuantizeOp refers to through its int64 "quant_info" attribute (``address``)."""

    def __init__(self):
        self._c = _abi.QcQuantizeInfoC()
        self._c.enabled = 1
        self._c.op_mode = int(OpMode.passThrough)
        self._c.is_int_data_type = 1
        self._q: Optional[BlockTensorQuantizer] = None
        self._name = b""

    @property
    def address(self) -> int:
        """The struct's address: the value of the node's "quant_info" attribute."""
        return ctypes.addressof(self._c)

    @property
    def c_struct(self) -> _abi.QcQuantizeInfoC:
        return self._c

    @property
    def tensorQuantizerRef(self) -> Optional[BlockTensorQuantizer]:  # noqa: N802
        return self._q

    @tensorQuantizerRef.setter
    def tensorQuantizerRef(self, q: Optional[BlockTensorQuantizer]) -> None:  # noqa: N802
        self._q = q
        self._c.tensor_quantizer = q.handle if q is not None else None

    @property
    def encoding(self) -> List[TfEncoding]:
        return self._q.getEncodings() if self._q is not None else []

    @encoding.setter
    def encoding(self, enc: Sequence[TfEncoding]) -> None:
        if self._q is None:
            raise RuntimeError("Cannot set encodings before instantiating tensor quantizer")
        self._q.setEncodings(enc)

    def _int_field(name, conv=int):  # noqa: N805
        def get(self):
            return conv(getattr(self._c, name))

        def set_(self, v):
            setattr(self._c, name, int(v))
        return property(get, set_)

    opMode = _int_field("op_mode", OpMode)
    useSymmetricEncoding = _int_field("use_symmetric_encoding", bool)
    enabled = _int_field("enabled", bool)
    isIntDataType = _int_field("is_int_data_type", bool)
    usePerChannelMode = _int_field("use_per_channel_mode", bool)
    channelAxis = _int_field("channel_axis")
    blockAxis = _int_field("block_axis")
    blockSize = _int_field("block_size")
    del _int_field

    @property
    def name(self) -> str:
        return self._name.decode()

    @name.setter
    def name(self, v: str) -> None:
        self._name = str(v).encode()
        self._c.name = self._name


def qc_quantize_op(info: QcQuantizeInfo, x: torch.Tensor) -> torch.Tensor:
    """One QcQuantizeOp node on a float32 / float16 CUDA tensor: allocates the output and runs
    QcQuantizeOp::computeImpl (QcQuantizeOp.cpp:101-170) on the current stream."""
    t, was_np = _device_tensor(x)
    y = torch.empty_like(t)
    arr, nd = _abi.dims(t.shape)
    _rx.call("rxmet_qc_quantize_compute", ctypes.byref(info.c_struct), t.data_ptr(),
             y.data_ptr(), _io(t), arr, nd, None, _stream(t))
    return y.cpu().numpy() if was_np else y
