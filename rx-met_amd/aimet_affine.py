"""aimet_torch affine-quantizer surface, restated over the MI355X backend.

aimet_torch cannot be imported in this environment (its backend module imports
``onnx``/``onnxscript`` at top level), so this module restates the pieces of its public
API that the fake-quantization hot path goes through, with the same names, argument
handling and encoding math, and routes every tensor-sized operation to
``mi355x_qdq`` (HIP kernels):

* backend registry — ``add_backend``, ``set_backend``, ``set_global_backend``,
  ``get_backend`` (``src/aimet_torch/v2/quantization/affine/backends/utils.py:76-113``);
* dispatchers ``quantize``, ``quantize_dequantize``, ``dequantize`` with ``_parse_args``
  (``backends/__init__.py:203-252, 403-440``);
* ``MinMaxEncodingAnalyzer`` (``v2/quantization/encoding_analyzer.py:92-272``) whose
  statistics pass is the fused min/max kernel;
* ``QuantizeDequantize`` (``v2/quantization/affine/quantizer.py:138-765, 947-1084``)
  parametrised by learnable ``min``/``max``, with ``get_scale`` / ``get_offset`` /
  ``set_range`` / ``compute_encodings``.

Only O(#encodings) bookkeeping (scale/offset from min/max, which autograd chains the
kernels' encoding gradients through) runs as PyTorch ops.
"""
from __future__ import annotations

import contextlib
import functools
import math
from itertools import chain, repeat
from typing import Optional, Tuple

import numpy as np
import torch
from torch import nn

import mi355x_qdq

# ---------------------------------------------------------------------------------
# Grid helpers (src/aimet_common/quantization_grid.py:10-21, quantsim.py:447-480)
# ---------------------------------------------------------------------------------


def integer_bounds(bitwidth: int, signed: bool, *, strict: bool = False):
    if type(bitwidth) is not int or not 1 <= bitwidth <= 64:
        raise ValueError("bitwidth must be an integer between 1 and 64")
    if type(signed) is not bool:
        raise ValueError("signed must be a boolean")
    low = -(1 << (bitwidth - 1)) if signed else 0
    high = (1 << (bitwidth - int(signed))) - 1
    return low + int(strict and signed), high


def symmetric_offset(qmin: int, qmax: int):
    return 0 if qmin >= 0 else -round((qmin + qmax) / 2)


def _get_minimum_scale(num_steps: int) -> float:
    """Smallest scale, rounded up to a power of two (quantsim.py:447-480)."""
    fp32_eps = float(np.finfo(np.float32).eps)
    raw_scale = min(fp32_eps, (0.005 - (-0.005)) / num_steps)
    return float(2.0 ** math.ceil(math.log2(raw_scale)))


class _StraightThroughEstimator(torch.autograd.Function):
    @staticmethod
    def forward(ctx, op, *args, **kwargs):  # pylint: disable=arguments-differ
        return op(*args, **kwargs)

    @staticmethod
    def backward(ctx, *grad):
        return (None, *grad)


def ste_round(*args, **kwargs):
    """Straight-through rounding (v2/utils.py:191-195)."""
    return _StraightThroughEstimator.apply(torch.round, *args, **kwargs)


# ---------------------------------------------------------------------------------
# Backend registry (backends/utils.py:76-113)
# ---------------------------------------------------------------------------------

_CURRENT_BACKEND = "mi355x"
_SUPPORTED_BACKENDS = {"mi355x": mi355x_qdq}


class _ContextManager:
    def __init__(self, action, cleanup):
        self._action = action
        self._cleanup = cleanup
        action()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self._cleanup()


def set_global_backend(name: str):
    global _CURRENT_BACKEND
    _CURRENT_BACKEND = name


def set_backend(name: str) -> _ContextManager:
    if name not in _SUPPORTED_BACKENDS:
        names = ", ".join(_SUPPORTED_BACKENDS.keys())
        raise RuntimeError(f"Backend '{name}' is not supported. Please choose one of: {names}")
    old = _CURRENT_BACKEND
    return _ContextManager(lambda: set_global_backend(name), lambda: set_global_backend(old))


def get_backend():
    return _SUPPORTED_BACKENDS[_CURRENT_BACKEND]


def add_backend(name: str, module):
    if name in _SUPPORTED_BACKENDS:
        return RuntimeError(f"{name} is exist.")
    _SUPPORTED_BACKENDS[name] = module
    return None


# ---------------------------------------------------------------------------------
# Dispatchers (backends/__init__.py:203-252, 403-440)
# ---------------------------------------------------------------------------------


def _derive_qmin_qmax(*, bitwidth: int = None, num_steps: int = None, signed: bool):
    if bitwidth is not None:
        num_steps = 2 ** bitwidth - 1
    if signed:
        return -math.ceil(num_steps / 2), math.floor(num_steps / 2)
    return 0, num_steps


def _parse_args(args, kwargs):
    args = tuple(chain(args, repeat(None, 4 - len(args))))
    arg0 = kwargs.get("qmin", kwargs.get("bitwidth", args[0]))
    arg1 = kwargs.get("qmax", kwargs.get("signed", args[1]))
    block_size = kwargs.get("block_size", None) or args[2]
    zero_point_shift = args[3] or kwargs.get("zero_point_shift", 0.0)
    if arg0 is None:
        qmin, qmax = _derive_qmin_qmax(num_steps=kwargs["num_steps"], signed=kwargs["signed"])
    elif arg1 is None or isinstance(arg1, bool):
        qmin, qmax = _derive_qmin_qmax(bitwidth=arg0, signed=bool(arg1))
    else:
        qmin, qmax = arg0, arg1
    return qmin, qmax, block_size, zero_point_shift


def quantize(tensor, scale, offset, *args, **kwargs):
    qmin, qmax, block_size, zps = _parse_args(args, kwargs)
    if zps != 0.0:
        raise RuntimeError("Nonzero zero_point_shift not supported for quantize()")
    return get_backend().quantize(tensor, scale, offset, qmin, qmax, block_size)


def quantize_dequantize(tensor, scale, offset, *args, **kwargs):
    qmin, qmax, block_size, zps = _parse_args(args, kwargs)
    return get_backend().quantize_dequantize(tensor, scale, offset, qmin, qmax, block_size, zps)


def dequantize(tensor, scale, offset, block_size=None):
    return get_backend().dequantize(tensor, scale, offset, block_size)


# ---------------------------------------------------------------------------------
# MinMax encoding analyzer (encoding_analyzer.py:92-272)
# ---------------------------------------------------------------------------------


class StatisticsNotFoundError(RuntimeError):
    pass


class _MinMaxRange:
    def __init__(self, mn=None, mx=None):
        self.min = mn
        self.max = mx


class _MinMaxObserver:
    def __init__(self, shape: tuple):
        self.shape = tuple(shape)
        self.stats = _MinMaxRange()

    @torch.no_grad()
    def collect_stats(self, input_tensor: torch.Tensor) -> _MinMaxRange:
        mn, mx = mi355x_qdq.minmax(input_tensor, self.shape)
        return _MinMaxRange(mn, mx)

    @torch.no_grad()
    def merge_stats(self, stats: _MinMaxRange):
        mn, mx = self.stats.min, self.stats.max
        if stats.min is not None:
            mn = stats.min.clone() if mn is None else torch.minimum(mn, stats.min)
        if stats.max is not None:
            mx = stats.max.clone() if mx is None else torch.maximum(mx, stats.max)
        self.stats = _MinMaxRange(mn, mx)

    def reset_stats(self):
        self.stats = _MinMaxRange()

    def get_stats(self):
        return self.stats


class MinMaxEncodingAnalyzer:
    def __init__(self, shape: tuple):
        self.observer = _MinMaxObserver(shape)

    @torch.no_grad()
    def update_stats(self, input_tensor: torch.Tensor):
        new = self.observer.collect_stats(input_tensor)
        self.observer.merge_stats(new)
        return new

    def reset_stats(self):
        self.observer.reset_stats()

    def compute_encodings(self, num_steps: int, is_symmetric: bool):
        return self.compute_encodings_from_stats(self.observer.get_stats(), num_steps, is_symmetric)

    @torch.no_grad()
    def compute_encodings_from_stats(self, stats: _MinMaxRange, num_steps: int, is_symmetric: bool):
        if num_steps <= 0:
            raise ValueError("The number of quantization bins cannot be less than or equal to 0.")
        if stats.min is None or stats.max is None:
            raise StatisticsNotFoundError("No statistics present to compute encodings.")
        minimum_scale = _get_minimum_scale(num_steps)
        min_with_zero = torch.clamp(stats.min, max=0)
        max_with_zero = torch.clamp(stats.max, min=0)
        tensor_diff = (max_with_zero - min_with_zero) / num_steps
        adjustment_step = minimum_scale * (tensor_diff < minimum_scale)
        if is_symmetric:
            updated_max = max_with_zero + math.floor(num_steps / 2) * adjustment_step
            updated_min = min_with_zero - math.ceil(num_steps / 2) * adjustment_step
            num_pos_steps = math.floor(num_steps / 2)
            num_neg_steps = math.ceil(num_steps / 2)
            extra = 1 if num_steps == 3 else 0
            delta = torch.maximum(updated_max / (num_pos_steps + extra), -updated_min / num_neg_steps)
            updated_min = -1 * num_neg_steps * delta
            updated_max = num_pos_steps * delta
        else:
            updated_max = max_with_zero + num_steps * adjustment_step
            updated_min = min_with_zero
        updated_max = torch.clamp(updated_max, max=torch.finfo(stats.min.dtype).max).to(stats.min.dtype)
        updated_min = torch.clamp(updated_min, min=torch.finfo(stats.max.dtype).min).to(stats.max.dtype)
        return updated_min, updated_max


# ---------------------------------------------------------------------------------
# QuantizeDequantize (quantizer.py:138-765, 947-1084)
# ---------------------------------------------------------------------------------


class QuantizeDequantize(nn.Module):
    """Fake-quantization module parametrised by learnable ``min``/``max``.

    ``QuantizeDequantize(shape, bitwidth, symmetric, encoding_analyzer=None,
    block_size=None, zero_point_shift=None, signed=True)`` or with explicit
    ``qmin``/``qmax`` — as in ``quantizer.py:138-219`` (``signed`` defaults to True).
    """

    def __init__(self, shape, *args, **kwargs):
        super().__init__()
        if isinstance(shape, int):
            shape = (shape,)
        self.shape = tuple(shape)
        signed = kwargs.pop("signed", True)
        args = tuple(chain(args, repeat(None, 6 - len(args))))
        arg0 = kwargs.pop("qmin", kwargs.pop("bitwidth", args[0]))
        arg1 = kwargs.pop("qmax", args[1])
        if arg1 is not None and not isinstance(arg1, bool):
            qmin, qmax = arg0, arg1
            symmetric = kwargs.pop("symmetric", True if args[2] is None else args[2])
            encoding_analyzer = kwargs.pop("encoding_analyzer", args[3])
            block_size = kwargs.pop("block_size", args[4])
            zero_point_shift = kwargs.pop("zero_point_shift", args[5])
        else:
            bitwidth = arg0
            symmetric = kwargs.pop("symmetric", True if args[1] is None else args[1])
            if bitwidth is None:
                raise TypeError("QuantizeDequantize needs a bitwidth or qmin/qmax")
            qmin, qmax = integer_bounds(bitwidth, signed)
            encoding_analyzer = kwargs.pop("encoding_analyzer", args[2])
            block_size = kwargs.pop("block_size", args[3])
            zero_point_shift = kwargs.pop("zero_point_shift", args[4])
        if kwargs:
            raise TypeError(f"QuantizeDequantize.__init__ got unexpected keyword argument: "
                            f"{', '.join(kwargs)}")
        if qmin >= qmax:
            raise ValueError(f"qmax should be strictly larger than qmin. Got qmax={qmax}, qmin={qmin}")
        self.qmin, self.qmax = int(qmin), int(qmax)
        self.symmetric = bool(symmetric)
        self.block_size = block_size
        self.zero_point_shift = zero_point_shift or 0.0
        if self.zero_point_shift not in (0.0, 0.5):
            raise ValueError(f"zero_point_shift should be 0.0 or 0.5. Got {self.zero_point_shift}")
        self.encoding_analyzer = encoding_analyzer or MinMaxEncodingAnalyzer(
            mi355x_qdq.get_encoding_shape_with_blocks(self.shape, self.block_size))
        self.min = nn.Parameter(-torch.ones(self.shape))
        self.max = nn.Parameter(torch.ones(self.shape))
        self._initialized = False

    @property
    def signed(self) -> bool:
        return self.qmin < 0

    @property
    def bitwidth(self) -> int:
        return int(math.log2(self.qmax - self.qmin + 1))

    def is_initialized(self) -> bool:
        return self._initialized

    def get_scale(self, dtype=None) -> Optional[torch.Tensor]:
        if not self.is_initialized():
            return None
        dtype = dtype or torch.float32
        num_steps = self.qmax - self.qmin
        scale = (self.max.to(dtype) - self.min.to(dtype)) / num_steps
        return scale.abs().clamp_min_(_get_minimum_scale(self.qmax - self.qmin)).to(dtype)

    def _get_offset(self, scale=None, dtype=None) -> Optional[torch.Tensor]:
        if not self.is_initialized():
            return None
        dtype = dtype or torch.float32
        if self.symmetric:
            offset = torch.full(self.shape, fill_value=symmetric_offset(self.qmin, self.qmax),
                                dtype=dtype, device=self.min.device)
        else:
            scale = scale if scale is not None else self.get_scale(dtype)
            offset = torch.clamp(ste_round(self.min / scale) - self.qmin, -self.qmax, -self.qmin)
        return offset.to(dtype)

    def get_offset(self, dtype=None):
        return self._get_offset(dtype=dtype)

    def get_min(self, dtype=None):
        if not self.is_initialized():
            return None
        return self.get_scale(dtype) * (self.get_offset(dtype) + self.qmin + self.zero_point_shift)

    def get_max(self, dtype=None):
        if not self.is_initialized():
            return None
        return self.get_scale(dtype) * (self.get_offset(dtype) + self.qmax + self.zero_point_shift)

    @torch.no_grad()
    def set_range(self, min, max):  # pylint: disable=redefined-builtin
        if min is None and max is None:
            return
        if min is not None:
            self.min.copy_(torch.as_tensor(min))
        if max is not None:
            self.max.copy_(torch.as_tensor(max))
        self._initialized = True

    @contextlib.contextmanager
    def compute_encodings(self):
        """Observe inputs; quantize with batch statistics meanwhile (quantizer.py:636-765)."""
        original_forward = self.forward
        shape = self.shape
        dtype, device = self.min.dtype, self.min.device

        @functools.wraps(original_forward)
        def forward_wrapper(input):  # pylint: disable=redefined-builtin
            expanded = mi355x_qdq.reshape_tensor_for_blocks(input, shape, self.block_size)
            observed = expanded.clamp_min(0) if self.symmetric and not self.signed else expanded
            stats = self.encoding_analyzer.update_stats(observed)
            num_steps = self.qmax - self.qmin - (1 if self.zero_point_shift == 0.5 else 0)
            dmin, dmax = self.encoding_analyzer.compute_encodings_from_stats(
                stats, num_steps, self.symmetric and self.signed)
            if self.block_size is not None:
                dmin, dmax = dmin.view(shape), dmax.view(shape)
            dmin = dmin.to(dtype=dtype, device=device).expand(shape)
            dmax = dmax.to(dtype=dtype, device=device).expand(shape)
            if self.symmetric and not self.signed:
                dmin = torch.zeros_like(dmin)
            saved = (self.min, self.max, self._initialized)
            try:
                self._parameters["min"], self._parameters["max"] = dmin, dmax
                self._initialized = True
                return original_forward(input)
            finally:
                self._parameters["min"], self._parameters["max"], self._initialized = saved

        self.encoding_analyzer.reset_stats()
        self.forward = forward_wrapper
        try:
            yield
        finally:
            del self.forward
        try:
            num_steps = self.qmax - self.qmin - (1 if self.zero_point_shift == 0.5 else 0)
            enc_min, enc_max = self.encoding_analyzer.compute_encodings(
                num_steps, self.symmetric and self.signed)
        except StatisticsNotFoundError:
            return
        if self.block_size is not None:
            enc_min, enc_max = enc_min.view(shape), enc_max.view(shape)
        if self.symmetric and not self.signed:
            enc_min = torch.zeros_like(enc_min)
        self.set_range(enc_min, enc_max)

    # True: with this build's backend, the encodings are derived from min / max inside the
    # quantize-dequantize kernels (rxmet_qdq_forward_minmax / _backward_minmax: one launch each
    # way plus the gradient fold); elsewhere (scale, offset) come from
    # rxmet_qdq_encoding_forward/_backward.  False: the reference's own get_encodings() tensor
    # expressions, i.e. what aimet_torch's QuantizeDequantize computes before it calls the
    # backend (quantizer.py:466-483, 1060-1082).
    fused_encodings = True

    def get_encodings(self) -> Optional[Tuple[torch.Tensor, torch.Tensor]]:
        if not self.is_initialized():
            return None
        scale = self.get_scale(dtype=torch.float32)
        offset = self._get_offset(scale=scale, dtype=torch.float32)
        return scale, offset

    def forward(self, input: torch.Tensor) -> torch.Tensor:  # pylint: disable=redefined-builtin
        if not self.is_initialized():
            raise RuntimeError(
                "Failed to run QuantizeDequantize since quantization parameters are not initialized."
                " Please initialize the quantization parameters using `compute_encodings()`.")
        mn, mx = self.min, self.max
        if self.fused_encodings and get_backend() is mi355x_qdq:
            y = mi355x_qdq.quantize_dequantize_minmax(
                input, mn, mx, self.qmin, self.qmax, self.symmetric,
                _get_minimum_scale(self.qmax - self.qmin),
                float(symmetric_offset(self.qmin, self.qmax)), self.block_size,
                self.zero_point_shift)
            if y is not None:
                return y
        if (self.fused_encodings and mn.is_cuda and mn.dtype == torch.float32
                and mx.dtype == torch.float32 and mn.is_contiguous() and mx.is_contiguous()):
            # get_encodings() in two launches instead of a chain of one-element tensor ops
            scale, offset = mi355x_qdq.minmax_encodings(
                mn, mx, self.qmin, self.qmax, self.symmetric,
                _get_minimum_scale(self.qmax - self.qmin),
                float(symmetric_offset(self.qmin, self.qmax)))
        else:
            scale, offset = self.get_encodings()
        return quantize_dequantize(input, scale, offset, self.qmin, self.qmax,
                                   block_size=self.block_size,
                                   zero_point_shift=self.zero_point_shift)
