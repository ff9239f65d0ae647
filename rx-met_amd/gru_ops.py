"""MI355X replacement of the reference's pybind module ``gru_interface_binding``
(``operators/quant-gru/pytorch/lib/gru_interface_binding.cc:1331-1788``), i.e. the
``gru_ops`` object quant_gru.py calls.  Same function names, argument names, tensor
shapes and return tuples for the QAT path; every call goes to librxmet.so
(``include/rxmet_gru.h``) on PyTorch's current stream.
"""
from __future__ import annotations

import ctypes
from typing import Optional

import numpy as np
import torch

import rxmet_gru_abi as A
import rxmet_lib as _rx

use_real_activation = False
cpu_only = False


class OperatorQuantConfig:
    """Bit-width configuration (quantize_bitwidth_config.h:56-122), attribute names as the
    reference binding exposes them: ``<op>_`` bits, ``<op>symmetric_``, ``<op>unsigned_``,
    ``W/R/bw/br_granularity_``, ``usePOT2_``, ``pot_scale_method_``, ``pot_scale_tolerance_``."""

    _OPS = {"x_": "x", "h_": "h", "weight_ih_linear_": "weight_ih_linear",
            "weight_hh_linear_": "weight_hh_linear", "update_gate_input_": "update_gate_input",
            "reset_gate_input_": "reset_gate_input", "new_gate_input_": "new_gate_input",
            "update_gate_output_": "update_gate_output", "reset_gate_output_": "reset_gate_output",
            "new_gate_output_": "new_gate_output", "mul_reset_hidden_": "mul_reset_hidden",
            "mul_new_contribution_": "mul_new_contribution",
            "mul_old_contribution_": "mul_old_contribution"}
    _CHANS = {"W_": 0, "R_": 1, "bw_": 2, "br_": 3}

    def __init__(self):
        object.__setattr__(self, "_c", A.default_config())

    def _spec(self, base):
        if base in self._OPS:
            return self._c.op[A.GRID[self._OPS[base]]]
        if base in self._CHANS:
            return self._c.chan[self._CHANS[base]]
        return None

    def __getattr__(self, name):
        c = object.__getattribute__(self, "_c")
        if name == "usePOT2_":
            return bool(c.use_pot2)
        if name == "pot_scale_method_":
            return int(c.pot_method)
        if name == "pot_scale_tolerance_":
            return float(c.pot_tolerance)
        if name.endswith("_granularity_"):
            return int(self._c.chan[self._CHANS[name[:-len("granularity_")]]].granularity)
        for suffix, field in (("symmetric_", "symmetric"), ("unsigned_", "is_unsigned")):
            if name.endswith(suffix):
                spec = self._spec(name[:-len(suffix)])
                if spec is not None:
                    return bool(getattr(spec, field))
        spec = self._spec(name)
        if spec is not None:
            return int(spec.bits)
        raise AttributeError(name)

    def __setattr__(self, name, value):
        c = self._c
        if name == "usePOT2_":
            c.use_pot2 = int(bool(value))
            return
        if name == "pot_scale_method_":
            c.pot_method = int(value)
            return
        if name == "pot_scale_tolerance_":
            c.pot_tolerance = float(value)
            return
        if name.endswith("_granularity_"):
            c.chan[self._CHANS[name[:-len("granularity_")]]].granularity = int(value)
            return
        for suffix, field in (("symmetric_", "symmetric"), ("unsigned_", "is_unsigned")):
            if name.endswith(suffix):
                spec = self._spec(name[:-len(suffix)])
                if spec is not None:
                    setattr(spec, field, int(bool(value)))
                    return
        spec = self._spec(name)
        if spec is not None:
            bits = int(value)
            if not 1 <= bits <= 32:
                raise ValueError(f"bitwidth must be in [1, 32], got {bits}")
            spec.bits = bits
            return
        raise AttributeError(name)

    def to_struct(self) -> A.GruConfig:
        return self._c


class GRUQuantizationRanges:
    """MinMax statistics of one direction: flat vector in the layout of
    rxmet_gru_forward_calibrate, kept on the device between calibration batches."""

    def __init__(self, hidden_size: int, device=None):
        self.hidden_ = int(hidden_size)
        self.stats = torch.from_numpy(A.empty_stats(self.hidden_))
        if device is not None:
            self.stats = self.stats.to(device)

    def reset(self, hidden: int = -1):
        if hidden > 0:
            self.hidden_ = hidden
        self.stats = torch.from_numpy(A.empty_stats(self.hidden_)).to(self.stats.device)

    def to_struct(self):
        return A.make_ranges(self.stats.detach().cpu().numpy(), self.hidden_)


class GRUQuantParams:
    """Quantisation grids of one direction (quantize_param_types.h:88-118)."""

    def __init__(self, hidden: int = 0):
        self.hidden_ = int(hidden)
        self._qp = A.new_qparams(max(self.hidden_, 1))
        self.bitwidth_config_ = None
        self._device_cache = {}

    @classmethod
    def from_struct(cls, qp) -> "GRUQuantParams":
        """Wrap an existing rxmet_gru_qparams (e.g. grids loaded from elsewhere)."""
        out = cls(int(qp.hidden))
        out._qp.use_pot2 = qp.use_pot2
        for i in range(A.NGRIDS):
            out._qp.g[i] = qp.g[i]
        for k in range(A.NCHAN):
            out._qp.chan_bits[k] = qp.chan_bits[k]
            out._qp.chan_unsigned[k] = qp.chan_unsigned[k]
            A.qparams_chan(out._qp, k)[:] = A.qparams_chan(qp, k)
        return out

    @property
    def struct(self):
        return self._qp

    def scale(self, name: str) -> float:
        return float(self._qp.g[A.GRID[name]].scale)

    def zero_point(self, name: str) -> int:
        return int(self._qp.g[A.GRID[name]].zero_point)

    def channel_scales(self, name: str) -> np.ndarray:
        return A.qparams_chan(self._qp, A.CHAN[name])


def calculate_gru_quantitative_parameters(quant_ranges: GRUQuantizationRanges,
                                          bitwidth_config: OperatorQuantConfig) -> GRUQuantParams:
    """calculateGRUQuantitativeParameters (src/gru_host.cc:13-124), host code in librxmet."""
    params = GRUQuantParams(quant_ranges.hidden_)
    ranges = quant_ranges.to_struct()
    _rx.call("rxmet_gru_make_params", ctypes.byref(ranges), ctypes.byref(bitwidth_config.to_struct()),
             ctypes.byref(params.struct))
    params.bitwidth_config_ = bitwidth_config
    return params


def _check_f32_cuda(name, t):
    if not (t.is_cuda and t.dtype == torch.float32):
        raise RuntimeError(f"{name} must be CUDA float32 tensor")


def _stream(dev):
    return _rx.stream_of(dev)


def _ws(nbytes: int, dev) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=dev)


def forward_calibrate(is_training, time_steps, batch_size, input_size, hidden_size, W, R, bw, br, x,
                      h0, calib_method="minmax", bitwidth_config=None, quant_ranges=None,
                      hist_collectors=None):
    """Float GRU forward + MinMax statistics merged into ``quant_ranges``
    (forwardWithCalibrationGPU, src/gru_interface.cc:930-1024).  Returns (h, v)."""
    if calib_method != "minmax":
        raise NotImplementedError("only MinMax calibration is implemented on MI355X")
    for n, t in (("W", W), ("R", R), ("bw", bw), ("br", br), ("x", x)):
        _check_f32_cuda(n, t)
    dev = x.device
    T, B, I, H = time_steps, batch_size, input_size, hidden_size
    h = torch.empty((T + 1, B, H), dtype=torch.float32, device=dev)
    # gate values are only materialised when asked for (is_training); the ranges never need them
    v = torch.empty((T, B, 4 * H) if is_training else (0,), dtype=torch.float32, device=dev)
    if quant_ranges is None:
        raise RuntimeError("forward_calibrate needs quant_ranges (MinMax statistics)")
    if quant_ranges.hidden_ != H:
        raise RuntimeError("quant_ranges hidden size does not match hidden_size")
    if tuple(x.shape) != (T, B, I) or tuple(W.shape) != (I, 3 * H) or tuple(R.shape) != (H, 3 * H):
        raise RuntimeError("x/W/R shapes do not match (time_steps, batch_size, input_size, "
                           "hidden_size)")
    if quant_ranges.stats.device != dev:
        quant_ranges.stats = quant_ranges.stats.to(dev)
    h0p = h0.data_ptr() if (h0 is not None and h0.numel() > 0) else None
    ws = _ws(_rx.load().rxmet_gru_calibrate_workspace_bytes(T, B, I, H), dev)
    _rx.call("rxmet_gru_forward_calibrate", T, B, I, H, W.data_ptr(), R.data_ptr(), bw.data_ptr(),
             br.data_ptr(), x.data_ptr(), h0p, h.data_ptr(), v.data_ptr() if is_training else None,
             quant_ranges.stats.data_ptr(), ws.data_ptr(), _stream(dev))
    return h, v


def forward_fp(is_training, time_steps, batch_size, input_size, hidden_size, W, R, bw, br, x,
               h0=None):
    """Float GRU forward (forward_fp_wrapper, gru_interface_binding.cc:656-697).
    Returns (h [T+1,B,H], v [T,B,4H]); v is empty when is_training is False."""
    for n, t in (("W", W), ("R", R), ("bw", bw), ("br", br), ("x", x)):
        _check_f32_cuda(n, t)
    T, B, I, H = time_steps, batch_size, input_size, hidden_size
    dev = x.device
    has_h0 = h0 is not None and h0.numel() > 0
    if has_h0:
        _check_f32_cuda("h0", h0)
        if tuple(h0.shape) != (B, H):
            raise RuntimeError("h0 must have shape [batch_size, hidden_size]")
    h = torch.empty((T + 1, B, H), dtype=torch.float32, device=dev)
    v = torch.empty((T, B, 4 * H) if is_training else (0,), dtype=torch.float32, device=dev)
    _rx.call("rxmet_gru_forward_fp", int(bool(is_training)), T, B, I, H, W.data_ptr(),
             R.data_ptr(), bw.data_ptr(), br.data_ptr(), x.data_ptr(),
             h0.data_ptr() if has_h0 else None, h.data_ptr(),
             v.data_ptr() if is_training else None, _stream(dev))
    return h, v


MASK_NAMES = ("x_mask", "h0_mask", "W_mask", "R_mask", "bw_mask", "br_mask",
              "weight_ih_linear_mask", "weight_hh_linear_mask", "gate_input_mask",
              "gate_output_mask", "h_mask")


def _forward_dir(is_training, T, B, I, H, W, R, bw, br, x, h0, quant_params):
    """Check one direction's inputs and allocate its outputs; returns (outputs, FwdDir)."""
    for n, t in (("W", W), ("R", R), ("bw", bw), ("br", br), ("x", x)):
        _check_f32_cuda(n, t)
    has_h0 = h0 is not None and h0.numel() > 0
    if has_h0:
        _check_f32_cuda("h0", h0)
        if tuple(h0.shape) != (B, H):
            raise RuntimeError("h0 must have shape [batch_size, hidden_size]")
    dev = x.device
    C = 3 * H
    f32 = dict(dtype=torch.float32, device=dev)
    u8 = dict(dtype=torch.uint8, device=dev)
    h = torch.empty((T + 1, B, H), **f32)
    v = torch.empty((T, B, 4 * H), **f32) if is_training else torch.empty((0,), **f32)
    W_q = torch.empty((I, C), **f32)
    R_q = torch.empty((H, C), **f32)
    bw_q = torch.empty((C,), **f32)
    br_q = torch.empty((C,), **f32)
    x_q = torch.empty((T, B, I), **f32)
    if is_training:
        masks = [torch.empty((T, B, I), **u8),
                 torch.empty((B, H), **u8) if has_h0 else torch.empty((0,), **u8),
                 torch.empty((I, C), **u8), torch.empty((H, C), **u8), torch.empty((C,), **u8),
                 torch.empty((C,), **u8)] + [torch.empty((T, B, C), **u8) for _ in range(4)] + \
                [torch.empty((T, B, H), **u8)]
    else:
        masks = [torch.empty((0,), **u8) for _ in range(11)]
    ws = _ws(_rx.load().rxmet_gru_forward_workspace_bytes(T, B, I, H), dev)
    mp = [m.data_ptr() if m.numel() > 0 else None for m in masks]
    d = A.FwdDir(W.data_ptr(), R.data_ptr(), bw.data_ptr(), br.data_ptr(), x.data_ptr(),
                 h0.data_ptr() if has_h0 else None, ctypes.addressof(quant_params.struct),
                 h.data_ptr(), v.data_ptr() if is_training else None, W_q.data_ptr(),
                 R_q.data_ptr(), bw_q.data_ptr(), br_q.data_ptr(), x_q.data_ptr(), *mp,
                 ws.data_ptr())
    outs = (h, v, W_q, R_q, bw_q, br_q, x_q, *masks)
    return outs, d, ws


def forward_quant_float_storage(is_training, time_steps, batch_size, input_size, hidden_size, W, R,
                                bw, br, x, h0, quant_params: GRUQuantParams):
    """forward_quant_float_storage_wrapper (gru_interface_binding.cc:306-448).

    Returns (h, v, W_q, R_q, bw_q, br_q, x_q, x_mask, h0_mask, W_mask, R_mask, bw_mask,
    br_mask, weight_ih_linear_mask, weight_hh_linear_mask, gate_input_mask,
    gate_output_mask, h_mask); masks are empty tensors when is_training is False."""
    T, B, I, H = time_steps, batch_size, input_size, hidden_size
    outs, d, ws = _forward_dir(is_training, T, B, I, H, W, R, bw, br, x, h0, quant_params)
    _rx.call("rxmet_gru_forward_quant", int(bool(is_training)), T, B, I, H, d.W, d.R, d.bw, d.br,
             d.x, d.h0, ctypes.byref(quant_params.struct), d.h, d.v, d.W_q, d.R_q, d.bw_q, d.br_q,
             d.x_q, d.x_mask, d.h0_mask, d.W_mask, d.R_mask, d.bw_mask, d.br_mask, d.ih_mask,
             d.hh_mask, d.gate_in_mask, d.gate_out_mask, d.h_mask, d.workspace, _stream(x.device))
    return outs


def forward_quant_float_storage_dirs(is_training, time_steps, batch_size, input_size, hidden_size,
                                     dirs):
    """Both directions of a bidirectional layer in one call (rxmet_gru_forward_quant_dirs):
    ``dirs`` is a list of (W, R, bw, br, x, h0, quant_params) per direction; returns one
    forward_quant_float_storage result tuple per direction."""
    T, B, I, H = time_steps, batch_size, input_size, hidden_size
    made = [_forward_dir(is_training, T, B, I, H, *d) for d in dirs]
    arr = (A.FwdDir * len(made))(*[m[1] for m in made])
    _rx.call("rxmet_gru_forward_quant_dirs", len(made), int(bool(is_training)), T, B, I, H, arr,
             _stream(dirs[0][4].device))
    return [m[0] for m in made]


def forward_quant_float_storage_dirs_x(is_training, time_steps, batch_size, input_size,
                                       hidden_size, dirs, x_layouts):
    """forward_quant_float_storage_dirs with each direction's x read in place
    (rxmet_gru_forward_quant_dirs_x): ``x_layouts[k]`` = (t stride, b stride, reversed, flags)
    of direction k's x in elements (feature stride 1); flags bit 0: W, R, bw, br given in
    PyTorch's layout (weight_ih [3H, I], weight_hh [3H, H], (r, z, n) gate order)."""
    T, B, I, H = time_steps, batch_size, input_size, hidden_size
    for k, d in enumerate(dirs):
        if d[4].dim() != 3 or d[4].stride(2) != 1:
            raise RuntimeError(f"x of direction {k} needs a unit feature stride")
    made = [_forward_dir(is_training, T, B, I, H, *d) for d in dirs]
    arr = (A.FwdDir * len(made))(*[m[1] for m in made])
    lay = (ctypes.c_int64 * (4 * len(made)))(*[int(v) for xl in x_layouts for v in xl])
    _rx.call("rxmet_gru_forward_quant_dirs_x", len(made), int(bool(is_training)), T, B, I, H, arr,
             lay, _stream(dirs[0][4].device))
    return [m[0] for m in made]


def bidir_assemble(h_f, h_r, batch_first: bool):
    """(output, h_n) of a bidirectional layer from both directions' h [T+1, B, H]
    (rxmet_gru_bidir_assemble): output [T, B, 2H], or [B, T, 2H] when batch_first."""
    T1, B, H = h_f.shape
    T = T1 - 1
    shape = (B, T, 2 * H) if batch_first else (T, B, 2 * H)
    out = torch.empty(shape, dtype=torch.float32, device=h_f.device)
    h_n = torch.empty((2, B, H), dtype=torch.float32, device=h_f.device)
    st, sb = (out.stride(1), out.stride(0)) if batch_first else (out.stride(0), out.stride(1))
    _rx.call("rxmet_gru_bidir_assemble", T, B, H, h_f.data_ptr(), h_r.data_ptr(), out.data_ptr(),
             st, sb, h_n.data_ptr(), _stream(h_f.device))
    return out, h_n


def bidir_split_grad(g_out, g_hn, T, B, H, batch_first: bool, device):
    """Each direction's dh_new [T+1, B, H] from the output gradient (any strides, or None)
    and the h_n gradient (rxmet_gru_bidir_split_grad)."""
    f32 = dict(dtype=torch.float32, device=device)
    dh_f, dh_r = torch.empty((T + 1, B, H), **f32), torch.empty((T + 1, B, H), **f32)
    gp, st, sb, sk = None, 0, 0, 0
    if g_out is not None:
        _check_f32_cuda("grad_output", g_out)
        gp = g_out.data_ptr()
        st, sb = (g_out.stride(1), g_out.stride(0)) if batch_first else (g_out.stride(0),
                                                                          g_out.stride(1))
        sk = g_out.stride(2)
    hp = None
    if g_hn is not None and g_hn.numel() > 0:
        _check_f32_cuda("grad_h_n", g_hn)
        g_hn = g_hn.contiguous()
        hp = g_hn.data_ptr()
    _rx.call("rxmet_gru_bidir_split_grad", T, B, H, gp, st, sb, sk, hp, dh_f.data_ptr(),
             dh_r.data_ptr(), _stream(device))
    return dh_f, dh_r, g_hn


def bidir_dx(dx_f, dx_r, batch_first: bool):
    """Input gradient of a bidirectional layer in the caller's layout (rxmet_gru_bidir_dx)."""
    T, B, I = dx_f.shape
    shape = (B, T, I) if batch_first else (T, B, I)
    dx = torch.empty(shape, dtype=torch.float32, device=dx_f.device)
    st, sb = (dx.stride(1), dx.stride(0)) if batch_first else (dx.stride(0), dx.stride(1))
    _rx.call("rxmet_gru_bidir_dx", T, B, I, dx_f.data_ptr(), dx_r.data_ptr(), dx.data_ptr(), st, sb,
             _stream(dx_f.device))
    return dx


def _backward_dir(T, B, I, H, W_q, R_q, bw_q, br_q, x_q, dh_new, h, v, quant_params, masks,
                  torch_layout=False):
    C = 3 * H
    dev = x_q.device
    for n, t, shp in (("W_q", W_q, (I, C)), ("R_q", R_q, (H, C)), ("bw_q", bw_q, (C,)),
                      ("br_q", br_q, (C,)), ("x_q", x_q, (T, B, I)),
                      ("dh_new", dh_new, (T + 1, B, H)), ("h", h, (T + 1, B, H)),
                      ("v", v, (T, B, 4 * H))):
        _check_f32_cuda(n, t)
        if tuple(t.shape) != shp:
            raise RuntimeError(f"{n} must have shape {list(shp)}")
    f32 = dict(dtype=torch.float32, device=dev)
    outs = (torch.empty((T, B, I), **f32),
            torch.empty((C, I) if torch_layout else (I, C), **f32),
            torch.empty((C, H) if torch_layout else (H, C), **f32),
            torch.empty((C,), **f32), torch.empty((C,), **f32), torch.empty((B, H), **f32))
    mp = [m.data_ptr() if (m is not None and m.numel() > 0) else None for m in masks]
    dh_new = dh_new.contiguous()
    ws = _ws(_rx.load().rxmet_gru_backward_workspace_bytes(T, B, I, H), dev)
    d = A.BwdDir(W_q.data_ptr(), R_q.data_ptr(), bw_q.data_ptr(), br_q.data_ptr(), x_q.data_ptr(),
                 dh_new.data_ptr(), h.data_ptr(), v.data_ptr(),
                 ctypes.addressof(quant_params.struct), *mp, *[o.data_ptr() for o in outs],
                 ws.data_ptr())
    return outs, d, (ws, dh_new)


def backward_quant_float_storage(time_steps, batch_size, input_size, hidden_size, W_q, R_q, bw_q,
                                 br_q, x_q, dh_new, h, v, quant_params: GRUQuantParams, x_mask,
                                 h0_mask, W_mask, R_mask, bw_mask, br_mask, weight_ih_linear_mask,
                                 weight_hh_linear_mask, gate_input_mask, gate_output_mask, h_mask):
    """backward_quant_float_storage_wrapper (gru_interface_binding.cc:789-920).
    Returns (dx, dW, dR, dbw, dbr, dh).  The saved codes are not modified."""
    T, B, I, H = time_steps, batch_size, input_size, hidden_size
    masks = (x_mask, h0_mask, W_mask, R_mask, bw_mask, br_mask, weight_ih_linear_mask,
             weight_hh_linear_mask, gate_input_mask, gate_output_mask, h_mask)
    outs, d, keep = _backward_dir(T, B, I, H, W_q, R_q, bw_q, br_q, x_q, dh_new, h, v,
                                  quant_params, masks)
    _rx.call("rxmet_gru_backward_quant", T, B, I, H, d.W_q, d.R_q, d.bw_q, d.br_q, d.x_q,
             d.dh_new, d.h, d.v, ctypes.byref(quant_params.struct), d.x_mask, d.h0_mask, d.W_mask,
             d.R_mask, d.bw_mask, d.br_mask, d.ih_mask, d.hh_mask, d.gate_in_mask,
             d.gate_out_mask, d.h_mask, d.dx, d.dW, d.dR, d.dbw, d.dbr, d.dh0, d.workspace,
             _stream(x_q.device))
    return outs


def backward_quant_float_storage_dirs(time_steps, batch_size, input_size, hidden_size, dirs):
    """Both directions' backward in one call (rxmet_gru_backward_quant_dirs): ``dirs`` is a
    list of (W_q, R_q, bw_q, br_q, x_q, dh_new, h, v, quant_params, masks) per direction;
    returns one (dx, dW, dR, dbw, dbr, dh) tuple per direction."""
    T, B, I, H = time_steps, batch_size, input_size, hidden_size
    made = [_backward_dir(T, B, I, H, *d) for d in dirs]
    arr = (A.BwdDir * len(made))(*[m[1] for m in made])
    _rx.call("rxmet_gru_backward_quant_dirs", len(made), T, B, I, H, arr,
             _stream(dirs[0][4].device))
    return [m[0] for m in made]


def backward_quant_float_storage_dirs_x(time_steps, batch_size, input_size, hidden_size, dirs):
    """backward_quant_float_storage_dirs with the weight gradients in PyTorch's layout
    (rxmet_gru_backward_quant_dirs_x): per direction (dx, dW [3H, I], dR [3H, H], dbw [3H],
    dbr [3H], dh) in (r, z, n) gate order."""
    T, B, I, H = time_steps, batch_size, input_size, hidden_size
    made = [_backward_dir(T, B, I, H, *d, torch_layout=True) for d in dirs]
    arr = (A.BwdDir * len(made))(*[m[1] for m in made])
    _rx.call("rxmet_gru_backward_quant_dirs_x", len(made), T, B, I, H, arr, 1,
             _stream(dirs[0][4].device))
    return [m[0] for m in made]
