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
        if name in ("usePOT2_", "usePO2_"):
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
        if name in ("usePOT2_", "usePO2_"):
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

    def copy(self) -> "OperatorQuantConfig":
        out = OperatorQuantConfig()
        ctypes.pointer(out._c)[0] = self._c
        return out


# Reference attribute stems of the 13 activation grids (gru_interface_binding.cc:1365-1410
# names the two linear grids Wx / Rh in GRUQuantizationRanges).
_RANGE_GRID = {n: n for n in A.GRID_NAMES}
_RANGE_GRID.update(Wx="weight_ih_linear", Rh="weight_hh_linear")
del _RANGE_GRID["weight_ih_linear"], _RANGE_GRID["weight_hh_linear"]


_EMPTY_STATS = {}


def _empty_stats(hidden: int, device) -> torch.Tensor:
    """A fresh empty statistics vector; on a GPU a copy of a cached device template, so that
    a new calibration does not wait for the stream on a pageable host copy."""
    if device is None or torch.device(device).type == "cpu":
        return torch.from_numpy(A.empty_stats(hidden))
    key = (hidden, str(device))
    t = _EMPTY_STATS.get(key)
    if t is None:
        t = _EMPTY_STATS[key] = torch.from_numpy(A.empty_stats(hidden)).to(device)
    return t.clone()


class GRUQuantizationRanges:
    """MinMax statistics of one direction (GRUQuantizationRanges, gru_interface_binding.cc:
    1365-1410): a flat vector in the layout of rxmet_gru_forward_calibrate, kept on the device
    between calibration batches.  The reference's attributes read and write it: ``hidden_``,
    ``min_<op>_`` / ``max_<op>_`` for the 13 grids (``Wx``, ``Rh`` for the two linears) and
    per-channel lists ``min_W_``, ``max_W_``, ``min_R_``, .., ``max_br_`` of length 3H."""

    def __init__(self, hidden_size: int = 0, device=None):
        object.__setattr__(self, "hidden_", int(hidden_size))
        object.__setattr__(self, "stats", _empty_stats(self.hidden_, device))

    def reset(self, hidden: int = -1):
        if hidden > 0:
            object.__setattr__(self, "hidden_", int(hidden))
        self.stats = _empty_stats(self.hidden_, self.stats.device)

    def to_struct(self):
        return A.make_ranges(self.stats.detach().cpu().numpy(), self.hidden_)

    def _slot(self, name):
        for side, off in (("min_", 0), ("max_", A.NGRIDS)):
            if name.startswith(side) and name.endswith("_"):
                stem = name[len(side):-1]
                if stem in _RANGE_GRID:
                    return ("grid", off + A.GRID[_RANGE_GRID[stem]])
                if stem in A.CHAN:
                    C = 3 * self.hidden_
                    base = 2 * A.NGRIDS + 2 * A.CHAN[stem] * C + (C if side == "max_" else 0)
                    return ("chan", base)
        return None

    def __getattr__(self, name):
        slot = GRUQuantizationRanges._slot(self, name) if not name.startswith("__") else None
        if slot is None:
            raise AttributeError(name)
        kind, i = slot
        st = self.stats.detach().cpu()
        if kind == "grid":
            return float(st[i])
        return [float(v) for v in st[i:i + 3 * self.hidden_]]

    def __setattr__(self, name, value):
        slot = self._slot(name)
        if slot is None:
            if name == "hidden_":
                self.reset(int(value))
                return
            object.__setattr__(self, name, value)
            return
        kind, i = slot
        if kind == "grid":
            self.stats[i] = float(value)
        else:
            vals = torch.as_tensor(np.asarray(value, np.float32))
            if vals.numel() != 3 * self.hidden_:
                raise ValueError(f"{name} needs {3 * self.hidden_} values")
            self.stats[i:i + 3 * self.hidden_] = vals.to(self.stats.device)


class GRUQuantParams:
    """Quantisation grids of one direction (GRUQuantParams, quantize_param_types.h:88-118;
    binding attributes gru_interface_binding.cc:1480-1522): ``hidden_``, ``scale_<op>_`` /
    ``zp_<op>_`` for the 13 activation grids, per-channel lists ``scale_W_``, ``scale_R_``,
    ``scale_bw_``, ``scale_br_`` (3H values, zero points 0) and ``bitwidth_config_``, whose
    bit widths, signedness and power-of-two flag the grids take (as the reference's to_cpp)."""

    def __init__(self, hidden: int = 0):
        object.__setattr__(self, "_qp", A.new_qparams(max(int(hidden), 1)))
        self._qp.hidden = int(hidden)
        object.__setattr__(self, "_cfg", None)

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

    def _sync_config(self):
        cfg = self._cfg
        if cfg is None:
            return
        c = cfg.to_struct()
        for i in range(A.NGRIDS):
            self._qp.g[i].bits = c.op[i].bits
            self._qp.g[i].is_unsigned = c.op[i].is_unsigned
        for k in range(A.NCHAN):
            self._qp.chan_bits[k] = c.chan[k].bits
            self._qp.chan_unsigned[k] = c.chan[k].is_unsigned
        self._qp.use_pot2 = c.use_pot2

    @property
    def struct(self):
        self._sync_config()
        return self._qp

    @property
    def hidden_(self) -> int:
        return int(self._qp.hidden)

    @hidden_.setter
    def hidden_(self, value: int):
        value = int(value)
        if value == self._qp.hidden:
            return
        old = self._qp
        qp = A.new_qparams(max(value, 1))
        qp.hidden = value
        qp.use_pot2 = old.use_pot2
        for i in range(A.NGRIDS):
            qp.g[i] = old.g[i]
        for k in range(A.NCHAN):
            qp.chan_bits[k] = old.chan_bits[k]
            qp.chan_unsigned[k] = old.chan_unsigned[k]
        object.__setattr__(self, "_qp", qp)

    @property
    def bitwidth_config_(self):
        return self._cfg

    @bitwidth_config_.setter
    def bitwidth_config_(self, cfg):
        # stored by value, as the reference's C++ member: later changes to the caller's object
        # do not reach these grids; changes made through this attribute's value do
        object.__setattr__(self, "_cfg", None if cfg is None else cfg.copy())
        self._sync_config()

    def scale(self, name: str) -> float:
        return float(self._qp.g[A.GRID[name]].scale)

    def zero_point(self, name: str) -> int:
        return int(self._qp.g[A.GRID[name]].zero_point)

    def channel_scales(self, name: str) -> np.ndarray:
        return A.qparams_chan(self._qp, A.CHAN[name])

    @staticmethod
    def _attr(name):
        for pre, kind in (("scale_", "scale"), ("zp_", "zp")):
            if name.startswith(pre) and name.endswith("_"):
                stem = name[len(pre):-1]
                if stem in A.GRID:
                    return kind, "grid", stem
                if stem in A.CHAN:
                    return kind, "chan", stem
        return None

    def __getattr__(self, name):
        a = GRUQuantParams._attr(name) if not name.startswith("_") else None
        if a is None:
            raise AttributeError(name)
        kind, where, stem = a
        if where == "grid":
            g = self._qp.g[A.GRID[stem]]
            return float(g.scale) if kind == "scale" else int(g.zero_point)
        if kind == "zp":  # weights and biases are symmetric: zero points are 0 per channel
            return [0] * (3 * self.hidden_)
        return [float(v) for v in A.qparams_chan(self._qp, A.CHAN[stem])[:3 * self.hidden_]]

    def __setattr__(self, name, value):
        a = self._attr(name)
        if a is None:
            object.__setattr__(self, name, value)
            return
        kind, where, stem = a
        if where == "grid":
            g = self._qp.g[A.GRID[stem]]
            if kind == "scale":
                g.scale = float(value)
            else:
                g.zero_point = int(value)
            return
        if kind == "zp":
            if any(int(v) != 0 for v in np.atleast_1d(value)):
                raise ValueError(f"{name}: per-channel weight grids are symmetric (zero point 0)")
            return
        vals = np.asarray(value, np.float32).reshape(-1)
        if vals.size != 3 * self.hidden_:
            raise ValueError(f"{name} needs {3 * self.hidden_} values (3 * hidden_)")
        A.qparams_chan(self._qp, A.CHAN[stem])[:vals.size] = vals


def decode_effective_scale(scale: float, usePOT2: bool) -> float:
    """The scale the kernels quantise and dequantise with: the 16-bit-mantissa M·2^-shift
    encoding of ``scale`` decoded, or its power of two with usePOT2
    (decode_effective_scale_wrapper, gru_interface_binding.cc:1349)."""
    return float(_rx.load().rxmet_gru_effective_scale(float(scale), int(bool(usePOT2))))


def init_gru_cublas():
    """The reference creates its cuBLAS handle here (gru_interface_binding.cc:1357); the
    MI355X build has no library handle to create, so this only checks the library loads."""
    _rx.load()


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


# ---------------------------------------------------------------------------------------
# Hidden sizes that are not a multiple of 16.  The library's recurrences work on tiles of 16
# hidden units; any other H runs as Hp = H rounded up to 16 with inert padded units: their
# weight columns, recurrent rows and biases are zero, so they never feed a real unit, and
# their outputs (and gradients) are dropped.  Channel c = g H + j of a gate-major [.., 3H]
# axis becomes g Hp + j.
# ---------------------------------------------------------------------------------------

_UNIT_TILE = 16


def _padded_hidden(H: int) -> int:
    return (H + _UNIT_TILE - 1) // _UNIT_TILE * _UNIT_TILE


def pad_blocks(t: torch.Tensor, H: int, Hp: int, axis: int, groups: int, fill=0) -> torch.Tensor:
    """``groups`` consecutive blocks of H along ``axis``, each widened to Hp with ``fill``."""
    if t is None or t.numel() == 0:
        return t
    shape = list(t.shape)
    shape[axis] = groups * Hp
    out = torch.full(shape, fill, dtype=t.dtype, device=t.device)
    for g in range(groups):
        out.narrow(axis, g * Hp, H).copy_(t.narrow(axis, g * H, H))
    return out


def unpad_blocks(t: torch.Tensor, H: int, Hp: int, axis: int, groups: int) -> torch.Tensor:
    """Inverse of pad_blocks: the first H of each of ``groups`` blocks of Hp along ``axis``."""
    if t is None or t.numel() == 0:
        return t
    return torch.cat([t.narrow(axis, g * Hp, H) for g in range(groups)], dim=axis).contiguous()


def _padded_params(qp: "GRUQuantParams", H: int, Hp: int) -> "GRUQuantParams":
    """The same grids for Hp units: real channels keep their scales, padded ones get 1.0."""
    out = GRUQuantParams(Hp)
    src = qp.struct
    out._qp.use_pot2 = src.use_pot2
    for i in range(A.NGRIDS):
        out._qp.g[i] = src.g[i]
    for k in range(A.NCHAN):
        out._qp.chan_bits[k] = src.chan_bits[k]
        out._qp.chan_unsigned[k] = src.chan_unsigned[k]
        dst = A.qparams_chan(out._qp, k)
        dst[:] = 1.0
        s = A.qparams_chan(src, k)
        for g in range(3):
            dst[g * Hp:g * Hp + H] = s[g * H:(g + 1) * H]
    out.bitwidth_config_ = qp.bitwidth_config_
    return out


def _forward_padded(is_training, T, B, I, H, W, R, bw, br, x, h0, quant_params):
    Hp = _padded_hidden(H)
    Wp = pad_blocks(W, H, Hp, 1, 3)
    Rp = pad_blocks(pad_blocks(R, H, Hp, 1, 3), H, Hp, 0, 1)
    bwp, brp = pad_blocks(bw, H, Hp, 0, 3), pad_blocks(br, H, Hp, 0, 3)
    h0p = h0 if (h0 is None or h0.numel() == 0) else pad_blocks(h0, H, Hp, 1, 1)
    outs = forward_quant_float_storage(is_training, T, B, I, Hp, Wp, Rp, bwp, brp, x, h0p,
                                       _padded_params(quant_params, H, Hp))
    (h, v, W_q, R_q, bw_q, br_q, x_q, x_m, h0_m, W_m, R_m, bw_m, br_m, ih_m, hh_m, gi_m, go_m,
     h_m) = outs
    un = lambda t, axis, groups: unpad_blocks(t, H, Hp, axis, groups)
    return (un(h, 2, 1), un(v, 2, 4), un(W_q, 1, 3), un(un(R_q, 1, 3), 0, 1), un(bw_q, 0, 3),
            un(br_q, 0, 3), x_q, x_m, un(h0_m, 1, 1), un(W_m, 1, 3), un(un(R_m, 1, 3), 0, 1),
            un(bw_m, 0, 3), un(br_m, 0, 3), un(ih_m, 2, 3), un(hh_m, 2, 3), un(gi_m, 2, 3),
            un(go_m, 2, 3), un(h_m, 2, 1))


def _backward_padded(T, B, I, H, W_q, R_q, bw_q, br_q, x_q, dh_new, h, v, quant_params, masks):
    Hp = _padded_hidden(H)
    pb = lambda t, axis, groups: pad_blocks(t, H, Hp, axis, groups)
    x_m, h0_m, W_m, R_m, bw_m, br_m, ih_m, hh_m, gi_m, go_m, h_m = masks
    pmasks = (x_m, pb(h0_m, 1, 1), pb(W_m, 1, 3), pb(pb(R_m, 1, 3), 0, 1), pb(bw_m, 0, 3),
              pb(br_m, 0, 3), pb(ih_m, 2, 3), pb(hh_m, 2, 3), pb(gi_m, 2, 3), pb(go_m, 2, 3),
              pb(h_m, 2, 1))
    dx, dW, dR, dbw, dbr, dh0 = backward_quant_float_storage(
        T, B, I, Hp, pb(W_q, 1, 3), pb(pb(R_q, 1, 3), 0, 1), pb(bw_q, 0, 3), pb(br_q, 0, 3), x_q,
        pb(dh_new.contiguous(), 2, 1), pb(h, 2, 1), pb(v, 2, 4),
        _padded_params(quant_params, H, Hp), *pmasks)
    un = lambda t, axis, groups: unpad_blocks(t, H, Hp, axis, groups)
    return dx, un(dW, 1, 3), un(un(dR, 1, 3), 0, 1), un(dbw, 0, 3), un(dbr, 0, 3), un(dh0, 1, 1)


MASK_NAMES = ("x_mask", "h0_mask", "W_mask", "R_mask", "bw_mask", "br_mask",
              "weight_ih_linear_mask", "weight_hh_linear_mask", "gate_input_mask",
              "gate_output_mask", "h_mask")


def _forward_dir(is_training, T, B, I, H, W, R, bw, br, x, h0, quant_params, codes=False):
    """Check one direction's inputs and allocate its outputs; returns (outputs, FwdDir,
    workspace), and with ``codes`` (training) the SavedCodes of the direction as well: the
    outputs are then (h, v_codes, W_q, .., x_q, the six x / h0 / W / R / bias masks,
    mask_bits)."""
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
    codes = codes and is_training
    v = torch.empty((T, B, 4 * H), **f32) if is_training and not codes else torch.empty((0,), **f32)
    W_q = torch.empty((I, C), **f32)
    R_q = torch.empty((H, C), **f32)
    bw_q = torch.empty((C,), **f32)
    br_q = torch.empty((C,), **f32)
    x_q = torch.empty((T, B, I), **f32)
    if is_training:
        masks = [torch.empty((T, B, I), **u8),
                 torch.empty((B, H), **u8) if has_h0 else torch.empty((0,), **u8),
                 torch.empty((I, C), **u8), torch.empty((H, C), **u8), torch.empty((C,), **u8),
                 torch.empty((C,), **u8)]
        if codes:
            masks += [torch.empty((0,), **u8) for _ in range(5)]
        else:
            masks += [torch.empty((T, B, C), **u8) for _ in range(4)] + \
                [torch.empty((T, B, H), **u8)]
    else:
        masks = [torch.empty((0,), **u8) for _ in range(11)]
    ws = _ws(_rx.load().rxmet_gru_forward_workspace_bytes(T, B, I, H), dev)
    mp = [m.data_ptr() if m.numel() > 0 else None for m in masks]
    d = A.FwdDir(W.data_ptr(), R.data_ptr(), bw.data_ptr(), br.data_ptr(), x.data_ptr(),
                 h0.data_ptr() if has_h0 else None, ctypes.addressof(quant_params.struct),
                 h.data_ptr(), v.data_ptr() if v.numel() else None, W_q.data_ptr(),
                 R_q.data_ptr(), bw_q.data_ptr(), br_q.data_ptr(), x_q.data_ptr(), *mp,
                 ws.data_ptr())
    if codes:
        i16 = dict(dtype=torch.int16, device=dev)
        Bp = (B + 15) // 16 * 16
        vc = torch.empty((T, Bp * 4 * H), **i16)
        mb = torch.empty((T, Bp * H), **i16)
        sc = A.SavedCodes(vc.data_ptr(), mb.data_ptr())
        return (h, vc, W_q, R_q, bw_q, br_q, x_q, *masks[:6], mb), d, ws, sc
    outs = (h, v, W_q, R_q, bw_q, br_q, x_q, *masks)
    return outs, d, ws


def forward_quant_float_storage(is_training, time_steps, batch_size, input_size, hidden_size, W, R,
                                bw, br, x, h0, quant_params: GRUQuantParams):
    """forward_quant_float_storage_wrapper (gru_interface_binding.cc:306-448).

    Returns (h, v, W_q, R_q, bw_q, br_q, x_q, x_mask, h0_mask, W_mask, R_mask, bw_mask,
    br_mask, weight_ih_linear_mask, weight_hh_linear_mask, gate_input_mask,
    gate_output_mask, h_mask); masks are empty tensors when is_training is False."""
    T, B, I, H = time_steps, batch_size, input_size, hidden_size
    if H % _UNIT_TILE:
        return _forward_padded(is_training, T, B, I, H, W, R, bw, br, x, h0, quant_params)
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
    if H % _UNIT_TILE:
        raise RuntimeError("the two-direction entry points need hidden_size % 16 == 0; call "
                           "the per-direction functions, which take any hidden size")
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
    if H % _UNIT_TILE:
        raise RuntimeError("the two-direction entry points need hidden_size % 16 == 0; call "
                           "the per-direction functions, which take any hidden size")
    for k, d in enumerate(dirs):
        if d[4].dim() != 3 or d[4].stride(2) != 1:
            raise RuntimeError(f"x of direction {k} needs a unit feature stride")
    made = [_forward_dir(is_training, T, B, I, H, *d) for d in dirs]
    arr = (A.FwdDir * len(made))(*[m[1] for m in made])
    lay = (ctypes.c_int64 * (4 * len(made)))(*[int(v) for xl in x_layouts for v in xl])
    _rx.call("rxmet_gru_forward_quant_dirs_x", len(made), int(bool(is_training)), T, B, I, H, arr,
             lay, _stream(dirs[0][4].device))
    return [m[0] for m in made]


def forward_quant_codes_dirs(is_training, time_steps, batch_size, input_size, hidden_size, dirs,
                             x_layouts=None):
    """forward_quant_float_storage_dirs(_x) keeping the saved state as codes
    (rxmet_gru_forward_quant_dirs_codes), for callers that only hand it to
    backward_quant_codes_dirs.  Per direction (h, v_codes [T, Bp 4H] int16, W_q, R_q, bw_q,
    br_q, x_q, x_mask, h0_mask, W_mask, R_mask, bw_mask, br_mask, mask_bits [T, Bp H] int16),
    Bp = B rounded up to 16; v_codes holds each of z, r, n, hh_n as code minus grid minimum
    (read as unsigned 16 bits), mask_bits the 13 per-step masks of an element, both in blocks
    of 16 sequences x 16 units (rxmet_gru_saved_codes; ``unblock_codes`` restores [T, B, .]).
    Not training: as the float-storage call.
    ``x_layouts`` as in forward_quant_float_storage_dirs_x, or None for [T, B, I] inputs."""
    T, B, I, H = time_steps, batch_size, input_size, hidden_size
    if H % _UNIT_TILE:
        raise RuntimeError("the saved-codes entry points need hidden_size % 16 == 0")
    made = [_forward_dir(is_training, T, B, I, H, *d, codes=True) for d in dirs]
    arr = (A.FwdDir * len(made))(*[m[1] for m in made])
    lay = None
    if x_layouts is not None:
        lay = (ctypes.c_int64 * (4 * len(made)))(*[int(v) for xl in x_layouts for v in xl])
    codes = None
    if is_training:
        codes = (A.SavedCodes * len(made))(*[m[3] for m in made])
    _rx.call("rxmet_gru_forward_quant_dirs_codes", len(made), int(bool(is_training)), T, B, I, H,
             arr, lay, codes, _stream(dirs[0][4].device))
    return [m[0] for m in made]


def grad_views(g_out, g_hn, T, B, H, batch_first: bool, ndir: int):
    """Each direction's rxmet_gru_grad_view of the layer's output gradient ([T, B, D H], or
    [B, T, D H] batch-first; any strides, or None) and of the h_n gradient [D, B, H] (or None):
    the backward reads its dh in place instead of a dh_new buffer.  Returns (views, keep)."""
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
    views = [A.GradView(gp, st, sb, sk, k * H, k, None if hp is None else hp + 4 * k * B * H)
             for k in range(ndir)]
    return views, (g_out, g_hn)


def backward_quant_codes_dirs(time_steps, batch_size, input_size, hidden_size, dirs,
                              torch_layout=True, views=None):
    """The backward of forward_quant_codes_dirs (rxmet_gru_backward_quant_dirs_codes): ``dirs``
    is a list of (W_q, R_q, bw_q, br_q, x_q, dh_new, h, v_codes, quant_params, masks) with
    masks = (x_mask, h0_mask, W_mask, R_mask, bw_mask, br_mask, mask_bits); returns one
    (dx, dW, dR, dbw, dbr, dh) tuple per direction, the weight gradients in PyTorch's layout
    and gate order unless ``torch_layout`` is False.  With ``views`` (grad_views), each
    direction reads its dh from the output gradient and its dh_new entry may be None."""
    T, B, I, H = time_steps, batch_size, input_size, hidden_size
    made, codes = [], []
    Bp = (B + 15) // 16 * 16
    for (W_q, R_q, bw_q, br_q, x_q, dh_new, h, vc, qp, masks) in dirs:
        if vc.dtype != torch.int16 or tuple(vc.shape) != (T, Bp * 4 * H) or not vc.is_contiguous():
            raise RuntimeError("v_codes must be a contiguous int16 tensor of shape [T, Bp 4H]")
        mb = masks[6]
        if mb.dtype != torch.int16 or tuple(mb.shape) != (T, Bp * H) or not mb.is_contiguous():
            raise RuntimeError("mask_bits must be a contiguous int16 tensor of shape [T, Bp H]")
        outs, d, keep = _backward_dir(T, B, I, H, W_q, R_q, bw_q, br_q, x_q, dh_new, h, None,
                                      qp, tuple(masks[:6]) + (None,) * 5,
                                      torch_layout=torch_layout)
        made.append((outs, d, keep))
        codes.append(A.SavedCodes(vc.data_ptr(), mb.data_ptr()))
    arr = (A.BwdDir * len(made))(*[m[1] for m in made])
    carr = (A.SavedCodes * len(made))(*codes)
    varr = None
    if views is not None:
        if len(views) != len(made):
            raise RuntimeError("one grad view per direction")
        varr = (A.GradView * len(made))(*views)
    _rx.call("rxmet_gru_backward_quant_dirs_codes", len(made), T, B, I, H, arr,
             1 if torch_layout else 0, carr, varr, _stream(dirs[0][4].device))
    return [m[0] for m in made]


def unblock_codes(codes, B, H, fields):
    """[T, B, fields H] view order of blocked saved codes (forward_quant_codes_dirs): ``codes``
    [T, Bp fields H] with blocks of [16 rows][fields][16 units] (fields 4 for v_codes, 1 for
    mask_bits).  Works on torch tensors and numpy arrays."""
    T = codes.shape[0]
    nt = (B + 15) // 16
    blk = codes.reshape(T, nt, H // 16, 16, fields, 16)
    perm = (0, 1, 3, 4, 2, 5)
    blk = blk.permute(*perm) if isinstance(blk, torch.Tensor) else blk.transpose(perm)
    return blk.reshape(T, nt * 16, fields * H)[:, :B]


def bidir_assemble(h_f, h_r, batch_first: bool):
    """(output, h_n) of a bidirectional layer from both directions' h [T+1, B, H]
    (rxmet_gru_bidir_assemble): output [T, B, 2H], or [B, T, 2H] when batch_first.  The
    assembly copies 4-byte elements, so float32 states and int32 codes alike."""
    T1, B, H = h_f.shape
    T = T1 - 1
    shape = (B, T, 2 * H) if batch_first else (T, B, 2 * H)
    out = torch.empty(shape, dtype=h_f.dtype, device=h_f.device)
    h_n = torch.empty((2, B, H), dtype=h_f.dtype, device=h_f.device)
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
        if t is None and n in ("v", "dh_new"):  # saved codes / a grad view instead
            continue
        _check_f32_cuda(n, t)
        if tuple(t.shape) != shp:
            raise RuntimeError(f"{n} must have shape {list(shp)}")
    f32 = dict(dtype=torch.float32, device=dev)
    outs = (torch.empty((T, B, I), **f32),
            torch.empty((C, I) if torch_layout else (I, C), **f32),
            torch.empty((C, H) if torch_layout else (H, C), **f32),
            torch.empty((C,), **f32), torch.empty((C,), **f32), torch.empty((B, H), **f32))
    mp = [m.data_ptr() if (m is not None and m.numel() > 0) else None for m in masks]
    dh_new = dh_new.contiguous() if dh_new is not None else None
    ws = _ws(_rx.load().rxmet_gru_backward_workspace_bytes(T, B, I, H), dev)
    d = A.BwdDir(W_q.data_ptr(), R_q.data_ptr(), bw_q.data_ptr(), br_q.data_ptr(), x_q.data_ptr(),
                 dh_new.data_ptr() if dh_new is not None else None, h.data_ptr(),
                 v.data_ptr() if v is not None else None,
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
    if H % _UNIT_TILE:
        return _backward_padded(T, B, I, H, W_q, R_q, bw_q, br_q, x_q, dh_new, h, v, quant_params,
                                masks)
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
    if H % _UNIT_TILE:
        raise RuntimeError("the two-direction entry points need hidden_size % 16 == 0; call "
                           "the per-direction functions, which take any hidden size")
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
    if H % _UNIT_TILE:
        raise RuntimeError("the two-direction entry points need hidden_size % 16 == 0; call "
                           "the per-direction functions, which take any hidden size")
    made = [_backward_dir(T, B, I, H, *d, torch_layout=True) for d in dirs]
    arr = (A.BwdDir * len(made))(*[m[1] for m in made])
    _rx.call("rxmet_gru_backward_quant_dirs_x", len(made), T, B, I, H, arr, 1,
             _stream(dirs[0][4].device))
    return [m[0] for m in made]


# ---------------------------------------------------------------------------------------
# int32 carrier
# ---------------------------------------------------------------------------------------

def _check_i32_cuda(name, t):
    if not (t.is_cuda and t.dtype == torch.int32):
        raise RuntimeError(f"{name} must be CUDA int32 tensor")


def forward_quant_int_storage(is_training, time_steps, batch_size, input_size, hidden_size, W, R,
                              bw, br, x, h0, quant_params: GRUQuantParams):
    """forward_quant_int_storage_wrapper (gru_interface_binding.cc:451-586): the int32 carrier
    (quantGRUForwardInt), rxmet_gru_forward_quant_int.

    Returns the 18 tensors of forward_quant_float_storage with W_q, R_q, bw_q, br_q and x_q as
    int32 codes; h and v are dequantised float32; masks are empty when is_training is False."""
    T, B, I, H = time_steps, batch_size, input_size, hidden_size
    for n, t in (("W", W), ("R", R), ("bw", bw), ("br", br), ("x", x)):
        _check_f32_cuda(n, t)
    has_h0 = h0 is not None and h0.numel() > 0
    if has_h0:
        _check_f32_cuda("h0", h0)
        if tuple(h0.shape) != (B, H):
            raise RuntimeError("h0 must have shape [batch_size, hidden_size]")
    if tuple(x.shape) != (T, B, I) or tuple(W.shape) != (I, 3 * H) or tuple(R.shape) != (H, 3 * H):
        raise RuntimeError("x/W/R shapes do not match (time_steps, batch_size, input_size, "
                           "hidden_size)")
    dev = x.device
    C = 3 * H
    f32 = dict(dtype=torch.float32, device=dev)
    i32 = dict(dtype=torch.int32, device=dev)
    u8 = dict(dtype=torch.uint8, device=dev)
    h = torch.empty((T + 1, B, H), **f32)
    v = torch.empty((T, B, 4 * H), **f32)
    W_q, R_q = torch.empty((I, C), **i32), torch.empty((H, C), **i32)
    bw_q, br_q = torch.empty((C,), **i32), torch.empty((C,), **i32)
    x_q = torch.empty((T, B, I), **i32)
    if is_training:
        masks = [torch.empty((T, B, I), **u8),
                 torch.empty((B, H), **u8) if has_h0 else torch.empty((0,), **u8),
                 torch.empty((I, C), **u8), torch.empty((H, C), **u8), torch.empty((C,), **u8),
                 torch.empty((C,), **u8)] + [torch.empty((T, B, C), **u8) for _ in range(4)] + \
                [torch.empty((T, B, H), **u8)]
    else:
        masks = [torch.empty((0,), **u8) for _ in range(11)]
    ws = _ws(_rx.load().rxmet_gru_forward_int_workspace_bytes(T, B, I, H), dev)
    mp = [m.data_ptr() if m.numel() > 0 else None for m in masks]
    _rx.call("rxmet_gru_forward_quant_int", int(bool(is_training)), T, B, I, H, W.data_ptr(),
             R.data_ptr(), bw.data_ptr(), br.data_ptr(), x.data_ptr(),
             h0.data_ptr() if has_h0 else None, ctypes.byref(quant_params.struct), h.data_ptr(),
             v.data_ptr(), W_q.data_ptr(), R_q.data_ptr(), bw_q.data_ptr(), br_q.data_ptr(),
             x_q.data_ptr(), *mp, ws.data_ptr(), _stream(dev))
    return (h, v, W_q, R_q, bw_q, br_q, x_q, *masks)


def _int_dir_struct(**fields):
    d = A.IntDir()
    for k, v in fields.items():
        setattr(d, k, v)
    return d


def forward_int_bidir(T, B, I, H, dirs, int_io=False):
    """Both directions of a bidirectional layer on the int32 carrier in one call
    (rxmet_gru_forward_quant_int_dirs; no counterpart in the reference, which calls the
    per-direction wrappers): one clustered recurrence launch covers both directions.  dirs: two
    tuples (W, R, bw, br, x, h0, quant_params), each direction's x in its own time order (x
    int32 codes when int_io).  Inference only: returns, per direction, h [T+1,B,H] float32
    (int_io: h_q [T+1,B,H] int32 codes)."""
    dev = dirs[0][4].device
    C = 3 * H
    i32 = dict(dtype=torch.int32, device=dev)
    f32 = dict(dtype=torch.float32, device=dev)
    structs, keep, outs = [], [], []
    for W, R, bw, br, x, h0, qp in dirs:
        for n, t in (("W", W), ("R", R), ("bw", bw), ("br", br)):
            _check_f32_cuda(n, t)
        (_check_i32_cuda if int_io else _check_f32_cuda)("x", x)
        if tuple(x.shape) != (T, B, I):
            raise RuntimeError("x must have shape [time_steps, batch_size, input_size]")
        has_h0 = h0 is not None and h0.numel() > 0
        if has_h0:
            (_check_i32_cuda if int_io else _check_f32_cuda)("h0", h0)
            if tuple(h0.shape) != (B, H):
                raise RuntimeError("h0 must have shape [batch_size, hidden_size]")
        codes = [torch.empty(s_, **i32) for s_ in ((I, C), (H, C), (C,), (C,))]
        ws = _ws(_rx.load().rxmet_gru_forward_int_workspace_bytes(T, B, I, H), dev)
        x = x.contiguous()
        h0c = h0.contiguous() if has_h0 else None
        f = dict(W=W.data_ptr(), R=R.data_ptr(), bw=bw.data_ptr(), br=br.data_ptr(),
                 params=ctypes.addressof(qp.struct),
                 W_q=codes[0].data_ptr(), R_q=codes[1].data_ptr(), bw_q=codes[2].data_ptr(),
                 br_q=codes[3].data_ptr(), workspace=ws.data_ptr())
        if int_io:
            h = torch.empty((T + 1, B, H), **i32)
            f.update(x_q_in=x.data_ptr(), h0_q_in=h0c.data_ptr() if has_h0 else None,
                     h_q=h.data_ptr())
            keep += [x, h0c, ws, codes]
        else:
            h = torch.empty((T + 1, B, H), **f32)
            x_q = torch.empty((T, B, I), **i32)
            f.update(x=x.data_ptr(), h0=h0c.data_ptr() if has_h0 else None, h=h.data_ptr(),
                     x_q=x_q.data_ptr())
            keep += [x, h0c, ws, codes, x_q]
        structs.append(_int_dir_struct(**f))
        outs.append(h)
    arr = (A.IntDir * 2)(*structs)
    _rx.call("rxmet_gru_forward_quant_int_dirs", 2, 0, T, B, I, H, arr, _stream(dev))
    return outs


def backward_quant_int_storage(time_steps, batch_size, input_size, hidden_size, W_q, R_q, bw_q,
                               br_q, x_q, dh_new, h, v, quant_params: GRUQuantParams, x_mask,
                               h0_mask, W_mask, R_mask, bw_mask, br_mask, weight_ih_linear_mask,
                               weight_hh_linear_mask, gate_input_mask, gate_output_mask, h_mask):
    """backward_quant_int_storage_wrapper (gru_interface_binding.cc:923-963): the int32 codes the
    forward saved, converted to float32 codes, through backward_quant_float_storage."""
    for n, t in (("W_q", W_q), ("R_q", R_q), ("bw_q", bw_q), ("br_q", br_q), ("x_q", x_q)):
        _check_i32_cuda(n, t)
    return backward_quant_float_storage(
        time_steps, batch_size, input_size, hidden_size, W_q.float(), R_q.float(), bw_q.float(),
        br_q.float(), x_q.float(), dh_new, h, v, quant_params, x_mask, h0_mask, W_mask, R_mask,
        bw_mask, br_mask, weight_ih_linear_mask, weight_hh_linear_mask, gate_input_mask,
        gate_output_mask, h_mask)


def forward_quantized_int_io(time_steps, batch_size, input_size, hidden_size, W, R, bw, br, x_q,
                             h0_q, quant_params: GRUQuantParams):
    """forward_quantized_int_io_wrapper (gru_interface_binding.cc:588-646): int32 codes in and
    out (quantGRUForwardIntIO), rxmet_gru_forward_int_io.  x_q [T,B,I] and h0_q [B,H] (may be
    empty) lie on the x and h grids.  Returns (output_q [T,B,H], h_n_q [1,B,H]) int32."""
    T, B, I, H = time_steps, batch_size, input_size, hidden_size
    for n, t in (("W", W), ("R", R), ("bw", bw), ("br", br)):
        _check_f32_cuda(n, t)
    _check_i32_cuda("x_q", x_q)
    if tuple(x_q.shape) != (T, B, I):
        raise RuntimeError("x_q must have shape [time_steps, batch_size, input_size]")
    has_h0 = h0_q is not None and h0_q.numel() > 0
    if has_h0:
        _check_i32_cuda("h0_q", h0_q)
        if tuple(h0_q.shape) != (B, H):
            raise RuntimeError("h0_q must have shape [batch_size, hidden_size]")
    dev = x_q.device
    C = 3 * H
    i32 = dict(dtype=torch.int32, device=dev)
    h_q = torch.empty((T + 1, B, H), **i32)
    codes = [torch.empty(s, **i32) for s in ((I, C), (H, C), (C,), (C,))]
    ws = _ws(_rx.load().rxmet_gru_forward_int_workspace_bytes(T, B, I, H), dev)
    x_q = x_q.contiguous()
    h0c = h0_q.contiguous() if has_h0 else None
    _rx.call("rxmet_gru_forward_int_io", T, B, I, H, W.data_ptr(), R.data_ptr(), bw.data_ptr(),
             br.data_ptr(), x_q.data_ptr(), h0c.data_ptr() if has_h0 else None,
             ctypes.byref(quant_params.struct), h_q.data_ptr(), *[c.data_ptr() for c in codes],
             ws.data_ptr(), _stream(dev))
    return h_q[1:].contiguous(), h_q[T:T + 1].contiguous()
