"""MI355X replacement of the reference's QuantLSTM native module ``_quant_lstm``
(``operators/quant-lstm/pytorch/lib/lstm_interface_binding.cc:917-975``) on the QAT path:
MinMax calibration, parameter finalisation, the quantised forward with its saved state and
the STE backward.  Every call goes to librxmet.so (``include/rxmet_lstm.h``) on PyTorch's
current stream; tensors are time-major ``[T, B, *]`` with PyTorch weight layouts and gate
order (i, f, g, o).
"""
from __future__ import annotations

import ctypes
from typing import Optional

import numpy as np
import torch

import rxmet_lstm_abi as L
import rxmet_lib as _rx

_F32 = torch.float32


def _dev_f32(name: str, t: torch.Tensor) -> torch.Tensor:
    if not (t.is_cuda and t.dtype == _F32):
        raise RuntimeError(f"{name} must be a CUDA float32 tensor")
    return t.contiguous()


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


def _stream(dev) -> int:
    return _rx.stream_of(dev)


def _ws(nbytes: int, dev) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=dev)


class LstmQuantParams:
    """Finalised standard scales / zero points of one direction (LstmQuantParams,
    include/lstm/quant_params.h), wrapping the C struct with owned channel arrays."""

    def __init__(self, hidden: int):
        self.hidden = int(hidden)
        self._p = L.new_params(self.hidden)

    @property
    def struct(self) -> L.Params:
        return self._p

    @property
    def bias_enabled(self) -> bool:
        return bool(self._p.bias_enabled)

    def scale(self, name: str) -> float:
        return float(self._p.scale[L.OP[name]])

    def zero_point(self, name: str) -> int:
        return int(self._p.zero_point[L.OP[name]])

    def channel_scales(self, name: str) -> np.ndarray:
        return L.chan_scales(self._p, L.PARAM_OPS.index(name)).copy()

    def to_dict(self) -> dict:
        d = {"hidden": self.hidden, "bias_enabled": self.bias_enabled,
             "scale_mode": int(self._p.config.scale_mode), "operators": {}}
        for i, n in enumerate(L.OP_NAMES):
            t = self._p.config.op[i]
            e = {"bits": int(t.bits), "is_unsigned": bool(t.is_unsigned),
                 "is_symmetric": bool(t.is_symmetric), "granularity": int(t.granularity)}
            if n in L.PARAM_OPS:
                e["scale"] = [float(v) for v in self.channel_scales(n)]
                e["zero_point"] = 0
            else:
                e["scale"] = self.scale(n)
                e["zero_point"] = self.zero_point(n)
            d["operators"][n] = e
        return d

    @classmethod
    def from_dict(cls, d: dict) -> "LstmQuantParams":
        p = cls(int(d["hidden"]))
        s = p._p
        s.bias_enabled = int(bool(d["bias_enabled"]))
        s.config.scale_mode = int(d["scale_mode"])
        for i, n in enumerate(L.OP_NAMES):
            e = d["operators"][n]
            s.config.op[i] = L.OpConfig(int(e["bits"]), int(e["is_unsigned"]),
                                        int(e["is_symmetric"]), int(e["granularity"]))
            if n in L.PARAM_OPS:
                L.chan_scales(s, L.PARAM_OPS.index(n))[:] = np.asarray(e["scale"], np.float32)
            else:
                s.scale[i] = float(e["scale"])
                s.zero_point[i] = int(e["zero_point"])
        return p


_EMPTY_STATS = {}


def new_stats(hidden: int, device) -> torch.Tensor:
    """Empty MinMax statistics (layout of rxmet_lstm_stats_size) on ``device``; on a GPU a copy
    of a cached device template, so that a new calibration does not wait for the stream on a
    pageable host copy."""
    if torch.device(device).type == "cpu":
        return torch.from_numpy(L.empty_stats(hidden))
    key = (hidden, str(device))
    t = _EMPTY_STATS.get(key)
    if t is None:
        t = _EMPTY_STATS[key] = torch.from_numpy(L.empty_stats(hidden)).to(device)
    return t.clone()


def forward_calibrate(x, W_ih, W_hh, b_ih, b_hh, h0, c0, stats: torch.Tensor):
    """Float forward + MinMax statistics merged into ``stats`` (CalibrationSession.collect).
    Returns (output [T,B,H], h_n [B,H], c_n [B,H])."""
    T, B, I = x.shape
    H = W_hh.shape[1]
    x, W_ih, W_hh = (_dev_f32(n, t) for n, t in (("x", x), ("weight_ih", W_ih), ("weight_hh", W_hh)))
    b_ih = _dev_f32("bias_ih", b_ih) if b_ih is not None else None
    b_hh = _dev_f32("bias_hh", b_hh) if b_hh is not None else None
    h0 = _dev_f32("h0", h0) if h0 is not None else None
    c0 = _dev_f32("c0", c0) if c0 is not None else None
    dev = x.device
    out = torch.empty((T, B, H), dtype=_F32, device=dev)
    hn = torch.empty((B, H), dtype=_F32, device=dev)
    cn = torch.empty((B, H), dtype=_F32, device=dev)
    ws = _ws(_rx.load().rxmet_lstm_calibrate_workspace_bytes(T, B, I, H), dev)
    _rx.call("rxmet_lstm_forward_calibrate", T, B, I, H, _ptr(W_ih), _ptr(W_hh), _ptr(b_ih),
             _ptr(b_hh), _ptr(x), _ptr(h0), _ptr(c0), _ptr(out), _ptr(hn), _ptr(cn),
             _ptr(stats), _ptr(ws), _stream(dev))
    return out, hn, cn


def finalize_params(stats: torch.Tensor, config: L.Config, hidden: int,
                    bias: bool) -> LstmQuantParams:
    """MinMax finalisation (LstmCalibrationSession::finalize, src/lstm/calibration.cc:374-427)."""
    host = stats.detach().cpu().numpy().astype(np.float32)
    p = LstmQuantParams(hidden)
    _rx.call("rxmet_lstm_finalize_params", host.ctypes.data_as(ctypes.c_void_p),
             ctypes.byref(config), hidden, int(bool(bias)), ctypes.byref(p.struct))
    return p


def check_params(params: LstmQuantParams, input_size: int) -> None:
    """Validate ``params`` by deriving its integer execution encodings on the host
    (rxmet_lstm_derive_exec); raises RxmetError for an inconsistent set."""
    C = 4 * params.hidden
    acc = (L.Rescale * (2 * C))()
    bias = (L.Rescale * (2 * C))()
    gate = (L.Rescale * 8)()
    cell = (L.Q31 * 2)()
    hid = (L.Rescale * 1)()
    _rx.call("rxmet_lstm_derive_exec", ctypes.byref(params.struct), int(input_size),
             ctypes.addressof(acc), ctypes.addressof(bias), ctypes.addressof(gate),
             ctypes.addressof(cell), ctypes.addressof(hid))


def forward_float(x, W_ih, W_hh, b_ih, b_hh, h0, c0):
    """Float forward (lstm_forward).  Returns (output, h_n, c_n)."""
    T, B, I = x.shape
    H = W_hh.shape[1]
    x, W_ih, W_hh = (_dev_f32(n, t) for n, t in (("x", x), ("weight_ih", W_ih), ("weight_hh", W_hh)))
    b_ih = _dev_f32("bias_ih", b_ih) if b_ih is not None else None
    b_hh = _dev_f32("bias_hh", b_hh) if b_hh is not None else None
    h0 = _dev_f32("h0", h0) if h0 is not None else None
    c0 = _dev_f32("c0", c0) if c0 is not None else None
    dev = x.device
    out = torch.empty((T, B, H), dtype=_F32, device=dev)
    hn = torch.empty((B, H), dtype=_F32, device=dev)
    cn = torch.empty((B, H), dtype=_F32, device=dev)
    _rx.call("rxmet_lstm_forward_float", T, B, I, H, _ptr(W_ih), _ptr(W_hh), _ptr(b_ih),
             _ptr(b_hh), _ptr(x), _ptr(h0), _ptr(c0), _ptr(out), _ptr(hn), _ptr(cn), _stream(dev))
    return out, hn, cn


# the saved-codes form's entries (rxmet_lstm_saved_codes) and the reference-format entries they
# replace
CODE_KEYS = ("codes_blocks", "cell_codes")
CODED_FIELDS = ("gate_out", "cell", "cell_tanh", "hh_linear_m", "gate_in_m", "gate_out_m",
                "cell_m", "cell_tanh_m", "hidden_m")


def _saved_tensors(T, B, I, H, bias, dev, codes=False) -> dict:
    C = 4 * H
    f = dict(dtype=_F32, device=dev)
    u = dict(dtype=torch.uint8, device=dev)
    s = {"x_q": torch.empty((T, B, I), **f), "w_ih_q": torch.empty((C, I), **f),
         "w_hh_q": torch.empty((C, H), **f), "h0_q": torch.empty((B, H), **f),
         "c0_q": torch.empty((B, H), **f), "x_m": torch.empty((T, B, I), **u),
         "w_ih_m": torch.empty((C, I), **u), "w_hh_m": torch.empty((C, H), **u),
         "h0_m": torch.empty((B, H), **u), "c0_m": torch.empty((B, H), **u),
         "hidden": torch.empty((T, B, H), **f), "ih_linear_m": torch.empty((T, B, C), **u)}
    if codes:
        nb = (B + 15) // 16 * (H // 16)
        s["codes_blocks"] = torch.empty((T * nb * L.CODES_BLOCK,), **u)
        s["cell_codes"] = torch.empty(((T + 1) * nb * L.CELL_BLOCK,), dtype=torch.int16, device=dev)
    else:
        s.update({"gate_out": torch.empty((T, B, C), **f), "cell": torch.empty((T, B, H), **f),
                  "cell_tanh": torch.empty((T, B, H), **f)})
        for k in ("hh_linear_m", "gate_in_m", "gate_out_m"):
            s[k] = torch.empty((T, B, C), **u)
        for k in ("cell_m", "cell_tanh_m", "hidden_m"):
            s[k] = torch.empty((T, B, H), **u)
    if bias:
        s["b_ih_q"] = torch.empty((C,), **f)
        s["b_hh_q"] = torch.empty((C,), **f)
        s["b_ih_m"] = torch.empty((C,), **u)
        s["b_hh_m"] = torch.empty((C,), **u)
    return s


def _saved_struct(saved: dict) -> L.Saved:
    s = L.Saved()
    for k in L.SAVED_FIELDS:
        t = saved.get(k)
        setattr(s, k, None if t is None else t.data_ptr())
    return s


def _codes_struct(saved: dict):
    if "codes_blocks" not in saved:
        return None
    return L.SavedCodes(saved["codes_blocks"].data_ptr(), saved["cell_codes"].data_ptr())


def codes_fit(params: LstmQuantParams) -> bool:
    """The saved codes hold the gate-output, cell and tanh grids (at most 16 bits)."""
    op = params.struct.config.op
    return all(int(op[L.OP[n]].bits) <= 16 for n in _GATE_OUTPUTS + ("cell_state", "cell_tanh_output"))


_GATE_OUTPUTS = ("input_gate_output", "forget_gate_output", "cell_gate_output",
                 "output_gate_output")


def _grid_lo(params: LstmQuantParams, name: str) -> int:
    t = params.struct.config.op[L.OP[name]]
    return 0 if t.is_unsigned else -(1 << (int(t.bits) - 1))


def decode_saved_codes(saved: dict, params: LstmQuantParams, B: int) -> dict:
    """The reference-format entries (gate_out, cell, cell_tanh as fp32 codes; the six masks as
    uint8, 1 = clamped) of a saved-codes forward, from its blocks (rxmet_lstm_saved_codes)."""
    T, H = saved["hidden"].shape[0], saved["hidden"].shape[2]
    nt, nu = (B + 15) // 16, H // 16
    blk = saved["codes_blocks"].view(T, nt, nu, L.CODES_BLOCK)
    u16 = lambda t: t.contiguous().view(torch.int16).to(torch.int32) & 0xFFFF

    def unblock(x, fields):  # [T, nt, nu, 16 r, fields, 16 e] -> [T, B, fields H]
        y = x.reshape(T, nt, nu, 16, fields, 16).permute(0, 1, 3, 4, 2, 5)
        return y.reshape(T, nt * 16, fields * H)[:, :B]

    gates = u16(blk[..., :2048]).view(T, nt, nu, 16, 4, 16)
    lo_g = torch.tensor([_grid_lo(params, n) for n in _GATE_OUTPUTS], dtype=torch.int32,
                        device=gates.device).view(1, 1, 1, 1, 4, 1)
    out = {"gate_out": unblock(gates + lo_g, 4).to(_F32)}
    gm = blk[..., 2048:3072].reshape(T, nt, nu, 4, 16, 16).permute(0, 1, 2, 4, 3, 5)
    for bit, k in enumerate(("hh_linear_m", "gate_in_m", "gate_out_m")):
        out[k] = unblock((gm >> bit) & 1, 4).contiguous()
    tanh = u16(blk[..., 3072:3584]).view(T, nt, nu, 16, 1, 16) + _grid_lo(params, "cell_tanh_output")
    out["cell_tanh"] = unblock(tanh, 1).to(_F32)
    cm = blk[..., 3584:].reshape(T, nt, nu, 16, 1, 16)
    for bit, k in enumerate(("cell_m", "cell_tanh_m", "hidden_m")):
        out[k] = unblock((cm >> bit) & 1, 1).contiguous()
    cells = u16(saved["cell_codes"].view(T + 1, nt, nu, L.CELL_BLOCK)).view(T + 1, nt, nu, 16, 1, 16)
    cells = cells + _grid_lo(params, "cell_state")
    y = cells.permute(0, 1, 3, 4, 2, 5).reshape(T + 1, nt * 16, H)[:, :B]
    out["cell"] = y[1:].to(_F32).contiguous()
    return out


# ---------------------------------------------------------------------------------------
# Hidden sizes that are not a multiple of 16.  The recurrences work on tiles of 16 hidden
# units; any other H runs as Hp = H rounded up to 16 with inert padded units: their rows of
# W_ih / W_hh, their columns of W_hh and their biases are zero, so they never feed a real
# unit, and their outputs and gradients are dropped.  Channel c = g H + j of a gate-major
# [4H] axis becomes g Hp + j.
# ---------------------------------------------------------------------------------------

_UNIT_TILE = 16


def _padded_hidden(H: int) -> int:
    return (H + _UNIT_TILE - 1) // _UNIT_TILE * _UNIT_TILE


def _pad(t, H, Hp, axis, groups, fill=0):
    if t is None or t.numel() == 0:
        return t
    shape = list(t.shape)
    shape[axis] = groups * Hp
    out = torch.full(shape, fill, dtype=t.dtype, device=t.device)
    for g in range(groups):
        out.narrow(axis, g * Hp, H).copy_(t.narrow(axis, g * H, H))
    return out


def _unpad(t, H, Hp, axis, groups):
    if t is None or t.numel() == 0:
        return t
    return torch.cat([t.narrow(axis, g * Hp, H) for g in range(groups)], dim=axis).contiguous()


# (axis, gate groups) of each saved tensor's hidden axes, in the order they are padded
_SAVED_HIDDEN_AXES = {
    "w_ih_q": ((0, 4),), "w_hh_q": ((0, 4), (1, 1)), "b_ih_q": ((0, 4),), "b_hh_q": ((0, 4),),
    "h0_q": ((1, 1),), "c0_q": ((1, 1),), "w_ih_m": ((0, 4),), "w_hh_m": ((0, 4), (1, 1)),
    "b_ih_m": ((0, 4),), "b_hh_m": ((0, 4),), "h0_m": ((1, 1),), "c0_m": ((1, 1),),
    "gate_out": ((2, 4),), "cell": ((2, 1),), "cell_tanh": ((2, 1),), "hidden": ((2, 1),),
    "ih_linear_m": ((2, 4),), "hh_linear_m": ((2, 4),), "gate_in_m": ((2, 4),),
    "gate_out_m": ((2, 4),), "cell_m": ((2, 1),), "cell_tanh_m": ((2, 1),), "hidden_m": ((2, 1),)}


def _padded_params(params: LstmQuantParams, H: int, Hp: int) -> LstmQuantParams:
    """The same grids for Hp units: real channels keep their scales, padded ones get 1.0."""
    out = LstmQuantParams(Hp)
    src, dst = params.struct, out.struct
    dst.bias_enabled = src.bias_enabled
    dst.config = src.config
    for i in range(L.NOPS):
        dst.scale[i] = src.scale[i]
        dst.zero_point[i] = src.zero_point[i]
    for k in range(4):
        d = L.chan_scales(dst, k)
        d[:] = 1.0
        sk = L.chan_scales(src, k)
        for g in range(4):
            d[g * Hp:g * Hp + H] = sk[g * H:(g + 1) * H]
    return out


def _forward_padded(x, W_ih, W_hh, b_ih, b_hh, h0, c0, params, save_checkpoints):
    H = W_hh.shape[1]
    Hp = _padded_hidden(H)
    pw = _pad(_pad(W_hh, H, Hp, 0, 4), H, Hp, 1, 1)
    out, hn, cn, saved = forward_quant(
        x, _pad(W_ih, H, Hp, 0, 4), pw, _pad(b_ih, H, Hp, 0, 4), _pad(b_hh, H, Hp, 0, 4),
        _pad(h0, H, Hp, 1, 1), _pad(c0, H, Hp, 1, 1), _padded_params(params, H, Hp),
        save_checkpoints)
    if saved is not None:
        for k, axes in _SAVED_HIDDEN_AXES.items():
            if k in saved:
                for axis, groups in axes:
                    saved[k] = _unpad(saved[k], H, Hp, axis, groups)
    return (_unpad(out, H, Hp, 2, 1), _unpad(hn, H, Hp, 1, 1), _unpad(cn, H, Hp, 1, 1), saved)


def _backward_padded(saved, params, grad_output, grad_h_n, grad_c_n):
    H = saved["h0_q"].shape[1]
    Hp = _padded_hidden(H)
    padded = dict(saved)
    for k, axes in _SAVED_HIDDEN_AXES.items():
        if k in padded:
            # padded masks read "clamped" (1), so no gradient passes through a padded unit
            fill = 1 if padded[k].dtype == torch.uint8 else 0
            for axis, groups in axes:
                padded[k] = _pad(padded[k], H, Hp, axis, groups, fill)
    dx, dwi, dwh, dbi, dbh, dh0, dc0 = backward_quant(
        padded, _padded_params(params, H, Hp), _pad(grad_output.contiguous(), H, Hp, 2, 1),
        _pad(grad_h_n, H, Hp, 1, 1), _pad(grad_c_n, H, Hp, 1, 1))
    un = lambda t, axis, groups: _unpad(t, H, Hp, axis, groups)
    return (dx, un(dwi, 0, 4), un(un(dwh, 0, 4), 1, 1), un(dbi, 0, 4), un(dbh, 0, 4),
            un(dh0, 1, 1), un(dc0, 1, 1))


def forward_quant(x, W_ih, W_hh, b_ih, b_hh, h0, c0, params: LstmQuantParams,
                  save_checkpoints: bool, codes: bool = False):
    """Quantised FP32-carrier forward (lstm_forward_quantized).  Returns (output, h_n, c_n,
    saved) where ``saved`` holds the masters, checkpoints and clamp masks (1 = clamped) when
    ``save_checkpoints`` is set, else None.  With ``codes`` the checkpoints other than hidden
    and the recurrence masks are kept as the blocked codes of rxmet_lstm_forward_quant_codes
    (``codes_blocks``, ``cell_codes``; decode_saved_codes restores them), for backward_quant
    only."""
    T, B, I = x.shape
    H = W_hh.shape[1]
    if H % _UNIT_TILE:
        return _forward_padded(x, W_ih, W_hh, b_ih, b_hh, h0, c0, params, save_checkpoints)
    x, W_ih, W_hh = (_dev_f32(n, t) for n, t in (("x", x), ("weight_ih", W_ih), ("weight_hh", W_hh)))
    bias = params.bias_enabled
    if bias and (b_ih is None or b_hh is None):
        raise RuntimeError("quant params enable bias but the module has no bias")
    b_ih = _dev_f32("bias_ih", b_ih) if bias else None
    b_hh = _dev_f32("bias_hh", b_hh) if bias else None
    h0 = _dev_f32("h0", h0) if h0 is not None else None
    c0 = _dev_f32("c0", c0) if c0 is not None else None
    dev = x.device
    out = torch.empty((T, B, H), dtype=_F32, device=dev)
    hn = torch.empty((B, H), dtype=_F32, device=dev)
    cn = torch.empty((B, H), dtype=_F32, device=dev)
    codes = bool(codes and save_checkpoints)
    saved = _saved_tensors(T, B, I, H, bias, dev, codes) if save_checkpoints else None
    sv = _saved_struct(saved) if saved is not None else None
    ws = _ws(_rx.load().rxmet_lstm_forward_workspace_bytes(T, B, I, H), dev)
    head = (T, B, I, H, _ptr(W_ih), _ptr(W_hh), _ptr(b_ih), _ptr(b_hh), _ptr(x), _ptr(h0),
            _ptr(c0), ctypes.byref(params.struct), _ptr(out), _ptr(hn), _ptr(cn),
            ctypes.byref(sv) if sv is not None else None)
    if codes:
        cs = _codes_struct(saved)
        _rx.call("rxmet_lstm_forward_quant_codes", *head, ctypes.byref(cs), _ptr(ws), _stream(dev))
    else:
        _rx.call("rxmet_lstm_forward_quant", *head, _ptr(ws), _stream(dev))
    return out, hn, cn, saved


def backward_quant(saved: dict, params: LstmQuantParams, grad_output, grad_h_n=None,
                   grad_c_n=None):
    """STE backward (lstm_backward_qat).  grad_output [T,B,H] time-major.  Returns
    (dx, dW_ih, dW_hh, db_ih, db_hh, dh0, dc0); bias grads are None without bias."""
    T, B, I = saved["x_q"].shape
    H = saved["h0_q"].shape[1]
    if H % _UNIT_TILE:
        return _backward_padded(saved, params, grad_output, grad_h_n, grad_c_n)
    C = 4 * H
    dev = saved["x_q"].device
    grad_output = _dev_f32("grad_output", grad_output)
    grad_h_n = _dev_f32("grad_h_n", grad_h_n) if grad_h_n is not None else None
    grad_c_n = _dev_f32("grad_c_n", grad_c_n) if grad_c_n is not None else None
    f = dict(dtype=_F32, device=dev)
    dx = torch.empty((T, B, I), **f)
    dwi = torch.empty((C, I), **f)
    dwh = torch.empty((C, H), **f)
    bias = params.bias_enabled
    dbi = torch.empty((C,), **f) if bias else None
    dbh = torch.empty((C,), **f) if bias else None
    dh0 = torch.empty((B, H), **f)
    dc0 = torch.empty((B, H), **f)
    sv = _saved_struct(saved)
    cs = _codes_struct(saved)
    ws = _ws(_rx.load().rxmet_lstm_backward_workspace_bytes(T, B, I, H), dev)
    tail = (_ptr(grad_output), _ptr(grad_h_n), _ptr(grad_c_n), _ptr(dx), _ptr(dwi), _ptr(dwh),
            _ptr(dbi), _ptr(dbh), _ptr(dh0), _ptr(dc0), _ptr(ws), _stream(dev))
    if cs is not None:
        _rx.call("rxmet_lstm_backward_quant_codes", T, B, I, H, ctypes.byref(params.struct),
                 ctypes.byref(sv), ctypes.byref(cs), *tail)
    else:
        _rx.call("rxmet_lstm_backward_quant", T, B, I, H, ctypes.byref(params.struct),
                 ctypes.byref(sv), *tail)
    return dx, dwi, dwh, dbi, dbh, dh0, dc0
