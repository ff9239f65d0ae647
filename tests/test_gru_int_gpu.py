"""GPU parity of the int32-carrier QuantGRU forward (rxmet_gru_forward_quant_int,
rxmet_gru_forward_int_io) against the oracle's int32 carrier, which equals the reference's
compiled CPU carrier code for code (tests/test_gru_int_oracle.py).

Bar: every code, mask and dequantised output bit-exact.  The int-IO forward on the codes of
the float-input forward returns exactly its h codes (the reference's
test_cpu_ptq_integer_carrier_and_encoding_roundtrip, operators/quant-gru/tests/
test_cpu_ptq.py:35-77, asserts the same identity).  The int32-storage backward equals the
float-storage backward on the converted codes.
"""
import numpy as np
import pytest
import torch

import gru_ops
import gru_oracle as GO
import rxmet_gru_abi as A
from test_gru_gpu import _case

pytestmark = pytest.mark.gpu
f32 = np.float32
CODES = ("W_q", "R_q", "bw_q", "br_q", "x_q")


def _t(dev, a):
    return None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _gpu_int(dev, W, R, bw, br, x, h0, qp, training):
    T, B, I = x.shape
    H = R.shape[0]
    out = gru_ops.forward_quant_int_storage(
        training, T, B, I, H, _t(dev, W), _t(dev, R), _t(dev, bw), _t(dev, br), _t(dev, x),
        _t(dev, h0) if h0 is not None else torch.empty(0, device=dev),
        gru_ops.GRUQuantParams.from_struct(qp))
    torch.cuda.synchronize()
    return out


def _dequant(codes, qp, grid):
    return GO.dequant_int(codes, qp.g[A.GRID[grid]], bool(qp.use_pot2))


def _v_dequant(v_q, qp, H):
    out = np.empty(v_q.shape, f32)
    for k, grid in enumerate(("update_gate_output", "reset_gate_output", "new_gate_output",
                              "weight_hh_linear")):
        out[..., k * H:(k + 1) * H] = _dequant(v_q[..., k * H:(k + 1) * H], qp, grid)
    return out


SHAPES = [(5, 20, 7, 32), (4, 16, 80, 256), (3, 33, 300, 64), (6, 3, 2, 1), (4, 7, 5, 33),
          (2, 70, 9, 24)]
CONFIGS = ["8b-sym", "8b-asym", "c3", "16b-act-pot2", "h-unsigned", "c5", "16b-all", "r12-pot2"]


@pytest.mark.parametrize("shape", SHAPES, ids=[str(s) for s in SHAPES])
@pytest.mark.parametrize("cfg_name", CONFIGS)
@pytest.mark.parametrize("with_h0", [False, True])
def test_int_storage_forward_bit_exact(cuda, shape, cfg_name, with_h0):
    T, B, I, H = shape
    print(f"[gru int fwd] shape={shape} cfg={cfg_name} h0={with_h0}", flush=True)
    W, R, bw, br, x, h0, qp = _case(T, B, I, H, cfg_name, 2, with_h0)
    exp = GO.forward_int(W, R, bw, br, x, qp, h0=h0, training=True)
    got = dict(zip(("h", "v") + CODES + GO.MASKS, _gpu_int(cuda, W, R, bw, br, x, h0, qp, True)))
    for k in CODES:
        assert got[k].dtype == torch.int32, k
        np.testing.assert_array_equal(got[k].cpu().numpy(), exp[k], err_msg=k)
    for k in GO.MASKS:
        if exp[k] is None:
            assert got[k].numel() == 0, k
        else:
            np.testing.assert_array_equal(got[k].cpu().numpy(), exp[k], err_msg=k)
    np.testing.assert_array_equal(got["h"].cpu().numpy(), _dequant(exp["h_q"], qp, "h"))
    np.testing.assert_array_equal(got["v"].cpu().numpy(), _v_dequant(exp["v_q"], qp, H))
    # inference: the same states, no masks
    ev = dict(zip(("h", "v") + CODES + GO.MASKS, _gpu_int(cuda, W, R, bw, br, x, h0, qp, False)))
    np.testing.assert_array_equal(ev["h"].cpu().numpy(), got["h"].cpu().numpy())
    assert all(ev[k].numel() == 0 for k in GO.MASKS)


@pytest.mark.parametrize("cfg_name", ["h-unsigned", "c3"])
def test_int_storage_clusters_walking_several_tiles(cuda, cfg_name):
    """B = 160 gives 10 batch tiles; the clustered recurrence rounds its cluster count down to
    a multiple of 8, so 8 clusters walk the 10 tiles (cluster 0 and 1 take a second tile, with
    h0 published afresh).  One h plane (8-bit unsigned h) and two (16-bit h)."""
    T, B, I, H = 4, 160, 7, 32
    print(f"[gru int fwd multi-tile] B={B} cfg={cfg_name}", flush=True)
    W, R, bw, br, x, h0, qp = _case(T, B, I, H, cfg_name, 8, True)
    exp = GO.forward_int(W, R, bw, br, x, qp, h0=h0, training=True)
    got = dict(zip(("h", "v") + CODES + GO.MASKS, _gpu_int(cuda, W, R, bw, br, x, h0, qp, True)))
    for k in CODES:
        np.testing.assert_array_equal(got[k].cpu().numpy(), exp[k], err_msg=k)
    for k in GO.MASKS:
        np.testing.assert_array_equal(got[k].cpu().numpy(), exp[k], err_msg=k)
    np.testing.assert_array_equal(got["h"].cpu().numpy(), _dequant(exp["h_q"], qp, "h"))
    np.testing.assert_array_equal(got["v"].cpu().numpy(), _v_dequant(exp["v_q"], qp, H))


@pytest.mark.parametrize("shape", [(5, 20, 7, 32), (3, 33, 300, 64), (4, 7, 5, 33)],
                         ids=str)
@pytest.mark.parametrize("cfg_name", ["8b-asym", "c3", "16b-all", "c5"])
def test_int_io_equals_int_storage(cuda, shape, cfg_name):
    """forward_quantized_int_io on the x and h0 codes of the float-input forward returns its h
    codes: output_q = h_q[1:], h_n_q = h_q[T]."""
    T, B, I, H = shape
    print(f"[gru int io] shape={shape} cfg={cfg_name}", flush=True)
    W, R, bw, br, x, h0, qp = _case(T, B, I, H, cfg_name, 3, True)
    exp = GO.forward_int(W, R, bw, br, x, qp, h0=h0, training=False)
    h0_q = exp["h_q"][0]
    io = GO.forward_int(W, R, bw, br, None, qp, training=False, x_q=exp["x_q"], h0_q=h0_q)
    np.testing.assert_array_equal(io["h_q"], exp["h_q"])
    out_q, hn_q = gru_ops.forward_quantized_int_io(
        T, B, I, H, _t(cuda, W), _t(cuda, R), _t(cuda, bw), _t(cuda, br), _t(cuda, exp["x_q"]),
        _t(cuda, h0_q), gru_ops.GRUQuantParams.from_struct(qp))
    assert out_q.dtype == torch.int32 and tuple(out_q.shape) == (T, B, H)
    assert tuple(hn_q.shape) == (1, B, H)
    np.testing.assert_array_equal(out_q.cpu().numpy(), exp["h_q"][1:])
    np.testing.assert_array_equal(hn_q.cpu().numpy()[0], exp["h_q"][T])
    # no h0_q: the state starts at the zero point of h
    exp0 = GO.forward_int(W, R, bw, br, None, qp, training=False, x_q=exp["x_q"])
    out0, _ = gru_ops.forward_quantized_int_io(
        T, B, I, H, _t(cuda, W), _t(cuda, R), _t(cuda, bw), _t(cuda, br), _t(cuda, exp["x_q"]),
        torch.empty(0, dtype=torch.int32, device=cuda), gru_ops.GRUQuantParams.from_struct(qp))
    np.testing.assert_array_equal(out0.cpu().numpy(), exp0["h_q"][1:])


def test_int_io_rejects_codes_off_the_grid(cuda):
    """Codes outside the x grid are refused with an error (checked on the device, reported on
    the host) rather than summed into a wrong result."""
    T, B, I, H = 3, 4, 5, 16
    W, R, bw, br, x, h0, qp = _case(T, B, I, H, "8b-asym", 4, False)
    exp = GO.forward_int(W, R, bw, br, x, qp, training=False)
    bad = exp["x_q"].copy()
    bad[1, 2, 3] = 1000  # an 8-bit x grid ends at 127
    args = (T, B, I, H, _t(cuda, W), _t(cuda, R), _t(cuda, bw), _t(cuda, br))
    with pytest.raises(RuntimeError, match="outside the x / h grids"):
        gru_ops.forward_quantized_int_io(*args, _t(cuda, bad), None,
                                         gru_ops.GRUQuantParams.from_struct(qp))
    # the same call with the codes back on the grid works
    out, _ = gru_ops.forward_quantized_int_io(*args, _t(cuda, exp["x_q"]), None,
                                              gru_ops.GRUQuantParams.from_struct(qp))
    np.testing.assert_array_equal(out.cpu().numpy(), exp["h_q"][1:])


@pytest.mark.parametrize("cfg_name", ["c3", "16b-all"])
def test_int_storage_backward_matches_oracle(cuda, cfg_name):
    """backward_quant_int_storage on the int forward's saved tensors: the oracle's backward on
    the same (float-converted) codes and masks, within 1e-4 relative."""
    T, B, I, H = 5, 12, 9, 32
    print(f"[gru int bwd] cfg={cfg_name}", flush=True)
    W, R, bw, br, x, h0, qp = _case(T, B, I, H, cfg_name, 5, True)
    got = _gpu_int(cuda, W, R, bw, br, x, h0, qp, True)
    h, v, W_q, R_q, bw_q, br_q, x_q = got[:7]
    masks = got[7:]
    g = np.random.default_rng(6)
    dh_new = g.standard_normal((T + 1, B, H)).astype(f32)
    dh_new[0] = 0
    P = gru_ops.GRUQuantParams.from_struct(qp)
    grads = gru_ops.backward_quant_int_storage(T, B, I, H, W_q, R_q, bw_q, br_q, x_q,
                                               _t(cuda, dh_new), h, v, P, *masks)
    torch.cuda.synchronize()
    fwd = {"h": h.cpu().numpy(), "v": v.cpu().numpy()}
    for k, tt in zip(CODES, (W_q, R_q, bw_q, br_q, x_q)):
        fwd[k] = tt.cpu().numpy().astype(f32)
    for k, m in zip(GO.MASKS, masks):
        fwd[k] = m.cpu().numpy() if m.numel() else None
    exp = GO.backward_quant(fwd, dh_new, qp)
    for name, tensor in zip(("dx", "dW", "dR", "dbw", "dbr", "dh0"), grads):
        e = exp[name]
        a = tensor.cpu().numpy()
        np.testing.assert_allclose(a, e, rtol=1e-4, atol=1e-5 * max(np.abs(e).max(), 1e-30),
                                   err_msg=name)
    with pytest.raises(RuntimeError, match="int32"):
        gru_ops.backward_quant_int_storage(T, B, I, H, W_q.float(), R_q, bw_q, br_q, x_q,
                                           _t(cuda, dh_new), h, v, P, *masks)
