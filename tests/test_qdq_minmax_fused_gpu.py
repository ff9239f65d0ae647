"""QuantizeDequantize's fused min / max path on the GPU (rxmet_qdq_forward_minmax /
rxmet_qdq_backward_minmax): the kernels derive scale and offset from the learnable min / max
themselves and the backward's fold takes the encoding gradients on to min and max.

Bar: bit for bit equal to the two-step path the module took before — the encodings from
rxmet_qdq_encoding_forward (minmax_encodings, whose values equal get_scale / _get_offset and are
pinned against the oracle in tests/test_qdq_gpu.py) followed by the backend's
quantize_dequantize, with autograd chaining the scale / offset gradients through
rxmet_qdq_encoding_backward — for y, dx, min.grad and max.grad, across tensor types, signed and
unsigned grids, per-tensor / per-channel / block encodings and the zero-point shift."""
import numpy as np
import pytest
import torch

import aimet_affine as A
import mi355x_qdq as Q

pytestmark = pytest.mark.gpu

CASES = [  # dtype, shape, module (encoding) shape, bits, symmetric, signed, block_size, shift
    (torch.float32, (96, 257), (), 8, False, True, None, 0.0),
    (torch.float32, (96, 257), (96, 1), 4, True, True, None, 0.0),
    (torch.float32, (96, 257), (), 8, False, False, None, 0.0),
    (torch.float32, (96, 257), (1, 257), 8, True, False, None, 0.0),
    (torch.float32, (96, 257), (), 8, False, True, None, 0.5),
    (torch.float16, (96, 257), (), 8, False, True, None, 0.0),
    (torch.bfloat16, (96, 256), (1, 256), 2, True, True, None, 0.0),
    (torch.float16, (96, 257), (96, 1), 16, True, True, None, 0.0),
    (torch.float32, (96, 257), (), 16, False, True, None, 0.5),
    (torch.float32, (64, 256), (4, 8), 8, False, True, (16, 32), 0.0),
    (torch.float32, (3, 40, 24), (3, 1, 24), 6, False, True, None, 0.0),
]


def _ids(c):
    return f"{str(c[0])[6:]}-{c[1]}-enc{c[2]}-{c[3]}b-{'sym' if c[4] else 'asym'}-" \
           f"{'s' if c[5] else 'u'}-blk{c[6]}-shift{c[7]}"


@pytest.mark.parametrize("case", CASES, ids=[_ids(c) for c in CASES])
def test_fused_minmax_equals_two_step_path(cuda, case):
    dtype, shape, enc, bits, sym, signed, block, shift = case
    print(f"[qdq minmax fused] {_ids(case)}", flush=True)
    gen = torch.Generator().manual_seed(bits * 7 + len(shape))
    x = (torch.randn(shape, generator=gen) * 2.0).to(dtype).to(cuda)
    x.view(-1)[:2] = torch.tensor([float("nan"), 50.0], dtype=dtype)  # a NaN and an outlier
    g = torch.randn(shape, generator=gen).to(dtype).to(cuda)
    q = A.QuantizeDequantize(enc, bits, sym, block_size=block, zero_point_shift=shift,
                             signed=signed).to(cuda)
    with q.compute_encodings():
        q(x.nan_to_num())
    with torch.no_grad():  # narrow the ranges a little so that every clamp fires
        q.min.mul_(0.8)
        q.max.mul_(0.7)

    xf = x.clone().requires_grad_(True)
    y = q(xf)
    y.backward(g)
    got = (y.detach(), xf.grad, q.min.grad.clone(), q.max.grad.clone())

    mn = q.min.detach().clone().requires_grad_(True)
    mx = q.max.detach().clone().requires_grad_(True)
    xs = x.clone().requires_grad_(True)
    s, o = Q.minmax_encodings(mn, mx, q.qmin, q.qmax, q.symmetric,
                              A._get_minimum_scale(q.qmax - q.qmin),
                              float(A.symmetric_offset(q.qmin, q.qmax)))
    y2 = Q.quantize_dequantize(xs, s, o, q.qmin, q.qmax, block_size=block,
                               zero_point_shift=shift)
    y2.backward(g)
    exp = (y2.detach(), xs.grad, mn.grad, mx.grad)
    for name, a, e in zip(("y", "dx", "d_min", "d_max"), got, exp):
        assert a.shape == e.shape and a.dtype == e.dtype, name
        assert torch.equal(torch.isnan(a), torch.isnan(e)), name
        assert torch.equal(a.nan_to_num(), e.nan_to_num()), name
    # the NaN element makes its own encoding's gradients NaN (in both paths); the others stay
    # finite
    fin = np.isfinite(got[2].cpu().numpy()).mean()
    assert fin == 0.0 if got[2].numel() == 1 else fin > 0.5


def test_fused_minmax_without_encoding_gradients(cuda):
    """Frozen min / max (requires_grad off): the fused forward, dx only."""
    x = torch.randn(64, 130, device=cuda)
    q = A.QuantizeDequantize((), 8, False).to(cuda)
    with q.compute_encodings():
        q(x)
    q.requires_grad_(False)
    xf = x.clone().requires_grad_(True)
    q(xf).sum().backward()
    s, o = q.get_encodings()
    xs = x.clone().requires_grad_(True)
    Q.quantize_dequantize(xs, s, o, q.qmin, q.qmax).sum().backward()
    assert torch.equal(xf.grad, xs.grad)
