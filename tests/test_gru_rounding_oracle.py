"""The reference's GRU rounding and saturation table (tests/recurrent/test_gru_rounding.py:12-195)
restated against the oracle's FP-carrier forward, at the reference's own fixture: hidden size 1,
one step, every grid of one bit width, gate outputs unsigned, weights symmetric with scale 1/32.

* x and h0 round the centred value half-to-even *before* the zero point is added, at 8 and 16
  bits, affine and power-of-two scales, zero points +-3 (:49-96);
* x saturates before any integer conversion and records its mask, for 8/16/26/32-bit signed
  and 31-bit unsigned grids, at the nextafter neighbours of both ends and at +-2^32; the FP32
  carrier stores the greatest fp32 code inside the integer domain (:140-191).

Expected values are the reference test's own closed forms.  The real-activation half-step test
(:97-138) needs the reference's USE_REAL_ACTIVATION build and is skipped there too.
"""
import numpy as np
import pytest
import torch

import gru_oracle as GO
import rxmet_gru_abi as A

f32 = np.float32
_UNSIGNED = ("update_gate_output", "reset_gate_output")


def _fixture(bits, pot2):
    qp = A.new_qparams(1)
    qp.use_pot2 = int(pot2)
    for name in A.GRID_NAMES:
        g = qp.g[A.GRID[name]]
        g.bits = bits
        g.is_unsigned = int(name in _UNSIGNED)
        g.scale = 1.0
        g.zero_point = 0
    for k in range(A.NCHAN):
        qp.chan_bits[k] = bits
        qp.chan_unsigned[k] = 0
        A.qparams_chan(qp, k)[:] = 1.0 / 32
    return qp


def _run(qp, x, h0, training=True):
    z3 = np.zeros((1, 3), f32)
    return GO.forward_quant(z3, z3, np.zeros(3, f32), np.zeros(3, f32), x, qp, h0=h0,
                            training=training)


@pytest.mark.parametrize("bits", [8, 16])
@pytest.mark.parametrize("pot2", [False, True])
@pytest.mark.parametrize("zero_point", [-3, 3])
def test_input_and_initial_state_round_before_zero_point(bits, pot2, zero_point):
    qp = _fixture(bits, pot2)
    lower, upper = -(1 << (bits - 1)), (1 << (bits - 1)) - 1

    def centered(zp):
        return np.array([lower - zp - 1.5, lower - zp - .5, lower - zp + .5, -2.5, -1.5, -.5, .5,
                         1.5, 2.5, upper - zp - .5, upper - zp + .5, upper - zp + 1.5], f32)

    xc = centered(zero_point)
    hc = centered(-zero_point)[::-1].copy()
    scale = .5 if pot2 else .75
    gx, gh = qp.g[A.GRID["x"]], qp.g[A.GRID["h"]]
    gx.scale = gh.scale = scale
    gx.zero_point = zero_point
    gh.zero_point = -zero_point
    x = (xc * f32(scale)).reshape(1, -1, 1)
    h0 = (hc * f32(scale)).reshape(-1, 1)
    out = _run(qp, x, h0)
    x_raw = (np.round(xc.astype(np.float64)) + zero_point).reshape(1, -1, 1)
    h_raw = (np.round(hc.astype(np.float64)) - zero_point).reshape(-1, 1)
    np.testing.assert_array_equal(out["x_q"], np.clip(x_raw, lower, upper).astype(f32))
    np.testing.assert_array_equal(out["h"][0],
                                  ((np.clip(h_raw, lower, upper) + zero_point) * scale).astype(f32))
    np.testing.assert_array_equal(out["x_mask"], ((x_raw >= lower) & (x_raw <= upper)).astype(np.uint8))
    np.testing.assert_array_equal(out["h0_mask"], ((h_raw >= lower) & (h_raw <= upper)).astype(np.uint8))
    ev = _run(qp, x, h0, training=False)
    np.testing.assert_array_equal(ev["x_q"], out["x_q"])
    np.testing.assert_array_equal(ev["h"], out["h"])


@pytest.mark.parametrize("bits,unsigned,float_upper", [
    (8, False, 127), (16, False, 32767), (26, False, 33554430), (32, False, 2147483520),
    (31, True, 2147483520)])
@pytest.mark.parametrize("pot2", [False, True])
def test_input_saturates_before_integer_conversion_and_records_mask(bits, unsigned, float_upper,
                                                                    pot2):
    qp = _fixture(8, pot2)
    gx = qp.g[A.GRID["x"]]
    gx.bits = bits
    gx.is_unsigned = int(unsigned)
    gx.scale = .5 if pot2 else 1.0
    lower = 0 if unsigned else -(1 << (bits - 1))
    upper = (1 << bits) - 1 if unsigned else (1 << (bits - 1)) - 1
    lo = torch.tensor(float(lower))
    hi = torch.tensor(float(upper))
    ninf, pinf = torch.tensor(float("-inf")), torch.tensor(float("inf"))
    codes = torch.stack([torch.tensor(float(-(1 << 32))), torch.nextafter(lo, ninf), lo,
                         torch.nextafter(lo, pinf), lo - 1, torch.tensor(-1.), torch.tensor(0.),
                         torch.tensor(1.), torch.nextafter(hi, ninf), hi, torch.nextafter(hi, pinf),
                         hi + 1, torch.tensor(float(1 << 32))]).numpy().astype(f32)
    x = (codes * f32(gx.scale)).reshape(1, -1, 1)
    out = _run(qp, x, np.zeros((codes.size, 1), f32))
    rounded = np.round(codes.astype(np.float64)).reshape(1, -1, 1)
    expected = np.clip(rounded, lower, float_upper).astype(f32)
    np.testing.assert_array_equal(out["x_q"], expected)
    assert (out["x_q"].astype(np.float64) <= upper).all()
    assert (out["x_q"].astype(np.float64) >= lower).all()
    assert np.isfinite(out["h"]).all()
    np.testing.assert_array_equal(out["x_mask"],
                                  ((rounded >= lower) & (rounded <= upper)).astype(np.uint8))
    ev = _run(qp, x, np.zeros((codes.size, 1), f32), training=False)
    np.testing.assert_array_equal(ev["x_q"], out["x_q"])
