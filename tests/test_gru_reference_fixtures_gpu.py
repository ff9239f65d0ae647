"""The reference's own QuantGRU tests, restated at their own tiny fixtures (hidden size 1) and run
through the MI355X drop-in boundary with the reference's argument and attribute names.

* tests/recurrent/test_gru_rounding.py:12-96 — x and h0 round the centred value half-to-even
  before the zero point is added (8 and 16 bits, affine and power-of-two, zero points +-3),
  with the masks; :140-191 — x saturates and records its mask at the nextafter neighbours of
  its grid ends;
* tests/recurrent/test_gru_autograd.py:57-93 — on tests/support/recurrent.py:62-87's
  fixed_gru_model (I = H = 1, power-of-two grids, one operator optionally squeezed to a tiny
  scale so that it clamps) the module's gradients equal autograd through the straight-through
  surrogate built from the module's own saved tensors, for output, hidden and combined losses;
* :121-133 — the eval forward keeps the same saved tensors and gradients as training.

Bars: codes and masks bit-exact against the reference test's closed forms; gradients within the
reference test's own tolerance (atol 1e-6, rtol 1e-5)."""
import json

import numpy as np
import pytest
import torch

import gru_ops
import quant_gru as Q

pytestmark = pytest.mark.gpu

_FIELDS = ("x", "h", "W", "R", "bw", "br", "weight_ih_linear", "weight_hh_linear",
           "update_gate_input", "update_gate_output", "reset_gate_input", "reset_gate_output",
           "new_gate_input", "new_gate_output", "mul_reset_hidden", "mul_old_contribution",
           "mul_new_contribution")
_CHANNEL_FIELDS = ("W", "R", "bw", "br")


def _fixture(bits, pot2, cuda):
    config = gru_ops.OperatorQuantConfig()
    for field in _FIELDS:
        setattr(config, field + "_", bits)
        setattr(config, field + "_unsigned_", field in ("update_gate_output", "reset_gate_output"))
        setattr(config, field + "_symmetric_", field in _CHANNEL_FIELDS)
    config.usePOT2_ = pot2
    parameters = gru_ops.GRUQuantParams()
    parameters.hidden_ = 1
    parameters.bitwidth_config_ = config
    for field in _FIELDS:
        setattr(parameters, "scale_" + field + "_",
                [1.0 / 32] * 3 if field in _CHANNEL_FIELDS else 1.0)
        if field not in _CHANNEL_FIELDS:
            setattr(parameters, "zp_" + field + "_", 0)
    arguments = dict(is_training=True, time_steps=1, batch_size=1, input_size=1, hidden_size=1,
                     W=torch.zeros(1, 3, device=cuda), R=torch.zeros(1, 3, device=cuda),
                     bw=torch.zeros(3, device=cuda), br=torch.zeros(3, device=cuda),
                     x=torch.zeros(1, 1, 1, device=cuda), h0=torch.zeros(1, 1, device=cuda),
                     quant_params=parameters)
    return arguments, parameters


@pytest.mark.parametrize("bits", [8, 16])
@pytest.mark.parametrize("pot2", [False, True])
@pytest.mark.parametrize("zero_point", [-3, 3])
def test_input_and_initial_state_round_before_zero_point(cuda, bits, pot2, zero_point):
    print(f"[gru rounding] bits={bits} pot2={pot2} zp={zero_point}", flush=True)
    arguments, parameters = _fixture(bits, pot2, cuda)
    lower, upper = -(1 << (bits - 1)), (1 << (bits - 1)) - 1

    def centered_values(zp):
        return torch.tensor([lower - zp - 1.5, lower - zp - .5, lower - zp + .5, -2.5, -1.5, -.5,
                             .5, 1.5, 2.5, upper - zp - .5, upper - zp + .5, upper - zp + 1.5],
                            device=cuda)

    x_centered = centered_values(zero_point)
    h_centered = centered_values(-zero_point).flip(0)
    scale = .5 if pot2 else .75
    parameters.scale_x_ = scale
    parameters.scale_h_ = scale
    parameters.zp_x_ = zero_point
    parameters.zp_h_ = -zero_point
    arguments["batch_size"] = x_centered.numel()
    arguments["x"] = (x_centered * scale).reshape(1, -1, 1)
    arguments["h0"] = (h_centered * scale).reshape(-1, 1)
    result = gru_ops.forward_quant_float_storage(**arguments)
    x_raw = (torch.round(x_centered) + zero_point).reshape(1, -1, 1)
    h_raw = (torch.round(h_centered) - zero_point).reshape(-1, 1)
    torch.testing.assert_close(result[6].float(), x_raw.clamp(lower, upper), rtol=0, atol=0)
    torch.testing.assert_close(result[0][0], (h_raw.clamp(lower, upper) + zero_point) * scale,
                               rtol=0, atol=0)
    torch.testing.assert_close(result[7], ((x_raw >= lower) & (x_raw <= upper)).to(torch.uint8),
                               rtol=0, atol=0)
    torch.testing.assert_close(result[8], ((h_raw >= lower) & (h_raw <= upper)).to(torch.uint8),
                               rtol=0, atol=0)
    arguments["is_training"] = False
    evaluated = gru_ops.forward_quant_float_storage(**arguments)
    torch.testing.assert_close(evaluated[6], result[6], rtol=0, atol=0)
    torch.testing.assert_close(evaluated[0], result[0], rtol=0, atol=0)


@pytest.mark.parametrize("bits,unsigned,float_upper", [(8, False, 127), (16, False, 32767)])
@pytest.mark.parametrize("pot2", [False, True])
def test_input_saturates_before_integer_conversion_and_records_mask(cuda, bits, unsigned,
                                                                    float_upper, pot2):
    print(f"[gru saturation] bits={bits} unsigned={unsigned} pot2={pot2}", flush=True)
    arguments, parameters = _fixture(8, pot2, cuda)
    config = parameters.bitwidth_config_
    config.x_ = bits
    config.x_unsigned_ = unsigned
    parameters.bitwidth_config_ = config
    parameters.scale_x_ = .5 if pot2 else 1.0
    lower = 0 if unsigned else -(1 << (bits - 1))
    upper = (1 << bits) - 1 if unsigned else (1 << (bits - 1)) - 1
    lo = torch.tensor(float(lower), device=cuda)
    hi = torch.tensor(float(upper), device=cuda)
    ninf = torch.tensor(float("-inf"), device=cuda)
    pinf = torch.tensor(float("inf"), device=cuda)
    codes = torch.stack([torch.tensor(float(-(1 << 32)), device=cuda), torch.nextafter(lo, ninf),
                         lo, torch.nextafter(lo, pinf), lo - 1, torch.tensor(-1., device=cuda),
                         torch.tensor(0., device=cuda), torch.tensor(1., device=cuda),
                         torch.nextafter(hi, ninf), hi, torch.nextafter(hi, pinf), hi + 1,
                         torch.tensor(float(1 << 32), device=cuda)])
    arguments["batch_size"] = codes.numel()
    arguments["x"] = (codes * parameters.scale_x_).reshape(1, -1, 1)
    arguments["h0"] = torch.zeros(codes.numel(), 1, device=cuda)
    result = gru_ops.forward_quant_float_storage(**arguments)
    rounded = torch.round(codes).double().reshape(1, -1, 1)
    torch.testing.assert_close(result[6], rounded.clamp(lower, float_upper).float(), rtol=0,
                               atol=0)
    assert torch.isfinite(result[0]).all()
    torch.testing.assert_close(result[7], ((rounded >= lower) & (rounded <= upper)).to(torch.uint8),
                               rtol=0, atol=0)
    arguments["is_training"] = False
    evaluated = gru_ops.forward_quant_float_storage(**arguments)
    torch.testing.assert_close(evaluated[6], result[6], rtol=0, atol=0)


def _fixed_gru_model(directory, cuda, clipped=None):
    """tests/support/recurrent.py:62-87: QuantGRU(1, 1) with fixed weights, calibrated on one
    value, its document rewritten to power-of-two grids (one operator squeezed to 1/4096 so that
    it clamps) and loaded back; QAT training mode."""
    m = Q.QuantGRU(1, 1).to(cuda)
    m.set_all_bitwidth(8)
    with torch.no_grad():
        m.weight_ih_l0.copy_(torch.tensor([[.2], [.1], [.3]], device=cuda))
        m.weight_hh_l0.copy_(torch.tensor([[.1], [.1], [.2]], device=cuda))
        m.bias_ih_l0.copy_(torch.tensor([.1, .1, .2], device=cuda))
        m.bias_hh_l0.copy_(torch.tensor([.1, .1, .4], device=cuda))
    m.calibrating = True
    with torch.no_grad():
        m(torch.tensor([[[.5]]], device=cuda))
    m.calibrating = False
    m.finalize_calibration()
    path = directory / "encodings.json"
    m.export_quant_params(str(path))
    data = json.loads(path.read_text())
    data["model_info"]["use_pot2_scale"] = True
    for name, e in data["operators"].items():
        scale = 1 / 32 if name.endswith("_input") or name.endswith("_linear") else 1 / 128
        if name in ("update_gate_output", "reset_gate_output"):
            scale = 1 / 256
        if name == clipped:
            scale = 1 / 4096
        channels = len(e["scale"]) if isinstance(e["scale"], list) else None
        lo, hi = (0, 255) if e["dtype"].startswith("U") else (-128, 127)
        e.update(scale=[scale] * channels if channels else scale,
                 zero_point=[0] * channels if channels else 0, symmetric=True,
                 real_min=[scale * lo] * channels if channels else scale * lo,
                 real_max=[scale * hi] * channels if channels else scale * hi)
    path.write_text(json.dumps(data))
    m.load_quant_params(str(path))
    m.use_quantization = True
    m.train()
    return m, data


def _swap_gates(t):
    r, z, n = t.chunk(3, dim=0)
    return torch.cat((z, r, n), dim=0)


def _surrogate(saved, enc):
    """Autograd through the straight-through construction of test_gru_autograd.py:21-48 on the
    module's saved tensors: every clamp masks its own input; gate derivatives use the
    dequantised gate outputs; values stay anchored to the kernel's."""
    (wq, rq, bwq, brq, xq, h, v, xmask, h0mask, wmask, rmask, bwmask, brmask, pmask, qmask,
     imask, omask, hmask) = saved

    def leaf(q, key):
        s = torch.tensor(enc["operators"][key]["scale"], device=q.device)
        return (q * s).detach().requires_grad_()

    w, r, bw, br = leaf(wq, "weight_ih"), leaf(rq, "weight_hh"), leaf(bwq, "bias_ih"), \
        leaf(brq, "bias_hh")
    x = leaf(xq, "input")
    h0 = h[0].detach().clone().requires_grad_()

    def masked(value, mask):
        return value.detach() + (value - value.detach()) * mask

    def anchor(value, actual):
        return actual.detach() + (value - value.detach())

    mw, mr, mbw, mbr, mx = (masked(w, wmask), masked(r, rmask), masked(bw, bwmask),
                            masked(br, brmask), masked(x, xmask))
    prev = masked(h0, h0mask)
    ys = []
    for t in range(x.shape[0]):
        p = masked(mx[t] @ mw + mbw, pmask[t])
        q = masked(prev @ mr + mbr, qmask[t])
        z0, r0, n0, qg = v[t].chunk(4, dim=-1)
        iz, ir, ig = imask[t].chunk(3, dim=-1)
        oz, orr, og = omask[t].chunk(3, dim=-1)
        pz, pr, pg = p.chunk(3, dim=-1)
        qz, qr, qn = q.chunk(3, dim=-1)

        def activation(pre, out, mask, derivative):
            return out.detach() + (pre - pre.detach()) * mask * derivative.detach()

        z = activation(pz + qz, z0, iz * oz, z0 * (1 - z0))
        reset = activation(pr + qr, r0, ir * orr, r0 * (1 - r0))
        candidate = activation(pg + reset * anchor(qn, qg), n0, ig * og, 1 - n0 * n0)
        prev = anchor(masked(z * prev + (1 - z) * candidate, hmask[t]), h[t + 1])
        ys.append(prev)
    return torch.stack(ys), prev.unsqueeze(0), (w, r, bw, br, x, h0)


@pytest.mark.parametrize("clipped", [None, "new_gate_input", "new_gate_output", "weight_ih_linear"])
@pytest.mark.parametrize("steps,batch", [(1, 1), (4, 2)])
@pytest.mark.parametrize("loss_source", ["output", "hidden", "both"])
def test_clamp_chain_rule_matches_surrogate(cuda, tmp_path, clipped, steps, batch, loss_source):
    print(f"[gru fixed model] clipped={clipped} steps={steps} batch={batch} loss={loss_source}",
          flush=True)
    m, enc = _fixed_gru_model(tmp_path, cuda, clipped)
    x = torch.linspace(.35, .65, steps * batch, device=cuda).reshape(steps, batch, 1)
    x.requires_grad_()
    h0 = torch.full((1, batch, 1), .2, device=cuda, requires_grad=True)
    y, hn = m(x, h0)
    saved = tuple(t.detach().clone() for t in y.grad_fn.saved_tensors)
    assert len(saved) == 18
    reference, reference_hn, leaves = _surrogate(saved, enc)
    if clipped in ("new_gate_input", "new_gate_output"):
        mask = saved[15 if clipped == "new_gate_input" else 16][..., 2]
        assert torch.all(mask == 0)
    if clipped == "weight_ih_linear":
        assert torch.all(saved[13] == 0)

    def loss(output, last):
        weights = torch.linspace(.3, 1.1, output.numel(), device=cuda).reshape_as(output)
        if loss_source == "output":
            return (output * weights).sum()
        if loss_source == "hidden":
            return last.square().sum()
        return (output * weights).sum() + last.square().sum()

    loss(y, hn).backward()
    loss(reference, reference_hn).backward()
    actual = [_swap_gates(m.weight_ih_l0.grad).t(), _swap_gates(m.weight_hh_l0.grad).t(),
              _swap_gates(m.bias_ih_l0.grad), _swap_gates(m.bias_hh_l0.grad), x.grad,
              h0.grad.squeeze(0)]
    for name, a, b in zip(["W", "R", "bias_ih", "bias_hh", "input", "h0"], actual, leaves):
        torch.testing.assert_close(a, b.grad, atol=1e-6, rtol=1e-5, msg=lambda s: f"{name}: {s}")


def _backward(model, value, h0):
    model.zero_grad(set_to_none=True)
    value = value.detach().clone().requires_grad_()
    h0 = h0.detach().clone().requires_grad_()
    y, last = model(value, h0)
    saved = [t.detach().clone() for t in y.grad_fn.saved_tensors]
    (y.square().sum() + last.sum()).backward()
    grads = {name: p.grad.detach().clone() for name, p in model.named_parameters()}
    grads.update(input=value.grad, hidden=h0.grad)
    return (y.detach(), last.detach()), saved, grads


@pytest.mark.parametrize("clipped", [None, "weight_ih_linear", "new_gate_input", "new_gate_output"])
def test_eval_saturation_uses_the_same_masks(cuda, tmp_path, clipped):
    """test_gru_autograd.py:121-133: eval keeps training's saved tensors and gradients."""
    model, _ = _fixed_gru_model(tmp_path, cuda, clipped)
    x = torch.tensor([[[.5]], [[.4]]], device=cuda)
    h = torch.tensor([[[.2]]], device=cuda)
    model.train()
    expected, cache, gradients = _backward(model, x, h)
    model.eval()
    actual, actual_cache, actual_gradients = _backward(model, x, h)
    for left, right in zip(expected, actual):
        torch.testing.assert_close(left, right, rtol=0, atol=0)
    for left, right in zip(cache, actual_cache):
        torch.testing.assert_close(left, right, rtol=0, atol=0)
    for name in gradients:
        torch.testing.assert_close(gradients[name], actual_gradients[name], rtol=0, atol=0)
