// ref_shim.cpp — C entry points over the reference's own CPU QuantGRU code, compiled
// from /root/reference/operators/quant-gru/src into oracle/_ref/libgru_ref.so by
// oracle/Makefile.  TEST INFRASTRUCTURE: used by tests/ (to pin the oracle's parameter
// derivation, LUT generation, calibration forward and the int-carrier agreement) and by
// bench.py's CPU-baseline legs, which time the reference's calibration and PTQ forwards;
// ref_gru_forward_int_codes pins the oracle's int32-carrier forward.
// Nothing here is part of the product.
#include <cstring>
#include <stdexcept>

#include "gru_host.h"
#include "gru_quant_cpu.h"
#include "quantize_ops_helper.h"
#include "rxmet_gru.h"

namespace {

QuantBitWidth bw_of(const rxmet_bitspec &b) {
  return QuantBitWidth(static_cast<int8_t>(b.bits), b.is_unsigned != 0);
}

OperatorQuantConfig::QuantizationGranularity gran_of(int g) {
  return g == RXMET_PER_TENSOR ? OperatorQuantConfig::PER_TENSOR
       : g == RXMET_PER_GATE   ? OperatorQuantConfig::PER_GATE
                               : OperatorQuantConfig::PER_CHANNEL;
}

OperatorQuantConfig config_of(const rxmet_gru_config &c) {
  OperatorQuantConfig o;
  QuantBitWidth *ops[RXMET_GRU_NGRIDS] = {
      &o.x_, &o.h_, &o.weight_ih_linear_, &o.weight_hh_linear_, &o.update_gate_input_,
      &o.reset_gate_input_, &o.new_gate_input_, &o.update_gate_output_, &o.reset_gate_output_,
      &o.new_gate_output_, &o.mul_reset_hidden_, &o.mul_new_contribution_,
      &o.mul_old_contribution_};
  bool *syms[RXMET_GRU_NGRIDS] = {
      &o.x_symmetric_, &o.h_symmetric_, &o.weight_ih_linear_symmetric_,
      &o.weight_hh_linear_symmetric_, &o.update_gate_input_symmetric_,
      &o.reset_gate_input_symmetric_, &o.new_gate_input_symmetric_,
      &o.update_gate_output_symmetric_, &o.reset_gate_output_symmetric_,
      &o.new_gate_output_symmetric_, &o.mul_reset_hidden_symmetric_,
      &o.mul_new_contribution_symmetric_, &o.mul_old_contribution_symmetric_};
  for (int i = 0; i < RXMET_GRU_NGRIDS; ++i) {
    *ops[i] = bw_of(c.op[i]);
    *syms[i] = c.op[i].symmetric != 0;
  }
  QuantBitWidth *ch[4] = {&o.W_, &o.R_, &o.bw_, &o.br_};
  bool *chs[4] = {&o.W_symmetric_, &o.R_symmetric_, &o.bw_symmetric_, &o.br_symmetric_};
  OperatorQuantConfig::QuantizationGranularity *chg[4] = {&o.W_granularity_, &o.R_granularity_,
                                                          &o.bw_granularity_, &o.br_granularity_};
  for (int k = 0; k < 4; ++k) {
    *ch[k] = bw_of(c.chan[k]);
    *chs[k] = c.chan[k].symmetric != 0;
    *chg[k] = gran_of(c.chan[k].granularity);
  }
  o.usePOT2_ = c.use_pot2 != 0;
  o.pot_scale_method_ = static_cast<PotScaleMethod>(c.pot_method);
  o.pot_scale_tolerance_ = c.pot_tolerance;
  return o;
}

void lut_out(const SigmoidLUT &l, rxmet_pwl_lut *o) {
  for (int i = 0; i < 16; ++i) {
    o->seg[i].q_b = l.segments[i].q_b;
    o->seg[i].n = l.segments[i].n_BX_total;
    o->seg[i].c = l.segments[i].term_c_precomputed;
    o->seg[i].threshold = l.segments[i].threshold;
  }
  o->zp_x = l.zp_x;
}

// GRUQuantParams straight from a parameter block (scales, zero points, bit widths; weights
// per channel), with the LUTs the reference generates from them.
GRUQuantParams params_of(const rxmet_gru_qparams &qp) {
  GRUQuantParams p;
  const int H = qp.hidden, C = 3 * H;
  OperatorQuantConfig &o = p.bitwidth_config_;
  QuantBitWidth *ops[RXMET_GRU_NGRIDS] = {
      &o.x_, &o.h_, &o.weight_ih_linear_, &o.weight_hh_linear_, &o.update_gate_input_,
      &o.reset_gate_input_, &o.new_gate_input_, &o.update_gate_output_, &o.reset_gate_output_,
      &o.new_gate_output_, &o.mul_reset_hidden_, &o.mul_new_contribution_,
      &o.mul_old_contribution_};
  QuantParam *g[RXMET_GRU_NGRIDS] = {
      &p.x_, &p.h_, &p.weight_ih_linear_, &p.weight_hh_linear_, &p.update_gate_input_,
      &p.reset_gate_input_, &p.new_gate_input_, &p.update_gate_output_,
      &p.reset_gate_output_, &p.new_gate_output_, &p.mul_reset_hidden_,
      &p.mul_new_contribution_, &p.mul_old_contribution_};
  for (int i = 0; i < RXMET_GRU_NGRIDS; ++i) {
    *ops[i] = QuantBitWidth(static_cast<int8_t>(qp.g[i].bits), qp.g[i].is_unsigned != 0);
    g[i]->scale = qp.g[i].scale;
    g[i]->zero_point = qp.g[i].zero_point;
  }
  QuantBitWidth *ch[4] = {&o.W_, &o.R_, &o.bw_, &o.br_};
  ChannelQuantParam *cp[4] = {&p.W_, &p.R_, &p.bw_, &p.br_};
  for (int k = 0; k < 4; ++k) {
    *ch[k] = QuantBitWidth(static_cast<int8_t>(qp.chan_bits[k]), qp.chan_unsigned[k] != 0);
    cp[k]->hidden = H;
    cp[k]->resize(C);
    for (int c = 0; c < C; ++c) cp[k]->channel(c).scale = qp.chan_scale[k][c];
  }
  o.usePOT2_ = qp.use_pot2 != 0;
  p.hidden_ = H;
  generate_piecewise_linear_lut_to_params(p);
  return p;
}

}  // namespace

extern "C" {

// calculateGRUQuantitativeParameters; qparams->chan_scale[k] are caller arrays [3H].
int ref_gru_make_params(const rxmet_gru_ranges *r, const rxmet_gru_config *c,
                        rxmet_gru_qparams *out, rxmet_pwl_lut luts[3]) {
  try {
    const int H = r->hidden, C = 3 * H;
    GRUQuantizationRanges q(H);
    float *mins[RXMET_GRU_NGRIDS] = {
        &q.min_x_, &q.min_h_, &q.min_Wx_, &q.min_Rh_, &q.min_update_gate_input_,
        &q.min_reset_gate_input_, &q.min_new_gate_input_, &q.min_update_gate_output_,
        &q.min_reset_gate_output_, &q.min_new_gate_output_, &q.min_mul_reset_hidden_,
        &q.min_mul_new_contribution_, &q.min_mul_old_contribution_};
    float *maxs[RXMET_GRU_NGRIDS] = {
        &q.max_x_, &q.max_h_, &q.max_Wx_, &q.max_Rh_, &q.max_update_gate_input_,
        &q.max_reset_gate_input_, &q.max_new_gate_input_, &q.max_update_gate_output_,
        &q.max_reset_gate_output_, &q.max_new_gate_output_, &q.max_mul_reset_hidden_,
        &q.max_mul_new_contribution_, &q.max_mul_old_contribution_};
    for (int i = 0; i < RXMET_GRU_NGRIDS; ++i) {
      *mins[i] = r->min[i];
      *maxs[i] = r->max[i];
    }
    std::vector<float> *cmin[4] = {&q.min_W_, &q.min_R_, &q.min_bw_, &q.min_br_};
    std::vector<float> *cmax[4] = {&q.max_W_, &q.max_R_, &q.max_bw_, &q.max_br_};
    for (int k = 0; k < 4; ++k) {
      cmin[k]->assign(r->chan_min[k], r->chan_min[k] + C);
      cmax[k]->assign(r->chan_max[k], r->chan_max[k] + C);
    }
    GRUQuantParams p = calculateGRUQuantitativeParameters(q, config_of(*c));
    const QuantParam *g[RXMET_GRU_NGRIDS] = {
        &p.x_, &p.h_, &p.weight_ih_linear_, &p.weight_hh_linear_, &p.update_gate_input_,
        &p.reset_gate_input_, &p.new_gate_input_, &p.update_gate_output_,
        &p.reset_gate_output_, &p.new_gate_output_, &p.mul_reset_hidden_,
        &p.mul_new_contribution_, &p.mul_old_contribution_};
    out->hidden = H;
    out->use_pot2 = c->use_pot2;
    for (int i = 0; i < RXMET_GRU_NGRIDS; ++i) {
      out->g[i].scale = g[i]->scale;
      out->g[i].zero_point = g[i]->zero_point;
      out->g[i].bits = c->op[i].bits;
      out->g[i].is_unsigned = c->op[i].bits >= 32 ? 0 : c->op[i].is_unsigned;
    }
    const ChannelQuantParam *ch[4] = {&p.W_, &p.R_, &p.bw_, &p.br_};
    for (int k = 0; k < 4; ++k) {
      out->chan_bits[k] = c->chan[k].bits;
      out->chan_unsigned[k] = c->chan[k].bits >= 32 ? 0 : c->chan[k].is_unsigned;
      for (int i = 0; i < C; ++i) out->chan_scale[k][i] = ch[k]->channel(i).scale;
    }
    if (luts) {
      lut_out(p.sigmoid_update_gate_lut_, &luts[0]);
      lut_out(p.sigmoid_reset_gate_lut_, &luts[1]);
      lut_out(p.tanh_new_gate_lut_, &luts[2]);
    }
    return 0;
  } catch (const std::exception &) {
    return -1;
  }
}

// forwardWithCalibrationCPU with MINMAX; stats laid out as rxmet_gru_forward_calibrate.
int ref_gru_forward_calibrate(int T, int B, int I, int H, const float *W, const float *R,
                              const float *bw, const float *br, const float *x, const float *h0,
                              float *h, float *v, float *stats) {
  try {
    const int C = 3 * H;
    GRUQuantizationRanges q(H);
    OperatorQuantConfig cfg;
    forwardWithCalibrationCPU(T, B, I, H, W, R, bw, br, x, h0, CalibrationMethod::MINMAX, &q,
                              nullptr, cfg, h, v);
    const float mins[RXMET_GRU_NGRIDS] = {
        q.min_x_, q.min_h_, q.min_Wx_, q.min_Rh_, q.min_update_gate_input_,
        q.min_reset_gate_input_, q.min_new_gate_input_, q.min_update_gate_output_,
        q.min_reset_gate_output_, q.min_new_gate_output_, q.min_mul_reset_hidden_,
        q.min_mul_new_contribution_, q.min_mul_old_contribution_};
    const float maxs[RXMET_GRU_NGRIDS] = {
        q.max_x_, q.max_h_, q.max_Wx_, q.max_Rh_, q.max_update_gate_input_,
        q.max_reset_gate_input_, q.max_new_gate_input_, q.max_update_gate_output_,
        q.max_reset_gate_output_, q.max_new_gate_output_, q.max_mul_reset_hidden_,
        q.max_mul_new_contribution_, q.max_mul_old_contribution_};
    for (int i = 0; i < RXMET_GRU_NGRIDS; ++i) {
      stats[i] = mins[i];
      stats[RXMET_GRU_NGRIDS + i] = maxs[i];
    }
    const std::vector<float> *cmin[4] = {&q.min_W_, &q.min_R_, &q.min_bw_, &q.min_br_};
    const std::vector<float> *cmax[4] = {&q.max_W_, &q.max_R_, &q.max_bw_, &q.max_br_};
    float *chan = stats + 2 * RXMET_GRU_NGRIDS;
    for (int k = 0; k < 4; ++k) {
      std::memcpy(chan + 2 * k * C, cmin[k]->data(), sizeof(float) * C);
      std::memcpy(chan + 2 * k * C + C, cmax[k]->data(), sizeof(float) * C);
    }
    return 0;
  } catch (const std::exception &) {
    return -1;
  }
}

// Reference CPU PTQ forward (integer carrier): quantitativeWeightCPU + quantGRUForwardCPU.
int ref_gru_forward_ptq(int T, int B, int I, int H, const float *W, const float *R,
                        const float *bw, const float *br, const float *x, const float *h0,
                        const rxmet_gru_ranges *r, const rxmet_gru_config *c, float *h, float *v) {
  try {
    const int C = 3 * H;
    std::vector<float> s[4];
    rxmet_gru_qparams tmp{};
    for (int k = 0; k < 4; ++k) {
      s[k].resize(C);
      tmp.chan_scale[k] = s[k].data();
    }
    GRUQuantizationRanges q(H);
    (void)q;
    // Build GRUQuantParams through the reference itself.
    rxmet_pwl_lut luts[3];
    if (ref_gru_make_params(r, c, &tmp, luts)) return -1;
    GRUQuantizationRanges rq(H);
    float *mins[RXMET_GRU_NGRIDS] = {
        &rq.min_x_, &rq.min_h_, &rq.min_Wx_, &rq.min_Rh_, &rq.min_update_gate_input_,
        &rq.min_reset_gate_input_, &rq.min_new_gate_input_, &rq.min_update_gate_output_,
        &rq.min_reset_gate_output_, &rq.min_new_gate_output_, &rq.min_mul_reset_hidden_,
        &rq.min_mul_new_contribution_, &rq.min_mul_old_contribution_};
    float *maxs[RXMET_GRU_NGRIDS] = {
        &rq.max_x_, &rq.max_h_, &rq.max_Wx_, &rq.max_Rh_, &rq.max_update_gate_input_,
        &rq.max_reset_gate_input_, &rq.max_new_gate_input_, &rq.max_update_gate_output_,
        &rq.max_reset_gate_output_, &rq.max_new_gate_output_, &rq.max_mul_reset_hidden_,
        &rq.max_mul_new_contribution_, &rq.max_mul_old_contribution_};
    for (int i = 0; i < RXMET_GRU_NGRIDS; ++i) {
      *mins[i] = r->min[i];
      *maxs[i] = r->max[i];
    }
    std::vector<float> *cmin[4] = {&rq.min_W_, &rq.min_R_, &rq.min_bw_, &rq.min_br_};
    std::vector<float> *cmax[4] = {&rq.max_W_, &rq.max_R_, &rq.max_bw_, &rq.max_br_};
    for (int k = 0; k < 4; ++k) {
      cmin[k]->assign(r->chan_min[k], r->chan_min[k] + C);
      cmax[k]->assign(r->chan_max[k], r->chan_max[k] + C);
    }
    GRUQuantParams p = calculateGRUQuantitativeParameters(rq, config_of(*c));
    // the reference writes v (gate codes, dequantised) only in training mode, the only
    // difference training makes to its CPU forward (gru_forward_cpu_quant.cc:199)
    quantGRUForwardCPU(v != nullptr, T, B, I, H, W, R, bw, br, x, h0, p, h, v);
    return 0;
  } catch (const std::exception &) {
    return -1;
  }
}

// The reference's CPU int32 carrier on codes: quantitativeWeightCPU, the boundary
// quantisation of quantGRUForwardCPU (src/gru_host.cc:161-216) unless x_q / h0_q are given
// (then as quantGRUForwardIntIO, src/gru_interface.cc:561-627, on the CPU carrier), and
// ForwardPassQuantCPU::Run.  Writes the int32 h codes [T+1, B, H], the v codes [T, B, 4H]
// (when v_q is non-null; training mode) and, when non-null, the weight and input codes.
int ref_gru_forward_int_codes(int T, int B, int I, int H, const float *W, const float *R,
                              const float *bw, const float *br, const float *x,
                              const int32_t *x_q_in, const float *h0, const int32_t *h0_q_in,
                              const rxmet_gru_qparams *qp, int32_t *h_q, int32_t *v_q,
                              int32_t *W_q, int32_t *R_q, int32_t *bw_q, int32_t *br_q,
                              int32_t *x_q) {
  try {
    const int C = 3 * H;
    const GRUQuantParams p = params_of(*qp);
    std::vector<int32_t> wq(static_cast<size_t>(I) * C), rq(static_cast<size_t>(H) * C), bwq(C),
        brq(C);
    quantitativeWeightCPU(I, H, W, R, bw, br, p, wq.data(), rq.data(), bwq.data(), brq.data());
    const bool pot = p.bitwidth_config_.usePOT2_;
    const size_t nx = static_cast<size_t>(T) * B * I, nh = static_cast<size_t>(B) * H;
    std::vector<int32_t> xq(nx);
    if (x_q_in) {
      std::memcpy(xq.data(), x_q_in, sizeof(int32_t) * nx);
    } else {
      for (size_t i = 0; i < nx; ++i)
        xq[i] = quantize(x[i], toFixedScale(p.x_, pot), p.x_.zero_point, p.bitwidth_config_.x_);
    }
    for (size_t i = 0; i < nh; ++i) {
      if (h0_q_in)
        h_q[i] = h0_q_in[i];
      else if (h0)
        h_q[i] = quantize(h0[i], toFixedScale(p.h_, pot), p.h_.zero_point, p.bitwidth_config_.h_);
      else
        h_q[i] = p.h_.zero_point;
    }
    cpu::ForwardPassQuantCPU fwd(v_q != nullptr, B, I, H);
    fwd.setRescaleParam(p);
    fwd.Run(T, wq.data(), rq.data(), bwq.data(), brq.data(), xq.data(), h_q, v_q, 0.0f, nullptr);
    if (W_q) std::memcpy(W_q, wq.data(), sizeof(int32_t) * wq.size());
    if (R_q) std::memcpy(R_q, rq.data(), sizeof(int32_t) * rq.size());
    if (bw_q) std::memcpy(bw_q, bwq.data(), sizeof(int32_t) * C);
    if (br_q) std::memcpy(br_q, brq.data(), sizeof(int32_t) * C);
    if (x_q) std::memcpy(x_q, xq.data(), sizeof(int32_t) * nx);
    return 0;
  } catch (const std::exception &) {
    return -1;
  }
}

}  // extern "C"
