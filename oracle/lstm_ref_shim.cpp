// lstm_ref_shim.cpp — extern "C" entry points over the reference's own QuantLSTM CPU code,
// compiled from /root/reference by oracle/Makefile into oracle/_ref/liblstm_ref.so.
//
// TEST INFRASTRUCTURE ONLY: used by tests/ to pin oracle/lstm_oracle.c against the
// reference's finalizeQuantParams (src/lstm/quant_params.cc), deriveLstmExecutionParams
// (src/lstm/lstm_execution_params.cc), lstmForwardQuantizedFpCpuReference
// (src/lstm/forward_quantized_fp_cpu.cc), lstmForwardFloatCpu (src/lstm/forward_float_cpu.cc),
// LstmCalibrationCollector (src/lstm/calibration.cc) and lstmBackwardFloatCpu
// (src/lstm/backward_float_cpu.cc).  Only data crosses this file; no reference source is
// reproduced here.
#include <cstring>
#include <exception>
#include <string>
#include <vector>

#include "lstm/backward_float_cpu.h"
#include "lstm/calibration.h"
#include "lstm/forward_cpu.h"
#include "lstm/forward_float.h"
#include "lstm/lstm_execution_params.h"
#include "lstm/quant_params.h"
#include "quantization/float_carrier_ops.h"
#include "rxmet_lstm.h"

using namespace quant_lstm;

namespace {

thread_local std::string g_err;

LstmOperatorQuantConfig to_config(const rxmet_lstm_config &c) {
  LstmOperatorQuantConfig r;
  r.schema_version = 1;
  r.scale_mode = c.scale_mode == RXMET_LSTM_POT2 ? quantization::ScaleMode::Pot2
                                                 : quantization::ScaleMode::Affine;
  for (int i = 0; i < RXMET_LSTM_NOPS; ++i) {
    r.operators[i].type.bitwidth = static_cast<std::uint8_t>(c.op[i].bits);
    r.operators[i].type.is_unsigned = c.op[i].is_unsigned != 0;
    r.operators[i].type.is_symmetric = c.op[i].is_symmetric != 0;
    r.operators[i].granularity = static_cast<QuantGranularity>(c.op[i].granularity);
  }
  return r;
}

LstmQuantParams to_params(const rxmet_lstm_params &p) {
  LstmQuantParams q;
  q.hidden_size = p.hidden;
  q.bias_enabled = p.bias_enabled != 0;
  const int C = 4 * p.hidden;
  for (int op = 0; op < RXMET_LSTM_NOPS; ++op) {
    auto &d = q.operators[op];
    d.source_granularity = static_cast<QuantGranularity>(p.config.op[op].granularity);
    const bool param = op >= RXMET_LSTM_W_IH && op <= RXMET_LSTM_B_HH;
    const bool bias = op == RXMET_LSTM_B_IH || op == RXMET_LSTM_B_HH;
    if (bias && !p.bias_enabled) continue;
    const std::size_t groups = quantizationGroupCount(static_cast<QuantOperator>(op),
                                                      d.source_granularity, p.hidden);
    d.group_diagnostics.assign(groups, {});
    if (param) {
      for (int c = 0; c < C; ++c)
        d.values.push_back({p.chan_scale[op - RXMET_LSTM_W_IH][c], 0});
    } else {
      d.values.push_back({p.scale[op], p.zero_point[op]});
    }
  }
  return q;
}

void put_rescale(const ExecutionRescale &e, rxmet_lstm_rescale *o) {
  o->is_mshift = e.kind == ExecutionRescaleKind::MShift;
  o->multiplier = o->is_mshift ? e.m_shift.multiplier : 0;
  o->shift = o->is_mshift ? e.m_shift.shift : e.pot2.shift;
}

}  // namespace

extern "C" {

const char *ref_lstm_error() { return g_err.c_str(); }

int ref_lstm_finalize(const float *stats, const rxmet_lstm_config *cfg, int H, int bias,
                      rxmet_lstm_params *out) {
  try {
    const auto config = to_config(*cfg);
    LstmQuantizationRanges ranges;
    ranges.reset(config, H, bias != 0);
    const int C = 4 * H;
    for (int op = 0; op < RXMET_LSTM_NOPS; ++op) {
      auto &groups = ranges.operators[op];
      if (groups.empty()) continue;
      const bool param = op >= RXMET_LSTM_W_IH && op <= RXMET_LSTM_B_HH;
      if (!param) {
        groups[0].minimum = stats[op];
        groups[0].maximum = stats[RXMET_LSTM_NOPS + op];
        groups[0].sample_count = 1;
        continue;
      }
      const float *mn = stats + 2 * RXMET_LSTM_NOPS + static_cast<std::size_t>(op - RXMET_LSTM_W_IH) * 2 * C;
      const float *mx = mn + C;
      const std::size_t span = C / groups.size();
      for (std::size_t g = 0; g < groups.size(); ++g)
        for (std::size_t c = g * span; c < (g + 1) * span; ++c) {
          CalibrationRange r;
          r.minimum = mn[c];
          r.maximum = mx[c];
          r.sample_count = 1;
          groups[g].merge(r);
        }
    }
    const auto q = finalizeQuantParams(config, ranges, H, bias != 0);
    out->hidden = H;
    out->bias_enabled = bias;
    out->config = *cfg;
    for (int op = 0; op < RXMET_LSTM_NOPS; ++op) {
      const auto &v = q.operators[op].values;
      const bool param = op >= RXMET_LSTM_W_IH && op <= RXMET_LSTM_B_HH;
      if (param) {
        out->scale[op] = 0.0f;
        out->zero_point[op] = 0;
        for (std::size_t c = 0; c < v.size(); ++c) out->chan_scale[op - RXMET_LSTM_W_IH][c] = v[c].scale;
      } else {
        out->scale[op] = v[0].scale;
        out->zero_point[op] = v[0].zero_point;
      }
    }
    return 0;
  } catch (const std::exception &e) {
    g_err = e.what();
    return -1;
  }
}

int ref_lstm_exec(const rxmet_lstm_params *p, int I, rxmet_lstm_rescale *acc_to_lin,
                  rxmet_lstm_rescale *bias_to_acc, rxmet_lstm_rescale *lin_to_gate,
                  rxmet_lstm_q31 *cell, rxmet_lstm_rescale *hid) {
  try {
    const auto config = to_config(p->config);
    const auto q = to_params(*p);
    const auto e = deriveLstmExecutionParams(config, q, I, false);
    const int C = 4 * p->hidden;
    for (int c = 0; c < C; ++c) {
      put_rescale(e.input_hidden_linear.accumulator_to_output[c], &acc_to_lin[c]);
      put_rescale(e.hidden_hidden_linear.accumulator_to_output[c], &acc_to_lin[C + c]);
      if (p->bias_enabled) {
        put_rescale(e.input_hidden_linear.bias_to_accumulator[c], &bias_to_acc[c]);
        put_rescale(e.hidden_hidden_linear.bias_to_accumulator[c], &bias_to_acc[C + c]);
      }
    }
    for (int g = 0; g < 4; ++g) {
      put_rescale(e.gates[g].input_hidden_to_gate, &lin_to_gate[g]);
      put_rescale(e.gates[g].hidden_hidden_to_gate, &lin_to_gate[4 + g]);
    }
    const Q31Scale *cs[2] = {&e.cell.forget_scale, &e.cell.input_scale};
    for (int k = 0; k < 2; ++k) {
      cell[k].multiplier = cs[k]->multiplier;
      cell[k].mantissa = cs[k]->fp_mantissa;
      cell[k].exponent = cs[k]->fp_exponent;
      cell[k].uses_fp = cs[k]->uses_fp_scale ? 1 : 0;
    }
    put_rescale(e.hidden.product_to_output, hid);
    return 0;
  } catch (const std::exception &e) {
    g_err = e.what();
    return -1;
  }
}

// Quantised forward of the reference: float inputs are quantised with the reference's
// own quantizeFp, then lstmForwardQuantizedFpCpuReference runs on the codes.  Outputs
// are codes; traces [T,B,4H] / [T,B,H] as in LstmFpReferenceTrace.
int ref_lstm_forward_fp(int T, int B, int I, int H, const float *W_ih, const float *W_hh,
                        const float *b_ih, const float *b_hh, const float *x, const float *h0,
                        const float *c0, const rxmet_lstm_params *p, float *out_codes,
                        float *hn_codes, float *cn_codes, float *ih_lin, float *hh_lin,
                        float *gate_in, float *gate_out, float *cell, float *cell_tanh) {
  try {
    const auto config = to_config(p->config);
    const auto q = to_params(*p);
    const auto e = deriveLstmExecutionParams(config, q, I, false);
    const int C = 4 * H;
    auto quant = [&](float v, QuantOperator id, int channel) {
      const auto &pt = q.at(id).values.at(channel);
      return quantization::quantizeFp(v, pt, config.at(id).type);
    };
    std::vector<float> xq(static_cast<std::size_t>(T) * B * I), wi(static_cast<std::size_t>(C) * I),
        wh(static_cast<std::size_t>(C) * H), bi(C), bh(C), hq(static_cast<std::size_t>(B) * H),
        cq(static_cast<std::size_t>(B) * H);
    for (std::size_t i = 0; i < xq.size(); ++i) xq[i] = quant(x[i], QuantOperator::Input, 0);
    for (int c = 0; c < C; ++c) {
      for (int k = 0; k < I; ++k)
        wi[static_cast<std::size_t>(c) * I + k] =
            quant(W_ih[static_cast<std::size_t>(c) * I + k], QuantOperator::WeightInputHidden, c);
      for (int k = 0; k < H; ++k)
        wh[static_cast<std::size_t>(c) * H + k] =
            quant(W_hh[static_cast<std::size_t>(c) * H + k], QuantOperator::WeightHiddenHidden, c);
      if (p->bias_enabled) {
        bi[c] = quant(b_ih[c], QuantOperator::BiasInputHidden, c);
        bh[c] = quant(b_hh[c], QuantOperator::BiasHiddenHidden, c);
      }
    }
    if (h0) {
      for (int i = 0; i < B * H; ++i) {
        hq[i] = quant(h0[i], QuantOperator::Output, 0);
        cq[i] = quant(c0[i], QuantOperator::CellState, 0);
      }
    }
    LstmFpCarrierWeights w{wi.data(), wh.data(), p->bias_enabled ? bi.data() : nullptr,
                           p->bias_enabled ? bh.data() : nullptr};
    LstmFpReferenceTrace trace;
    LstmShape shape{T, B, I, H};
    lstmForwardQuantizedFpCpuReference(shape, w, xq.data(), h0 ? hq.data() : nullptr,
                                       h0 ? cq.data() : nullptr, config, q, e, out_codes, hn_codes,
                                       cn_codes, &trace);
    auto cp = [](const std::vector<float> &v, float *d) {
      if (d) std::memcpy(d, v.data(), sizeof(float) * v.size());
    };
    cp(trace.weight_ih_linear, ih_lin);
    cp(trace.weight_hh_linear, hh_lin);
    cp(trace.gate_inputs, gate_in);
    cp(trace.gate_outputs, gate_out);
    cp(trace.cell_states, cell);
    cp(trace.cell_tanh_outputs, cell_tanh);
    return 0;
  } catch (const std::exception &e) {
    g_err = e.what();
    return -1;
  }
}

int ref_lstm_forward_float(int T, int B, int I, int H, const float *W_ih, const float *W_hh,
                           const float *b_ih, const float *b_hh, const float *x, const float *h0,
                           const float *c0, float *out, float *hn, float *cn) {
  try {
    LstmShape shape{T, B, I, H};
    LstmFloatWeights w{W_ih, W_hh, b_ih, b_hh};
    lstmForwardFloatCpu(shape, w, x, h0, c0, out, hn, cn, nullptr);
    return 0;
  } catch (const std::exception &e) {
    g_err = e.what();
    return -1;
  }
}

// One calibration batch through the reference collector (parameters per channel), written
// into the rxmet stats layout (merged with the existing contents).
int ref_lstm_calibrate(int T, int B, int I, int H, const float *W_ih, const float *W_hh,
                       const float *b_ih, const float *b_hh, const float *x, const float *h0,
                       const float *c0, float *stats) {
  try {
    rxmet_lstm_config rc{};
    rc.scale_mode = RXMET_LSTM_AFFINE;
    for (int op = 0; op < RXMET_LSTM_NOPS; ++op) {
      const bool param = op >= RXMET_LSTM_W_IH && op <= RXMET_LSTM_B_HH;
      rc.op[op] = {8, 0, 1, param ? RXMET_LSTM_PER_CHANNEL : RXMET_LSTM_PER_TENSOR};
    }
    LstmCalibrationCollector col(to_config(rc), I, H, b_ih != nullptr);
    LstmShape shape{T, B, I, H};
    LstmFloatWeights w{W_ih, W_hh, b_ih, b_hh};
    col.collect(shape, w, x, h0, c0);
    const auto &r = col.ranges();
    const int C = 4 * H;
    for (int op = 0; op < RXMET_LSTM_NOPS; ++op) {
      const auto &g = r.operators[op];
      if (g.empty()) continue;
      const bool param = op >= RXMET_LSTM_W_IH && op <= RXMET_LSTM_B_HH;
      if (!param) {
        stats[op] = std::min(stats[op], g[0].minimum);
        stats[RXMET_LSTM_NOPS + op] = std::max(stats[RXMET_LSTM_NOPS + op], g[0].maximum);
        continue;
      }
      float *mn = stats + 2 * RXMET_LSTM_NOPS + static_cast<std::size_t>(op - RXMET_LSTM_W_IH) * 2 * C;
      float *mx = mn + C;
      for (int c = 0; c < C; ++c) {
        mn[c] = std::min(mn[c], g[c].minimum);
        mx[c] = std::max(mx[c], g[c].maximum);
      }
    }
    return 0;
  } catch (const std::exception &e) {
    g_err = e.what();
    return -1;
  }
}

int ref_lstm_backward_float(int T, int B, int I, int H, const float *W_ih, const float *W_hh,
                            const float *x, const float *h0, const float *c0,
                            const float *gate_out, const float *cell, const float *cell_tanh,
                            const float *hidden, const float *grad_out, const float *grad_hn,
                            const float *grad_cn, float *dx, float *dwi, float *dwh, float *dbi,
                            float *dbh, float *dh0, float *dc0) {
  try {
    LstmShape shape{T, B, I, H};
    LstmFloatWeights w{W_ih, W_hh, nullptr, nullptr};
    LstmFloatCpuBackwardTrace tr{gate_out, cell, cell_tanh, hidden};
    LstmFloatCpuGradients g{dx, dwi, dwh, dbi, dbh, dh0, dc0};
    lstmBackwardFloatCpu(shape, w, x, h0, c0, tr, grad_out, grad_hn, grad_cn, g);
    return 0;
  } catch (const std::exception &e) {
    g_err = e.what();
    return -1;
  }
}

}  // extern "C"
