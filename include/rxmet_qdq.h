/*
 * rxmet_qdq.h — C ABI of the MI355X fake-quantization (QuantizeDequantize) kernels.
 *
 * Every entry point takes plain device pointers, element counts and a hipStream_t
 * (passed as void*), enqueues its kernels on that stream and returns 0 on success or a
 * negative status; rxmet_last_error() then holds the message.  Nothing here allocates
 * device memory: reductions take a caller-provided workspace of
 * rxmet_qdq_workspace_bytes() bytes.
 *
 * Tensor layout.  A tensor of N = outer * C * inner fp32 elements is addressed as
 * [outer, C, inner] (row-major); element i uses encoding c = (i / inner) % C.  This
 * covers per-tensor encodings (C = 1) and any single-axis per-channel encoding, which
 * are the two encoding shapes aimet_torch's fast path distinguishes
 * (reference: src/aimet_torch/v2/quantization/affine/backends/torch_builtins.py:287-361).
 *
 * Modes.
 *   RXMET_QDQ_LEARNABLE  — QuantDequantFunc semantics: q = rint(x / s) - o,
 *                          y = (clamp(q, qmin, qmax) + o) * s
 *                          (torch_builtins.py:640-672); offset o is AIMET's offset,
 *                          i.e. the negated zero point.
 *   RXMET_QDQ_FROZEN     — torch.fake_quantize_per_{tensor,channel}_affine semantics
 *                          used by the frozen-encoding fast path: q = rint(x * (1/s)) + zp,
 *                          zp = -(int)o, y = (clamp(q) - zp) * s  (torch_builtins.py:221-249),
 *                          with NaN kept (:249).
 * Rounding is round-half-to-even throughout.  NaN inputs give NaN outputs and zero
 * gradients; +-inf saturate to the grid ends with zero gradient.
 */
#ifndef RXMET_QDQ_H_
#define RXMET_QDQ_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  RXMET_QDQ_LEARNABLE = 0,
  RXMET_QDQ_FROZEN = 1,
};

/* Message of the last failing call on this thread ("" if none). */
const char *rxmet_last_error(void);

/* Library/ABI version, for loaders that check compatibility. */
int rxmet_abi_version(void);

/* Bytes of workspace the reductions below need for this layout. */
int64_t rxmet_qdq_workspace_bytes(int64_t outer, int64_t C, int64_t inner);

/*
 * Per-encoding min and max of x (NaN propagates, like torch.min/torch.max).
 * Replaces _MinMaxObserver.collect_stats
 * (src/aimet_torch/v2/quantization/encoding_analyzer.py:101-105) and the
 * permute/reshape/reduce it goes through (src/aimet_torch/v2/utils.py:69-89).
 * out_min/out_max: [C] fp32.
 */
int rxmet_qdq_minmax(const float *x, int64_t outer, int64_t C, int64_t inner,
                     float *out_min, float *out_max, void *workspace, void *stream);

/*
 * Fake-quantize forward.  y may alias x.  scale/offset: [C] fp32.
 * Replaces QuantDequantFunc.forward (torch_builtins.py:640-672) for
 * mode = RXMET_QDQ_LEARNABLE and _torch_fake_quantize (torch_builtins.py:287-361)
 * for mode = RXMET_QDQ_FROZEN.
 */
int rxmet_qdq_forward(const float *x, float *y, int64_t outer, int64_t C, int64_t inner,
                      const float *scale, const float *offset, int64_t qmin, int64_t qmax,
                      int mode, void *stream);

/*
 * Fused fake-quantize backward: dx = g * mask, and (when dscale/doffset are non-null)
 * the encoding gradients already reduced over the broadcast dimensions to [C]:
 *   dscale[c]  = sum g * (clamp(rint(x/s), o+qmin, o+qmax) - (x/s) * mask)
 *   doffset[c] = sum g * (!mask * s)
 * Replaces QuantDequantFunc.backward (torch_builtins.py:675-691) plus autograd's
 * broadcast reduction of its scale/offset gradients.  The mask is recomputed from x
 * exactly as the forward computes it.  Sums are accumulated in fp64 and reduced in a
 * fixed order (deterministic).  dx may alias g.
 */
int rxmet_qdq_backward(const float *x, const float *g, float *dx, float *dscale,
                       float *doffset, int64_t outer, int64_t C, int64_t inner,
                       const float *scale, const float *offset, int64_t qmin, int64_t qmax,
                       int mode, void *workspace, void *stream);

/*
 * Size of the device scratch array rxmet_qdq_backward_noalloc works in (4 MiB: the
 * encoding-gradient partials of tensors up to about 2^31 elements in the per-tensor case).
 */
#define RXMET_QDQ_NOALLOC_SCRATCH_BYTES (4LL << 20)

/*
 * rxmet_qdq_backward without a workspace argument and without any device allocation: the
 * partial sums of the encoding gradients live in a 4 MiB file-scope device array
 * (RXMET_QDQ_NOALLOC_SCRATCH_BYTES), one per GPU, held until the process ends.  No
 * counterpart in the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments, kernels and results as rxmet_qdq_backward (bit for bit).
 * Limits: a layout whose partials need more than the scratch (rxmet_qdq_workspace_bytes >
 * RXMET_QDQ_NOALLOC_SCRATCH_BYTES) is rejected with -22 and a message; calls that overlap on
 * one GPU (different streams, or host threads) share the array and race; the stream must
 * belong to the current device.  Nothing in the array needs clearing between calls.  (The
 * library's optional kernel timing, off unless rxmet_prof_enable turns it on, creates hipEvents;
 * with it off this call makes no allocating call at all.)
 */
int rxmet_qdq_backward_noalloc(const float *x, const float *g, float *dx, float *dscale,
                               float *doffset, int64_t outer, int64_t C, int64_t inner,
                               const float *scale, const float *offset, int64_t qmin,
                               int64_t qmax, int mode, void *stream);

/*
 * Quantize forward: q = clamp(rint(x / s) - o, qmin, qmax) (codes as fp32).
 * Replaces QuantizeFunc.forward (torch_builtins.py:527-552).
 */
int rxmet_quantize_forward(const float *x, float *q, int64_t outer, int64_t C,
                           int64_t inner, const float *scale, const float *offset,
                           int64_t qmin, int64_t qmax, void *stream);

/*
 * Quantize backward (QuantizeFunc.backward, torch_builtins.py:555-571):
 *   dx = g*mask/s, dscale[c] = sum -(g*mask/s)*(x/s), doffset[c] = sum -g*mask.
 */
int rxmet_quantize_backward(const float *x, const float *g, float *dx, float *dscale,
                            float *doffset, int64_t outer, int64_t C, int64_t inner,
                            const float *scale, const float *offset, int64_t qmin,
                            int64_t qmax, void *workspace, void *stream);

/*
 * Dequantize forward: y = (q + o) * s  (DequantizeFunc.forward, torch_builtins.py:589-603).
 */
int rxmet_dequantize_forward(const float *q, float *y, int64_t outer, int64_t C,
                             int64_t inner, const float *scale, const float *offset,
                             void *stream);

/*
 * Dequantize backward (DequantizeFunc.backward, torch_builtins.py:607-615):
 *   dq = g*s, dscale[c] = sum g*(q+o), doffset[c] = sum g*s.
 */
int rxmet_dequantize_backward(const float *q, const float *g, float *dq, float *dscale,
                              float *doffset, int64_t outer, int64_t C, int64_t inner,
                              const float *scale, const float *offset, void *workspace,
                              void *stream);

/*
 * Encodings of learnable min/max (QuantizeDequantize.get_scale / _get_offset,
 * quantizer.py:345-464), n encodings in one launch instead of the reference's chain of
 * one-element tensor operations:
 *   scale  = max(|(max - min) * fl(1 / (qmax - qmin))|, min_scale),
 *   offset = symmetric ? sym_offset : clamp(round_half_even(min / scale) - qmin, -qmax, -qmin),
 * the float operations PyTorch performs for the reference's tensor expressions on the GPU (a
 * tensor divided by a scalar is a product with the scalar's rounded reciprocal there).
 */
int rxmet_qdq_encoding_forward(const float *mn, const float *mx, int64_t n, int64_t qmin,
                               int64_t qmax, int32_t symmetric, float sym_offset,
                               float min_scale, float *scale, float *offset, void *stream);

/*
 * Gradients of the above with respect to min and max, given those of scale (g_scale) and of
 * offset (g_offset, ignored when symmetric; either may be null = zero), with the
 * reference's autograd rules: straight-through rounding, clamp and clamp_min pass the
 * gradient inside their range (bounds included), |x|' = sign(x).
 */
int rxmet_qdq_encoding_backward(const float *mn, const float *mx, const float *g_scale,
                                const float *g_offset, int64_t n, int64_t qmin, int64_t qmax,
                                int32_t symmetric, float min_scale, float *d_min, float *d_max,
                                void *stream);

#ifdef __cplusplus
}
#endif

#endif /* RXMET_QDQ_H_ */
