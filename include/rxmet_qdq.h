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

/* ---------------------------------------------------------------------------------------
 * General entry points: fp16 / bf16 tensors, the reference's internal arithmetic type,
 * zero_point_shift, and encodings over two separated groups of axes.
 * ------------------------------------------------------------------------------------- */

/* Element types (tensors and internal arithmetic; an F64 tensor computes in F64). */
enum {
  RXMET_QDQ_F32 = 0,
  RXMET_QDQ_F16 = 1,
  RXMET_QDQ_BF16 = 2,
  RXMET_QDQ_F64 = 3,
};

/*
 * Tensor layout [outer, C0, mid, C1, inner] (row-major): element (o, c0, m, c1, k) uses
 * encoding c0 * C1 + c1, so scale/offset hold C0 * C1 values.  The three-argument layout
 * [outer, C, inner] above is {1, 1, outer, C, inner}.  Two separated encoding groups cover
 * per-channel encodings on two non-adjacent axes and two-dimensional block quantization
 * (torch_builtins.py:694-754 reshapes a [R, Cc] tensor with block sizes (br, bc) to
 * [R/br, br, Cc/bc, bc] with encodings [R/br, 1, Cc/bc, 1]: {1, R/br, br, Cc/bc, bc}).
 */
typedef struct rxmet_qdq_layout {
  int64_t outer, C0, mid, C1, inner;
} rxmet_qdq_layout;

/*
 * Arithmetic of one call, as the reference's backend evaluates it:
 *   io_dtype        element type of x, y, g and dx (F32, F16, BF16 or F64; F64 pairs with
 *                   internal_dtype F64 only, the reference's internal type for an fp64
 *                   tensor);
 *   internal_dtype  type QuantizeFunc / QuantDequantFunc compute in (io_dtype, F32 or F64:
 *                   torch_builtins.py:171-174, 255-262 widen it while the grid is not
 *                   numerically stable in the narrower type); every operation's result is
 *                   rounded to it, and the result to io_dtype.  Dequantize computes in
 *                   io_dtype (internal_dtype must equal it); the frozen mode computes as
 *                   torch.fake_quantize does, in fp32, whatever the io type (an F64 tensor's
 *                   x * (1 / scale) and its rounding in fp64, as aten's kernel promotes it).
 *                   Min / max statistics of an F64 tensor are fp32 (each value rounded).
 *   zero_point_shift  quantize_dequantize only (learnable mode): y = qdq(x - shift * s) +
 *                   shift * s (torch_builtins.py:276-284); 0 for none.
 *   scalar_scale    the reference's scale is a 0-dim tensor.  PyTorch then evaluates binary
 *                   operations between the input tensor and the scale in the input's type
 *                   (the scale rounded to it first): the shift's subtraction and
 *                   QuantizeFunc.backward's tensor / scale.  Only matters when
 *                   internal_dtype is wider than io_dtype.
 * scale and offset always arrive as fp32 arrays holding the internal-type values
 * (scale.to(internal) of the reference; with an F64 internal type the values must be exact
 * in fp32, which fp32/fp16/bf16 parameters are).
 */
typedef struct rxmet_qdq_numerics {
  int32_t io_dtype;
  int32_t internal_dtype;
  double zero_point_shift;
  int32_t scalar_scale;
  int32_t reserved; /* 0 */
} rxmet_qdq_numerics;

/* Workspace bytes of the _ex reductions for this layout and io type. */
int64_t rxmet_qdq_workspace_bytes_ex(const rxmet_qdq_layout *layout, int32_t io_dtype);

/* rxmet_qdq_minmax for any io type and layout; out_min/out_max: [C0 * C1] fp32 (exact). */
int rxmet_qdq_minmax_ex(const void *x, int32_t io_dtype, const rxmet_qdq_layout *layout,
                        float *out_min, float *out_max, void *workspace, void *stream);

/*
 * quantize_dequantize forward / backward (torch_builtins.py:199-284 with QuantDequantFunc
 * :618-691, or the frozen fast path :221-249 + :287-361).  Gradients of the shift's own
 * terms are included: dscale[c] gains shift * sum g * (1 - mask).  dscale / doffset come back
 * rounded to the internal type (stored as fp32).
 */
int rxmet_qdq_forward_ex(const void *x, void *y, const rxmet_qdq_layout *layout,
                         const rxmet_qdq_numerics *numerics, const float *scale,
                         const float *offset, int64_t qmin, int64_t qmax, int mode,
                         void *stream);
int rxmet_qdq_backward_ex(const void *x, const void *g, void *dx, float *dscale, float *doffset,
                          const rxmet_qdq_layout *layout, const rxmet_qdq_numerics *numerics,
                          const float *scale, const float *offset, int64_t qmin, int64_t qmax,
                          int mode, void *workspace, void *stream);

/* quantize forward / backward (torch_builtins.py:151-194 with QuantizeFunc :505-571); q in
 * io_dtype (the grid must be exact in it). */
int rxmet_quantize_forward_ex(const void *x, void *q, const rxmet_qdq_layout *layout,
                              const rxmet_qdq_numerics *numerics, const float *scale,
                              const float *offset, int64_t qmin, int64_t qmax, void *stream);
int rxmet_quantize_backward_ex(const void *x, const void *g, void *dx, float *dscale,
                               float *doffset, const rxmet_qdq_layout *layout,
                               const rxmet_qdq_numerics *numerics, const float *scale,
                               const float *offset, int64_t qmin, int64_t qmax,
                               void *workspace, void *stream);

/*
 * QuantizeDequantize.forward with learnable min / max (quantizer.py:1048-1082: get_encodings()
 * then the backend's quantize_dequantize, learnable mode) in one launch each way: the kernels
 * derive every encoding's scale and offset from min and max as rxmet_qdq_encoding_forward does
 * (then take them to the internal type), so no scale / offset tensors are made; the backward
 * folds the encoding gradients straight on to min and max (rxmet_qdq_encoding_backward's rules
 * applied to the folded, internal-type-rounded gradients of scale and offset).  y, dx, d_min
 * and d_max equal those of rxmet_qdq_encoding_forward + rxmet_qdq_forward_ex and
 * rxmet_qdq_backward_ex + rxmet_qdq_encoding_backward bit for bit.  min / max: [C0 * C1] fp32;
 * d_min / d_max: both or neither (then dx only, no workspace needed).
 */
typedef struct rxmet_qdq_minmax_enc {
  const float *min, *max;
  int32_t symmetric;  /* offset = sym_offset, else derived from min */
  float sym_offset;
  float min_scale;    /* lower clamp of the scale (quantsim's minimum scale) */
  int32_t reserved;   /* 0 */
} rxmet_qdq_minmax_enc;

int rxmet_qdq_forward_minmax(const void *x, void *y, const rxmet_qdq_layout *layout,
                             const rxmet_qdq_numerics *numerics, const rxmet_qdq_minmax_enc *enc,
                             int64_t qmin, int64_t qmax, void *stream);
int rxmet_qdq_backward_minmax(const void *x, const void *g, void *dx, float *d_min,
                              float *d_max, const rxmet_qdq_layout *layout,
                              const rxmet_qdq_numerics *numerics, const rxmet_qdq_minmax_enc *enc,
                              int64_t qmin, int64_t qmax, void *workspace, void *stream);

/* dequantize forward / backward (torch_builtins.py:459-488 with DequantizeFunc :574-615). */
int rxmet_dequantize_forward_ex(const void *q, void *y, const rxmet_qdq_layout *layout,
                                const rxmet_qdq_numerics *numerics, const float *scale,
                                const float *offset, void *stream);
int rxmet_dequantize_backward_ex(const void *q, const void *g, void *dq, float *dscale,
                                 float *doffset, const rxmet_qdq_layout *layout,
                                 const rxmet_qdq_numerics *numerics, const float *scale,
                                 const float *offset, void *workspace, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* RXMET_QDQ_H_ */
