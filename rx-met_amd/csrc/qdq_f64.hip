// qdq_f64.hip — the fake-quantization kernels instantiated for f64 tensors (arithmetic in
// fp64, the frozen path in torch's fake_quantize arithmetic); the entry points in qdq.hip
// dispatch here.
#include "qdq_kernels.h"

namespace rxmet {
namespace qdq {

int run_f64(const Call &c, int what) { return run_typed<double>(c, what); }

}  // namespace qdq
}  // namespace rxmet
