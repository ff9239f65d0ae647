// qdq_f16.hip — the fake-quantization kernels instantiated for f16 tensors (every op and
// internal type that pairs with f16); the entry points in qdq.hip dispatch here.
#include "qdq_kernels.h"

namespace rxmet {
namespace qdq {

int run_f16(const Call &c, int what) { return run_typed<half_t>(c, what); }

}  // namespace qdq
}  // namespace rxmet
