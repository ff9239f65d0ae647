// qdq_f32.hip — the fake-quantization kernels instantiated for f32 tensors (every op and
// internal type that pairs with f32); the entry points in qdq.hip dispatch here.
#include "qdq_kernels.h"

namespace rxmet {
namespace qdq {

int run_f32(const Call &c, int what) { return run_typed<float>(c, what); }

}  // namespace qdq
}  // namespace rxmet
