// qdq_bf16.hip — the fake-quantization kernels instantiated for bf16 tensors (every op and
// internal type that pairs with bf16); the entry points in qdq.hip dispatch here.
#include "qdq_kernels.h"

namespace rxmet {
namespace qdq {

int run_bf16(const Call &c, int what) { return run_typed<bf16_t>(c, what); }

}  // namespace qdq
}  // namespace rxmet
