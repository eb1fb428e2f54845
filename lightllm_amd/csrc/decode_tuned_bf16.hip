// Tuned paged decode instantiations for bf16_t pools.
#include "decode_sched.h"

namespace llkv {
Kernels tuned_kernels_bf16(int D, int G, bool append) { return tuned<bf16_t>(D, G, append); }
}  // namespace llkv
