// Tuned paged decode instantiations for float pools.
#include "decode_sched.h"

namespace llkv {
Kernels tuned_kernels_f32(int D, int G, bool append) { return tuned<float>(D, G, append); }
}  // namespace llkv
