// Tuned paged decode instantiations for _Float16 pools.
#include "decode_sched.h"

namespace llkv {
Kernels tuned_kernels_f16(int D, int G, bool append) { return tuned<_Float16>(D, G, append); }
}  // namespace llkv
