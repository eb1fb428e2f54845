// Tuned paged decode kernels: the entry points the dispatcher (decode.hip)
// picks from.  Each pool type's instantiations live in their own translation
// unit (decode_tuned_f32.hip, _f16, _bf16) so that they compile in parallel.
#pragma once

#include "attn_common.h"

namespace llkv {

typedef void (*DecodeFn)(DecodeArgs);

// The schedules of one MFMA body: fixed split and balanced (kDecodeWaves
// waves per work-group), and unit: the fixed-split kernel with kUnitWaves
// waves per work-group, launched with one split (no partials, no merge) for
// small batches of short sequences.
struct Kernels {
    DecodeFn split = nullptr;
    DecodeFn balanced = nullptr;
    DecodeFn unit = nullptr;
};

// Tuned kernels for head_dim D and G query heads per kv head, plain or with
// the fused append of the step's new row; both null when the shape has no
// tuned body (the dispatcher then runs the generic kernel).  Tuned: D 64 or
// 128 with G in {1, 2, 3, 4, 5, 6, 7, 8, 12, 16}; D 96 or 256 with G in {1, 2, 4, 8}.
Kernels tuned_kernels_f32(int D, int G, bool append);
Kernels tuned_kernels_f16(int D, int G, bool append);
Kernels tuned_kernels_bf16(int D, int G, bool append);

}  // namespace llkv
