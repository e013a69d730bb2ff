// Instantiations of the single-launch MoE decode kernel (moe_fused.hpp) for
// f32 activations and 2 or 4 tokens (token-major slots).
#include "moe_fused_batch.hpp"

namespace swq {

FusedKernel fused_select_f32_batch(int gfmt, bool rc2, int M) {
    if (gfmt == kFusedQ4) return rc2 ? fused_batch_by_m<SWQ_F32, 4, 1, kXF32, 4, 2>(M) : fused_batch_by_m<SWQ_F32, 4, 1, kXF32, 4, 1>(M);
    if (gfmt == kFusedQ8C2) return rc2 ? fused_batch_by_m<SWQ_F32, 8, 2, kXF32, 8, 2>(M) : fused_batch_by_m<SWQ_F32, 8, 2, kXF32, 8, 1>(M);
    if (gfmt == kFusedQ8C1) return rc2 ? fused_batch_by_m<SWQ_F32, 8, 1, kXF32, 8, 2>(M) : fused_batch_by_m<SWQ_F32, 8, 1, kXF32, 8, 1>(M);
    return nullptr;
}

}  // namespace swq
