// Instantiations of the single-launch MoE decode kernel (moe_fused.hpp) for
// f32 activations.
#include "moe_fused.hpp"

namespace swq {

FusedKernel fused_select_f32(int gfmt, bool rc2, int M) {
    if (gfmt == kFusedQ4) return rc2 ? fused_by_m<SWQ_F32, 4, 1, kXF32, 4, 2, false>(M) : fused_by_m<SWQ_F32, 4, 1, kXF32, 4, 1, false>(M);
    if (gfmt == kFusedQ8C2) return rc2 ? fused_by_m<SWQ_F32, 8, 2, kXF32, 8, 2, false>(M) : fused_by_m<SWQ_F32, 8, 2, kXF32, 8, 1, false>(M);
    if (gfmt == kFusedQ8C1) return rc2 ? fused_by_m<SWQ_F32, 8, 1, kXF32, 8, 2, false>(M) : fused_by_m<SWQ_F32, 8, 1, kXF32, 8, 1, false>(M);
    return nullptr;
}

}  // namespace swq
