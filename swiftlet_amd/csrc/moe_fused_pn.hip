// Instantiations of the single-launch MoE decode kernel (moe_fused.hpp) for
// the post-attention RMSNorm folded in (f32 activations normalised into LDS).
#include "moe_fused.hpp"

namespace swq {

FusedKernel fused_select_pn(int gfmt, bool rc2, int M) {
    if (gfmt == kFusedQ4) return rc2 ? fused_by_m<SWQ_F32, 4, 1, kXF32, 4, 2, true>(M) : fused_by_m<SWQ_F32, 4, 1, kXF32, 4, 1, true>(M);
    if (gfmt == kFusedQ8C2) return rc2 ? fused_by_m<SWQ_F32, 8, 2, kXF32, 8, 2, true>(M) : fused_by_m<SWQ_F32, 8, 2, kXF32, 8, 1, true>(M);
    if (gfmt == kFusedQ8C1) return rc2 ? fused_by_m<SWQ_F32, 8, 1, kXF32, 8, 2, true>(M) : fused_by_m<SWQ_F32, 8, 1, kXF32, 8, 1, true>(M);
    return nullptr;
}

}  // namespace swq
