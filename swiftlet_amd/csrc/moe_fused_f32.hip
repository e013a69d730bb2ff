// Instantiations of the single-launch MoE decode kernel (moe_fused.hpp) for
// f32 activations.
#include "moe_fused.hpp"

namespace swq {

FusedKernel fused_select_f32(int gfmt, bool rc2, int M, int wpc) {
    if (gfmt == kFusedQ4) return rc2 ? fused_by_m<SWQ_F32, 4, 1, kXF32, 4, 2, false>(M, wpc) : fused_by_m<SWQ_F32, 4, 1, kXF32, 4, 1, false>(M, wpc);
    if (gfmt == kFusedQ8C2) return rc2 ? fused_by_m<SWQ_F32, 8, 2, kXF32, 8, 2, false>(M, wpc) : fused_by_m<SWQ_F32, 8, 2, kXF32, 8, 1, false>(M, wpc);
    if (gfmt == kFusedQ8C1) return rc2 ? fused_by_m<SWQ_F32, 8, 1, kXF32, 8, 2, false>(M, wpc) : fused_by_m<SWQ_F32, 8, 1, kXF32, 8, 1, false>(M, wpc);
    return nullptr;
}

}  // namespace swq
