// Instantiations of the single-launch MoE decode kernel (moe_fused.hpp) for
// bf16 activations (4-bit rows as packed bf16 dot products).
#include "moe_fused.hpp"

namespace swq {

FusedKernel fused_select_bf16(int gfmt, bool rc2, int M) {
    if (gfmt == kFusedQ4) return rc2 ? fused_by_m<SWQ_BF16, 4, 2, kXBF16, 4, 2, false>(M) : fused_by_m<SWQ_BF16, 4, 2, kXBF16, 4, 1, false>(M);
    if (gfmt == kFusedQ8C2) return rc2 ? fused_by_m<SWQ_BF16, 8, 2, kXF32, 8, 2, false>(M) : fused_by_m<SWQ_BF16, 8, 2, kXF32, 8, 1, false>(M);
    if (gfmt == kFusedQ8C1) return rc2 ? fused_by_m<SWQ_BF16, 8, 1, kXF32, 8, 2, false>(M) : fused_by_m<SWQ_BF16, 8, 1, kXF32, 8, 1, false>(M);
    return nullptr;
}

}  // namespace swq

#ifdef SWQ_FUSED_TRACE
SWQ_TRACE_ACCESSOR(swq_fused_trace_bf16)
#endif
