// Instantiations of the single-launch MoE decode kernel (moe_fused.hpp) for
// bf16 activations and 2 or 4 tokens (token-major slots).
#include "moe_fused_batch.hpp"

namespace swq {

FusedKernel fused_select_bf16_batch(int gfmt, bool rc2, int M) {
    if (gfmt == kFusedQ4) return rc2 ? fused_batch_by_m<SWQ_BF16, 4, 2, kXBF16, 4, 2>(M) : fused_batch_by_m<SWQ_BF16, 4, 2, kXBF16, 4, 1>(M);
    if (gfmt == kFusedQ8C2) return rc2 ? fused_batch_by_m<SWQ_BF16, 8, 2, kXF32, 8, 2>(M) : fused_batch_by_m<SWQ_BF16, 8, 2, kXF32, 8, 1>(M);
    if (gfmt == kFusedQ8C1) return rc2 ? fused_batch_by_m<SWQ_BF16, 8, 1, kXF32, 8, 2>(M) : fused_batch_by_m<SWQ_BF16, 8, 1, kXF32, 8, 1>(M);
    return nullptr;
}

}  // namespace swq

#ifdef SWQ_FUSED_TRACE
SWQ_TRACE_ACCESSOR(swq_fused_trace_bf16_batch)
#endif
