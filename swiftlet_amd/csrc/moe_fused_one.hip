// Instantiations of the one-expert single launch (moe_fused_one.hpp) for bf16
// and f32 activations, in the gate/up formats of moe_fused.
#include "moe_fused_one.hpp"

namespace swq {

FusedKernel fused_select_one(int x_dtype, int gfmt, bool rc2) {
    if (x_dtype == SWQ_BF16) {
        if (gfmt == kFusedQ4) return rc2 ? moe_fused_one<SWQ_BF16, 4, 2, kXBF16, gate_passes(4, 2), 4, 2> : moe_fused_one<SWQ_BF16, 4, 2, kXBF16, gate_passes(4, 2), 4, 1>;
        if (gfmt == kFusedQ8C2) return rc2 ? moe_fused_one<SWQ_BF16, 8, 2, kXF32, gate_passes(8, 2), 8, 2> : moe_fused_one<SWQ_BF16, 8, 2, kXF32, gate_passes(8, 2), 8, 1>;
        if (gfmt == kFusedQ8C1) return rc2 ? moe_fused_one<SWQ_BF16, 8, 1, kXF32, gate_passes(8, 1), 8, 2> : moe_fused_one<SWQ_BF16, 8, 1, kXF32, gate_passes(8, 1), 8, 1>;
    } else if (x_dtype == SWQ_F32) {
        if (gfmt == kFusedQ4) return rc2 ? moe_fused_one<SWQ_F32, 4, 1, kXF32, gate_passes(4, 1), 4, 2> : moe_fused_one<SWQ_F32, 4, 1, kXF32, gate_passes(4, 1), 4, 1>;
        if (gfmt == kFusedQ8C2) return rc2 ? moe_fused_one<SWQ_F32, 8, 2, kXF32, gate_passes(8, 2), 8, 2> : moe_fused_one<SWQ_F32, 8, 2, kXF32, gate_passes(8, 2), 8, 1>;
        if (gfmt == kFusedQ8C1) return rc2 ? moe_fused_one<SWQ_F32, 8, 1, kXF32, gate_passes(8, 1), 8, 2> : moe_fused_one<SWQ_F32, 8, 1, kXF32, gate_passes(8, 1), 8, 1>;
    }
    return nullptr;
}

}  // namespace swq

#ifdef SWQ_FUSED_TRACE
SWQ_TRACE_ACCESSOR(swq_fused_trace_one)
#endif
