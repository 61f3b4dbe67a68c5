// q38_moe_grp.hip — dispatch of the grouped-scale (VALU) expert projections by codebook
// geometry; the kernels are instantiated per dimension in q38_moe_grp{8,4,2}.hip.
#include "q38_moe_grp.hpp"

namespace q38 {

hipError_t launch_grouped_d8(const LayerDev& L, const MoeBufs& B, int M, bool down, hipStream_t st);
hipError_t launch_grouped_d4(const LayerDev& L, const MoeBufs& B, int M, bool down, hipStream_t st);
hipError_t launch_grouped_d2(const LayerDev& L, const MoeBufs& B, int M, bool down, hipStream_t st);

static hipError_t launch_grouped(const LayerDev& L, const MoeBufs& B, int M, bool down, hipStream_t st) {
    const ProjDev& P = L.p[down ? 2 : 0];
    if (P.dim == 8 && P.bits == 14) return launch_grouped_d8(L, B, M, down, st);
    if (P.dim == 4 && P.bits == 8) return launch_grouped_d4(L, B, M, down, st);
    if (P.dim == 2 && P.bits == 8) return launch_grouped_d2(L, B, M, down, st);
    return hipErrorInvalidValue;
}

// Prefill widths on these kernels: the uniform layouts they take (d8/14, d4/8, d2/8 with
// row or group scales, fp16 or INT8 books), the plan sort's expert count, and 16 staged
// rows of H in LDS.
bool moe_supports_grouped_prefill(const LayerDev& L) {
    if (L.mixed || L.E > 1024) return false;
    for (int p = 0; p < 3; ++p) {
        const ProjDev& P = L.p[p];
        const bool geo = (P.dim == 8 && P.bits == 14) || (P.dim == 4 && P.bits == 8) || (P.dim == 2 && P.bits == 8);
        if (!geo || !(P.book || P.book_i8)) return false;
    }
    return static_cast<size_t>(kMaxRows) * fin_stride(L.H) * sizeof(fin_t) <= kFinLdsMax &&
           L.I % kGuRowsPerBlock == 0 && L.H % kDownRowsPerBlock == 0;
}

hipError_t launch_gate_up_grouped(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st) {
    return launch_grouped(L, B, M, false, st);
}
hipError_t launch_down_grouped(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st) {
    return launch_grouped(L, B, M, true, st);
}

} // namespace q38
