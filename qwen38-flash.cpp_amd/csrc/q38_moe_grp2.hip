// The grouped-scale kernels (q38_moe_grp.hpp) for 2-dimensional codebooks with 8-bit codes.
#include "q38_moe_grp.hpp"

namespace q38 {

hipError_t launch_grouped_d2(const LayerDev& L, const MoeBufs& B, int M, bool down, hipStream_t st) {
    if (!down) {
        const int lpr = next_pow2((L.H / 2 + 15) / 16);
        if (lpr == 64) return launch_gu_grouped_g<2, 8, 64>(L, B, M, st);
        if (lpr == 32) return launch_gu_grouped_g<2, 8, 32>(L, B, M, st);
        if (lpr <= 16) return launch_gu_grouped_g<2, 8, 16>(L, B, M, st);
        return hipErrorInvalidValue;
    }
    const int lpr = next_pow2((L.I / 2 + 15) / 16);
    if (lpr == 16) return launch_down_grouped_g<2, 8, 16>(L, B, M, st);
    if (lpr == 32) return launch_down_grouped_g<2, 8, 32>(L, B, M, st);
    if (lpr <= 8) return launch_down_grouped_g<2, 8, 8>(L, B, M, st);
    return hipErrorInvalidValue;
}

} // namespace q38
