// The grouped-scale kernels (q38_moe_grp.hpp) for 4-dimensional codebooks with 8-bit codes.
#include "q38_moe_grp.hpp"

namespace q38 {

hipError_t launch_grouped_d4(const LayerDev& L, const MoeBufs& B, int M, bool down, hipStream_t st) {
    if (!down) {
        const int lpr = next_pow2((L.H / 4 + 15) / 16);
        if (lpr == 32) return launch_gu_grouped_g<4, 8, 32>(L, B, M, st);
        if (lpr == 64) return launch_gu_grouped_g<4, 8, 64>(L, B, M, st);
        if (lpr == 16) return launch_gu_grouped_g<4, 8, 16>(L, B, M, st);
        if (lpr <= 8) return launch_gu_grouped_g<4, 8, 8>(L, B, M, st);
        return hipErrorInvalidValue;
    }
    const int lpr = next_pow2((L.I / 4 + 15) / 16);
    if (lpr == 8) return launch_down_grouped_g<4, 8, 8>(L, B, M, st);
    if (lpr == 16) return launch_down_grouped_g<4, 8, 16>(L, B, M, st);
    if (lpr == 4) return launch_down_grouped_g<4, 8, 4>(L, B, M, st);
    if (lpr <= 2) return launch_down_grouped_g<4, 8, 2>(L, B, M, st);
    return hipErrorInvalidValue;
}

} // namespace q38
