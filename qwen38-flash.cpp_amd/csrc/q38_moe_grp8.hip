// The grouped-scale kernels (q38_moe_grp.hpp) for 8-dimensional codebooks with 14-bit codes.
#include "q38_moe_grp.hpp"

namespace q38 {

hipError_t launch_grouped_d8(const LayerDev& L, const MoeBufs& B, int M, bool down, hipStream_t st) {
    if (!down) {
        const int lpr = next_pow2((L.H / 8 + 15) / 16);
        if (lpr == 16) return launch_gu_grouped_g<8, 14, 16>(L, B, M, st);
        if (lpr == 32) return launch_gu_grouped_g<8, 14, 32>(L, B, M, st);
        if (lpr == 8) return launch_gu_grouped_g<8, 14, 8>(L, B, M, st);
        if (lpr <= 4) return launch_gu_grouped_g<8, 14, 4>(L, B, M, st);
        return hipErrorInvalidValue;
    }
    const int lpr = next_pow2((L.I / 8 + 15) / 16);
    if (lpr == 4) return launch_down_grouped_g<8, 14, 4>(L, B, M, st);
    if (lpr == 8) return launch_down_grouped_g<8, 14, 8>(L, B, M, st);
    if (lpr <= 2) return launch_down_grouped_g<8, 14, 2>(L, B, M, st);
    return hipErrorInvalidValue;
}

} // namespace q38
