// q38_affine.hip — the shared expert in MLX affine form (R10 in the layout of the reference's
// checkpoints: the affine branch of SparseMoe::load_projection, src/sparse_moe.cpp:474-480,
// 662-700, applied by SparseMoe::forward_shared, :1306-1313, through quantized_matmul).
//
// Two launches per layer call, before the routed experts' kernels (the row dot products of
// q38_affine.hpp):
//   k_sa_gu  gate and up rows of the shared expert for the call's rows, SwiGLU with the
//            reference's rounding points, into the workspace's SwiGLU rows (bf16-exact values);
//   k_sa_dn  the down projection of those rows into the shared expert's down-output rows of
//            the partial-sum planes (value in plane 0, 0 in plane 1), which the combine reads
//            as it reads a VQ shared expert's.
#include "q38_affine.hpp"

namespace q38 {
namespace {

// Gate and up rows o of the shared expert, SwiGLU: hs[r][o] (bf16) for the workgroup's rows.
template <int BITS, int LPR>
__global__ __launch_bounds__(kSaThreads) void k_sa_gu(LayerDev L, MoeBufs B, int M) {
    extern __shared__ __align__(16) uint16_t xs[];  // [kSaRows][H]
    const int H = L.H, Is = L.sa_inter;
    const int r0 = blockIdx.y * kSaRows, nr = M - r0 < kSaRows ? M - r0 : kSaRows;
    sa_stage(B.x, H, r0, nr, xs);
    __syncthreads();
    constexpr int OPW = 64 / LPR;  // weight rows per wave
    const int o = (blockIdx.x * (kSaThreads / 64) + (threadIdx.x >> 6)) * OPW + (threadIdx.x & 63) / LPR;
    if (o >= Is) return;
    const int wpr = H * BITS / 32, ngrp = H / L.sa_group;
    float g[kSaRows], u[kSaRows];
    sa_row_dot<BITS, LPR>(L.sa[0].w + static_cast<size_t>(o) * wpr, L.sa[0].s + static_cast<size_t>(o) * ngrp,
                          L.sa[0].b + static_cast<size_t>(o) * ngrp, H, L.sa_group, L.sa_f16, xs, nr, g);
    sa_row_dot<BITS, LPR>(L.sa[1].w + static_cast<size_t>(o) * wpr, L.sa[1].s + static_cast<size_t>(o) * ngrp,
                          L.sa[1].b + static_cast<size_t>(o) * ngrp, H, L.sa_group, L.sa_f16, xs, nr, u);
    if ((threadIdx.x & 63) % LPR == 0)
#pragma unroll
        for (int r = 0; r < kSaRows; ++r)
            if (r < nr) B.h16[static_cast<size_t>(r0 + r) * Is + o] = f2bf(swiglu(g[r], u[r]));
}

// Down rows o of the shared expert over the SwiGLU rows: the shared expert's rows of the down
// partial-sum planes, d[M*K + r][o] (plane 0; plane 1 gets 0).
template <int BITS, int LPR>
__global__ __launch_bounds__(kSaThreads) void k_sa_dn(LayerDev L, MoeBufs B, int M) {
    extern __shared__ __align__(16) uint16_t xs[];  // [kSaRows][Is]
    const int H = L.H, Is = L.sa_inter;
    const int r0 = blockIdx.y * kSaRows, nr = M - r0 < kSaRows ? M - r0 : kSaRows;
    sa_stage(B.h16, Is, r0, nr, xs);
    __syncthreads();
    constexpr int OPW = 64 / LPR;
    const int o = (blockIdx.x * (kSaThreads / 64) + (threadIdx.x >> 6)) * OPW + (threadIdx.x & 63) / LPR;
    if (o >= H) return;
    const int wpr = Is * BITS / 32, ngrp = Is / L.sa_group;
    float d[kSaRows];
    sa_row_dot<BITS, LPR>(L.sa[2].w + static_cast<size_t>(o) * wpr, L.sa[2].s + static_cast<size_t>(o) * ngrp,
                          L.sa[2].b + static_cast<size_t>(o) * ngrp, Is, L.sa_group, L.sa_f16, xs, nr, d);
    const int MK = M * L.K;
    if ((threadIdx.x & 63) % LPR == 0)
#pragma unroll
        for (int r = 0; r < kSaRows; ++r)
            if (r < nr) {
                const size_t at = static_cast<size_t>(MK + r0 + r) * H + o;
                B.d[at] = d[r];
                B.d[B.d_plane + at] = 0.0f;
            }
}

template <int BITS, int LPR>
hipError_t launch_sa_gu_t(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st) {
    const size_t lds = static_cast<size_t>(kSaRows) * L.H * 2;
    if (const hipError_t e = ensure_lds<k_sa_gu<BITS, LPR>>(lds); e != hipSuccess) return e;
    constexpr int OPB = kSaThreads / 64 * (64 / LPR);
    return launch(k_sa_gu<BITS, LPR>, dim3((L.sa_inter + OPB - 1) / OPB, (M + kSaRows - 1) / kSaRows),
                  dim3(kSaThreads), lds, st, L, B, M);
}
template <int BITS, int LPR>
hipError_t launch_sa_dn_t(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st) {
    const size_t lds = static_cast<size_t>(kSaRows) * L.sa_inter * 2;
    if (const hipError_t e = ensure_lds<k_sa_dn<BITS, LPR>>(lds); e != hipSuccess) return e;
    constexpr int OPB = kSaThreads / 64 * (64 / LPR);
    return launch(k_sa_dn<BITS, LPR>, dim3((L.H + OPB - 1) / OPB, (M + kSaRows - 1) / kSaRows), dim3(kSaThreads), lds,
                  st, L, B, M);
}
// Lanes per weight row: the row's 32-input chunks over at most 64 lanes.
template <int BITS>
hipError_t launch_sa(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st) {
    const int cg = L.H / 32, cd = L.sa_inter / 32;
    hipError_t e = cg >= 64 ? launch_sa_gu_t<BITS, 64>(L, B, M, st)
                   : cg >= 32 ? launch_sa_gu_t<BITS, 32>(L, B, M, st)
                              : launch_sa_gu_t<BITS, 16>(L, B, M, st);
    if (e != hipSuccess) return e;
    return cd >= 64 ? launch_sa_dn_t<BITS, 64>(L, B, M, st)
           : cd >= 32 ? launch_sa_dn_t<BITS, 32>(L, B, M, st)
           : cd >= 16 ? launch_sa_dn_t<BITS, 16>(L, B, M, st)
                      : launch_sa_dn_t<BITS, 8>(L, B, M, st);
}
} // namespace

hipError_t launch_shared_affine(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st) {
    if (!L.shared_affine) return hipSuccess;
    switch (L.sa_bits) {
        case 2: return launch_sa<2>(L, B, M, st);
        case 4: return launch_sa<4>(L, B, M, st);
        case 8: return launch_sa<8>(L, B, M, st);
        default: return hipErrorInvalidValue;
    }
}

} // namespace q38
