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
// Rows of several affine projections of the same S input rows in one launch: workgroup
// blocks [p.first_block, next first_block) take projection p's weight rows, a lane group of
// LPR lanes per weight row, up to 16 input rows staged in LDS with their 32-input sums.
template <int BITS, int LPR>
__global__ __launch_bounds__(kSaThreads) void k_affine_rows(AffineRowSet set, const uint16_t* __restrict__ x, int S,
                                                         int IN, int G, int f16, int rows_wg) {
    extern __shared__ __align__(16) uint16_t xs[];  // [rows_wg][IN], then the chunk sums [rows_wg][IN / 32]
    const int r0 = blockIdx.y * rows_wg, nr = S - r0 < rows_wg ? S - r0 : rows_wg;
    float* sxs = reinterpret_cast<float*>(xs + static_cast<size_t>(rows_wg) * IN);
    // the projection of this block (uniform selects over the argument block)
    const int bx = static_cast<int>(blockIdx.x);
    const int pi = set.n > 3 && bx >= set.p[3].first_block ? 3
                   : set.n > 2 && bx >= set.p[2].first_block ? 2
                   : set.n > 1 && bx >= set.p[1].first_block ? 1
                                                             : 0;
    const AffineRows P = pi == 3 ? set.p[3] : pi == 2 ? set.p[2] : pi == 1 ? set.p[1] : set.p[0];
    sa_stage(x, IN, r0, nr, xs);
    __syncthreads();
    sa_chunk_sums(xs, IN, nr, sxs, kSaThreads);
    __syncthreads();
    constexpr int OPW = 64 / LPR;
    const int o = ((bx - P.first_block) * (kSaThreads / 64) + (threadIdx.x >> 6)) * OPW + (threadIdx.x & 63) / LPR;
    if (o >= P.out) return;
    const int wpr = IN * BITS / 32, ngrp = IN / G;
    float acc[kSaRows];
    sa_row_dot_sx<BITS, LPR>(P.w + static_cast<size_t>(o) * wpr, P.s + static_cast<size_t>(o) * ngrp,
                             P.b + static_cast<size_t>(o) * ngrp, IN, G, f16, xs, sxs, nr, acc);
    if ((threadIdx.x & 63) % LPR == 0)
#pragma unroll
        for (int r = 0; r < kSaRows; ++r)
            if (r < nr) P.dst[static_cast<size_t>(r0 + r) * P.dst_stride + o] = f2bf(acc[r]);
}

int proj_lpr(int IN, int out) {
    const int c = IN / 32;
    const int lpr = c >= 256 ? 64 : c >= 128 ? 32 : c >= 64 ? 16 : 8;
    // (fewer weight rows per workgroup where the projection has few rows: at least ~512
    // workgroups for 256 CUs)
    return out / (kSaThreads / 64 * (64 / lpr)) < 512 && lpr < 64 && c >= 2 * lpr ? 2 * lpr : lpr;
}

template <int BITS, int LPR>
hipError_t launch_proj_t(AffineRowSet set, int blocks, const uint16_t* x, int S, int IN, int G, int f16,
                         hipStream_t st) {
    // staged rows: up to 16, fewer for wide inputs (the staging stays within 144 KiB of LDS)
    int rows = static_cast<int>((144 * 1024) / (static_cast<size_t>(IN) * 2 + static_cast<size_t>(IN) / 8));
    rows = rows > kSaRows ? kSaRows : rows;
    rows = rows > S ? S : rows;
    if (rows < 1) return hipErrorInvalidValue;
    const size_t lds = static_cast<size_t>(rows) * IN * 2 + static_cast<size_t>(rows) * (IN / 32) * 4;
    if (const hipError_t e = ensure_lds<k_affine_rows<BITS, LPR>>(lds); e != hipSuccess) return e;
    return launch(k_affine_rows<BITS, LPR>, dim3(blocks, (S + rows - 1) / rows), dim3(kSaThreads), lds, st, set, x, S, IN,
                  G, f16, rows);
}
template <int BITS>
hipError_t launch_proj_b(AffineRowSet set, const uint16_t* x, int S, int IN, int G, int f16, hipStream_t st) {
    int rows_out = 0;
    for (int i = 0; i < set.n; ++i) rows_out += set.p[i].out;
    const int lpr = proj_lpr(IN, rows_out);
    int blocks = 0;
    const int per = kSaThreads / 64 * (64 / lpr);
    for (int i = 0; i < set.n; ++i) {
        set.p[i].first_block = blocks;
        blocks += (set.p[i].out + per - 1) / per;
    }
    switch (lpr) {
        case 64: return launch_proj_t<BITS, 64>(set, blocks, x, S, IN, G, f16, st);
        case 32: return launch_proj_t<BITS, 32>(set, blocks, x, S, IN, G, f16, st);
        case 16: return launch_proj_t<BITS, 16>(set, blocks, x, S, IN, G, f16, st);
        default: return launch_proj_t<BITS, 8>(set, blocks, x, S, IN, G, f16, st);
    }
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

hipError_t launch_affine_rows(const AffineRowSet& set, const uint16_t* x, int S, int IN, int G, int bits, int f16,
                              hipStream_t st) {
    switch (bits) {
        case 2: return launch_proj_b<2>(set, x, S, IN, G, f16, st);
        case 4: return launch_proj_b<4>(set, x, S, IN, G, f16, st);
        case 8: return launch_proj_b<8>(set, x, S, IN, G, f16, st);
        default: return hipErrorInvalidValue;
    }
}

} // namespace q38
