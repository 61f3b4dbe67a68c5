// q38_moe_grp.hpp — the grouped-scale expert projections (VALU): layers whose scales are per
// 64-input group in a geometry the MFMA kernels do not take (d4 and d2 projections, wider
// calls), the reference checkpoints' layout (src/sparse_moe.cpp:641-647). The kernels and
// their launchers; each codebook dimension is instantiated in a translation unit of its own
// (q38_moe_grp{8,4,2}.hip), since their many (bits, lanes-per-row, routes) instantiations
// dominate the build.
#pragma once

#include "q38_moe_dev.hpp"

namespace q38 {
namespace {

inline int next_pow2(int v) {
    int p = 1;
    while (p < v) p <<= 1;
    return p;
}

// ============================================================== grouped-scale path
// Layers whose scales are per 64-input group (the reference checkpoint layout,
// src/sparse_moe.cpp:641-647) take this path: VALU dot products with codebook reads
// through the cache, per-group scaling in the lane. Same fp32 g/u/d outputs.
template <int D>
struct Vec;
template <>
struct Vec<8> {
    // fp16 codebook, or INT8 codebook x one fp16 scale (value = q * scale, exact in float)
    static __device__ __forceinline__ void load_book(const ProjDev& P, uint32_t code, float* v) {
        if (P.book_i8) {
            const uint2 b = *reinterpret_cast<const uint2*>(P.book_i8 + code * 8);
            const uint32_t w[2] = {b.x, b.y};
#pragma unroll
            for (int i = 0; i < 8; ++i)
                v[i] = static_cast<float>(static_cast<int8_t>(w[i >> 2] >> (8 * (i & 3)))) * P.book_scale;
            return;
        }
        const uint4 b = *reinterpret_cast<const uint4*>(P.book + code * 8);
        const uint32_t w[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[2 * i] = h2f(static_cast<uint16_t>(w[i]));
            v[2 * i + 1] = h2f(static_cast<uint16_t>(w[i] >> 16));
        }
    }
};
template <>
struct Vec<4> {
    static __device__ __forceinline__ void load_book(const ProjDev& P, uint32_t code, float* v) {
        const uint2 b = *reinterpret_cast<const uint2*>(P.book + code * 4);
        v[0] = h2f(static_cast<uint16_t>(b.x));
        v[1] = h2f(static_cast<uint16_t>(b.x >> 16));
        v[2] = h2f(static_cast<uint16_t>(b.y));
        v[3] = h2f(static_cast<uint16_t>(b.y >> 16));
    }
};

template <>
struct Vec<2> {
    // d2/K256: the byte codes of the reference checkpoint's first layers
    static __device__ __forceinline__ void load_book(const ProjDev& P, uint32_t code, float* v) {
        const uint32_t b = *reinterpret_cast<const uint32_t*>(P.book + code * 2);
        v[0] = h2f(static_cast<uint16_t>(b));
        v[1] = h2f(static_cast<uint16_t>(b >> 16));
    }
};

constexpr int kGuRowsPerBlock = 64;
constexpr int kDownRowsPerBlock = 128;

// Staged input rows of the grouped kernels, fp16: row j, column c at fin_at(j, c, IN). Two
// pad halves (one bank) after every 64 columns, so that the lanes of a row (16 codes each,
// 64 or 128 columns apart) read different LDS banks instead of one. fp16 keeps 16 rows of
// H = 2048 at 66.5 KiB, two workgroups per CU. (Inputs are bf16 values or SwiGLU outputs
// rounded to bf16: fp16 holds them exactly in the normal range; the MFMA paths take the
// same fp16 operand.)
typedef _Float16 fin_t;
__host__ __device__ constexpr int fin_stride(int IN) { return IN + 2 * (IN / 64); }
constexpr size_t kFinLdsMax = 68 * 1024;  // 16 rows of H = 2048 (68,096 bytes)
__device__ __forceinline__ int fin_at(int j, int c, int IN) { return j * fin_stride(IN) + c + 2 * (c / 64); }

// Lane mapping: a lane owns 16 consecutive codes of a row (BITS/2 words); LPR lanes
// (power of two, padded) cover one row; 64/LPR rows per wave. in_f: n rows staged at fin_at. Output row
// pos0 + j, or its route index when rplan (the plan) is given (down projections).
template <int D, int BITS, int LPR, int MAXN>
__device__ __forceinline__ void grouped_rows(const ProjDev& P, int expert, int IN, int OUT, int o_base,
                                             int rows_per_block, const fin_t* in_f, int n, float* out,
                                             int pos0, int wave, int lane, const int32_t* rplan = nullptr,
                                             int MK = 0) {
    const int nsub = IN / D;
    const int lanes_used = (nsub + 15) / 16;
    const int sub_lane = lane % LPR;
    const bool active = sub_lane < lanes_used;
    const int s0 = sub_lane * 16;
    const int spg = IN / P.ngrp / D;
    const bool row_scale = P.ngrp == 1;
    constexpr int WPL = BITS / 2;
    constexpr int RPW = 64 / LPR;
    for (int it = 0; it < rows_per_block / (4 * RPW); ++it) {
        const int o = o_base + it * 4 * RPW + wave * RPW + lane / LPR;
        float acc[MAXN];
#pragma unroll
        for (int j = 0; j < MAXN; ++j) acc[j] = 0.0f;
        if (active && o < OUT) {
            const size_t rowi = static_cast<size_t>(expert) * OUT + o;
            const uint32_t* pw = P.codes + rowi * P.words + (s0 / 32) * BITS + ((s0 % 32) / 16) * WPL;
            uint32_t wr[WPL + 1];
#pragma unroll
            for (int i = 0; i < WPL; ++i) wr[i] = pw[i];
            wr[WPL] = 0;
            float pp[MAXN];
#pragma unroll
            for (int j = 0; j < MAXN; ++j) pp[j] = 0.0f;
#pragma unroll
            for (int qq = 0; qq < 16; ++qq) {
                const int s = s0 + qq;
                const uint32_t c = code_from<BITS>(wr, qq);
                float bk[D];
                Vec<D>::load_book(P, c, bk);
#pragma unroll
                for (int j = 0; j < MAXN; ++j)
                    if (j < n)
#pragma unroll
                        for (int dd = 0; dd < D; ++dd) pp[j] = fmaf(static_cast<float>(in_f[fin_at(j, s * D + dd, IN)]), bk[dd], pp[j]);
                // a group ends here, or the lane's span ends inside a group of more than 16 codes
                if (!row_scale && (((s + 1) % spg) == 0 || qq == 15)) {
                    const float sc = h2f(P.scales[rowi * P.ngrp + s / spg]);
#pragma unroll
                    for (int j = 0; j < MAXN; ++j) {
                        acc[j] = fmaf(sc, pp[j], acc[j]);
                        pp[j] = 0.0f;
                    }
                }
            }
            if (row_scale) {
#pragma unroll
                for (int j = 0; j < MAXN; ++j) acc[j] = pp[j];
            }
        }
#pragma unroll
        for (int j = 0; j < MAXN; ++j) acc[j] = group_sum_xor<LPR>(acc[j]);
        if (sub_lane == 0 && o < OUT) {
            const float sc = row_scale ? h2f(P.scales[static_cast<size_t>(expert) * OUT + o]) : 1.0f;
#pragma unroll
            for (int j = 0; j < MAXN; ++j)
                if (j < n) out[static_cast<size_t>(rplan ? route_of_pos(rplan, MK, pos0 + j) : pos0 + j) * OUT + o] = acc[j] * sc;
        }
    }
}

// grouped_rows for a slot of n routes, with the route loop sized for n (1, 2, 4 or up to
// kMaxRows) rather than always unrolled to kMaxRows with a guard per route (most slots of
// a 16-row call have one or two routes).
template <int D, int BITS, int LPR>
__device__ __forceinline__ void grouped_rows_n(const ProjDev& P, int expert, int IN, int OUT, int o_base,
                                               int rows_per_block, const fin_t* in_f, int n, float* out, int pos0,
                                               int wave, int lane, const int32_t* rplan = nullptr, int MK = 0) {
    if (n <= 1)
        grouped_rows<D, BITS, LPR, 1>(P, expert, IN, OUT, o_base, rows_per_block, in_f, n, out, pos0, wave, lane, rplan, MK);
    else if (n <= 2)
        grouped_rows<D, BITS, LPR, 2>(P, expert, IN, OUT, o_base, rows_per_block, in_f, n, out, pos0, wave, lane, rplan, MK);
    else if (n <= 4)
        grouped_rows<D, BITS, LPR, 4>(P, expert, IN, OUT, o_base, rows_per_block, in_f, n, out, pos0, wave, lane, rplan, MK);
    else
        grouped_rows<D, BITS, LPR, kMaxRows>(P, expert, IN, OUT, o_base, rows_per_block, in_f, n, out, pos0, wave, lane,
                                             rplan, MK);
}

// Work units of a call. Up to kMaxRows rows, a unit is a slot of the plan (blockIdx.y). At
// prefill widths (more rows, the plan of k_plan_sort, same layout) a slot can hold up to M
// routes, more than the kMaxRows staged rows: a unit is then one pass over up to kMaxRows
// of a slot's routes, the slots' passes in slot order (routed experts ascending, then the
// shared expert). Block-wide (256 threads, uniform result); false past the last unit.
constexpr int kUnitSlotsPerThread = 5;  // 256 x 5 >= 1025 slots (E <= 1024 + the shared expert)
__device__ bool grouped_unit(const int32_t* plan, int M, int K, int has_shared, int u, int* slot, int* pass) {
    __shared__ int wsum[4];
    __shared__ int found[2];
    const int MK = M * K, nu = plan[0];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int cnt[kUnitSlotsPerThread], tot = 0;
#pragma unroll
    for (int c = 0; c < kUnitSlotsPerThread; ++c) {
        const int s = tid * kUnitSlotsPerThread + c;
        const int n = s < nu ? plan[2 + MK + s] - plan[1 + MK + s] : (s == nu && has_shared ? M : 0);
        cnt[c] = (n + kMaxRows - 1) / kMaxRows;
        tot += cnt[c];
    }
    int incl = tot;  // inclusive scan over the wave, then the waves in order
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int t = __shfl_up(incl, off, 64);
        if (lane >= off) incl += t;
    }
    if (lane == 63) wsum[wave] = incl;
    if (tid == 0) found[0] = -1;
    __syncthreads();
    int start = incl - tot;
    for (int w = 0; w < wave; ++w) start += wsum[w];
    const int total = wsum[0] + wsum[1] + wsum[2] + wsum[3];
#pragma unroll
    for (int c = 0; c < kUnitSlotsPerThread; ++c) {
        if (u >= start && u < start + cnt[c]) {
            found[0] = tid * kUnitSlotsPerThread + c;
            found[1] = u - start;
        }
        start += cnt[c];
    }
    __syncthreads();
    *slot = found[0];
    *pass = found[1];
    return u < total && found[0] >= 0;
}

// The unit's expert, routes (n <= kMaxRows, from sorted position pos0) and its first route's
// index j0 within the slot; false for no work.
__device__ __forceinline__ bool grouped_routes(const LayerDev& L, const MoeBufs& B, int M, int* expert, int* n,
                                               int* pos0, int* j0, bool* shared) {
    int slot = static_cast<int>(blockIdx.y), pass = 0;
    if (M > kMaxRows && !grouped_unit(B.plan, M, L.K, L.has_shared, slot, &slot, &pass)) return false;
    if (!slot_rows(B.plan, M, L.K, L.has_shared, slot, L.E, expert, n, pos0)) return false;
    *shared = slot == B.plan[0];
    *j0 = pass * kMaxRows;
    *n = *n - *j0 < kMaxRows ? *n - *j0 : kMaxRows;
    *pos0 += *j0;
    return *n > 0;
}

template <int D, int BITS, int LPR>
__global__ __launch_bounds__(256) void k_gu_grouped(LayerDev L, MoeBufs B, int M) {
    extern __shared__ __align__(16) fin_t fin[];  // n rows of H, at fin_at
    int expert, n, pos0, j0;
    bool shared;
    if (!grouped_routes(L, B, M, &expert, &n, &pos0, &j0, &shared)) return;
    const int H = L.H, I = L.I;
    for (int i = threadIdx.x; i < n * H; i += 256) {
        const int j = i / H, c = i % H;
        const int row = shared ? j0 + j : route_row(B.plan, M, L.K, pos0, j, false);
        fin[fin_at(j, c, H)] = static_cast<fin_t>(bf2f(B.x[static_cast<size_t>(row) * H + c]));
    }
    __syncthreads();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int o_base = blockIdx.x * kGuRowsPerBlock;
    grouped_rows_n<D, BITS, LPR>(L.p[0], expert, H, I, o_base, kGuRowsPerBlock, fin, n, B.g, pos0, wave, lane);
    grouped_rows_n<D, BITS, LPR>(L.p[1], expert, H, I, o_base, kGuRowsPerBlock, fin, n, B.u, pos0, wave, lane);
}

template <int D, int BITS, int LPR>
__global__ __launch_bounds__(256) void k_down_grouped(LayerDev L, MoeBufs B, int M) {
    extern __shared__ __align__(16) fin_t fin[];  // n rows of I, at fin_at
    int expert, n, pos0, j0;
    bool shared;
    if (!grouped_routes(L, B, M, &expert, &n, &pos0, &j0, &shared)) return;
    const int H = L.H, I = L.I;
    for (int i = threadIdx.x; i < n * I; i += 256) {
        const size_t at = static_cast<size_t>(pos0) * I + i;
        float g = B.g[at], u = B.u[at];
        if (L.gu_parts == 2) {
            g += B.g[B.gu_plane + at];
            u += B.u[B.gu_plane + at];
        }
        fin[fin_at(i / I, i % I, I)] = static_cast<fin_t>(swiglu(g, u));
    }
    __syncthreads();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    grouped_rows_n<D, BITS, LPR>(L.p[2], expert, I, H, blockIdx.x * kDownRowsPerBlock, kDownRowsPerBlock,
                                         fin, n, B.d, pos0, wave, lane, B.plan, M * L.K);
}


// Units of a call (grid.y): its slots up to kMaxRows rows; at prefill widths a bound on the
// passes, sum over slots of ceil(n / kMaxRows) <= MK / kMaxRows + slots + the shared
// expert's passes (units past the last exit at once).
inline int grouped_units(const LayerDev& L, int M) {
    const int MK = M * L.K;
    if (M <= kMaxRows) return MK + 1;
    const int slots = MK < L.E ? MK : L.E;
    return (MK + kMaxRows - 1) / kMaxRows + slots + (M + kMaxRows - 1) / kMaxRows + 1;
}

template <int D, int BITS, int LPR>
hipError_t launch_gu_grouped_g(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st) {
    const int rows = M < kMaxRows ? M : kMaxRows;
    const size_t lds = static_cast<size_t>(rows) * fin_stride(L.H) * sizeof(fin_t);
    if (lds > kFinLdsMax) return hipErrorInvalidValue;
    if (const hipError_t e = ensure_lds<k_gu_grouped<D, BITS, LPR>>(kFinLdsMax); e != hipSuccess) return e;
    return launch(k_gu_grouped<D, BITS, LPR>, dim3(L.I / kGuRowsPerBlock, grouped_units(L, M)), dim3(256), lds, st, L,
                  B, M);
}
template <int D, int BITS, int LPR>
hipError_t launch_down_grouped_g(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st) {
    const int rows = M < kMaxRows ? M : kMaxRows;
    const size_t lds = static_cast<size_t>(rows) * fin_stride(L.I) * sizeof(fin_t);
    if (lds > kFinLdsMax) return hipErrorInvalidValue;
    if (const hipError_t e = ensure_lds<k_down_grouped<D, BITS, LPR>>(kFinLdsMax); e != hipSuccess) return e;
    return launch(k_down_grouped<D, BITS, LPR>, dim3(L.H / kDownRowsPerBlock, grouped_units(L, M)), dim3(256), lds, st,
                  L, B, M);
}
} // namespace
} // namespace q38
