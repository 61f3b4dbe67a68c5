// q38_affine.hpp — dot products of bf16 rows with MLX affine-quantized weight rows, shared
// by the affine shared expert (q38_affine.hip) and the GatedDeltaNet projections
// (q38_gdn.hip): quantized_matmul's arithmetic as this build computes it.
//
// Row o of a [OUT, IN] projection holds IN values q in [0, 2^bits) packed LSB-first in 32-bit
// words (32 / bits per word); w[o, c] = scale[o, c / G] * q[o, c] + bias[o, c / G], scales and
// biases bf16 or fp16. A lane group of LPR lanes takes one weight row: lane k of the group
// takes the 32-input chunks k, k + LPR, ... (each chunk inside one scale group: G is a
// multiple of 32); per chunk and request row it forms scale * sum(q x) + bias * sum(x) in
// float and accumulates; the group's partial sums meet in an xor butterfly. Up to kSaRows
// request rows are staged in LDS as bf16.
#pragma once

#include "q38_moe_dev.hpp"

namespace q38 {
namespace {

constexpr int kSaRows = 16;     // request rows per workgroup
constexpr int kSaThreads = 256;

__device__ __forceinline__ float sa_param(const uint16_t* p, size_t i, int f16) {
    const uint16_t v = p[i];
    return f16 ? h2f(v) : bf2f(v);
}

// Rows [r0, r0 + nr) of src ([rows][n] bf16) into xs ([nr][n]), 16-byte units.
__device__ __forceinline__ void sa_stage(const uint16_t* src, int n, int r0, int nr, uint16_t* xs) {
    const uint4* s4 = reinterpret_cast<const uint4*>(src + static_cast<size_t>(r0) * n);
    uint4* d4 = reinterpret_cast<uint4*>(xs);
    for (int i = threadIdx.x; i < nr * n / 8; i += kSaThreads) d4[i] = s4[i];
}

// acc[r] = sum over the row's inputs of w * x_r for the nr staged rows (every lane of the
// lane group ends with the totals).
template <int BITS, int LPR>
__device__ __forceinline__ void sa_row_dot(const uint32_t* wrow, const uint16_t* srow, const uint16_t* brow, int IN,
                                           int G, int f16, const uint16_t* xs, int nr, float (&acc)[kSaRows]) {
    const int gl = (threadIdx.x & 63) % LPR;
    constexpr uint32_t kMask = (1u << BITS) - 1u;
#pragma unroll
    for (int r = 0; r < kSaRows; ++r) acc[r] = 0.0f;
    for (int c = gl; c < IN / 32; c += LPR) {
        uint32_t wq[BITS];
#pragma unroll
        for (int k = 0; k < BITS; ++k) wq[k] = wrow[c * BITS + k];
        const int g = c * 32 / G;
        const float sc = sa_param(srow, g, f16), bi = sa_param(brow, g, f16);
        float q[32];
#pragma unroll
        for (int j = 0; j < 32; ++j)
            q[j] = static_cast<float>((wq[j * BITS / 32] >> ((j * BITS) % 32)) & kMask);
#pragma unroll
        for (int r = 0; r < kSaRows; ++r) {
            if (r >= nr) continue;
            const uint4* x4 = reinterpret_cast<const uint4*>(xs + static_cast<size_t>(r) * IN + c * 32);
            float qx = 0.0f, sx = 0.0f;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const uint4 u = x4[v];
                const uint32_t w4[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const float a = bflo(w4[k]), b = bfhi(w4[k]);
                    qx = fmaf(q[8 * v + 2 * k], a, qx);
                    qx = fmaf(q[8 * v + 2 * k + 1], b, qx);
                    sx += a;
                    sx += b;
                }
            }
            acc[r] = fmaf(sc, qx, fmaf(bi, sx, acc[r]));
        }
    }
#pragma unroll
    for (int m = LPR / 2; m > 0; m >>= 1)
#pragma unroll
        for (int r = 0; r < kSaRows; ++r) acc[r] += __shfl_xor(acc[r], m, 64);
}

// sa_row_dot with the staged rows' 32-input chunk sums given (sxs [nr][IN / 32], each the
// same sequential float sum sa_row_dot forms): the sums are formed once per workgroup instead
// of once per weight row; the results are the same bits.
template <int BITS, int LPR>
__device__ __forceinline__ void sa_row_dot_sx(const uint32_t* wrow, const uint16_t* srow, const uint16_t* brow, int IN,
                                              int G, int f16, const uint16_t* xs, const float* sxs, int nr,
                                              float (&acc)[kSaRows]) {
    const int gl = (threadIdx.x & 63) % LPR;
    constexpr uint32_t kMask = (1u << BITS) - 1u;
    const int nc = IN / 32;
#pragma unroll
    for (int r = 0; r < kSaRows; ++r) acc[r] = 0.0f;
    for (int c = gl; c < nc; c += LPR) {
        uint32_t wq[BITS];
#pragma unroll
        for (int k = 0; k < BITS; ++k) wq[k] = wrow[c * BITS + k];
        const int g = c * 32 / G;
        const float sc = sa_param(srow, g, f16), bi = sa_param(brow, g, f16);
        float q[32];
#pragma unroll
        for (int j = 0; j < 32; ++j)
            q[j] = static_cast<float>((wq[j * BITS / 32] >> ((j * BITS) % 32)) & kMask);
#pragma unroll
        for (int r = 0; r < kSaRows; ++r) {
            if (r >= nr) continue;
            const uint4* x4 = reinterpret_cast<const uint4*>(xs + static_cast<size_t>(r) * IN + c * 32);
            float qx = 0.0f;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const uint4 u = x4[v];
                const uint32_t w4[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    qx = fmaf(q[8 * v + 2 * k], bflo(w4[k]), qx);
                    qx = fmaf(q[8 * v + 2 * k + 1], bfhi(w4[k]), qx);
                }
            }
            acc[r] = fmaf(sc, qx, fmaf(bi, sxs[r * nc + c], acc[r]));
        }
    }
#pragma unroll
    for (int m = LPR / 2; m > 0; m >>= 1)
#pragma unroll
        for (int r = 0; r < kSaRows; ++r) acc[r] += __shfl_xor(acc[r], m, 64);
}

// The chunk sums of nr staged rows (xs [nr][IN]) into sxs [nr][IN / 32], in sa_row_dot's order.
__device__ __forceinline__ void sa_chunk_sums(const uint16_t* xs, int IN, int nr, float* sxs, int nthreads) {
    const int nc = IN / 32;
    for (int i = threadIdx.x; i < nr * nc; i += nthreads) {
        const uint4* x4 = reinterpret_cast<const uint4*>(xs + static_cast<size_t>(i / nc) * IN + (i % nc) * 32);
        float sx = 0.0f;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const uint4 u = x4[v];
            const uint32_t w4[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                sx += bflo(w4[k]);
                sx += bfhi(w4[k]);
            }
        }
        sxs[i] = sx;
    }
}

} // namespace
} // namespace q38
