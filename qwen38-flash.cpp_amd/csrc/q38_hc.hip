// q38_hc.hip — the HyperConnection stream mixer at verify widths (1..16 rows): the read
// that turns a row's HC residual streams into the block input, and the write that adds the
// block output back into every stream (HyperConnection::read / write,
// src/hyper_connection.cpp:309-493, 692-709; the rounding points of the reference's fused
// read, src/hc_metal_kernels.hpp:10-36, 85-128, 270-308).
//
//   k_hc_norm   per (row, stream): RMSNorm over H and the learned norm weight,
//               xn = T(T(x * inv_rms) * T(1 + w))                     (T = round to BF16)
//   k_hc_down   one workgroup per output: the rank projection of the row's flat normalised
//               streams (MLX affine weights: q * scale + bias per group, 4 or 8 bits),
//               a = T(v * T(sigmoid(v))) with v = T(dot / HC); the injection outputs in the
//               same launch, inj = T(2 * T(sigmoid(T(T(dot) * T(1 / HC)))))
//   k_hc_up     eight lanes per (stream, column): u = T(dot over the rank), gate = T(sigmoid(u)),
//               the stream's term T(gate * xn); the workgroup adds the HC terms in stream
//               order in float: mixed = T(T(sum) / HC)
//   k_hc_write  stream <- T(stream + T(block_output * inj[stream]))
// Memory per call is tiny next to the MoE block (R x HC x H x bits / 8 bytes per projection:
// 1 MiB each at H 2048, HC 4, R 256, 4 bits); the kernels are latency-bound, so each launch
// spreads its weight rows over many waves and issues a thread's loads before its products.
#include "q38_device.hpp"
#include "q38_internal.hpp"

#include <algorithm>

namespace q38 {
namespace {

__device__ __forceinline__ float sigmoid_f(float v) { return 1.0f / (1.0f + expf(-v)); }

// ------------------------------------------------------------------ read: normalisation
// Workgroup (stream s, row m), 256 threads: thread t holds the 8-column runs t + 256 i of the
// stream (H / 8 runs; at most 2 per thread for H <= 4096), loaded with the matching norm
// weights in one go; squares summed run by run with fmaf, the wave totals (xor butterfly)
// added in wave order.
__global__ __launch_bounds__(256) void k_hc_norm(HcDev D, const uint16_t* __restrict__ stream, uint16_t* __restrict__ xn) {
    constexpr int kRuns = kHcMaxPerThread / 8;
    __shared__ float red[4];
    const int s = blockIdx.x, m = blockIdx.y, tid = threadIdx.x;
    const int H = D.H, runs = H / 8;
    const size_t base = (static_cast<size_t>(m) * D.HC + s) * H;
    uint4 xv[kRuns], wv[kRuns];
#pragma unroll
    for (int i = 0; i < kRuns; ++i) {
        const int r = tid + 256 * i < runs ? tid + 256 * i : 0;  // (past the stream: run 0, unused)
        xv[i] = *reinterpret_cast<const uint4*>(stream + base + 8 * r);
        wv[i] = *reinterpret_cast<const uint4*>(D.wn + static_cast<size_t>(s) * H + 8 * r);
    }
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < kRuns; ++i)
        if (tid + 256 * i < runs) {
            const uint32_t q[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                ss = fmaf(bflo(q[k]), bflo(q[k]), ss);
                ss = fmaf(bfhi(q[k]), bfhi(q[k]), ss);
            }
        }
    ss = wave_sum_xor(ss);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    lds_barrier();
    const float total = ((red[0] + red[1]) + red[2]) + red[3];
    const float inv = 1.0f / sqrtf(total / static_cast<float>(H) + D.eps);
#pragma unroll
    for (int i = 0; i < kRuns; ++i)
        if (tid + 256 * i < runs) {
            const uint32_t q[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
            const uint32_t w[4] = {wv[i].x, wv[i].y, wv[i].z, wv[i].w};
            uint32_t o[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t lo = f2bf(rbf(bflo(q[k]) * inv) * bflo(w[k]));
                const uint32_t hi = f2bf(rbf(bfhi(q[k]) * inv) * bfhi(w[k]));
                o[k] = lo | (hi << 16);
            }
            *reinterpret_cast<uint4*>(xn + base + 8 * (tid + 256 * i)) = make_uint4(o[0], o[1], o[2], o[3]);
        }
}

// Values t of one packed word as weights: q * scale + bias (fmaf).
template <int BITS>
__device__ __forceinline__ void dequant_word(uint32_t w, float s, float b, float (&out)[32 / BITS]) {
#pragma unroll
    for (int t = 0; t < 32 / BITS; ++t)
        out[t] = fmaf(static_cast<float>((w >> (BITS * t)) & ((1u << BITS) - 1u)), s, b);
}

// ------------------------------------------------------------------ read: rank projection
// Workgroup o (256 threads): output o (o < R: a rank row; R <= o < R + HC: injection row
// o - R). Thread t takes the packed words t + 256 i of the output's row and every row's
// matching normalised inputs (read from L2: xn is M x HC x H x 2 bytes); UNR words' loads
// are issued before their products. The four waves' totals are added in wave order.
template <int BITS, int MR>
__global__ __launch_bounds__(256) void k_hc_down(HcDev D, int M, const uint16_t* __restrict__ xn, float* __restrict__ act,
                                                 uint16_t* __restrict__ inj) {
    constexpr int VPW = 32 / BITS, XW = VPW / 2, UNR = MR <= 4 ? 4 : MR <= 8 ? 2 : 1;
    __shared__ float red[4][MR];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int o = blockIdx.x;
    const int K = D.HC * D.H, words = K / VPW, groups = K / D.G;
    const bool rank_row = o < D.R;
    const int row = rank_row ? o : o - D.R;
    const uint32_t* W = (rank_row ? D.dw : D.iw) + static_cast<size_t>(row) * words;
    const uint16_t* S = (rank_row ? D.ds : D.is) + static_cast<size_t>(row) * groups;
    const uint16_t* Bi = (rank_row ? D.db : D.ib) + static_cast<size_t>(row) * groups;
    float acc[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = 0.0f;
    for (int j0 = tid; j0 < words; j0 += 256 * UNR) {
        uint32_t wv[UNR], xr[UNR][MR][XW];
        float sv[UNR], bv[UNR];
#pragma unroll
        for (int u = 0; u < UNR; ++u) {
            const int j = j0 + 256 * u < words ? j0 + 256 * u : j0;  // (past the end: repeated, unused)
            const int g = j * VPW / D.G;
            wv[u] = W[j];
            sv[u] = bf2f(S[g]);
            bv[u] = bf2f(Bi[g]);
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                const uint16_t* p = xn + static_cast<size_t>(m < M ? m : M - 1) * K + j * VPW;
                if constexpr (XW == 4) {
                    const uint4 q = *reinterpret_cast<const uint4*>(p);
                    xr[u][m][0] = q.x; xr[u][m][1] = q.y; xr[u][m][2] = q.z; xr[u][m][3] = q.w;
                } else {
                    const uint2 q = *reinterpret_cast<const uint2*>(p);
                    xr[u][m][0] = q.x; xr[u][m][1] = q.y;
                }
            }
        }
#pragma unroll
        for (int u = 0; u < UNR; ++u)
            if (j0 + 256 * u < words) {
                float wq[VPW];
                dequant_word<BITS>(wv[u], sv[u], bv[u], wq);
#pragma unroll
                for (int m = 0; m < MR; ++m)
#pragma unroll
                    for (int t = 0; t < XW; ++t) {
                        acc[m] = fmaf(bflo(xr[u][m][t]), wq[2 * t], acc[m]);
                        acc[m] = fmaf(bfhi(xr[u][m][t]), wq[2 * t + 1], acc[m]);
                    }
            }
    }
    if constexpr (MR == 1) {
        const float t = wave_sum_xor(acc[0]);
        if (lane == 0) red[wave][0] = t;
    } else {
        wave_sum_xor_scatter<MR>(acc);
#pragma unroll
        for (int s = 0; s < scatter_slots<MR>(); ++s)
            if (scatter_leader<MR>(lane)) red[wave][scatter_value<MR>(s, lane >> 4)] = acc[s];
    }
    lds_barrier();
    if (tid < M) {
        const int m = tid;
        const float total = ((red[0][m] + red[1][m]) + red[2][m]) + red[3][m];
        if (rank_row) {
            const float v = rbf(total / static_cast<float>(D.HC));
            act[static_cast<size_t>(m) * D.R + row] = rbf(v * rbf(sigmoid_f(v)));
        } else {
            const float v = rbf(rbf(total) * rbf(1.0f / static_cast<float>(D.HC)));
            inj[static_cast<size_t>(m) * D.HC + row] = f2bf(rbf(sigmoid_f(v)) * 2.0f);
        }
    }
}

// ------------------------------------------------------------------ read: expansion + mix
// Workgroup b, HC waves: wave h = stream h; lanes 8c' .. 8c' + 7 share column c = 8 b + c',
// whose weight row is h H + c (R / VPW packed words, R / G groups), lane octant q taking the
// row's 16-byte quads q, q + 8, ... (each inside one scale group). The octants' partial sums
// meet by three DPP steps (((q0 + q1) + (q2 + q3)) + ((q4 + q5) + (q6 + q7))). The rows' rank
// activations are staged in LDS and read 16 bytes at a time (the 8 columns of a wave read
// the same ones); the streams' terms meet in LDS and are added in stream order.
template <int BITS, int MR>
__global__ __launch_bounds__(1024) void k_hc_up(HcDev D, int M, const uint16_t* __restrict__ xn,
                                                const float* __restrict__ act, uint16_t* __restrict__ mixed) {
    constexpr int VPW = 32 / BITS, QMAX = kHcMaxRank / VPW / 32;
    extern __shared__ __align__(16) float hc_lds[];
    float* acts = hc_lds;                                     // [M][R]
    float* terms = hc_lds + static_cast<size_t>(MR) * D.R;    // [MR][HC][8]
    const int tid = threadIdx.x, lane = tid & 63, h = tid >> 6;
    const int H = D.H, R = D.R, HC = D.HC;
    const int cl = lane >> 3, q = lane & 7;
    const int c = blockIdx.x * 8 + cl;
    const size_t wrow = static_cast<size_t>(h) * H + c;
    const int nq = R / VPW / 4, groups = R / D.G;
    const uint4* W4 = reinterpret_cast<const uint4*>(D.uw + wrow * (R / VPW));
    const uint16_t* S = D.us + wrow * groups;
    const uint16_t* Bi = D.ub + wrow * groups;
    uint4 wv[QMAX];
    float sv[QMAX], bv[QMAX];
#pragma unroll
    for (int i = 0; i < QMAX; ++i) {
        const int qi = q + 8 * i < nq ? q + 8 * i : 0;  // (past the row's quads: quad 0, unused)
        const int g = qi * 4 * VPW / D.G;
        wv[i] = W4[qi];
        sv[i] = bf2f(S[g]);
        bv[i] = bf2f(Bi[g]);
    }
    // the epilogue's normalised stream values (lanes q == 0), requested with the weights
    uint16_t xe[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) xe[m] = xn[(static_cast<size_t>(m < M ? m : M - 1) * HC + h) * H + c];
    {   // the activations into LDS, 16 bytes a thread and four loads in flight before the stores
        const int n4 = M * R / 4, nt = 64 * HC;
        const uint4* src = reinterpret_cast<const uint4*>(act);
        uint4* dst = reinterpret_cast<uint4*>(acts);
        for (int b = tid; b < n4; b += 4 * nt) {
            uint4 v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) v[u] = src[b + u * nt < n4 ? b + u * nt : b];
#pragma unroll
            for (int u = 0; u < 4; ++u)
                if (b + u * nt < n4) dst[b + u * nt] = v[u];
        }
    }
    lds_barrier();
    float acc[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = 0.0f;
#pragma unroll
    for (int i = 0; i < QMAX; ++i)
        if (q + 8 * i < nq) {
            const uint32_t w4[4] = {wv[i].x, wv[i].y, wv[i].z, wv[i].w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int r0 = ((q + 8 * i) * 4 + k) * VPW;
                float wq[VPW];
                dequant_word<BITS>(w4[k], sv[i], bv[i], wq);
#pragma unroll
                for (int m = 0; m < MR; ++m) {
                    const float4* a4 = reinterpret_cast<const float4*>(acts + (m < M ? m : M - 1) * R + r0);
#pragma unroll
                    for (int t4 = 0; t4 < VPW / 4; ++t4) {
                        const float4 av = a4[t4];
                        acc[m] = fmaf(av.x, wq[4 * t4], acc[m]);
                        acc[m] = fmaf(av.y, wq[4 * t4 + 1], acc[m]);
                        acc[m] = fmaf(av.z, wq[4 * t4 + 2], acc[m]);
                        acc[m] = fmaf(av.w, wq[4 * t4 + 3], acc[m]);
                    }
                }
            }
        }
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        acc[m] = acc[m] + xor_lane_f<1>(acc[m]);
        acc[m] = acc[m] + xor_lane_f<2>(acc[m]);
        acc[m] = acc[m] + xor_lane_f<4>(acc[m]);
    }
    if (q == 0) {
#pragma unroll
        for (int m = 0; m < MR; ++m)
            if (m < M) {
                const float u = rbf(acc[m]);
                const float gate = rbf(sigmoid_f(u));
                terms[(m * HC + h) * 8 + cl] = rbf(gate * bf2f(xe[m]));
            }
    }
    lds_barrier();
    for (int i = tid; i < M * 8; i += 64 * HC) {
        const int m = i >> 3, cc = i & 7;
        float s = 0.0f;
        for (int hh = 0; hh < HC; ++hh) s += terms[(m * HC + hh) * 8 + cc];
        mixed[static_cast<size_t>(m) * H + blockIdx.x * 8 + cc] = f2bf(rbf(s) / static_cast<float>(HC));
    }
}

// ------------------------------------------------------------------ write and stream set-up
// Thread: 8 consecutive stream elements of row blockIdx.y.
__global__ __launch_bounds__(256) void k_hc_write(int H, int HC, const uint16_t* __restrict__ stream,
                                                  const uint16_t* __restrict__ block_out,
                                                  const uint16_t* __restrict__ inj, uint16_t* __restrict__ out) {
    const int m = blockIdx.y;
    const int k0 = (blockIdx.x * 256 + threadIdx.x) * 8;
    if (k0 >= HC * H) return;
    const int h = k0 / H, c0 = k0 - h * H;
    const float g = bf2f(inj[static_cast<size_t>(m) * HC + h]);
    const size_t at = static_cast<size_t>(m) * HC * H + k0;
    const uint4 sv = *reinterpret_cast<const uint4*>(stream + at);
    const uint4 bv = *reinterpret_cast<const uint4*>(block_out + static_cast<size_t>(m) * H + c0);
    const uint32_t s4[4] = {sv.x, sv.y, sv.z, sv.w}, b4[4] = {bv.x, bv.y, bv.z, bv.w};
    uint32_t o4[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t lo = f2bf(bflo(s4[i]) + rbf(bflo(b4[i]) * g));
        const uint32_t hi = f2bf(bfhi(s4[i]) + rbf(bfhi(b4[i]) * g));
        o4[i] = lo | (hi << 16);
    }
    *reinterpret_cast<uint4*>(out + at) = make_uint4(o4[0], o4[1], o4[2], o4[3]);
}

// out[m][s][c] = emb[m][c] (HyperConnection::initialize_stream: the embedding tiled HC times).
__global__ __launch_bounds__(256) void k_hc_tile(int H, int HC, const uint16_t* __restrict__ emb,
                                                 uint16_t* __restrict__ out) {
    const int m = blockIdx.y;
    const int k0 = (blockIdx.x * 256 + threadIdx.x) * 8;
    if (k0 >= HC * H) return;
    const int c0 = k0 % H;
    *reinterpret_cast<uint4*>(out + static_cast<size_t>(m) * HC * H + k0) =
        *reinterpret_cast<const uint4*>(emb + static_cast<size_t>(m) * H + c0);
}

// T(raw + 1): the norm weight the mixer multiplies by (src/hyper_connection.cpp:182-189).
__global__ void k_hc_norm_weight(const uint16_t* __restrict__ raw, int n, uint16_t* __restrict__ wn) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
        wn[i] = f2bf(bf2f(raw[i]) + 1.0f);
}

template <int BITS, int MR>
hipError_t launch_hc_read_mr(const HcDev& D, int M, const uint16_t* stream, uint16_t* xn, float* act,
                             uint16_t* mixed, uint16_t* inj, hipStream_t st) {
    hipError_t e = launch(k_hc_norm, dim3(D.HC, M), dim3(256), 0, st, D, stream, xn);
    if (e != hipSuccess) return e;
    const int n_out = D.R + (D.with_inj ? D.HC : 0);
    e = launch(k_hc_down<BITS, MR>, dim3(n_out), dim3(256), 0, st, D, M, xn, act, inj);
    if (e != hipSuccess) return e;
    const size_t lds = (static_cast<size_t>(MR) * D.R + static_cast<size_t>(MR) * D.HC * 8) * sizeof(float);
    if ((e = ensure_lds<k_hc_up<BITS, MR>>(hc_up_lds_max())) != hipSuccess) return e;
    return launch(k_hc_up<BITS, MR>, dim3(D.H / 8), dim3(64 * D.HC), lds, st, D, M, xn, act, mixed);
}

template <int BITS>
hipError_t launch_hc_read_b(const HcDev& D, int M, const uint16_t* stream, uint16_t* xn, float* act, uint16_t* mixed,
                            uint16_t* inj, hipStream_t st) {
    if (M <= 1) return launch_hc_read_mr<BITS, 1>(D, M, stream, xn, act, mixed, inj, st);
    if (M <= 2) return launch_hc_read_mr<BITS, 2>(D, M, stream, xn, act, mixed, inj, st);
    if (M <= 4) return launch_hc_read_mr<BITS, 4>(D, M, stream, xn, act, mixed, inj, st);
    if (M <= 8) return launch_hc_read_mr<BITS, 8>(D, M, stream, xn, act, mixed, inj, st);
    return launch_hc_read_mr<BITS, 16>(D, M, stream, xn, act, mixed, inj, st);
}

} // namespace

size_t hc_up_lds_max() {
    return (static_cast<size_t>(kMaxRows) * kHcMaxRank + static_cast<size_t>(kMaxRows) * kHcMaxStreams * 8) *
           sizeof(float);
}

hipError_t launch_hc_read(const HcDev& D, int M, const uint16_t* stream, uint16_t* xn, float* act, uint16_t* mixed,
                          uint16_t* inj, hipStream_t st) {
    return D.bits == 4 ? launch_hc_read_b<4>(D, M, stream, xn, act, mixed, inj, st)
                       : launch_hc_read_b<8>(D, M, stream, xn, act, mixed, inj, st);
}

hipError_t launch_hc_write(int H, int HC, int M, const uint16_t* stream, const uint16_t* block_out,
                           const uint16_t* inj, uint16_t* out, hipStream_t st) {
    return launch(k_hc_write, dim3((HC * H / 8 + 255) / 256, M), dim3(256), 0, st, H, HC, stream, block_out, inj, out);
}

hipError_t launch_hc_tile(int H, int HC, int M, const uint16_t* emb, uint16_t* out, hipStream_t st) {
    return launch(k_hc_tile, dim3((HC * H / 8 + 255) / 256, M), dim3(256), 0, st, H, HC, emb, out);
}

hipError_t launch_hc_norm_weight(const uint16_t* raw, int n, uint16_t* wn, hipStream_t st) {
    return launch(k_hc_norm_weight, dim3(std::min(1024, (n + 255) / 256)), dim3(256), 0, st, raw, n, wn);
}

} // namespace q38
