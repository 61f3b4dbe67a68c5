// q38_hc.hip — the HyperConnection stream mixer at verify widths (1..16 rows): the read
// that turns a row's HC residual streams into the block input, and the write that adds the
// block output back into every stream (HyperConnection::read / write,
// src/hyper_connection.cpp:309-493, 692-709; the rounding points of the reference's fused
// read, src/hc_metal_kernels.hpp:10-36, 85-128, 270-308).
//
//   k_hc_norm   per (row, stream): RMSNorm over H and the learned norm weight,
//               xn = T(T(x * inv_rms) * T(1 + w))                     (T = round to BF16)
//   k_hc_down   one wave per output: the rank projection of the row's flat normalised
//               streams (MLX affine weights: q * scale + bias per group, 4 or 8 bits),
//               a = T(v * T(sigmoid(v))) with v = T(dot / HC); the injection outputs in the
//               same launch, inj = T(2 * T(sigmoid(T(T(dot) * T(1 / HC)))))
//   k_hc_up     one lane per (stream, column): u = T(dot over the rank), gate = T(sigmoid(u)),
//               the stream's term T(gate * xn); the workgroup adds the HC terms in stream
//               order in float: mixed = T(T(sum) / HC)
//   k_hc_write  stream <- T(stream + T(block_output * inj[stream]))
// Memory per call is tiny next to the MoE block (R x HC x H x bits / 8 bytes per projection:
// 1 MiB each at H 2048, HC 4, R 256, 4 bits); the kernels are latency-bound, so each launch
// spreads its weight rows over as many waves as there are outputs.
#include "q38_device.hpp"
#include "q38_internal.hpp"

#include <algorithm>

namespace q38 {
namespace {

__device__ __forceinline__ float sigmoid_f(float v) { return 1.0f / (1.0f + expf(-v)); }

// ------------------------------------------------------------------ read: normalisation
// Workgroup (stream s, row m), 256 threads: thread t holds columns t + 256 i of the stream,
// squares summed in i order with fmaf, the wave totals (xor butterfly) added in wave order.
__global__ __launch_bounds__(256) void k_hc_norm(HcDev D, const uint16_t* __restrict__ stream, uint16_t* __restrict__ xn) {
    __shared__ float red[4];
    const int s = blockIdx.x, m = blockIdx.y, tid = threadIdx.x;
    const int H = D.H, npt = H / 256;
    const size_t base = (static_cast<size_t>(m) * D.HC + s) * H;
    float v[kHcMaxPerThread];
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < kHcMaxPerThread; ++i)
        if (i < npt) {
            v[i] = bf2f(stream[base + tid + 256 * i]);
            ss = fmaf(v[i], v[i], ss);
        }
    ss = wave_sum_xor(ss);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    lds_barrier();
    const float total = ((red[0] + red[1]) + red[2]) + red[3];
    const float inv = 1.0f / sqrtf(total / static_cast<float>(H) + D.eps);
#pragma unroll
    for (int i = 0; i < kHcMaxPerThread; ++i)
        if (i < npt) {
            const size_t k = base + tid + 256 * i;
            xn[k] = f2bf(rbf(v[i] * inv) * bf2f(D.wn[static_cast<size_t>(s) * H + tid + 256 * i]));
        }
}

// Values t of one packed word as weights: q * scale + bias (fmaf).
template <int BITS>
__device__ __forceinline__ void dequant_word(uint32_t w, float s, float b, float (&out)[32 / BITS]) {
#pragma unroll
    for (int t = 0; t < 32 / BITS; ++t)
        out[t] = fmaf(static_cast<float>((w >> (BITS * t)) & ((1u << BITS) - 1u)), s, b);
}

// 32 / BITS bf16 values of row m at column k0 (k0 a multiple of 32 / BITS).
template <int BITS>
__device__ __forceinline__ void load_bf16_run(const uint16_t* p, float (&x)[32 / BITS]) {
    if constexpr (BITS == 4) {
        const uint4 q = *reinterpret_cast<const uint4*>(p);
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            x[2 * i] = bflo(w[i]);
            x[2 * i + 1] = bfhi(w[i]);
        }
    } else {
        const uint2 q = *reinterpret_cast<const uint2*>(p);
        x[0] = bflo(q.x); x[1] = bfhi(q.x); x[2] = bflo(q.y); x[3] = bfhi(q.y);
    }
}

// ------------------------------------------------------------------ read: rank projection
// Wave w of workgroup b: output o = 4 b + w (o < R: a rank row; R <= o < R + HC: injection
// row o - R). Lane l takes the packed words l + 64 j of the output's row and every row's
// matching normalised inputs (read from L2: xn is M x HC x H x 2 bytes).
template <int BITS, int MR>
__global__ __launch_bounds__(256) void k_hc_down(HcDev D, int M, const uint16_t* __restrict__ xn, float* __restrict__ act,
                                                 uint16_t* __restrict__ inj) {
    constexpr int VPW = 32 / BITS;
    const int lane = threadIdx.x & 63;
    const int o = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int n_out = D.R + (D.with_inj ? D.HC : 0);
    if (o >= n_out) return;  // wave-uniform
    const int K = D.HC * D.H, words = K / VPW, groups = K / D.G;
    const bool rank_row = o < D.R;
    const int row = rank_row ? o : o - D.R;
    const uint32_t* W = (rank_row ? D.dw : D.iw) + static_cast<size_t>(row) * words;
    const uint16_t* S = (rank_row ? D.ds : D.is) + static_cast<size_t>(row) * groups;
    const uint16_t* Bi = (rank_row ? D.db : D.ib) + static_cast<size_t>(row) * groups;
    float acc[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = 0.0f;
    for (int j = lane; j < words; j += 64) {
        const int k0 = j * VPW, g = k0 / D.G;
        float wq[VPW];
        dequant_word<BITS>(W[j], bf2f(S[g]), bf2f(Bi[g]), wq);
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            const int mm = m < M ? m : M - 1;  // (rows past M repeat the last one; unused)
            float x[VPW];
            load_bf16_run<BITS>(xn + static_cast<size_t>(mm) * K + k0, x);
#pragma unroll
            for (int t = 0; t < VPW; ++t) acc[m] = fmaf(x[t], wq[t], acc[m]);
        }
    }
    const float inv_hc = 1.0f / static_cast<float>(D.HC);
    auto finish = [&](int m, float total) {
        if (rank_row) {
            const float v = rbf(total / static_cast<float>(D.HC));
            act[static_cast<size_t>(m) * D.R + row] = rbf(v * rbf(sigmoid_f(v)));
        } else {
            const float v = rbf(rbf(total) * rbf(inv_hc));
            inj[static_cast<size_t>(m) * D.HC + row] = f2bf(rbf(sigmoid_f(v)) * 2.0f);
        }
    };
    if constexpr (MR == 1) {
        const float t = wave_sum_xor(acc[0]);
        if (lane == 0) finish(0, t);
    } else {
        wave_sum_xor_scatter<MR>(acc);
#pragma unroll
        for (int s = 0; s < scatter_slots<MR>(); ++s) {
            const int m = scatter_value<MR>(s, lane >> 4);
            if (scatter_leader<MR>(lane) && m < M) finish(m, acc[s]);
        }
    }
}

// ------------------------------------------------------------------ read: expansion + mix
// Workgroup b, HC waves: wave h = stream h, lane l = column c = 64 b + l, whose weight row is
// h H + c (R / VPW packed words, R / G groups). The rows' rank activations are staged in LDS
// (every lane reads the same one: broadcast); the streams' terms meet in LDS and lane l of
// wave 0 adds them in stream order.
template <int BITS, int MR>
__global__ __launch_bounds__(1024) void k_hc_up(HcDev D, int M, const uint16_t* __restrict__ xn,
                                                const float* __restrict__ act, uint16_t* __restrict__ mixed) {
    constexpr int VPW = 32 / BITS;
    extern __shared__ __align__(16) float hc_lds[];
    float* acts = hc_lds;                                     // [M][R]
    float* terms = hc_lds + static_cast<size_t>(MR) * D.R;    // [MR][HC][64]
    const int tid = threadIdx.x, lane = tid & 63, h = tid >> 6;
    const int H = D.H, R = D.R, HC = D.HC;
    for (int i = tid; i < M * R; i += 64 * HC) acts[i] = act[i];
    const int c = blockIdx.x * 64 + lane;
    const size_t wrow = static_cast<size_t>(h) * H + c;
    const int words = R / VPW, groups = R / D.G;
    const uint32_t* W = D.uw + wrow * words;
    const uint16_t* S = D.us + wrow * groups;
    const uint16_t* Bi = D.ub + wrow * groups;
    lds_barrier();
    float acc[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = 0.0f;
    for (int j4 = 0; j4 < words; j4 += 4) {
        const uint4 q = *reinterpret_cast<const uint4*>(W + j4);
        const uint32_t w4[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r0 = (j4 + i) * VPW, g = r0 / D.G;
            float wq[VPW];
            dequant_word<BITS>(w4[i], bf2f(S[g]), bf2f(Bi[g]), wq);
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                const int mm = m < M ? m : M - 1;
#pragma unroll
                for (int t = 0; t < VPW; ++t) acc[m] = fmaf(acts[mm * R + r0 + t], wq[t], acc[m]);
            }
        }
    }
#pragma unroll
    for (int m = 0; m < MR; ++m)
        if (m < M) {
            const float u = rbf(acc[m]);
            const float gate = rbf(sigmoid_f(u));
            const float x = bf2f(xn[(static_cast<size_t>(m) * HC + h) * H + c]);
            terms[(m * HC + h) * 64 + lane] = rbf(gate * x);
        }
    lds_barrier();
    if (h == 0) {
        for (int m = 0; m < M; ++m) {
            float s = 0.0f;
            for (int hh = 0; hh < HC; ++hh) s += terms[(m * HC + hh) * 64 + lane];
            mixed[static_cast<size_t>(m) * H + c] = f2bf(rbf(s) / static_cast<float>(HC));
        }
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
    e = launch(k_hc_down<BITS, MR>, dim3((n_out + 3) / 4), dim3(256), 0, st, D, M, xn, act, inj);
    if (e != hipSuccess) return e;
    const size_t lds = (static_cast<size_t>(MR) * D.R + static_cast<size_t>(MR) * D.HC * 64) * sizeof(float);
    if ((e = ensure_lds<k_hc_up<BITS, MR>>(hc_up_lds_max())) != hipSuccess) return e;
    return launch(k_hc_up<BITS, MR>, dim3(D.H / 64), dim3(64 * D.HC), lds, st, D, M, xn, act, mixed);
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
    return (static_cast<size_t>(kMaxRows) * kHcMaxRank + static_cast<size_t>(kMaxRows) * kHcMaxStreams * 64) *
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
