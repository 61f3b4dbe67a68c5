// q38_head.hip — gfx950 kernels of the verify tail: the Q8 target LM head with an exact
// greedy argmax (R12, R13), the Q4/g64 draft head logits (R14), and rejection-sampling
// acceptance (R16), and the row argmax + FC join of the MTP draft head.
//
// Greedy argmax. The reference takes argmax_all over MLX quantized_matmul logits
// (src/model.cpp:470-480, src/mtp_verifier.cpp:30-55). Greedy acceptance must be
// bit-exact, so the argmax is defined on an exact logit contract (double partial sums in
// a fixed order, see oracle/q38_oracle.cpp head_q8_logit) and computed in two passes:
//   1. k_head_i8: the bandwidth pass. Every int8 vocab row is read once and multiplied
//      with all request rows on the int8 matrix cores; per-row maxima are kept.
//   2. k_head_cand + k_head_exact: every vocab row whose fast logit lies within twice a
//      proven bound of the fast pass's error of the row maximum is recomputed under the
//      contract and the best (logit desc, index asc) key wins. The true contract argmax
//      always lies in that window, so the result equals the contract argmax; the window
//      holds one or a few rows in practice. More than kHeadCap candidates fall back to
//      recomputing all rows of that request row.
//
// Fast pass arithmetic. k_head_prep writes each request row h (bf16) as three int8
// planes, h ~= s * (a + b / 2^7 + c / 2^14), s = 2^(e-6) with max|h| = f * 2^e, so that
// |a|, |b|, |c| <= 64 and the planes are exact for every element with
// |h| >= s * 2^-6; R = sum |h - s (a + b/2^7 + c/2^14)| is measured exactly (double).
// The MFMA sums sum_k w_k a_k (etc.) are exact int32; A * 2^14 + B * 2^7 + C is exact in
// int64 and, scaled by s * 2^-14 and the fp16 row scale, exact in double, so the fast
// logit is the float rounding of scale_v * sum_k w_k h^_k, and
//   |fast_v - contract_v| <= s_max * 128 * (R + 2^-22 * (sum|h| + R)),
// which head_window doubles.
#include "q38_device.hpp"
#include "q38_internal.hpp"

#include <algorithm>

namespace q38 {

namespace {
constexpr size_t al256(size_t b) { return (b + 255) / 256 * 256; }
}

size_t head_work_bytes(const HeadDev& hd, int M, bool greedy) {
    size_t b = al256(3ull * M * hd.H) + 7 * 256;  // planes; hscale, res, tsum, rowmax, cnt, best
    if (greedy) b += al256(static_cast<size_t>(M) * kHeadCap * 4) + al256(static_cast<size_t>(M) * hd.V * 4);
    return b;
}
HeadWork head_work_carve(void* base, const HeadDev& hd, int M, bool greedy) {
    char* p = static_cast<char*>(base);
    HeadWork w{};
    w.planes = reinterpret_cast<int8_t*>(p); p += al256(3ull * M * hd.H);
    w.hscale = reinterpret_cast<float*>(p); p += 256;
    w.res = reinterpret_cast<float*>(p); p += 256;
    w.tsum = reinterpret_cast<float*>(p); p += 256;
    w.rowmax = reinterpret_cast<uint32_t*>(p); p += 256;
    w.cnt = reinterpret_cast<int32_t*>(p); p += 256;
    w.best = reinterpret_cast<unsigned long long*>(p); p += 256;
    if (greedy) {
        w.cand = reinterpret_cast<int32_t*>(p); p += al256(static_cast<size_t>(M) * kHeadCap * 4);
        w.fast = reinterpret_cast<float*>(p);
    }
    return w;
}

// The int8 planes of one request row hr (H values, global or LDS), its plane scale, the
// residual R and sum|h| (double, fixed order), and the reset of the pass state for row r of
// an M-row call (kernel stores, no memset nodes, so the sequence can be captured in a graph).
// Called by every thread of a workgroup of 256 or more (threads past 256 take no part but
// the barriers); may be called repeatedly in one workgroup.
__device__ void head_prep_row(const uint16_t* hr, int H, int M, int r, const HeadWork& w) {
    __shared__ float redm[4];
    __shared__ double redt[4], redr[4];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int cend = tid < 256 ? H : 0;
    float m = 0.0f;
    for (int c = tid; c < cend; c += 256) m = fmaxf(m, fabsf(bf2f(hr[c])));
    m = wave_max(m);
    if (lane == 0 && wv < 4) redm[wv] = m;
    __syncthreads();
    m = fmaxf(fmaxf(redm[0], redm[1]), fmaxf(redm[2], redm[3]));
    int e = 0;
    (void)frexpf(m, &e);
    const float s = m > 0.0f ? ldexpf(1.0f, e - 6) : 1.0f;
    const double sd = s;
    double tsum = 0.0, res = 0.0;
    for (int c = tid; c < cend; c += 256) {
        const double x = bf2f(hr[c]);
        const double y = x / sd;                  // exact: power-of-two scale, |y| < 64
        const double a = rint(y);
        const double t1 = (y - a) * 128.0;        // |t1| <= 64
        const double b = rint(t1);
        const double t2 = (t1 - b) * 128.0;
        const double cc = rint(t2);
        w.planes[(static_cast<size_t>(0) * M + r) * H + c] = static_cast<int8_t>(a);
        w.planes[(static_cast<size_t>(1) * M + r) * H + c] = static_cast<int8_t>(b);
        w.planes[(static_cast<size_t>(2) * M + r) * H + c] = static_cast<int8_t>(cc);
        tsum += fabs(x);
        res += fabs(x - sd * (a + b * 0x1.0p-7 + cc * 0x1.0p-14));
    }
    tsum = wave_sum_xor(tsum);
    res = wave_sum_xor(res);
    if (lane == 0 && wv < 4) { redt[wv] = tsum; redr[wv] = res; }
    __syncthreads();
    if (tid == 0) {
        // rounded up so that the window bound stays an upper bound
        w.tsum[r] = static_cast<float>(((redt[0] + redt[1]) + (redt[2] + redt[3])) * (1.0 + 0x1.0p-20));
        w.res[r] = static_cast<float>(((redr[0] + redr[1]) + (redr[2] + redr[3])) * (1.0 + 0x1.0p-20));
        w.hscale[r] = s;
        w.rowmax[r] = 0u;
        w.cnt[r] = 0;
        w.best[r] = 0ull;
    }
    __syncthreads();
}

// One block per request row.
__global__ __launch_bounds__(256) void k_head_prep(const uint16_t* __restrict__ h, int H, int M, HeadWork w) {
    head_prep_row(h + static_cast<size_t>(blockIdx.x) * H, H, M, blockIdx.x, w);
}

// Fast pass on v_mfma_i32_16x16x64_i8. A tile is 16 vocab rows; the TB groups of four
// waves of a block take one tile each, and the four waves of a group split the tile's K
// range into quarters. Lane (i = l % 16, q = l / 16) of wave wq loads, for step s, the 16
// weight bytes of row i at columns wq * H/4 + 64 s + 16 q (the MFMA A operand, used as
// loaded); B is the same columns of the three request planes, the same for every tile, so
// each lane holds its B operands in registers for the whole launch. The weights and row
// scales of the group's next tile are loaded before the cross-wave reduction of the
// current one. Output lane (vocab 4q + r, request row i).
typedef int i4_t __attribute__((ext_vector_type(4)));

// Two blocks per CU (2 waves per SIMD): room for the B operands in registers, and 8 tiles of
// weight loads in flight per CU.
constexpr int kHeadBlocksPerCu = 2;

template <int NS, int MR, int TB>
__global__ __launch_bounds__(256 * TB) __attribute__((amdgpu_waves_per_eu(MR == 4 ? kHeadBlocksPerCu : 2)))
void k_head_i8(HeadDev hd, int M, HeadWork w, float* __restrict__ out_logits) {
    constexpr int H = 256 * NS;
    __shared__ long long red[2][TB][4][4][MR][4];  // [buffer][group][wave][q][row][r]
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = (tid >> 6) & 3, grp = tid >> 8, i16 = lane & 15, q = lane >> 4;
    const int jj = i16 < M ? i16 : 0;
    const int64_t V = hd.V;
    const int64_t tiles = (V + 15) / 16;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * TB;
    uint4 wv[NS];
    uint16_t sv[4];  // raw fp16 row scales of vocab rows 4q + r of the tile
    auto load = [&](int64_t tt) {
        int64_t vr = tt * 16 + i16;
        if (vr >= V) vr = V - 1;  // ragged last tile: a valid row, never stored
        const uint4* src = reinterpret_cast<const uint4*>(hd.w + vr * H + wave * (H / 4)) + q;
#pragma unroll
        for (int k = 0; k < NS; ++k) wv[k] = src[4 * k];
        if (wave == 0) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                int64_t v = tt * 16 + 4 * q + r;
                if (v >= V) v = V - 1;
                sv[r] = hd.scales[v];
            }
        }
    };
    int64_t base = static_cast<int64_t>(blockIdx.x) * TB;
    if (base + grp < tiles) load(base + grp);
    i4_t bq[NS][3];
    {
        const int8_t* pb = w.planes + static_cast<size_t>(jj) * H + wave * (H / 4) + 16 * q;
#pragma unroll
        for (int k = 0; k < NS; ++k)
#pragma unroll
            for (int p = 0; p < 3; ++p)
                bq[k][p] = *reinterpret_cast<const i4_t*>(pb + static_cast<size_t>(p) * M * H + 64 * k);
    }
    const bool jact = i16 < M;
    const double hsc = jact ? static_cast<double>(w.hscale[i16]) * 0x1.0p-14 : 0.0;
    float* dst = out_logits ? out_logits : w.fast;
    float mx = -INFINITY;
    int buf = 0;
    for (; base < tiles; base += stride) {  // trip count uniform over the block
        const int64_t t = base + grp;
        i4_t a0 = {0, 0, 0, 0}, a1 = {0, 0, 0, 0}, a2 = {0, 0, 0, 0};
        if (t < tiles) {
#pragma unroll
            for (int k = 0; k < NS; ++k) {
                const i4_t av = __builtin_bit_cast(i4_t, wv[k]);
                a0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bq[k][0], a0, 0, 0, 0);
                a1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bq[k][1], a1, 0, 0, 0);
                a2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bq[k][2], a2, 0, 0, 0);
            }
        }
        uint16_t sc[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) sc[r] = sv[r];
        if (t < tiles && t + stride < tiles) load(t + stride);
        if (i16 < MR) {
#pragma unroll
            for (int r = 0; r < 4; ++r)
                red[buf][grp][wave][q][i16][r] = static_cast<long long>(a0[r]) * 16384 +
                                                 static_cast<long long>(a1[r]) * 128 + a2[r];
        }
        __syncthreads();
        if (wave == 0 && jact && t < tiles) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t v = t * 16 + 4 * q + r;
                if (v < V) {
                    const long long acc = (red[buf][grp][0][q][i16][r] + red[buf][grp][1][q][i16][r]) +
                                          (red[buf][grp][2][q][i16][r] + red[buf][grp][3][q][i16][r]);
                    const float lg =
                        static_cast<float>(static_cast<double>(h2f(sc[r])) * (static_cast<double>(acc) * hsc));
                    mx = fmaxf(mx, lg);
                    dst[static_cast<size_t>(i16) * V + v] = lg;
                }
            }
        }
        buf ^= 1;  // the other buffer is free: its readers passed this iteration's barrier
    }
    if (!out_logits) {
        // one atomic per request row and group: the four lanes of a row (q) merged first
        // (same-address atomics from every lane of the grid serialise at the kernel's end)
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        if (wave == 0 && jact && q == 0) atomicMax(&w.rowmax[i16], orderable(mx));
    }
}

// Window: fast >= max - 2E with E = 2 * s_max * 128 * (R + 2^-22 (sum|h| + R)), twice the
// bound on |fast - contract| derived above (|w| <= 128 for int8 weights).
__device__ __forceinline__ float head_window(const HeadDev& hd, const HeadWork& w, int r) {
    const float E = 2.0f * hd.s_max * 128.0f * (w.res[r] + 0x1.0p-22f * (w.tsum[r] + w.res[r])) + 1e-30f;
    return from_orderable(w.rowmax[r]) - 2.0f * E;
}

__global__ __launch_bounds__(256) void k_head_cand(HeadDev hd, int M, HeadWork w) {
    const int64_t total = static_cast<int64_t>(M) * hd.V;
    for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < total; i += static_cast<int64_t>(gridDim.x) * 256) {
        const int r = static_cast<int>(i / hd.V);
        const int64_t v = i % hd.V;
        if (w.fast[i] >= head_window(hd, w, r)) {
            const int slot = atomicAdd(&w.cnt[r], 1);
            if (slot < kHeadCap) w.cand[r * kHeadCap + slot] = static_cast<int32_t>(v);
        }
    }
}

// Exact contract logit of vocab row v for request row r: lane l sums w[64j+l]*h[64j+l]
// in double for j = 0.. in order, xor butterfly, float(double(scale) * dot).
__device__ __forceinline__ float head_exact_logit(const HeadDev& hd, const uint16_t* h, int64_t v, int lane) {
    const int8_t* row = hd.w + v * hd.H;
    double acc = 0.0;
    for (int j = 0; j * 64 + lane < hd.H; ++j) {
        const int c = j * 64 + lane;
        acc += static_cast<double>(row[c]) * static_cast<double>(bf2f(h[c]));
    }
    acc = wave_sum_xor(acc);
    return static_cast<float>(static_cast<double>(h2f(hd.scales[v])) * acc);
}

__global__ __launch_bounds__(256) void k_head_exact(HeadDev hd, const uint16_t* __restrict__ h, HeadWork w) {
    const int r = blockIdx.y;
    const int lane = threadIdx.x & 63;
    const int gw = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int nw = gridDim.x * 4;
    const int n = w.cnt[r];
    const uint16_t* hrow = h + static_cast<size_t>(r) * hd.H;
    unsigned long long best = 0ull;
    if (n <= kHeadCap) {
        for (int i = gw; i < n; i += nw) {
            const int64_t v = w.cand[r * kHeadCap + i];
            const float lg = head_exact_logit(hd, hrow, v, lane);
            const unsigned long long key = (static_cast<unsigned long long>(orderable(lg)) << 32) |
                                           (0xFFFFFFFFull - static_cast<unsigned long long>(v));
            best = key > best ? key : best;
        }
    } else {
        for (int64_t v = gw; v < hd.V; v += nw) {
            const float lg = head_exact_logit(hd, hrow, v, lane);
            const unsigned long long key = (static_cast<unsigned long long>(orderable(lg)) << 32) |
                                           (0xFFFFFFFFull - static_cast<unsigned long long>(v));
            best = key > best ? key : best;
        }
    }
    if (lane == 0 && best) atomicMax(&w.best[r], best);
}

__global__ void k_head_final(int M, HeadWork w, uint32_t* __restrict__ argmax, float* __restrict__ logit) {
    const int r = threadIdx.x;
    if (r >= M) return;
    const unsigned long long b = w.best[r];
    argmax[r] = 0xFFFFFFFFu - static_cast<uint32_t>(b);
    logit[r] = from_orderable(static_cast<uint32_t>(b >> 32));
}

// Q4/g64 draft head logits: signed nibbles (low first), u = nibble ^ 8 = w + 8, bias
// removed per 32-column lane span with the span's sum of h. The products run on
// v_dot2_f32_f16: each nibble becomes the fp16 value 1 + u/16 (exact; products with the fp16
// copy of h are exact in fp32), so sum w h = 16 sum (1 + u/16) h - 24 sum h. Lane l owns columns
// [32l, 32l + 32) (half a scale group) of every row; a wave takes 8 vocab rows per step and
// has the next step's 8 rows (weights and scales) in flight while it computes. The 8 x M
// per-lane partials are reduce-scattered across the wave (each butterfly step halves the
// values a lane keeps) instead of one full butterfly per (row, request).
// Reduce-scatter over the wave with DPP / permlane exchanges: at offset O a lane keeps the
// half of its KEEP values selected by (lane & O) and adds the partner's copy of that half;
// once one value is left, plain butterfly steps finish the sum.
template <int O, int KEEP, int NP>
__device__ __forceinline__ void reduce_scatter(float (&part)[NP]) {
    if constexpr (O >= 1) {
        if constexpr (KEEP > 1) {
            constexpr int half = KEEP / 2;
            const bool up = (threadIdx.x & O) != 0;
#pragma unroll
            for (int i = 0; i < half; ++i) {
                const float mine = up ? part[half + i] : part[i];
                const float send = up ? part[i] : part[half + i];
                part[i] = mine + xor_lane_f<O>(send);
            }
            reduce_scatter<O / 2, half, NP>(part);
        } else {
            part[0] += xor_lane_f<O>(part[0]);
            reduce_scatter<O / 2, 1, NP>(part);
        }
    }
}

// part (or null): also each workgroup's argmax key per row, orderable(logit) << 32 | ~index
// as k_argmax_rows forms them (0: none), at part[r * gridDim.x + block]; the consumer takes
// the maximum (no atomics: one address per row would serialise the grid's waves).
template <int M>
__global__ __launch_bounds__(256) void k_head_q4(HeadDev hd, const uint16_t* __restrict__ h,
                                                 float* __restrict__ out_logits, unsigned long long* __restrict__ part) {
    constexpr int CPL = 32, RPS = 8;            // columns per lane, rows per step
    constexpr int N = RPS * M;                  // partials per lane per step
    constexpr int NP = N <= 8 ? 8 : N <= 16 ? 16 : 32;  // padded to a power of two
    typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
    const int lane = threadIdx.x & 63;
    const int64_t gw = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const int64_t nw = static_cast<int64_t>(gridDim.x) * 4;
    const int H = hd.H, G = H / 64;
    const int64_t V = hd.V;
    // h as fp16 pairs in the order the nibbles are paired below: word i of the lane's 16
    // bytes holds columns 8i..8i+7 (nibble n = column 8i + n); pair k = columns (8i+k, 8i+k+4).
    half2_t hp[M][16];
    float hs[M];
#pragma unroll
    for (int r = 0; r < M; ++r) {
        float t[CPL];
        hs[r] = 0.0f;
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            t[c] = bf2f(h[static_cast<size_t>(r) * H + CPL * lane + c]);
            hs[r] += t[c];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int k = 0; k < 4; ++k)
                hp[r][4 * i + k] = half2_t{static_cast<_Float16>(t[8 * i + k]), static_cast<_Float16>(t[8 * i + k + 4])};
    }
    uint4 wq[RPS], wn[RPS];
    uint16_t sq[RPS], sn[RPS];
    auto load = [&](int64_t base, uint4 (&w)[RPS], uint16_t (&sc)[RPS]) {
#pragma unroll
        for (int j = 0; j < RPS; ++j) {
            const int64_t v = base + j < V ? base + j : V - 1;  // a ragged step reads a valid row
            w[j] = reinterpret_cast<const uint4*>(hd.w + v * (H / 2) + (CPL / 2) * lane)[0];
            sc[j] = hd.scales[v * G + lane / 2];
        }
    };
    int64_t base = gw * RPS;
    uint64_t kbest = 0;  // this lane's best key (its values all belong to one row)
    if (base < V) load(base, wq, sq);
    for (; base < V; base += nw * RPS) {
        if (base + nw * RPS < V) load(base + nw * RPS, wn, sn);
        float part[NP];
#pragma unroll
        for (int i = 0; i < NP; ++i) part[i] = 0.0f;
#pragma unroll
        for (int j = 0; j < RPS; ++j) {
            const uint32_t wd[4] = {wq[j].x, wq[j].y, wq[j].z, wq[j].w};
            float acc[M];
#pragma unroll
            for (int r = 0; r < M; ++r) acc[r] = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t bw = wd[i] ^ 0x88888888u;  // u = w + 8 in 0..15
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    // nibbles k and k + 4 into bits 6..9 of the two fp16 halves: 1 + u / 16
                    const uint32_t sh = k < 2 ? bw << (6 - 4 * k) : bw >> (4 * k - 6);
                    const uint32_t pr = (sh & 0x03C003C0u) | 0x3C003C00u;
                    const half2_t wv = __builtin_bit_cast(half2_t, pr);
#pragma unroll
                    for (int r = 0; r < M; ++r) acc[r] = __builtin_amdgcn_fdot2(wv, hp[r][4 * i + k], acc[r], false);
                }
            }
            // sum (w) h = sum (u - 8) h = 16 sum (1 + u/16) h - 24 sum h
            const float sc = h2f(sq[j]);
#pragma unroll
            for (int r = 0; r < M; ++r) part[j * M + r] = sc * fmaf(16.0f, acc[r], -24.0f * hs[r]);
        }
        reduce_scatter<32, NP, NP>(part);
        // the value index a lane holds: its bits of the halving offsets, high offset first
        int idx = 0;
        {
            int bitv = NP / 2;
            for (int o = 32; bitv >= 1; o >>= 1, bitv >>= 1)
                if (lane & o) idx += bitv;
        }
        const int lsb = 64 / NP;  // lanes sharing an index: the low log2(64 / NP) lane bits
        if ((lane & (lsb - 1)) == 0 && idx < N) {
            const int j = idx / M, r = idx % M;
            if (base + j < V) {
                out_logits[static_cast<size_t>(r) * V + base + j] = part[0];
                const uint64_t k = (static_cast<uint64_t>(orderable(part[0])) << 32) |
                                   (0xFFFFFFFFu - static_cast<uint32_t>(base + j));
                kbest = k > kbest ? k : kbest;
            }
        }
#pragma unroll
        for (int j = 0; j < RPS; ++j) {
            wq[j] = wn[j];
            sq[j] = sn[j];
        }
    }
    if (part) {
        __shared__ uint64_t wk[4][M];
        int idx = 0;
        {
            int bitv = NP / 2;
            for (int o = 32; bitv >= 1; o >>= 1, bitv >>= 1)
                if (lane & o) idx += bitv;
        }
#pragma unroll
        for (int r = 0; r < M; ++r) {
            const uint64_t k = wave_max_u64(idx % M == r ? kbest : 0);
            if (lane == 0) wk[threadIdx.x >> 6][r] = k;
        }
        __syncthreads();
        if (threadIdx.x < M) {
            const int r = threadIdx.x;
            uint64_t k = wk[0][r];
#pragma unroll
            for (int w = 1; w < 4; ++w) k = wk[w][r] > k ? wk[w][r] : k;
            part[static_cast<size_t>(r) * gridDim.x + blockIdx.x] = k;
        }
    }
}

// The maximum of n partial keys (block-wide; every thread gets it).
__device__ __forceinline__ uint64_t max_keys(const unsigned long long* p, int n) {
    __shared__ uint64_t wk[16];  // (up to 1024 threads)
    uint64_t k = 0;
    for (int i = threadIdx.x; i < n; i += blockDim.x) k = p[i] > k ? p[i] : k;
    k = wave_max_u64(k);
    if ((threadIdx.x & 63) == 0) wk[threadIdx.x >> 6] = k;
    __syncthreads();
    k = wk[0];
    for (int w = 1; w < static_cast<int>(blockDim.x >> 6); ++w) k = wk[w] > k ? wk[w] : k;
    return k;
}

// Row r's key from the Q4 head's partials, decoded as k_argmax_final does.
__global__ __launch_bounds__(256) void k_argmax_part_final(const unsigned long long* __restrict__ part, int n,
                                                           uint32_t* __restrict__ tokens, float* __restrict__ values,
                                                           uint32_t* __restrict__ drafts, int depth, int step) {
    const int r = blockIdx.x;
    const uint64_t b = max_keys(part + static_cast<size_t>(r) * n, n);
    if (threadIdx.x != 0) return;
    const uint32_t t = 0xFFFFFFFFu - static_cast<uint32_t>(b);
    if (tokens) tokens[r] = t;
    if (values) values[r] = from_orderable(static_cast<uint32_t>(b >> 32));
    if (drafts) drafts[static_cast<size_t>(r) * depth + step] = t;
}

__global__ void k_gen_head(HeadDev hd, uint64_t wkey, uint64_t skey, int8_t* __restrict__ w,
                           uint16_t* __restrict__ scales) {
    const int64_t H = hd.H;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    const int64_t t0 = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (hd.kind == 0) {
        const int64_t n = hd.V * H;
        for (int64_t i = t0; i < n; i += stride)
            w[i] = static_cast<int8_t>(static_cast<int>(((bits_at(wkey, i) >> 32) * 255ull) >> 32) - 127);
        for (int64_t v = t0; v < hd.V; v += stride) scales[v] = f2h(uniform_f32(skey, v, 1e-4, 1e-3));
    } else {
        const int64_t n = hd.V * H / 2;
        for (int64_t i = t0; i < n; i += stride) {
            const int lo = static_cast<int>(bits_at(wkey, 2 * i) >> 60) - 8;
            const int hi = static_cast<int>(bits_at(wkey, 2 * i + 1) >> 60) - 8;
            w[i] = static_cast<int8_t>((lo & 0xf) | ((hi & 0xf) << 4));
        }
        const int64_t ns = hd.V * (H / 64);
        for (int64_t i = t0; i < ns; i += stride) scales[i] = f2h(uniform_f32(skey, i, 1.6e-3, 1.6e-2));
    }
}

__global__ void k_scale_absmax(const uint16_t* __restrict__ s, int64_t n, float* out) {
    __shared__ float red[16];
    float m = 0.0f;
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) m = fmaxf(m, fabsf(h2f(s[i])));
    m = wave_max(m);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        float t = 0.0f;
        for (int i = 0; i < static_cast<int>(blockDim.x >> 6); ++i) t = fmaxf(t, red[i]);
        *out = t;
    }
}

// ---------------------------------------------------------------- rejection sampling
// Spread over the chip in four launches (graph-capturable, no host round trip):
//   k_samp_stats   (chunks x rows) workgroups: online softmax partials (max, sum exp) of each
//                  256-thread chunk of every target row 0..k and draft row 0..k-1;
//   k_samp_decide  one wave: each row's (max, sum) from its partials in a fixed tree order,
//                  then the accept test of drafts 0..k-1 in order (u * q(d) < p(d));
//   k_samp_mass    one workgroup per chunk: the residual mass max(0, p - q) of the first
//                  rejected position (or p of the bonus row) per chunk, and the chunk's last
//                  positive index;
//   k_samp_draw    one workgroup: the chunk where the inclusive prefix first exceeds v * total,
//                  then the index inside it (thread sub-ranges in index order); when rounding
//                  leaves no crossing, the last index with positive mass.
// Every sum runs in a fixed order, so a call is deterministic.
namespace {
constexpr int kSampChunks = 64;  // chunks per row (fewer for small vocabularies)

struct SampCtl {
    int32_t row;       // first rejected position, or k (all accepted: the bonus row)
    float v;           // the residual draw's uniform
    float pm, ps;      // target row stats (max, sum exp) of `row`
    float qm, qs;      // draft row stats (row < k)
};

__device__ __forceinline__ void softmax_merge(float& m, float& s, float m2, float s2, float invT) {
    if (m2 == -INFINITY) return;
    if (m == -INFINITY) { m = m2; s = s2; return; }
    if (m2 > m) {
        s = s * expf((m - m2) * invT) + s2;
        m = m2;
    } else {
        s += s2 * expf((m2 - m) * invT);
    }
}

__global__ __launch_bounds__(256) void k_samp_stats(const float* __restrict__ tl, const float* __restrict__ dl, int k,
                                                    int64_t V, int64_t cs, float invT, float2* __restrict__ part) {
    __shared__ float2 sh[4];
    const int c = blockIdx.x, r = blockIdx.y, tid = threadIdx.x;
    const float* l = r <= k ? tl + static_cast<int64_t>(r) * V : dl + static_cast<int64_t>(r - k - 1) * V;
    const int64_t a = static_cast<int64_t>(c) * cs, b = a + cs < V ? a + cs : V;
    float m = -INFINITY, s = 0.0f;
    auto take = [&](float v) {
        if (!(v > -INFINITY)) return;  // a -inf logit has probability 0
        if (v > m) {
            s = (m == -INFINITY ? 0.0f : s * expf((m - v) * invT)) + 1.0f;
            m = v;
        } else {
            s += expf((v - m) * invT);
        }
    };
    int64_t x = a + tid;
    for (; x + 3 * 256 < b; x += 4 * 256) {  // four loads in flight, taken in index order
        const float v0 = l[x], v1 = l[x + 256], v2 = l[x + 512], v3 = l[x + 768];
        take(v0);
        take(v1);
        take(v2);
        take(v3);
    }
    for (; x < b; x += 256) take(l[x]);
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const float m2 = __shfl_xor(m, off, kWave), s2 = __shfl_xor(s, off, kWave);
        softmax_merge(m, s, m2, s2, invT);
    }
    if ((tid & 63) == 0) sh[tid >> 6] = make_float2(m, s);
    __syncthreads();
    if (tid == 0) {
        float M = sh[0].x, S = sh[0].y;
        for (int w = 1; w < 4; ++w) softmax_merge(M, S, sh[w].x, sh[w].y, invT);
        part[static_cast<size_t>(r) * gridDim.x + c] = make_float2(M, S);
    }
}

__global__ __launch_bounds__(64) void k_samp_decide(const float* __restrict__ tl, const float* __restrict__ dl,
                                                    const uint32_t* __restrict__ drafts, int k, int64_t V, int nc,
                                                    float invT, uint64_t seed, uint64_t slot, uint64_t round,
                                                    const float2* __restrict__ part, SampCtl* __restrict__ ctl) {
    __shared__ float2 st[2 * 24 + 1];
    const int lane = threadIdx.x;
    for (int r = 0; r < 2 * k + 1; ++r) {
        float m = -INFINITY, s = 0.0f;
        if (lane < nc) {
            const float2 p = part[static_cast<size_t>(r) * nc + lane];
            m = p.x;
            s = p.y;
        }
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const float m2 = __shfl_xor(m, off, kWave), s2 = __shfl_xor(s, off, kWave);
            softmax_merge(m, s, m2, s2, invT);
        }
        if (lane == 0) st[r] = make_float2(m, s);
    }
    __syncthreads();
    // lane i: position i's uniforms and p(d_i), q(d_i) (all positions at once), then lane 0
    // walks the accept chain in order
    __shared__ float su[25], sv[25], spd[24], sqd[24];
    if (lane <= k) {
        float u, v;
        round_uniforms(seed, slot, round, static_cast<uint32_t>(lane), &u, &v);
        su[lane] = u;
        sv[lane] = v;
        if (lane < k) {
            const float2 ps = st[lane], qs = st[k + 1 + lane];
            const uint32_t d = drafts[lane];
            // an out-of-vocabulary draft is rejected (never read out of bounds)
            spd[lane] = d < V ? expf((tl[static_cast<int64_t>(lane) * V + d] - ps.x) * invT) / ps.y : 0.0f;
            sqd[lane] = d < V ? expf((dl[static_cast<int64_t>(lane) * V + d] - qs.x) * invT) / qs.y : 1.0f;
        }
    }
    __syncthreads();
    if (lane != 0) return;
    for (int i = 0; i <= k; ++i) {
        const float2 ps = st[i];
        if (i == k) {
            *ctl = SampCtl{k, sv[i], ps.x, ps.y, 0.0f, 1.0f};
            return;
        }
        if (su[i] * sqd[i] < spd[i]) continue;
        const float2 qs = st[k + 1 + i];
        *ctl = SampCtl{i, sv[i], ps.x, ps.y, qs.x, qs.y};
        return;
    }
}

// The residual weights of indices x0 .. x1 - 1 in index order, 8 indices' logits loaded at a
// time; f(x, w) returns true to stop.
template <typename F>
__device__ __forceinline__ void samp_weights(const float* tl, const float* dl, int k, int64_t V, const SampCtl& c,
                                             float invT, int64_t x0, int64_t x1, F&& f) {
    const float* pr = tl + static_cast<int64_t>(c.row) * V;
    const float* qr = c.row == k ? pr : dl + static_cast<int64_t>(c.row) * V;
    for (int64_t x = x0; x < x1; x += 8) {
        float pl[8], ql[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int64_t xi = x + j < x1 ? x + j : x1 - 1;
            pl[j] = pr[xi];
            ql[j] = qr[xi];
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if (x + j >= x1) return;
            const float p = expf((pl[j] - c.pm) * invT) / c.ps;
            const float w = c.row == k ? p : fmaxf(0.0f, p - expf((ql[j] - c.qm) * invT) / c.qs);
            if (f(x + j, w)) return;
        }
    }
}

// Thread t of a chunk owns the contiguous sub-range [a + t * sub, a + (t + 1) * sub).
__device__ __forceinline__ void samp_range(int64_t a, int64_t b, int64_t sub, int t, int64_t& x0, int64_t& x1) {
    x0 = a + t * sub < b ? a + t * sub : b;
    x1 = x0 + sub < b ? x0 + sub : b;
}

__device__ float block_sum_ordered(float v, float* sh) {
    v = wave_sum_xor(v);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
    __syncthreads();
    const float t = (sh[0] + sh[1]) + (sh[2] + sh[3]);
    __syncthreads();
    return t;
}

__global__ __launch_bounds__(256) void k_samp_mass(const float* __restrict__ tl, const float* __restrict__ dl, int k,
                                                   int64_t V, int64_t cs, float invT, const SampCtl* __restrict__ ctl,
                                                   float* __restrict__ csum, int64_t* __restrict__ clast) {
    __shared__ float sh[4];
    __shared__ unsigned long long last;
    const SampCtl c = *ctl;
    const int64_t a = static_cast<int64_t>(blockIdx.x) * cs, b = a + cs < V ? a + cs : V;
    const int64_t sub = (cs + 255) / 256;
    int64_t x0, x1;
    samp_range(a, b, sub, threadIdx.x, x0, x1);
    if (threadIdx.x == 0) last = 0ull;
    __syncthreads();
    float s = 0.0f;
    int64_t lp = -1;
    samp_weights(tl, dl, k, V, c, invT, x0, x1, [&](int64_t x, float w) {
        s += w;
        if (w > 0.0f) lp = x;
        return false;
    });
    if (lp >= 0) atomicMax(&last, static_cast<unsigned long long>(lp + 1));
    const float t = block_sum_ordered(s, sh);
    if (threadIdx.x == 0) {
        csum[blockIdx.x] = t;
        clast[blockIdx.x] = static_cast<int64_t>(last) - 1;
    }
}

__global__ __launch_bounds__(256) void k_samp_draw(const float* __restrict__ tl, const float* __restrict__ dl, int k,
                                                   int64_t V, int64_t cs, int nc, float invT,
                                                   const SampCtl* __restrict__ ctl, const float* __restrict__ csum,
                                                   const int64_t* __restrict__ clast, int64_t* __restrict__ out) {
    __shared__ float pre[256];
    __shared__ float cs_l[kSampChunks];
    __shared__ int chunk;
    __shared__ float base, target;
    __shared__ unsigned long long found;
    const SampCtl c = *ctl;
    const int tid = threadIdx.x;
    if (tid < nc) cs_l[tid] = csum[tid];
    __syncthreads();
    if (tid == 0) {
        float total = 0.0f;
        for (int i = 0; i < nc; ++i) total += cs_l[i];
        const float tg = c.v * total;
        float run = 0.0f;
        int ch = -1;
        for (int i = 0; i < nc; ++i) {
            if (cs_l[i] > 0.0f && run <= tg && tg < run + cs_l[i]) {
                ch = i;
                break;
            }
            run += cs_l[i];
        }
        chunk = ch;
        base = run;
        target = tg;
        found = ~0ull;
    }
    __syncthreads();
    int64_t pick = -1;
    if (chunk >= 0) {
        const int64_t a = static_cast<int64_t>(chunk) * cs, b = a + cs < V ? a + cs : V;
        const int64_t sub = (cs + 255) / 256;
        int64_t x0, x1;
        samp_range(a, b, sub, tid, x0, x1);
        float s = 0.0f;
        samp_weights(tl, dl, k, V, c, invT, x0, x1, [&](int64_t, float w) {
            s += w;
            return false;
        });
        pre[tid] = s;
        __syncthreads();
        if (tid == 0) {  // exclusive prefix over the threads, in index order
            float run = base;
            for (int t = 0; t < 256; ++t) {
                const float w = pre[t];
                pre[t] = run;
                run += w;
            }
        }
        __syncthreads();
        const float excl = pre[tid];
        if (s > 0.0f && excl <= target && target < excl + s) {
            float run = excl;
            int64_t p = -1;
            samp_weights(tl, dl, k, V, c, invT, x0, x1, [&](int64_t x, float w) {
                run += w;
                if (w > 0.0f) p = x;  // the last positive so far: the fallback of this range
                return run > target && w > 0.0f;
            });
            if (p >= 0) atomicMin(&found, static_cast<unsigned long long>(p));
        }
        __syncthreads();
        if (found != ~0ull) pick = static_cast<int64_t>(found);
    }
    if (tid == 0) {
        if (pick < 0) {  // no crossing under rounding: the last index with positive mass
            int64_t lp = -1;
            for (int i = 0; i < nc; ++i) lp = clast[i] > lp ? clast[i] : lp;
            pick = lp < 0 ? 0 : lp;
        }
        out[0] = c.row;
        out[1] = pick;
    }
}
} // namespace

// ---------------------------------------------------------------- launchers
namespace {

int cu_count() {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1)
        n = 256;
    return n;
}

// Request rows <= 4: one tile per block; up to 16 rows: two tiles per block (16-row B).
template <int NS, int MR, int TB>
hipError_t launch_i8_t(const HeadDev& hd, int M, const HeadWork& w, float* out, hipStream_t st) {
    const int64_t tiles = (hd.V + 15) / 16;
    int64_t grid = static_cast<int64_t>(cu_count()) * (MR == 4 ? kHeadBlocksPerCu : 1);
    if (grid > (tiles + TB - 1) / TB) grid = (tiles + TB - 1) / TB;
    return launch(k_head_i8<NS, MR, TB>, dim3(static_cast<unsigned>(grid)), dim3(256 * TB), 0, st, hd, M, w, out);
}
hipError_t launch_i8(const HeadDev& hd, int M, const HeadWork& w, float* out, hipStream_t st) {
    const bool wide = M > 4;
    switch (hd.H) {
        case 1024: return wide ? launch_i8_t<4, 16, 2>(hd, M, w, out, st) : launch_i8_t<4, 4, 1>(hd, M, w, out, st);
        case 2048: return wide ? launch_i8_t<8, 16, 2>(hd, M, w, out, st) : launch_i8_t<8, 4, 1>(hd, M, w, out, st);
        case 2560: return wide ? launch_i8_t<10, 16, 2>(hd, M, w, out, st) : launch_i8_t<10, 4, 1>(hd, M, w, out, st);
        default: return hipErrorInvalidValue;
    }
}
template <int M>
hipError_t launch_q4_m(const HeadDev& hd, const uint16_t* h, float* out, hipStream_t st,
                       unsigned long long* part = nullptr) {
    // one resident wave per SIMD slot (the kernel holds 4 waves per SIMD at M = 1, 3 at M = 2
    // and 3, 2 at M = 4): every wave streams
    // many 8-row steps, so its prologue (M rows of h) is paid once per ~9 steps
    return launch(k_head_q4<M>, dim3(q4_blocks(M)), dim3(256), 0, st, hd, h, out, part);
}
} // namespace

hipError_t head_init_attrs() { return hipSuccess; }

hipError_t launch_head_greedy(const HeadDev& hd, const uint16_t* h, int M, const HeadWork& w, uint32_t* argmax,
                              float* logit, hipStream_t st) {
    hipError_t e = launch(k_head_prep, dim3(M), dim3(256), 0, st, h, hd.H, M, w);
    if (e != hipSuccess) return e;
    if ((e = launch_i8(hd, M, w, nullptr, st)) != hipSuccess) return e;
    if ((e = launch(k_head_cand, dim3(2048), dim3(256), 0, st, hd, M, w)) != hipSuccess) return e;
    if ((e = launch(k_head_exact, dim3(16, M), dim3(256), 0, st, hd, h, w)) != hipSuccess) return e;
    return launch(k_head_final, dim3(1), dim3(64), 0, st, M, w, argmax, logit);
}

hipError_t launch_head_logits(const HeadDev& hd, const uint16_t* h, int M, const HeadWork& w, float* logits,
                              hipStream_t st) {
    if (hd.kind == 0) {
        const hipError_t e = launch(k_head_prep, dim3(M), dim3(256), 0, st, h, hd.H, M, w);
        if (e != hipSuccess) return e;
        return launch_i8(hd, M, w, logits, st);
    }
    if (hd.H != 2048) return hipErrorInvalidValue;
    switch (M) {
        case 1: return launch_q4_m<1>(hd, h, logits, st);
        case 2: return launch_q4_m<2>(hd, h, logits, st);
        case 3: return launch_q4_m<3>(hd, h, logits, st);
        case 4: return launch_q4_m<4>(hd, h, logits, st);
        default: return hipErrorInvalidValue;
    }
}

int q4_blocks(int M) {
    const int n = cu_count() * (M == 1 ? 4 : M == 4 ? 2 : 3);
    return n < kQ4MaxBlocks ? n : kQ4MaxBlocks;
}

hipError_t launch_head_q4_part(const HeadDev& hd, const uint16_t* h, int M, float* logits, unsigned long long* part,
                               hipStream_t st) {
    if (hd.kind == 0 || hd.H != 2048) return hipErrorInvalidValue;
    switch (M) {
        case 1: return launch_q4_m<1>(hd, h, logits, st, part);
        case 2: return launch_q4_m<2>(hd, h, logits, st, part);
        case 3: return launch_q4_m<3>(hd, h, logits, st, part);
        case 4: return launch_q4_m<4>(hd, h, logits, st, part);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gen_head(const HeadDev& hd, uint64_t seed, int8_t* w, uint16_t* scales, hipStream_t st) {
    const uint64_t wk = stream_key(seed, hd.kind == 0 ? kHeadLayer : kDraftLayer, hd.kind == 0 ? T_HEAD_W : T_DRAFT_W);
    const uint64_t sk = stream_key(seed, hd.kind == 0 ? kHeadLayer : kDraftLayer, hd.kind == 0 ? T_HEAD_S : T_DRAFT_S);
    hipLaunchKernelGGL(k_gen_head, dim3(8192), dim3(256), 0, st, hd, wk, sk, w, scales);
    return hipGetLastError();
}

hipError_t launch_scale_absmax(const uint16_t* scales, int64_t n, float* out, hipStream_t st) {
    hipLaunchKernelGGL(k_scale_absmax, dim3(1), dim3(1024), 0, st, scales, n, out);
    return hipGetLastError();
}

// ---------------------------------------------------------------- draft head helpers
// MTP draft head FC join: x = T(T(a) + T(b)) over n values (the embedding and hidden
// projections, each rounded to bf16, added in bf16: src/mtp_head.cpp:258-266). The sum of two
// bf16 values is exact in fp32 or below half a bf16 ulp of the larger, so one rounding of the
// fp32 sum is the correctly rounded bf16 sum. Also clears best[0..M) for the step's argmax.
// With HC streams a row holds HC stream projections b [M][HC][H] and one embedding
// projection a [M][H], added to every stream (the broadcast of src/mtp_head.cpp:261-266).
__global__ __launch_bounds__(256) void k_fc_join(const float* __restrict__ a, const float* __restrict__ b, int M,
                                                 int HC, int H, uint16_t* __restrict__ x,
                                                 unsigned long long* __restrict__ best) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    const int n = M * HC * H;
    if (i < n) {
        const int r = i / (HC * H), c = i % H;
        x[i] = f2bf(rbf(a[r * H + c]) + rbf(b[i]));
    }
    if (best && i < M) best[i] = 0ull;
}

__global__ void k_fill_u64(unsigned long long* __restrict__ p, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = 0ull;
}

// Row argmax of logits [M, V], ties to the lowest index (src/mtp_verifier.cpp:20-55 with the
// tie rule of src/mlx_backend.cpp:78-85): each thread keeps the largest key
// (orderable(value) << 32 | ~index) of a strided range, the wave reduces, one 64-bit atomic max
// per wave merges into best[row] (which starts at 0, below every key).
__global__ __launch_bounds__(256) void k_argmax_rows(const float* __restrict__ logits, int64_t V,
                                                     unsigned long long* __restrict__ best) {
    const int r = blockIdx.y;
    const float* row = logits + static_cast<int64_t>(r) * V;
    uint64_t k = 0;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < V;
         i += static_cast<int64_t>(gridDim.x) * 256) {
        const uint64_t c = (static_cast<uint64_t>(orderable(row[i])) << 32) | (0xFFFFFFFFu - static_cast<uint32_t>(i));
        k = c > k ? c : k;
    }
    k = wave_max_u64(k);
    if ((threadIdx.x & 63) == 0 && k != 0) atomicMax(&best[r], static_cast<unsigned long long>(k));
}

// Decodes best[r] into tokens[r] (and values[r]); with drafts, also drafts[r * depth + step].
__global__ void k_argmax_final(const unsigned long long* __restrict__ best, int M, uint32_t* __restrict__ tokens,
                               float* __restrict__ values, uint32_t* __restrict__ drafts, int depth, int step) {
    const int r = threadIdx.x;
    if (r >= M) return;
    const unsigned long long b = best[r];
    const uint32_t t = 0xFFFFFFFFu - static_cast<uint32_t>(b);
    if (tokens) tokens[r] = t;
    if (values) values[r] = from_orderable(static_cast<uint32_t>(b >> 32));
    if (drafts) drafts[static_cast<size_t>(r) * depth + step] = t;
}

hipError_t launch_fc_join(const float* a, const float* b, int M, int HC, int H, uint16_t* x, unsigned long long* best,
                          hipStream_t st) {
    const int n = M * HC * H;
    return launch(k_fc_join, dim3((n + 255) / 256), dim3(256), 0, st, a, b, M, HC, H, x, best);
}

// The row argmax keys alone (best must start at 0; no k_argmax_final).
hipError_t launch_argmax_rows(const float* logits, int M, int64_t V, unsigned long long* best, hipStream_t st) {
    if (M < 1 || M > 64 || V < 1) return hipErrorInvalidValue;
    const int64_t blocks = std::min<int64_t>(128, (V + 255) / 256);
    return launch(k_argmax_rows, dim3(static_cast<unsigned>(blocks), M), dim3(256), 0, st, logits, V, best);
}

hipError_t launch_argmax_part_final(const unsigned long long* part, int n, int M, uint32_t* tokens, float* values,
                                    uint32_t* drafts, int depth, int step, hipStream_t st) {
    if (M < 1 || M > 64 || n < 1) return hipErrorInvalidValue;
    return launch(k_argmax_part_final, dim3(M), dim3(256), 0, st, part, n, tokens, values, drafts, depth, step);
}

hipError_t launch_argmax(const float* logits, int M, int64_t V, unsigned long long* best, bool clear,
                         uint32_t* tokens, float* values, uint32_t* drafts, int depth, int step, hipStream_t st) {
    if (M < 1 || M > 64 || V < 1) return hipErrorInvalidValue;
    if (clear) {
        const hipError_t e = launch(k_fill_u64, dim3(1), dim3(256), 0, st, best, M);
        if (e != hipSuccess) return e;
    }
    const int64_t blocks = std::min<int64_t>(128, (V + 255) / 256);
    hipError_t e = launch(k_argmax_rows, dim3(static_cast<unsigned>(blocks), M), dim3(256), 0, st, logits, V, best);
    if (e != hipSuccess) return e;
    return launch(k_argmax_final, dim3(1), dim3(64), 0, st, best, M, tokens, values, drafts, depth, step);
}

// The draft step's inputs of its two FC projections in one launch (the embedding, the two
// RMSNorms and the Q8 planes of both projections' rows), one workgroup per projection row:
// (r, 0) forms request r's embedding row (token toks[r], or, in a chain, the previous step's
// argmax best[r], whose token it also records); (r, 1 + s) takes stream s of request r. Each
// RMS-normalises its row in k_rmsnorm's order (thread t sums the squares of values t, t + 256,
// ... of the whole H or HC * H row in order, then the wave and workgroup sums), the stream
// workgroups each over the whole stream row (read again from L2) but normalising only their
// own H values, with the offset weight when given, and prepares the Q8 planes of that row:
// the embedding row as row r of we, stream s as row g = r HC + s of the stream projection's
// passes (pass g / 16, row g % 16).
__global__ __launch_bounds__(1024) void k_draft_prologue(DraftPro P) {
    extern __shared__ __align__(16) uint16_t row[];  // [H] bf16
    __shared__ float red[4];
    const int r = blockIdx.x, which = blockIdx.y, tid = threadIdx.x;
    const int H = P.H, W = which ? P.HC * H : H;
    float ss = 0.0f;
    if (which == 0) {
        // (the 1024 threads generate the row; its sums stay on the first 256 in k_rmsnorm's order)
        uint32_t t;
        if (P.toks) {
            t = P.toks[r];
        } else {
            const uint64_t b = P.part ? max_keys(P.part + static_cast<size_t>(r) * P.nparts, P.nparts) : P.best[r];
            t = 0xFFFFFFFFu - static_cast<uint32_t>(b);
            if (tid == 0) {
                if (P.tokens_out) P.tokens_out[r] = t;
                if (P.drafts) P.drafts[static_cast<size_t>(r) * P.depth + P.prev_step] = t;
            }
        }
        for (int c = tid; c < H; c += 1024)
            row[c] = f2bf(static_cast<float>(normal_at(P.embed_key, static_cast<uint64_t>(t) * H + c)));
        __syncthreads();
        if (tid < 256)
            for (int c = tid; c < W; c += 256) {
                const float v = bf2f(row[c]);
                ss = fmaf(v, v, ss);
            }
    } else if (tid < 256) {
        // the whole stream row, 16 values per thread in flight, summed in order
        const int s0 = (which - 1) * H;
        const uint16_t* src = P.stream + static_cast<size_t>(r) * W;
        constexpr int B16 = 16;
        for (int c0 = 0; c0 < W; c0 += 256 * B16) {
            uint16_t e[B16];
#pragma unroll
            for (int k = 0; k < B16; ++k) {
                const int c = c0 + tid + 256 * k;
                e[k] = c < W ? src[c] : 0;
            }
#pragma unroll
            for (int k = 0; k < B16; ++k) {
                const int c = c0 + tid + 256 * k;
                if (c < W) {
                    const float v = bf2f(e[k]);
                    ss = fmaf(v, v, ss);
                    if (c >= s0 && c < s0 + H) row[c - s0] = e[k];
                }
            }
        }
    }
    ss = wave_sum_xor(ss);
    if ((tid & 63) == 0 && tid < 256) red[tid >> 6] = ss;
    __syncthreads();
    const float tot = (red[0] + red[1]) + (red[2] + red[3]);
    const float inv = 1.0f / sqrtf(tot / static_cast<float>(W) + P.eps);
    const uint16_t* wn = which ? P.hid_norm + (which - 1) * H : P.emb_norm;
    for (int c = tid; c < H; c += 1024) {
        const float n = rbf(bf2f(row[c]) * inv);
        row[c] = f2bf((which ? P.hid_norm : P.emb_norm) ? n * bf2f(wn[c]) : n);
    }
    __syncthreads();
    if (which == 0) {
        head_prep_row(row, H, P.M, r, P.we);
    } else {
        const int g = r * P.HC + which - 1, pass = g / kHeadMaxRows;
        head_prep_row(row, H, P.mh[pass], g % kHeadMaxRows, P.wh[pass]);
    }
}

hipError_t launch_draft_prologue(const DraftPro& P, hipStream_t st) {
    const size_t lds = static_cast<size_t>(P.H) * 2;
    if (const hipError_t e = ensure_lds<k_draft_prologue>(lds); e != hipSuccess) return e;
    return launch(k_draft_prologue, dim3(P.M, 1 + P.HC), dim3(1024), lds, st, P);
}

hipError_t launch_head_logits_prepared(const HeadDev& hd, int M, const HeadWork& w, float* logits, hipStream_t st) {
    if (hd.kind != 0) return hipErrorInvalidValue;
    return launch_i8(hd, M, w, logits, st);
}

namespace {
struct SampLayout {
    int nc;
    int64_t cs;
    float2* part;
    float* csum;
    int64_t* clast;
    SampCtl* ctl;
    size_t bytes;
};
size_t a256(size_t v) { return (v + 255) / 256 * 256; }
SampLayout samp_layout(int k, int64_t V, void* base) {
    SampLayout L{};
    L.nc = static_cast<int>(std::min<int64_t>(kSampChunks, (V + 255) / 256));
    L.cs = (V + L.nc - 1) / L.nc;
    char* b = static_cast<char*>(base);
    size_t off = 0;
    L.part = reinterpret_cast<float2*>(b + off);
    off += a256(static_cast<size_t>(2 * k + 1) * L.nc * sizeof(float2));
    L.csum = reinterpret_cast<float*>(b + off);
    off += a256(static_cast<size_t>(L.nc) * 4);
    L.clast = reinterpret_cast<int64_t*>(b + off);
    off += a256(static_cast<size_t>(L.nc) * 8);
    L.ctl = reinterpret_cast<SampCtl*>(b + off);
    off += a256(sizeof(SampCtl));
    L.bytes = off;
    return L;
}
} // namespace

size_t accept_sampled_workspace(int k, int64_t V) { return samp_layout(k, V, nullptr).bytes; }

hipError_t launch_accept_sampled(const float* tl, const float* dl, const uint32_t* drafts, int k, int64_t V,
                                 float T, uint64_t seed, uint64_t slot, uint64_t round, int64_t* out, void* ws,
                                 hipStream_t st) {
    const SampLayout L = samp_layout(k, V, ws);
    const float invT = 1.0f / T;
    hipError_t e = launch(k_samp_stats, dim3(L.nc, 2 * k + 1), dim3(256), 0, st, tl, dl, k, V, L.cs, invT, L.part);
    if (e == hipSuccess)
        e = launch(k_samp_decide, dim3(1), dim3(64), 0, st, tl, dl, drafts, k, V, L.nc, invT, seed, slot, round,
                   static_cast<const float2*>(L.part), L.ctl);
    if (e == hipSuccess)
        e = launch(k_samp_mass, dim3(L.nc), dim3(256), 0, st, tl, dl, k, V, L.cs, invT,
                   static_cast<const SampCtl*>(L.ctl), L.csum, L.clast);
    if (e == hipSuccess)
        e = launch(k_samp_draw, dim3(1), dim3(256), 0, st, tl, dl, k, V, L.cs, L.nc, invT,
                   static_cast<const SampCtl*>(L.ctl), static_cast<const float*>(L.csum),
                   static_cast<const int64_t*>(L.clast), out);
    return e;
}

namespace {
// Softmax rows: per row the chunk partials (k_samp_stats) merged in chunk order into
// (max, sum of exp((l - max) / T)); then, when asked, the probabilities.
__global__ __launch_bounds__(64) void k_softmax_stats(const float2* __restrict__ part, int nc, float invT,
                                                      float* __restrict__ stats) {
    if (threadIdx.x != 0) return;
    const int r = blockIdx.x;
    float m = -INFINITY, s = 0.0f;
    for (int c = 0; c < nc; ++c) {
        const float2 v = part[static_cast<size_t>(r) * nc + c];
        softmax_merge(m, s, v.x, v.y, invT);
    }
    stats[2 * r] = m;
    stats[2 * r + 1] = s;
}

// probs[r][x] = exp((l[r][x] - max) / T) / sum (0 for a -inf logit); probs may be l.
__global__ __launch_bounds__(256) void k_softmax_probs(const float* l, int64_t V, int64_t cs, float invT,
                                                      const float* __restrict__ stats, float* probs) {
    const int c = blockIdx.x, r = blockIdx.y;
    const int64_t a = static_cast<int64_t>(c) * cs, b = a + cs < V ? a + cs : V;
    const float m = stats[2 * r], s = stats[2 * r + 1];
    for (int64_t x = a + threadIdx.x; x < b; x += 256) {
        const float v = l[static_cast<int64_t>(r) * V + x];
        probs[static_cast<int64_t>(r) * V + x] = v > -INFINITY ? expf((v - m) * invT) / s : 0.0f;
    }
}
} // namespace

size_t softmax_rows_workspace(int rows, int64_t V) {
    const int nc = static_cast<int>(std::min<int64_t>(kSampChunks, (V + 255) / 256));
    return a256(static_cast<size_t>(rows) * nc * sizeof(float2));
}

hipError_t launch_softmax_rows(const float* logits, int rows, int64_t V, float T, float* stats, float* probs, void* ws,
                               hipStream_t st) {
    const int nc = static_cast<int>(std::min<int64_t>(kSampChunks, (V + 255) / 256));
    const int64_t cs = (V + nc - 1) / nc;
    const float invT = 1.0f / T;
    auto* part = static_cast<float2*>(ws);
    hipError_t e = launch(k_samp_stats, dim3(nc, rows), dim3(256), 0, st, logits, logits, rows - 1, V, cs, invT, part);
    if (e == hipSuccess)
        e = launch(k_softmax_stats, dim3(rows), dim3(64), 0, st, static_cast<const float2*>(part), nc, invT, stats);
    if (e == hipSuccess && probs)
        e = launch(k_softmax_probs, dim3(nc, rows), dim3(256), 0, st, logits, V, cs, invT,
                   static_cast<const float*>(stats), probs);
    return e;
}

} // namespace q38
