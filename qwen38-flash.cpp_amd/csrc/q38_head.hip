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

// One block per request row: the int8 planes of h, its plane scale, the residual R and
// sum|h| (double, fixed order), and the reset of the pass state (kernel stores, no memset
// nodes, so the sequence can be captured in a graph).
__global__ __launch_bounds__(256) void k_head_prep(const uint16_t* __restrict__ h, int H, int M, HeadWork w) {
    __shared__ float redm[4];
    __shared__ double redt[4], redr[4];
    const int r = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const uint16_t* hr = h + static_cast<size_t>(r) * H;
    float m = 0.0f;
    for (int c = tid; c < H; c += 256) m = fmaxf(m, fabsf(bf2f(hr[c])));
    m = wave_max(m);
    if (lane == 0) redm[wv] = m;
    __syncthreads();
    m = fmaxf(fmaxf(redm[0], redm[1]), fmaxf(redm[2], redm[3]));
    int e = 0;
    (void)frexpf(m, &e);
    const float s = m > 0.0f ? ldexpf(1.0f, e - 6) : 1.0f;
    const double sd = s;
    double tsum = 0.0, res = 0.0;
    for (int c = tid; c < H; c += 256) {
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
    if (lane == 0) { redt[wv] = tsum; redr[wv] = res; }
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
    if (wave == 0 && jact && !out_logits) atomicMax(&w.rowmax[i16], orderable(mx));
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
// removed per 64-column group with the group's column sum of h.
template <int M>
__global__ __launch_bounds__(256) void k_head_q4(HeadDev hd, const uint16_t* __restrict__ h,
                                                 float* __restrict__ out_logits) {
    constexpr int CPL = 32;  // H = 2048: lane l owns columns [32l, 32l+32) = half a group
    const int lane = threadIdx.x & 63;
    const int gw = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int nw = gridDim.x * 4;
    const int H = hd.H, G = H / 64;
    float hr[M][CPL];
    float hs[M];
#pragma unroll
    for (int r = 0; r < M; ++r) {
        hs[r] = 0.0f;
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            hr[r][c] = bf2f(h[static_cast<size_t>(r) * H + CPL * lane + c]);
            hs[r] += hr[r][c];
        }
    }
    for (int64_t v = gw; v < hd.V; v += nw) {
        const uint4 q = reinterpret_cast<const uint4*>(hd.w + v * (H / 2) + (CPL / 2) * lane)[0];
        const uint32_t wd[4] = {q.x, q.y, q.z, q.w};
        float acc[M];
#pragma unroll
        for (int r = 0; r < M; ++r) acc[r] = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t b = wd[i] ^ 0x88888888u;
#pragma unroll
            for (int n = 0; n < 8; ++n) {
                const float u = static_cast<float>((b >> (4 * n)) & 0xfu);
#pragma unroll
                for (int r = 0; r < M; ++r) acc[r] = fmaf(u, hr[r][8 * i + n], acc[r]);
            }
        }
        const float sc = h2f(hd.scales[v * G + lane / 2]);
#pragma unroll
        for (int r = 0; r < M; ++r) {
            const float s = wave_sum_xor(sc * fmaf(-8.0f, hs[r], acc[r]));
            if (lane == 0) out_logits[static_cast<size_t>(r) * hd.V + v] = s;
        }
    }
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
// One workgroup. Row statistics are block reductions in a fixed order; the residual /
// bonus draw is an inverse CDF over the vocab in index order (chunked prefix sums).
namespace {
constexpr int kSampThreads = 1024;

__device__ float block_reduce(float v, float* sh, bool is_max) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    if (is_max) v = wave_max(v);
    else v = wave_sum_xor(v);
    __syncthreads();
    if (lane == 0) sh[wv] = v;
    __syncthreads();
    float t = sh[0];
    for (int i = 1; i < kSampThreads / 64; ++i) t = is_max ? fmaxf(t, sh[i]) : t + sh[i];
    __syncthreads();
    return t;
}

struct RowStat { float mx, sum; };
__device__ RowStat row_stat(const float* l, int64_t V, float invT, float* sh) {
    float m = -INFINITY;
    for (int64_t i = threadIdx.x; i < V; i += kSampThreads) m = fmaxf(m, l[i]);
    m = block_reduce(m, sh, true);
    float s = 0.0f;
    for (int64_t i = threadIdx.x; i < V; i += kSampThreads) s += expf((l[i] - m) * invT);
    s = block_reduce(s, sh, false);
    return {m, s};
}

// weight(x) = max(0, p(x) - q(x)) when dl != null, else p(x). Returns the smallest x whose
// inclusive prefix sum exceeds v * total (thread chunks in index order); when rounding
// leaves no crossing, the last x with positive weight.
__device__ int64_t draw_cdf(const float* tl, RowStat ps, const float* dl, RowStat qs, int64_t V, float invT,
                            float v, float* sh, unsigned long long* found, unsigned long long* lastp) {
    const int tid = threadIdx.x;
    const int64_t chunk = (V + kSampThreads - 1) / kSampThreads;
    const int64_t a = tid * chunk < V ? tid * chunk : V;
    const int64_t b = a + chunk < V ? a + chunk : V;
    auto wgt = [&](int64_t x) {
        const float p = expf((tl[x] - ps.mx) * invT) / ps.sum;
        if (!dl) return p;
        const float q = expf((dl[x] - qs.mx) * invT) / qs.sum;
        return fmaxf(0.0f, p - q);
    };
    float s = 0.0f;
    int64_t last = -1;
    for (int64_t x = a; x < b; ++x) {
        const float wv = wgt(x);
        s += wv;
        if (wv > 0.0f) last = x;
    }
    if (tid == 0) { *found = ~0ull; *lastp = 0ull; }
    sh[tid] = s;
    __syncthreads();
    for (int off = 1; off < kSampThreads; off <<= 1) {
        const float t = tid >= off ? sh[tid - off] : 0.0f;
        __syncthreads();
        sh[tid] += t;
        __syncthreads();
    }
    const float incl = sh[tid];
    const float total = sh[kSampThreads - 1];
    const float excl = incl - s;
    const float target = v * total;
    if (last >= 0) atomicMax(lastp, static_cast<unsigned long long>(last + 1));
    if (s > 0.0f && excl <= target && target < incl) {
        float c = excl;
        int64_t pick = last;
        for (int64_t x = a; x < b; ++x) {
            const float wv = wgt(x);
            c += wv;
            if (c > target && wv > 0.0f) { pick = x; break; }
        }
        atomicMin(found, static_cast<unsigned long long>(pick));
    }
    __syncthreads();
    const unsigned long long f = *found, l = *lastp;
    __syncthreads();
    if (f != ~0ull) return static_cast<int64_t>(f);
    return l ? static_cast<int64_t>(l - 1) : 0;
}
} // namespace

__global__ __launch_bounds__(kSampThreads) void k_accept_sampled(const float* __restrict__ tl,
                                                                const float* __restrict__ dl,
                                                                const uint32_t* __restrict__ drafts, int k, int64_t V,
                                                                float T, uint64_t seed, uint64_t slot, uint64_t round,
                                                                int64_t* __restrict__ out) {
    __shared__ float sh[kSampThreads];
    __shared__ unsigned long long found, lastp;
    const float invT = 1.0f / T;
    for (int i = 0; i < k; ++i) {
        const float* ti = tl + static_cast<size_t>(i) * V;
        const float* di = dl + static_cast<size_t>(i) * V;
        const RowStat ps = row_stat(ti, V, invT, sh);
        const RowStat qs = row_stat(di, V, invT, sh);
        float u, v;
        round_uniforms(seed, slot, round, static_cast<uint32_t>(i), &u, &v);
        const uint32_t d = drafts[i];
        // an out-of-vocabulary draft is rejected (never read out of bounds)
        const float pd = d < V ? expf((ti[d] - ps.mx) * invT) / ps.sum : 0.0f;
        const float qd = d < V ? expf((di[d] - qs.mx) * invT) / qs.sum : 1.0f;
        if (u * qd < pd) continue;
        const int64_t x = draw_cdf(ti, ps, di, qs, V, invT, v, sh, &found, &lastp);
        if (threadIdx.x == 0) { out[0] = i; out[1] = x; }
        return;
    }
    const float* tk = tl + static_cast<size_t>(k) * V;
    const RowStat ps = row_stat(tk, V, invT, sh);
    float u, v;
    round_uniforms(seed, slot, round, static_cast<uint32_t>(k), &u, &v);
    const int64_t x = draw_cdf(tk, ps, nullptr, ps, V, invT, v, sh, &found, &lastp);
    if (threadIdx.x == 0) { out[0] = k; out[1] = x; }
}

// ---------------------------------------------------------------- launchers
namespace {
int head_grid() { return 256 * 8; }

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
hipError_t launch_q4_m(const HeadDev& hd, const uint16_t* h, float* out, hipStream_t st) {
    return launch(k_head_q4<M>, dim3(head_grid()), dim3(256), 0, st, hd, h, out);
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
__global__ __launch_bounds__(256) void k_fc_join(const float* __restrict__ a, const float* __restrict__ b, int n,
                                                 uint16_t* __restrict__ x, unsigned long long* __restrict__ best,
                                                 int M) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) x[i] = f2bf(rbf(a[i]) + rbf(b[i]));
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

hipError_t launch_fc_join(const float* a, const float* b, int n, uint16_t* x, unsigned long long* best, int M,
                          hipStream_t st) {
    return launch(k_fc_join, dim3((n + 255) / 256), dim3(256), 0, st, a, b, n, x, best, M);
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

hipError_t launch_accept_sampled(const float* tl, const float* dl, const uint32_t* drafts, int k, int64_t V,
                                 float T, uint64_t seed, uint64_t slot, uint64_t round, int64_t* out,
                                 hipStream_t st) {
    return launch(k_accept_sampled, dim3(1), dim3(kSampThreads), 0, st, tl, dl, drafts, k, V, T, seed, slot, round,
                  out);
}

} // namespace q38
