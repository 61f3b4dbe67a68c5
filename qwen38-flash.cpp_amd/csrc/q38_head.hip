// q38_head.hip — gfx950 kernels of the verify tail: the Q8 target LM head with an exact
// greedy argmax (R12, R13), the Q4/g64 draft head logits (R14), and rejection-sampling
// acceptance (R16).
//
// Greedy argmax. The reference takes argmax_all over MLX quantized_matmul logits
// (src/model.cpp:470-480, src/mtp_verifier.cpp:30-55). Greedy acceptance must be
// bit-exact, so the argmax is defined on an exact logit contract (double partial sums in
// a fixed order, see oracle/q38_oracle.cpp head_q8_logit) and computed in two passes:
//   1. k_head_fast: the bandwidth pass. Every int8 row is read once and dotted with all
//      rows of h in float; per-row maxima are kept.
//   2. k_head_cand + k_head_exact: every vocab row whose fast logit lies within twice the
//      proven float error bound of the row maximum is recomputed under the contract and
//      the best (logit desc, index asc) key wins. The true contract argmax always lies in
//      that window, so the result equals the contract argmax; the window holds one or a
//      few rows in practice. More than kHeadCap candidates fall back to recomputing all
//      rows of that request row.
#include "q38_device.hpp"
#include "q38_internal.hpp"

namespace q38 {

size_t head_work_bytes(int64_t V, int M) {
    size_t b = 0;
    b += static_cast<size_t>(M) * V * 4;            // fast
    b += 256;                                        // rowmax
    b += 256;                                        // tsum
    b += 256;                                        // cnt
    b += static_cast<size_t>(M) * kHeadCap * 4;     // cand
    b += 256;                                        // best
    return b + 1024;
}
HeadWork head_work_carve(void* base, int64_t V, int M) {
    char* p = static_cast<char*>(base);
    HeadWork w{};
    w.fast = reinterpret_cast<float*>(p);
    p += (static_cast<size_t>(M) * V * 4 + 255) / 256 * 256;
    w.rowmax = reinterpret_cast<uint32_t*>(p); p += 256;
    w.tsum = reinterpret_cast<float*>(p); p += 256;
    w.cnt = reinterpret_cast<int32_t*>(p); p += 256;
    w.cand = reinterpret_cast<int32_t*>(p); p += (static_cast<size_t>(M) * kHeadCap * 4 + 255) / 256 * 256;
    w.best = reinterpret_cast<unsigned long long*>(p);
    return w;
}

// Per request row: sum |h| (fixed order) and reset of the pass state (no memset nodes,
// so the sequence can be captured in a graph).
__global__ void k_head_prep(const uint16_t* __restrict__ h, int H, HeadWork w) {
    __shared__ float red[4];
    const int r = blockIdx.x, tid = threadIdx.x;
    float s = 0.0f;
    for (int c = tid; c < H; c += 256) s += fabsf(bf2f(h[static_cast<size_t>(r) * H + c]));
    s = wave_sum_xor(s);
    if ((tid & 63) == 0) red[tid >> 6] = s;
    __syncthreads();
    if (tid == 0) {
        w.tsum[r] = (red[0] + red[1]) + (red[2] + red[3]);
        w.rowmax[r] = 0u;
        w.cnt[r] = 0;
        w.best[r] = 0ull;
    }
}

// Fast pass. Lane l owns columns [CPL*l, CPL*l + CPL); the int8 weights are biased by
// 128 (w ^ 0x80 -> u in [1, 255], converted exactly by v_cvt_f32_ubyte*) and the bias
// is removed with the lane's column sum of h.
template <int M, int CPL>
__global__ __launch_bounds__(256) void k_head_fast(HeadDev hd, const uint16_t* __restrict__ h, HeadWork w,
                                                   float* __restrict__ out_logits) {
    const int lane = threadIdx.x & 63;
    const int gw = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int nw = gridDim.x * 4;
    const int H = hd.H;
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
    float mx[M];
#pragma unroll
    for (int r = 0; r < M; ++r) mx[r] = -INFINITY;
    float* dst = out_logits ? out_logits : w.fast;
    for (int64_t v = gw; v < hd.V; v += nw) {
        const int8_t* row = hd.w + v * H + CPL * lane;
        uint32_t wd[CPL / 4];
        if constexpr ((CPL % 16) == 0) {
#pragma unroll
            for (int i = 0; i < CPL / 16; ++i) {
                const uint4 q = reinterpret_cast<const uint4*>(row)[i];
                wd[4 * i] = q.x; wd[4 * i + 1] = q.y; wd[4 * i + 2] = q.z; wd[4 * i + 3] = q.w;
            }
        } else {
#pragma unroll
            for (int i = 0; i < CPL / 8; ++i) {
                const uint2 q = reinterpret_cast<const uint2*>(row)[i];
                wd[2 * i] = q.x; wd[2 * i + 1] = q.y;
            }
        }
        float acc[M];
#pragma unroll
        for (int r = 0; r < M; ++r) acc[r] = 0.0f;
#pragma unroll
        for (int i = 0; i < CPL / 4; ++i) {
            const uint32_t b = wd[i] ^ 0x80808080u;
            const float u0 = static_cast<float>(b & 0xffu);
            const float u1 = static_cast<float>((b >> 8) & 0xffu);
            const float u2 = static_cast<float>((b >> 16) & 0xffu);
            const float u3 = static_cast<float>(b >> 24);
#pragma unroll
            for (int r = 0; r < M; ++r) {
                acc[r] = fmaf(u0, hr[r][4 * i], acc[r]);
                acc[r] = fmaf(u1, hr[r][4 * i + 1], acc[r]);
                acc[r] = fmaf(u2, hr[r][4 * i + 2], acc[r]);
                acc[r] = fmaf(u3, hr[r][4 * i + 3], acc[r]);
            }
        }
        const float sc = h2f(hd.scales[v]);
#pragma unroll
        for (int r = 0; r < M; ++r) {
            const float s = wave_sum_xor(fmaf(-128.0f, hs[r], acc[r]));
            const float lg = s * sc;
            mx[r] = fmaxf(mx[r], lg);
            if (lane == 0) dst[static_cast<size_t>(r) * hd.V + v] = lg;
        }
    }
    if (lane == 0 && !out_logits) {
#pragma unroll
        for (int r = 0; r < M; ++r) atomicMax(&w.rowmax[r], orderable(mx[r]));
    }
}

// MFMA fast pass (v_mfma_f32_16x16x32_bf16). A wave owns 16-row vocab tiles; lane
// (i = l % 16, q = l / 16) loads 16 weight bytes of row i per 64-column superstep s
// (columns 64s + 16q .. +15) and feeds them to two MFMAs as bf16 (u = w ^ 0x80 = w + 128 is
// exact in bf16); B holds the same columns of the request rows, from LDS. The bias is
// removed per request row with 128 * sum(h). Output lane (i' = 4q + r, j = l % 16).
typedef __bf16 bh8_t __attribute__((ext_vector_type(8)));
typedef float hf4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t pack_bf16_hi(float lo, float hi) {
    return (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xffff0000u);
}

template <int H>
__global__ __launch_bounds__(256) void k_head_mfma(HeadDev hd, const uint16_t* __restrict__ h, int M, HeadWork w,
                                                   float* __restrict__ out_logits) {
    __shared__ __align__(16) uint16_t hs[5 * H];   // request rows 0..3, then a zero row
    __shared__ float hsum_s[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int i = tid; i < 5 * H / 8; i += 256) {
        uint4 v = make_uint4(0u, 0u, 0u, 0u);
        if (i < M * H / 8) v = reinterpret_cast<const uint4*>(h)[i];
        reinterpret_cast<uint4*>(hs)[i] = v;
    }
    if (wave < M) {
        float sacc = 0.0f;
        for (int c = lane; c < H; c += 64) sacc += bf2f(h[wave * H + c]);
        sacc = wave_sum_xor(sacc);
        if (lane == 0) hsum_s[wave] = sacc;
    }
    __syncthreads();
    const int i16 = lane & 15, q = lane >> 4;
    const int j = i16;                       // request row of this lane's B / D column
    const bool jact = j < M;
    const float hsum = jact ? hsum_s[j] : 0.0f;
    const uint4* hrow = reinterpret_cast<const uint4*>(hs + (jact ? j : 4) * H) + 2 * q;  // branch-free B
    float* dst = out_logits ? out_logits : w.fast;
    const int64_t tiles = (hd.V + 15) / 16;
    float mx = -INFINITY;
    constexpr int S = H / 64;
    constexpr int BATCH = 8;
    for (int64_t t = blockIdx.x * 4 + wave; t < tiles; t += gridDim.x * 4) {
        const int64_t v0 = t * 16;
        int64_t vr = v0 + i16;
        if (vr >= hd.V) vr = hd.V - 1;       // ragged last tile: recompute a valid row, not stored
        const uint4* wrow = reinterpret_cast<const uint4*>(hd.w + vr * H) + q;
        hf4_t acc = {0.f, 0.f, 0.f, 0.f};
        for (int s0 = 0; s0 < S; s0 += BATCH) {
            uint4 wv[BATCH];
#pragma unroll
            for (int k = 0; k < BATCH; ++k) wv[k] = wrow[4 * (s0 + k)];
#pragma unroll
            for (int k = 0; k < BATCH; ++k) {
                const uint32_t b4[4] = {wv[k].x ^ 0x80808080u, wv[k].y ^ 0x80808080u, wv[k].z ^ 0x80808080u,
                                        wv[k].w ^ 0x80808080u};
                uint32_t a[8];
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    const float f0 = static_cast<float>(b4[m] & 0xffu), f1 = static_cast<float>((b4[m] >> 8) & 0xffu);
                    const float f2 = static_cast<float>((b4[m] >> 16) & 0xffu), f3 = static_cast<float>(b4[m] >> 24);
                    a[2 * m] = pack_bf16_hi(f0, f1);
                    a[2 * m + 1] = pack_bf16_hi(f2, f3);
                }
                const uint4 b0 = hrow[8 * (s0 + k)];
                const uint4 b1 = hrow[8 * (s0 + k) + 1];
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    __builtin_bit_cast(bh8_t, make_uint4(a[0], a[1], a[2], a[3])), __builtin_bit_cast(bh8_t, b0), acc,
                    0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    __builtin_bit_cast(bh8_t, make_uint4(a[4], a[5], a[6], a[7])), __builtin_bit_cast(bh8_t, b1), acc,
                    0, 0, 0);
            }
        }
        if (jact) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t v = v0 + 4 * q + r;
                if (v < hd.V) {
                    const float lg = fmaf(-128.0f, hsum, acc[r]) * h2f(hd.scales[v]);
                    mx = fmaxf(mx, lg);
                    dst[static_cast<size_t>(j) * hd.V + v] = lg;
                }
            }
        }
    }
    if (jact && !out_logits) atomicMax(&w.rowmax[j], orderable(mx));
}

// Window: fast >= max - 2E, E = 2 * s_max * 383 * sum|h| * 80 * 2^-24 + 1e-30 (the float
// error bound of the fast pass and of the contract's own rounding, with a factor 2).
// Window: fast >= max - 2E with E a bound on |fast - contract|: the fast pass sums 2048
// terms |u*h| <= 255|h| (plus the 128*sum(h) correction) in float in an unspecified order,
// so |error| <= 2^-24 * s_max * sum|h| * (2047 * 383 + 2 * 383); taken with a factor 4.
__device__ __forceinline__ float head_window(const HeadDev& hd, const HeadWork& w, int r) {
    const float E = 4.0f * hd.s_max * w.tsum[r] * 0x1.0p-24f * (2047.0f * 383.0f + 766.0f) + 1e-30f;
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

template <int M>
hipError_t launch_fast_m(const HeadDev& hd, const uint16_t* h, const HeadWork& w, float* out, hipStream_t st) {
    if (hd.H == 2048)
        hipLaunchKernelGGL((k_head_fast<M, 32>), dim3(head_grid()), dim3(256), 0, st, hd, h, w, out);
    else if (hd.H == 2560)
        hipLaunchKernelGGL((k_head_fast<M, 40>), dim3(head_grid()), dim3(256), 0, st, hd, h, w, out);
    else if (hd.H == 1024)
        hipLaunchKernelGGL((k_head_fast<M, 16>), dim3(head_grid()), dim3(256), 0, st, hd, h, w, out);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}
hipError_t launch_fast(const HeadDev& hd, const uint16_t* h, int M, const HeadWork& w, float* out, hipStream_t st) {
    if (M >= 1 && M <= 4 && (hd.H == 2048 || hd.H == 1024)) {
        if (hd.H == 2048)
            hipLaunchKernelGGL(k_head_mfma<2048>, dim3(256 * 4), dim3(256), 0, st, hd, h, M, w, out);
        else
            hipLaunchKernelGGL(k_head_mfma<1024>, dim3(256 * 4), dim3(256), 0, st, hd, h, M, w, out);
        return hipGetLastError();
    }
    switch (M) {
        case 1: return launch_fast_m<1>(hd, h, w, out, st);
        case 2: return launch_fast_m<2>(hd, h, w, out, st);
        case 3: return launch_fast_m<3>(hd, h, w, out, st);
        case 4: return launch_fast_m<4>(hd, h, w, out, st);
        default: return hipErrorInvalidValue;
    }
}
template <int M>
hipError_t launch_q4_m(const HeadDev& hd, const uint16_t* h, float* out, hipStream_t st) {
    hipLaunchKernelGGL((k_head_q4<M>), dim3(head_grid()), dim3(256), 0, st, hd, h, out);
    return hipGetLastError();
}
} // namespace

hipError_t launch_head_greedy(const HeadDev& hd, const uint16_t* h, int M, const HeadWork& w, uint32_t* argmax,
                              float* logit, hipStream_t st) {
    hipLaunchKernelGGL(k_head_prep, dim3(M), dim3(256), 0, st, h, hd.H, w);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if ((e = launch_fast(hd, h, M, w, nullptr, st)) != hipSuccess) return e;
    hipLaunchKernelGGL(k_head_cand, dim3(2048), dim3(256), 0, st, hd, M, w);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL(k_head_exact, dim3(16, M), dim3(256), 0, st, hd, h, w);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL(k_head_final, dim3(1), dim3(64), 0, st, M, w, argmax, logit);
    return hipGetLastError();
}

hipError_t launch_head_logits(const HeadDev& hd, const uint16_t* h, int M, float* logits, hipStream_t st) {
    if (hd.kind == 0) {
        HeadWork dummy{};
        return launch_fast(hd, h, M, dummy, logits, st);
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

hipError_t launch_accept_sampled(const float* tl, const float* dl, const uint32_t* drafts, int k, int64_t V,
                                 float T, uint64_t seed, uint64_t slot, uint64_t round, int64_t* out,
                                 hipStream_t st) {
    hipLaunchKernelGGL(k_accept_sampled, dim3(1), dim3(kSampThreads), 0, st, tl, dl, drafts, k, V, T, seed, slot,
                       round, out);
    return hipGetLastError();
}

} // namespace q38
