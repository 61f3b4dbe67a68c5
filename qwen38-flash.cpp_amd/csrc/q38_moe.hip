// q38_moe.hip — gfx950 kernels of one packed-VQ sparse-MoE layer at verify width
// (rows <= 16), plus the synthetic-weight generators.
//
// Per layer the launch sequence is
//   k_router      RMSNorm (chain mode) + router logits with the fixed-order contract
//                 (R1) + the shared-expert gate logit; one wave per expert row of Wr.
//   k_topk_plan   softmax/top-k/normalise per row (R2) and the gather-by-expert plan
//                 (R3): unique experts ascending, each with its routes in (row, slot)
//                 order; one workgroup.
//   k_gate_up     per (unique expert, 64 output rows): every packed code row is read
//                 once and applied to all rows routed to that expert (R4, R5, R7);
//                 SwiGLU epilogue with the reference's rounding points.
//   k_down        per (unique expert, 128 output rows): down projection of the expert's
//                 SwiGLU rows, rounded to BF16 per route (R8).
//   k_combine     ordered route reduction (slot order) + shared expert x sigmoid gate +
//                 merge (R8, R10, R11), and in chain mode the residual add.
#include "q38_device.hpp"
#include "q38_internal.hpp"

namespace q38 {

// ============================================================== generators
__global__ void k_gen_codes(uint64_t key, int e0, int n_experts, int out_dim, int nsub, int bits, int words,
                            uint32_t* __restrict__ codes) {
    // one thread per (expert, row, 32-code block)
    const int nblk = (nsub + 31) / 32;
    const int64_t total = static_cast<int64_t>(n_experts) * out_dim * nblk;
    for (int64_t t = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; t < total;
         t += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int blk = static_cast<int>(t % nblk);
        const int64_t row = t / nblk;  // local (expert, o)
        const int o = static_cast<int>(row % out_dim);
        const int e = e0 + static_cast<int>(row / out_dim);
        uint32_t w[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) w[i] = 0;
        for (int q = 0; q < 32; ++q) {
            const int s = blk * 32 + q;
            if (s >= nsub) break;
            const uint64_t idx = (static_cast<uint64_t>(e) * out_dim + o) * 1024ull + s;
            const uint64_t code = bits_at(key, idx) >> (64 - bits);
            const int bit = q * bits, wi = bit >> 5, sh = bit & 31;
            const uint64_t v = code << sh;
            for (int i = 0; i < 16; ++i) {
                if (i == wi) w[i] |= static_cast<uint32_t>(v);
                if (i == wi + 1 && sh + bits > 32) w[i] |= static_cast<uint32_t>(v >> 32);
            }
        }
        uint32_t* dst = codes + row * words + static_cast<int64_t>(blk) * bits;
        for (int i = 0; i < bits; ++i) dst[i] = w[i];
    }
}

__global__ void k_gen_uniform_f16(uint64_t key, int64_t idx0, int64_t n, double lo, double hi,
                                  uint16_t* __restrict__ out) {
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x)
        out[i] = f2h(uniform_f32(key, static_cast<uint64_t>(idx0 + i), lo, hi));
}

__global__ void k_gen_normal(uint64_t key, int64_t n, double sd, int f16, uint16_t* __restrict__ out) {
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const double z = normal_at(key, static_cast<uint64_t>(i));
        const double v = z * sd;
        const float f = static_cast<float>(v);
        out[i] = f16 ? f2h(f) : f2bf(f);
    }
}

struct TokenList { uint32_t t[32]; };
__global__ void k_gen_embed(uint64_t key, TokenList toks, int n, int H, uint16_t* __restrict__ out) {
    const int64_t total = static_cast<int64_t>(n) * H;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int r = static_cast<int>(i / H), c = static_cast<int>(i % H);
        const double z = normal_at(key, static_cast<uint64_t>(toks.t[r]) * H + c);
        out[i] = f2bf(static_cast<float>(z));
    }
}

// Approximate INT8 codebook with one FP16 scale per codebook: scale = f16(max|v| / 127),
// q = clamp(rint(v / scale), -127, 127). One workgroup; v = the FP16 N(0,1) book.
__global__ void k_book_to_int8(const uint16_t* __restrict__ book16, int n, int8_t* __restrict__ q8,
                               uint16_t* __restrict__ scale) {
    __shared__ float red[16];
    float mx = 0.0f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) mx = fmaxf(mx, fabsf(h2f(book16[i])));
    mx = wave_max(mx);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    float m = 0.0f;
    for (int w = 0; w < static_cast<int>(blockDim.x >> 6); ++w) m = fmaxf(m, red[w]);
    const uint16_t s16 = f2h(m / 127.0f);
    const float s = h2f(s16);
    if (threadIdx.x == 0) *scale = s16;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        float q = rintf(h2f(book16[i]) / s);
        q = fminf(127.0f, fmaxf(-127.0f, q));
        q8[i] = static_cast<int8_t>(q);
    }
}

// ============================================================== router (R1)
// One wave per row of Wr (plus one for w_sg). Lane l accumulates c = 512t + 8l + j
// (t outer, j inner) with fmaf, then the xor butterfly; rounded to BF16.
template <int MAXM>
__global__ __launch_bounds__(256) void k_router(LayerDev L, const uint16_t* __restrict__ hin, int M, int do_norm,
                                                float eps, uint16_t* __restrict__ xn_out,
                                                float* __restrict__ logits, float* __restrict__ sgate) {
    extern __shared__ __align__(16) uint16_t xs[];  // [M][H]
    __shared__ float red[4][MAXM];
    const int H = L.H;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (do_norm) {
#pragma unroll
        for (int r = 0; r < MAXM; ++r) {
            if (r < M) {
                float ss = 0.0f;
                for (int c = tid; c < H; c += 256) {
                    const float v = bf2f(hin[r * H + c]);
                    ss = fmaf(v, v, ss);
                }
                ss = wave_sum_xor(ss);
                if (lane == 0) red[wave][r] = ss;
            }
        }
        __syncthreads();
        for (int i = tid; i < M * H; i += 256) {
            const int r = i / H;
            const float ss = (red[0][r] + red[1][r]) + (red[2][r] + red[3][r]);
            const float inv = 1.0f / sqrtf(ss / static_cast<float>(H) + eps);
            const uint16_t x = f2bf(bf2f(hin[i]) * inv);
            xs[i] = x;
            if (blockIdx.x == 0 && xn_out) xn_out[i] = x;
        }
    } else {
        const uint4* src = reinterpret_cast<const uint4*>(hin);
        uint4* dst = reinterpret_cast<uint4*>(xs);
        for (int i = tid; i < M * H / 8; i += 256) dst[i] = src[i];
    }
    __syncthreads();
    const int e = blockIdx.x * 4 + wave;
    const int n_rows = L.E + (L.has_shared ? 1 : 0);
    if (e >= n_rows) return;
    const uint16_t* w = e < L.E ? L.router + static_cast<size_t>(e) * H : L.wsg;
    float acc[MAXM];
#pragma unroll
    for (int r = 0; r < MAXM; ++r) acc[r] = 0.0f;
    for (int t = 0; t < H / 512; ++t) {
        const uint4 wv = *reinterpret_cast<const uint4*>(w + 512 * t + 8 * lane);
        const float wf[8] = {bflo(wv.x), bfhi(wv.x), bflo(wv.y), bfhi(wv.y),
                             bflo(wv.z), bfhi(wv.z), bflo(wv.w), bfhi(wv.w)};
#pragma unroll
        for (int r = 0; r < MAXM; ++r) {
            if (r < M) {
                const uint4 xv = *reinterpret_cast<const uint4*>(xs + r * H + 512 * t + 8 * lane);
                const float xf[8] = {bflo(xv.x), bfhi(xv.x), bflo(xv.y), bfhi(xv.y),
                                     bflo(xv.z), bfhi(xv.z), bflo(xv.w), bfhi(xv.w)};
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[r] = __builtin_fmaf(xf[j], wf[j], acc[r]);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < MAXM; ++r) {
        if (r < M) {
            const float s = wave_sum_xor(acc[r]);
            if (lane == 0) {
                if (e < L.E) {
                    logits[r * L.E + e] = rbf(s);
                } else {
                    const float lg = rbf(s);
                    sgate[r] = rbf(1.0f / (1.0f + expf(-lg)));
                }
            }
        }
    }
}

// ============================================================== top-k + plan (R2, R3)
// One workgroup of 1024 threads; wave r handles row r (rows <= 16). Lane l owns experts
// i = 64j + l. Plan: per expert (one thread each) count its routes, scan, and list them
// in (row, slot) order.
__global__ __launch_bounds__(1024) void k_topk_plan(const float* __restrict__ logits, int M, int E, int K,
                                                    int normalize, int32_t* __restrict__ experts,
                                                    float* __restrict__ weights, int32_t* __restrict__ plan) {
    __shared__ int32_t ex_s[kMaxRows * kMaxTopK];
    __shared__ int32_t sc_a[1024], sc_b[1024];
    const int tid = threadIdx.x, lane = tid & 63, r = tid >> 6;
    const int NJ = E / 64;
    if (r < M) {
        float lg[16];
        float mx = -INFINITY;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            lg[j] = j < NJ ? logits[r * E + 64 * j + lane] : -INFINITY;
            mx = fmaxf(mx, lg[j]);
        }
        mx = wave_max(mx);
        float ev[16];
        double ds = 0.0;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            if (j < NJ) {
                ev[j] = exp_contract(lg[j] - mx);
                ds += static_cast<double>(ev[j]);
            }
        }
        ds = wave_sum_xor(ds);
        uint64_t key[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            if (j < NJ) {
                const float p = static_cast<float>(static_cast<double>(ev[j]) / ds);
                key[j] = (static_cast<uint64_t>(__float_as_uint(p)) << 32) |
                         static_cast<uint64_t>(0xFFFFFFFFu - static_cast<uint32_t>(64 * j + lane));
            } else {
                key[j] = 0;
            }
        }
        float psel[kMaxTopK];
        int isel[kMaxTopK];
        for (int s = 0; s < K; ++s) {
            uint64_t best = 0;
#pragma unroll
            for (int j = 0; j < 16; ++j) best = key[j] > best ? key[j] : best;
            best = wave_max_u64(best);
#pragma unroll
            for (int j = 0; j < 16; ++j)
                if (key[j] == best) key[j] = 0;
            psel[s] = __uint_as_float(static_cast<uint32_t>(best >> 32));
            isel[s] = static_cast<int>(0xFFFFFFFFu - static_cast<uint32_t>(best));
        }
        if (lane == 0) {
            float sum = 0.0f;
            for (int s = 0; s < K; ++s) sum += psel[s];
            for (int s = 0; s < K; ++s) {
                experts[r * K + s] = isel[s];
                weights[r * K + s] = normalize ? psel[s] / sum : psel[s];
                ex_s[r * K + s] = isel[s];
            }
        }
    }
    __syncthreads();
    const int MK = M * K;
    int cnt = 0;
    if (tid < E)
        for (int i = 0; i < MK; ++i) cnt += ex_s[i] == tid;
    // inclusive scans of cnt (offsets) and of (cnt > 0) (ranks)
    sc_a[tid] = cnt;
    sc_b[tid] = cnt > 0;
    __syncthreads();
    for (int off = 1; off < 1024; off <<= 1) {
        const int a = tid >= off ? sc_a[tid - off] : 0;
        const int b = tid >= off ? sc_b[tid - off] : 0;
        __syncthreads();
        sc_a[tid] += a;
        sc_b[tid] += b;
        __syncthreads();
    }
    int32_t* uexp = plan + 1;
    int32_t* uoff = plan + 1 + MK;
    int32_t* rlist = plan + 2 + 2 * MK;
    int32_t* rpos = plan + 2 + 3 * MK;
    if (tid < E && cnt > 0) {
        const int off = sc_a[tid] - cnt;
        const int rank = sc_b[tid] - 1;
        uexp[rank] = tid;
        uoff[rank] = off;
        int n = 0;
        for (int i = 0; i < MK; ++i)
            if (ex_s[i] == tid) {
                rlist[off + n] = i;
                rpos[i] = off + n;
                ++n;
            }
    }
    if (tid == 0) {
        const int nu = sc_b[1023];
        plan[0] = nu;
        uoff[nu] = MK;
    }
}

// ============================================================== expert projections
// Lane mapping: a lane owns 16 consecutive codes of a row (a half 32-code block: BITS/2
// words); LPR lanes (power of two, padded) cover one row; 64/LPR rows per wave.
template <int D>
struct Vec;
template <>
struct Vec<8> {
    static __device__ __forceinline__ void load_book(const uint16_t* book, uint32_t code, float* v) {
        const uint4 b = *reinterpret_cast<const uint4*>(book + code * 8);
        const uint32_t w[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[2 * i] = h2f(static_cast<uint16_t>(w[i]));
            v[2 * i + 1] = h2f(static_cast<uint16_t>(w[i] >> 16));
        }
    }
    static __device__ __forceinline__ void load_x(const uint16_t* x, float* v) {
        const uint4 b = *reinterpret_cast<const uint4*>(x);
        v[0] = bflo(b.x); v[1] = bfhi(b.x); v[2] = bflo(b.y); v[3] = bfhi(b.y);
        v[4] = bflo(b.z); v[5] = bfhi(b.z); v[6] = bflo(b.w); v[7] = bfhi(b.w);
    }
};
template <>
struct Vec<4> {
    static __device__ __forceinline__ void load_book(const uint16_t* book, uint32_t code, float* v) {
        const uint2 b = *reinterpret_cast<const uint2*>(book + code * 4);
        v[0] = h2f(static_cast<uint16_t>(b.x));
        v[1] = h2f(static_cast<uint16_t>(b.x >> 16));
        v[2] = h2f(static_cast<uint16_t>(b.y));
        v[3] = h2f(static_cast<uint16_t>(b.y >> 16));
    }
    static __device__ __forceinline__ void load_x(const uint16_t* x, float* v) {
        const uint2 b = *reinterpret_cast<const uint2*>(x);
        v[0] = bflo(b.x); v[1] = bfhi(b.x); v[2] = bflo(b.y); v[3] = bfhi(b.y);
    }
};

// Resolve the rows of unique-expert slot ui. Returns false when the slot is empty.
__device__ __forceinline__ bool slot_rows(const int32_t* plan, int M, int K, int has_shared, int ui, int E,
                                          int* expert, int* n, int* first_pos, bool* shared) {
    const int nu = plan[0];
    const int MK = M * K;
    if (ui < nu) {
        *expert = plan[1 + ui];
        const int a = plan[1 + MK + ui], b = plan[1 + MK + ui + 1];
        *n = b - a;
        *first_pos = a;
        *shared = false;
        return true;
    }
    if (ui == nu && has_shared) {
        *expert = E;
        *n = M;
        *first_pos = MK;
        *shared = true;
        return true;
    }
    return false;
}

constexpr int kGuRowsPerBlock = 64;
constexpr int kDownRowsPerBlock = 128;

template <int D, int BITS, int LPR, int MAXN>
__global__ __launch_bounds__(256) void k_gate_up(LayerDev L, const uint16_t* __restrict__ xn, int M,
                                                 const int32_t* __restrict__ plan, uint16_t* __restrict__ hbuf) {
    extern __shared__ __align__(16) uint16_t xs[];  // [n][H]
    int expert, n, pos0;
    bool shared;
    if (!slot_rows(plan, M, L.K, L.has_shared, blockIdx.y, L.E, &expert, &n, &pos0, &shared)) return;
    const int H = L.H, I = L.I, MK = M * L.K;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // stage the expert's input rows
    for (int i = tid; i < n * H / 8; i += 256) {
        const int j = i / (H / 8), c8 = i % (H / 8);
        const int row = shared ? j : plan[2 + 2 * MK + pos0 + j] / L.K;
        reinterpret_cast<uint4*>(xs)[i] = reinterpret_cast<const uint4*>(xn + static_cast<size_t>(row) * H)[c8];
    }
    __syncthreads();
    const ProjDev& G = L.p[0];
    const ProjDev& U = L.p[1];
    const int nsub = H / D;
    const int lanes_used = nsub / 16;
    const int sub_lane = lane % LPR;
    const bool active = sub_lane < lanes_used;
    const int s0 = sub_lane * 16;
    const bool row_scale = G.ngrp == 1;
    const int spg = H / G.ngrp / D;  // subvectors per scale group
    constexpr int WPL = BITS / 2;    // words per 16 codes
    constexpr int RPW = 64 / LPR;
    for (int it = 0; it < kGuRowsPerBlock / (4 * RPW); ++it) {
        const int o = blockIdx.x * kGuRowsPerBlock + it * 4 * RPW + wave * RPW + lane / LPR;
        float ga[MAXN], ua[MAXN];
#pragma unroll
        for (int j = 0; j < MAXN; ++j) { ga[j] = 0.0f; ua[j] = 0.0f; }
        if (active && o < I) {
            const size_t rowi = static_cast<size_t>(expert) * I + o;
            const uint32_t* gw = G.codes + rowi * G.words + (s0 / 32) * BITS + ((s0 % 32) / 16) * WPL;
            const uint32_t* uw = U.codes + rowi * U.words + (s0 / 32) * BITS + ((s0 % 32) / 16) * WPL;
            uint32_t gwr[WPL + 1], uwr[WPL + 1];
#pragma unroll
            for (int i = 0; i < WPL; ++i) { gwr[i] = gw[i]; uwr[i] = uw[i]; }
            gwr[WPL] = 0; uwr[WPL] = 0;
            float gp[MAXN], up[MAXN];
#pragma unroll
            for (int j = 0; j < MAXN; ++j) { gp[j] = 0.0f; up[j] = 0.0f; }
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const uint32_t gc = code_from<BITS>(gwr, q);
                const uint32_t uc = code_from<BITS>(uwr, q);
                float gb[D], ub[D];
                Vec<D>::load_book(G.book, gc, gb);
                Vec<D>::load_book(U.book, uc, ub);
                const int s = s0 + q;
#pragma unroll
                for (int j = 0; j < MAXN; ++j) {
                    if (j < n) {
                        float xv[D];
                        Vec<D>::load_x(xs + j * H + s * D, xv);
#pragma unroll
                        for (int d = 0; d < D; ++d) {
                            gp[j] = fmaf(xv[d], gb[d], gp[j]);
                            up[j] = fmaf(xv[d], ub[d], up[j]);
                        }
                    }
                }
                if (!row_scale && ((s + 1) % spg) == 0) {
                    const int g = s / spg;
                    const float gs = h2f(G.scales[rowi * G.ngrp + g]);
                    const float us = h2f(U.scales[rowi * U.ngrp + g]);
#pragma unroll
                    for (int j = 0; j < MAXN; ++j) {
                        ga[j] = fmaf(gs, gp[j], ga[j]);
                        ua[j] = fmaf(us, up[j], ua[j]);
                        gp[j] = 0.0f;
                        up[j] = 0.0f;
                    }
                }
            }
            if (row_scale) {
#pragma unroll
                for (int j = 0; j < MAXN; ++j) { ga[j] = gp[j]; ua[j] = up[j]; }
            }
        }
#pragma unroll
        for (int j = 0; j < MAXN; ++j) {
            ga[j] = group_sum_xor<LPR>(ga[j]);
            ua[j] = group_sum_xor<LPR>(ua[j]);
        }
        if (sub_lane == 0 && o < I) {
            const size_t rowi = static_cast<size_t>(expert) * I + o;
            const float gsc = row_scale ? h2f(G.scales[rowi]) : 1.0f;
            const float usc = row_scale ? h2f(U.scales[rowi]) : 1.0f;
#pragma unroll
            for (int j = 0; j < MAXN; ++j) {
                if (j < n) {
                    const float g = rbf(ga[j] * gsc);
                    const float u = rbf(ua[j] * usc);
                    const float s = rbf(g / (1.0f + expf(-g)));
                    hbuf[static_cast<size_t>(pos0 + j) * I + o] = f2bf(s * u);
                }
            }
        }
    }
    (void)MK;
}

template <int D, int BITS, int LPR, int MAXN>
__global__ __launch_bounds__(256) void k_down(LayerDev L, int M, const int32_t* __restrict__ plan,
                                              const uint16_t* __restrict__ hbuf, uint16_t* __restrict__ dbuf) {
    extern __shared__ __align__(16) uint16_t hs[];  // [n][I]
    int expert, n, pos0;
    bool shared;
    if (!slot_rows(plan, M, L.K, L.has_shared, blockIdx.y, L.E, &expert, &n, &pos0, &shared)) return;
    const int H = L.H, I = L.I;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int i = tid; i < n * I / 8; i += 256)
        reinterpret_cast<uint4*>(hs)[i] = reinterpret_cast<const uint4*>(hbuf + static_cast<size_t>(pos0) * I)[i];
    __syncthreads();
    const ProjDev& P = L.p[2];
    const int nsub = I / D;
    const int lanes_used = (nsub + 15) / 16;
    const int sub_lane = lane % LPR;
    const bool active = sub_lane < lanes_used;
    const int s0 = sub_lane * 16;
    const bool row_scale = P.ngrp == 1;
    const int spg = I / P.ngrp / D;
    constexpr int WPL = BITS / 2;
    constexpr int RPW = 64 / LPR;
    for (int it = 0; it < kDownRowsPerBlock / (4 * RPW); ++it) {
        const int o = blockIdx.x * kDownRowsPerBlock + it * 4 * RPW + wave * RPW + lane / LPR;
        float acc[MAXN];
#pragma unroll
        for (int j = 0; j < MAXN; ++j) acc[j] = 0.0f;
        if (active && o < H) {
            const size_t rowi = static_cast<size_t>(expert) * H + o;
            const uint32_t* pw = P.codes + rowi * P.words + (s0 / 32) * BITS + ((s0 % 32) / 16) * WPL;
            uint32_t wr[WPL + 1];
#pragma unroll
            for (int i = 0; i < WPL; ++i) wr[i] = pw[i];
            wr[WPL] = 0;
            float pp[MAXN];
#pragma unroll
            for (int j = 0; j < MAXN; ++j) pp[j] = 0.0f;
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const int s = s0 + q;
                const uint32_t c = code_from<BITS>(wr, q);
                float b[D];
                Vec<D>::load_book(P.book, c, b);
#pragma unroll
                for (int j = 0; j < MAXN; ++j) {
                    if (j < n) {
                        float xv[D];
                        Vec<D>::load_x(hs + j * I + s * D, xv);
#pragma unroll
                        for (int d = 0; d < D; ++d) pp[j] = fmaf(xv[d], b[d], pp[j]);
                    }
                }
                if (!row_scale && ((s + 1) % spg) == 0) {
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
        if (sub_lane == 0 && o < H) {
            const size_t rowi = static_cast<size_t>(expert) * H + o;
            const float sc = row_scale ? h2f(P.scales[rowi]) : 1.0f;
#pragma unroll
            for (int j = 0; j < MAXN; ++j)
                if (j < n) dbuf[static_cast<size_t>(pos0 + j) * H + o] = f2bf(acc[j] * sc);
        }
    }
}

// ============================================================== combine (R8, R10, R11)
__global__ __launch_bounds__(256) void k_combine(LayerDev L, int M, const int32_t* __restrict__ plan,
                                                 const float* __restrict__ weights, const float* __restrict__ sgate,
                                                 const uint16_t* __restrict__ dbuf, const uint16_t* hin,
                                                 uint16_t* out) {
    const int r = blockIdx.y;
    const int o = blockIdx.x * 256 + threadIdx.x;
    const int H = L.H, K = L.K, MK = M * K;
    if (o >= H) return;
    const int32_t* rpos = plan + 2 + 3 * MK;
    float routed = 0.0f;
    for (int s = 0; s < K; ++s)
        routed = fmaf(weights[r * K + s], bf2f(dbuf[static_cast<size_t>(rpos[r * K + s]) * H + o]), routed);
    float y = rbf(routed);
    if (L.has_shared) {
        const float sh = rbf(bf2f(dbuf[static_cast<size_t>(MK + r) * H + o]) * sgate[r]);
        y = rbf(y + sh);
    }
    const size_t i = static_cast<size_t>(r) * H + o;
    out[i] = hin ? f2bf(bf2f(hin[i]) + y) : f2bf(y);
}

__global__ __launch_bounds__(256) void k_rmsnorm(const uint16_t* __restrict__ x, int H, float eps,
                                                 uint16_t* __restrict__ y) {
    __shared__ float red[4];
    const int r = blockIdx.x, tid = threadIdx.x;
    float ss = 0.0f;
    for (int c = tid; c < H; c += 256) {
        const float v = bf2f(x[static_cast<size_t>(r) * H + c]);
        ss = fmaf(v, v, ss);
    }
    ss = wave_sum_xor(ss);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    const float t = (red[0] + red[1]) + (red[2] + red[3]);
    const float inv = 1.0f / sqrtf(t / static_cast<float>(H) + eps);
    for (int c = tid; c < H; c += 256)
        y[static_cast<size_t>(r) * H + c] = f2bf(bf2f(x[static_cast<size_t>(r) * H + c]) * inv);
}

// ============================================================== launchers
namespace {
template <int MAXM>
hipError_t launch_router_m(const LayerDev& L, const uint16_t* hin, int M, int do_norm, float eps, uint16_t* xn,
                           float* logits, float* sgate, hipStream_t st) {
    const int rows = L.E + (L.has_shared ? 1 : 0);
    const size_t lds = static_cast<size_t>(M) * L.H * 2;
    static bool attr = false;
    if (!attr) {
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&k_router<MAXM>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, 96 * 1024);
        attr = true;
    }
    hipLaunchKernelGGL(k_router<MAXM>, dim3((rows + 3) / 4), dim3(256), lds, st, L, hin, M, do_norm, eps, xn,
                       logits, sgate);
    return hipGetLastError();
}

template <int D, int BITS, int LPR>
hipError_t launch_gate_up_g(const LayerDev& L, const uint16_t* xn, int M, const int32_t* plan, uint16_t* hbuf,
                            hipStream_t st) {
    const dim3 grid((L.I + kGuRowsPerBlock - 1) / kGuRowsPerBlock, M * L.K + 1);
    const size_t lds = static_cast<size_t>(M) * L.H * 2;
    if (M <= 4) {
        static bool attr = false;
        if (!attr) { (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&k_gate_up<D, BITS, LPR, 4>), hipFuncAttributeMaxDynamicSharedMemorySize, 96 * 1024); attr = true; }
        hipLaunchKernelGGL((k_gate_up<D, BITS, LPR, 4>), grid, dim3(256), lds, st, L, xn, M, plan, hbuf);
    } else {
        static bool attr = false;
        if (!attr) { (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&k_gate_up<D, BITS, LPR, 16>), hipFuncAttributeMaxDynamicSharedMemorySize, 96 * 1024); attr = true; }
        hipLaunchKernelGGL((k_gate_up<D, BITS, LPR, 16>), grid, dim3(256), lds, st, L, xn, M, plan, hbuf);
    }
    return hipGetLastError();
}

template <int D, int BITS, int LPR>
hipError_t launch_down_g(const LayerDev& L, int M, const int32_t* plan, const uint16_t* hbuf, uint16_t* dbuf,
                         hipStream_t st) {
    const dim3 grid((L.H + kDownRowsPerBlock - 1) / kDownRowsPerBlock, M * L.K + 1);
    const size_t lds = static_cast<size_t>(M) * L.I * 2;
    if (M <= 4)
        hipLaunchKernelGGL((k_down<D, BITS, LPR, 4>), grid, dim3(256), lds, st, L, M, plan, hbuf, dbuf);
    else
        hipLaunchKernelGGL((k_down<D, BITS, LPR, 16>), grid, dim3(256), lds, st, L, M, plan, hbuf, dbuf);
    return hipGetLastError();
}

int next_pow2(int v) {
    int p = 1;
    while (p < v) p <<= 1;
    return p;
}
} // namespace

hipError_t launch_router(const LayerDev& L, const uint16_t* hin, int M, int do_norm, float eps, uint16_t* xn,
                         float* logits, float* sgate, hipStream_t st) {
    if (M <= 1) return launch_router_m<1>(L, hin, M, do_norm, eps, xn, logits, sgate, st);
    if (M <= 2) return launch_router_m<2>(L, hin, M, do_norm, eps, xn, logits, sgate, st);
    if (M <= 4) return launch_router_m<4>(L, hin, M, do_norm, eps, xn, logits, sgate, st);
    if (M <= 8) return launch_router_m<8>(L, hin, M, do_norm, eps, xn, logits, sgate, st);
    return launch_router_m<16>(L, hin, M, do_norm, eps, xn, logits, sgate, st);
}

hipError_t launch_topk_plan(const LayerDev& L, const float* logits, int M, int32_t* experts, float* weights,
                            int32_t* plan, hipStream_t st) {
    hipLaunchKernelGGL(k_topk_plan, dim3(1), dim3(1024), 0, st, logits, M, L.E, L.K, L.normalize, experts, weights,
                       plan);
    return hipGetLastError();
}

hipError_t launch_gate_up(const LayerDev& L, const uint16_t* xn, int M, const int32_t* plan, uint16_t* hbuf,
                          hipStream_t st) {
    const int D = L.p[0].dim, B = L.p[0].bits;
    const int lpr = next_pow2((L.H / D + 15) / 16);
    if (D == 8 && B == 14) {
        if (lpr == 16) return launch_gate_up_g<8, 14, 16>(L, xn, M, plan, hbuf, st);
        if (lpr == 32) return launch_gate_up_g<8, 14, 32>(L, xn, M, plan, hbuf, st);
        if (lpr == 8) return launch_gate_up_g<8, 14, 8>(L, xn, M, plan, hbuf, st);
        if (lpr <= 4) return launch_gate_up_g<8, 14, 4>(L, xn, M, plan, hbuf, st);
    } else if (D == 4 && B == 8) {
        if (lpr == 32) return launch_gate_up_g<4, 8, 32>(L, xn, M, plan, hbuf, st);
        if (lpr == 64) return launch_gate_up_g<4, 8, 64>(L, xn, M, plan, hbuf, st);
        if (lpr == 16) return launch_gate_up_g<4, 8, 16>(L, xn, M, plan, hbuf, st);
        if (lpr <= 8) return launch_gate_up_g<4, 8, 8>(L, xn, M, plan, hbuf, st);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_down(const LayerDev& L, int M, const int32_t* plan, const uint16_t* hbuf, uint16_t* dbuf,
                       hipStream_t st) {
    const int D = L.p[2].dim, B = L.p[2].bits;
    const int lpr = next_pow2((L.I / D + 15) / 16);
    if (D == 8 && B == 14) {
        if (lpr == 4) return launch_down_g<8, 14, 4>(L, M, plan, hbuf, dbuf, st);
        if (lpr == 8) return launch_down_g<8, 14, 8>(L, M, plan, hbuf, dbuf, st);
        if (lpr <= 2) return launch_down_g<8, 14, 2>(L, M, plan, hbuf, dbuf, st);
    } else if (D == 4 && B == 8) {
        if (lpr == 8) return launch_down_g<4, 8, 8>(L, M, plan, hbuf, dbuf, st);
        if (lpr == 16) return launch_down_g<4, 8, 16>(L, M, plan, hbuf, dbuf, st);
        if (lpr == 4) return launch_down_g<4, 8, 4>(L, M, plan, hbuf, dbuf, st);
        if (lpr <= 2) return launch_down_g<4, 8, 2>(L, M, plan, hbuf, dbuf, st);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_combine(const LayerDev& L, int M, const int32_t* plan, const float* weights, const float* sgate,
                          const uint16_t* dbuf, const uint16_t* hin, uint16_t* out, hipStream_t st) {
    hipLaunchKernelGGL(k_combine, dim3((L.H + 255) / 256, M), dim3(256), 0, st, L, M, plan, weights, sgate, dbuf,
                       hin, out);
    return hipGetLastError();
}

hipError_t launch_rmsnorm(const uint16_t* x, int M, int H, float eps, uint16_t* y, hipStream_t st) {
    hipLaunchKernelGGL(k_rmsnorm, dim3(M), dim3(256), 0, st, x, H, eps, y);
    return hipGetLastError();
}

hipError_t launch_gen_codes(uint64_t key, int e0, int n_experts, int out_dim, int nsub, int bits, int words,
                            uint32_t* codes, hipStream_t st) {
    hipLaunchKernelGGL(k_gen_codes, dim3(4096), dim3(256), 0, st, key, e0, n_experts, out_dim, nsub, bits, words,
                       codes);
    return hipGetLastError();
}
hipError_t launch_gen_uniform_f16(uint64_t key, int64_t idx0, int64_t n, double lo, double hi, uint16_t* out,
                                  hipStream_t st) {
    hipLaunchKernelGGL(k_gen_uniform_f16, dim3(2048), dim3(256), 0, st, key, idx0, n, lo, hi, out);
    return hipGetLastError();
}
hipError_t launch_gen_normal(uint64_t key, int64_t n, double sd, int f16, uint16_t* out, hipStream_t st) {
    hipLaunchKernelGGL(k_gen_normal, dim3(2048), dim3(256), 0, st, key, n, sd, f16, out);
    return hipGetLastError();
}
hipError_t launch_gen_embed(uint64_t seed, const uint32_t* tokens, int n, int H, uint16_t* out, hipStream_t st) {
    if (n > 32) return hipErrorInvalidValue;
    TokenList tl{};
    for (int i = 0; i < n; ++i) tl.t[i] = tokens[i];
    hipLaunchKernelGGL(k_gen_embed, dim3((n * H + 255) / 256), dim3(256), 0, st,
                       stream_key(seed, kEmbedLayer, T_EMBED), tl, n, H, out);
    return hipGetLastError();
}
hipError_t launch_book_to_int8(const uint16_t* book16, int n, int8_t* q8, uint16_t* scale, hipStream_t st) {
    hipLaunchKernelGGL(k_book_to_int8, dim3(1), dim3(1024), 0, st, book16, n, q8, scale);
    return hipGetLastError();
}

} // namespace q38
