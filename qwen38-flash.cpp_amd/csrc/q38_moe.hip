// q38_moe.hip — gfx950 kernels of one packed-VQ sparse-MoE layer at verify width
// (rows <= 16), plus the synthetic-weight generators.
//
// Per layer the launch sequence is
//   k_route_norm  router logits with the fixed-order contract (R1) + the shared-expert
//                 gate logit, with the layer-input RMSNorm of the verify chain folded in;
//                 one wave per row of Wr, H/4 threads per workgroup.
//   k_topk_plan   softmax / top-k / normalise per row (R2) and the gather-by-expert plan
//                 (R3): unique experts ascending, each with its routes in (row, slot)
//                 order; one workgroup.
//   k_gu_mfma     gate and up projections (R4, R5, R7): persistent workgroups, each with
//                 one 4-dim chunk of one codebook resident in LDS, MFMA tiles over every
//                 routed row of an expert, so each packed code row is read once per chunk.
//   k_down_mfma   SwiGLU of the gate/up sums + down projection (R7, R8), same scheme.
//   k_combine     ordered route reduction (slot order) + shared expert x sigmoid gate +
//                 merge (R8, R10, R11); in a chain it adds the residual in place.
// Rows <= 4 take the narrow kernels of q38_moe4.hip instead of k_topk_plan + k_*_mfma.
// Mixed layers (two codebook geometries by expert parity) run k_gu_mfma / k_down_mfma once
// per bank. Layers with per-64-input scale groups use the k_*_grouped VALU kernels.
#ifdef Q38_TRACE
#define g_trace g_trace_route  // (each code object holds its own stamp buffer)
#endif
#include "q38_device.hpp"
#include "q38_internal.hpp"
#include "q38_moe_dev.hpp"

#include <mutex>

namespace q38 {

// ============================================================== generators
__global__ void k_gen_codes(uint64_t key, int e0, int e_stride, int n_experts, int out_dim, int nsub, int bits,
                            int words, uint32_t* __restrict__ codes) {
    // one thread per (expert, row, 32-code block)
    const int nblk = (nsub + 31) / 32;
    const int64_t total = static_cast<int64_t>(n_experts) * out_dim * nblk;
    for (int64_t t = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; t < total;
         t += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int blk = static_cast<int>(t % nblk);
        const int64_t row = t / nblk;  // local (expert, o)
        const int o = static_cast<int>(row % out_dim);
        const int e = e0 + e_stride * static_cast<int>(row / out_dim);
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

__global__ void k_gen_scales(uint64_t key, int e0, int e_stride, int n_experts, int out_dim, double lo, double hi,
                             uint16_t* __restrict__ out) {
    const int64_t n = static_cast<int64_t>(n_experts) * out_dim;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t e = e0 + static_cast<int64_t>(e_stride) * (i / out_dim);
        out[i] = f2h(uniform_f32(key, static_cast<uint64_t>(e * out_dim + i % out_dim), lo, hi));
    }
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

__global__ void k_gen_embed_dev(uint64_t key, const uint32_t* __restrict__ toks, int n, int H,
                                uint16_t* __restrict__ out) {
    const int64_t total = static_cast<int64_t>(n) * H;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int r = static_cast<int>(i / H), c = static_cast<int>(i % H);
        const double z = normal_at(key, static_cast<uint64_t>(toks[r]) * H + c);
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

// SparseMoe::prepare_u8_codebook (src/sparse_moe.cpp:750-804) of a [K, 8] fp16 book in one
// workgroup: per-dimension min/max (order-free), scale = (max - min) / 255 (1 when not > 0),
// centred q = clamp(lround(v / scale), -128, 127) or affine q = clamp(lround((v - min) /
// scale), 0, 255), fp16 scale and bias (= min). The book the kernels read is the float decode
// q * f16(scale) (+ f16(min)) (src/vq_metal_kernels.hpp:564-579) rounded to fp16.
__global__ __launch_bounds__(1024) void k_prepare_u8(const uint16_t* __restrict__ book16, int K, int centered,
                                                      uint8_t* __restrict__ q, uint16_t* __restrict__ s16,
                                                      uint16_t* __restrict__ b16, uint16_t* __restrict__ dec) {
    constexpr int D = 8;
    __shared__ float red[2][16][D];
    __shared__ float sc[D], mn[D];
    float lo[D], hi[D];
#pragma unroll
    for (int d = 0; d < D; ++d) {
        lo[d] = INFINITY;
        hi[d] = -INFINITY;
    }
    for (int r = threadIdx.x; r < K; r += blockDim.x) {
        const uint4 v = reinterpret_cast<const uint4*>(book16)[r];
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const float x = h2f(static_cast<uint16_t>(w[d / 2] >> (16 * (d & 1))));
            lo[d] = fminf(lo[d], x);
            hi[d] = fmaxf(hi[d], x);
        }
    }
#pragma unroll
    for (int d = 0; d < D; ++d) {
        for (int off = 32; off >= 1; off >>= 1) {
            lo[d] = fminf(lo[d], __shfl_xor(lo[d], off, kWave));
            hi[d] = fmaxf(hi[d], __shfl_xor(hi[d], off, kWave));
        }
        if ((threadIdx.x & 63) == 0) {
            red[0][threadIdx.x >> 6][d] = lo[d];
            red[1][threadIdx.x >> 6][d] = hi[d];
        }
    }
    __syncthreads();
    if (threadIdx.x < D) {
        const int d = threadIdx.x;
        float a = INFINITY, b = -INFINITY;
        for (int w = 0; w < static_cast<int>(blockDim.x >> 6); ++w) {
            a = fminf(a, red[0][w][d]);
            b = fmaxf(b, red[1][w][d]);
        }
        float s = (b - a) / 255.0f;
        if (!(s > 0.0f)) s = 1.0f;
        sc[d] = s;
        mn[d] = a;
        s16[d] = f2h(s);
        b16[d] = f2h(a);
    }
    __syncthreads();
    for (int i = threadIdx.x; i < K * D; i += blockDim.x) {
        const int d = i % D;
        const float v = h2f(book16[i]);
        const float t = centered ? v / sc[d] : (v - mn[d]) / sc[d];
        const float r = roundf(t);  // (half away from zero, as lround)
        const float qf = centered ? fminf(127.0f, fmaxf(-128.0f, r)) : fminf(255.0f, fmaxf(0.0f, r));
        const int qi = static_cast<int>(qf);
        q[i] = static_cast<uint8_t>(qi);
        float wv = static_cast<float>(qi) * h2f(f2h(sc[d]));
        if (!centered) wv = wv + h2f(f2h(mn[d]));
        dec[i] = f2h(wv);
    }
}

// ============================================================== router (R1) + layer-input RMSNorm
// One workgroup of H/4 threads per NW = H/256 router rows (wave w: row blockIdx.x * NW + w;
// row E is w_sg). The router rows are requested first: they do not depend on the previous
// kernel. NORM: the layer input is x = T(h * inv_rms(h)) of the residual stream h, formed
// in every workgroup in one fixed order: thread t owns columns t + (H/4) i (i < 4) and
// accumulates fmaf(v, v) in i order; the waves' xor-butterfly totals are added in wave
// order; inv_rms = 1 / sqrt(total / H + eps). Otherwise src is x itself.
// Logit contract: lane l holds the columns c = 512t + 8l + j and accumulates x*w over them
// (t outer, j inner) with fmaf, then the xor butterfly and BF16 rounding; a router bias,
// when set, is added to the rounded logit in float. Workgroup 0 stores x in the workspace
// (bf16) with its fp16 copy (the MFMA operand) unless src already is that copy.
// reset_gu: the gate/up and down chunk planes of the call ([2][M*K + M][I] each for g and u,
// [2][M*K + M][H] for d) are set to the all-ones pattern that the fused layer kernel (k_gd4)
// waits on.
template <int T, bool NORM, int MR>
__global__ __launch_bounds__(128 * T) void k_route_norm(LayerDev L, MoeBufs B, int M, const uint16_t* __restrict__ src,
                                                        float eps, int reset_gu) {
    constexpr int H = 512 * T, NT = 128 * T, NW = NT / 64;
    extern __shared__ __align__(16) uint16_t xs[];  // [M][H] bf16
    __shared__ float red[MR][NW];
    touch_kernargs<sizeof(LayerDev) + sizeof(MoeBufs) + 2 * sizeof(void*) + sizeof(float) + sizeof(int)>();
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nr = L.E + (L.has_shared ? 1 : 0);
    const int e = blockIdx.x * NW + wave;
    Q38_STAMP(0, 0);
    const bool store = blockIdx.x == 0 && src != B.x;
    // The layer input is requested first (it gates the norm); the router rows are needed
    // only for the dot products and stream in behind it. MR >= M rows are loaded without
    // branches (rows past M repeat row M - 1) so that every load is in flight at once.
    uint16_t hraw[NORM ? MR : 1][4];
    if constexpr (NORM) {
#pragma unroll
        for (int r = 0; r < MR; ++r) {
            const int rr = r < M ? r : M - 1;
#pragma unroll
            for (int i = 0; i < 4; ++i) hraw[r][i] = src[static_cast<size_t>(rr) * H + tid + NT * i];
        }
    }
    __builtin_amdgcn_sched_barrier(0);  // (the input's loads stay ahead of the router rows')
    uint4 wv[T];
    {
        const int ew = e < nr ? e : nr - 1;
        const uint16_t* w = ew < L.E ? L.router + static_cast<size_t>(ew) * H : L.wsg;
#pragma unroll
        for (int t = 0; t < T; ++t) wv[t] = *reinterpret_cast<const uint4*>(w + 512 * t + 8 * lane);
    }
    // (the scheduler would otherwise sink the router-row loads below the norm's wait for
    // the layer input, and the two memory latencies would add up)
    __builtin_amdgcn_sched_barrier(0);
    float v[NORM ? MR : 1][4];
    if constexpr (NORM) {
#pragma unroll
        for (int r = 0; r < MR; ++r)
#pragma unroll
            for (int i = 0; i < 4; ++i) v[r][i] = bf2f(hraw[r][i]);
        Q38_STAMPV(0, 1, v[0][0]);
        norm_partials<NT, MR>(v, red);
        lds_barrier();
        Q38_STAMP(0, 6);
        // Lane r forms row r's total (wave totals in wave order) and 1 / rms, one chain for
        // all rows instead of MR chains in every lane (the phase is VALU-bound); the results
        // are read back from lanes 0..MR-1.
        float inv[MR];
        norm_inv<NT, MR>(red, H, eps, inv);
#pragma unroll
        for (int r = 0; r < MR; ++r)
            if (r < M) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const size_t at = static_cast<size_t>(r) * H + tid + NT * i;
                    const uint16_t b = f2bf(v[r][i] * inv[r]);
                    xs[at] = b;
                    if (store) {
                        B.x[at] = b;
                        B.x16[at] = f2h(bf2f(b));
                    }
                }
            }
        Q38_STAMP(0, 7);
    } else {
        const uint4* s4 = reinterpret_cast<const uint4*>(src);
        for (int i = tid; i < M * H / 8; i += NT) {
            const uint4 q4 = s4[i];
            reinterpret_cast<uint4*>(xs)[i] = q4;
            if (store) {
                reinterpret_cast<uint4*>(B.x)[i] = q4;
                const uint32_t q[4] = {q4.x, q4.y, q4.z, q4.w};
                uint32_t hq[4];
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    hq[k] = static_cast<uint32_t>(f2h(bflo(q[k]))) | (static_cast<uint32_t>(f2h(bfhi(q[k]))) << 16);
                reinterpret_cast<uint4*>(B.x16)[i] = make_uint4(hq[0], hq[1], hq[2], hq[3]);
            }
        }
    }
    lds_barrier();
    Q38_STAMP(0, 2);
    if (reset_gu) {
        const size_t n4 = B.gu_plane / 2, d4 = B.d_plane / 2;  // 16-byte stores per [2][rows][I or H] block
        const uint4 ones = make_uint4(~0u, ~0u, ~0u, ~0u);
        for (size_t i = static_cast<size_t>(blockIdx.x) * NT + tid; i < 2 * n4 + d4;
             i += static_cast<size_t>(gridDim.x) * NT) {
            uint4* dst = i < n4 ? reinterpret_cast<uint4*>(B.g) + i
                                : i < 2 * n4 ? reinterpret_cast<uint4*>(B.u) + (i - n4)
                                             : reinterpret_cast<uint4*>(B.d) + (i - 2 * n4);
            *dst = ones;
        }
    }
    Q38_STAMP(0, 4);
    if (e >= nr) return;
    // all rows' products first (independent chains), then the butterflies
    float acc[MR];
    router_dots<T, MR>(xs, M, wv, acc);
    Q38_STAMPV(0, 5, acc[0]);
#pragma unroll
    for (int s = 0; s < scatter_slots<MR>(); ++s) {
        const int r = MR > 1 ? scatter_value<MR>(s, lane >> 4) : 0;
        const float sres = acc[s];
        if (scatter_leader<MR>(lane) && r < M) {
            if (e < L.E) {
                B.logits[r * L.E + e] = L.rbias ? rbf(sres) + L.rbias[e] : rbf(sres);
            } else {
                const float lg = rbf(sres);
                B.sgate[r] = rbf(1.0f / (1.0f + expf(-lg)));
            }
        }
    }
    Q38_STAMP(0, 3);
}

__global__ __launch_bounds__(1024) void k_topk_plan(LayerDev L, MoeBufs B, int M) {
    __shared__ TopkLds t;
    topk_plan_block(L, B, M, true, B.plan, t, 0);
}

// ============================================================== MFMA expert projections
// A workgroup holds one 4-dim chunk of one projection's codebook in LDS (128 KiB for
// d8/14-bit) for the whole launch and walks its share of (expert slot, 128-row tile)
// items. A wave computes a 16-row x (up to 8 routed rows) tile with
// v_mfma_f32_16x16x32_f16: A = codebook entries looked up in LDS by the packed codes of
// the 16 rows (lane (r, q) decodes the codes of row r for subvectors [q*S4, (q+1)*S4)),
// B = the chunk's dims of the routed rows' inputs (fp16, staged in LDS). Every code row
// is read once per chunk; the next item's code words are loaded while the current item
// computes. Chunk partial sums (times the row scale) are added into fp32 accumulators,
// two addends each for d8 (order-independent).
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));

constexpr int kMfmaThreads = 512;       // 8 waves
constexpr int kMfmaRowsPerItem = 128;   // 8 waves x 16 rows
constexpr int kMfmaMaxCols = 8;         // routed rows staged per pass
// Gate/up: routed rows staged per pass. With an 8-bit codebook (2 KiB) the LDS holds all 16
// B columns of the MFMA tile, so up to 16 request rows are staged once per workgroup; a
// 14-bit codebook chunk (128 KiB) leaves room for 8.
__host__ __device__ constexpr int gu_mfma_cols(int bits) { return bits <= 8 ? 16 : kMfmaMaxCols; }

template <int BITS, int NSUB>
__device__ __forceinline__ void load_lane_words(const uint32_t* src, uint32_t* w) {
    constexpr int WPL = (NSUB / 4) * BITS / 32;
    if constexpr (WPL % 4 == 0) {
#pragma unroll
        for (int i = 0; i < WPL / 4; ++i) {
            const uint4 v = reinterpret_cast<const uint4*>(src)[i];
            w[4 * i] = v.x; w[4 * i + 1] = v.y; w[4 * i + 2] = v.z; w[4 * i + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < WPL; ++i) w[i] = src[i];
    }
    w[WPL] = 0;
}

// One 16-row MFMA tile over all subvectors of one chunk. xlane: this lane's B row in LDS
// (a zeroed row for lanes without a routed row), already offset to its q block.
template <int BITS, int NSUB>
__device__ __forceinline__ f4_t mfma_tile(const uint32_t* w, const uint2* book, const uint4* xlane) {
    constexpr int S4 = NSUB / 4;
    f4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < S4 / 2; ++t) {
        const uint32_t c1 = code_from<BITS>(w, 2 * t);
        const uint32_t c2 = code_from<BITS>(w, 2 * t + 1);
        const uint2 a1 = book[c1];
        const uint2 a2 = book[c2];
        const uint4 av = make_uint4(a1.x, a1.y, a2.x, a2.y);
        const uint4 bv = xlane[t];
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8_t, av), __builtin_bit_cast(h8_t, bv),
                                                     acc, 0, 0, 0);
    }
    return acc;
}
// Staged B rows: row r, lane quarter q (subvectors q S4 .. q S4 + S4 - 1, 8 bytes each) at
// byte r * RB + q * QB. The strides are padded so that one B read of the MFMA loop (16
// columns x 4 quarters, 16 bytes each) spreads over the LDS banks: with unpadded rows every
// lane of it lands in the same 16-byte bank group. Row strides are 16 mod 256 bytes and
// quarter strides 64 or 192 mod 256 (128 for 16-subvector quarters), so distinct rows and
// quarters take distinct 16-byte slots of a 256-byte bank cycle, four lanes per slot.
template <int NSUB>
struct XsLayout {
    static constexpr int S4 = NSUB / 4;
    static constexpr int QB = S4 * 8 >= 256 ? S4 * 8 + 64 : S4 * 8;
    static constexpr int RB = 4 * QB + 16;
    __device__ static uint2* at(uint4* xs, int row, int sv) {
        return reinterpret_cast<uint2*>(reinterpret_cast<unsigned char*>(xs) + row * RB + (sv / S4) * QB +
                                        (sv % S4) * 8);
    }
};
// B row base for lane (row xrow, block q) or the zero row when inactive.
template <int NSUB>
__device__ __forceinline__ const uint4* xs_lane(const uint4* xs, int xrow, int zero_row, int q, bool active) {
    return reinterpret_cast<const uint4*>(reinterpret_cast<const unsigned char*>(xs) +
                                          (active ? xrow : zero_row) * XsLayout<NSUB>::RB + q * XsLayout<NSUB>::QB);
}

constexpr int kPlanSlots = kMaxRows * kMaxTopK + 1;  // unique-expert slots + the shared one

// Mixed layers: the index of expert e in its bank (even experts and the shared expert E
// in bank 0, odd experts in bank 1, both at e / 2); uniform layers: e.
template <int PAR>
__device__ __forceinline__ int bank_index(int e) { return PAR < 0 ? e : e >> 1; }

// The plan's slots (unique experts ascending, then the shared expert E, which is even)
// whose expert has parity par, in slot order, into out; returns their count. Every
// thread calls it; the list is complete after the block barrier inside.
__device__ __forceinline__ int parity_slots(const int32_t* plan, int nu, int has_shared, int E, int par,
                                            int32_t* out) {
    __shared__ int32_t cnt;
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        const int ns = nu + (has_shared ? 1 : 0);
        int base = 0;
        for (int u0 = 0; u0 < ns; u0 += 64) {
            const int u = u0 + lane;
            const int e = u < nu ? plan[1 + u] : E;
            const bool take = u < ns && (e & 1) == par;
            const uint64_t m = __ballot(take);
            if (take) out[base + __popcll(m & ((1ull << lane) - 1ull))] = u;
            base += __popcll(m);
        }
        if (lane == 0) cnt = base;
    }
    __syncthreads();
    return cnt;
}

// PAR >= 0 (mixed layers): only the slots whose expert has that parity, with the
// geometry of that bank (L.pb[proj][PAR], expert index e / 2); the even bank (one codebook
// chunk) also clears plane 1 of its outputs, so a consumer can add both planes for every
// route. The even bank's launch routes and publishes the plan; the odd bank's launch,
// which follows it, reads the plan.
template <int BITS, int NSUB, int NCHUNK, int PAR = -1>
__global__ __launch_bounds__(kMfmaThreads) void k_gu_mfma(LayerDev L, MoeBufs B, int M) {
    extern __shared__ __align__(16) unsigned char lds[];
    __shared__ TopkLds tk;
    __shared__ int32_t plan[kPlanInts];
    __shared__ int32_t pslots[PAR < 0 ? 1 : kPlanSlots];
    constexpr int KENT = 1 << BITS;
    constexpr int MAXC = gu_mfma_cols(BITS);
    const uint2* book = reinterpret_cast<const uint2*>(lds);       // [KENT] x 4 fp16
    uint4* xs = reinterpret_cast<uint4*>(lds + KENT * 8);          // [MAXC + 1 zero] rows (XsLayout), 4 fp16 per subvector
    constexpr int TYPES = 2 * NCHUNK;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int x8 = blockIdx.x & 7, kk = blockIdx.x >> 3;
    const int type = kk % TYPES;
    const int proj = type / NCHUNK, chunk = type % NCHUNK;
    const int per_type = (gridDim.x / (8 * TYPES)) * 8;
    const int idx = (kk / TYPES) * 8 + x8;
    const ProjDev& P = PAR < 0 ? L.p[proj] : L.pb[proj][PAR < 0 ? 0 : PAR];
    // waves 0-3 load the codebook chunk while waves 4-7 route; every workgroup derives
    // the same plan and workgroup 0 publishes it
    if (PAR == 1) {
        // the odd bank runs right after the even bank's launch, which routed and published
        // the plan (and the routes) on the same stream
        for (int i = tid; i < 2 + 4 * M * L.K; i += kMfmaThreads) plan[i] = B.plan[i];
        fill_book<KENT>(P.book4 + static_cast<size_t>(chunk) * KENT * 4, lds, tid, kMfmaThreads);
        __syncthreads();
    } else {
        // an 8-bit book (2 KiB) is one load per thread of waves 0-3, which then route too
        constexpr int route_wave0 = KENT <= 256 ? 0 : 4;
        if (wave < 4) fill_book<KENT>(P.book4 + static_cast<size_t>(chunk) * KENT * 4, lds, tid, 256);
        topk_plan_block(L, B, M, blockIdx.x == 0, plan, tk, route_wave0);
        if (blockIdx.x == 0)
            for (int i = tid; i < 2 + 4 * M * L.K; i += kMfmaThreads) B.plan[i] = plan[i];
    }
    const int H = L.H, I = L.I, K = L.K;
    const int nu = plan[0];
    const int nslots = PAR < 0 ? nu + (L.has_shared ? 1 : 0) : parity_slots(plan, nu, L.has_shared, L.E, PAR, pslots);
    const int n_items = nslots * (I / kMfmaRowsPerItem);
    const int tiles = I / kMfmaRowsPerItem;
    auto slot_of = [&](int item) { return PAR < 0 ? item / tiles : pslots[item / tiles]; };
    float* out = (proj == 0 ? B.g : B.u) + chunk * B.gu_plane;
    const int r16 = lane & 15, q = lane >> 4;
    constexpr int S4 = NSUB / 4;
    constexpr int WPL = S4 * BITS / 32;
    // Verify widths (M <= MAXC): the chunk's dims of every request row are staged once.
    const bool stage_all = M <= MAXC;
    if (stage_all) {
        for (int i = tid; i < M * NSUB; i += kMfmaThreads) {
            const int row = i / NSUB, sv = i % NSUB;
            *XsLayout<NSUB>::at(xs, row, sv) =
                *reinterpret_cast<const uint2*>(B.x16 + static_cast<size_t>(row) * H + sv * (4 * NCHUNK) + 4 * chunk);
        }
    }
    for (int i = tid; i < NSUB; i += kMfmaThreads)
        *XsLayout<NSUB>::at(xs, MAXC, i) = make_uint2(0u, 0u);
    lds_barrier();
    auto code_src = [&](int item) {
        int expert, n, pos0;
        slot_rows(plan, M, K, L.has_shared, slot_of(item), L.E, &expert, &n, &pos0);
        const size_t rowi =
            static_cast<size_t>(bank_index<PAR>(expert)) * I + (item % tiles) * kMfmaRowsPerItem + wave * 16 + r16;
        return P.codes + rowi * P.words + q * WPL;
    };
    // Mixed banks: a contiguous range of items, so that consecutive items mostly share a slot
    // and its staged rows (restaged only when the slot or the pass changes). Uniform layers:
    // items strided over the workgroups (the shared slot's 16 rows take two passes per tile,
    // and a contiguous range would put all its tiles on one workgroup).
    constexpr bool CONTIG = PAR >= 0;
    const int i0 = CONTIG ? static_cast<int>(static_cast<int64_t>(idx) * n_items / per_type) : idx;
    const int i1 = CONTIG ? static_cast<int>(static_cast<int64_t>(idx + 1) * n_items / per_type) : n_items;
    const int istep = CONTIG ? 1 : per_type;
    int staged_slot = -1, staged_j0 = -1;
    uint32_t w[WPL + 1], wn[WPL + 1];
    if (i0 < i1) load_lane_words<BITS, NSUB>(code_src(i0), w);
    for (int item = i0; item < i1; item += istep) {
        if (item + istep < i1) load_lane_words<BITS, NSUB>(code_src(item + istep), wn);
        const int ui = slot_of(item), tile = item % tiles;
        int expert, n, pos0;
        slot_rows(plan, M, K, L.has_shared, ui, L.E, &expert, &n, &pos0);
        const bool shared = ui == nu;
        const int o0 = tile * kMfmaRowsPerItem + wave * 16;
        for (int j0 = 0; j0 < n; j0 += MAXC) {
            const int nj = n - j0 < MAXC ? n - j0 : MAXC;
            int xrow = r16;
            if (stage_all) {
                if (r16 < nj) xrow = route_row(plan, M, K, pos0, j0 + r16, shared);
            } else if (ui != staged_slot || j0 != staged_j0) {
                staged_slot = ui;
                staged_j0 = j0;
                lds_barrier();
                for (int i = tid; i < nj * NSUB; i += kMfmaThreads) {
                    const int jj = i / NSUB, sv = i % NSUB;
                    const int row = route_row(plan, M, K, pos0, j0 + jj, shared);
                    *XsLayout<NSUB>::at(xs, jj, sv) = *reinterpret_cast<const uint2*>(
                        B.x16 + static_cast<size_t>(row) * H + sv * (4 * NCHUNK) + 4 * chunk);
                }
                lds_barrier();
            }
            const f4_t acc = mfma_tile<BITS, NSUB>(w, book, xs_lane<NSUB>(xs, xrow, MAXC, q, r16 < nj));
            if (r16 < nj) {
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) {
                    const int o = o0 + 4 * q + rr;
                    const float sc = h2f(P.scales[static_cast<size_t>(bank_index<PAR>(expert)) * I + o]);
                    out[static_cast<size_t>(pos0 + j0 + r16) * I + o] = sc * acc[rr];
                    if (PAR >= 0 && NCHUNK == 1) out[B.gu_plane + static_cast<size_t>(pos0 + j0 + r16) * I + o] = 0.0f;
                }
            }
        }
#pragma unroll
        for (int i = 0; i <= WPL; ++i) w[i] = wn[i];
    }
}

constexpr int kDownStageRoutes = 48;  // routes whose SwiGLU rows are staged once (M <= 4 with k = 10)

// PAR >= 0: one bank of a mixed layer, as in k_gu_mfma (the even bank clears plane 1).
template <int BITS, int NSUB, int NCHUNK, int PAR = -1>
__global__ __launch_bounds__(kMfmaThreads) void k_down_mfma(LayerDev L, MoeBufs B, int M) {
    extern __shared__ __align__(16) unsigned char lds[];
    __shared__ int32_t plan[kPlanInts];
    __shared__ int32_t pslots[PAR < 0 ? 1 : kPlanSlots];
    constexpr int KENT = 1 << BITS;
    const uint2* book = reinterpret_cast<const uint2*>(lds);
    uint4* xs = reinterpret_cast<uint4*>(lds + KENT * 8);   // [routes + 1 zero] SwiGLU rows (XsLayout), 4 fp16 each
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int x8 = blockIdx.x & 7, kk = blockIdx.x >> 3;
    const int chunk = kk % NCHUNK;
    const int per_type = (gridDim.x / (8 * NCHUNK)) * 8;
    const int idx = (kk / NCHUNK) * 8 + x8;
    const ProjDev& P = PAR < 0 ? L.p[2] : L.pb[2][PAR < 0 ? 0 : PAR];
    const int H = L.H, I = L.I, K = L.K;
    const int n_routes = M * K + (L.has_shared ? M : 0);
    for (int i = tid; i < 2 + 4 * M * K; i += kMfmaThreads) plan[i] = B.plan[i];
    fill_book<KENT>(P.book4 + static_cast<size_t>(chunk) * KENT * 4, lds, tid, kMfmaThreads);
    // SwiGLU rows of every route, once (verify widths)
    const bool stage_all = n_routes <= kDownStageRoutes;
    auto stage = [&](int r0, int nr) {
        for (int i = tid; i < nr * NSUB; i += kMfmaThreads) {
            const int j = i / NSUB, sv = i % NSUB;
            const size_t base = static_cast<size_t>(r0 + j) * I + sv * (4 * NCHUNK) + 4 * chunk;
            float4 gv = *reinterpret_cast<const float4*>(B.g + base);
            float4 uv = *reinterpret_cast<const float4*>(B.u + base);
            if (L.gu_parts == 2) {
                const float4 g1 = *reinterpret_cast<const float4*>(B.g + B.gu_plane + base);
                const float4 u1 = *reinterpret_cast<const float4*>(B.u + B.gu_plane + base);
                gv = make_float4(gv.x + g1.x, gv.y + g1.y, gv.z + g1.z, gv.w + g1.w);
                uv = make_float4(uv.x + u1.x, uv.y + u1.y, uv.z + u1.z, uv.w + u1.w);
            }
            const uint32_t h0 = f2h(swiglu(gv.x, uv.x)), h1 = f2h(swiglu(gv.y, uv.y));
            const uint32_t h2 = f2h(swiglu(gv.z, uv.z)), h3 = f2h(swiglu(gv.w, uv.w));
            *XsLayout<NSUB>::at(xs, j, sv) = make_uint2(h0 | (h1 << 16), h2 | (h3 << 16));
        }
    };
    if (stage_all) stage(0, n_routes);
    for (int i = tid; i < NSUB; i += kMfmaThreads)
        *XsLayout<NSUB>::at(xs, kDownStageRoutes, i) = make_uint2(0u, 0u);
    lds_barrier();
    float* dout = B.d + chunk * B.d_plane;
    const int nu = plan[0];
    const int tiles = H / kMfmaRowsPerItem;
    const int nslots = PAR < 0 ? nu + (L.has_shared ? 1 : 0) : parity_slots(plan, nu, L.has_shared, L.E, PAR, pslots);
    const int n_items = nslots * tiles;
    auto slot_of = [&](int item) { return PAR < 0 ? item / tiles : pslots[item / tiles]; };
    const int r16 = lane & 15, q = lane >> 4;
    constexpr int S4 = NSUB / 4;
    constexpr int WPL = S4 * BITS / 32;
    auto code_src = [&](int item) {
        int expert, n, pos0;
        slot_rows(plan, M, K, L.has_shared, slot_of(item), L.E, &expert, &n, &pos0);
        const size_t rowi =
            static_cast<size_t>(bank_index<PAR>(expert)) * H + (item % tiles) * kMfmaRowsPerItem + wave * 16 + r16;
        return P.codes + rowi * P.words + q * WPL;
    };
    // a contiguous range of items (see k_gu_mfma): a slot's routes (all of them when they fit
    // the staging rows) are staged once for its consecutive items
    const int i0 = static_cast<int>(static_cast<int64_t>(idx) * n_items / per_type);
    const int i1 = static_cast<int>(static_cast<int64_t>(idx + 1) * n_items / per_type);
    int staged_slot = -1, staged_j0 = -1;
    uint32_t w[WPL + 1], wn[WPL + 1];
    if (i0 < i1) load_lane_words<BITS, NSUB>(code_src(i0), w);
    for (int item = i0; item < i1; ++item) {
        if (item + 1 < i1) load_lane_words<BITS, NSUB>(code_src(item + 1), wn);
        const int ui = slot_of(item), tile = item % tiles;
        int expert, n, pos0;
        slot_rows(plan, M, K, L.has_shared, ui, L.E, &expert, &n, &pos0);
        const int o0 = tile * kMfmaRowsPerItem + wave * 16;
        const bool whole = n <= kDownStageRoutes;  // (always at verify widths: n <= 16)
        for (int j0 = 0; j0 < n; j0 += kMfmaMaxCols) {
            const int nj = n - j0 < kMfmaMaxCols ? n - j0 : kMfmaMaxCols;
            int xrow = r16;
            if (stage_all) {
                xrow = pos0 + j0 + r16;
            } else {
                const int sj0 = whole ? 0 : j0;
                if (ui != staged_slot || sj0 != staged_j0) {
                    staged_slot = ui;
                    staged_j0 = sj0;
                    lds_barrier();
                    stage(pos0 + sj0, whole ? n : nj);
                    lds_barrier();
                }
                xrow = j0 - sj0 + r16;
            }
            const f4_t acc = mfma_tile<BITS, NSUB>(w, book, xs_lane<NSUB>(xs, xrow, kDownStageRoutes, q, r16 < nj));
            if (r16 < nj) {
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) {
                    const int o = o0 + 4 * q + rr;
                    const float sc = h2f(P.scales[static_cast<size_t>(bank_index<PAR>(expert)) * H + o]);
                    const size_t at = static_cast<size_t>(route_of_pos(plan, M * K, pos0 + j0 + r16)) * H + o;
                    dout[at] = sc * acc[rr];
                    if (PAR >= 0 && NCHUNK == 1) B.d[B.d_plane + at] = 0.0f;
                }
            }
        }
#pragma unroll
        for (int i = 0; i <= WPL; ++i) w[i] = wn[i];
    }
}

// ============================================================== U8 books (R6, verify widths)
// The reference's verify-width decode (src/vq_metal_kernels.hpp:564-579) reads a d8
// projection's per-dimension INT8/U8 book: w = q s[d] (+ b[d]), s and b fp16 per dimension.
// Here the book is kept as bytes u = q + 128 (centred gate book) or u = q (affine books), so
// that w = (u - 128) s[d] + c[d] with c = 0 (centred) or b + 128 s (affine). One 8-byte entry
// holds all 8 dims, so the whole book (16384 x 8 bytes) sits in one workgroup's LDS: one
// gather per subvector, where the fp16 book takes two (one per 4-dim chunk, in two
// workgroups). v_mfma_f32_16x16x32_f16 takes A = u - 128, exact in fp16 (v_perm pairs two
// bytes with the exponent byte of 1024, giving 1024 + u, then a packed fp16 add of -1152),
// and B = x' = fp16(s[d] x) per input, so for each B column (input row or route)
//   sum_k w_k x_k = sum_k (u_k - 128) x'_k + sum_k c[d_k] x_k
// up to the rounding of x' (relative 2^-12 per input, carried by |u - 128| s, about |w|).
// The second sum is formed once per column in a fixed order. Lane (c, q) of a 16-row tile:
// A = row c's entry for subvector q S4 + t, B = column c's x' of that subvector (8 fp16),
// t = 0 .. S4 - 1 (S4 = subvectors / 4).
__device__ __forceinline__ void wait_vm_all_moe() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

constexpr int kU8Cols = 4;  // gate/up: request rows staged per pass (the book leaves room for 4)
constexpr uint32_t kF16Exp1024 = 0x64646464u;

__device__ __forceinline__ h8_t u8_entry_f16(uint2 e) {
    // bytes u0..u7 -> fp16 1024 + u0 .. 1024 + u7 (dims in order) -> u - 128, exact
    const uint4 v = make_uint4(__builtin_amdgcn_perm(kF16Exp1024, e.x, 0x04010400u),
                               __builtin_amdgcn_perm(kF16Exp1024, e.x, 0x04030402u),
                               __builtin_amdgcn_perm(kF16Exp1024, e.y, 0x04010400u),
                               __builtin_amdgcn_perm(kF16Exp1024, e.y, 0x04030402u));
    return __builtin_bit_cast(h8_t, v) - static_cast<_Float16>(1152.0f);
}

// x' of one subvector (8 fp16 inputs) and its share of the column sum sum_k c[d_k] x_k (in c,
// dimension order).
__device__ __forceinline__ uint4 u8_scale_sub(uint4 xv, const float (&s)[8], const float (&b)[8], float& c) {
    const uint32_t w[4] = {xv.x, xv.y, xv.z, xv.w};
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t pr = 0;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int d = 2 * i + k;
            const float x = h2f(static_cast<uint16_t>(w[i] >> (16 * k)));
            const uint16_t xp = f2h(x * s[d]);
            c = fmaf(b[d], x, c);
            pr |= static_cast<uint32_t>(xp) << (16 * k);
        }
        o[i] = pr;
    }
    return make_uint4(o[0], o[1], o[2], o[3]);
}

__device__ __forceinline__ void u8_load_sb(const float* sb, float (&s)[8], float (&b)[8]) {
#pragma unroll
    for (int d = 0; d < 8; ++d) {
        s[d] = sb[d];
        b[d] = sb[8 + d];
    }
}

// One 16-row tile over all NSUB subvectors: A from the U8 book, B = xlane[t] (this lane's
// column, q block) from LDS or registers. Two accumulators (even and odd steps), added.
template <int NSUB, typename XB>
__device__ __forceinline__ f4_t mfma_tile_u8(const uint32_t* w, const uint2* book, const XB& xlane) {
    constexpr int S4 = NSUB / 4;
    f4_t acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < S4; t += 2) {
        const h8_t a0 = u8_entry_f16(book[code_from<14>(w, t)]);
        const h8_t a1 = u8_entry_f16(book[code_from<14>(w, t + 1)]);
        acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, __builtin_bit_cast(h8_t, xlane[t]), acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, __builtin_bit_cast(h8_t, xlane[t + 1]), acc1, 0, 0, 0);
    }
    return acc0 + acc1;
}

// Gate and up from the U8 books: workgroup type = projection (the whole book in LDS), items
// (slot, 128-row tile of I). Waves 0-3 copy the book into LDS over the direct global-to-LDS
// path while waves 4-7 stage x' of the request rows (M <= kU8Cols: lane l of those 256
// threads takes subvector l of every row) with their shares of each row's column sum C =
// sum_k c[d_k] x_k (wave butterflies, then the four waves' sums in order); then routing and
// the plan as in k_gu_mfma, and the first item's codes are requested before the copy is
// waited for. Wider calls stage x' per pass of up to kU8Cols of a slot's routes, and C comes
// from one wave per row. The x' rows are padded per q block (S4 + 1 entries), so the 16
// columns x 4 blocks of one B read fall in different LDS banks. Output: one plane,
// scale * (acc + C), at the route's sorted position.
template <int NSUB>
__global__ __launch_bounds__(kMfmaThreads) void k_gu_u8(LayerDev L, MoeBufs B, int M) {
    extern __shared__ __align__(16) unsigned char lds[];
    __shared__ TopkLds tk;
    __shared__ int32_t plan[kPlanInts];
    __shared__ float cx[kMaxRows];          // C of each request row (this projection)
    __shared__ float cpart[4][kU8Cols];     // staging waves' shares of C
    __shared__ int32_t exf[kNarrowMaxRoutes];          // (fast routing) the rows' experts
    __shared__ uint64_t cand[kU8Cols][64];             // (fast routing) candidates per row wave
    constexpr int KENT = 1 << 14;
    constexpr int S4 = NSUB / 4, WPL = S4 * 14 / 32, XR = 4 * (S4 + 1);
    static_assert(NSUB == 256, "one staging thread per subvector");
    const uint2* book = reinterpret_cast<const uint2*>(lds);
    uint4* xs = reinterpret_cast<uint4*>(lds + KENT * 8);  // [kU8Cols + 1 zero][4][S4 + 1] x'
    auto xat = [](int row, int sv) { return row * XR + (sv / S4) * (S4 + 1) + sv % S4; };
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int x8 = blockIdx.x & 7, kk = blockIdx.x >> 3;
    const int proj = kk & 1;
    const int per_type = (gridDim.x / 16) * 8;
    const int idx = (kk >> 1) * 8 + x8;
    const ProjDev& P = L.p[proj];
    const int H = L.H, I = L.I, K = L.K;
    float s[8], b[8];
    u8_load_sb(P.u8_sb, s, b);
    const bool stage_all = M <= kU8Cols;
    if (wave < 4) {
        dma_book<KENT>(reinterpret_cast<const uint16_t*>(P.book_u8), lds, wave, 4);
    } else if (stage_all) {
        const int sv = tid - 256;
        uint4 xv[kU8Cols];
#pragma unroll
        for (int r = 0; r < kU8Cols; ++r)
            if (r < M) xv[r] = *reinterpret_cast<const uint4*>(B.x16 + static_cast<size_t>(r) * H + 8 * sv);
#pragma unroll
        for (int r = 0; r < kU8Cols; ++r)
            if (r < M) {
                float c = 0.0f;
                xs[xat(r, sv)] = u8_scale_sub(xv[r], s, b, c);
#pragma unroll
                for (int o = 32; o >= 1; o >>= 1) c += __shfl_xor(c, o, 64);
                if (lane == 0) cpart[wave - 4][r] = c;
            }
    }
    // Routing: up to 4 rows of E = 512 by the one-wave routines of the four-row kernels
    // (row r on wave 4 + r, the plan by wave 4), otherwise the block routine.
    if (stage_all && L.E == 512 && M * K <= kNarrowMaxRoutes) {
        if (wave >= 4 && wave - 4 < M) {
            float lg[8];
            topk_load_row_t<8, true>(L, B, wave - 4, lg);
            topk_select_row_fast<8>(L, B, wave - 4, lg, exf, blockIdx.x == 0, cand[wave - 4]);
        }
        lds_barrier();
        if (wave == 4) plan_wave(M, K, exf, plan);
        lds_barrier();
    } else {
        topk_plan_block(L, B, M, blockIdx.x == 0, plan, tk, 4);
    }
    if (blockIdx.x == 0)
        for (int i = tid; i < 2 + 4 * M * L.K; i += kMfmaThreads) B.plan[i] = plan[i];
    if (stage_all) {
        if (tid < M) cx[tid] = ((cpart[0][tid] + cpart[1][tid]) + cpart[2][tid]) + cpart[3][tid];
    } else {
        for (int r = wave; r < M; r += 8) {
            float c = 0.0f;
#pragma unroll
            for (int i = 0; i < NSUB / 64; ++i) {
                const uint4 xv = *reinterpret_cast<const uint4*>(B.x16 + static_cast<size_t>(r) * H + 8 * (lane + 64 * i));
                (void)u8_scale_sub(xv, s, b, c);
            }
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) c += __shfl_xor(c, o, 64);
            if (lane == 0) cx[r] = c;
        }
    }
    for (int i = tid; i < XR; i += kMfmaThreads) xs[kU8Cols * XR + i] = make_uint4(0u, 0u, 0u, 0u);
    const int nu = plan[0];
    const int nslots = nu + (L.has_shared ? 1 : 0);
    const int tiles = I / kMfmaRowsPerItem;
    const int n_items = nslots * tiles;
    float* out = proj == 0 ? B.g : B.u;
    const int r16 = lane & 15, q = lane >> 4;
    auto code_src = [&](int item) {
        int expert, n, pos0;
        slot_rows(plan, M, K, L.has_shared, item / tiles, L.E, &expert, &n, &pos0);
        const size_t rowi = static_cast<size_t>(expert) * I + (item % tiles) * kMfmaRowsPerItem + wave * 16 + r16;
        return P.codes + rowi * P.words + q * WPL;
    };
    // items strided over the workgroups (as k_gu_mfma's uniform layers); wider calls restage
    // x' only when the slot or the pass changes
    int staged_slot = -1, staged_j0 = -1;
    uint32_t w[WPL + 1], wn[WPL + 1];
    if (idx < n_items) load_lane_words<14, NSUB>(code_src(idx), w);
    wait_vm_all_moe();  // (the book copy of waves 0-3)
    lds_barrier();
    for (int item = idx; item < n_items; item += per_type) {
        if (item + per_type < n_items) load_lane_words<14, NSUB>(code_src(item + per_type), wn);
        const int ui = item / tiles, tile = item % tiles;
        int expert, n, pos0;
        slot_rows(plan, M, K, L.has_shared, ui, L.E, &expert, &n, &pos0);
        const bool shared = ui == nu;
        const int o0 = tile * kMfmaRowsPerItem + wave * 16;
        for (int j0 = 0; j0 < n; j0 += kU8Cols) {
            const int nj = n - j0 < kU8Cols ? n - j0 : kU8Cols;
            const int crow = r16 < nj ? route_row(plan, M, K, pos0, j0 + r16, shared) : 0;
            const int xrow = stage_all ? crow : r16;
            if (!stage_all && (ui != staged_slot || j0 != staged_j0)) {
                staged_slot = ui;
                staged_j0 = j0;
                lds_barrier();
                for (int i = tid; i < nj * NSUB; i += kMfmaThreads) {
                    const int jj = i / NSUB, sv = i % NSUB;
                    const int row = route_row(plan, M, K, pos0, j0 + jj, shared);
                    float c = 0.0f;
                    xs[xat(jj, sv)] = u8_scale_sub(
                        *reinterpret_cast<const uint4*>(B.x16 + static_cast<size_t>(row) * H + 8 * sv), s, b, c);
                }
                lds_barrier();
            }
            const uint4* xlane = xs + (r16 < nj ? xrow : kU8Cols) * XR + q * (S4 + 1);
            const f4_t acc = mfma_tile_u8<NSUB>(w, book, xlane);
            if (r16 < nj) {
                const float c = cx[crow];
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) {
                    const int o = o0 + 4 * q + rr;
                    const float sc = h2f(P.scales[static_cast<size_t>(expert) * I + o]);
                    out[static_cast<size_t>(pos0 + j0 + r16) * I + o] = sc * (acc[rr] + c);
                }
            }
        }
#pragma unroll
        for (int i = 0; i <= WPL; ++i) w[i] = wn[i];
    }
}

// SwiGLU rows of every route as the U8 down kernel's B operand: one wave per sorted position
// (I = 512: lane l = subvector l), h = fp16(swiglu(g, u)) as on the fp16-book path, then
// h' = fp16(s[d] h) into B.h16 ([position][I], subvector-major) and the route's column sum
// C = sum_k c[d_k] h_k into B.dcorr (lane order, then a fixed butterfly).
__global__ __launch_bounds__(256) void k_swiglu_u8(LayerDev L, MoeBufs B, int n_routes) {
    const int pos = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (pos >= n_routes) return;
    float s[8], b[8];
    u8_load_sb(L.p[2].u8_sb, s, b);
    const size_t at = static_cast<size_t>(pos) * L.I + 8 * lane;
    const float4 g0 = *reinterpret_cast<const float4*>(B.g + at), g1 = *reinterpret_cast<const float4*>(B.g + at + 4);
    const float4 u0 = *reinterpret_cast<const float4*>(B.u + at), u1 = *reinterpret_cast<const float4*>(B.u + at + 4);
    const float gv[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
    const float uv[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
    uint32_t hw[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        hw[i] = static_cast<uint32_t>(f2h(swiglu(gv[2 * i], uv[2 * i]))) |
                (static_cast<uint32_t>(f2h(swiglu(gv[2 * i + 1], uv[2 * i + 1]))) << 16);
    float c = 0.0f;
    const uint4 hp = u8_scale_sub(make_uint4(hw[0], hw[1], hw[2], hw[3]), s, b, c);
    *reinterpret_cast<uint4*>(B.h16 + at) = hp;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) c += __shfl_xor(c, o, 64);
    if (lane == 0) B.dcorr[pos] = c;
}

// Down from the U8 book: every workgroup holds the book; items (slot, 128-row tile of H); B =
// the slot's h' rows straight from the workspace (lane (c, q): 16 x 16 bytes of route c's row),
// loaded with the item's codes one item ahead. Routes in passes of 16 (one pass at <= 16 rows).
// Output: one plane, scale * (acc + C), at the route index.
template <int NSUB>
__global__ __launch_bounds__(kMfmaThreads) void k_dn_u8(LayerDev L, MoeBufs B, int M) {
    extern __shared__ __align__(16) unsigned char lds[];
    __shared__ int32_t plan[kPlanInts];
    constexpr int KENT = 1 << 14;
    constexpr int S4 = NSUB / 4, WPL = S4 * 14 / 32;
    static_assert(NSUB == 64, "I = 512");
    const uint2* book = reinterpret_cast<const uint2*>(lds);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int idx = blockIdx.x, per_type = gridDim.x;
    const ProjDev& P = L.p[2];
    const int H = L.H, I = L.I, K = L.K, MK = M * K;
    // the plan first (a wave's loads complete in order), then the book over the direct
    // global-to-LDS path; the first item's loads go out before the copy is waited for
    constexpr int PV = (kPlanInts + kMfmaThreads - 1) / kMfmaThreads;
    const int plan_n = 2 + 4 * MK;
    int pv[PV];
#pragma unroll
    for (int k = 0; k < PV; ++k) pv[k] = tid + k * kMfmaThreads < plan_n ? B.plan[tid + k * kMfmaThreads] : 0;
    dma_book<KENT>(reinterpret_cast<const uint16_t*>(P.book_u8), lds, wave, 8);
#pragma unroll
    for (int k = 0; k < PV; ++k)
        if (tid + k * kMfmaThreads < plan_n) plan[tid + k * kMfmaThreads] = pv[k];
    lds_barrier();
    const int nu = plan[0];
    const int tiles = H / kMfmaRowsPerItem;
    const int n_items = (nu + (L.has_shared ? 1 : 0)) * tiles;
    const int r16 = lane & 15, q = lane >> 4;
    struct Item {
        uint32_t w[WPL + 1];
        uint4 bx[S4];
    };
    auto load = [&](int item, int j0, Item& it) {
        int expert, n, pos0;
        slot_rows(plan, M, K, L.has_shared, item / tiles, L.E, &expert, &n, &pos0);
        const size_t rowi = static_cast<size_t>(expert) * H + (item % tiles) * kMfmaRowsPerItem + wave * 16 + r16;
        load_lane_words<14, NSUB>(P.codes + rowi * P.words + q * WPL, it.w);
        if (j0 + r16 < n) {
            const uint4* src = reinterpret_cast<const uint4*>(B.h16 + static_cast<size_t>(pos0 + j0 + r16) * I) + q * S4;
#pragma unroll
            for (int t = 0; t < S4; ++t) it.bx[t] = src[t];
        } else {
#pragma unroll
            for (int t = 0; t < S4; ++t) it.bx[t] = make_uint4(0u, 0u, 0u, 0u);
        }
    };
    Item cur, nxt;
    if (idx < n_items) load(idx, 0, cur);
    wait_vm_all_moe();  // (the book copy)
    lds_barrier();
    for (int item = idx; item < n_items; item += per_type) {
        int expert, n, pos0;
        slot_rows(plan, M, K, L.has_shared, item / tiles, L.E, &expert, &n, &pos0);
        const int o0 = (item % tiles) * kMfmaRowsPerItem + wave * 16;
        for (int j0 = 0; j0 < n; j0 += 16) {
            // the next load: this item's next pass, else the next item's first
            const bool more = j0 + 16 < n;
            if (more) load(item, j0 + 16, nxt);
            else if (item + per_type < n_items) load(item + per_type, 0, nxt);
            const f4_t acc = mfma_tile_u8<NSUB>(cur.w, book, cur.bx);
            if (j0 + r16 < n) {
                const int pos = pos0 + j0 + r16;
                const float c = B.dcorr[pos];
                const size_t rt = static_cast<size_t>(route_of_pos(plan, MK, pos)) * H;
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) {
                    const int o = o0 + 4 * q + rr;
                    const float sc = h2f(P.scales[static_cast<size_t>(expert) * H + o]);
                    B.d[rt + o] = sc * (acc[rr] + c);
                }
            }
            cur = nxt;
        }
    }
}

// u = q (+ 128 when centred) and the 16 floats s[8], c[8] of one per-dimension book (c = 0
// centred, bias + 128 s affine).
__global__ void k_u8_operands(const uint8_t* __restrict__ q, int n, int centered, const uint16_t* __restrict__ s16,
                              const uint16_t* __restrict__ b16, uint8_t* __restrict__ u, float* __restrict__ sb) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) u[i] = static_cast<uint8_t>(q[i] ^ (centered ? 0x80u : 0u));
    if (i < 8) {
        const float sv = h2f(s16[i]);
        sb[i] = sv;
        sb[8 + i] = centered ? 0.0f : h2f(b16[i]) + 128.0f * sv;
    }
}

// ============================================================== combine (R8, R10, R11)
// One thread per (row, column): routed = T(sum_slot w_slot * T(d_slot)) in slot order,
// shared = T(T(d_shared) * gate), y = T(routed + shared); chain mode adds the residual in
// place (h <- T(h + y)), otherwise out <- y. The down kernels write route r * k + s at row
// r * k + s and the shared expert's row r at M * k + r, so every load here is independent
// of the plan and all of them are issued before the first use.

// Every load is unconditional and issued up front, the row's route weights and gate first
// (each wait below then covers only what it needs); with no shared expert the shared read
// repeats route 0 (that route is opaque to the optimizer, so it cannot split the code on it).
template <int KT, bool TWO>
__device__ __forceinline__ void combine_load(const LayerDev& L, const MoeBufs& B, int M, int r, int o,
                                             CombineIn<KT, TWO>& in) {
    const int H = L.H, MK = M * KT;
#pragma unroll
    for (int s = 0; s < KT; ++s) in.wts[s] = B.weights[r * KT + s];
    in.wts[KT] = B.sgate[r];
    int shared_route = L.has_shared ? MK + r : r * KT;
    asm("" : "+s"(shared_route));
#pragma unroll
    for (int s = 0; s <= KT; ++s) {
        const int route = s < KT ? r * KT + s : shared_route;
        const size_t at = static_cast<size_t>(route) * H + o;
        in.dv[s][0] = B.d[at];
        in.dv[s][1] = TWO ? B.d[B.d_plane + at] : 0.0f;
    }
}


template <int KT, bool TWO>
__global__ __launch_bounds__(256) void k_combine(LayerDev L, MoeBufs B, int M, uint16_t* h, uint16_t* out) {
    touch_kernargs<sizeof(LayerDev) + sizeof(MoeBufs) + 3 * sizeof(void*)>();
    const int r = blockIdx.y;
    const int o = blockIdx.x * 256 + threadIdx.x;
    const int H = L.H;
    Q38_STAMP(24576, 0);
    if (o >= H) return;
    CombineIn<KT, TWO> in;
    combine_load<KT, TWO>(L, B, M, r, o, in);
    // the residual comes from the output row when there is none (unused then)
    const uint16_t hraw = (h ? h : out)[static_cast<size_t>(r) * H + o];
    const float y = combine_value<KT, TWO>(L, in);
    const size_t i = static_cast<size_t>(r) * H + o;
    if (h) h[i] = f2bf(rbf(bf2f(hraw) + y));
    else out[i] = f2bf(y);
    Q38_STAMP(24576, 1);
}

// The same combine followed by the HyperConnection write of the layer output into the row's
// HC streams (HyperConnection::write, src/hyper_connection.cpp:692-709): stream s of row r
// becomes T(stream + T(y * inj[r][s])), y never leaves registers.
template <int KT, bool TWO>
__global__ __launch_bounds__(256) void k_combine_hc(LayerDev L, MoeBufs B, int M, uint16_t* hs, const uint16_t* inj,
                                                    int HC) {
    touch_kernargs<sizeof(LayerDev) + sizeof(MoeBufs) + 3 * sizeof(void*)>();
    const int r = blockIdx.y;
    const int o = blockIdx.x * 256 + threadIdx.x;
    const int H = L.H;
    if (o >= H) return;
    CombineIn<KT, TWO> in;
    combine_load<KT, TWO>(L, B, M, r, o, in);
    uint16_t sv[kHcMaxStreams], gv[kHcMaxStreams];
    const size_t row = static_cast<size_t>(r) * HC * H + o;
#pragma unroll
    for (int s = 0; s < kHcMaxStreams; ++s)
        if (s < HC) {
            sv[s] = hs[row + static_cast<size_t>(s) * H];
            gv[s] = inj[r * HC + s];
        }
    const float y = combine_value<KT, TWO>(L, in);
#pragma unroll
    for (int s = 0; s < kHcMaxStreams; ++s)
        if (s < HC) hs[row + static_cast<size_t>(s) * H] = f2bf(bf2f(sv[s]) + rbf(y * bf2f(gv[s])));
}

__global__ __launch_bounds__(256) void k_rmsnorm(const uint16_t* __restrict__ x, int H, float eps,
                                                 const uint16_t* __restrict__ w, uint16_t* __restrict__ y) {
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
    for (int c = tid; c < H; c += 256) {
        const float n = rbf(bf2f(x[static_cast<size_t>(r) * H + c]) * inv);
        y[static_cast<size_t>(r) * H + c] = f2bf(w ? n * bf2f(w[c]) : n);
    }
}

// Split a [entries, dim] fp16 codebook into [dim/4][entries][4] chunks.
__global__ void k_split_book(const uint16_t* __restrict__ book, int entries, int dim, uint16_t* __restrict__ out) {
    const int n = entries * dim;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        const int e = i / dim, d = i % dim;
        out[(static_cast<size_t>(d / 4) * entries + e) * 4 + d % 4] = book[i];
    }
}

// The same split of an INT8 codebook, decoded to fp16: value = fp16(q * scale) (the MFMA
// operand type; q * scale itself is exact in float, the fp16 rounding is the only change).
__global__ void k_split_book_i8(const int8_t* __restrict__ book, float scale, int entries, int dim,
                                uint16_t* __restrict__ out) {
    const int n = entries * dim;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        const int e = i / dim, d = i % dim;
        out[(static_cast<size_t>(d / 4) * entries + e) * 4 + d % 4] = f2h(static_cast<float>(book[i]) * scale);
    }
}

// Tiled copy of packed codes (the layout of ProjDev::codes_t): one thread per (64-row tile,
// 32-code block, row of the tile).
__global__ void k_tile_codes(const uint32_t* __restrict__ codes, int64_t n_tiles, int words, int bits,
                             uint32_t* __restrict__ out) {
    const int nblk = words / bits;
    const int64_t total = n_tiles * nblk * 64;
    for (int64_t t = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; t < total;
         t += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int lane = static_cast<int>(t % 64);
        const int64_t tw = t / 64;
        const int w = static_cast<int>(tw % nblk);
        const int64_t tile = tw / nblk;
        const uint32_t* src = codes + (tile * 64 + lane) * words + static_cast<int64_t>(w) * bits;
        uint32_t* blk = out + (tile * nblk + w) * bits * 64;
        for (int q = 0; q < bits; ++q) {
            const int c = q / 4, cw = bits - 4 * c < 4 ? bits - 4 * c : 4;
            blk[c * 256 + lane * cw + q % 4] = src[q];
        }
    }
}

// ============================================================== launchers
namespace {
int g_mfma_grid = 256;  // one persistent workgroup per CU (set from the device at first use)

void init_grid() {
    // (every device of the process is an MI355X with the same CU count; the value is the
    // same whichever thread stores it first)
    static std::once_flag once;
    std::call_once(once, [] {
        int dev = 0, cus = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cus >= 64)
            g_mfma_grid = cus / 32 * 32;
    });
}

template <int T, bool NORM, int MR>
hipError_t launch_route_norm_t(const LayerDev& L, const MoeBufs& B, int M, const uint16_t* src, float eps,
                               hipStream_t st) {
    constexpr int NW = 2 * T;  // waves of H/4 threads
    const size_t lds = static_cast<size_t>(M) * 512 * T * 2;
    if (const hipError_t e = ensure_lds<k_route_norm<T, NORM, MR>>(MR * 512 * T * 2); e != hipSuccess) return e;
    const int rows = L.E + (L.has_shared ? 1 : 0);
    const int reset = moe_uses_fused(L, M) ? 1 : 0;
    return launch(k_route_norm<T, NORM, MR>, dim3((rows + NW - 1) / NW), dim3(128 * T), lds, st, L, B, M, src, eps,
                  reset);
}
template <int T, bool NORM>
hipError_t launch_route_norm_m(const LayerDev& L, const MoeBufs& B, int M, const uint16_t* src, float eps,
                               hipStream_t st) {
    if (M <= 1) return launch_route_norm_t<T, NORM, 1>(L, B, M, src, eps, st);
    if (M <= 2) return launch_route_norm_t<T, NORM, 2>(L, B, M, src, eps, st);
    if (M <= 4) return launch_route_norm_t<T, NORM, 4>(L, B, M, src, eps, st);
    if (M <= 8) return launch_route_norm_t<T, NORM, 8>(L, B, M, src, eps, st);
    return launch_route_norm_t<T, NORM, 16>(L, B, M, src, eps, st);
}
template <int T>
hipError_t launch_route_norm_h(const LayerDev& L, const MoeBufs& B, int M, const uint16_t* src, bool norm, float eps,
                               hipStream_t st) {
    return norm ? launch_route_norm_m<T, true>(L, B, M, src, eps, st) : launch_route_norm_m<T, false>(L, B, M, src, eps, st);
}

template <int BITS, int NSUB, int NCHUNK, int PAR = -1>
hipError_t launch_gu_mfma_g(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st) {
    const size_t lds = (size_t{1} << BITS) * 8 + static_cast<size_t>(gu_mfma_cols(BITS) + 1) * XsLayout<NSUB>::RB;
    if (const hipError_t e = ensure_lds<k_gu_mfma<BITS, NSUB, NCHUNK, PAR>>(lds); e != hipSuccess) return e;
    return launch(k_gu_mfma<BITS, NSUB, NCHUNK, PAR>, dim3(g_mfma_grid), dim3(kMfmaThreads), lds, st, L, B, M);
}
template <int BITS, int NSUB, int NCHUNK, int PAR = -1>
hipError_t launch_down_mfma_g(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st) {
    const size_t lds = (size_t{1} << BITS) * 8 + static_cast<size_t>(kDownStageRoutes + 1) * XsLayout<NSUB>::RB;
    if (const hipError_t e = ensure_lds<k_down_mfma<BITS, NSUB, NCHUNK, PAR>>(lds); e != hipSuccess) return e;
    return launch(k_down_mfma<BITS, NSUB, NCHUNK, PAR>, dim3(g_mfma_grid), dim3(kMfmaThreads), lds, st, L, B, M);
}

hipError_t launch_gu_u8(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st) {
    constexpr int NSUB = 256;
    constexpr size_t lds = (size_t{1} << 14) * 8 + static_cast<size_t>(kU8Cols + 1) * (NSUB + 4) * 16;
    if (L.H != 8 * NSUB || L.I % kMfmaRowsPerItem) return hipErrorInvalidValue;
    if (const hipError_t e = ensure_lds<k_gu_u8<NSUB>>(lds); e != hipSuccess) return e;
    return launch(k_gu_u8<NSUB>, dim3(g_mfma_grid), dim3(kMfmaThreads), lds, st, L, B, M);
}

hipError_t launch_down_u8(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st) {
    constexpr size_t lds = (size_t{1} << 14) * 8;
    if (L.I != 512 || L.H % kMfmaRowsPerItem) return hipErrorInvalidValue;
    const int n_routes = M * L.K + (L.has_shared ? M : 0);
    hipError_t e = launch(k_swiglu_u8, dim3((n_routes + 3) / 4), dim3(256), 0, st, L, B, n_routes);
    if (e != hipSuccess) return e;
    if ((e = ensure_lds<k_dn_u8<64>>(lds)) != hipSuccess) return e;
    return launch(k_dn_u8<64>, dim3(g_mfma_grid), dim3(kMfmaThreads), lds, st, L, B, M);
}

std::atomic<int> g_u8_native{1};

} // namespace

void set_u8_native(int mode) { g_u8_native.store(mode < 0 ? 0 : mode > 2 ? 2 : mode, std::memory_order_relaxed); }

bool moe_u8_call(const LayerDev& L, int M) {
    if (!L.u8_native || L.shared_affine || L.mixed || M < 1 || M > kMaxRows) return false;
    const int mode = g_u8_native.load(std::memory_order_relaxed);
    if (mode == 0) return false;
    if (mode == 2 || M > 4) return true;
    // 1-4 rows: the one-launch layer on the decoded book is faster wherever it is taken
    LayerDev d = L;
    d.fused_mode = 0;
    return !moe_uses_fused(d, M);
}

hipError_t launch_u8_operands(const void* q, int K, int centered, const uint16_t* s16, const uint16_t* b16,
                              uint8_t* u, float* sb, hipStream_t st) {
    const int n = K * 8;
    hipLaunchKernelGGL(k_u8_operands, dim3((n + 255) / 256), dim3(256), 0, st, static_cast<const uint8_t*>(q), n,
                       centered, s16, b16, u, sb);
    return hipGetLastError();
}

// Mixed layers run their two banks on the MFMA kernels: H = 2048, I = 512, per-row scales,
// chunked fp16 codebooks prepared for both banks.
bool moe_mixed_mfma(const LayerDev& L) {
    if (!L.mixed || L.H != 2048 || L.I != 512) return false;
    for (int p = 0; p < 3; ++p)
        for (int b = 0; b < 2; ++b)
            if (L.pb[p][b].ngrp != 1 || !L.pb[p][b].book4) return false;
    return true;
}

bool moe_plans_in_gate_up(const LayerDev& L, int M) {
    return moe_uses_mfma(L) || moe_mixed_mfma(L) || moe_uses_narrow(L, M);
}

bool moe_uses_mfma(const LayerDev& L) {
    // MFMA tiles: per-row scales and the geometry below
    if (L.p[0].ngrp != 1 || L.p[1].ngrp != 1 || L.p[2].ngrp != 1) return false;
    return moe_uses_mfma_geometry(L);
}

bool moe_uses_mfma_geometry(const LayerDev& L) {
    if (L.mixed) return false;
    // 128-row tiles, and lane code spans of whole 16-code half-blocks (gate/up: d8 with H/8
    // in {256, 320} or d4 with H/4 = 512; down: d8 with I/8 = 64 or d4 with I/4 = 128).
    if (L.p[1].dim != L.p[0].dim || L.p[1].bits != L.p[0].bits) return false;
    if (L.I % kMfmaRowsPerItem || L.H % kMfmaRowsPerItem) return false;
    const int gd = L.p[0].dim, gb = L.p[0].bits, dd = L.p[2].dim, db = L.p[2].bits;
    const bool gu_ok = (gd == 8 && gb == 14 && (L.H == 2048 || L.H == 2560)) || (gd == 4 && gb == 8 && L.H == 2048);
    const bool dn_ok = (dd == 8 && db == 14 && L.I == 512) || (dd == 4 && db == 8 && L.I == 512);
    return gu_ok && dn_ok;
}

hipError_t launch_router(const LayerDev& L, const MoeBufs& B, int M, const uint16_t* src, bool norm, float eps,
                         hipStream_t st) {
    if (M < 1 || M > kMaxRows) return hipErrorInvalidValue;
    switch (L.H / 512) {
        case 1: return launch_route_norm_h<1>(L, B, M, src, norm, eps, st);
        case 2: return launch_route_norm_h<2>(L, B, M, src, norm, eps, st);
        case 3: return launch_route_norm_h<3>(L, B, M, src, norm, eps, st);
        case 4: return launch_route_norm_h<4>(L, B, M, src, norm, eps, st);
        case 5: return launch_route_norm_h<5>(L, B, M, src, norm, eps, st);
        case 6: return launch_route_norm_h<6>(L, B, M, src, norm, eps, st);
        case 8: return launch_route_norm_h<8>(L, B, M, src, norm, eps, st);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_topk_plan(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st) {
    return launch(k_topk_plan, dim3(1), dim3(1024), 0, st, L, B, M);
}

KernelTimer& kernel_timer() {
    static thread_local KernelTimer t;
    return t;
}

int mfma_grid() {
    init_grid();
    return g_mfma_grid;
}

hipError_t launch_gate_up(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st) {
    init_grid();
    if (L.mixed) {  // the two banks on the MFMA kernels: even experts d4/8-bit, odd d8/14-bit
        if (!moe_mixed_mfma(L)) return hipErrorInvalidValue;
        const hipError_t e = launch_gu_mfma_g<8, 512, 1, 0>(L, B, M, st);
        if (e != hipSuccess) return e;
        return launch_gu_mfma_g<14, 256, 2, 1>(L, B, M, st);
    }
    if (L.u8_call) return launch_gu_u8(L, B, M, st);
    if (moe_uses_fused(L, M)) return launch_gate_down4(L, B, M, nullptr, nullptr, st);
    if (moe_uses_narrow(L, M)) return launch_gate_up4(L, B, M, st);
    const int D = L.p[0].dim;
    if (moe_uses_mfma(L)) {
        const int nsub = L.H / D;
        if (D == 8 && nsub == 256) return launch_gu_mfma_g<14, 256, 2>(L, B, M, st);
        if (D == 8 && nsub == 320) return launch_gu_mfma_g<14, 320, 2>(L, B, M, st);
        if (D == 4 && nsub == 512) return launch_gu_mfma_g<8, 512, 1>(L, B, M, st);
        return hipErrorInvalidValue;
    }
    return launch_gate_up_grouped(L, B, M, st);
}

hipError_t launch_down(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st) {
    init_grid();
    if (L.mixed) {
        if (!moe_mixed_mfma(L)) return hipErrorInvalidValue;
        const hipError_t e = launch_down_mfma_g<8, 128, 1, 0>(L, B, M, st);
        if (e != hipSuccess) return e;
        return launch_down_mfma_g<14, 64, 2, 1>(L, B, M, st);
    }
    if (L.u8_call) return launch_down_u8(L, B, M, st);
    if (moe_uses_fused(L, M)) return hipSuccess;  // (the fused gate/up launch ran the down half)
    if (moe_uses_narrow(L, M)) return launch_down4(L, B, M, st);
    const int D = L.p[2].dim;
    if (moe_uses_mfma(L)) {
        const int nsub = L.I / D;
        if (D == 8 && nsub == 64) return launch_down_mfma_g<14, 64, 2>(L, B, M, st);
        if (D == 4 && nsub == 128) return launch_down_mfma_g<8, 128, 1>(L, B, M, st);
        return hipErrorInvalidValue;
    }
    return launch_down_grouped(L, B, M, st);
}

template <int KT>
hipError_t launch_combine_k(const LayerDev& L, const MoeBufs& B, int M, uint16_t* h, uint16_t* out, const uint16_t* inj,
                            int HC, hipStream_t st) {
    const dim3 grid((L.H + 255) / 256, M);
    if (inj) {
        if (L.d_parts == 2) return launch(k_combine_hc<KT, true>, grid, dim3(256), 0, st, L, B, M, h, inj, HC);
        return launch(k_combine_hc<KT, false>, grid, dim3(256), 0, st, L, B, M, h, inj, HC);
    }
    if (L.d_parts == 2) return launch(k_combine<KT, true>, grid, dim3(256), 0, st, L, B, M, h, out);
    return launch(k_combine<KT, false>, grid, dim3(256), 0, st, L, B, M, h, out);
}

static hipError_t launch_combine_any(const LayerDev& L, const MoeBufs& B, int M, uint16_t* h, uint16_t* out,
                                     const uint16_t* inj, int HC, hipStream_t st) {
    switch (L.K) {
        case 1: return launch_combine_k<1>(L, B, M, h, out, inj, HC, st);
        case 2: return launch_combine_k<2>(L, B, M, h, out, inj, HC, st);
        case 3: return launch_combine_k<3>(L, B, M, h, out, inj, HC, st);
        case 4: return launch_combine_k<4>(L, B, M, h, out, inj, HC, st);
        case 5: return launch_combine_k<5>(L, B, M, h, out, inj, HC, st);
        case 6: return launch_combine_k<6>(L, B, M, h, out, inj, HC, st);
        case 7: return launch_combine_k<7>(L, B, M, h, out, inj, HC, st);
        case 8: return launch_combine_k<8>(L, B, M, h, out, inj, HC, st);
        case 9: return launch_combine_k<9>(L, B, M, h, out, inj, HC, st);
        case 10: return launch_combine_k<10>(L, B, M, h, out, inj, HC, st);
        case 11: return launch_combine_k<11>(L, B, M, h, out, inj, HC, st);
        case 12: return launch_combine_k<12>(L, B, M, h, out, inj, HC, st);
        case 13: return launch_combine_k<13>(L, B, M, h, out, inj, HC, st);
        case 14: return launch_combine_k<14>(L, B, M, h, out, inj, HC, st);
        case 15: return launch_combine_k<15>(L, B, M, h, out, inj, HC, st);
        case 16: return launch_combine_k<16>(L, B, M, h, out, inj, HC, st);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_combine(const LayerDev& L, const MoeBufs& B, int M, uint16_t* h, uint16_t* out, hipStream_t st) {
    return launch_combine_any(L, B, M, h, out, nullptr, 0, st);
}

hipError_t launch_combine_hc(const LayerDev& L, const MoeBufs& B, int M, uint16_t* hs, const uint16_t* inj, int HC,
                             hipStream_t st) {
    return launch_combine_any(L, B, M, hs, nullptr, inj, HC, st);
}

hipError_t launch_rmsnorm(const uint16_t* x, int M, int H, float eps, uint16_t* y, hipStream_t st) {
    return launch(k_rmsnorm, dim3(M), dim3(256), 0, st, x, H, eps, static_cast<const uint16_t*>(nullptr), y);
}
hipError_t launch_rmsnorm_w(const uint16_t* x, int M, int H, float eps, const uint16_t* w, uint16_t* y,
                            hipStream_t st) {
    return launch(k_rmsnorm, dim3(M), dim3(256), 0, st, x, H, eps, w, y);
}

hipError_t launch_tile_codes(const uint32_t* codes, int64_t rows, int words, int bits, uint32_t* out, hipStream_t st) {
    if (rows % 64 || words % bits) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_tile_codes, dim3(4096), dim3(256), 0, st, codes, rows / 64, words, bits, out);
    return hipGetLastError();
}

hipError_t launch_split_book(const uint16_t* book, int entries, int dim, uint16_t* book4, hipStream_t st) {
    hipLaunchKernelGGL(k_split_book, dim3(512), dim3(256), 0, st, book, entries, dim, book4);
    return hipGetLastError();
}
hipError_t launch_split_book_i8(const int8_t* book, float scale, int entries, int dim, uint16_t* book4,
                                hipStream_t st) {
    hipLaunchKernelGGL(k_split_book_i8, dim3(512), dim3(256), 0, st, book, scale, entries, dim, book4);
    return hipGetLastError();
}

hipError_t launch_gen_codes(uint64_t key, int e0, int e_stride, int n_experts, int out_dim, int nsub, int bits,
                            int words, uint32_t* codes, hipStream_t st) {
    hipLaunchKernelGGL(k_gen_codes, dim3(4096), dim3(256), 0, st, key, e0, e_stride, n_experts, out_dim, nsub, bits,
                       words, codes);
    return hipGetLastError();
}
hipError_t launch_gen_scales(uint64_t key, int e0, int e_stride, int n_experts, int out_dim, double lo, double hi,
                             uint16_t* out, hipStream_t st) {
    hipLaunchKernelGGL(k_gen_scales, dim3(2048), dim3(256), 0, st, key, e0, e_stride, n_experts, out_dim, lo, hi, out);
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
hipError_t launch_gen_embed_dev(uint64_t seed, const uint32_t* tokens, int n, int H, uint16_t* out, hipStream_t st) {
    hipLaunchKernelGGL(k_gen_embed_dev, dim3((n * H + 255) / 256), dim3(256), 0, st,
                       stream_key(seed, kEmbedLayer, T_EMBED), tokens, n, H, out);
    return hipGetLastError();
}
hipError_t launch_prepare_u8(const uint16_t* book16, int K, int centered, uint8_t* q, uint16_t* s16, uint16_t* b16,
                             uint16_t* dec, hipStream_t st) {
    return launch(k_prepare_u8, dim3(1), dim3(1024), 0, st, book16, K, centered, q, s16, b16, dec);
}
hipError_t launch_book_to_int8(const uint16_t* book16, int n, int8_t* q8, uint16_t* scale, hipStream_t st) {
    hipLaunchKernelGGL(k_book_to_int8, dim3(1), dim3(1024), 0, st, book16, n, q8, scale);
    return hipGetLastError();
}

#ifdef Q38_TRACE
__device__ unsigned long long g_trace_route[32768];
#endif
} // namespace q38

#ifdef Q38_TRACE
extern "C" int q38_trace_read_route(unsigned long long* out) {
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(q38::g_trace_route), sizeof(unsigned long long) * 32768) == hipSuccess
               ? 0
               : -1;
}
#endif
