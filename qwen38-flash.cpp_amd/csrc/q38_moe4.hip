// q38_moe4.hip — expert projections for verify widths of up to four rows (R4, R5, R7, R8)
// on v_mfma_f32_4x4x4_16b_f16.
//
// Operand layout of the 16-block 4x4x4 instruction: A lane 4b + i holds row i of block b
// (4 k values), B lane 4b + j holds column j of block b, D lane 4b + j register r holds
// D[b][r][j]. Here A lane l is one codebook entry (the 4 fp16 dims of one subvector held
// by the workgroup's codebook chunk) of weight row l of a 64-row tile, and B lane 4b + j
// is the same 4 dims of input row j (identical in every block), so one instruction
// accumulates one subvector of 64 weight rows against 4 input rows. A wave owns one
// 32-subvector K slice (one whole 32-code block of each of its rows, one contiguous code
// span per lane); the slices are summed across waves through LDS in a fixed order.
//
// Each workgroup keeps one 4-dim chunk of one codebook in LDS for the whole launch (as in
// the wide-row kernels) and walks its share of (expert slot, tile) items. The prologue
// issues every independent load before it waits on any: the routing wave's logits, the
// codebook chunk, the input operand; the first item's code span is requested as soon as
// the plan exists, and each item's span is prefetched while the previous item computes.
#include "q38_moe_dev.hpp"

namespace q38 {
namespace {

typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef float v4f_t __attribute__((ext_vector_type(4)));

constexpr int kNarrow = 4;  // input rows per instruction (the B columns)

// One 32-code block (BITS words) plus a zero pad word for code_from.
template <int BITS>
__device__ __forceinline__ void load_code_block(const uint32_t* src, uint32_t* w) {
    if constexpr (BITS % 4 == 0) {
#pragma unroll
        for (int i = 0; i < BITS / 4; ++i) {
            const uint4 v = reinterpret_cast<const uint4*>(src)[i];
            w[4 * i] = v.x; w[4 * i + 1] = v.y; w[4 * i + 2] = v.z; w[4 * i + 3] = v.w;
        }
    } else if constexpr (BITS % 2 == 0) {
#pragma unroll
        for (int i = 0; i < BITS / 2; ++i) {
            const uint2 v = reinterpret_cast<const uint2*>(src)[i];
            w[2 * i] = v.x; w[2 * i + 1] = v.y;
        }
    } else {
#pragma unroll
        for (int i = 0; i < BITS; ++i) w[i] = src[i];
    }
    w[BITS] = 0;
}

// 32 steps of one K slice: A = codebook entries of the lane's row, B = bops[t].
template <int BITS>
__device__ __forceinline__ v4f_t slice_mfma(const uint32_t* cw, const uint2* book, const uint2* bops) {
    v4f_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < 32; ++t) {
        const uint2 a = book[code_from<BITS>(cw, t)];
        acc = __builtin_amdgcn_mfma_f32_4x4x4f16(__builtin_bit_cast(h4_t, a), __builtin_bit_cast(h4_t, bops[t]), acc,
                                                  0, 0, 0);
    }
    return acc;
}

// Gate and up projections. Workgroup type = (projection, codebook chunk); waves = K slices.
// Items are 64-row tiles of I; the 4 B columns are the request rows (rows not routed to the
// item's expert are computed and discarded). Output: partial sums of this chunk, times the
// row scale, at the route's sorted position (the gate/up chunk planes).
// One workgroup per CU (the LDS codebook chunk), so a SIMD runs at most ceil(waves / 4)
// of its waves: the register budget is set by that, not by a higher occupancy target.
template <int BITS, int NSUB, int NCHUNK>
__global__ __launch_bounds__(2 * NSUB) __attribute__((amdgpu_waves_per_eu(1, (NSUB / 32 + 3) / 4)))
void k_gu4(LayerDev L, MoeBufs B, int M) {
    constexpr int KS = NSUB / 32;
    constexpr int NT = 64 * KS;
    constexpr int KENT = 1 << BITS;
    constexpr int TYPES = 2 * NCHUNK;
    constexpr int NF = (KENT / 2 + NT - 1) / NT;  // codebook uint4 per thread
    extern __shared__ __align__(16) unsigned char lds[];
    __shared__ TopkLds tk;
    __shared__ int32_t plan[kPlanInts];
    const uint2* book = reinterpret_cast<const uint2*>(lds);
    float* red = reinterpret_cast<float*>(lds + KENT * 8);  // [2][KS][64][4]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int x8 = blockIdx.x & 7, kk = blockIdx.x >> 3;
    const int type = kk % TYPES;
    const int proj = type / NCHUNK, chunk = type % NCHUNK;
    const int per_type = (gridDim.x / (8 * TYPES)) * 8;
    const int idx = (kk / TYPES) * 8 + x8;  // items of one index run on one XCD for all types
    const ProjDev& P = L.p[proj];
    const int H = L.H, I = L.I, K = L.K;

    // Loads in the order they are consumed (a wave's vector loads complete in order).
    // E = 512: 64 lanes x 8 keys, branch-free routing code (moe_uses_narrow checks E).
    float lg[8];
    if (wave < M) topk_load_row_t<8, true>(L, B, wave, lg);
    uint4 fv[NF];
    const uint4* fsrc = reinterpret_cast<const uint4*>(P.book4 + static_cast<size_t>(chunk) * KENT * 4);
#pragma unroll
    for (int k = 0; k < NF; ++k) {
        const int i = tid + k * NT;
        fv[k] = (KENT / 2) % NT == 0 || i < KENT / 2 ? fsrc[i] : make_uint4(0u, 0u, 0u, 0u);
    }
    uint2 xb[32];
    {
        const int jx = (lane & 3) < M ? (lane & 3) : 0;
        const uint16_t* xr =
            B.x16 + static_cast<size_t>(jx) * H + static_cast<size_t>(wave) * 32 * (4 * NCHUNK) + 4 * chunk;
#pragma unroll
        for (int t = 0; t < 32; ++t) xb[t] = *reinterpret_cast<const uint2*>(xr + t * 4 * NCHUNK);
    }
    if (wave < M) topk_select_row_t<8, true>(L, B, wave, lg, tk.ex, blockIdx.x == 0);
    topk_build_plan(M, K, plan, tk);  // barriers on entry and exit

    const int tiles = I / 64;
    const int nu = plan[0];
    const int n_items = (nu + (L.has_shared ? 1 : 0)) * tiles;
    auto code_src = [&](int item) {
        int expert, n, pos0;
        slot_rows(plan, M, K, L.has_shared, item / tiles, L.E, &expert, &n, &pos0);
        const size_t row = static_cast<size_t>(expert) * I + (item % tiles) * 64 + lane;
        return P.codes + row * P.words + wave * BITS;
    };
    uint32_t cw[BITS + 1], cn[BITS + 1];
    if (idx < n_items) load_code_block<BITS>(code_src(idx), cw);
    uint4* bdst = reinterpret_cast<uint4*>(lds);
#pragma unroll
    for (int k = 0; k < NF; ++k) {
        const int i = tid + k * NT;
        if ((KENT / 2) % NT == 0 || i < KENT / 2) bdst[i] = fv[k];
    }
    if (blockIdx.x == 0)
        for (int i = tid; i < 2 + 4 * M * K; i += NT) B.plan[i] = plan[i];
    __syncthreads();

    float* out = (proj == 0 ? B.g : B.u) + chunk * B.gu_plane;
    int buf = 0;
    for (int item = idx; item < n_items; item += per_type) {
        if (item + per_type < n_items) load_code_block<BITS>(code_src(item + per_type), cn);
        const v4f_t acc = slice_mfma<BITS>(cw, book, xb);
        reinterpret_cast<v4f_t*>(red)[(buf * KS + wave) * 64 + lane] = acc;
        __syncthreads();
        if (tid < 64 * kNarrow) {
            const int r = tid >> 2, j = tid & 3;  // weight row of the tile, request row
            const int ui = item / tiles;
            int expert, n, pos0;
            slot_rows(plan, M, K, L.has_shared, ui, L.E, &expert, &n, &pos0);
            int pos = -1;
            if (j < M) {
                if (ui == nu) {
                    pos = pos0 + j;
                } else {
                    for (int p = 0; p < n; ++p)
                        if (route_row(plan, M, K, pos0, p, false) == j) pos = pos0 + p;
                }
            }
            if (pos >= 0) {
                const int src = (r & ~3) | j, reg = r & 3;
                float s = 0.0f;
#pragma unroll
                for (int w = 0; w < KS; ++w) s += red[((buf * KS + w) * 64 + src) * 4 + reg];
                const int o = (item % tiles) * 64 + r;
                out[static_cast<size_t>(pos) * I + o] = h2f(P.scales[static_cast<size_t>(expert) * I + o]) * s;
            }
        }
        buf ^= 1;  // the other buffer's readers have passed this item's barrier
#pragma unroll
        for (int i = 0; i <= BITS; ++i) cw[i] = cn[i];
    }
}

// Down projection. Workgroup type = codebook chunk; 8 waves = KS K slices x RG row groups,
// items are (slot, TR = 64 RG rows of H). The B columns are the slot's routes: their SwiGLU
// rows (this chunk's dims, fp16) are formed per item from the gate/up chunk planes, which
// are prefetched one item ahead with the code spans.
template <int BITS, int NSUB, int NCHUNK>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(1, 2))) void k_dn4(LayerDev L, MoeBufs B, int M) {
    constexpr int KS = NSUB / 32, RG = 8 / KS, TR = 64 * RG;
    constexpr int NT = 512, KENT = 1 << BITS;
    constexpr int NF = (KENT / 2 + NT - 1) / NT;
    static_assert(KS * RG == 8, "8 waves");
    static_assert(kNarrow * NSUB <= NT, "one SwiGLU quad per thread");
    extern __shared__ __align__(16) unsigned char lds[];
    __shared__ int32_t plan[kPlanInts];
    __shared__ __align__(16) uint2 hs[kNarrow][NSUB];  // SwiGLU rows of the item's routes (fp16)
    const uint2* book = reinterpret_cast<const uint2*>(lds);
    float* red = reinterpret_cast<float*>(lds + KENT * 8);  // [RG][KS-1][64][4]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int x8 = blockIdx.x & 7, kk = blockIdx.x >> 3;
    const int chunk = kk % NCHUNK;
    const int per_type = (gridDim.x / (8 * NCHUNK)) * 8;
    const int idx = (kk / NCHUNK) * 8 + x8;
    const ProjDev& P = L.p[2];
    const int H = L.H, I = L.I, K = L.K, MK = M * K;
    const int kh = wave % KS, rg = wave / KS;

    int32_t pv = 0;
    const int plan_n = 2 + 4 * MK;
    if (tid < plan_n) pv = B.plan[tid];
    uint4 fv[NF];
    const uint4* fsrc = reinterpret_cast<const uint4*>(P.book4 + static_cast<size_t>(chunk) * KENT * 4);
#pragma unroll
    for (int k = 0; k < NF; ++k) {
        const int i = tid + k * NT;
        fv[k] = (KENT / 2) % NT == 0 || i < KENT / 2 ? fsrc[i] : make_uint4(0u, 0u, 0u, 0u);
    }
    if (tid < plan_n) plan[tid] = pv;
    __syncthreads();

    const int nu = plan[0];
    const int tiles = H / TR;
    const int n_items = (nu + (L.has_shared ? 1 : 0)) * tiles;
    const bool two = L.gu_parts == 2;
    auto code_src = [&](int item) {
        int expert, n, pos0;
        slot_rows(plan, M, K, L.has_shared, item / tiles, L.E, &expert, &n, &pos0);
        const size_t row = static_cast<size_t>(expert) * H + (item % tiles) * TR + rg * 64 + lane;
        return P.codes + row * P.words + kh * BITS;
    };
    // gate/up chunk-plane quads of SwiGLU element (route tid / NSUB, subvector tid % NSUB)
    float4 gq[2], uq[2];
    auto load_gu = [&](int item) {
        int expert, n, pos0;
        slot_rows(plan, M, K, L.has_shared, item / tiles, L.E, &expert, &n, &pos0);
        if (tid < n * NSUB) {
            const size_t at = static_cast<size_t>(pos0 + tid / NSUB) * I + (tid % NSUB) * (4 * NCHUNK) + 4 * chunk;
            gq[0] = *reinterpret_cast<const float4*>(B.g + at);
            uq[0] = *reinterpret_cast<const float4*>(B.u + at);
            if (two) {
                gq[1] = *reinterpret_cast<const float4*>(B.g + B.gu_plane + at);
                uq[1] = *reinterpret_cast<const float4*>(B.u + B.gu_plane + at);
            }
        }
    };
    uint32_t cw[BITS + 1], cn[BITS + 1];
    if (idx < n_items) {
        load_code_block<BITS>(code_src(idx), cw);
        load_gu(idx);
    }
    uint4* bdst = reinterpret_cast<uint4*>(lds);
#pragma unroll
    for (int k = 0; k < NF; ++k) {
        const int i = tid + k * NT;
        if ((KENT / 2) % NT == 0 || i < KENT / 2) bdst[i] = fv[k];
    }

    float* dout = B.d + chunk * B.d_plane;
    for (int item = idx; item < n_items; item += per_type) {
        int expert, n, pos0;
        slot_rows(plan, M, K, L.has_shared, item / tiles, L.E, &expert, &n, &pos0);
        if (tid < n * NSUB) {
            float4 g = gq[0], u = uq[0];
            if (two) {
                g = make_float4(g.x + gq[1].x, g.y + gq[1].y, g.z + gq[1].z, g.w + gq[1].w);
                u = make_float4(u.x + uq[1].x, u.y + uq[1].y, u.z + uq[1].z, u.w + uq[1].w);
            }
            const uint32_t h0 = f2h(swiglu(g.x, u.x)), h1 = f2h(swiglu(g.y, u.y));
            const uint32_t h2 = f2h(swiglu(g.z, u.z)), h3 = f2h(swiglu(g.w, u.w));
            hs[tid / NSUB][tid % NSUB] = make_uint2(h0 | (h1 << 16), h2 | (h3 << 16));
        }
        if (item + per_type < n_items) {
            load_code_block<BITS>(code_src(item + per_type), cn);
            load_gu(item + per_type);
        }
        __syncthreads();  // SwiGLU rows (and, the first time, the codebook) in LDS
        const int jb = (lane & 3) < n ? (lane & 3) : 0;
        v4f_t acc = slice_mfma<BITS>(cw, book, &hs[jb][kh * 32]);
        if (kh > 0) reinterpret_cast<v4f_t*>(red)[(rg * (KS - 1) + kh - 1) * 64 + lane] = acc;
        __syncthreads();
        if (kh == 0) {
#pragma unroll
            for (int w = 1; w < KS; ++w) acc += reinterpret_cast<const v4f_t*>(red)[(rg * (KS - 1) + w - 1) * 64 + lane];
            const int j = lane & 3;
            if (j < n) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int o = (item % tiles) * TR + rg * 64 + (lane & ~3) + r;
                    dout[static_cast<size_t>(pos0 + j) * H + o] =
                        h2f(P.scales[static_cast<size_t>(expert) * H + o]) * acc[r];
                }
            }
        }
#pragma unroll
        for (int i = 0; i <= BITS; ++i) cw[i] = cn[i];
    }
}

template <typename Kern>
hipError_t set_lds4(Kern k, size_t bytes) {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize,
                               static_cast<int>(bytes));
}

template <int BITS, int NSUB, int NCHUNK>
hipError_t launch_gu4_t(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st) {
    constexpr size_t lds = (size_t{1} << BITS) * 8 + 2 * (NSUB / 32) * 64 * 16;
    static bool attr = false;
    if (!attr) {
        const hipError_t e = set_lds4(&k_gu4<BITS, NSUB, NCHUNK>, lds);
        if (e != hipSuccess) return e;
        attr = true;
    }
    return launch(k_gu4<BITS, NSUB, NCHUNK>, dim3(mfma_grid()), dim3(2 * NSUB), lds, st, L, B, M);
}
template <int BITS, int NSUB, int NCHUNK>
hipError_t launch_dn4_t(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st) {
    constexpr int KS = NSUB / 32, RG = 8 / KS;
    constexpr size_t lds = (size_t{1} << BITS) * 8 + static_cast<size_t>(RG) * (KS - 1) * 64 * 16;
    static bool attr = false;
    if (!attr) {
        const hipError_t e = set_lds4(&k_dn4<BITS, NSUB, NCHUNK>, lds);
        if (e != hipSuccess) return e;
        attr = true;
    }
    return launch(k_dn4<BITS, NSUB, NCHUNK>, dim3(mfma_grid()), dim3(512), lds, st, L, B, M);
}
} // namespace

bool moe_uses_narrow(const LayerDev& L, int M) {
    if (M < 1 || M > kNarrow || L.E != 512 || !moe_uses_mfma(L)) return false;
    const int gn = L.H / L.p[0].dim, dn = L.I / L.p[2].dim;
    const bool gu = (L.p[0].dim == 8 && (gn == 256 || gn == 320)) || (L.p[0].dim == 4 && gn == 512);
    const bool dw = (L.p[2].dim == 8 && dn == 64) || (L.p[2].dim == 4 && dn == 128);
    return gu && dw && L.I % 64 == 0 && L.H % 256 == 0;
}

hipError_t launch_gate_up4(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st) {
    const int nsub = L.H / L.p[0].dim;
    if (L.p[0].dim == 8 && nsub == 256) return launch_gu4_t<14, 256, 2>(L, B, M, st);
    if (L.p[0].dim == 8 && nsub == 320) return launch_gu4_t<14, 320, 2>(L, B, M, st);
    if (L.p[0].dim == 4 && nsub == 512) return launch_gu4_t<8, 512, 1>(L, B, M, st);
    return hipErrorInvalidValue;
}

hipError_t launch_down4(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st) {
    const int nsub = L.I / L.p[2].dim;
    if (L.p[2].dim == 8 && nsub == 64) return launch_dn4_t<14, 64, 2>(L, B, M, st);
    if (L.p[2].dim == 4 && nsub == 128) return launch_dn4_t<8, 128, 1>(L, B, M, st);
    return hipErrorInvalidValue;
}

} // namespace q38
