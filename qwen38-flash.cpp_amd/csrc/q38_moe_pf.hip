// q38_moe_pf.hip — prefill-width sparse MoE (R1-R3, R9): 17..2048 rows per call, the
// SparseMoe::forward_prefill_impl segmented path (src/sparse_moe.cpp:2199-2624).
//
//   k_logits_rows  router logits, NE router rows per workgroup held in registers across
//                  64 request rows (the per-lane summation contract of the verify router)
//   k_topk_rows    softmax + top-k of every row (one wave per row, R2)
//   k_plan_sort    gather-by-expert plan of all routes (R3, the stable sort of
//                  src/sparse_moe.cpp:2260-2271): a counting sort by expert in one
//                  workgroup, ranks within 64-route batches from wave ballots, so every
//                  expert's routes come out in route order; unique experts and their
//                  offsets by a block scan
//   k_gu_pf        gate / up segmented GEMM (R9): one workgroup per (64-row output tile,
//                  expert slot, projection). Per 256-input K block the VQ weight tile
//                  (64 x 256) is decoded once into LDS as fp16 and used for every route of
//                  the slot, 64 routes at a time, on v_mfma_f32_16x16x32_f16 (B = the
//                  routes' fp16 inputs staged in LDS); the next K block's code words are
//                  loaded while the current block is decoded and multiplied
//   k_swiglu_pf    SwiGLU of every route with the reference's rounding points, fp16
//   k_dn_pf        down segmented GEMM over the SwiGLU rows, same scheme
// Row scales multiply the accumulated tile at the end. Layers: d8/14-bit, one scale per
// output row, fp16 codebooks.
#include "q38_moe_dev.hpp"

namespace q38 {
namespace {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));

// ============================================================== router (R1)
// Workgroup (gx, gy): router rows [NE gx, NE gx + NE) (row E is w_sg) against request rows
// [64 gy, 64 gy + 64), wave w taking rows 64 gy + w, + 4, ... Lane l accumulates
// x*w over the columns 512t + 8l + j (t outer, j inner) with fmaf, then the xor butterfly
// and BF16 rounding: the logits equal the verify router's bit for bit.
template <int T, int NE>
__global__ __launch_bounds__(256) void k_logits_rows(LayerDev L, MoeBufs B, int M, const uint16_t* __restrict__ x) {
    constexpr int H = 512 * T;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int e0 = blockIdx.x * NE;
    const int nr = L.E + (L.has_shared ? 1 : 0);
    uint4 wv[NE][T];
#pragma unroll
    for (int n = 0; n < NE; ++n) {
        const int e = e0 + n < nr ? e0 + n : nr - 1;
        const uint16_t* w = e < L.E ? L.router + static_cast<size_t>(e) * H : L.wsg;
#pragma unroll
        for (int t = 0; t < T; ++t) wv[n][t] = *reinterpret_cast<const uint4*>(w + 512 * t + 8 * lane);
    }
    const bool store_x = blockIdx.x == 0 && x != B.x;
    const int r1 = (static_cast<int>(blockIdx.y) + 1) * 64 < M ? (blockIdx.y + 1) * 64 : M;
    // the next request row's inputs are loaded while this row's dot products run (the
    // prefetch of the last row repeats it: always in bounds)
    uint4 xn[T];
    {
        const int r0 = blockIdx.y * 64 + wave < r1 ? blockIdx.y * 64 + wave : r1 - 1;
#pragma unroll
        for (int t = 0; t < T; ++t)
            xn[t] = *reinterpret_cast<const uint4*>(x + static_cast<size_t>(r0) * H + 512 * t + 8 * lane);
    }
    for (int r = blockIdx.y * 64 + wave; r < r1; r += 4) {
        uint4 xv[T];
#pragma unroll
        for (int t = 0; t < T; ++t) xv[t] = xn[t];
        const int rn = r + 4 < r1 ? r + 4 : r;
#pragma unroll
        for (int t = 0; t < T; ++t)
            xn[t] = *reinterpret_cast<const uint4*>(x + static_cast<size_t>(rn) * H + 512 * t + 8 * lane);
        float acc[NE];
#pragma unroll
        for (int n = 0; n < NE; ++n) acc[n] = 0.0f;
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const uint32_t xq[4] = {xv[t].x, xv[t].y, xv[t].z, xv[t].w};
#pragma unroll
            for (int n = 0; n < NE; ++n) {
                const uint32_t wq[4] = {wv[n][t].x, wv[n][t].y, wv[n][t].z, wv[n][t].w};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    acc[n] = __builtin_fmaf(bflo(xq[k]), bflo(wq[k]), acc[n]);
                    acc[n] = __builtin_fmaf(bfhi(xq[k]), bfhi(wq[k]), acc[n]);
                }
            }
        }
        float mine = 0.0f;
#pragma unroll
        for (int n = 0; n < NE; ++n) {
            const float s = wave_sum_xor(acc[n]);
            if (lane == n) mine = s;
        }
        const int e = e0 + lane;
        if (lane < NE && e < nr) {
            const float lg = rbf(mine);
            if (e < L.E) B.logits[static_cast<size_t>(r) * L.E + e] = L.rbias ? lg + L.rbias[e] : lg;
            else B.sgate[r] = rbf(1.0f / (1.0f + expf(-lg)));
        }
        if (store_x) {
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const size_t at = static_cast<size_t>(r) * H + 512 * t + 8 * lane;
                *reinterpret_cast<uint4*>(B.x + at) = xv[t];
                const uint32_t q[4] = {xv[t].x, xv[t].y, xv[t].z, xv[t].w};
                uint32_t hq[4];
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    hq[k] = static_cast<uint32_t>(f2h(bflo(q[k]))) | (static_cast<uint32_t>(f2h(bfhi(q[k]))) << 16);
                *reinterpret_cast<uint4*>(B.x16 + at) = make_uint4(hq[0], hq[1], hq[2], hq[3]);
            }
        }
    }
}

// ============================================================== routing (R2, R3)
template <int NJ, bool EXACT>
__global__ __launch_bounds__(256) void k_topk_rows(LayerDev L, MoeBufs B, int M) {
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= M) return;  // wave-uniform
    float lg[NJ];
    topk_load_row_t<NJ, EXACT>(L, B, r, lg);
    topk_select_row_t<NJ, EXACT>(L, B, r, lg, nullptr, true);
}

constexpr int kSortMax = 32768;  // routes per call (rows x k); route ids fit 16 bits

// Plan layout (shared with the verify kernels): [0] unique experts nu, [1 + u] expert of
// slot u, [1 + MK + u] first sorted position of slot u (u <= nu, the last is MK),
// [2 + 2MK + i] route at sorted position i, [2 + 3MK + route] its sorted position.
//
// The plan is a stable counting sort of the routes by expert (routes keep ascending order
// within an expert), in one workgroup of 16 waves. Wave w owns the contiguous routes
// [w c, w c + c) and walks them 64 at a time in order; within such a batch, lanes with the
// same expert find each other with one ballot per expert-id bit, and a lane's rank is the
// number of lower lanes in its group.
//   A: every group's last lane adds the group size to cnt[w][e];
//   B: per expert, a scan over experts of the totals (and of the nonzero flags: the slot
//      numbers) gives its first position, and a scan over waves turns cnt[w][e] into wave
//      w's first position within the expert;
//   C: the walk again: position = cnt[w][e] + rank, the group's last lane advances cnt.
// Counts and positions are below 2^16 (MK <= kSortMax), so cnt holds 16-bit values.
constexpr int kPlanWaves = 16;
constexpr int kPlanExperts = 1024;  // expert ids < 2^10

__device__ __forceinline__ void plan_group(int e, bool valid, int lane, int& rank, int& cnt) {
    uint64_t same = __ballot(valid);
#pragma unroll
    for (int bit = 0; bit < 10; ++bit) {
        const bool on = (e >> bit) & 1;
        const uint64_t bal = __ballot(on);
        same &= on ? bal : ~bal;
    }
    rank = __popcll(same & ((1ull << lane) - 1ull));
    cnt = __popcll(same);
}

__global__ __launch_bounds__(1024) void k_plan_sort(MoeBufs B, int MK, int E) {
    __shared__ uint16_t cnt[kPlanWaves][kPlanExperts];
    __shared__ uint32_t scan[kPlanExperts];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    for (int i = tid; i < kPlanWaves * kPlanExperts; i += 1024) (&cnt[0][0])[i] = 0;
    __syncthreads();
    const int c = (MK + kPlanWaves - 1) / kPlanWaves;
    const int r0 = w * c < MK ? w * c : MK, r1 = r0 + c < MK ? r0 + c : MK;
    for (int b = r0; b < r1; b += 64) {  // A
        const int i = b + lane;
        const bool valid = i < r1;
        const int e = valid ? B.experts[i] : 0;
        int rank, n;
        plan_group(e, valid, lane, rank, n);
        if (valid && rank == n - 1) cnt[w][e] = static_cast<uint16_t>(cnt[w][e] + n);
    }
    __syncthreads();
    // B: tid = expert. scan holds total | (total > 0) << 16 (totals sum to MK < 2^16).
    uint32_t tot = 0;
    if (tid < E)
        for (int v = 0; v < kPlanWaves; ++v) tot += cnt[v][tid];
    const uint32_t own = tot | (tot ? 1u << 16 : 0u);
    scan[tid] = own;
    __syncthreads();
    for (int off = 1; off < 1024; off <<= 1) {  // inclusive scan
        const uint32_t t = tid >= off ? scan[tid - off] : 0u;
        __syncthreads();
        scan[tid] += t;
        __syncthreads();
    }
    const uint32_t excl = scan[tid] - own;
    int32_t* plan = B.plan;
    if (tid < E && tot) {
        const int slot = static_cast<int>(excl >> 16);
        plan[1 + slot] = tid;
        plan[1 + MK + slot] = static_cast<int>(excl & 0xFFFFu);
    }
    if (tid == 1023) {
        const int nu = static_cast<int>(scan[1023] >> 16);
        plan[0] = nu;
        plan[1 + MK + nu] = MK;
    }
    if (tid < E) {
        uint32_t run = excl & 0xFFFFu;
        for (int v = 0; v < kPlanWaves; ++v) {
            const uint32_t n = cnt[v][tid];
            cnt[v][tid] = static_cast<uint16_t>(run);
            run += n;
        }
    }
    __syncthreads();
    for (int b = r0; b < r1; b += 64) {  // C
        const int i = b + lane;
        const bool valid = i < r1;
        const int e = valid ? B.experts[i] : 0;
        int rank, n;
        plan_group(e, valid, lane, rank, n);
        if (valid) {
            const int pos = cnt[w][e] + rank;
            plan[2 + 2 * MK + pos] = i;
            plan[2 + 3 * MK + i] = pos;
        }
        // every lane has read cnt before the group's last lane advances it
        __builtin_amdgcn_wave_barrier();
        if (valid && rank == n - 1) cnt[w][e] = static_cast<uint16_t>(cnt[w][e] + n);
    }
}

// ============================================================== segmented GEMM (R9)
constexpr int kPfRows = 64;     // output rows per workgroup (4 waves x 16)
constexpr int kPfK = 256;       // inputs per K block (32 d8 codes: one packed code block)
constexpr int kPfRoutes = 64;   // routes per staged B tile
constexpr int kPfChunks = 4;    // B tiles per accumulation pass
constexpr int kPfPass = kPfRoutes * kPfChunks;
constexpr int kPfLd = kPfK + 8; // fp16 row pitch of the LDS tiles

typedef _Float16 Tile[kPfLd];

// The 64 x 256 fp16 weight tile of rows [o0, o0 + 64) of `expert`, K block kb, is decoded
// into As in two steps so that the code words of block kb + 1 can be in flight while block
// kb is decoded and multiplied: load_codes reads the 14 packed words (32 d8 codes) of row
// t / 4 into registers; decode_gather picks codes [8 (t % 4), 8 (t % 4) + 8) out of them and
// issues their fp16 codebook entries (16 bytes each, read through the cache); store_tile
// writes the entries to As.
__device__ __forceinline__ void load_codes(const ProjDev& P, int expert, int OUT, int o0, int kb,
                                           uint32_t (&w)[14]) {
    const int row = threadIdx.x >> 2;
    const uint32_t* src = P.codes + (static_cast<size_t>(expert) * OUT + o0 + row) * P.words + kb * 14;
#pragma unroll
    for (int i = 0; i < 7; ++i) {
        const uint2 v = reinterpret_cast<const uint2*>(src)[i];
        w[2 * i] = v.x;
        w[2 * i + 1] = v.y;
    }
}

__device__ __forceinline__ void decode_gather(const ProjDev& P, const uint32_t (&wc)[14], uint4 (&e)[8]) {
    const int qq = threadIdx.x & 3;
    uint32_t w[15];
#pragma unroll
    for (int i = 0; i < 14; ++i) w[i] = wc[i];
    w[14] = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t c0 = code_from<14>(w, i), c1 = code_from<14>(w, 8 + i);
        const uint32_t c2 = code_from<14>(w, 16 + i), c3 = code_from<14>(w, 24 + i);
        const uint32_t c = qq == 0 ? c0 : qq == 1 ? c1 : qq == 2 ? c2 : c3;
        e[i] = *reinterpret_cast<const uint4*>(P.book + static_cast<size_t>(c) * 8);
    }
}

__device__ __forceinline__ void store_tile(const uint4 (&e)[8], Tile* As) {
    const int t = threadIdx.x, row = t >> 2, qq = t & 3;
#pragma unroll
    for (int i = 0; i < 8; ++i) *reinterpret_cast<uint4*>(&As[row][64 * qq + 8 * i]) = e[i];
}

// Stage routes [64 ch, 64 ch + 64) of the pass (K block kb) in two steps, loads then LDS
// stores: thread t moves 8 fp16 of columns 8 (t % 32) for routes t / 32 + 8 m (m < 8); rows
// past np are zeros. src_row(j) gives the source row of pass route j in `src` ([*, IN] fp16).
template <typename SrcRow>
__device__ __forceinline__ void stage_load(const uint16_t* src, int IN, int kb, int ch, int np, uint4 (&v)[8],
                                           SrcRow src_row) {
    const int j0 = threadIdx.x >> 5, c8 = threadIdx.x & 31;
#pragma unroll
    for (int m = 0; m < 8; ++m) {
        const int route = ch * kPfRoutes + j0 + 8 * m;
        v[m] = make_uint4(0u, 0u, 0u, 0u);
        if (route < np)
            v[m] = *reinterpret_cast<const uint4*>(src + static_cast<size_t>(src_row(route)) * IN + kb * kPfK + 8 * c8);
    }
}

__device__ __forceinline__ void stage_store(const uint4 (&v)[8], Tile* Bt) {
    const int j0 = threadIdx.x >> 5, c8 = threadIdx.x & 31;
#pragma unroll
    for (int m = 0; m < 8; ++m) *reinterpret_cast<uint4*>(&Bt[j0 + 8 * m][8 * c8]) = v[m];
}

// One accumulation pass over all K blocks for routes [0, np) of the pass (np <= kPfPass):
// acc[4 ch + t] = rows 16 wave + (0..15) x routes 64 ch + 16 t + (0..15). Per K block: the
// codebook gathers of the block and the loads of its first B tile are issued together, then
// the next block's code words (clamped to the last block: always in bounds), which stay in
// flight through the block's MFMAs. The barriers wait only for LDS traffic, so they do not
// drain those prefetches. 16-route B sub-tiles with no route are skipped.
template <typename StageLoad>
__device__ __forceinline__ void pf_pass(const ProjDev& P, int expert, int OUT, int IN, int o0, int np, Tile* As,
                                        Tile* Bs, f4_t (&acc)[4 * kPfChunks], StageLoad stage_b) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, r16 = lane & 15, q = lane >> 4;
#pragma unroll
    for (int i = 0; i < 4 * kPfChunks; ++i) acc[i] = f4_t{0.f, 0.f, 0.f, 0.f};
    const int nch = (np + kPfRoutes - 1) / kPfRoutes;
    const int nkb = IN / kPfK;
    uint32_t w[14];
    load_codes(P, expert, OUT, o0, 0, w);
    for (int kb = 0; kb < nkb; ++kb) {
        lds_barrier_dma_pending();  // the previous K block's tiles are consumed
        {
            uint4 e[8], bv[8];
            decode_gather(P, w, e);
            stage_b(kb, 0, bv);
            load_codes(P, expert, OUT, o0, kb + 1 < nkb ? kb + 1 : kb, w);
            store_tile(e, As);
            stage_store(bv, Bs);
        }
        lds_barrier_dma_pending();
        h8_t af[8];
#pragma unroll
        for (int s = 0; s < 8; ++s) af[s] = *reinterpret_cast<const h8_t*>(&As[16 * wave + r16][32 * s + 8 * q]);
#pragma unroll
        for (int ch = 0; ch < kPfChunks; ++ch) {
            if (ch < nch) {  // workgroup-uniform
                if (ch) {
                    uint4 bv[8];
                    stage_b(kb, ch, bv);
                    lds_barrier_dma_pending();  // the previous B tile is consumed
                    stage_store(bv, Bs);
                    lds_barrier_dma_pending();
                }
                const int nv = np - ch * kPfRoutes;  // routes of this B tile (> 0)
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    if (16 * t < nv) {  // workgroup-uniform
#pragma unroll
                        for (int s = 0; s < 8; ++s) {
                            const h8_t bf = *reinterpret_cast<const h8_t*>(&Bs[16 * t + r16][32 * s + 8 * q]);
                            acc[4 * ch + t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[s], bf, acc[4 * ch + t], 0, 0, 0);
                        }
                    }
                }
            }
        }
    }
}

// D lane (c16 = l % 16, q = l / 16) register r of acc[i]: row 16 wave + 4q + r, route
// 64 (i / 4) + 16 (i % 4) + c16 of the pass; out row = sorted position pos0 + p0 + route, or
// that position's route index when rplan (the plan) is given (the down projection).
__device__ __forceinline__ void pf_store(const ProjDev& P, int expert, int OUT, int o0, int p0, int np, int pos0,
                                         const f4_t (&acc)[4 * kPfChunks], float* out, const int32_t* rplan = nullptr,
                                         int MK = 0) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, c16 = lane & 15, q = lane >> 4;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int o = o0 + 16 * wave + 4 * q + r;
        const float sc = h2f(P.scales[static_cast<size_t>(expert) * OUT + o]);
#pragma unroll
        for (int i = 0; i < 4 * kPfChunks; ++i) {
            const int j = (i >> 2) * kPfRoutes + (i & 3) * 16 + c16;
            if (j < np) {
                const int row = pos0 + p0 + j;
                out[static_cast<size_t>(rplan ? route_of_pos(rplan, MK, row) : row) * OUT + o] = sc * acc[i][r];
            }
        }
    }
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_gu_pf(LayerDev L, MoeBufs B, int M) {
    __shared__ __align__(16) Tile As[kPfRows];
    __shared__ __align__(16) Tile Bs[kPfRoutes];
    __shared__ int src_rows[kPfPass];  // source row of each route of the pass
    int expert, n, pos0;
    if (!slot_rows(B.plan, M, L.K, L.has_shared, blockIdx.y, L.E, &expert, &n, &pos0)) return;
    const bool shared = static_cast<int>(blockIdx.y) == B.plan[0];
    const int proj = blockIdx.z;
    const ProjDev& P = L.p[proj];
    const int o0 = blockIdx.x * kPfRows;
    float* out = proj == 0 ? B.g : B.u;
    f4_t acc[4 * kPfChunks];
    for (int p0 = 0; p0 < n; p0 += kPfPass) {
        const int np = n - p0 < kPfPass ? n - p0 : kPfPass;
        lds_barrier();  // the previous pass's row table is consumed
        for (int j = threadIdx.x; j < np; j += 256) src_rows[j] = route_row(B.plan, M, L.K, pos0, p0 + j, shared);
        // (published by the first barrier of the pass)
        pf_pass(P, expert, L.I, L.H, o0, np, As, Bs, acc, [&](int kb, int ch, uint4 (&v)[8]) {
            stage_load(B.x16, L.H, kb, ch, np, v, [&](int j) { return src_rows[j]; });
        });
        pf_store(P, expert, L.I, o0, p0, np, pos0, acc, out);
    }
}

__global__ __launch_bounds__(256) void k_swiglu_pf(MoeBufs B, int64_t total) {
    for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < total; i += static_cast<int64_t>(gridDim.x) * 256)
        B.h16[i] = f2h(swiglu(B.g[i], B.u[i]));
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_dn_pf(LayerDev L, MoeBufs B, int M) {
    __shared__ __align__(16) Tile As[kPfRows];
    __shared__ __align__(16) Tile Bs[kPfRoutes];
    int expert, n, pos0;
    if (!slot_rows(B.plan, M, L.K, L.has_shared, blockIdx.y, L.E, &expert, &n, &pos0)) return;
    const ProjDev& P = L.p[2];
    const int o0 = blockIdx.x * kPfRows;
    f4_t acc[4 * kPfChunks];
    for (int p0 = 0; p0 < n; p0 += kPfPass) {
        const int np = n - p0 < kPfPass ? n - p0 : kPfPass;
        pf_pass(P, expert, L.H, L.I, o0, np, As, Bs, acc, [&](int kb, int ch, uint4 (&v)[8]) {
            stage_load(B.h16, L.I, kb, ch, np, v, [&](int j) { return pos0 + p0 + j; });
        });
        pf_store(P, expert, L.H, o0, p0, np, pos0, acc, B.d, B.plan, M * L.K);
    }
}

template <int T>
hipError_t launch_router_rows_t(const LayerDev& L, const MoeBufs& B, int M, const uint16_t* x, hipStream_t st) {
    constexpr int NE = T <= 2 ? 8 : T <= 4 ? 4 : 2;  // router rows in registers: 16 T NE <= 128 VGPRs
    const int nr = L.E + (L.has_shared ? 1 : 0);
    return launch(k_logits_rows<T, NE>, dim3((nr + NE - 1) / NE, (M + 63) / 64), dim3(256), 0, st, L, B, M, x);
}

} // namespace

bool moe_supports_prefill(const LayerDev& L) {
    if (L.mixed) return false;
    for (int p = 0; p < 3; ++p)
        if (L.p[p].dim != 8 || L.p[p].bits != 14 || L.p[p].ngrp != 1 || !L.p[p].book) return false;
    return L.H % kPfK == 0 && L.I % kPfK == 0 && L.H % kPfRows == 0 && L.I % kPfRows == 0 && L.H % 512 == 0 &&
           L.H <= 4096 && L.E <= 65535;
}

hipError_t launch_router_rows(const LayerDev& L, const MoeBufs& B, int M, const uint16_t* x, hipStream_t st) {
    switch (L.H / 512) {
        case 1: return launch_router_rows_t<1>(L, B, M, x, st);
        case 2: return launch_router_rows_t<2>(L, B, M, x, st);
        case 3: return launch_router_rows_t<3>(L, B, M, x, st);
        case 4: return launch_router_rows_t<4>(L, B, M, x, st);
        case 5: return launch_router_rows_t<5>(L, B, M, x, st);
        case 6: return launch_router_rows_t<6>(L, B, M, x, st);
        case 8: return launch_router_rows_t<8>(L, B, M, x, st);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_topk_rows(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st) {
    if (M * L.K > kSortMax || L.E > 1024) return hipErrorInvalidValue;
    if (L.E == 512) return launch(k_topk_rows<8, true>, dim3((M + 3) / 4), dim3(256), 0, st, L, B, M);
    return launch(k_topk_rows<16, false>, dim3((M + 3) / 4), dim3(256), 0, st, L, B, M);
}

hipError_t launch_plan_sort(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st) {
    if (M * L.K > kSortMax || L.E > kPlanExperts) return hipErrorInvalidValue;
    return launch(k_plan_sort, dim3(1), dim3(1024), 0, st, B, M * L.K, L.E);
}

static int pf_slots(const LayerDev& L, int M) {
    const int MK = M * L.K;
    return (MK < L.E ? MK : L.E) + (L.has_shared ? 1 : 0);
}

hipError_t launch_gate_up_pf(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st) {
    return launch(k_gu_pf, dim3(L.I / kPfRows, pf_slots(L, M), 2), dim3(256), 0, st, L, B, M);
}

hipError_t launch_swiglu_pf(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st) {
    const int64_t total = static_cast<int64_t>(M * L.K + (L.has_shared ? M : 0)) * L.I;
    return launch(k_swiglu_pf, dim3(2048), dim3(256), 0, st, B, total);
}

hipError_t launch_down_pf(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st) {
    return launch(k_dn_pf, dim3(L.H / kPfRows, pf_slots(L, M), 1), dim3(256), 0, st, L, B, M);
}

} // namespace q38
