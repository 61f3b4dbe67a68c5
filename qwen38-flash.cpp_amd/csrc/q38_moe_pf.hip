// q38_moe_pf.hip — prefill-width sparse MoE (R1-R3, R9): 17..2048 rows per call, the
// SparseMoe::forward_prefill_impl segmented path (src/sparse_moe.cpp:2199-2624).
//
//   k_logits_rows  router logits, NE router rows per workgroup held in registers across
//                  the workgroup's request rows (the per-lane summation contract of the
//                  verify router), and the shared expert's gate
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
// Workgroup (gx, gy): routed router rows [NE gx, NE gx + NE) against request rows
// [rpw gy, rpw gy + rpw), wave w taking rows rpw gy + w, + 8, ... Lane l accumulates
// x*w over the columns 512t + 8l + j (t outer, j inner) with fmaf, then the xor butterfly
// and BF16 rounding: the logits equal the verify router's bit for bit. The launch sizes rpw
// so that the grid is resident at once (one pass of workgroups per CU slot, no partial
// second pass).
// planar: the fp16 copy of x is stored chunk-planar ([2][M][H / 2]: dims 4c..4c+3 of every
// subvector in plane c), the layout the LDS-codebook gate/up kernel reads its B operand from.
constexpr int kLogitsWaves = 8;

template <int T, int NE>
__global__ __launch_bounds__(64 * kLogitsWaves) void k_logits_rows(LayerDev L, MoeBufs B, int M, const uint16_t* __restrict__ x,
                                                     int planar, int rpw) {
    constexpr int H = 512 * T;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int e0 = blockIdx.x * NE;
    const int nr = L.E;
    uint4 wv[NE][T];
#pragma unroll
    for (int n = 0; n < NE; ++n) {
        const int e = e0 + n < nr ? e0 + n : nr - 1;
        const uint16_t* w = L.router + static_cast<size_t>(e) * H;
#pragma unroll
        for (int t = 0; t < T; ++t) wv[n][t] = *reinterpret_cast<const uint4*>(w + 512 * t + 8 * lane);
    }
    const bool store_x = blockIdx.x == 0 && x != B.x;
    const int rb = static_cast<int>(blockIdx.y) * rpw;
    const int r1 = rb + rpw < M ? rb + rpw : M;
    if (rb >= r1) return;
    auto load_row = [&](int r, uint4 (&v)[T]) {
#pragma unroll
        for (int t = 0; t < T; ++t) v[t] = *reinterpret_cast<const uint4*>(x + static_cast<size_t>(r) * H + 512 * t + 8 * lane);
    };
    // the request rows two and one steps ahead are in flight while a row's dot products run
    // (past the end the last row again: always in bounds)
    uint4 xa[T], xb[T];
    load_row(rb + wave < r1 ? rb + wave : r1 - 1, xa);
    load_row(rb + wave + kLogitsWaves < r1 ? rb + wave + kLogitsWaves : r1 - 1, xb);
    // the router bias of the lane's logits (loop-invariant: loaded once, so that no load in the
    // loop waits behind the prefetches)
    float rbias[scatter_slots<NE>()];
#pragma unroll
    for (int s = 0; s < scatter_slots<NE>(); ++s) {
        const int e = e0 + scatter_value<NE>(s, lane >> 4);
        rbias[s] = L.rbias ? L.rbias[e < nr ? e : nr - 1] : 0.0f;
    }
    // The shared expert's gate row (w_sg), spread over the grid's columns: wave 0 of column gx
    // takes request rows rb + gx, rb + gx + gridDim.x, ... of its range, with the same lane
    // contract; sgate = T(sigmoid(T(logit))).
    if (L.has_shared && wave == 0) {
        uint4 ws[T];
#pragma unroll
        for (int t = 0; t < T; ++t) ws[t] = *reinterpret_cast<const uint4*>(L.wsg + 512 * t + 8 * lane);
        for (int r = rb + static_cast<int>(blockIdx.x); r < r1; r += gridDim.x) {
            uint4 xs[T];
            load_row(r, xs);
            float a = 0.0f;
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const uint32_t xq[4] = {xs[t].x, xs[t].y, xs[t].z, xs[t].w};
                const uint32_t wq[4] = {ws[t].x, ws[t].y, ws[t].z, ws[t].w};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    a = __builtin_fmaf(bflo(xq[k]), bflo(wq[k]), a);
                    a = __builtin_fmaf(bfhi(xq[k]), bfhi(wq[k]), a);
                }
            }
            a = wave_sum_xor(a);
            if (lane == 0) B.sgate[r] = rbf(1.0f / (1.0f + expf(-rbf(a))));
        }
    }
    for (int r = rb + wave; r < r1; r += kLogitsWaves) {
        uint4 xv[T];
#pragma unroll
        for (int t = 0; t < T; ++t) {
            xv[t] = xa[t];
            xa[t] = xb[t];
        }
        load_row(r + 2 * kLogitsWaves < r1 ? r + 2 * kLogitsWaves : r1 - 1, xb);
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
        // the NE butterflies at once: 16-lane row q of acc[s] ends with router row
        // e0 + scatter_value<NE>(s, q)
        wave_sum_xor_scatter<NE>(acc);
#pragma unroll
        for (int s = 0; s < scatter_slots<NE>(); ++s) {
            const int e = e0 + scatter_value<NE>(s, lane >> 4);
            if ((lane & 15) == 0 && e < nr) {
                const float lg = rbf(acc[s]);
                B.logits[static_cast<size_t>(r) * L.E + e] = L.rbias ? lg + rbias[s] : lg;
            }
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
                if (planar) {
                    const size_t pa = static_cast<size_t>(r) * (H / 2) + (64 * t + lane) * 4;
                    *reinterpret_cast<uint2*>(B.x16 + pa) = make_uint2(hq[0], hq[1]);
                    *reinterpret_cast<uint2*>(B.x16 + static_cast<size_t>(M) * (H / 2) + pa) = make_uint2(hq[2], hq[3]);
                } else {
                    *reinterpret_cast<uint4*>(B.x16 + at) = make_uint4(hq[0], hq[1], hq[2], hq[3]);
                }
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
// within an expert), in one workgroup of 16 waves; the routes' experts are first copied into
// LDS (every load in flight at once), so neither walk waits on memory. Wave w owns the contiguous routes
// [w c, w c + c) and walks them 64 at a time in order; within such a batch, lanes with the
// same expert find each other with one ballot per expert-id bit, and a lane's rank is the
// number of lower lanes in its group.
//   A: every group's last lane adds the group size to cnt[w][e];
//   B: per expert, a scan over experts of the totals (and of the nonzero flags: the slot
//      numbers; shuffles within a wave, then the wave totals) gives its first position,
//      and a scan over waves turns cnt[w][e] into wave
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
    __shared__ uint32_t wtot[kPlanWaves];
    extern __shared__ uint16_t ex[];  // [MK] expert of every route
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    // Every route's expert into LDS at once (all loads in flight before the first store), the
    // counters cleared behind them; the walks then read LDS only.
    {
        constexpr int PT = kSortMax / 1024;
        int v[PT];
#pragma unroll
        for (int k = 0; k < PT; ++k) {
            const int i = tid + 1024 * k;
            v[k] = i < MK ? B.experts[i] : 0;
        }
        for (int i = tid; i < kPlanWaves * kPlanExperts / 8; i += 1024)
            reinterpret_cast<uint4*>(&cnt[0][0])[i] = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
        for (int k = 0; k < PT; ++k) {
            const int i = tid + 1024 * k;
            if (i < MK) ex[i] = static_cast<uint16_t>(v[k]);
        }
    }
    __syncthreads();
    const int c = (MK + kPlanWaves - 1) / kPlanWaves;
    const int r0 = w * c < MK ? w * c : MK, r1 = r0 + c < MK ? r0 + c : MK;
    for (int b = r0; b < r1; b += 64) {  // A
        const int i = b + lane;
        const bool valid = i < r1;
        const int e = valid ? ex[i] : 0;
        int rank, n;
        plan_group(e, valid, lane, rank, n);
        if (valid && rank == n - 1) cnt[w][e] = static_cast<uint16_t>(cnt[w][e] + n);
    }
    __syncthreads();
    // B: tid = expert. The scanned value is total | (total > 0) << 16 (totals sum to MK <
    // 2^16): an inclusive scan within each wave by shuffles, then the wave totals in order.
    uint32_t tot = 0;
    if (tid < E)
        for (int v = 0; v < kPlanWaves; ++v) tot += cnt[v][tid];
    const uint32_t own = tot | (tot ? 1u << 16 : 0u);
    uint32_t incl = own;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t t = __shfl_up(incl, o);
        if (lane >= o) incl += t;
    }
    if (lane == 63) wtot[w] = incl;
    __syncthreads();
    for (int v = 0; v < w; ++v) incl += wtot[v];
    const uint32_t excl = incl - own;
    int32_t* plan = B.plan;
    if (tid < E && tot) {
        const int slot = static_cast<int>(excl >> 16);
        plan[1 + slot] = tid;
        plan[1 + MK + slot] = static_cast<int>(excl & 0xFFFFu);
    }
    if (tid == 1023) {
        const int nu = static_cast<int>(incl >> 16);
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
        const int e = valid ? ex[i] : 0;
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

// ============================================================== segmented GEMM on LDS codebook chunks (R9)
// The same products with the codebook decode moved from the vector cache into LDS: a
// workgroup holds one 4-dim chunk of one projection's codebook (128 KiB, d8/14-bit, at LDS
// address 0) for the whole launch, so every decoded entry is an 8-byte LDS gather instead of
// a 16-byte cache line read. Work units are (expert slot, pass of up to 16 of the slot's
// routes); items are (unit, tile of output rows), and each workgroup walks a contiguous
// range of items, so the B operand (the pass's 16 route rows, this chunk's dims) stays in
// registers for all tiles of a unit. Wave (kh, rg): K part kh (lane quarter q owns one 16-
// or 32-code span of each of its rows) x row group rg (32 rows = two 16-row MFMA tiles);
// v_mfma_f32_16x16x32_f16 with A = the two gathered 4-dim entries of subvectors 2t, 2t + 1
// of the lane's span and B = the same subvectors' dims of route c16, read as one 16-byte
// word from the chunk-planar fp16 inputs. K parts are summed through LDS in part order.
// Each chunk writes its own partial-sum plane (times the row scale); the consumers add the
// two planes.
// At entry the workgroup derives the units' first item (ustart, a scan over the slots) and
// a table of its own units: expert, route count, first sorted position, first route, and
// per route of the unit the row it reads (gate/up: the request row) or writes (down: the
// route index), so a unit change costs LDS reads only. The code spans of item k + 1 are in
// flight while item k computes (two register sets, the loop unrolled by two, no copies);
// the next unit's B operand likewise.
constexpr int kSegThreads = 512;
constexpr int kSegRoutes = 16;                   // routes per unit (the MFMA's B columns)
constexpr int kSegMaxSlots = kPlanExperts + 1;   // routed slots + the shared one
constexpr int kSegKent = 1 << 14;                // d8/14-bit codebook entries
constexpr int kSegTab = 64;                      // units one workgroup walks (checked on the host)

struct SegTab {
    int32_t ustart[kSegMaxSlots + 1];
    int4 unit[kSegTab];                 // expert, route count, first sorted position, first route
    int32_t row[kSegTab][kSegRoutes];   // per route of the unit (-1 past the slot's routes)
};

__device__ __forceinline__ void seg_wait_vm() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// ustart[s] = the first unit of slot s (ustart[ns] = the unit count): slot s has
// ceil(n_s / 16) units. One wave, 64 slots per step (inclusive scan by shuffles).
__device__ __forceinline__ void seg_unit_scan(const int32_t* plan, int M, int K, int has_shared, int32_t* ustart) {
    const int lane = threadIdx.x & 63;
    const int nu = plan[0], ns = nu + (has_shared ? 1 : 0), MK = M * K;
    int base = 0;
    for (int s0 = 0; s0 < ns; s0 += 64) {
        const int s = s0 + lane;
        int n = 0;
        if (s < nu) n = plan[1 + MK + s + 1] - plan[1 + MK + s];
        else if (s < ns) n = M;
        int v = (n + kSegRoutes - 1) / kSegRoutes;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int t = __shfl_up(v, o);
            if (lane >= o) v += t;
        }
        if (s < ns) ustart[s + 1] = base + v;
        base += __shfl(v, 63);
    }
    if (lane == 0) ustart[0] = 0;
}

// Slot of unit u: the last s with ustart[s] <= u (every slot has at least one unit).
__device__ __forceinline__ int seg_slot(const int32_t* ustart, int ns, int u) {
    int lo = 0, hi = ns;
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (ustart[mid] <= u) lo = mid;
        else hi = mid;
    }
    return lo;
}

// The table of units [u0, u0 + nt) (every thread of the workgroup; ustart published).
template <bool DOWN>
__device__ __forceinline__ void seg_build_tab(const int32_t* plan, int M, int K, int has_shared, int E, int ns,
                                              int u0, int nt, SegTab& T) {
    const int MK = M * K, nu = plan[0];
    for (int t = threadIdx.x; t < nt * kSegRoutes; t += kSegThreads) {
        const int k = t / kSegRoutes, l = t % kSegRoutes;
        const int u = u0 + k;
        const int s = seg_slot(T.ustart, ns, u);
        int expert, n, pos0;
        slot_rows(plan, M, K, has_shared, s, E, &expert, &n, &pos0);
        const int j0 = (u - T.ustart[s]) * kSegRoutes, j = j0 + l;
        if (l == 0) T.unit[k] = make_int4(expert, n, pos0, j0);
        int r = -1;
        if (j < n) r = DOWN ? route_of_pos(plan, MK, pos0 + j) : route_row(plan, M, K, pos0, j, s == nu);
        T.row[k][l] = r;
    }
}

// Words [7 h, 7 h + 7) of the lane's 32-code block (h = half, for 16-code spans) or the
// whole block (14 words), from the tiled code layout: tile64 = the row's 64-row tile,
// rr = the row inside it; chunk c of a (tile, block) holds words 4c.. of its 64 rows.
template <int SPL>
__device__ __forceinline__ void seg_load_codes(const uint32_t* codes_t, int KS, size_t tile64, int rr, int blk,
                                               int half, uint32_t (&w)[SPL == 32 ? 14 : 7]) {
    const uint32_t* base = codes_t + (tile64 * KS + blk) * (14 * 64);
    if constexpr (SPL == 32) {
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            const uint4 v = *reinterpret_cast<const uint4*>(base + c * 256 + rr * 4);
            w[4 * c] = v.x; w[4 * c + 1] = v.y; w[4 * c + 2] = v.z; w[4 * c + 3] = v.w;
        }
        const uint2 v = *reinterpret_cast<const uint2*>(base + 768 + rr * 2);
        w[12] = v.x; w[13] = v.y;
    } else {
        // half 0: words 0..6 = chunk 0 + chunk 1 (three of four); half 1: words 7..13 =
        // chunk 1's last word + chunk 2 + chunk 3. The same three loads for every lane.
        const uint4 a = *reinterpret_cast<const uint4*>(base + (half ? 256 : 0) + rr * 4);
        const uint4 b = *reinterpret_cast<const uint4*>(base + (half ? 512 : 256) + rr * 4);
        const uint2 c = *reinterpret_cast<const uint2*>(base + 768 + rr * 2);
        w[0] = half ? a.w : a.x;
        w[1] = half ? b.x : a.y;
        w[2] = half ? b.y : a.z;
        w[3] = half ? b.z : a.w;
        w[4] = half ? b.w : b.x;
        w[5] = half ? c.x : b.y;
        w[6] = half ? c.y : b.z;
    }
}

// 8 x code q of a packed 32-code block (the LDS byte offset of its 4-dim entry): one shift
// (or funnel shift, for a code that spans two words) and one mask.
__device__ __forceinline__ uint32_t code14_x8(const uint32_t* w, int q) {
    const int bit = q * 14;
    const int wi = bit >> 5, sh = bit & 31;
    uint32_t v;
    if (sh < 3) v = w[wi] << (3 - sh);
    else if (sh + 14 > 32) v = __builtin_amdgcn_alignbit(w[wi + 1], w[wi], sh - 3);
    else v = w[wi] >> (sh - 3);
    return v & (((1u << 14) - 1u) << 3);
}

// Two 16-row tiles of one item: acc[i] += A(rows of w[i]) x B over NB16 16-byte B words (two
// subvectors each). MFMA m (step m / 2, tile m % 2) uses the gathers issued LA MFMAs
// earlier: scheduling barriers keep that order (left alone, the scheduler waits for each
// MFMA's two gathers right before it, and the LDS latency is exposed on every step).
template <int NB16, int NW>
__device__ __forceinline__ void seg_mfma(const uint32_t (&w)[2][NW], const uint4 (&bx)[NB16],
                                         const unsigned char* book, f4_t (&acc)[2]) {
    constexpr int NM = 2 * NB16, LA = 4;
    uint4 a[NM];
    auto gather = [&](int m) {
        const int t = m >> 1, i = m & 1;
        const uint2 a0 = *reinterpret_cast<const uint2*>(book + code14_x8(w[i], 2 * t));
        const uint2 a1 = *reinterpret_cast<const uint2*>(book + code14_x8(w[i], 2 * t + 1));
        a[m] = make_uint4(a0.x, a0.y, a1.x, a1.y);
    };
#pragma unroll
    for (int m = 0; m < LA; ++m) gather(m);
#pragma unroll
    for (int m = 0; m < NM; ++m) {
        __builtin_amdgcn_sched_barrier(0);
        if (m + LA < NM) gather(m + LA);
        acc[m & 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8_t, a[m]),
                                                            __builtin_bit_cast(h8_t, bx[m >> 1]), acc[m & 1], 0, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
}

__device__ __forceinline__ float4 seg_scaled(uint2 sc, const f4_t& a) {
    return make_float4(h2f(static_cast<uint16_t>(sc.x)) * a[0], h2f(static_cast<uint16_t>(sc.x >> 16)) * a[1],
                       h2f(static_cast<uint16_t>(sc.y)) * a[2], h2f(static_cast<uint16_t>(sc.y >> 16)) * a[3]);
}

// Items [i0, i1) of this workgroup.
__device__ __forceinline__ void seg_range(int n_items, int per_type, int idx, int& i0, int& i1) {
    i0 = static_cast<int>(static_cast<int64_t>(idx) * n_items / per_type);
    i1 = static_cast<int>(static_cast<int64_t>(idx + 1) * n_items / per_type);
}

// Gate/up (NSUB = H / 8 subvectors per row: 128 or 256; at 512 the K-part partial sums of
// four K parts would not fit in LDS beside the 128 KiB codebook chunk). Output rows of an item:
// TR = 32 * RG rows of I; chunk `chunk` of projection `proj` per workgroup type. B = rows of
// the chunk-planar fp16 inputs ([2][M][H / 2]).
template <int NSUB>
__global__ __launch_bounds__(kSegThreads) void k_gu_seg(LayerDev L, MoeBufs B, int M) {
    constexpr int KP = NSUB / 128, RG = 8 / KP, TR = 32 * RG, KS = NSUB / 32;
    static_assert(NSUB % 128 == 0 && KP * RG == 8, "8 waves = K parts x row groups");
    // One static LDS block (the codebook chunk at offset 0, known when compiling, so a gather's
    // address is its code offset alone), the K-part partial sums ([2][KP - 1][RG][2][64]) and
    // the unit table.
    constexpr int RED = 2 * (KP - 1) * RG * 2 * 64;
    struct Lds {
        uint2 book[kSegKent];
        f4_t red[RED > 0 ? RED : 1];
        SegTab T;
    };
    __shared__ Lds S;
    unsigned char* lds = reinterpret_cast<unsigned char*>(S.book);
    const unsigned char* book = lds;
    f4_t* red = S.red;
    SegTab& T = S.T;
    touch_kernargs<sizeof(LayerDev) + sizeof(MoeBufs) + sizeof(int)>();
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kh = wave % KP, rg = wave / KP;
    const int r16 = lane & 15, q = lane >> 4;
    const int x8 = blockIdx.x & 7, kk = blockIdx.x >> 3;
    const int type = kk & 3, proj = type >> 1, chunk = type & 1;
    const int per_type = (gridDim.x / 32) * 8;
    const int idx = (kk >> 2) * 8 + x8;  // the chunk-0 and chunk-1 workgroups of an index share an XCD
    const ProjDev& P = L.p[proj];
    const int H = L.H, I = L.I, K = L.K, E = L.E, hs = L.has_shared;
    const int32_t* plan = B.plan;
    if (wave == 0) seg_unit_scan(plan, M, K, hs, T.ustart);
    else dma_book<kSegKent>(P.book4 + static_cast<size_t>(chunk) * kSegKent * 4, lds, wave - 1, 7);
    lds_barrier_dma_pending();  // ustart published; the codebook copy still in flight
    const int ns = plan[0] + (hs ? 1 : 0);
    const int tiles = I / TR;
    int i0, i1;
    seg_range(T.ustart[ns] * tiles, per_type, idx, i0, i1);
    if (i0 >= i1) {
        seg_wait_vm();  // (the copy into LDS ends before the workgroup does)
        return;
    }
    const int u0 = i0 / tiles;
    seg_build_tab<false>(plan, M, K, hs, E, ns, u0, (i1 - 1) / tiles - u0 + 1, T);
    seg_wait_vm();
    lds_barrier();
    float* out = (proj == 0 ? B.g : B.u) + chunk * B.gu_plane;
    const uint16_t* xplane = B.x16 + static_cast<size_t>(chunk) * M * (H / 2);

    // B operand of unit k: request row T.row[k][r16], subvectors kh * 128 + 32 q + (0..31)
    auto load_b = [&](int k, uint4 (&bx)[16]) {
        const int row = T.row[k][r16];
        if (row >= 0) {
            const uint4* src = reinterpret_cast<const uint4*>(xplane + static_cast<size_t>(row) * (H / 2) +
                                                              (kh * 128 + 32 * q) * 4);
#pragma unroll
            for (int i = 0; i < 16; ++i) bx[i] = src[i];
        } else {
#pragma unroll
            for (int i = 0; i < 16; ++i) bx[i] = make_uint4(0u, 0u, 0u, 0u);
        }
    };
    auto load_codes = [&](int expert, int tile, uint32_t (&w)[2][14]) {
        const size_t row0 = static_cast<size_t>(expert) * I + tile * TR + rg * 32;
#pragma unroll
        for (int i = 0; i < 2; ++i)
            seg_load_codes<32>(P.codes_t, KS, row0 >> 6, static_cast<int>(row0 & 63) + 16 * i + r16, kh * 4 + q, 0,
                               w[i]);
    };
    uint4 bx[16];
    load_b(0, bx);
    // (k, tile): the current item's unit (table index) and tile, advanced without divisions
    int k = 0, tile = i0 - u0 * tiles;
    auto body = [&](int item, const uint32_t (&w)[2][14], uint32_t (&wn)[2][14]) {
        const int4 un = T.unit[k];  // expert, n, pos0, j0
        const int o0 = tile * TR + rg * 32 + 4 * q;
        // loads in the order they are needed: this item's row scales, the next unit's B
        // operand (when the unit changes), the next item's code spans (the last item: its
        // own again)
        uint2 sc[2];
        sc[0] = *reinterpret_cast<const uint2*>(P.scales + static_cast<size_t>(un.x) * I + o0);
        sc[1] = *reinterpret_cast<const uint2*>(P.scales + static_cast<size_t>(un.x) * I + o0 + 16);
        const bool last = item + 1 >= i1;
        const bool new_unit = !last && tile + 1 == tiles;
        load_codes(new_unit ? T.unit[k + 1].x : un.x, last ? tile : new_unit ? 0 : tile + 1, wn);
        f4_t acc[2] = {f4_t{0.f, 0.f, 0.f, 0.f}, f4_t{0.f, 0.f, 0.f, 0.f}};
        seg_mfma<16, 14>(w, bx, book, acc);
        // the next unit's B operand replaces this one as soon as the MFMAs have read it (a
        // second register set would not fit), in flight through the reduction and stores
        if (new_unit) load_b(k + 1, bx);
        const int buf = item & 1;
        if (KP > 1) {
            if (kh > 0)
#pragma unroll
                for (int i = 0; i < 2; ++i) red[(((buf * (KP - 1) + kh - 1) * RG + rg) * 2 + i) * 64 + lane] = acc[i];
            lds_barrier();  // (the other buffer was read before the previous item's barrier)
        }
        if (kh == 0) {
            const int j = un.w + r16;
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                f4_t sum = acc[i];
#pragma unroll
                for (int p = 1; p < KP; ++p) sum += red[(((buf * (KP - 1) + p - 1) * RG + rg) * 2 + i) * 64 + lane];
                if (j < un.y)
                    *reinterpret_cast<float4*>(out + static_cast<size_t>(un.z + j) * I + o0 + 16 * i) =
                        seg_scaled(sc[i], sum);
            }
        }
        if (new_unit) {
            ++k;
            tile = 0;
        } else {
            ++tile;
        }
    };
    uint32_t wa[2][14], wb[2][14];
    load_codes(T.unit[0].x, tile, wa);
    for (int item = i0; item < i1; item += 2) {
        body(item, wa, wb);
        if (item + 1 < i1) body(item + 1, wb, wa);
    }
}

// Down (NSUB = I / 8 subvectors per row: 64 or 128; SPL = NSUB / 4 per lane quarter, 16 =
// half a code block). One K part: wave rg owns rows 32 rg .. + 31 of a TR = 256-row tile of
// H. B = the pass's SwiGLU rows (chunk-planar fp16 at sorted positions); outputs at the
// route index.
template <int NSUB>
__global__ __launch_bounds__(kSegThreads) void k_dn_seg(LayerDev L, MoeBufs B, int M) {
    constexpr int SPL = NSUB / 4, TR = 256, KS = NSUB / 32;
    static_assert(SPL == 16 || SPL == 32, "16-code or 32-code lane spans");
    constexpr int NW = SPL == 32 ? 14 : 7, NB = SPL / 2;
    // one static LDS block: the codebook chunk at offset 0 (a gather's address is its code
    // offset alone), then the unit table
    struct Lds {
        uint2 book[kSegKent];
        SegTab T;
    };
    __shared__ Lds S;
    unsigned char* lds = reinterpret_cast<unsigned char*>(S.book);
    const unsigned char* book = lds;
    SegTab& T = S.T;
    touch_kernargs<sizeof(LayerDev) + sizeof(MoeBufs) + sizeof(int)>();
    const int tid = threadIdx.x, lane = tid & 63, rg = tid >> 6;
    const int r16 = lane & 15, q = lane >> 4;
    const int x8 = blockIdx.x & 7, kk = blockIdx.x >> 3;
    const int chunk = kk & 1;
    const int per_type = (gridDim.x / 16) * 8;
    const int idx = (kk >> 1) * 8 + x8;
    const ProjDev& P = L.p[2];
    const int H = L.H, I = L.I, K = L.K, E = L.E, hs = L.has_shared;
    const int32_t* plan = B.plan;
    if (rg == 0) seg_unit_scan(plan, M, K, hs, T.ustart);
    else dma_book<kSegKent>(P.book4 + static_cast<size_t>(chunk) * kSegKent * 4, lds, rg - 1, 7);
    lds_barrier_dma_pending();
    const int ns = plan[0] + (hs ? 1 : 0);
    const int tiles = H / TR;
    int i0, i1;
    seg_range(T.ustart[ns] * tiles, per_type, idx, i0, i1);
    if (i0 >= i1) {
        seg_wait_vm();
        return;
    }
    const int u0 = i0 / tiles;
    seg_build_tab<true>(plan, M, K, hs, E, ns, u0, (i1 - 1) / tiles - u0 + 1, T);
    seg_wait_vm();
    lds_barrier();
    float* dout = B.d + chunk * B.d_plane;
    const int MKM = M * K + (hs ? M : 0);
    const uint16_t* hplane = B.h16 + static_cast<size_t>(chunk) * MKM * (I / 2);
    const int blk = SPL * q / 32, half = SPL == 16 ? (q & 1) : 0;

    // B operand of unit k: SwiGLU row (sorted position) of route j0 + r16, subvectors
    // SPL q + (0..SPL-1)
    auto load_b = [&](int k, uint4 (&bx)[NB]) {
        const int4 un = T.unit[k];
        const int j = un.w + r16;
        if (j < un.y) {
            const uint4* src =
                reinterpret_cast<const uint4*>(hplane + static_cast<size_t>(un.z + j) * (I / 2) + SPL * q * 4);
#pragma unroll
            for (int i = 0; i < NB; ++i) bx[i] = src[i];
        } else {
#pragma unroll
            for (int i = 0; i < NB; ++i) bx[i] = make_uint4(0u, 0u, 0u, 0u);
        }
    };
    auto load_codes = [&](int expert, int tile, uint32_t (&w)[2][NW]) {
        const size_t row0 = static_cast<size_t>(expert) * H + tile * TR + rg * 32;
#pragma unroll
        for (int i = 0; i < 2; ++i)
            seg_load_codes<SPL>(P.codes_t, KS, row0 >> 6, static_cast<int>(row0 & 63) + 16 * i + r16, blk, half,
                                w[i]);
    };
    uint4 bx[NB];
    load_b(0, bx);
    int k = 0, tile = i0 - u0 * tiles;
    auto body = [&](int item, const uint32_t (&w)[2][NW], uint32_t (&wn)[2][NW]) {
        const int expert = T.unit[k].x;
        const int rt = T.row[k][r16];  // route index of the lane's route (-1: none)
        const int o0 = tile * TR + rg * 32 + 4 * q;
        uint2 sc[2];
        sc[0] = *reinterpret_cast<const uint2*>(P.scales + static_cast<size_t>(expert) * H + o0);
        sc[1] = *reinterpret_cast<const uint2*>(P.scales + static_cast<size_t>(expert) * H + o0 + 16);
        const bool last = item + 1 >= i1;
        const bool new_unit = !last && tile + 1 == tiles;
        load_codes(new_unit ? T.unit[k + 1].x : expert, last ? tile : new_unit ? 0 : tile + 1, wn);
        f4_t acc[2] = {f4_t{0.f, 0.f, 0.f, 0.f}, f4_t{0.f, 0.f, 0.f, 0.f}};
        seg_mfma<NB, NW>(w, bx, book, acc);
        if (new_unit) load_b(k + 1, bx);
        if (rt >= 0)
#pragma unroll
            for (int i = 0; i < 2; ++i)
                *reinterpret_cast<float4*>(dout + static_cast<size_t>(rt) * H + o0 + 16 * i) = seg_scaled(sc[i], acc[i]);
        if (new_unit) {
            ++k;
            tile = 0;
        } else {
            ++tile;
        }
    };
    uint32_t wa[2][NW], wb[2][NW];
    load_codes(T.unit[0].x, tile, wa);
    for (int item = i0; item < i1; item += 2) {
        body(item, wa, wb);
        if (item + 1 < i1) body(item + 1, wb, wa);
    }
}

// SwiGLU of every route, the two chunk planes of g and u added; the output is chunk-planar
// ([2][rows][I / 2]) for the down kernel's B operand.
__global__ __launch_bounds__(256) void k_swiglu_seg(MoeBufs B, int I, int64_t total) {
    const int64_t plane = total / 2;
    for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < total; i += static_cast<int64_t>(gridDim.x) * 256) {
        const int64_t pos = i / I;
        const int o = static_cast<int>(i - pos * I);
        const int64_t at = ((o >> 2) & 1) * plane + pos * (I / 2) + (o >> 3) * 4 + (o & 3);
        B.h16[at] = f2h(swiglu(B.g[i] + B.g[B.gu_plane + i], B.u[i] + B.u[B.gu_plane + i]));
    }
}

int router_cus() {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1)
        n = 256;
    return n;
}

template <int T>
hipError_t launch_router_rows_t(const LayerDev& L, const MoeBufs& B, int M, const uint16_t* x, hipStream_t st) {
    constexpr int NE = T <= 2 ? 8 : T <= 4 ? 4 : 2;  // router rows in registers: 16 T NE <= 128 VGPRs
    // workgroups resident at once (per instantiation; every device here is the same part)
    static std::atomic<int> resident{0};
    int slots = resident.load(std::memory_order_relaxed);
    if (slots == 0) {
        int nb = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, reinterpret_cast<const void*>(k_logits_rows<T, NE>),
                                                         64 * kLogitsWaves, 0) != hipSuccess || nb < 1)
            nb = 1;
        slots = nb * router_cus();
        resident.store(slots, std::memory_order_relaxed);
    }
    // request rows per workgroup: the grid fills the resident slots once (at least one row
    // per wave)
    const int gx = (L.E + NE - 1) / NE;
    int gy = slots / gx;
    gy = gy < 1 ? 1 : gy > (M + kLogitsWaves - 1) / kLogitsWaves ? (M + kLogitsWaves - 1) / kLogitsWaves : gy;
    const int rpw = (M + gy - 1) / gy;
    gy = (M + rpw - 1) / rpw;
    const int planar = prefill_planes(L, M) == 2 ? 1 : 0;
    return launch(k_logits_rows<T, NE>, dim3(gx, gy), dim3(64 * kLogitsWaves), 0, st, L, B, M, x, planar, rpw);
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
    const size_t lds = static_cast<size_t>(M * L.K) * 2;
    if (const hipError_t e = ensure_lds<k_plan_sort>(kSortMax * 2); e != hipSuccess) return e;
    return launch(k_plan_sort, dim3(1), dim3(1024), lds, st, B, M * L.K, L.E);
}

static int pf_slots(const LayerDev& L, int M) {
    const int MK = M * L.K;
    return (MK < L.E ? MK : L.E) + (L.has_shared ? 1 : 0);
}

// The LDS-codebook kernels serve layers with 4-dim codebook chunks and the tiled codes
// (d8/14-bit, H / 8 = 128 or 256, I / 8 = 64 or 128) when every workgroup's units fit
// its table; others take the tile kernels.
static int64_t seg_units_per_wg(const LayerDev& L, int M, int tiles, int per_type) {
    const int64_t MK = static_cast<int64_t>(M) * L.K;
    const int64_t ns = (MK < L.E ? MK : L.E) + (L.has_shared ? 1 : 0);
    const int64_t units = (MK + (L.has_shared ? M : 0) + (kSegRoutes - 1) * ns) / kSegRoutes;  // >= sum ceil(n/16)
    const int64_t items = (units * tiles + per_type - 1) / per_type;
    return (items + tiles - 1) / tiles + 1;
}

int prefill_planes(const LayerDev& L, int M) {
    for (int p = 0; p < 3; ++p)
        if (!L.p[p].book4 || !L.p[p].codes_t) return 1;
    const int gn = L.H / 8, dn = L.I / 8;
    if ((gn != 128 && gn != 256) || (dn != 64 && dn != 128)) return 1;
    const int gu_rows = 32 * (8 / (gn / 128));  // output rows of a gate/up item
    if (L.I % gu_rows || L.H % 256 || L.E + 1 > kSegMaxSlots) return 1;
    const int grid = mfma_grid();
    if (seg_units_per_wg(L, M, L.I / gu_rows, grid / 32 * 8) > kSegTab ||
        seg_units_per_wg(L, M, L.H / 256, grid / 16 * 8) > kSegTab)
        return 1;
    return 2;
}

template <int NSUB>
hipError_t launch_gu_seg_t(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st) {
    return launch(k_gu_seg<NSUB>, dim3(mfma_grid()), dim3(kSegThreads), 0, st, L, B, M);
}
template <int NSUB>
hipError_t launch_dn_seg_t(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st) {
    return launch(k_dn_seg<NSUB>, dim3(mfma_grid()), dim3(kSegThreads), 0, st, L, B, M);
}

hipError_t launch_gate_up_pf(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st) {
    if (prefill_planes(L, M) == 2) {
        switch (L.H / 8) {
            case 128: return launch_gu_seg_t<128>(L, B, M, st);
            case 256: return launch_gu_seg_t<256>(L, B, M, st);
            default: return hipErrorInvalidValue;
        }
    }
    return launch(k_gu_pf, dim3(L.I / kPfRows, pf_slots(L, M), 2), dim3(256), 0, st, L, B, M);
}

hipError_t launch_swiglu_pf(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st) {
    const int64_t total = static_cast<int64_t>(M * L.K + (L.has_shared ? M : 0)) * L.I;
    if (prefill_planes(L, M) == 2) return launch(k_swiglu_seg, dim3(2048), dim3(256), 0, st, B, L.I, total);
    return launch(k_swiglu_pf, dim3(2048), dim3(256), 0, st, B, total);
}

hipError_t launch_down_pf(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st) {
    if (prefill_planes(L, M) == 2) {
        if (L.I / 8 == 64) return launch_dn_seg_t<64>(L, B, M, st);
        if (L.I / 8 == 128) return launch_dn_seg_t<128>(L, B, M, st);
        return hipErrorInvalidValue;
    }
    return launch(k_dn_pf, dim3(L.H / kPfRows, pf_slots(L, M), 1), dim3(256), 0, st, L, B, M);
}

} // namespace q38
