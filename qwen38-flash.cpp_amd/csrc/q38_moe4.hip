// q38_moe4.hip — expert projections for verify widths of up to four rows (R2-R5, R7, R8)
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
// Each workgroup keeps one 4-dim chunk of one codebook in LDS for the whole launch and
// walks its share of (expert slot, tile) items. The kernels are built around the latency
// chain of a verify layer:
//   k_gu4  the non-routing waves start the codebook chunk's copy into LDS (the direct
//          global-to-LDS path) at kernel entry; the routing waves (one per request row)
//          load their logits, their row's chunk dims and a share of the down codebook's
//          lines (so the down kernel finds them in L2), and run softmax + top-k as soon as
//          the logits are in; wave 0 turns the rows' experts into the plan while the copy
//          finishes; then every wave walks its items over a ring of three in flight (item
//          k computes, then item k + 3's code spans are requested into its slot).
//   k_dn4  the plan is read first; the codebook chunk (into registers) follows at once and
//          the code spans, gate/up partial sums and scales of the first D items as soon as
//          the plan is in LDS; the chunk is stored to LDS behind them.
//          Down outputs are written at the route index (request row * k + slot; the
//          shared expert's rows after the routed ones), so the combine needs no plan.
//   k_gd4  both bodies in one launch, then the combine (the config-1 geometry): the down
//          kernel's launch, plan read and first waits leave the layer's latency chain, and
//          values cross workgroups through agent-coherent stores and polled loads.
#include "q38_moe_dev.hpp"

namespace q38 {
namespace {

typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef float v4f_t __attribute__((ext_vector_type(4)));
typedef uint32_t u4_t __attribute__((ext_vector_type(4)));

constexpr int kNarrow = 4;  // input rows per instruction (the B columns)
constexpr int kNarrowPlan = 2 + 4 * kNarrow * kMaxTopK;

// One 32-code block (BITS words) of the lane's row plus a zero pad word for code_from, from
// the tiled copy (ProjDev::codes_t): blk is the (64-row tile, block) base; chunk c holds
// words 4c.. of the 64 rows interleaved, so each load is contiguous across the wave.
template <int BITS>
__device__ __forceinline__ void load_code_block_tiled(const uint32_t* blk, int lane, uint32_t* w) {
#pragma unroll
    for (int c = 0; c < (BITS + 3) / 4; ++c) {
        const int cw = BITS - 4 * c < 4 ? BITS - 4 * c : 4;
        const uint32_t* src = blk + c * 256 + lane * cw;
        if (cw == 4) {
            const uint4 v = *reinterpret_cast<const uint4*>(src);
            w[4 * c] = v.x; w[4 * c + 1] = v.y; w[4 * c + 2] = v.z; w[4 * c + 3] = v.w;
        } else if (cw == 2) {
            const uint2 v = *reinterpret_cast<const uint2*>(src);
            w[4 * c] = v.x; w[4 * c + 1] = v.y;
        } else {
            for (int i = 0; i < cw; ++i) w[4 * c + i] = src[i];
        }
    }
    w[BITS] = 0;
}

// 32 steps of one K slice: A = codebook entries of the lane's row, B = bops[t]. Even and
// odd steps accumulate separately (two independent MFMA chains), added at the end.
template <int BITS>
__device__ __forceinline__ v4f_t slice_mfma(const uint32_t* cw, const uint2* book, const uint2* bops) {
    v4f_t acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < 32; t += 2) {
        const uint2 a0 = book[code_from<BITS>(cw, t)];
        const uint2 a1 = book[code_from<BITS>(cw, t + 1)];
        acc0 = __builtin_amdgcn_mfma_f32_4x4x4f16(__builtin_bit_cast(h4_t, a0), __builtin_bit_cast(h4_t, bops[t]), acc0,
                                                   0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_4x4x4f16(__builtin_bit_cast(h4_t, a1), __builtin_bit_cast(h4_t, bops[t + 1]),
                                                   acc1, 0, 0, 0);
    }
    return acc0 + acc1;
}

// The same 32 steps with one scale per 8 subvectors (64 inputs of d8 codes, the checkpoint
// layout): the four groups of the slice accumulate separately (t within a group in order,
// the groups interleaved), then each lane's rows (lane & ~3) + r are scaled per group and
// the groups added in order: gs[r] holds row r's four fp16 group scales.
template <int BITS>
__device__ __forceinline__ v4f_t slice_mfma_g8(const uint32_t* cw, const uint2* book, const uint2* bops,
                                               const uint2 (&gs)[4]) {
    v4f_t acc[4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const uint2 a = book[code_from<BITS>(cw, 8 * g + t)];
            acc[g] = __builtin_amdgcn_mfma_f32_4x4x4f16(__builtin_bit_cast(h4_t, a),
                                                        __builtin_bit_cast(h4_t, bops[8 * g + t]), acc[g], 0, 0, 0);
        }
    v4f_t out;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const uint16_t s4[4] = {static_cast<uint16_t>(gs[r].x), static_cast<uint16_t>(gs[r].x >> 16),
                                static_cast<uint16_t>(gs[r].y), static_cast<uint16_t>(gs[r].y >> 16)};
        float v = 0.0f;
#pragma unroll
        for (int g = 0; g < 4; ++g) v = fmaf(h2f(s4[g]), acc[g][r], v);
        out[r] = v;
    }
    return out;
}

// Scales an item needs. Per row (G8 = 0): k_gu4 keeps the aligned word holding its output
// thread's row scale, k_dn4 the four rows' scales of its output lanes. Per group (G8 = 8):
// the lane's rows (lane & ~3) + 0..3, the four groups of its wave's K slice.
template <int G8>
struct ItemScales {
    uint2 g[4];
};
template <>
struct ItemScales<0> {
    uint2 w;
};
// Group scales of rows row0 + (lane & ~3) + 0..3, groups g0 .. g0 + 3 ([rows, ngrp] fp16).
__device__ __forceinline__ void load_group_scales(const uint16_t* scales, size_t row0, int lane, int ngrp, int g0,
                                                  uint2 (&gs)[4]) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
        gs[r] = *reinterpret_cast<const uint2*>(scales + (row0 + (lane & ~3) + r) * ngrp + g0);
}

__device__ __forceinline__ void wait_vm_all() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Gate/up values inside k_gd4: agent-scope relaxed atomics (stores and loads that are
// coherent across the XCDs' L2s), plain accesses in the two-kernel path.
template <bool AGENT>
__device__ __forceinline__ void store_f32(float* p, float v) {
    if constexpr (AGENT) __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else *p = v;
}
template <bool AGENT>
__device__ __forceinline__ float load_f32(const float* p) {
    if constexpr (AGENT) return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else return *p;
}
// The reset pattern of the gate/up planes (all ones: a NaN that no arithmetic produces).
__device__ __forceinline__ bool gu_unset(float v) { return __float_as_uint(v) == 0xFFFFFFFFu; }
} // namespace

// Status of the bounded waits between workgroups (one word per device, in the code object):
// bit 0 is set by every thread whose wait gave up with a value still unset. The host reads
// and clears it (read_wait_status).
__device__ uint32_t g_wait_status;

namespace {
__device__ __forceinline__ void wait_gave_up() {
    __hip_atomic_fetch_or(&g_wait_status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Gate and up projections. Workgroup type = (projection, codebook chunk); waves = K slices.
// Items are 64-row tiles of I; the 4 B columns are the request rows (rows not routed to the
// item's expert are computed and discarded). Output: partial sums of this chunk, times the
// row scale, at the route's sorted position (the gate/up chunk planes).
// One workgroup per CU (the LDS codebook chunk), so a SIMD runs at most ceil(waves / 4)
// of its waves: the register budget is set by that, not by a higher occupancy target.
// LDS: codebook chunk [KENT][4] fp16, cross-wave partial sums [2][KS][64][4] f32; before
// the items, the chunk's dims of the request rows [4][NSUB][4] fp16 and the routing waves'
// top-k candidates [4][64] u64 share the partial-sum area.
// (the x staging and the routing waves' candidate lists live inside the partial-sum area,
// which the items use only after both are consumed)
template <int BITS, int NSUB, int NCHUNK>
constexpr size_t gu4_lds_bytes() {
    return (size_t{1} << BITS) * 8 + 2 * (NSUB / 32) * 64 * 16;
}

// FUSED: the gate/up half of k_gd4, whose outputs are read by the down half of other
// workgroups of the same launch (agent-coherent stores, see k_gd4).
// dn_fill (FUSED): receives the workgroup's down codebook chunk for the down half (16-byte
// granules tid + NT q), requested a few granules per item behind the items' own loads, while
// the items keep the CU's LDS busy and leave its memory path mostly idle.
// wt (FUSED): the rows' route weights in LDS, for the fused kernel's combine tail.
template <int BITS, int NSUB, int NCHUNK, int D, int G8, bool FUSED>
__device__ __forceinline__ void gu4_body(const LayerDev& L, const MoeBufs& B, int M, unsigned char* lds,
                                         int32_t* ex, int32_t* plan, int32_t* slot_pos, u4_t* dn_fill, float* wt) {
    constexpr int KS = NSUB / 32;
    constexpr int NT = 64 * KS;
    constexpr int KENT = 1 << BITS;
    constexpr int TYPES = 2 * NCHUNK;
    static_assert(kNarrow * NSUB * 8 + kNarrow * 64 * 8 <= 2 * KS * 64 * 16, "staging fits the partial sums");
    const uint2* book = reinterpret_cast<const uint2*>(lds);
    float* red = reinterpret_cast<float*>(lds + KENT * 8);  // [2][KS][64][4]
    uint2* xs = reinterpret_cast<uint2*>(lds + KENT * 8);                       // [4][NSUB], in red
    uint64_t* cand = reinterpret_cast<uint64_t*>(lds + KENT * 8 + kNarrow * NSUB * 8);  // [4][64], in red
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int x8 = blockIdx.x & 7, kk = blockIdx.x >> 3;
    const int type = kk % TYPES;
    const int proj = type / NCHUNK, chunk = type % NCHUNK;
    const int per_type = (gridDim.x / (8 * TYPES)) * 8;
    const int idx = (kk / TYPES) * 8 + x8;  // items of one index run on one XCD for all types
    const ProjDev& P = L.p[proj];
    const int H = L.H, I = L.I, K = L.K, MK = M * K;

    // 1. The routing waves load their row's logits (E = 512: 64 lanes x 8), behind them their
    //    row's dims of the chunk (NSUB / 64 8-byte loads per lane) and one word per 128-byte
    //    line of a share of the down projection's codebook (same geometry; the workgroups of
    //    an XCD cover it, so the down kernel's chunk fills find it in the XCD's L2; the words
    //    are dropped), wait for the logits only, select their row's experts and stage their
    //    row's chunk dims. The non-routing waves skip that block and copy the codebook chunk
    //    into LDS at once (the copy's block comes second, so no copy is pending in the code
    //    of the routing waves as the compiler sees it).
    static_assert(NSUB % 64 == 0, "whole 64-lane passes over the subvectors");
    constexpr int XPW = NSUB / 64;
    Q38_STAMP(8192, 0);
    uint32_t warm = 0;
    if (wave < M) {
        float lg[8];
        uint2 xv[XPW];
        topk_load_row_t<8, true>(L, B, wave, lg);
#pragma unroll
        for (int q = 0; q < XPW; ++q)
            xv[q] = *reinterpret_cast<const uint2*>(B.x16 + static_cast<size_t>(wave) * H +
                                                    (lane + 64 * q) * (4 * NCHUNK) + 4 * chunk);
        // (lines of the down book itself: (1 << bits) entries of dim fp16 values; the gate/up
        // book's geometry may differ, e.g. d8/14-bit gate/up over a d4/8-bit down)
        const int lines = ((1 << L.p[2].bits) * L.p[2].dim * 2) >> 7;
        warm = reinterpret_cast<const uint32_t*>(L.p[2].book4)[(((kk * M + wave) * 64 + lane) % lines) * 32];
#pragma unroll
        for (int j = 0; j < 8; ++j) asm volatile("" ::"v"(lg[j]));
        Q38_STAMP(8192, 1);
        Q38_STAMP(8192, 2);
        topk_select_row_fast<8>(L, B, wave, lg, ex, blockIdx.x == 0, cand + 64 * wave, FUSED ? wt : nullptr);
#pragma unroll
        for (int q = 0; q < XPW; ++q) xs[wave * NSUB + lane + 64 * q] = xv[q];
    }
    if (wave >= M) dma_book<KENT>(P.book4 + static_cast<size_t>(chunk) * KENT * 4, lds, wave - M, KS - M);
    Q38_STAMP(8192, 3);
    // 3. The plan of every row's routes (R3), published by workgroup 0. Wave 0 (a routing
    //    wave: no copy of its own in flight) builds it while the copy finishes; the barrier
    //    before it waits for LDS writes only, the one after it for every wave's copy too.
    lds_barrier_dma_pending();
    if (wave == 0) plan_wave(M, K, ex, plan, slot_pos);
    Q38_STAMP(8192, 14);
    wait_vm_all();
    Q38_STAMP_T(8192, 15, 64 * M);
    lds_barrier();
    asm volatile("" ::"v"(warm));
    Q38_STAMP(8192, 4);
    if (blockIdx.x == 0)
        for (int i = tid; i < 2 + 4 * MK; i += NT) B.plan[i] = plan[i];

    // 4. The code spans and row scales of this workgroup's first D items and the B operand
    //    from LDS (lane 4b + j: the 4 chunk dims of request row j for each of the wave's 32
    //    subvectors). Item k waits only for its own loads (they complete in order).
    const int tiles = I / 64;
    const int nu = plan[0];
    const int n_items = (nu + (L.has_shared ? 1 : 0)) * tiles;
    const int r_out = (tid >> 2) & 63;  // output role (tid < 256): weight row of the tile
    const int E = L.E;
    // (the plan entry is read from LDS before the value select, so that the compiler cannot
    // turn it into one generic load from either LDS or the kernel arguments)
    auto item_expert = [&](int item) {
        const int ui = item / tiles;
        const int pe = plan[1 + (ui < nu ? ui : 0)];
        return ui < nu ? pe : E;
    };
    // This workgroup's items are idx + j * per_type, j < my_n. Their loads are issued
    // unconditionally (past the end: the last item again, an L2 hit), so the compiler counts
    // them exactly and item k waits only for its own.
    const int my_n = n_items > idx ? (n_items - idx + per_type - 1) / per_type : 0;
    auto load_item = [&](int j, uint32_t* cw, ItemScales<G8>& sc) {
        const int item = my_n > 0 ? idx + (j < my_n ? j : my_n - 1) * per_type : 0;
        const int expert = item_expert(item);
        const size_t row = static_cast<size_t>(expert) * I + (item % tiles) * 64;
        load_code_block_tiled<BITS>(P.codes_t + ((row >> 6) * KS + wave) * (BITS * 64), lane, cw);
        if constexpr (G8 == 0) {
            // the aligned 32-bit word holding the row's fp16 scale (no 16-bit load to widen)
            sc.w.x = *reinterpret_cast<const uint32_t*>(P.scales + ((row + r_out) & ~size_t{1}));
        } else {
            load_group_scales(P.scales, row, lane, P.ngrp, wave * (32 / G8), sc.g);
        }
    };
    constexpr int PF = D < 3 ? D : 3;  // items in flight
    uint32_t cw[PF][BITS + 1];
    ItemScales<G8> sc[PF];
#pragma unroll
    for (int k = 0; k < PF; ++k) load_item(k, cw[k], sc[k]);  // (no items: item 0, unused)
    uint2 xb[32];
    {
        const int jx = (lane & 3) < M ? (lane & 3) : 0;
#pragma unroll
        for (int t = 0; t < 32; ++t) xb[t] = xs[jx * NSUB + wave * 32 + t];
    }
    lds_barrier();  // every wave has its B operand before the items overwrite the staging
    Q38_STAMP(8192, 5);

    // 5. Items. The first D run as straight-line code over a ring of PF slots: item k's
    //    compute, then the loads of item k + PF into its slot (unconditional, clamped), with
    //    no other memory instruction in between (results stay in registers until all D are
    //    done), so item k waits only for its own loads while later items stream in behind
    //    the compute. Items past D (more per workgroup than the launch planned) take a loop.
    //    Output thread tid < 256: weight row r_out of the tile x request row tid & 3.
    float* out = (proj == 0 ? B.g : B.u) + chunk * B.gu_plane;
    auto item_compute = [&](int j, const uint32_t* cwj, const ItemScales<G8>& scj, float& ov, int& oat) {
        const int item = idx + j * per_type;
        const int buf = j & 1;
        v4f_t acc;
        if constexpr (G8 == 0) acc = slice_mfma<BITS>(cwj, book, xb);
        else acc = slice_mfma_g8<BITS>(cwj, book, xb, scj.g);
        if (j == 0) Q38_STAMPV(8192, 6, acc[0]);
        reinterpret_cast<v4f_t*>(red)[(buf * KS + wave) * 64 + lane] = acc;
        lds_barrier();  // (the other buffer's readers passed the previous item's barrier)
        if (j == 0) Q38_STAMP(8192, 7);
        oat = -1;
        if (tid < 64 * kNarrow) {
            const int jr = tid & 3;  // request row
            const int pos = jr < M ? slot_pos[(item / tiles) * 4 + jr] : -1;
            if (pos >= 0) {
                const int src = (r_out & ~3) | jr, reg = r_out & 3;
                float s = 0.0f;
#pragma unroll
                for (int w = 0; w < KS; ++w) s += red[((buf * KS + w) * 64 + src) * 4 + reg];
                if constexpr (G8 == 0) ov = h2f(static_cast<uint16_t>(scj.w.x >> (16 * (r_out & 1)))) * s;
                else ov = s;  // (the group scales are applied in the slices)
                oat = pos * I + (item % tiles) * 64 + r_out;
            }
        }
    };
    float ov[D];
    int oat[D];
    // (FUSED: the down chunk has the gate/up geometry; its granules are spread over the first
    // FI items, so that the last ones still have two items' time to arrive)
    constexpr int NFILL = FUSED ? KENT / 2 / NT : 0, FI = D > 3 ? D - 2 : 1;
    const u4_t* dsrc = reinterpret_cast<const u4_t*>(L.p[2].book4 + static_cast<size_t>(kk % NCHUNK) * KENT * 4);
#pragma unroll
    for (int k = 0; k < D; ++k) {
        oat[k] = -1;
        if (k < my_n) item_compute(k, cw[k % PF], sc[k % PF], ov[k], oat[k]);
        if (k + PF < D) load_item(k + PF, cw[k % PF], sc[k % PF]);
        if constexpr (FUSED) {
#pragma unroll
            for (int q = NFILL * k / FI; q < (k < FI ? NFILL * (k + 1) / FI : 0); ++q) dn_fill[q] = dsrc[tid + q * NT];
        }
        if (k == 0) Q38_STAMP(8192, 8);
    }
#pragma unroll
    for (int k = 0; k < D; ++k)
        if (oat[k] >= 0) store_f32<FUSED>(out + oat[k], ov[k]);
    for (int jj = D; jj < my_n; ++jj) {
        uint32_t c1[BITS + 1];
        ItemScales<G8> s1;
        load_item(jj, c1, s1);
        float o1;
        int a1;
        item_compute(jj, c1, s1, o1, a1);
        if (a1 >= 0) store_f32<FUSED>(out + a1, o1);
    }
    Q38_STAMP(8192, 9);
#ifdef Q38_TRACE
    if (threadIdx.x == 0) g_trace[8192 + 16 * blockIdx.x + 10] = my_n;
#endif
}

template <int BITS, int NSUB, int NCHUNK, int D, int G8 = 0>
__global__ __launch_bounds__(2 * NSUB) __attribute__((amdgpu_waves_per_eu(1, (NSUB / 32 + 3) / 4)))
void k_gu4(LayerDev L, MoeBufs B, int M) {
    extern __shared__ __align__(16) unsigned char lds[];
    __shared__ int32_t ex[kNarrowMaxRoutes];
    __shared__ int32_t plan[kNarrowPlan];
    __shared__ int32_t slot_pos[(kNarrowMaxRoutes + 1) * 4];
    touch_kernargs<sizeof(LayerDev) + sizeof(MoeBufs) + sizeof(int)>();
    gu4_body<BITS, NSUB, NCHUNK, D, G8, false>(L, B, M, lds, ex, plan, slot_pos, nullptr, nullptr);
}

// Down projection. Workgroup type = codebook chunk; 8 waves = KS K slices x RG row groups,
// items are (slot, TR = 64 RG rows of H). The B columns are the slot's routes: their SwiGLU
// rows (this chunk's dims, fp16) are formed per item from the gate/up chunk planes, which
// are requested with the item's code spans, D items ahead.
// FUSED: the down half of k_gd4. The plan is already in LDS (built by this workgroup's
// gate/up half), and the gate/up values are read agent-coherent and re-read until none
// holds the reset pattern (the gate/up half of another workgroup has not stored it yet).
// hs: SwiGLU rows of the item's routes, [kNarrow][NSUB] fp16 quads.
template <int BITS, int NSUB, int NCHUNK, int D, int G8, bool FUSED>
__device__ __forceinline__ void dn4_body(const LayerDev& L, const MoeBufs& B, int M, unsigned char* lds,
                                         int32_t* plan, uint2* hs, const u4_t* pre_fill) {
    constexpr int KS = NSUB / 32, RG = 8 / KS, TR = 64 * RG;
    constexpr int NT = 512, KENT = 1 << BITS;
    static_assert(KS * RG == 8, "8 waves");
    const uint2* book = reinterpret_cast<const uint2*>(lds);
    float* red = reinterpret_cast<float*>(lds + KENT * 8);  // [RG][KS-1][64][4]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int x8 = blockIdx.x & 7, kk = blockIdx.x >> 3;
    const int chunk = kk % NCHUNK;
    const int per_type = (gridDim.x / (8 * NCHUNK)) * 8;
    const int idx = (kk / NCHUNK) * 8 + x8;
    const ProjDev& P = L.p[2];
    const int H = L.H, I = L.I, K = L.K, MK = M * K;
    // (E as a register value: a select between an LDS plan entry and an argument held in
    // memory would otherwise become one generic load, whose wait drains every load in flight)
    const int E = __builtin_amdgcn_readfirstlane(L.E);
    const int kh = wave % KS, rg = wave / KS;

    // 1. The plan (written by the gate/up kernel) into LDS, then the codebook chunk loads
    //    into registers (a wave's loads complete in order: the plan must not queue behind
    //    them). The chunk is stored to LDS after the item loads below have been issued, so
    //    every wait is on registers and the compiler counts it exactly.
    const int plan_n = 2 + 4 * MK;
    Q38_STAMP(16384, 0);
    if (!FUSED && tid < plan_n) plan[tid] = B.plan[tid];
    constexpr int NG = KENT / 2;  // 16-byte granules of the chunk
    constexpr int NFILL = (NG + NT - 1) / NT;
    u4_t fv[NFILL];
    if constexpr (FUSED) {  // (requested by the gate/up half)
#pragma unroll
        for (int q = 0; q < NFILL; ++q) fv[q] = pre_fill[q];
    } else {
        const u4_t* src = reinterpret_cast<const u4_t*>(P.book4 + static_cast<size_t>(chunk) * KENT * 4);
#pragma unroll
        for (int q = 0; q < NFILL; ++q) {
            const int i = tid + q * NT;
            fv[q] = src[i < NG ? i : NG - 1];
        }
    }
    lds_barrier();
    Q38_STAMP(16384, 1);

    // 2. Code spans and gate/up quads of the first D items.
    const int nu = plan[0];
    const int tiles = FUSED ? 2048 / TR : H / TR;  // (the fused layers have H = 2048)
    const int n_items = (nu + (L.has_shared ? 1 : 0)) * tiles;
    const bool two = FUSED || L.gu_parts == 2;  // (the fused layers' gate/up write two planes)
    // An item's slot (expert, route count, first route position), read from the plan once.
    struct Slot {
        int expert, n, pos0;
    };
    auto slot_of = [&](int item) {
        Slot t;
        slot_rows(plan, M, K, L.has_shared, item / tiles, E, &t.expert, &t.n, &t.pos0);
        return t;
    };
    auto code_src = [&](int item, const Slot& t) {  // this wave's (64-row tile, block) in the tiled codes
        const size_t row0 = static_cast<size_t>(t.expert) * H + (item % tiles) * TR + rg * 64;
        return P.codes_t + ((row0 >> 6) * KS + kh) * (BITS * 64);
    };
    // Gate/up chunk-plane values of the SwiGLU elements this thread forms: element e = tid
    // + 512 q (q < GQ) of the slot's n routes x NSUB subvectors x 4 chunk dims (route e /
    // (4 NSUB), subvector e / 4 % NSUB, dim e % 4). Loads are unconditional: elements past
    // the slot's routes repeat its last element, so the compiler counts every load.
    constexpr int GQ = (kNarrow * NSUB * 4 + NT - 1) / NT;
    auto load_gu = [&](const Slot& t, float (&g)[GQ][2], float (&u)[GQ][2]) {
        const int n = t.n, pos0 = t.pos0;
#pragma unroll
        for (int q = 0; q < GQ; ++q) {
            // (FUSED: a pass wholly past the slot's routes is not loaded: its values are never
            // used, and the load instructions are what the down half's start waits on)
            if (FUSED && q > 0 && NT * q >= n * NSUB * 4) {
                g[q][0] = u[q][0] = g[q][1] = u[q][1] = 0.0f;
                continue;
            }
            const int e = tid + NT * q < n * NSUB * 4 ? tid + NT * q : n * NSUB * 4 - 1;
            const size_t at = static_cast<size_t>(pos0 + e / (4 * NSUB)) * I + (e / 4 % NSUB) * (4 * NCHUNK) +
                              4 * chunk + (e & 3);
            g[q][0] = load_f32<FUSED>(B.g + at);
            u[q][0] = load_f32<FUSED>(B.u + at);
            g[q][1] = load_f32<FUSED>(B.g + (two ? B.gu_plane : 0) + at);
            u[q][1] = load_f32<FUSED>(B.u + (two ? B.gu_plane : 0) + at);
        }
    };
    // row scales of the output lanes (kh == 0): rows (lane & ~3) + 0..3 of the row group; or
    // the group scales of every lane's rows for its wave's K slice
    auto load_sc = [&](int item, const Slot& t, ItemScales<G8>& sc) {
        const size_t row0 = static_cast<size_t>(t.expert) * H + (item % tiles) * TR + rg * 64;
        if constexpr (G8 == 0) sc.w = *reinterpret_cast<const uint2*>(P.scales + row0 + (lane & ~3));
        else load_group_scales(P.scales, row0, lane, P.ngrp, kh * (32 / G8), sc.g);
    };
    // Items j = idx + j * per_type (j < my_n); loads are unconditional (past the end: the last
    // item again) so the compiler counts them exactly.
    const int my_n = n_items > idx ? (n_items - idx + per_type - 1) / per_type : 0;
    auto item_of = [&](int j) { return my_n > 0 ? idx + (j < my_n ? j : my_n - 1) * per_type : 0; };
    constexpr int PF = D;  // items in flight (all: the item loads are the ones that wait longest)
    uint32_t cw[PF][BITS + 1];
    float gq[PF][GQ][2], uq[PF][GQ][2];
    ItemScales<G8> sc[PF];
    auto load_slot = [&](int j, int k) {
        const int it = item_of(j);
        const Slot t = slot_of(it);
        load_code_block_tiled<BITS>(code_src(it, t), lane, cw[k]);
        load_gu(t, gq[k], uq[k]);
        load_sc(it, t, sc[k]);
    };
#pragma unroll
    for (int k = 0; k < PF; ++k) {
        load_slot(k, k);  // (no items: item 0, unused)
        if (k < 3) Q38_STAMP(16384, 6 + k);
    }
#pragma unroll
    for (int q = 0; q < NFILL; ++q) {
        const int i = tid + q * NT;
        if (NG % NT == 0 || i < NG) reinterpret_cast<u4_t*>(lds)[i] = fv[q];
    }
    Q38_STAMP(16384, 2);

    // 3. Items: the first D as straight-line code over a ring of PF slots (as in k_gu4: item
    //    k's compute, then item k + PF's loads into its slot; results stay in registers),
    //    items past D in a plain loop. Output lanes (kh == 0): weight rows (lane & ~3) +
    //    0..3 of the row group x route lane & 3.
    float* dout = B.d + chunk * B.d_plane;
    auto item_compute = [&](int jj, const uint32_t* cwj, const float (&g2)[GQ][2], const float (&u2)[GQ][2],
                            const ItemScales<G8>& scj, float (&o4)[4], int& oroute, int& obase) {
        const int item = idx + jj * per_type;
        int expert, n, pos0;
        const int ui = item / tiles;
        slot_rows(plan, M, K, L.has_shared, ui, E, &expert, &n, &pos0);
        float gl[GQ][2], ul[GQ][2];
#pragma unroll
        for (int q = 0; q < GQ; ++q)
#pragma unroll
            for (int i = 0; i < 2; ++i) gl[q][i] = g2[q][i], ul[q][i] = u2[q][i];
        if constexpr (FUSED) {
            auto pending = [&] {
                bool p = false;
#pragma unroll
                for (int q = 0; q < GQ; ++q)
                    if (tid + NT * q < n * NSUB * 4)
#pragma unroll
                        for (int i = 0; i < 2; ++i) p |= gu_unset(gl[q][i]) || gu_unset(ul[q][i]);
                return p;
            };
            // (bounded: a value still unset at the limit stays NaN, and so does the output, and
            // the device's wait status records it)
            int spin = 0;
            for (; pending() && spin < B.wait_limit; ++spin) {
                __builtin_amdgcn_s_sleep(2);
                load_gu(Slot{expert, n, pos0}, gl, ul);
            }
            if (pending()) wait_gave_up();
#ifdef Q38_TRACE
            if (jj == 0) {
                Q38_STAMP(16384, 5);
                if (threadIdx.x == 0) g_trace[16384 + 16 * blockIdx.x + 11] = spin;
            }
#endif
        }
#pragma unroll
        for (int q = 0; q < GQ; ++q) {
            const int e = tid + NT * q;
            if (e < n * NSUB * 4) {
                const float g = two ? gl[q][0] + gl[q][1] : gl[q][0];
                const float u = two ? ul[q][0] + ul[q][1] : ul[q][0];
                reinterpret_cast<uint16_t*>(hs)[e] = f2h(swiglu(g, u));
            }
        }
        lds_barrier();  // SwiGLU rows (and, the first time, the codebook chunk) in LDS
        if (jj == 0) Q38_STAMP(16384, 12);
        const int jb = (lane & 3) < n ? (lane & 3) : 0;
        uint2 bop[32];
#pragma unroll
        for (int t = 0; t < 32; t += 2) {
            const uint4 v2 = *reinterpret_cast<const uint4*>(&hs[jb * NSUB + kh * 32 + t]);
            bop[t] = make_uint2(v2.x, v2.y);
            bop[t + 1] = make_uint2(v2.z, v2.w);
        }
        v4f_t acc;
        if constexpr (G8 == 0) acc = slice_mfma<BITS>(cwj, book, bop);
        else acc = slice_mfma_g8<BITS>(cwj, book, bop, scj.g);
        if (jj == 0) Q38_STAMPV(16384, 13, acc[0]);
        if (kh > 0) reinterpret_cast<v4f_t*>(red)[(rg * (KS - 1) + kh - 1) * 64 + lane] = acc;
        lds_barrier();  // (the next item's SwiGLU rows are written after this barrier)
        if (jj == 0) Q38_STAMP(16384, 14);
        oroute = -1;
        if (kh == 0) {
#pragma unroll
            for (int w = 1; w < KS; ++w)
                acc += reinterpret_cast<const v4f_t*>(red)[(rg * (KS - 1) + w - 1) * 64 + lane];
            const int jr = lane & 3;
            if (jr < n) {
                oroute = ui == nu ? MK + jr : plan[2 + 2 * MK + pos0 + jr];
                obase = (item % tiles) * TR + rg * 64 + (lane & ~3);
                if constexpr (G8 == 0) {
                    const uint16_t s4[4] = {static_cast<uint16_t>(scj.w.x), static_cast<uint16_t>(scj.w.x >> 16),
                                            static_cast<uint16_t>(scj.w.y), static_cast<uint16_t>(scj.w.y >> 16)};
#pragma unroll
                    for (int r = 0; r < 4; ++r) o4[r] = h2f(s4[r]) * acc[r];
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r) o4[r] = acc[r];
                }
            }
        }
    };
    float o4[D][4];
    int oroute[D], obase[D];
#pragma unroll
    for (int k = 0; k < D; ++k) {
        oroute[k] = -1;
        if (k < my_n) item_compute(k, cw[k % PF], gq[k % PF], uq[k % PF], sc[k % PF], o4[k], oroute[k], obase[k]);
        if (k + PF < D) load_slot(k + PF, k % PF);
        if (k == 0) Q38_STAMP(16384, 3);
    }
#pragma unroll
    for (int k = 0; k < D; ++k)
        if (oroute[k] >= 0)
#pragma unroll
            for (int r = 0; r < 4; ++r) store_f32<FUSED>(dout + static_cast<size_t>(oroute[k]) * H + obase[k] + r, o4[k][r]);
    for (int jj = D; jj < my_n; ++jj) {
        const int it = item_of(jj);
        uint32_t c1[BITS + 1];
        float g1[GQ][2], u1[GQ][2];
        ItemScales<G8> s1;
        const Slot t = slot_of(it);
        load_code_block_tiled<BITS>(code_src(it, t), lane, c1);
        load_gu(t, g1, u1);
        load_sc(it, t, s1);
        float p4[4];
        int rt, bs;
        item_compute(jj, c1, g1, u1, s1, p4, rt, bs);
        if (rt >= 0)
#pragma unroll
            for (int r = 0; r < 4; ++r) store_f32<FUSED>(dout + static_cast<size_t>(rt) * H + bs + r, p4[r]);
    }
    Q38_STAMP(16384, 4);
#ifdef Q38_TRACE
    if (threadIdx.x == 0) g_trace[16384 + 16 * blockIdx.x + 10] = my_n;
#endif
}

template <int BITS, int NSUB, int NCHUNK, int D, int G8 = 0>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(1, 2))) void k_dn4(LayerDev L, MoeBufs B, int M) {
    extern __shared__ __align__(16) unsigned char lds[];
    __shared__ int32_t plan[kNarrowPlan];
    __shared__ __align__(16) uint2 hs[kNarrow * NSUB];
    touch_kernargs<sizeof(LayerDev) + sizeof(MoeBufs) + sizeof(int)>();
    dn4_body<BITS, NSUB, NCHUNK, D, G8, false>(L, B, M, lds, plan, hs, nullptr);
}

// Gate/up and down of a verify layer in one launch (d8/14-bit, H 2048, I 512, top-10,
// per-row scales), optionally with the combine. Every workgroup first runs the gate/up half
// of k_gu4 (routing, plan, its gate/up items), then replaces its LDS codebook chunk with a
// down chunk (requested during its gate/up items) and runs the down half of k_dn4: the down
// kernel's launch, plan read and first loads are gone from the layer's latency chain. With
// h or out set, the last kCombineWgs workgroups (those with the fewest down items) then form
// the layer output: y = combine of the rows' routes and the shared expert (combine_value,
// the combine kernel's arithmetic); h <- T(h + y) in place, or out <- y.
// Values cross workgroups (and XCDs) inside the launch: the gate/up and down partial sums
// are stored with agent-scope atomic stores and read with agent-scope atomic loads, both
// coherent at the device's memory side, so no L2 write-back is needed. The router kernel
// before this one sets every value of those planes to the all-ones pattern (a NaN that no
// arithmetic produces), and a reader re-reads the values it needs until none holds it. The
// wait is bounded (kWaitLimit re-reads, ~0.1 s): every workgroup of the grid is resident at
// once (one per CU, grid <= CUs, checked against the kernel's occupancy before it is chosen),
// so it ends long before that unless the device is shared with other work or something is
// broken; then the affected outputs are NaN instead of the kernel hanging, and the device's
// wait status records it for the API to report (q38_ctx_synchronize).
constexpr int kCombineWgs = 32;
// HC > 0: h is the rows' HyperConnection streams ([M][HC][H]) and the output goes into every
// stream as k_combine_hc writes it, T(stream + T(y * inj[r][s])), instead of h <- T(h + y).
template <int KT>
__device__ __forceinline__ void combine_tail(const LayerDev& L, const MoeBufs& B, int M, const float* wt, uint16_t* h,
                                             uint16_t* out, const uint16_t* inj, int HC) {
    const int w = static_cast<int>(blockIdx.x) - static_cast<int>(gridDim.x - kCombineWgs);
    Q38_STAMP(24576, 0);
    const int H = L.H, MK = M * KT;
    const int per = (M * H + kCombineWgs - 1) / kCombineWgs;  // (<= 512: M <= 4, H = 2048)
    const int p = w * per + static_cast<int>(threadIdx.x);
    if (w < 0 || static_cast<int>(threadIdx.x) >= per || p >= M * H) return;
    const int r = p / H, o = p % H;
    CombineIn<KT, true> in;
#pragma unroll
    for (int s = 0; s < KT; ++s) in.wts[s] = wt[r * KT + s];
    in.wts[KT] = B.sgate[r];
    const uint16_t hraw = HC > 0 ? 0 : (h ? h : out)[static_cast<size_t>(r) * H + o];  // (unused without h)
    uint16_t sv[kHcMaxStreams], gv[kHcMaxStreams];
    const size_t srow = (static_cast<size_t>(r) * HC) * H + o;
    if (HC > 0) {
#pragma unroll
        for (int s = 0; s < kHcMaxStreams; ++s)
            if (s < HC) {
                sv[s] = h[srow + static_cast<size_t>(s) * H];
                gv[s] = inj[r * HC + s];
            }
    }
    auto load = [&] {
#pragma unroll
        for (int s = 0; s <= KT; ++s) {
            const int route = s < KT ? r * KT + s : (L.has_shared ? MK + r : r * KT);
            const size_t at = static_cast<size_t>(route) * H + o;
            in.dv[s][0] = load_f32<true>(B.d + at);
            in.dv[s][1] = load_f32<true>(B.d + B.d_plane + at);
        }
    };
    auto pending = [&] {
        bool q = false;
#pragma unroll
        for (int s = 0; s <= KT; ++s) q |= gu_unset(in.dv[s][0]) || gu_unset(in.dv[s][1]);
        return q;
    };
    load();
    Q38_STAMPV(24576, 1, in.dv[0][0]);
    for (int spin = 0; pending() && spin < B.wait_limit; ++spin) {
        __builtin_amdgcn_s_sleep(2);
        load();
    }
    if (pending()) wait_gave_up();
    Q38_STAMPV(24576, 2, in.dv[0][0]);
    const float y = combine_value<KT, true>(L, in);
    const size_t i = static_cast<size_t>(r) * H + o;
    if (HC > 0) {
#pragma unroll
        for (int s = 0; s < kHcMaxStreams; ++s)
            if (s < HC) h[srow + static_cast<size_t>(s) * H] = f2bf(bf2f(sv[s]) + rbf(y * bf2f(gv[s])));
    } else if (h) {
        h[i] = f2bf(rbf(bf2f(hraw) + y));
    } else {
        out[i] = f2bf(y);
    }
    Q38_STAMP(24576, 3);
}

// G8: per-row scales (0) or one scale per 64 inputs in both projections (8, the checkpoint
// layout; the two kernels' G8 = 8 item code).
template <int BITS, int NSUB_GU, int NSUB_DN, int NCHUNK, int DG, int DD, int KT, int G8 = 0>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(1, 2))) void k_gd4(LayerDev L, MoeBufs B, int M,
                                                                                         uint16_t* h, uint16_t* out,
                                                                                         const uint16_t* inj, int HC) {
    static_assert(2 * NSUB_GU == 512, "the gate/up half uses the 8 waves of the down half");
    extern __shared__ __align__(16) unsigned char lds[];
    __shared__ int32_t ex[kNarrowMaxRoutes];
    __shared__ float wt[kNarrowMaxRoutes];
    __shared__ int32_t plan[kNarrowPlan];
    __shared__ int32_t slot_pos[(kNarrowMaxRoutes + 1) * 4];
    __shared__ __align__(16) uint2 hs[kNarrow * NSUB_DN];
    touch_kernargs<sizeof(LayerDev) + sizeof(MoeBufs) + 2 * sizeof(int) + 3 * sizeof(void*)>();
    u4_t fill[(1 << BITS) / 2 / 512];  // the down codebook chunk, requested by the gate/up half
    gu4_body<BITS, NSUB_GU, NCHUNK, DG, G8, true>(L, B, M, lds, ex, plan, slot_pos, fill, wt);
    lds_barrier();  // every wave is done with the gate/up codebook chunk
    dn4_body<BITS, NSUB_DN, NCHUNK, DD, G8, true>(L, B, M, lds, plan, hs, fill);
    if (h || out) combine_tail<KT>(L, B, M, wt, h, out, inj, HC);
    Q38_STAMP(24576, 4);
}

template <int BITS, int NSUB, int NCHUNK, int D, int G8 = 0>
hipError_t launch_gu4_t(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st) {
    constexpr size_t lds = gu4_lds_bytes<BITS, NSUB, NCHUNK>();
    if (const hipError_t e = ensure_lds<k_gu4<BITS, NSUB, NCHUNK, D, G8>>(lds); e != hipSuccess) return e;
    return launch(k_gu4<BITS, NSUB, NCHUNK, D, G8>, dim3(mfma_grid()), dim3(2 * NSUB), lds, st, L, B, M);
}
template <int DG, int DD, int G8>
hipError_t launch_gd4_t(const LayerDev& L, const MoeBufs& B, int M, uint16_t* h, uint16_t* out, hipStream_t st,
                        const uint16_t* inj, int HC) {
    constexpr size_t lds = gu4_lds_bytes<14, 256, 2>();
    static_assert(lds >= (size_t{1} << 14) * 8 + 4 * 64 * 16, "the down half's LDS fits the gate/up half's");
    if (const hipError_t e = ensure_lds<k_gd4<14, 256, 64, 2, DG, DD, 10, G8>>(lds); e != hipSuccess) return e;
    return launch(k_gd4<14, 256, 64, 2, DG, DD, 10, G8>, dim3(mfma_grid()), dim3(512), lds, st, L, B, M, h, out, inj,
                  HC);
}
template <int BITS, int NSUB, int NCHUNK, int D, int G8 = 0>
hipError_t launch_dn4_t(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st) {
    constexpr int KS = NSUB / 32, RG = 8 / KS;
    constexpr size_t lds = (size_t{1} << BITS) * 8 + static_cast<size_t>(RG) * (KS - 1) * 64 * 16;
    if (const hipError_t e = ensure_lds<k_dn4<BITS, NSUB, NCHUNK, D, G8>>(lds); e != hipSuccess) return e;
    return launch(k_dn4<BITS, NSUB, NCHUNK, D, G8>, dim3(mfma_grid()), dim3(512), lds, st, L, B, M);
}

// Scales the four-row kernels take: one per output row, or one per 64 inputs for the d8
// gate/up projections of H / 8 = 256 subvectors and the d8 down projection (the layout of the
// reference's checkpoints, src/sparse_moe.cpp:641-647).
bool gu_groups64(const LayerDev& L) {
    return L.p[0].dim == 8 && L.H / 8 == 256 && L.p[0].ngrp == L.H / 64 && L.p[1].ngrp == L.H / 64;
}
bool dn_groups64(const LayerDev& L) { return L.p[2].dim == 8 && L.p[2].ngrp == L.I / 64; }
} // namespace

bool moe_uses_narrow(const LayerDev& L, int M) {
    if (M < 1 || M > kNarrow || L.E != 512 || L.mixed) return false;
    if (M * L.K > 64) return false;  // the plan is built by one wave
    // the MFMA layers' geometry (moe_uses_mfma), with per-64-input scale groups allowed
    const bool rows = L.p[0].ngrp == 1 && L.p[1].ngrp == 1 && L.p[2].ngrp == 1;
    if (rows ? !moe_uses_mfma(L) : !(moe_uses_mfma_geometry(L) && (L.p[0].ngrp == 1 ? L.p[1].ngrp == 1 : gu_groups64(L)) &&
                                     (L.p[2].ngrp == 1 || dn_groups64(L))))
        return false;
    const int gn = L.H / L.p[0].dim, dn = L.I / L.p[2].dim;
    const bool gu = (L.p[0].dim == 8 && (gn == 256 || gn == 320)) || (L.p[0].dim == 4 && gn == 512);
    const bool dw = (L.p[2].dim == 8 && dn == 64) || (L.p[2].dim == 4 && dn == 128);
    return gu && dw && L.I % 64 == 0 && L.H % 256 == 0;
}

LayerDev moe_call_dev(const LayerDev& L, int M) {
    LayerDev d = L;
    d.u8_call = 0;
    if (moe_u8_call(L, M)) {  // the U8 kernels: one plane each, no one-launch layer
        d.u8_call = 1;
        d.gu_parts = d.d_parts = 1;
        d.fused_mode = 2;
        return d;
    }
    if (moe_uses_narrow(L, M)) {
        d.gu_parts = L.p[0].dim / 4;
        d.d_parts = L.p[2].dim / 4;
    }
    d.fused_mode = 0;
    d.fused_mode = moe_uses_fused(d, M) ? 1 : 2;
    return d;
}

// Ring depth: the most items one workgroup can get (every route on its own expert, plus the
// shared expert), so that the item loads are all in flight before the first item; deeper
// rings cost registers (8 waves: 256 VGPRs a wave; 10 or 16 waves: fewer), so they stop at
// 6 (4 for the wider workgroups) and further items take the loop.
static int ring_items(const LayerDev& L, int M, int tiles, int per_type) {
    return ((M * L.K + 1) * tiles + per_type - 1) / per_type;
}

namespace {
std::atomic<int> g_fused_enabled{1};
std::atomic<int> g_wait_limit{kWaitLimit};

// Occupancy of one k_gd4 instantiation: at least one workgroup of 512 threads with its LDS
// per CU, and the planned grid no larger than the CUs that many workgroups cover.
template <int DG, int DD, int G8>
bool gd4_fits(int cus) {
    constexpr size_t lds = gu4_lds_bytes<14, 256, 2>();
    auto kern = k_gd4<14, 256, 64, 2, DG, DD, 10, G8>;
    if (ensure_lds<k_gd4<14, 256, 64, 2, DG, DD, 10, G8>>(lds) != hipSuccess) return false;
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, reinterpret_cast<const void*>(kern), 512, lds) != hipSuccess)
        return false;
    return nb >= 1 && static_cast<int64_t>(mfma_grid()) <= static_cast<int64_t>(cus) * nb;
}

// Whether every k_gd4 instantiation fits the current device as planned (once per device).
bool fused_resident() {
    static std::atomic<uint64_t> checked{0}, ok{0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return false;
    const uint64_t bit = uint64_t{1} << (dev & 63);
    if (checked.load(std::memory_order_acquire) & bit) return (ok.load(std::memory_order_acquire) & bit) != 0;
    int cus = 0;
    bool fits = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cus > 0;
    fits = fits && gd4_fits<2, 1, 0>(cus) && gd4_fits<3, 2, 0>(cus) && gd4_fits<4, 2, 0>(cus) &&
           gd4_fits<6, 3, 0>(cus) && gd4_fits<2, 1, 8>(cus) && gd4_fits<3, 2, 8>(cus) && gd4_fits<4, 2, 8>(cus) &&
           gd4_fits<6, 3, 8>(cus);
    (void)hipGetLastError();  // (a failed query leaves no error behind for the next launch)
    if (fits) ok.fetch_or(bit, std::memory_order_acq_rel);
    checked.fetch_or(bit, std::memory_order_acq_rel);
    return fits;
}
} // namespace

void set_fused_enabled(bool on) { g_fused_enabled.store(on ? 1 : 0, std::memory_order_relaxed); }
void set_wait_limit(int spins) { g_wait_limit.store(spins < 0 ? kWaitLimit : spins, std::memory_order_relaxed); }
int wait_limit() { return g_wait_limit.load(std::memory_order_relaxed); }
hipError_t read_wait_status(uint32_t* status, bool clear) {
    hipError_t e = hipMemcpyFromSymbol(status, HIP_SYMBOL(g_wait_status), sizeof(uint32_t), 0, hipMemcpyDeviceToHost);
    if (e == hipSuccess && clear && *status != 0) {
        const uint32_t zero = 0;
        e = hipMemcpyToSymbol(HIP_SYMBOL(g_wait_status), &zero, sizeof(uint32_t), 0, hipMemcpyHostToDevice);
    }
    return e;
}

bool moe_uses_fused(const LayerDev& L, int M) {
    if (L.fused_mode != 0) return L.fused_mode == 1;
    if (!g_fused_enabled.load(std::memory_order_relaxed)) return false;
    if (!moe_uses_narrow(L, M)) return false;
    // per-row scales everywhere, or per-64-input groups in both projections
    const bool rows = L.p[0].ngrp == 1 && L.p[1].ngrp == 1 && L.p[2].ngrp == 1;
    if (!rows && !(gu_groups64(L) && dn_groups64(L))) return false;
    for (int p = 0; p < 3; ++p)
        if (L.p[p].dim != 8 || L.p[p].bits != 14 || !L.p[p].codes_t) return false;
    return L.H == 2048 && L.I == 512 && L.K == 10 && mfma_grid() >= kCombineWgs && fused_resident();
}

// Ring depths of the two halves (as the two kernels pick them: every item's loads in flight
// at once where registers allow; items beyond take the loop).
hipError_t launch_gate_down4(const LayerDev& L, const MoeBufs& B, int M, uint16_t* h, uint16_t* out, hipStream_t st,
                             const uint16_t* inj, int HC) {
    if (!moe_uses_fused(L, M)) return hipErrorInvalidValue;
    if (HC < 0 || HC > kHcMaxStreams || (HC > 0 && (!h || !inj || out))) return hipErrorInvalidValue;
    const int grid = mfma_grid();
    const int c = ring_items(L, M, L.I / 64, grid / 32 * 8);
    if (L.p[0].ngrp != 1) {  // 64-input scale groups
        if (c <= 2) return launch_gd4_t<2, 1, 8>(L, B, M, h, out, st, inj, HC);
        if (c <= 3) return launch_gd4_t<3, 2, 8>(L, B, M, h, out, st, inj, HC);
        if (c <= 4) return launch_gd4_t<4, 2, 8>(L, B, M, h, out, st, inj, HC);
        return launch_gd4_t<6, 3, 8>(L, B, M, h, out, st, inj, HC);
    }
    if (c <= 2) return launch_gd4_t<2, 1, 0>(L, B, M, h, out, st, inj, HC);
    if (c <= 3) return launch_gd4_t<3, 2, 0>(L, B, M, h, out, st, inj, HC);
    if (c <= 4) return launch_gd4_t<4, 2, 0>(L, B, M, h, out, st, inj, HC);
    return launch_gd4_t<6, 3, 0>(L, B, M, h, out, st, inj, HC);
}

hipError_t launch_gate_up4(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st) {
    const int nsub = L.H / L.p[0].dim;
    if (!L.p[0].codes_t || !L.p[1].codes_t) return hipErrorInvalidValue;
    const int grid = mfma_grid();
    if (L.p[0].dim == 8 && nsub == 256 && gu_groups64(L)) {
        const int c = ring_items(L, M, L.I / 64, grid / 32 * 8);
        if (c <= 2) return launch_gu4_t<14, 256, 2, 2, 8>(L, B, M, st);
        if (c <= 3) return launch_gu4_t<14, 256, 2, 3, 8>(L, B, M, st);
        if (c <= 4) return launch_gu4_t<14, 256, 2, 4, 8>(L, B, M, st);
        return launch_gu4_t<14, 256, 2, 6, 8>(L, B, M, st);
    }
    if (L.p[0].ngrp != 1 || L.p[1].ngrp != 1) return hipErrorInvalidValue;
    if (L.p[0].dim == 8 && nsub == 256) {
        const int c = ring_items(L, M, L.I / 64, grid / 32 * 8);
        if (c <= 2) return launch_gu4_t<14, 256, 2, 2>(L, B, M, st);
        if (c <= 3) return launch_gu4_t<14, 256, 2, 3>(L, B, M, st);
        if (c <= 4) return launch_gu4_t<14, 256, 2, 4>(L, B, M, st);
        return launch_gu4_t<14, 256, 2, 6>(L, B, M, st);
    }
    if (L.p[0].dim == 8 && nsub == 320) {
        const int c = ring_items(L, M, L.I / 64, grid / 32 * 8);
        if (c <= 2) return launch_gu4_t<14, 320, 2, 2>(L, B, M, st);
        return launch_gu4_t<14, 320, 2, 4>(L, B, M, st);
    }
    if (L.p[0].dim == 4 && nsub == 512) {
        const int c = ring_items(L, M, L.I / 64, grid / 16 * 8);
        if (c <= 2) return launch_gu4_t<8, 512, 1, 2>(L, B, M, st);
        return launch_gu4_t<8, 512, 1, 4>(L, B, M, st);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_down4(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st) {
    const int nsub = L.I / L.p[2].dim;
    if (!L.p[2].codes_t) return hipErrorInvalidValue;
    const int grid = mfma_grid();
    if (L.p[2].dim == 8 && nsub == 64 && dn_groups64(L)) {
        const int c = ring_items(L, M, L.H / 256, grid / 16 * 8);
        if (c <= 1) return launch_dn4_t<14, 64, 2, 1, 8>(L, B, M, st);
        if (c <= 2) return launch_dn4_t<14, 64, 2, 2, 8>(L, B, M, st);
        return launch_dn4_t<14, 64, 2, 3, 8>(L, B, M, st);
    }
    if (L.p[2].ngrp != 1) return hipErrorInvalidValue;
    if (L.p[2].dim == 8 && nsub == 64) {
        const int c = ring_items(L, M, L.H / 256, grid / 16 * 8);
        if (c <= 1) return launch_dn4_t<14, 64, 2, 1>(L, B, M, st);
        if (c <= 2) return launch_dn4_t<14, 64, 2, 2>(L, B, M, st);
        return launch_dn4_t<14, 64, 2, 3>(L, B, M, st);
    }
    if (L.p[2].dim == 4 && nsub == 128) {
        const int c = ring_items(L, M, L.H / 128, grid / 8 * 8);
        if (c <= 1) return launch_dn4_t<8, 128, 1, 1>(L, B, M, st);
        if (c <= 2) return launch_dn4_t<8, 128, 1, 2>(L, B, M, st);
        return launch_dn4_t<8, 128, 1, 3>(L, B, M, st);
    }
    return hipErrorInvalidValue;
}

#ifdef Q38_TRACE
// The phase stamps of this code object (Q38_STAMP in q38_moe_dev.hpp) and their reader.
__device__ unsigned long long g_trace[32768];
#endif
} // namespace q38

#ifdef Q38_TRACE
extern "C" int q38_trace_read(unsigned long long* out) {
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(q38::g_trace), sizeof(unsigned long long) * 32768) == hipSuccess ? 0 : -1;
}
#endif
