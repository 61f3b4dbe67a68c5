// q38_moe_dev.hpp — device routines shared by the MoE kernels: DPP wave reductions, the
// top-k routing + gather-by-expert plan (R2, R3), the plan accessors, codebook fills and
// the SwiGLU rounding contract.
#pragma once

#include "q38_device.hpp"
#include "q38_internal.hpp"

// Phase stamps for timing a kernel from the inside: with Q38_TRACE defined (the separate
// build of the Makefile's trace target, read by trace/phases.py), thread 0 of each workgroup records the 100 MHz real-time
// counter at a numbered point into q38::g_trace[base + 16 * workgroup + i]; Q38_STAMPV
// first waits for value v. Without Q38_TRACE they compile to nothing.
#ifdef Q38_TRACE
namespace q38 {
extern __device__ unsigned long long g_trace[32768];
}
#define Q38_STAMP(base, i)                                                                                    \
    do {                                                                                                      \
        if (threadIdx.x == 0)                                                                                 \
            ::q38::g_trace[(base) + 16 * (blockIdx.y * gridDim.x + blockIdx.x) + (i)] =                       \
                __builtin_amdgcn_s_memrealtime();                                                             \
    } while (0)
#define Q38_STAMPV(base, i, v)          \
    do {                                \
        asm volatile("" ::"v"(v));      \
        Q38_STAMP(base, i);             \
    } while (0)
#define Q38_STAMP_T(base, i, t)                                                                               \
    do {                                                                                                      \
        if (static_cast<int>(threadIdx.x) == (t))                                                             \
            ::q38::g_trace[(base) + 16 * (blockIdx.y * gridDim.x + blockIdx.x) + (i)] =                       \
                __builtin_amdgcn_s_memrealtime();                                                             \
    } while (0)
#else
#define Q38_STAMP_T(base, i, t) \
    do {                        \
    } while (0)
#define Q38_STAMP(base, i) \
    do {                   \
    } while (0)
#define Q38_STAMPV(base, i, v) \
    do {                       \
    } while (0)
#endif

namespace q38 {

constexpr int kNarrowMaxRoutes = 64;  // routes of the one-wave plan (4 rows x 16)
constexpr int kPlanInts = 2 + 4 * kMaxRows * kMaxTopK;

// ============================================================== DPP wave reductions
// Order-independent reductions (max) use DPP row operations and readlane; the summations
// whose order is part of a contract keep the xor butterfly of q38_device.hpp.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp32(uint32_t v) {
    return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(static_cast<int>(v), static_cast<int>(v), CTRL, 0xF,
                                                             0xF, false));
}
template <int CTRL>
__device__ __forceinline__ uint64_t max_step_u64(uint64_t k) {
    const uint32_t h = dpp32<CTRL>(static_cast<uint32_t>(k >> 32));
    const uint32_t l = dpp32<CTRL>(static_cast<uint32_t>(k));
    const uint64_t o = (static_cast<uint64_t>(h) << 32) | l;
    return o > k ? o : k;
}
__device__ __forceinline__ uint64_t readlane_u64(uint64_t k, int lane) {
    const uint32_t h = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(k >> 32), lane));
    const uint32_t l = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(k), lane));
    return (static_cast<uint64_t>(h) << 32) | l;
}
// quad_perm(1,0,3,2), quad_perm(2,3,0,1), row_half_mirror, row_mirror, then rows via readlane.
__device__ __forceinline__ uint64_t wave_max_u64_dpp(uint64_t k) {
    k = max_step_u64<0xB1>(k);
    k = max_step_u64<0x4E>(k);
    k = max_step_u64<0x141>(k);
    k = max_step_u64<0x140>(k);
    uint64_t m = readlane_u64(k, 0);
    const uint64_t a = readlane_u64(k, 16), b = readlane_u64(k, 32), c = readlane_u64(k, 48);
    m = a > m ? a : m;
    m = b > m ? b : m;
    m = c > m ? c : m;
    return m;
}
__device__ __forceinline__ uint32_t wave_max_u32_dpp(uint32_t v) {
    auto step = [](uint32_t x, uint32_t o) { return x > o ? x : o; };
    v = step(v, dpp32<0xB1>(v));
    v = step(v, dpp32<0x4E>(v));
    v = step(v, dpp32<0x141>(v));
    v = step(v, dpp32<0x140>(v));
    uint32_t m = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 0));
    const uint32_t a = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 16));
    const uint32_t b = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 32));
    const uint32_t c = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 48));
    m = a > m ? a : m;
    m = b > m ? b : m;
    m = c > m ? c : m;
    return m;
}
__device__ __forceinline__ float wave_max_dpp(float v) {
    auto step = [](float x, uint32_t o) { return fmaxf(x, __uint_as_float(o)); };
    v = step(v, dpp32<0xB1>(__float_as_uint(v)));
    v = step(v, dpp32<0x4E>(__float_as_uint(v)));
    v = step(v, dpp32<0x141>(__float_as_uint(v)));
    v = step(v, dpp32<0x140>(__float_as_uint(v)));
    float m = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16)));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32)));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48)));
    return m;
}

// ============================================================== top-k + plan (R2, R3)
// Block-level routine (any block of >= 256 threads). Wave w takes rows w, w + waves, ...:
// lane l owns experts 64j + l as (p bits << 32 | ~index) keys; K rounds of a DPP wave max
// pick (p desc, index asc). The plan is built by counting: route i lands at
// #{routes (e, i') < (e_i, i)}; expert groups are marked with a ballot. The plan is left
// in `plan` (LDS or global); `global_out` also receives experts and weights.
struct TopkLds {
    int32_t ex[kMaxRows * kMaxTopK];
    int32_t sorted_e[kMaxRows * kMaxTopK];
    int32_t wave_cnt[16];
};

// Logits of request row r, lane l holding experts 64j + l (j < NJ; E = 64 NJ when EXACT).
template <int NJ, bool EXACT>
__device__ __forceinline__ void topk_load_row_t(const LayerDev& L, const MoeBufs& B, int r, float* lg) {
    const int lane = threadIdx.x & 63;
    const int E = EXACT ? 64 * NJ : L.E, nj = E / 64;
#pragma unroll
    for (int j = 0; j < NJ; ++j) lg[j] = EXACT || j < nj ? B.logits[r * E + 64 * j + lane] : -INFINITY;
}
__device__ __forceinline__ void topk_load_row(const LayerDev& L, const MoeBufs& B, int r, float* lg) {
    topk_load_row_t<16, false>(L, B, r, lg);
}

// Softmax (exp contract, double denominator) of one row by one wave, for E <= 64 * NJ
// experts (lane l: experts 64j + l): keys (p bits << 32 | ~index), unique, ordered as (p
// desc, index asc); experts past E get key 0.
template <int NJ, bool EXACT>
__device__ __forceinline__ void topk_keys_t(const LayerDev& L, const float* lg, uint64_t* key) {
    const int lane = threadIdx.x & 63;
    const int nj = EXACT ? NJ : L.E / 64;
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < NJ; ++j) mx = fmaxf(mx, lg[j]);
    mx = wave_max_dpp(mx);
    double ds = 0.0;
    float ev[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        ev[j] = 0.0f;
        if (EXACT || j < nj) {
            ev[j] = exp_contract(lg[j] - mx);
            ds += static_cast<double>(ev[j]);
        }
    }
    ds = wave_sum_xor(ds);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        key[j] = 0;
        if (EXACT || j < nj) {
            const float p = static_cast<float>(static_cast<double>(ev[j]) / ds);
            key[j] = (static_cast<uint64_t>(__float_as_uint(p)) << 32) |
                     static_cast<uint64_t>(0xFFFFFFFFu - static_cast<uint32_t>(64 * j + lane));
        }
    }
}

// Rank-ordered outputs of one row: lane s < K holds the s-th key (weight p / sum of the
// selected p in rank order when normalising).
// wt_lds (optional): the row's route weights in LDS beside ex_lds.
__device__ __forceinline__ void topk_write_row(const LayerDev& L, const MoeBufs& B, int r, int32_t* ex_lds,
                                               bool global_out, float psel, int isel, float sum,
                                               float* wt_lds = nullptr) {
    const int lane = threadIdx.x & 63;
    const int K = L.K;
    if (lane < K) {
        if (ex_lds) ex_lds[r * K + lane] = isel;
        if (wt_lds) wt_lds[r * K + lane] = L.normalize ? psel / sum : psel;
        if (global_out) {
            B.experts[r * K + lane] = isel;
            B.weights[r * K + lane] = L.normalize ? psel / sum : psel;
        }
    }
}

// Top-k by tournament: each lane sorts its NJ keys (bitonic network), then K rounds take the
// DPP wave maximum of the lane heads and the winning lane advances its list, which yields the
// keys in (p desc, index asc) order. key[] is consumed.
template <int NJ>
__device__ __forceinline__ void topk_tournament(const LayerDev& L, const MoeBufs& B, int r, uint64_t* key,
                                                int32_t* ex_lds, bool global_out, float* wt_lds = nullptr) {
    const int lane = threadIdx.x & 63;
    const int K = L.K;
#pragma unroll
    for (int k = 2; k <= NJ; k <<= 1) {
#pragma unroll
        for (int h = k >> 1; h > 0; h >>= 1) {
#pragma unroll
            for (int i = 0; i < NJ; ++i) {
                const int m = i ^ h;
                if (m > i) {
                    const uint64_t x = key[i], y = key[m];
                    const bool sw = (i & k) == 0 ? x < y : x > y;  // descending overall
                    key[i] = sw ? y : x;
                    key[m] = sw ? x : y;
                }
            }
        }
    }
    // A round reduces the p word of the lane heads; the lanes holding the maximum are
    // balloted and, only when several tie, the index word breaks the tie (largest ~index).
    float psel = 0.0f, sum = 0.0f;
    int isel = 0;
    for (int s = 0; s < K; ++s) {
        const uint32_t hi = static_cast<uint32_t>(key[0] >> 32), lo = static_cast<uint32_t>(key[0]);
        const uint32_t mhi = wave_max_u32_dpp(hi);
        uint64_t tie = __ballot(hi == mhi);
        if (__popcll(tie) > 1) {
            const uint32_t mlo = wave_max_u32_dpp(hi == mhi ? lo : 0u);
            tie = __ballot(hi == mhi && lo == mlo);
        }
        const int win = __ffsll(static_cast<long long>(tie)) - 1;
        const uint32_t wlo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(lo), win));
        if (lane == win) {
#pragma unroll
            for (int i = 0; i + 1 < NJ; ++i) key[i] = key[i + 1];
            key[NJ - 1] = 0;
        }
        const float p = __uint_as_float(mhi);
        sum += p;
        if (lane == s) {
            psel = p;
            isel = static_cast<int>(0xFFFFFFFFu - wlo);
        }
    }
    topk_write_row(L, B, r, ex_lds, global_out, psel, isel, sum, wt_lds);
}

template <int NJ, bool EXACT>
__device__ __forceinline__ void topk_select_row_t(const LayerDev& L, const MoeBufs& B, int r, const float* lg,
                                                  int32_t* ex_lds, bool global_out) {
    uint64_t key[NJ];
    topk_keys_t<NJ, EXACT>(L, lg, key);
    topk_tournament<NJ>(L, B, r, key, ex_lds, global_out);
}

// The same top-k (E = 512, K <= 64) with a short dependent chain, by counting instead of
// sorting the keys. T = the K-th largest p word among the 64 lane maxima is a lower bound of
// the K-th largest key's p word (the K largest lane maxima are K distinct keys); so is T
// with its low bits cleared, which a bitwise search with ballot counts finds. The keys whose
// p word is >= that bound, typically a few more than K, are compacted into cand; each
// candidate's rank is the number of larger candidates (keys are unique) and a lane permute
// sends it to lane rank, so lanes 0..K-1 hold the top K in (p desc, index asc) order. More
// than 64 candidates (many equal p words) take the tournament. The selection and the
// rank-order weight sum equal topk_select_row_t's bit for bit. cand: 64 u64 of this wave's
// LDS.
template <int NJ>
__device__ __forceinline__ void topk_select_row_fast(const LayerDev& L, const MoeBufs& B, int r, const float* lg,
                                                     int32_t* ex_lds, bool global_out, uint64_t* cand,
                                                     float* wt_lds = nullptr) {
    const int lane = threadIdx.x & 63;
    const int K = L.K;
    uint64_t key[NJ];
    topk_keys_t<NJ, true>(L, lg, key);
    Q38_STAMPV(8192, 11, static_cast<uint32_t>(key[0]));
    uint64_t lm = key[0];
#pragma unroll
    for (int j = 1; j < NJ; ++j) lm = key[j] > lm ? key[j] : lm;
    const uint32_t mh = static_cast<uint32_t>(lm >> 32);
    // p words are those of floats in [0, 1]: below 2^30. Bits 29..17 only: T is then
    // within ~1/32 of the K-th lane maximum, and the chain is 13 ballots.
    uint32_t t = 0;
#pragma unroll
    for (int b = 29; b >= 17; --b) {
        const uint32_t c = t | (1u << b);
        if (__popcll(__ballot(mh >= c)) >= K) t = c;
    }
    Q38_STAMPV(8192, 12, t);
    const uint64_t lt = (1ull << lane) - 1ull;
    int total = 0;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const bool in = static_cast<uint32_t>(key[j] >> 32) >= t;
        const uint64_t bj = __ballot(in);
        const int at = total + __popcll(bj & lt);
        if (in && at < 64) cand[at] = key[j];
        total += __popcll(bj);
    }
    if (total > 64) {
        topk_tournament<NJ>(L, B, r, key, ex_lds, global_out, wt_lds);
        return;
    }
    // zero keys pad the list to a multiple of 16 (a zero key is below every real one); a
    // wave's LDS operations complete in order, so the reads below see every write
    const int total16 = (total + 15) & ~15;
    if (lane >= total && lane < total16) cand[lane] = 0;
    const uint64_t mine = lane < total ? cand[lane] : 0ull;
    int rank = 0;
    for (int i = 0; i < total16; i += 16) {
        ulonglong2 c[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) c[q] = *reinterpret_cast<const ulonglong2*>(cand + i + 2 * q);
#pragma unroll
        for (int q = 0; q < 8; ++q) rank += (c[q].x > mine) + (c[q].y > mine);
    }
    // candidates go to lane rank, the other lanes keep their own slot (a bijection)
    const int dst = (lane < total ? rank : lane) * 4;
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_ds_permute(dst, static_cast<int>(mine >> 32)));
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_ds_permute(dst, static_cast<int>(mine)));
    Q38_STAMPV(8192, 13, hi);
    float sum = 0.0f;
    for (int s = 0; s < K; ++s) sum += __uint_as_float(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(hi), s)));
    topk_write_row(L, B, r, ex_lds, global_out, __uint_as_float(hi), static_cast<int>(0xFFFFFFFFu - lo), sum,
                   wt_lds);
}
__device__ __forceinline__ void topk_select_row(const LayerDev& L, const MoeBufs& B, int r, const float* lg,
                                                int32_t* ex_lds, bool global_out) {
    if (L.E <= 512) topk_select_row_t<8, false>(L, B, r, lg, ex_lds, global_out);
    else topk_select_row_t<16, false>(L, B, r, lg, ex_lds, global_out);
}

// Gather-by-expert plan from t.ex (all rows selected); every thread of the block calls it.
__device__ __forceinline__ void topk_build_plan(int M, int K, int32_t* plan, TopkLds& t) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int waves = blockDim.x >> 6;
    const int MK = M * K;
    lds_barrier();
    if (tid < MK) {
        const int my_e = t.ex[tid];
        const int my_key = (my_e << 8) | tid;
        int pos = 0;
        for (int j = 0; j < MK; ++j) pos += ((t.ex[j] << 8) | j) < my_key;
        t.sorted_e[pos] = my_e;
        plan[2 + 2 * MK + pos] = tid;   // route_list
        plan[2 + 3 * MK + tid] = pos;   // route_pos
    }
    lds_barrier();
    const bool start = tid < MK && (tid == 0 || t.sorted_e[tid - 1] != t.sorted_e[tid]);
    const uint64_t bal = __ballot(start);
    if (lane == 0) t.wave_cnt[wave] = __popcll(bal);
    lds_barrier();
    int rank = __popcll(bal & ((1ull << lane) - 1ull));
    for (int w = 0; w < wave; ++w) rank += t.wave_cnt[w];
    int nu = 0;
    for (int w = 0; w < waves; ++w) nu += t.wave_cnt[w];
    if (start) {
        plan[1 + rank] = t.sorted_e[tid];
        plan[1 + MK + rank] = tid;
    }
    if (tid == 0) {
        plan[0] = nu;
        plan[1 + MK + nu] = MK;
    }
    // entries past the unique experts: expert -1, offset MK (every entry is written)
    if (tid < MK && tid >= nu) {
        plan[1 + tid] = -1;
        plan[1 + MK + tid + 1] = MK;
    }
    lds_barrier();
}

// Rows are taken by waves [row_wave0, waves); the other waves may do unrelated work
// (the MFMA gate/up kernel fills its codebook with them) before the first barrier.
__device__ __forceinline__ void topk_plan_block(const LayerDev& L, const MoeBufs& B, int M, bool global_out, int32_t* plan,
                                                TopkLds& t, int row_wave0) {
    const int wave = threadIdx.x >> 6;
    const int waves = blockDim.x >> 6;
    for (int r = wave - row_wave0; wave >= row_wave0 && r < M; r += waves - row_wave0) {
        float lg[16];
        topk_load_row(L, B, r, lg);
        topk_select_row(L, B, r, lg, t.ex, global_out);
    }
    topk_build_plan(M, L.K, plan, t);
}

// Gather-by-expert plan (R3) of up to 4 rows x K <= 16 routes over E <= 512 experts, built
// by one whole wave without loops over the routes (every lane calls it). ex: [M*K] expert
// ids in route order (route i = row * K + slot; the experts of one row are distinct). Same
// layout as topk_build_plan: routes sorted by (expert, route index), unique experts
// ascending. Lane 16 r + w builds the 32-bit mask of row r's experts in [32 w, 32 w + 32)
// and the exclusive prefix count of row r's experts below 32 w (a DPP scan within the 16-lane
// row); the union of the rows' masks gives the unique-expert ranks the same way. Route i
// (row r, expert e) then sits at sorted position #{routes with expert < e} + #{rows r' < r
// that chose e}, and opens its expert's group when no earlier row chose e. slot_pos, when
// given ([65][4] ints), receives the sorted position of row r's route in unique slot u at
// [4 u + r] (-1 where row r did not choose that expert; slot nu: the shared expert).
__device__ __forceinline__ uint32_t row_scan_incl(uint32_t x) {  // inclusive scan in 16-lane rows
    x += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0x111, 0xF, 0xF, false));
    x += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0x112, 0xF, 0xF, false));
    x += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0x114, 0xF, 0xF, false));
    x += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0x118, 0xF, 0xF, false));
    return x;
}
__device__ __forceinline__ void plan_wave(int M, int K, const int32_t* ex, int32_t* plan, int32_t* slot_pos = nullptr) {
    const int lane = threadIdx.x & 63;
    const int MK = M * K;
    if (slot_pos)
        for (int i = lane; i < (kNarrowMaxRoutes + 1) * 4; i += 64) slot_pos[i] = -1;
    // 1. row masks: lane 16 r + w
    const int mr = lane >> 4, mw = lane & 15;
    uint32_t m = 0;
#pragma unroll
    for (int s = 0; s < kMaxTopK; ++s) {  // slots past K repeat slot K - 1 (same bits)
        const int e = ex[(mr < M ? mr : 0) * K + (s < K ? s : K - 1)];
        m |= (e >> 5) == mw ? 1u << (e & 31) : 0u;
    }
    if (mr >= M) m = 0;
    const uint32_t pc = static_cast<uint32_t>(__popc(m));
    const uint32_t pref = row_scan_incl(pc) - pc;  // row mr's experts below 32 mw
    // 2. union of the rows' masks (every row of lanes ends with U[w]) and its prefix counts
    uint32_t u = m | static_cast<uint32_t>(__shfl_xor(static_cast<int>(m), 16, 64));
    u |= static_cast<uint32_t>(__shfl_xor(static_cast<int>(u), 32, 64));
    const uint32_t uc = static_cast<uint32_t>(__popc(u));
    const uint32_t upref = row_scan_incl(uc) - uc;
    const int nu = static_cast<int>(__builtin_amdgcn_readlane(static_cast<int>(upref + uc), 15));
    // 3. one lane per route
    const bool act = lane < MK;
    const int e = act ? ex[lane] : 0;
    const int r = (lane >= K ? 1 : 0) + (lane >= 2 * K ? 1 : 0) + (lane >= 3 * K ? 1 : 0);
    const int w = e >> 5, b = e & 31;
    const uint32_t low = (1u << b) - 1u;
    int below = 0, rank = 0;
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
        const uint32_t mk = static_cast<uint32_t>(__shfl(static_cast<int>(m), rr * 16 + w, 64));
        const uint32_t pk = static_cast<uint32_t>(__shfl(static_cast<int>(pref), rr * 16 + w, 64));
        if (rr < M) {
            below += static_cast<int>(pk) + __popc(mk & low);
            rank += (rr < r && ((mk >> b) & 1u)) ? 1 : 0;
        }
    }
    const uint32_t uw = static_cast<uint32_t>(__shfl(static_cast<int>(u), w, 64));
    const uint32_t upw = static_cast<uint32_t>(__shfl(static_cast<int>(upref), w, 64));
    const int pos = below + rank;
    const int urank = static_cast<int>(upw) + __popc(uw & low);
    if (act) {
        plan[2 + 2 * MK + pos] = lane;  // route at sorted position pos
        plan[2 + 3 * MK + lane] = pos;  // sorted position of route lane
        if (rank == 0) {
            plan[1 + urank] = e;
            plan[1 + MK + urank] = pos;
        }
        if (slot_pos) slot_pos[urank * 4 + r] = pos;
    }
    if (lane == 0) {
        plan[0] = nu;
        plan[1 + MK + nu] = MK;
    }
    // entries past the unique experts: expert -1, offset MK (every entry is written)
    if (act && lane >= nu) {
        plan[1 + lane] = -1;
        plan[1 + MK + lane + 1] = MK;
    }
    if (slot_pos && lane < M) slot_pos[nu * 4 + lane] = MK + lane;  // the shared expert's slot
}

// The route index of sorted position pos (shared-expert rows, pos >= MK, keep theirs).
__device__ __forceinline__ int route_of_pos(const int32_t* plan, int MK, int pos) {
    return pos < MK ? plan[2 + 2 * MK + pos] : pos;
}

// Codebook chunk -> LDS over the direct global-to-LDS path (no VGPR staging): waves
// w = 0..nw-1 of the caller copy KENT * 8 bytes, 1 KiB per wave instruction. The data is in
// LDS once the issuing wave's vmcnt drains; wait for that before the barrier that
// publishes it.
// The same copy by all NW waves of the workgroup with a compile-time instruction count per
// wave (unrolled), so the compiler can count the copy's vmcnt events exactly.
template <int KENT, int NW>
__device__ __forceinline__ void dma_book_all(const uint16_t* src4, unsigned char* lds) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const uint4* src = reinterpret_cast<const uint4*>(src4);
    constexpr int N = KENT / 2;
    constexpr int PER = (N + 64 * NW - 1) / (64 * NW);
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const int i = (k * NW + w) * 64;
        if (N % (64 * NW) == 0 || i < N)
            __builtin_amdgcn_global_load_lds(src + i + lane, reinterpret_cast<uint4*>(lds) + i, 16, 0, 0);
    }
}

template <int KENT>
__device__ __forceinline__ void dma_book(const uint16_t* src4, unsigned char* lds, int w, int nw) {
    const int lane = threadIdx.x & 63;
    const uint4* src = reinterpret_cast<const uint4*>(src4);
    constexpr int N = KENT / 2;  // 16-byte granules
    for (int i = w * 64; i < N; i += nw * 64)
        __builtin_amdgcn_global_load_lds(src + i + lane, reinterpret_cast<uint4*>(lds) + i, 16, 0, 0);
}

// Rows of unique-expert slot ui: the routed experts in ascending id, then the shared
// expert (all M rows). Returns false for an empty slot.
__device__ __forceinline__ bool slot_rows(const int32_t* plan, int M, int K, int has_shared, int ui, int E,
                                          int* expert, int* n, int* first_pos) {
    const int nu = plan[0];
    const int MK = M * K;
    // (the entries are read at a clamped index before any select, so that the compiler
    // cannot merge the LDS read with the caller's E into one generic load)
    const int uc = ui < nu ? ui : 0;
    const int pe = plan[1 + uc], a = plan[1 + MK + uc], b = plan[1 + MK + uc + 1];
    if (ui < nu) {
        *expert = pe;
        *n = b - a;
        *first_pos = a;
        return true;
    }
    if (ui == nu && has_shared) {
        *expert = E;
        *n = M;
        *first_pos = MK;
        return true;
    }
    return false;
}
// The combine's inputs for one (row, column) and its arithmetic (R8 reduce, R10, R11):
// routed = T(sum_slot w_slot * T(d_slot)) in slot order, shared = T(T(d_shared) * gate),
// y = T(routed + shared). Shared by the combine kernels and the fused layer kernel's tail.
template <int KT, bool TWO>
struct CombineIn {
    float wts[KT + 1];    // route weights in slot order, then the shared gate
    float dv[KT + 1][2];  // the routes' (and the shared expert's) down outputs, both planes
};

template <int KT, bool TWO>
__device__ __forceinline__ float combine_value(const LayerDev& L, const CombineIn<KT, TWO>& in) {
    float routed = 0.0f;
#pragma unroll
    for (int s = 0; s < KT; ++s) routed = fmaf(in.wts[s], rbf(TWO ? in.dv[s][0] + in.dv[s][1] : in.dv[s][0]), routed);
    float y = rbf(routed);
    if (L.has_shared) {
        const float sh = rbf(rbf(TWO ? in.dv[KT][0] + in.dv[KT][1] : in.dv[KT][0]) * in.wts[KT]);
        y = rbf(y + sh);
    }
    return y;
}

// The request row of the j-th route of slot ui.
__device__ __forceinline__ int route_row(const int32_t* plan, int M, int K, int pos0, int j, bool shared) {
    return shared ? j : plan[2 + 2 * M * K + pos0 + j] / K;
}

// Codebook chunk -> LDS by threads [0, nthreads): 16 loads in flight per thread.
template <int KENT>
__device__ __forceinline__ void fill_book(const uint16_t* src4, unsigned char* lds, int t, int nthreads) {
    const uint4* src = reinterpret_cast<const uint4*>(src4);
    uint4* dst = reinterpret_cast<uint4*>(lds);
    constexpr int N = KENT / 2;  // uint4 entries
    constexpr int G = 16;
    int i = t;
    for (; i + (G - 1) * nthreads < N; i += G * nthreads) {
        uint4 v[G];
#pragma unroll
        for (int k = 0; k < G; ++k) v[k] = src[i + k * nthreads];
#pragma unroll
        for (int k = 0; k < G; ++k) dst[i + k * nthreads] = v[k];
    }
    for (; i < N; i += nthreads) dst[i] = src[i];
}

// ============================================================== router rows (R1) + layer-input RMSNorm
// The arithmetic contracts of the router, shared by the router kernel (k_route_norm) and the
// one-launch layer kernel (k_gd4 with its router) so that the two give the same bits. A
// workgroup of NT = H / 4 threads forms the norm: thread t owns columns t + NT i (i < 4) of
// every row and accumulates fmaf(v, v) in i order; the wave xor-butterfly totals (MR > 1:
// reduced and scattered together) go to red[MR][NT / 64]; after a barrier, lane r of every
// wave adds row r's wave totals in wave order and forms inv_rms = 1 / sqrt(total / H + eps),
// which every lane reads back.
template <int NT, int MR>
__device__ __forceinline__ void norm_partials(const float (&v)[MR][4], float (*red)[NT / 64]) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float ss[MR];
#pragma unroll
    for (int r = 0; r < MR; ++r) {
        ss[r] = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) ss[r] = fmaf(v[r][i], v[r][i], ss[r]);
    }
    if constexpr (MR == 1) {
        ss[0] = wave_sum_xor(ss[0]);
        if (lane == 0) red[0][wave] = ss[0];
    } else {
        wave_sum_xor_scatter<MR>(ss);
#pragma unroll
        for (int s = 0; s < scatter_slots<MR>(); ++s)
            if (scatter_leader<MR>(lane)) red[scatter_value<MR>(s, lane >> 4)][wave] = ss[s];
    }
}
template <int NT, int MR>
__device__ __forceinline__ void norm_inv(const float (*red)[NT / 64], int H, float eps, float (&inv)[MR]) {
    const int lane = threadIdx.x & 63;
    const int rl = lane < MR ? lane : 0;
    float t = 0.0f;
#pragma unroll
    for (int w = 0; w < NT / 64; ++w) t += red[rl][w];
    const float il = 1.0f / sqrtf(t / static_cast<float>(H) + eps);
#pragma unroll
    for (int r = 0; r < MR; ++r) inv[r] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(il), r));
}
// Router logit contract: lane l holds the columns c = 512 t + 8 l + j of a router row (t < T
// outer, j < 8 inner) and accumulates x * w with fmaf for each of the MR request rows (rows
// past M repeat row 0); then the MR butterflies at once (reduced and scattered for MR > 1:
// 16-lane row q of acc[s] ends with request row scatter_value<MR>(s, q)). xs: [M][512 T] bf16.
template <int T, int MR>
__device__ __forceinline__ void router_dots(const uint16_t* xs, int M, const uint4 (&wv)[T], float (&acc)[MR]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int r = 0; r < MR; ++r) {
        acc[r] = 0.0f;
        const int rr = r < M ? r : 0;
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const uint4 xv = *reinterpret_cast<const uint4*>(xs + static_cast<size_t>(rr) * 512 * T + 512 * t + 8 * lane);
            const uint32_t xq[4] = {xv.x, xv.y, xv.z, xv.w};
            const uint32_t wq[4] = {wv[t].x, wv[t].y, wv[t].z, wv[t].w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                acc[r] = __builtin_fmaf(bflo(xq[k]), bflo(wq[k]), acc[r]);
                acc[r] = __builtin_fmaf(bfhi(xq[k]), bfhi(wq[k]), acc[r]);
            }
        }
    }
    if constexpr (MR > 1) wave_sum_xor_scatter<MR>(acc);
    else acc[0] = wave_sum_xor(acc[0]);
}

// SwiGLU with the reference's rounding points (src/vq_metal_kernels.hpp:589-595):
// h = T(T(silu(T(g))) * T(u)).
__device__ __forceinline__ float swiglu(float g, float u) {
    const float gt = rbf(g);
    const float s = rbf(gt / (1.0f + expf(-gt)));
    return rbf(s * rbf(u));
}

} // namespace q38
