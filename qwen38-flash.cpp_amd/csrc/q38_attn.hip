// q38_attn.hip — the full-attention verify step on its dense path: the attention half of a
// decoder layer for S verify rows (1..64) of one slot over the slot's KV cache, the cache
// extended by the rows (SelfAttention::forward_verify, src/self_attention.cpp:1450-1720; the
// QSA mask, built only once a context exceeds the indexer budget, :764-766, and the Q8 KV
// cache are not part of this path). A row's checkpoint is the cache prefix up to it, so the
// call writes no state copies.
//
// Seven launches:
//   k_affine_rows    q (each head's D query rows, then its D gate rows), k and v of the S
//                    rows in one launch (q38_affine.hip), rounded to bf16;
//   k_attn_prework   per (row, head): the q / k RMS norms T(w * T(x * inv)), RoPE on the first
//                    R dims with the bf16 cos / sin of position * theta^(-2i / R) formed in
//                    double (:641-679), T(sigmoid(gate)), and the new keys and values written
//                    into the cache at the row's token;
//   k_attn_scores    per (64-token tile, kv head): s = T(T(q . k) * T(1 / sqrt D)) for every
//                    token a query sees (t <= T0 + r) on bf16 MFMA (exact products, float
//                    sums), and per query the tile's max and float sum of exp(s - max);
//   k_attn_stats     per query: the max over its tiles and the sum of the tiles' sums scaled
//                    to it;
//   k_attn_pv        per (128-token tile, kv head, 64 queries): p = T(exp(s - max) / sum) as
//                    the A operand of bf16 MFMA against the tile's values (staged transposed in
//                    LDS, 64 tokens at a time), one float partial row per (tile, query);
//   k_attn_combine   per query: the tiles' partials added in a fixed order, rounded, times the
//                    gate, rounded;
//   k_affine_rows    the output projection.
// Tiles start at multiples of their size from token 0, so a query's sums do not depend on how
// many rows the call carries: S rows give the bits of S one-row calls.
// Cache layout (q38_attn_cache_bytes): keys [HKV][capacity][D] bf16, then values alike.
#include "q38_device.hpp"
#include "q38_internal.hpp"

namespace q38 {

namespace {

constexpr int kTok = 64;     // tokens per score tile (and per P.V sub-tile)
constexpr int kPvTok = 128;  // tokens per P.V tile (256: 70.6 -> 63.9 us per 4-row call at 4K tokens)
constexpr int kPvMt = 4;     // 16-query M-tiles per P.V workgroup

__device__ __forceinline__ float tbf(float v) { return bf2f(f2bf(v)); }
__device__ __forceinline__ float sigmoid_bf(float x) { return tbf(1.0f / (1.0f + expf(-x))); }

// q / k: norm + RoPE into B.q or the cache; gate: T(sigmoid); v: into the cache.
template <int CPL>
__global__ __launch_bounds__(64) void k_attn_prework(AttnDev A, AttnBufs B, uint16_t* __restrict__ keys,
                                                     uint16_t* __restrict__ values, int64_t cap, int64_t T0,
                                                     int64_t position) {
    __shared__ float nv[64 * CPL];
    __shared__ float csk[32 * CPL], snk[32 * CPL];  // the rotary table of this row: pair k's T(cos), T(sin)
    const int head = blockIdx.x, r = blockIdx.y, lane = threadIdx.x;
    const int HQ = A.hq, HKV = A.hkv, D = A.d, R = A.rot, half = R / 2;
    const int QW = HQ * D, KW = HKV * D;
    const int role = head < HQ ? 0 : head < HQ + HKV ? 1 : 2;  // query, key, value head
    const int h = role == 0 ? head : role == 1 ? head - HQ : head - HQ - HKV;
    const int64_t tok = T0 + r;
    if (role == 2) {
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const int i = lane * CPL + c;
            values[(static_cast<int64_t>(h) * cap + tok) * D + i] = B.vr[static_cast<size_t>(r) * KW + h * D + i];
        }
        return;
    }
    const uint16_t* src = role == 0 ? B.qg + static_cast<size_t>(r) * 2 * QW + static_cast<size_t>(h) * 2 * D
                                    : B.kr + static_cast<size_t>(r) * KW + h * D;
    const uint16_t* wn = role == 0 ? A.qn : A.kn;
    float x[CPL];
    float ss = 0.0f;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        x[c] = bf2f(src[lane * CPL + c]);
        ss = fmaf(x[c], x[c], ss);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
    const float inv = 1.0f / sqrtf(ss / static_cast<float>(D) + A.eps);
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        const int i = lane * CPL + c;
        nv[i] = tbf(bf2f(wn[i]) * tbf(x[c] * inv));
    }
    // one rotary pair per lane (the two elements of a pair share its angle), in double as
    // before: pos * theta^(-2k / R)
    const double pos = static_cast<double>(position + r);
    for (int k = lane; k < half; k += 64) {
        const double ang = pos * pow(A.theta, -2.0 * static_cast<double>(k) / static_cast<double>(R));
        csk[k] = tbf(static_cast<float>(cos(ang)));
        snk[k] = tbf(static_cast<float>(sin(ang)));
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        const int i = lane * CPL + c;
        float y = nv[i];
        if (i < R) {
            const int k = i < half ? i : i - half;
            const float cs = csk[k], sn = snk[k];
            const float rot = i < half ? -nv[i + half] : nv[i - half];
            y = tbf(tbf(nv[i] * cs) + tbf(rot * sn));
        }
        if (role == 0) {
            const size_t at = (static_cast<size_t>(r) * HQ + h) * D + i;
            B.q[at] = f2bf(y);
            B.gs[at] = f2bf(sigmoid_bf(bf2f(src[D + i])));
        } else {
            keys[(static_cast<int64_t>(h) * cap + tok) * D + i] = f2bf(y);
        }
    }
}

typedef __bf16 bf8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ f4_t mfma_bf16(uint4 a, uint4 b, f4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf8_t, a), __builtin_bit_cast(bf8_t, b), c, 0,
                                                   0, 0);
}

// Scores and tile statistics of one 64-token tile of kv head g for mt_per_wg 16-query M-tiles
// (from blockIdx.z * mt_per_wg) of the head's group (query j: row j / G, head g G + j % G), on
// v_mfma_f32_16x16x32_bf16: wave w takes tokens 16 w .. 16 w + 15 of the tile; A = the queries (lane
// (c, q): query row c, dims 8 q .. 8 q + 7 of each 32-dim step), B = the keys (lane (c, q):
// token c, the same dims), both read as 16-byte runs; the products are exact and the sums
// float. The lane then holds queries 4 q .. 4 q + 3 of the M-tile for token c. Per query the
// tile's max and the float sum of exp(s - max) over the tokens it sees go to B.stats.
template <int D>
__global__ __launch_bounds__(256) void k_attn_scores(AttnDev A, AttnBufs B, int S, const uint16_t* __restrict__ keys,
                                                     int64_t cap, int64_t T0, int64_t tpad, int mt_per_wg) {
    constexpr int KS = D / 32;
    __shared__ float red_m[4][16], red_s[4][16];
    const int tile = blockIdx.x, g = blockIdx.y, lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int c = lane & 15, q = lane >> 4;
    const int HQ = A.hq, G = HQ / A.hkv, NQ = S * G;
    const int64_t Ttot = T0 + S, tk = static_cast<int64_t>(tile) * kTok + 16 * w + c;
    const uint16_t* krow = keys + (static_cast<int64_t>(g) * cap + (tk < Ttot ? tk : Ttot - 1)) * D + 8 * q;
    uint4 kb[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) kb[ks] = *reinterpret_cast<const uint4*>(krow + 32 * ks);
    const float scale = tbf(static_cast<float>(1.0 / sqrt(static_cast<double>(D))));
    const size_t NQall = static_cast<size_t>(S) * HQ;
    const int mt_lo = blockIdx.z * mt_per_wg, mt_hi = min(mt_lo + mt_per_wg, (NQ + 15) / 16);
    for (int mt = mt_lo; mt < mt_hi; ++mt) {
        const int jr = mt * 16 + c;  // this lane's A row
        uint4 qa[KS];
        if (jr < NQ) {
            const uint16_t* qrow = B.q + (static_cast<size_t>(jr / G) * HQ + g * G + jr % G) * D + 8 * q;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) qa[ks] = *reinterpret_cast<const uint4*>(qrow + 32 * ks);
        } else {
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) qa[ks] = make_uint4(0u, 0u, 0u, 0u);
        }
        f4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) acc = mfma_bf16(qa[ks], kb[ks], acc);
        float sv[4], mm[4];
        bool ok[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int j = mt * 16 + 4 * q + i, r = j / G;
            ok[i] = j < NQ && tk <= T0 + r;
            sv[i] = ok[i] ? tbf(tbf(acc[i]) * scale) : -INFINITY;
            if (ok[i]) B.sc[(static_cast<size_t>(r) * HQ + g * G + j % G) * tpad + tk] = f2bf(sv[i]);
            float m = sv[i];
#pragma unroll
            for (int off = 1; off < 16; off <<= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
            mm[i] = m;
        }
        if (c == 0)
#pragma unroll
            for (int i = 0; i < 4; ++i) red_m[w][4 * q + i] = mm[i];
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = 4 * q + i;
            mm[i] = fmaxf(fmaxf(red_m[0][row], red_m[1][row]), fmaxf(red_m[2][row], red_m[3][row]));
            float e = ok[i] ? expf(sv[i] - mm[i]) : 0.0f;
#pragma unroll
            for (int off = 1; off < 16; off <<= 1) e += __shfl_xor(e, off, 64);
            if (c == 0) red_s[w][row] = e;
        }
        __syncthreads();
        if (w == 0 && c == 0)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int j = mt * 16 + 4 * q + i, row = 4 * q + i;
                if (j >= NQ) continue;
                const size_t qi = static_cast<size_t>(j / G) * HQ + g * G + j % G;
                B.stats[static_cast<size_t>(tile) * NQall + qi] =
                    make_float2(mm[i], (red_s[0][row] + red_s[1][row]) + (red_s[2][row] + red_s[3][row]));
            }
        __syncthreads();
    }
}

// Per query: max and sum over its tiles' statistics (m = max m_t, sum = sum s_t exp(m_t - m)).
__global__ __launch_bounds__(256) void k_attn_stats(AttnDev A, AttnBufs B, int S, int64_t T0) {
    __shared__ float red[4];
    const int qi = blockIdx.x, r = qi / A.hq, tid = threadIdx.x;
    const size_t NQall = static_cast<size_t>(S) * A.hq;
    const int64_t nt = (T0 + r + 1 + kTok - 1) / kTok;
    float m = -INFINITY;
    for (int64_t k = tid; k < nt; k += 256) m = fmaxf(m, B.stats[static_cast<size_t>(k) * NQall + qi].x);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    float s = 0.0f;
    for (int64_t k = tid; k < nt; k += 256) {
        const float2 st = B.stats[static_cast<size_t>(k) * NQall + qi];
        s += st.y * expf(st.x - m);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
    if ((tid & 63) == 0) red[tid >> 6] = s;
    __syncthreads();
    if (tid == 0) {
        B.mx[qi] = m;
        B.sm[qi] = (red[0] + red[1]) + (red[2] + red[3]);
    }
}

// P.V of one 128-token tile (two 64-token sub-tiles) of kv head g for a DW-dim slice and
// M-tiles mt0 .. mt0 + kPvMt - 1 of the group's queries, on v_mfma_f32_16x16x32_bf16: the
// sub-tile's values of the slice are staged transposed in LDS ([dim][token], rows padded by 16
// bytes; the next sub-tile's loads are in flight while the current one computes); A = p =
// T(exp(s - m) / sum) of 8 tokens of one query (0 for tokens the query does not see), B = 8
// tokens of one dim; wave w owns dims 16 NTW w .. 16 NTW (w + 1) - 1 of the slice. One float
// partial per (tile, query, dim).
template <int D, int DW>
__global__ __launch_bounds__(256) void k_attn_pv(AttnDev A, AttnBufs B, int S, const uint16_t* __restrict__ values,
                                                 int64_t cap, int64_t T0, int64_t tpad) {
    constexpr int VS = kTok + 8;        // transposed row (bf16)
    constexpr int NSL = D / DW;         // dim slices (DW dims per workgroup)
    constexpr int NTW = DW / 64;        // 16-dim N-tiles per wave
    constexpr int CPT = DW / 64;        // 8-dim chunks a thread stages per sub-tile (two tokens each)
    __shared__ __align__(16) uint16_t vt[DW * VS];
    const int tile = blockIdx.x, g = blockIdx.y, mt0 = (blockIdx.z / NSL) * kPvMt, d0 = (blockIdx.z % NSL) * DW;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, c = lane & 15, q = lane >> 4;
    const int HQ = A.hq, G = HQ / A.hkv, NQ = S * G;
    const int nmt = (NQ + 15) / 16 - mt0 < kPvMt ? (NQ + 15) / 16 - mt0 : kPvMt;
    const int64_t Ttot = T0 + S, tb = static_cast<int64_t>(tile) * kPvTok;
    const int64_t left = Ttot - tb;
    const int nsub = static_cast<int>(left >= kPvTok ? kPvTok / kTok : (left + kTok - 1) / kTok);
    // staging: thread (token pair tp, 8-dim chunks dc0 + 8 k) of the slice
    const int tp = tid & 31, dc0 = tid >> 5;
    uint4 va[CPT], vb[CPT];
    auto load = [&](int64_t ts) {
        const int64_t t = ts + 2 * tp;
#pragma unroll
        for (int k = 0; k < CPT; ++k) {
            const uint16_t* src = values + (static_cast<int64_t>(g) * cap + t) * D + d0 + 8 * (dc0 + 8 * k);
            va[k] = t < Ttot ? *reinterpret_cast<const uint4*>(src) : make_uint4(0u, 0u, 0u, 0u);
            vb[k] = t + 1 < Ttot ? *reinterpret_cast<const uint4*>(src + D) : make_uint4(0u, 0u, 0u, 0u);
        }
    };
    auto store = [&]() {
#pragma unroll
        for (int k = 0; k < CPT; ++k) {
            const uint32_t a[4] = {va[k].x, va[k].y, va[k].z, va[k].w}, b[4] = {vb[k].x, vb[k].y, vb[k].z, vb[k].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int d = 8 * (dc0 + 8 * k) + 2 * e;
                *reinterpret_cast<uint32_t*>(vt + d * VS + 2 * tp) = (a[e] & 0xFFFFu) | (b[e] << 16);
                *reinterpret_cast<uint32_t*>(vt + (d + 1) * VS + 2 * tp) = (a[e] >> 16) | (b[e] & 0xFFFF0000u);
            }
        }
    };
    f4_t acc[kPvMt][NTW];
#pragma unroll
    for (int mt = 0; mt < kPvMt; ++mt)
#pragma unroll
        for (int nt = 0; nt < NTW; ++nt) acc[mt][nt] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
    // per M-tile: this lane's A-row query, its softmax max and sum (read once)
    size_t qrow[kPvMt];
    int rrow[kPvMt];
    float mrow[kPvMt], srow[kPvMt];
#pragma unroll
    for (int mt = 0; mt < kPvMt; ++mt) {
        const int j = (mt0 + mt) * 16 + c;
        rrow[mt] = -1;
        if (mt < nmt && j < NQ) {
            rrow[mt] = j / G;
            qrow[mt] = static_cast<size_t>(rrow[mt]) * HQ + g * G + j % G;
            mrow[mt] = B.mx[qrow[mt]];
            srow[mt] = B.sm[qrow[mt]];
        }
    }
    // the scores of the lane's 2 x 8 tokens of a sub-tile, per M-tile (loaded with the values)
    uint4 scv[kPvMt][2];
    auto load_sc = [&](int64_t ts) {
#pragma unroll
        for (int mt = 0; mt < kPvMt; ++mt)
            if (rrow[mt] >= 0)
#pragma unroll
                for (int ks = 0; ks < 2; ++ks)
                    scv[mt][ks] = *reinterpret_cast<const uint4*>(B.sc + qrow[mt] * tpad + ts + 32 * ks + 8 * q);
    };
    load(tb);
    load_sc(tb);
    for (int s = 0; s < nsub; ++s) {
        const int64_t ts = tb + static_cast<int64_t>(kTok) * s;
        __syncthreads();  // the previous sub-tile's reads are done
        store();
        __syncthreads();
        uint4 pa[kPvMt][2];
#pragma unroll
        for (int mt = 0; mt < kPvMt; ++mt) {
            pa[mt][0] = pa[mt][1] = make_uint4(0u, 0u, 0u, 0u);
            if (rrow[mt] < 0) continue;
            const int64_t last = T0 + rrow[mt];
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                const int64_t t = ts + 32 * ks + 8 * q;
                const uint32_t u[4] = {scv[mt][ks].x, scv[mt][ks].y, scv[mt][ks].z, scv[mt][ks].w};
                uint32_t pk[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float s0 = __uint_as_float(u[e] << 16), s1 = __uint_as_float(u[e] & 0xFFFF0000u);
                    const uint32_t p0 = t + 2 * e <= last ? f2bf(expf(s0 - mrow[mt]) / srow[mt]) : 0u;
                    const uint32_t p1 = t + 2 * e + 1 <= last ? f2bf(expf(s1 - mrow[mt]) / srow[mt]) : 0u;
                    pk[e] = p0 | (p1 << 16);
                }
                pa[mt][ks] = make_uint4(pk[0], pk[1], pk[2], pk[3]);
            }
        }
        if (s + 1 < nsub) {  // the next sub-tile's values and scores are in flight during the MFMAs
            load(ts + kTok);
            load_sc(ts + kTok);
        }
#pragma unroll
        for (int mt = 0; mt < kPvMt; ++mt) {
            if (mt >= nmt) break;
#pragma unroll
            for (int nt = 0; nt < NTW; ++nt) {
                const uint16_t* col = vt + ((w * NTW + nt) * 16 + c) * VS + 8 * q;
#pragma unroll
                for (int ks = 0; ks < 2; ++ks)
                    acc[mt][nt] = mfma_bf16(pa[mt][ks], *reinterpret_cast<const uint4*>(col + 32 * ks), acc[mt][nt]);
            }
        }
    }
    const size_t NQall = static_cast<size_t>(S) * HQ;
#pragma unroll
    for (int mt = 0; mt < kPvMt; ++mt) {
        if (mt >= nmt) break;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int j = (mt0 + mt) * 16 + 4 * q + i;
            if (j >= NQ) continue;
            const size_t qi = static_cast<size_t>(j / G) * HQ + g * G + j % G;
#pragma unroll
            for (int nt = 0; nt < NTW; ++nt)
                B.part[(static_cast<size_t>(tile) * NQall + qi) * D + d0 + (w * NTW + nt) * 16 + c] = acc[mt][nt][i];
        }
    }
}

// attended = T(sum of the tiles' partials), gated = T(attended * gate): TG groups of D
// threads, group k adds tiles k, k + TG, .. (8 loads in flight), the groups added in order.
template <int D>
__global__ __launch_bounds__(1024) void k_attn_combine(AttnDev A, AttnBufs B, int S, int64_t T0) {
    constexpr int TG = 1024 / D;
    __shared__ float red[1024];
    const int qi = blockIdx.x, d = threadIdx.x % D, k = threadIdx.x / D;
    const int r = qi / A.hq, h = qi % A.hq;
    const int64_t ntile = (T0 + r + 1 + kPvTok - 1) / kPvTok;
    const size_t NQall = static_cast<size_t>(S) * A.hq;
    const float* src = B.part + static_cast<size_t>(qi) * D + d;
    const size_t step = NQall * D;
    float a = 0.0f;
    int64_t t = k;
    for (; t + 7 * TG < ntile; t += 8 * TG) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = src[static_cast<size_t>(t + u * TG) * step];
#pragma unroll
        for (int u = 0; u < 8; ++u) a += v[u];
    }
    for (; t < ntile; t += TG) a += src[static_cast<size_t>(t) * step];
    red[threadIdx.x] = a;
    __syncthreads();
    if (k != 0) return;
    float s = red[d];
#pragma unroll
    for (int kk = 1; kk < TG; ++kk) s += red[kk * D + d];
    B.gated[static_cast<size_t>(r) * A.hq * D + static_cast<size_t>(h) * D + d] =
        f2bf(tbf(s) * bf2f(B.gs[static_cast<size_t>(qi) * D + d]));
}

template <int D>
hipError_t launch_attn_core(const AttnDev& A, const AttnBufs& B, int S, uint16_t* keys, uint16_t* values, int64_t cap,
                            int64_t T0, int64_t position, int64_t tpad, hipStream_t st) {
    const int HQ = A.hq, HKV = A.hkv, G = HQ / HKV;
    const int64_t Ttot = T0 + S;
    hipError_t e = launch(k_attn_prework<D / 64>, dim3(HQ + 2 * HKV, S), dim3(64), 0, st, A, B, keys, values, cap, T0,
                          position);
    if (e != hipSuccess) return e;
    // short contexts: one M-tile per workgroup for parallelism; long ones: the workgroup takes
    // every M-tile of its tile (the keys are read once)
    const int nmt = (S * G + 15) / 16;
    const int64_t ntile = (Ttot + kTok - 1) / kTok;
    const int mt_per_wg = ntile * HKV < 1024 ? 1 : nmt;
    e = launch(k_attn_scores<D>, dim3(static_cast<unsigned>(ntile), HKV, (nmt + mt_per_wg - 1) / mt_per_wg), dim3(256),
               0, st, A, B, S, static_cast<const uint16_t*>(keys), cap, T0, tpad, mt_per_wg);
    if (e != hipSuccess) return e;
    e = launch(k_attn_stats, dim3(S * HQ), dim3(256), 0, st, A, B, S, T0);
    if (e != hipSuccess) return e;
    const unsigned mchunks = static_cast<unsigned>((nmt + kPvMt - 1) / kPvMt);
    const unsigned npv = static_cast<unsigned>((Ttot + kPvTok - 1) / kPvTok);
    if (npv * HKV * mchunks < 128)  // few tiles: 64-dim slices per workgroup for parallelism
        e = launch(k_attn_pv<D, 64>, dim3(npv, HKV, mchunks * (D / 64)), dim3(256), 0, st, A, B, S,
                   static_cast<const uint16_t*>(values), cap, T0, tpad);
    else
        e = launch(k_attn_pv<D, D>, dim3(npv, HKV, mchunks), dim3(256), 0, st, A, B, S,
                   static_cast<const uint16_t*>(values), cap, T0, tpad);
    if (e != hipSuccess) return e;
    return launch(k_attn_combine<D>, dim3(S * HQ), dim3(1024), 0, st, A, B, S, T0);
}

} // namespace

bool attn_geometry_ok(int hidden, int hq, int hkv, int d, int rot) {
    return hidden > 0 && hq > 0 && hkv > 0 && hq % hkv == 0 && (d == 64 || d == 128 || d == 256) && rot > 0 &&
           rot % 2 == 0 && rot <= d;
}

int64_t attn_score_stride(int64_t tokens) { return (tokens + kTok - 1) / kTok * kTok; }
int64_t attn_pv_tiles(int64_t tokens) { return (tokens + kPvTok - 1) / kPvTok; }
int64_t attn_score_tiles(int64_t tokens) { return (tokens + kTok - 1) / kTok; }

hipError_t launch_attn_verify(const AttnDev& A, const AttnBufs& B, int S, const uint16_t* x, uint16_t* keys,
                              uint16_t* values, int64_t cap, int64_t T0, int64_t position, uint16_t* out,
                              hipStream_t st) {
    const int QW = A.hq * A.d, KW = A.hkv * A.d;
    AffineRowSet in{};
    in.n = 3;
    in.p[0] = AffineRows{A.w[0], A.s[0], A.b[0], B.qg, 2 * QW, 2 * QW, 0};
    in.p[1] = AffineRows{A.w[1], A.s[1], A.b[1], B.kr, KW, KW, 0};
    in.p[2] = AffineRows{A.w[2], A.s[2], A.b[2], B.vr, KW, KW, 0};
    hipError_t e = launch_affine_rows(in, x, S, A.hidden, A.group, A.bits, A.f16, st);
    if (e != hipSuccess) return e;
    const int64_t tpad = attn_score_stride(T0 + S);
    switch (A.d) {
        case 64: e = launch_attn_core<64>(A, B, S, keys, values, cap, T0, position, tpad, st); break;
        case 128: e = launch_attn_core<128>(A, B, S, keys, values, cap, T0, position, tpad, st); break;
        case 256: e = launch_attn_core<256>(A, B, S, keys, values, cap, T0, position, tpad, st); break;
        default: return hipErrorInvalidValue;
    }
    if (e != hipSuccess) return e;
    AffineRowSet o{};
    o.n = 1;
    o.p[0] = AffineRows{A.w[3], A.s[3], A.b[3], out, A.hidden, A.hidden, 0};
    return launch_affine_rows(o, B.gated, S, QW, A.group, A.bits, A.f16, st);
}

} // namespace q38
