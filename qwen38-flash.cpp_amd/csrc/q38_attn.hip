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
//   k_attn_scores    per (64-token tile, kv head, chunk of 32 queries): the tile's keys staged
//                    in LDS (rows padded by 16 bytes), the queries as float; one lane per token,
//                    the waves splitting the queries; s = T(T(q . k) * T(1 / sqrt D)) for every
//                    token the query sees (t <= T0 + r);
//   k_attn_softmax   per query: the max and the float sum of exp(s - max) over its tokens;
//   k_attn_pv        per (256-token tile, kv head, chunk of 32 queries): p = T(e / sum) into
//                    LDS, then per dimension the tile's sum of p * v in float (token groups
//                    added in order), one partial row per (tile, query);
//   k_attn_combine   per query: the tiles' partials added in tile order, rounded, times the
//                    gate, rounded;
//   k_affine_rows    the output projection.
// Tiles start at multiples of their size from token 0, so a query's sums do not depend on how
// many rows the call carries: S rows give the bits of S one-row calls.
// Cache layout (q38_attn_cache_bytes): keys [HKV][capacity][D] bf16, then values alike.
#include "q38_device.hpp"
#include "q38_internal.hpp"

namespace q38 {

namespace {

constexpr int kTok = 64;     // tokens per score tile
constexpr int kPvTok = 256;  // tokens per P.V tile
constexpr int kQc = 32;      // queries per chunk

__device__ __forceinline__ float tbf(float v) { return bf2f(f2bf(v)); }
__device__ __forceinline__ float sigmoid_bf(float x) { return tbf(1.0f / (1.0f + expf(-x))); }

// q / k: norm + RoPE into B.q or the cache; gate: T(sigmoid); v: into the cache.
template <int CPL>
__global__ __launch_bounds__(64) void k_attn_prework(AttnDev A, AttnBufs B, uint16_t* __restrict__ keys,
                                                     uint16_t* __restrict__ values, int64_t cap, int64_t T0,
                                                     int64_t position) {
    __shared__ float nv[64 * CPL];
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
    __syncthreads();
    const double pos = static_cast<double>(position + r);
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        const int i = lane * CPL + c;
        float y = nv[i];
        if (i < R) {
            const int k = i < half ? i : i - half;
            const double ang = pos * pow(A.theta, -2.0 * static_cast<double>(k) / static_cast<double>(R));
            const float cs = tbf(static_cast<float>(cos(ang))), sn = tbf(static_cast<float>(sin(ang)));
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

// Scores of one 64-token tile of kv head g for queries j0 .. j0 + 31 of the head's group
// (query j: row j / G, head g G + j % G).
template <int D>
__global__ __launch_bounds__(256) void k_attn_scores(AttnDev A, AttnBufs B, int S, const uint16_t* __restrict__ keys,
                                                     int64_t cap, int64_t T0, int64_t tpad) {
    constexpr int KS = D + 8;  // padded key row (bf16): rows start 4 banks apart
    extern __shared__ __align__(16) char lds[];
    uint16_t* kt = reinterpret_cast<uint16_t*>(lds);                        // [64][KS]
    float* qs = reinterpret_cast<float*>(lds + kTok * KS * sizeof(uint16_t));  // [32][D]
    const int tile = blockIdx.x, g = blockIdx.y;
    const int G = A.hq / A.hkv, NQ = S * G, j0 = blockIdx.z * kQc;
    const int nq = NQ - j0 < kQc ? NQ - j0 : kQc;
    const int64_t t0 = static_cast<int64_t>(tile) * kTok, Ttot = T0 + S;
    constexpr int WPR = D / 8;  // 16-byte words per key row
    for (int w = threadIdx.x; w < kTok * WPR; w += 256) {
        const int tt = w / WPR, c = w % WPR;
        const int64_t t = t0 + tt < Ttot ? t0 + tt : Ttot - 1;
        *reinterpret_cast<uint4*>(kt + tt * KS + c * 8) =
            *reinterpret_cast<const uint4*>(keys + (static_cast<int64_t>(g) * cap + t) * D + c * 8);
    }
    for (int e = threadIdx.x; e < nq * D; e += 256) {
        const int jj = e / D, i = e % D, j = j0 + jj;
        qs[jj * D + i] = bf2f(B.q[(static_cast<size_t>(j / G) * A.hq + g * G + j % G) * D + i]);
    }
    __syncthreads();
    const int tt = threadIdx.x & 63, wv = threadIdx.x >> 6;
    constexpr int QPW = kQc / 4;  // queries per wave: jj = wv + 4 k
    float acc[QPW];
#pragma unroll
    for (int k = 0; k < QPW; ++k) acc[k] = 0.0f;
    for (int c = 0; c < D; c += 8) {
        const uint4 kw = *reinterpret_cast<const uint4*>(kt + tt * KS + c);
        const uint32_t u[4] = {kw.x, kw.y, kw.z, kw.w};
        float kf[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            kf[2 * e] = __uint_as_float(u[e] << 16);
            kf[2 * e + 1] = __uint_as_float(u[e] & 0xFFFF0000u);
        }
#pragma unroll
        for (int k = 0; k < QPW; ++k) {
            const int jj = wv + 4 * k;
            if (jj < nq) {
                const float4 a = *reinterpret_cast<const float4*>(qs + jj * D + c);
                const float4 b = *reinterpret_cast<const float4*>(qs + jj * D + c + 4);
                float s = acc[k];
                s = fmaf(a.x, kf[0], s);
                s = fmaf(a.y, kf[1], s);
                s = fmaf(a.z, kf[2], s);
                s = fmaf(a.w, kf[3], s);
                s = fmaf(b.x, kf[4], s);
                s = fmaf(b.y, kf[5], s);
                s = fmaf(b.z, kf[6], s);
                s = fmaf(b.w, kf[7], s);
                acc[k] = s;
            }
        }
    }
    const float scale = tbf(static_cast<float>(1.0 / sqrt(static_cast<double>(D))));
    const int64_t t = t0 + tt;
#pragma unroll
    for (int k = 0; k < QPW; ++k) {
        const int jj = wv + 4 * k;
        if (jj >= nq) continue;
        const int j = j0 + jj, r = j / G;
        if (t <= T0 + r) B.sc[(static_cast<size_t>(r) * A.hq + g * G + j % G) * tpad + t] = f2bf(tbf(acc[k]) * scale);
    }
}

// Max and sum of exp(s - max) of one query's scores (row r: tokens 0 .. T0 + r).
__global__ __launch_bounds__(256) void k_attn_softmax(AttnDev A, AttnBufs B, int64_t T0, int64_t tpad) {
    __shared__ float red[4];
    const int qi = blockIdx.x, r = qi / A.hq, tid = threadIdx.x;
    const int64_t T = T0 + r + 1;
    const uint16_t* row = B.sc + static_cast<size_t>(qi) * tpad;
    float m = -INFINITY;
    for (int64_t t = tid; t < T; t += 256) m = fmaxf(m, bf2f(row[t]));
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    float s = 0.0f;
    for (int64_t t = tid; t < T; t += 256) s += expf(bf2f(row[t]) - m);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
    if ((tid & 63) == 0) red[tid >> 6] = s;
    __syncthreads();
    if (tid == 0) {
        B.mx[qi] = m;
        B.sm[qi] = (red[0] + red[1]) + (red[2] + red[3]);
    }
}

// Partial P.V rows of one 256-token tile of kv head g for queries j0 .. j0 + 31.
template <int D>
__global__ __launch_bounds__(256) void k_attn_pv(AttnDev A, AttnBufs B, int S, const uint16_t* __restrict__ values,
                                                 int64_t cap, int64_t T0, int64_t tpad) {
    constexpr int TPD = 256 / D;  // token groups
    extern __shared__ __align__(16) char lds[];
    float* ps = reinterpret_cast<float*>(lds);           // [32][256]
    float* red = ps + kQc * kPvTok;                      // [TPD][32][D]
    const int tile = blockIdx.x, g = blockIdx.y;
    const int G = A.hq / A.hkv, NQ = S * G, j0 = blockIdx.z * kQc;
    const int nq = NQ - j0 < kQc ? NQ - j0 : kQc;
    const int64_t t0 = static_cast<int64_t>(tile) * kPvTok, Ttot = T0 + S;
    for (int e = threadIdx.x; e < nq * kPvTok; e += 256) {
        const int jj = e / kPvTok, tt = e % kPvTok, j = j0 + jj, r = j / G;
        const int64_t t = t0 + tt;
        const size_t qi = static_cast<size_t>(r) * A.hq + g * G + j % G;
        float p = 0.0f;
        if (t <= T0 + r) p = tbf(expf(bf2f(B.sc[qi * tpad + t]) - B.mx[qi]) / B.sm[qi]);
        ps[jj * kPvTok + tt] = p;
    }
    __syncthreads();
    const int tg = threadIdx.x / D, d = threadIdx.x % D;
    float acc[kQc];
#pragma unroll
    for (int jj = 0; jj < kQc; ++jj) acc[jj] = 0.0f;
    for (int tt = tg; tt < kPvTok; tt += TPD) {
        const int64_t t = t0 + tt;
        if (t >= Ttot) break;
        const float v = bf2f(values[(static_cast<int64_t>(g) * cap + t) * D + d]);
#pragma unroll
        for (int jj = 0; jj < kQc; ++jj)
            if (jj < nq) acc[jj] = fmaf(ps[jj * kPvTok + tt], v, acc[jj]);
    }
    if constexpr (TPD > 1) {
#pragma unroll
        for (int jj = 0; jj < kQc; ++jj)
            if (jj < nq) red[(tg * kQc + jj) * D + d] = acc[jj];
        __syncthreads();
        if (tg != 0) return;
#pragma unroll
        for (int jj = 0; jj < kQc; ++jj) {
            if (jj >= nq) continue;
            float s = red[jj * D + d];
            for (int k = 1; k < TPD; ++k) s += red[(k * kQc + jj) * D + d];
            acc[jj] = s;
        }
    }
    const size_t NQall = static_cast<size_t>(S) * A.hq;
    for (int jj = 0; jj < nq; ++jj) {
        const int j = j0 + jj, r = j / G;
        const size_t qi = static_cast<size_t>(r) * A.hq + g * G + j % G;
        B.part[(static_cast<size_t>(tile) * NQall + qi) * D + d] = acc[jj];
    }
}

// attended = T(sum of the tiles' partials, tile order), gated = T(attended * gate).
__global__ __launch_bounds__(256) void k_attn_combine(AttnDev A, AttnBufs B, int S, int64_t T0) {
    const int qi = blockIdx.x, d = threadIdx.x, D = A.d;
    if (d >= D) return;
    const int r = qi / A.hq, h = qi % A.hq;
    const int64_t ntile = (T0 + r + 1 + kPvTok - 1) / kPvTok;
    const size_t NQall = static_cast<size_t>(S) * A.hq;
    float a = 0.0f;
    for (int64_t tile = 0; tile < ntile; ++tile) a += B.part[(static_cast<size_t>(tile) * NQall + qi) * D + d];
    B.gated[static_cast<size_t>(r) * A.hq * D + static_cast<size_t>(h) * D + d] =
        f2bf(tbf(a) * bf2f(B.gs[static_cast<size_t>(qi) * D + d]));
}

template <int D>
hipError_t launch_attn_core(const AttnDev& A, const AttnBufs& B, int S, uint16_t* keys, uint16_t* values, int64_t cap,
                            int64_t T0, int64_t position, int64_t tpad, hipStream_t st) {
    const int HQ = A.hq, HKV = A.hkv, G = HQ / HKV;
    const int64_t Ttot = T0 + S;
    const unsigned qchunks = static_cast<unsigned>((S * G + kQc - 1) / kQc);
    hipError_t e = launch(k_attn_prework<D / 64>, dim3(HQ + 2 * HKV, S), dim3(64), 0, st, A, B, keys, values, cap, T0,
                          position);
    if (e != hipSuccess) return e;
    const size_t lds_s = static_cast<size_t>(kTok) * (D + 8) * 2 + static_cast<size_t>(kQc) * D * 4;
    if ((e = ensure_lds<k_attn_scores<D>>(lds_s)) != hipSuccess) return e;
    e = launch(k_attn_scores<D>, dim3(static_cast<unsigned>((Ttot + kTok - 1) / kTok), HKV, qchunks), dim3(256), lds_s,
               st, A, B, S, static_cast<const uint16_t*>(keys), cap, T0, tpad);
    if (e != hipSuccess) return e;
    e = launch(k_attn_softmax, dim3(S * HQ), dim3(256), 0, st, A, B, T0, tpad);
    if (e != hipSuccess) return e;
    const size_t lds_p = static_cast<size_t>(kQc) * kPvTok * 4 + static_cast<size_t>(256) * kQc * 4;
    if ((e = ensure_lds<k_attn_pv<D>>(lds_p)) != hipSuccess) return e;
    e = launch(k_attn_pv<D>, dim3(static_cast<unsigned>((Ttot + kPvTok - 1) / kPvTok), HKV, qchunks), dim3(256), lds_p,
               st, A, B, S, static_cast<const uint16_t*>(values), cap, T0, tpad);
    if (e != hipSuccess) return e;
    return launch(k_attn_combine, dim3(S * HQ), dim3(256), 0, st, A, B, S, T0);
}

} // namespace

bool attn_geometry_ok(int hidden, int hq, int hkv, int d, int rot) {
    return hidden > 0 && hq > 0 && hkv > 0 && hq % hkv == 0 && (d == 64 || d == 128 || d == 256) && rot > 0 &&
           rot % 2 == 0 && rot <= d;
}

int64_t attn_score_stride(int64_t tokens) { return (tokens + kTok - 1) / kTok * kTok; }
int64_t attn_pv_tiles(int64_t tokens) { return (tokens + kPvTok - 1) / kPvTok; }

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
