// q38_gdn.hip — the GatedDeltaNet verify step: the linear-attention half of a decoder layer
// for S verify rows (1..64) from an origin state, keeping the state after every row as that
// row's checkpoint (GatedDeltaNet::forward_verify, src/gated_delta_net.cpp:657-834).
//
// Five launches:
//   k_affine_rows   the affine projections qkv, z, b (beta) and a (decay) of the S rows in
//                   one launch (q38_affine.hip): a workgroup takes a block of one projection's
//                   weight rows for up to 16 staged rows; outputs rounded to bf16
//                   (quantized_matmul's output);
//   k_gdn_prework   per (row, head): the depthwise width-4 convolution over [origin conv rows ;
//                   qkv rows] and SiLU (T(c * T(sigmoid c))), the q / k RMS norms with the
//                   1/DK and 1/sqrt(DK) scales, v, and per value head beta = T(sigmoid b) and
//                   decay = T(exp(-exp(A_log) * softplus(T(a + dt_bias)))); the conv rows of
//                   every checkpoint;
//   k_gdn_recur     the delta-rule recurrence with the reference's bf16-sum rounding points
//                   (src/gdn_metal_kernels.hpp:498-562): one 64-lane wave per two value rows of
//                   a value head, 32 lanes per row with DK / 32 state items each, the state in
//                   registers across the S rows; every product, lane sum, residual, delta,
//                   update and state value rounded to bf16, the 32 lanes' sums added in float
//                   by an xor butterfly (offsets 16..1) and rounded once; writes y and the
//                   recurrent part of every row's checkpoint;
//   k_gdn_norm_gate per (row, value head): T(w * T(y / rms(y))) times the gate T(sigmoid z)
//                   or SiLU T(z * T(sigmoid z)), rounded (:809, :824-833);
//   k_affine_rows   the output projection.
// A state (q38_gdn_state_bytes) is the conv rows [3][C] bf16 followed by the recurrent state
// [HV][DV][DK] bf16, C = 2 HK DK + HV DV; value head h reads key head h / (HV / HK).
#include "q38_affine.hpp"

namespace q38 {

namespace {

__device__ __forceinline__ float tbf(float v) { return bf2f(f2bf(v)); }
__device__ __forceinline__ float sigmoid_bf(float x) { return tbf(1.0f / (1.0f + expf(-x))); }

// conv + SiLU of row t, channels cb + lane * CPL + i; q / k heads normalised.
template <int CPL>
__global__ __launch_bounds__(64) void k_gdn_prework(GdnDev G, GdnBufs B, int S, const uint16_t* __restrict__ origin,
                                                    uint16_t* __restrict__ ckpt, size_t state_elems) {
    const int head = blockIdx.x, t = blockIdx.y, lane = threadIdx.x;
    const int HK = G.hk, HV = G.hv, DK = G.dk, DV = G.dv, KW = HK * DK, VW = HV * DV, C = 2 * KW + VW;
    const int role = head < HK ? 0 : head < 2 * HK ? 1 : 2;  // q, k, v
    const int h = role == 0 ? head : role == 1 ? head - HK : head - 2 * HK;
    const int cb = role == 0 ? h * DK : role == 1 ? KW + h * DK : 2 * KW + h * DV;
    auto cin = [&](int r, int c) {  // row r of [origin conv rows ; qkv rows]
        if (r >= 3) return bf2f(B.qkv[static_cast<size_t>(r - 3) * C + c]);
        return origin ? bf2f(origin[static_cast<size_t>(r) * C + c]) : 0.0f;
    };
    float act[CPL];
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        const int c = cb + lane * CPL + i;
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) acc = fmaf(bf2f(G.conv_w[static_cast<size_t>(c) * 4 + j]), cin(t + j, c), acc);
        const float cv = tbf(acc);
        act[i] = tbf(cv * sigmoid_bf(cv));
        ss = fmaf(act[i], act[i], ss);
        if (ckpt)
#pragma unroll
            for (int j = 0; j < 3; ++j) ckpt[static_cast<size_t>(t) * state_elems + static_cast<size_t>(j) * C + c] =
                                             f2bf(cin(t + 1 + j, c));
    }
    if (role < 2) {
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
        const float inv = 1.0f / sqrtf(ss / static_cast<float>(DK) + 1e-6f);
        const float scale = role == 0 ? tbf(1.0f / static_cast<float>(DK)) : tbf(1.0f / sqrtf(static_cast<float>(DK)));
        uint16_t* dst = (role == 0 ? B.q : B.k) + static_cast<size_t>(t) * KW + h * DK + lane * CPL;
#pragma unroll
        for (int i = 0; i < CPL; ++i) dst[i] = f2bf(tbf(act[i] * inv) * scale);
    } else {
        uint16_t* dst = B.v + static_cast<size_t>(t) * VW + h * DV + lane * CPL;
#pragma unroll
        for (int i = 0; i < CPL; ++i) dst[i] = f2bf(act[i]);
        if (lane == 0) {
            const size_t at = static_cast<size_t>(t) * HV + h;
            B.beta[at] = sigmoid_bf(bf2f(B.bpr[at]));
            const float biased = tbf(bf2f(B.apr[at]) + bf2f(G.dt_bias[h]));
            const float softplus = log1pf(expf(biased));
            const float rate = expf(G.a_log[h]);
            B.decay[at] = tbf(expf(-(rate * softplus)));
        }
    }
}

// Lane sum of the 32 lanes of each half-wave in float (xor butterfly 16..1), rounded.
__device__ __forceinline__ float half_wave_sum(float v) {
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return tbf(v);
}

template <int ITEMS>
__global__ __launch_bounds__(64) void k_gdn_recur(GdnDev G, GdnBufs B, int S, const uint16_t* __restrict__ origin,
                                                  uint16_t* __restrict__ ckpt, size_t state_elems) {
    const int HK = G.hk, HV = G.hv, DK = G.dk, DV = G.dv, KW = HK * DK, VW = HV * DV, C = 2 * KW + VW;
    const int hv = blockIdx.y, lane = threadIdx.x, sl = lane & 31;
    const int dv = blockIdx.x * 2 + (lane >> 5);
    const int hk = hv / (HV / HK);
    const size_t rec = static_cast<size_t>(3) * C + (static_cast<size_t>(hv) * DV + dv) * DK + sl * ITEMS;
    float st[ITEMS];
    {
        typedef uint16_t items_t __attribute__((ext_vector_type(ITEMS)));
        items_t o0 = {};
        if (origin) o0 = *reinterpret_cast<const items_t*>(origin + rec);
#pragma unroll
        for (int i = 0; i < ITEMS; ++i) st[i] = bf2f(o0[i]);
    }
    // (row t + 1's inputs are requested before row t's arithmetic; a lane's DK / 32 items of
    // k, q and the state are one vector access each)
    static_assert(ITEMS == 2 || ITEMS == 4 || ITEMS == 8, "items per lane");
    typedef uint16_t items_t __attribute__((ext_vector_type(ITEMS)));
    struct RowIn {
        items_t k, q;
        uint16_t v;
        float g, b;
    };
    auto load_row = [&](int t, RowIn& r) {
        const int tt = t < S ? t : S - 1;
        r.k = *reinterpret_cast<const items_t*>(B.k + static_cast<size_t>(tt) * KW + hk * DK + sl * ITEMS);
        r.q = *reinterpret_cast<const items_t*>(B.q + static_cast<size_t>(tt) * KW + hk * DK + sl * ITEMS);
        r.v = B.v[static_cast<size_t>(tt) * VW + hv * DV + dv];
        r.g = B.decay[static_cast<size_t>(tt) * HV + hv];
        r.b = B.beta[static_cast<size_t>(tt) * HV + hv];
    };
    RowIn nxt;
    load_row(0, nxt);
    for (int t = 0; t < S; ++t) {
        const RowIn cur = nxt;
        load_row(t + 1, nxt);
        const float g = cur.g, bt = cur.b;
        float kv[ITEMS], qv[ITEMS];
#pragma unroll
        for (int i = 0; i < ITEMS; ++i) {
            kv[i] = bf2f(cur.k[i]);
            qv[i] = bf2f(cur.q[i]);
        }
        const float vv = bf2f(cur.v);
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < ITEMS; ++i) {
            st[i] = tbf(st[i] * g);
            acc = tbf(acc + tbf(st[i] * kv[i]));
        }
        const float recalled = half_wave_sum(acc);
        const float delta = tbf(tbf(vv - recalled) * bt);
        acc = 0.0f;
#pragma unroll
        for (int i = 0; i < ITEMS; ++i) {
            st[i] = tbf(st[i] + tbf(kv[i] * delta));
            acc = tbf(acc + tbf(st[i] * qv[i]));
        }
        const float y = half_wave_sum(acc);
        if (sl == 0) B.y[static_cast<size_t>(t) * VW + hv * DV + dv] = f2bf(y);
        if (ckpt) {
            typedef uint16_t items_t2 __attribute__((ext_vector_type(ITEMS)));
            items_t2 o;
#pragma unroll
            for (int i = 0; i < ITEMS; ++i) o[i] = f2bf(st[i]);
            *reinterpret_cast<items_t2*>(ckpt + static_cast<size_t>(t) * state_elems + rec) = o;
        }
    }
}

template <int CPL>
__global__ __launch_bounds__(64) void k_gdn_norm_gate(GdnDev G, GdnBufs B, int S) {
    const int hv = blockIdx.x, t = blockIdx.y, lane = threadIdx.x;
    const int DV = G.dv, VW = G.hv * DV;
    const size_t base = static_cast<size_t>(t) * VW + hv * DV + lane * CPL;
    float y[CPL];
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        y[i] = bf2f(B.y[base + i]);
        ss = fmaf(y[i], y[i], ss);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
    const float inv = 1.0f / sqrtf(ss / static_cast<float>(DV) + G.eps);
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        const float nrm = tbf(bf2f(G.norm_w[lane * CPL + i]) * tbf(y[i] * inv));
        const float z = bf2f(B.z[base + i]);
        const float gate = G.gate_silu ? tbf(z * sigmoid_bf(z)) : sigmoid_bf(z);
        B.gated[base + i] = f2bf(nrm * gate);
    }
}

// Lanes per weight row: about four 32-input chunks per lane (16 weight rows per workgroup at
// H = 2048), 8 to 64 lanes.
template <int CPL>
hipError_t launch_prework_t(const GdnDev& G, const GdnBufs& B, int S, const uint16_t* origin, uint16_t* ckpt,
                            size_t state_elems, hipStream_t st) {
    return launch(k_gdn_prework<CPL>, dim3(2 * G.hk + G.hv, S), dim3(64), 0, st, G, B, S, origin, ckpt, state_elems);
}
template <int CPL>
hipError_t launch_norm_gate_t(const GdnDev& G, const GdnBufs& B, int S, hipStream_t st) {
    return launch(k_gdn_norm_gate<CPL>, dim3(G.hv, S), dim3(64), 0, st, G, B, S);
}
template <int ITEMS>
hipError_t launch_recur_t(const GdnDev& G, const GdnBufs& B, int S, const uint16_t* origin, uint16_t* ckpt,
                          size_t state_elems, hipStream_t st) {
    return launch(k_gdn_recur<ITEMS>, dim3(G.dv / 2, G.hv), dim3(64), 0, st, G, B, S, origin, ckpt, state_elems);
}
} // namespace

bool gdn_geometry_ok(const GdnDev& G) {
    // (the prework gives a lane dk / 64 or dv / 64 channels; a recurrence lane dk / 32 items)
    return (G.dk == 64 || G.dk == 128 || G.dk == 256) && G.dk == G.dv && G.hk > 0 && G.hv % G.hk == 0;
}

hipError_t launch_gdn_verify(const GdnDev& G, const GdnBufs& B, int S, const uint16_t* x, const uint16_t* origin,
                             uint16_t* ckpt, uint16_t* out, hipStream_t st) {
    if (!gdn_geometry_ok(G)) return hipErrorInvalidValue;
    const int KW = G.hk * G.dk, VW = G.hv * G.dv, C = 2 * KW + VW;
    const size_t state_elems = static_cast<size_t>(3) * C + static_cast<size_t>(G.hv) * G.dv * G.dk;
    AffineRowSet in{};
    in.n = 4;
    in.p[0] = {G.w[0], G.s[0], G.b[0], B.qkv, C, C, 0};
    in.p[1] = {G.w[1], G.s[1], G.b[1], B.z, VW, VW, 0};
    in.p[2] = {G.w[2], G.s[2], G.b[2], B.bpr, G.hv, G.hv, 0};
    in.p[3] = {G.w[3], G.s[3], G.b[3], B.apr, G.hv, G.hv, 0};
    if (const hipError_t e = launch_affine_rows(in, x, S, G.hidden, G.group, G.bits, G.f16, st); e != hipSuccess) return e;
    hipError_t e = G.dk == 64    ? launch_prework_t<1>(G, B, S, origin, ckpt, state_elems, st)
                   : G.dk == 128 ? launch_prework_t<2>(G, B, S, origin, ckpt, state_elems, st)
                                 : launch_prework_t<4>(G, B, S, origin, ckpt, state_elems, st);
    if (e != hipSuccess) return e;
    e = G.dk == 64    ? launch_recur_t<2>(G, B, S, origin, ckpt, state_elems, st)
        : G.dk == 128 ? launch_recur_t<4>(G, B, S, origin, ckpt, state_elems, st)
                      : launch_recur_t<8>(G, B, S, origin, ckpt, state_elems, st);
    if (e != hipSuccess) return e;
    e = G.dv == 64 ? launch_norm_gate_t<1>(G, B, S, st)
        : G.dv == 128 ? launch_norm_gate_t<2>(G, B, S, st)
                      : launch_norm_gate_t<4>(G, B, S, st);
    if (e != hipSuccess) return e;
    AffineRowSet o{};
    o.n = 1;
    o.p[0] = {G.w[4], G.s[4], G.b[4], out, G.hidden, G.hidden, 0};
    return launch_affine_rows(o, B.gated, S, VW, G.group, G.bits, G.f16, st);
}

} // namespace q38
