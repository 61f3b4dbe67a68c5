// q38_oracle.cpp — CPU restatement of the qwen38-flash.cpp MTP verification round.
//
// TEST INFRASTRUCTURE ONLY. Nothing in the product library links, loads or calls this
// file; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it,
// and only as the checker (or the timed CPU baseline), never as the thing measured on
// the GPU.
//
// Every function cites the reference file:line it restates (paths relative to the
// reference checkout). Where the reference leaves an arithmetic detail to a third-party
// library (MLX's BF16 matmul, softmax, quantized_matmul) this file states the
// deterministic contract that the HIP kernels implement bit-for-bit, and the contract
// is named as such.
//
// Pins (tests/test_oracle_*.py):
//   pack/unpack            KAT from tests/quantization_geometry_test.cpp:48-84 and the
//                          compiled reference (oracle/_ref) on random codes.
//   decide_greedy / commit KAT from tests/mtp_lifecycle_test.cpp:39-71,
//                          tests/mlx_backend_test.cpp:711-769 and oracle/_ref.
//   router                 closed forms: all-equal logits -> experts 0..k-1 weight 1/k,
//                          planted top-k, ties -> lower index; brute force vs numpy.
//   VQ decode / MoE        closed-form banks of tests/vq_geometry_gpu_test.cpp:24-57;
//                          one-hot / zero codebooks; dense numpy float64 recomputation.
//   LM head                exact integer-product check vs numpy float64 + near-tie KAT.
//   Philox4x32-10          Random123 known-answer vectors.
//   rejection sampling     invariants (p == q accepts all; p(d) = 0 rejects); chi-square
//                          tests at k = 3 that every emitted position follows its p_i, that
//                          the draw after a first rejection at i follows norm(max(0, p_i -
//                          q_i)) and the all-accepted bonus follows p_k, and the acceptance
//                          rate sum_x min(p_i, q_i); planted wrong-row draws fail them.
//   residual add           float32 numpy restatement with its own RNE (ties, overflow,
//                          signed zeros, subnormals).
//   exp contract           error bound vs math.exp over the whole reduced range.
//   per-dim INT8/U8 books  independent numpy restatement (bit-exact tables and decode),
//                          closed forms (min/max round trip, lround ties away from zero,
//                          clamps, constant dimension), float64 numpy layer recomputation.
//   Q4 draft head          closed forms (nibble order, sign, group scales), numpy splitmix64
//                          regeneration + float64 logits.
//   RMSNorm                bit-exact float64 numpy restatement, closed forms, invariants.
//   HyperConnection mixer  independent numpy restatement, closed forms (zero and bias-only
//                          projections, packed-value order, the 1 + w norm weight, sign-only
//                          streams, injection of 1 and 2 in the write).
//   GatedDeltaNet verify   independent numpy restatement (float64 state, vectorised per
//                          head), closed forms (one row from a zero state: state = beta v k^T,
//                          output beta v (k . q); beta 0: the state decays by g per row;
//                          decay 1, beta 1 and a one-hot key: the delta rule replaces that
//                          column of the state by v), S rows = S single-row calls chained
//                          through the checkpoints; a planted wrong key-head mapping fails them.
//   attention verify       independent numpy restatement (float64, numpy cos / sin, the
//                          rotation as a 2 x 2 matrix per pair), closed forms (the bf16 RoPE
//                          table at position 0 and at R = 2; with an identity o_proj and zero
//                          gates: a zero query gives the mean of the visible values / 2, a
//                          one-hot query matched by one large key reads that token's value),
//                          S rows = S single-row calls through the cache; planted RoPE-pairing
//                          and causal-mask faults fail them.
//   MLP output map         closed forms (identity full map: out = y; zero right factor: out = y;
//                          rank-1 one-hot factors: column b gains column a, a transposed factor
//                          fails), float64 numpy within tolerance.

#include <pthread.h>
#include <sched.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <condition_variable>
#include <cstdint>
#include <cstring>
#include <functional>
#include <limits>
#include <mutex>
#include <numeric>
#include <thread>
#include <vector>

namespace {

// ---------------------------------------------------------------- number formats

inline uint32_t f32_bits(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }
inline float bits_f32(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }

inline uint16_t f32_to_bf16(float f) {
    uint32_t x = f32_bits(f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((x >> 16) | 0x40u);
    x += 0x7fffu + ((x >> 16) & 1u);
    return static_cast<uint16_t>(x >> 16);
}
inline float bf16_to_f32(uint16_t h) { return bits_f32(static_cast<uint32_t>(h) << 16); }
inline float rbf16(double v) { return bf16_to_f32(f32_to_bf16(static_cast<float>(v))); }

inline uint16_t f32_to_f16(float f) {
    uint32_t x = f32_bits(f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    x &= 0x7fffffffu;
    if (x >= 0x7f800000u) return static_cast<uint16_t>(sign | (x > 0x7f800000u ? 0x7e00u : 0x7c00u));
    if (x >= 0x477ff000u) return static_cast<uint16_t>(sign | 0x7c00u);
    if (x < 0x38800000u) {
        if (x < 0x33000000u) return static_cast<uint16_t>(sign);
        const uint32_t m = (x & 0x7fffffu) | 0x800000u;
        const uint32_t e = x >> 23;
        const uint32_t shift = 126u - e;
        uint32_t r = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (r & 1u))) ++r;
        return static_cast<uint16_t>(sign | r);
    }
    const uint32_t r = (x - 0x38000000u + 0xfffu + ((x >> 13) & 1u)) >> 13;
    return static_cast<uint16_t>(sign | r);
}
inline float f16_to_f32(uint16_t h) {
    const uint32_t sign = (static_cast<uint32_t>(h) & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    if (e == 0) {
        if (m == 0) return bits_f32(sign);
        // subnormal: m * 2^-24
        const float v = static_cast<float>(m) * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    if (e == 31) return bits_f32(sign | 0x7f800000u | (m << 13));
    return bits_f32(sign | ((e + 112u) << 23) | (m << 13));
}

// ---------------------------------------------------------------- synthetic generator
// Counter-based splitmix64 streams, so that any element can be regenerated alone (the
// device generator produces the same values in parallel). This is the measurement
// input generator, not a reference algorithm.

constexpr uint64_t kGolden = 0x9E3779B97F4A7C15ull;

inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
inline uint64_t stream_key(uint64_t seed, uint64_t layer, uint64_t tensor) {
    return mix64(mix64(mix64(seed) + kGolden * (layer + 1)) + kGolden * (tensor + 1));
}
inline uint64_t bits_at(uint64_t key, uint64_t i) { return mix64(key + kGolden * (i + 1)); }

inline double normal_at(uint64_t key, uint64_t i) {
    const double u1 = static_cast<double>((bits_at(key, 2 * i) >> 11) + 1) * 0x1.0p-53;
    const double u2 = static_cast<double>(bits_at(key, 2 * i + 1) >> 11) * 0x1.0p-53;
    return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
}
inline double uniform_at(uint64_t key, uint64_t i) {
    return static_cast<double>(bits_at(key, i) >> 11) * 0x1.0p-53;
}

// ---------------------------------------------------------------- geometry (R4)
// src/quantization_geometry.cpp:37-48 (packed_vq_word_count) and :50-67 (unpack_vq_code):
// 32-code blocks, each occupying BITS 32-bit words, code q of a block at bit q*BITS,
// LSB-first, possibly straddling two words.

inline int64_t word_count(int64_t n, int bits) {
    if (bits <= 0 || bits > 31 || n < 0) return -1;
    return ((n + 31) / 32) * bits;
}
inline uint32_t unpack(const uint32_t* words, int64_t i, int bits) {
    const int64_t bit = (i % 32) * bits;
    const int64_t w = (i / 32) * bits + bit / 32;
    const int shift = static_cast<int>(bit % 32);
    uint64_t v = static_cast<uint64_t>(words[w]) >> shift;
    if (shift + bits > 32) v |= static_cast<uint64_t>(words[w + 1]) << (32 - shift);
    return static_cast<uint32_t>(v & ((uint64_t{1} << bits) - 1));
}
inline void pack(const uint32_t* codes, int64_t n, int bits, uint32_t* words) {
    const int64_t nw = word_count(n, bits);
    std::fill(words, words + nw, 0u);
    for (int64_t i = 0; i < n; ++i) {
        const int64_t bit = (i % 32) * bits;
        const int64_t w = (i / 32) * bits + bit / 32;
        const int shift = static_cast<int>(bit % 32);
        const uint64_t v = static_cast<uint64_t>(codes[i]) << shift;
        words[w] |= static_cast<uint32_t>(v);
        if (shift + bits > 32) words[w + 1] |= static_cast<uint32_t>(v >> 32);
    }
}

// ---------------------------------------------------------------- exp contract
// The reference router takes std::exp of float (src/sparse_moe.cpp:1049); libm's
// last-bit behaviour is platform specific, so the build fixes its own: Cody-Waite
// reduction x = k*ln2 + r (k = rint(x*log2 e), ln2 split hi/lo) and a degree-7 Taylor
// polynomial in Horner form with fused multiply-adds, scaled by 2^k. Results below
// 2^-125 are flushed to zero. The HIP router evaluates the same float operations.
inline float exp_contract(float d) {
    if (!(d > -87.0f)) return 0.0f;
    const float kf = std::rint(d * 1.44269504088896341f);
    float r = std::fma(kf, -0.693145751953125f, d);
    r = std::fma(kf, -1.42860682030941723212e-06f, r);
    float p = 1.0f / 5040.0f;
    p = std::fma(p, r, 1.0f / 720.0f);
    p = std::fma(p, r, 1.0f / 120.0f);
    p = std::fma(p, r, 1.0f / 24.0f);
    p = std::fma(p, r, 1.0f / 6.0f);
    p = std::fma(p, r, 0.5f);
    p = std::fma(p, r, 1.0f);
    p = std::fma(p, r, 1.0f);
    const int k = static_cast<int>(kf);
    if (k < -125) return 0.0f;
    return std::ldexp(p, k);
}

// ---------------------------------------------------------------- router logit contract (R1)
// Reference: SparseMoe::router_logits -> project_linear (src/sparse_moe.cpp:945-960), a BF16
// x * Wr^T whose FP32 accumulation order is MLX's. Contract (shared with the HIP kernel):
// 64 partial sums, partial l accumulates c = 512t + 8l + j for t = 0.., j = 0..7 in that
// order with fmaf (each bf16*bf16 product is exact in float); the partials are then
// combined by an xor butterfly over offsets 32,16,8,4,2,1; the result is rounded to BF16.
inline float dot_contract(const uint16_t* x, const uint16_t* w, int H) {
    float part[64];
    for (int l = 0; l < 64; ++l) {
        float acc = 0.0f;
        for (int t = 0; t < H / 512; ++t)
            for (int j = 0; j < 8; ++j) {
                const int c = 512 * t + 8 * l + j;
                acc = std::fma(bf16_to_f32(x[c]), bf16_to_f32(w[c]), acc);
            }
        part[l] = acc;
    }
    for (int off = 32; off >= 1; off >>= 1) {
        float next[64];
        for (int l = 0; l < 64; ++l) next[l] = part[l] + part[l ^ off];
        std::memcpy(part, next, sizeof(part));
    }
    return part[0];
}

// ---------------------------------------------------------------- routing (R2)
// SparseMoe::route_decode_batch (src/sparse_moe.cpp:1032-1086): softmax with max
// subtraction, float exponentials, a double denominator, float probabilities,
// partial_sort by (p desc, index asc), then weights = p / sum of selected p (float, in
// rank order) when normalize_topk_probability. Contract refinements: exp_contract above,
// and the double denominator is summed as 64 lane partials (lane l adds e[64j + l] for
// j = 0.. in order) joined by the same xor butterfly (the reference sums sequentially;
// the difference is below one double ulp of the sum).
void route_rows(const float* logits, int M, int E, int k, int normalize,
                int32_t* experts, float* weights) {
    std::vector<float> e(E), p(E);
    for (int r = 0; r < M; ++r) {
        const float* l = logits + static_cast<int64_t>(r) * E;
        float mx = l[0];
        for (int i = 1; i < E; ++i) mx = std::max(mx, l[i]);
        for (int i = 0; i < E; ++i) e[i] = exp_contract(l[i] - mx);
        double part[64];
        for (int ln = 0; ln < 64; ++ln) {
            double acc = 0.0;
            for (int j = 0; j * 64 + ln < E; ++j) acc += static_cast<double>(e[j * 64 + ln]);
            part[ln] = acc;
        }
        for (int off = 32; off >= 1; off >>= 1) {
            double next[64];
            for (int ln = 0; ln < 64; ++ln) next[ln] = part[ln] + part[ln ^ off];
            std::memcpy(part, next, sizeof(part));
        }
        const double denom = part[0];
        for (int i = 0; i < E; ++i) p[i] = static_cast<float>(static_cast<double>(e[i]) / denom);
        std::vector<int> order(E);
        std::iota(order.begin(), order.end(), 0);
        std::partial_sort(order.begin(), order.begin() + k, order.end(), [&](int a, int b) {
            if (p[a] != p[b]) return p[a] > p[b];
            return a < b;
        });
        float sum = 0.0f;
        for (int s = 0; s < k; ++s) sum += p[order[s]];
        for (int s = 0; s < k; ++s) {
            experts[r * k + s] = order[s];
            weights[r * k + s] = normalize ? p[order[s]] / sum : p[order[s]];
        }
    }
}

// ---------------------------------------------------------------- route plan (R3)
// Gather-by-expert: the reference's wide path stable-sorts flat routes r*k+slot by expert
// (src/sparse_moe.cpp:2264-2271) and derives inverse_order (:2336-2345). The build uses
// the same plan at every width: unique experts ascending, each with its routes in
// ascending (row, slot) order.
int route_plan(const int32_t* experts, int M, int k, int E, int32_t* n_unique, int32_t* uexp,
               int32_t* uoff, int32_t* route_list, int32_t* route_pos) {
    const int R = M * k;
    std::vector<int> count(E, 0);
    for (int i = 0; i < R; ++i) {
        if (experts[i] < 0 || experts[i] >= E) return -1;
        ++count[experts[i]];
    }
    int nu = 0, off = 0;
    std::vector<int> start(E, 0);
    for (int e = 0; e < E; ++e) {
        if (!count[e]) continue;
        uexp[nu] = e;
        uoff[nu] = off;
        start[e] = off;
        off += count[e];
        ++nu;
    }
    uoff[nu] = off;
    *n_unique = nu;
    std::vector<int> fill(start);
    for (int i = 0; i < R; ++i) {
        const int pos = fill[experts[i]]++;
        route_list[pos] = i;
        route_pos[i] = pos;
    }
    return 0;
}

// ---------------------------------------------------------------- MoE layer (R5-R11)

struct Desc {  // field order is part of the ctypes contract (tests/oracle.py)
    int32_t hidden, inter, experts, top_k;
    int32_t gu_dim, gu_bits, down_dim, down_bits;
    int32_t gu_group, down_group;   // scale group along IN; == IN means one scale per row
    int32_t normalize, has_shared;
    int32_t mixed;                  // 1: even experts d4/8-bit FP16, odd d8/14-bit INT8 codebook
    int32_t book_format;            // 0: FP16 books; 2: per-dimension INT8/U8 books (d8/14 projections)
};

struct Proj {  // one projection of one expert, host pointers
    const uint32_t* codes;   // [OUT, words] (words = word_count(IN/D, BITS))
    const uint16_t* scales;  // [OUT, IN/G] fp16
    const float* book;       // [K, D] dequantized codebook values
    int in, out, dim, bits, group;
};

// Dense row o of a projection: W[o, c] = scale[o, c/G] * book[code(o, c/D)*D + c%D]
// (src/vq_metal_kernels.hpp:396-427; tests/vq_geometry_gpu_test.cpp:48-50), dotted with a
// float vector in double: per scale group sum x*book, times the group scale
// (src/vq_metal_kernels.hpp:493-588).
inline double proj_row_dot(const Proj& P, int o, const float* x) {
    const int nsub = P.in / P.dim;
    const int64_t words = word_count(nsub, P.bits);
    const uint32_t* row = P.codes + static_cast<int64_t>(o) * words;
    const int ngrp = P.in / P.group;
    double acc = 0.0;
    for (int g = 0; g < ngrp; ++g) {
        double gacc = 0.0;
        const int s0 = g * P.group / P.dim, s1 = (g + 1) * P.group / P.dim;
        for (int s = s0; s < s1; ++s) {
            const uint32_t code = unpack(row, s, P.bits);
            const float* b = P.book + static_cast<int64_t>(code) * P.dim;
            for (int d = 0; d < P.dim; ++d) gacc += static_cast<double>(x[s * P.dim + d]) * b[d];
        }
        acc += static_cast<double>(f16_to_f32(P.scales[static_cast<int64_t>(o) * ngrp + g])) * gacc;
    }
    return acc;
}

struct ExpertWeights { Proj gate, up, down; };

// One expert applied to one input row: SwiGLU with the reference's rounding points
// (gate/up rounded to T, T(silu(g)) * up rounded to T: src/vq_metal_kernels.hpp:589-595),
// then the down projection rounded to T per route (:753-756). Output: T(down) as float.
void expert_forward(const ExpertWeights& W, const float* x, float* dout) {
    const int I = W.gate.out, H = W.down.out;
    std::vector<float> h(I);
    for (int o = 0; o < I; ++o) {
        const float g = rbf16(proj_row_dot(W.gate, o, x));
        const float u = rbf16(proj_row_dot(W.up, o, x));
        const float s = rbf16(static_cast<double>(g) / (1.0 + std::exp(-static_cast<double>(g))));
        h[o] = rbf16(static_cast<double>(s) * u);
    }
    for (int o = 0; o < H; ++o) dout[o] = rbf16(proj_row_dot(W.down, o, h.data()));
}

// Shared expert in MLX affine form (the reference checkpoints' shared experts: the affine
// branch of SparseMoe::load_projection, src/sparse_moe.cpp:662-700, applied by
// SparseMoe::forward_shared, :1306-1313, through quantized_matmul). Row o of a [OUT, IN]
// projection: values q in [0, 2^bits) packed LSB-first in 32-bit words (32 / bits per word),
// w[o, c] = scale[o, c / G] * q[o, c] + bias[o, c / G] with bf16 (fmt 0) or fp16 (fmt 1) scales
// and biases. The dot product is taken per group as scale * sum(q x) + bias * sum(x), in
// double.
struct AffineProj {
    const uint32_t* w;
    const uint16_t* s;
    const uint16_t* b;
    int in, out, bits, group, fmt;
};
inline double affine_param(uint16_t v, int fmt) { return fmt ? f16_to_f32(v) : bf16_to_f32(v); }
inline double affine_row_dot(const AffineProj& P, int o, const float* x) {
    const int vpw = 32 / P.bits, ngrp = P.in / P.group;
    const uint32_t mask = (1u << P.bits) - 1u;
    const uint32_t* row = P.w + static_cast<size_t>(o) * (P.in / vpw);
    double acc = 0.0;
    for (int g = 0; g < ngrp; ++g) {
        double qx = 0.0, sx = 0.0;
        for (int c = g * P.group; c < (g + 1) * P.group; ++c) {
            const uint32_t q = (row[c / vpw] >> ((c % vpw) * P.bits)) & mask;
            qx += static_cast<double>(q) * x[c];
            sx += x[c];
        }
        acc += affine_param(P.s[static_cast<size_t>(o) * ngrp + g], P.fmt) * qx +
               affine_param(P.b[static_cast<size_t>(o) * ngrp + g], P.fmt) * sx;
    }
    return acc;
}
struct AffineExpert { AffineProj gate, up, down; };
// forward_shared's rounding points: gate and up T (quantized_matmul outputs), T(silu), the
// product T, the down projection T (the shared gate and the merge follow in moe_layer).
void affine_expert_forward(const AffineExpert& W, const float* x, float* dout) {
    const int I = W.gate.out, H = W.down.out;
    std::vector<float> h(I);
    for (int o = 0; o < I; ++o) {
        const float g = rbf16(affine_row_dot(W.gate, o, x));
        const float u = rbf16(affine_row_dot(W.up, o, x));
        const float sg = rbf16(static_cast<double>(g) / (1.0 + std::exp(-static_cast<double>(g))));
        h[o] = rbf16(static_cast<double>(sg) * u);
    }
    for (int o = 0; o < H; ++o) dout[o] = rbf16(affine_row_dot(W.down, o, h.data()));
}

struct LayerSource {
    virtual ~LayerSource() = default;
    virtual const uint16_t* router() = 0;       // [E, H] bf16
    virtual const uint16_t* wsg() = 0;          // [H] bf16 (may be null without shared)
    virtual ExpertWeights expert(int e) = 0;    // e == E: shared expert
    // the shared expert in affine form instead of expert(E), when the layer has one
    virtual const AffineExpert* shared_affine() { return nullptr; }
};

// Persistent worker pool: workers are created on first use, each pinned to one CPU of the
// process's affinity mask (worker t to the (t+1)-th allowed CPU, the caller's thread runs
// items too and is not pinned), and wait on a condition variable between jobs. One job at a
// time (callers serialise on `run_mu`); items are handed out by an atomic counter.
class Pool {
public:
    static Pool& get() {
        static Pool p;
        return p;
    }
    void run(int n, int threads, const std::function<void(int)>& f) {
        std::lock_guard<std::mutex> run_lock(run_mu_);
        const int helpers = std::min(threads, n) - 1;
        grow(helpers);
        std::atomic<int> next{0};
        const std::function<void()> body = [&] {
            for (int i = next.fetch_add(1); i < n; i = next.fetch_add(1)) f(i);
        };
        {
            std::lock_guard<std::mutex> lk(mu_);
            job_ = &body;
            active_ = helpers;
            pending_ = helpers;
            ++gen_;
        }
        cv_.notify_all();
        body();
        std::unique_lock<std::mutex> lk(mu_);
        done_cv_.wait(lk, [&] { return pending_ == 0; });
        job_ = nullptr;
    }
    ~Pool() {
        {
            std::lock_guard<std::mutex> lk(mu_);
            stop_ = true;
            ++gen_;
        }
        cv_.notify_all();
        for (auto& t : workers_) t.join();
    }

private:
    void grow(int want) {
        while (static_cast<int>(workers_.size()) < want) {
            const int id = static_cast<int>(workers_.size());
            workers_.emplace_back([this, id] { loop(id); });
            pin(workers_.back(), id + 1);
        }
    }
    static void pin(std::thread& t, int ordinal) {
        cpu_set_t allowed;
        CPU_ZERO(&allowed);
        if (sched_getaffinity(0, sizeof(allowed), &allowed) != 0) return;
        const int n = CPU_COUNT(&allowed);
        if (n == 0) return;
        int want = ordinal % n;
        for (int c = 0; c < CPU_SETSIZE; ++c) {
            if (!CPU_ISSET(c, &allowed)) continue;
            if (want-- == 0) {
                cpu_set_t one;
                CPU_ZERO(&one);
                CPU_SET(c, &one);
                pthread_setaffinity_np(t.native_handle(), sizeof(one), &one);
                return;
            }
        }
    }
    void loop(int id) {
        uint64_t seen = 0;
        for (;;) {
            const std::function<void()>* job = nullptr;
            {
                std::unique_lock<std::mutex> lk(mu_);
                cv_.wait(lk, [&] { return stop_ || (gen_ != seen && id < active_); });
                if (stop_) return;
                seen = gen_;
                job = job_;
            }
            (*job)();
            std::lock_guard<std::mutex> lk(mu_);
            if (--pending_ == 0) done_cv_.notify_one();
        }
    }
    std::mutex run_mu_, mu_;
    std::condition_variable cv_, done_cv_;
    std::vector<std::thread> workers_;
    const std::function<void()>* job_ = nullptr;
    int active_ = 0, pending_ = 0;
    uint64_t gen_ = 0;
    bool stop_ = false;
};

template <class F>
void parallel_for(int n, int threads, F&& f) {
    if (threads <= 1 || n <= 1) {
        for (int i = 0; i < n; ++i) f(i);
        return;
    }
    const std::function<void(int)> fn(std::ref(f));
    Pool::get().run(n, threads, fn);
}

// SparseMoe::forward_verify on the fused-VQ path (src/sparse_moe.cpp:2199-2247 routing,
// 2508-2610 gate/up and down-reduce, 2611-2623 shared + merge) with the routing contract
// of route_decode_batch and the shared expert of forward_shared (:1306-1313) as a VQ
// expert gated by sigmoid(x . w_sg).
// Rounding points: routed = T(sum_slot w_slot * T(down_slot)) in slot order (accumulated in
// double here), shared = T(T(down_shared) * T(sigmoid(T(x . w_sg)))), y = T(routed + shared).
int moe_layer(const Desc& d, LayerSource& src, const uint16_t* x, int M, uint16_t* y,
              int32_t* experts_out, float* weights_out, float* logits_out, int threads,
              const float* bias = nullptr) {
    const int H = d.hidden, E = d.experts, k = d.top_k;
    if (H % 512 != 0 || E % 64 != 0 || k < 1 || k > E || M < 1) return -1;
    const uint16_t* Wr = src.router();
    std::vector<float> logits(static_cast<size_t>(M) * E);
    parallel_for(E, threads, [&](int e) {
        for (int r = 0; r < M; ++r) {
            const float lg = rbf16(dot_contract(x + static_cast<size_t>(r) * H, Wr + static_cast<size_t>(e) * H, H));
            logits[static_cast<size_t>(r) * E + e] = bias ? lg + bias[e] : lg;
        }
    });
    std::vector<int32_t> ex(static_cast<size_t>(M) * k);
    std::vector<float> wt(static_cast<size_t>(M) * k);
    route_rows(logits.data(), M, E, k, d.normalize, ex.data(), wt.data());
    if (experts_out) std::copy(ex.begin(), ex.end(), experts_out);
    if (weights_out) std::copy(wt.begin(), wt.end(), weights_out);
    if (logits_out) std::copy(logits.begin(), logits.end(), logits_out);

    std::vector<float> xf(static_cast<size_t>(M) * H);
    for (size_t i = 0; i < xf.size(); ++i) xf[i] = bf16_to_f32(x[i]);
    const int n_routes = M * k + (d.has_shared ? M : 0);
    std::vector<float> dout(static_cast<size_t>(n_routes) * H);
    // Experts are materialised serially (a generating source is not thread-safe),
    // then applied in parallel.
    std::vector<int> uniq(ex.begin(), ex.end());
    std::sort(uniq.begin(), uniq.end());
    uniq.erase(std::unique(uniq.begin(), uniq.end()), uniq.end());
    const AffineExpert* sa = d.has_shared ? src.shared_affine() : nullptr;
    if (d.has_shared && !sa) uniq.push_back(E);
    std::vector<ExpertWeights> ew(uniq.size());
    std::vector<int> slot_of(E + 1, -1);
    for (size_t u = 0; u < uniq.size(); ++u) { ew[u] = src.expert(uniq[u]); slot_of[uniq[u]] = static_cast<int>(u); }
    parallel_for(n_routes, threads, [&](int i) {
        const int r = i < M * k ? i / k : i - M * k;
        const int e = i < M * k ? ex[i] : E;
        if (e == E && sa)
            affine_expert_forward(*sa, xf.data() + static_cast<size_t>(r) * H, dout.data() + static_cast<size_t>(i) * H);
        else
            expert_forward(ew[slot_of[e]], xf.data() + static_cast<size_t>(r) * H, dout.data() + static_cast<size_t>(i) * H);
    });
    const uint16_t* wsg = d.has_shared ? src.wsg() : nullptr;
    for (int r = 0; r < M; ++r) {
        float sg = 0.0f;
        if (d.has_shared) {
            const float lg = rbf16(dot_contract(x + static_cast<size_t>(r) * H, wsg, H));
            sg = rbf16(1.0 / (1.0 + std::exp(-static_cast<double>(lg))));
        }
        for (int o = 0; o < H; ++o) {
            double routed = 0.0;
            for (int s = 0; s < k; ++s)
                routed += static_cast<double>(wt[r * k + s]) * dout[static_cast<size_t>(r * k + s) * H + o];
            const float rt = rbf16(routed);
            float out = rt;
            if (d.has_shared) {
                const float sh = rbf16(static_cast<double>(dout[static_cast<size_t>(M * k + r) * H + o]) * sg);
                out = rbf16(static_cast<double>(rt) + sh);
            }
            y[static_cast<size_t>(r) * H + o] = f32_to_bf16(out);
        }
    }
    return 0;
}

// ---------------------------------------------------------------- synthetic layer source

enum Tensor : uint64_t {
    T_ROUTER = 1, T_WSG = 2, T_CB_GATE = 3, T_CB_UP = 4, T_CB_DOWN = 5,
    T_CODES_GATE = 6, T_CODES_UP = 7, T_CODES_DOWN = 8,
    T_SCALE_GATE = 9, T_SCALE_UP = 10, T_SCALE_DOWN = 11,
    T_CB4_GATE = 12, T_CB4_UP = 13, T_CB4_DOWN = 14,
    T_X = 20, T_EMBED = 21,
    T_HEAD_W = 30, T_HEAD_S = 31, T_DRAFT_W = 32, T_DRAFT_S = 33,
};
constexpr uint64_t kEmbedLayer = 0xFFFF, kHeadLayer = 0xFFFE, kDraftLayer = 0xFFFD;

inline uint16_t normal_bf16(uint64_t key, uint64_t i, double sd) {
    return f32_to_bf16(static_cast<float>(normal_at(key, i) * sd));
}
inline uint16_t normal_f16(uint64_t key, uint64_t i, double sd) {
    return f32_to_f16(static_cast<float>(normal_at(key, i) * sd));
}
inline uint16_t uniform_f16(uint64_t key, uint64_t i, double lo, double hi) {
    return f32_to_f16(static_cast<float>(lo + uniform_at(key, i) * (hi - lo)));
}
inline uint32_t code_at(uint64_t key, uint64_t e, uint64_t out, uint64_t o, uint64_t s, int bits) {
    return static_cast<uint32_t>(bits_at(key, (e * out + o) * 1024 + s) >> (64 - bits));
}

// Codebook values of the synthetic layer. FP16 ~N(0,1). The mixed layout's d8 book is the
// "approximate INT8 codebook with one FP16 scale per codebook": scale = f16(max|v|/127),
// q = clamp(rint(v/scale), -127, 127), value = q * scale.
void synth_book(uint64_t key, int K, int D, bool int8, std::vector<float>& vals,
                std::vector<uint16_t>* raw_f16, std::vector<int8_t>* raw_i8, uint16_t* scale_out) {
    const int n = K * D;
    std::vector<uint16_t> h(n);
    for (int i = 0; i < n; ++i) h[i] = normal_f16(key, i, 1.0);
    vals.resize(n);
    if (!int8) {
        for (int i = 0; i < n; ++i) vals[i] = f16_to_f32(h[i]);
        if (raw_f16) *raw_f16 = h;
        return;
    }
    float mx = 0.0f;
    for (int i = 0; i < n; ++i) mx = std::max(mx, std::fabs(f16_to_f32(h[i])));
    const uint16_t sc16 = f32_to_f16(mx / 127.0f);
    const float sc = f16_to_f32(sc16);
    if (scale_out) *scale_out = sc16;
    if (raw_i8) raw_i8->resize(n);
    for (int i = 0; i < n; ++i) {
        float q = std::rint(f16_to_f32(h[i]) / sc);
        q = std::min(127.0f, std::max(-127.0f, q));
        if (raw_i8) (*raw_i8)[i] = static_cast<int8_t>(q);
        vals[i] = q * sc;
    }
}

// SparseMoe::prepare_u8_codebook (src/sparse_moe.cpp:750-804): per-dimension min/max of the
// FP16 book (as float), scale = (max - min) / 255 (1 when not > 0); centred (the gate book):
// q = clamp(lround(v / scale), -128, 127); affine (up, down): q = clamp(lround((v - min) /
// scale), 0, 255); scales and biases (= min) stored as FP16. The kernels decode in float
// (src/vq_metal_kernels.hpp:564-579): w = q * f16(scale) (+ f16(min) when affine).
void prepare_u8_book(const uint16_t* book16, int K, int D, bool centered, std::vector<int32_t>& q,
                     std::vector<uint16_t>& s16, std::vector<uint16_t>& b16, std::vector<float>& vals) {
    std::vector<float> mn(D, std::numeric_limits<float>::infinity()), mx(D, -std::numeric_limits<float>::infinity());
    for (int r = 0; r < K; ++r)
        for (int d = 0; d < D; ++d) {
            const float v = f16_to_f32(book16[static_cast<size_t>(r) * D + d]);
            mn[d] = std::min(mn[d], v);
            mx[d] = std::max(mx[d], v);
        }
    std::vector<float> sc(D);
    s16.resize(D);
    b16.resize(D);
    for (int d = 0; d < D; ++d) {
        sc[d] = (mx[d] - mn[d]) / 255.0F;
        if (!(sc[d] > 0.0F)) sc[d] = 1.0F;
        s16[d] = f32_to_f16(sc[d]);
        b16[d] = f32_to_f16(mn[d]);
    }
    const size_t n = static_cast<size_t>(K) * D;
    q.resize(n);
    vals.resize(n);
    for (size_t i = 0; i < n; ++i) {
        const int d = static_cast<int>(i % D);
        const float v = f16_to_f32(book16[i]);
        const long r = centered ? std::lround(v / sc[d]) : std::lround((v - mn[d]) / sc[d]);
        q[i] = static_cast<int32_t>(centered ? std::clamp<long>(r, -128, 127) : std::clamp<long>(r, 0, 255));
        vals[i] = static_cast<float>(q[i]) * f16_to_f32(s16[d]);
        if (!centered) vals[i] = vals[i] + f16_to_f32(b16[d]);
    }
}
// The book the kernels read for projection p: the FP16 values, or with book_format 2 and a
// d8/14-bit projection the decoded per-dimension INT8 (gate) / U8 (up, down) book
// (src/sparse_moe.cpp:528-544).
void layer_book(const Desc& d, int p, const uint16_t* book16, int K, int D, int bits, std::vector<float>& vals) {
    if (d.book_format == 2 && D == 8 && bits == 14) {
        std::vector<int32_t> q;
        std::vector<uint16_t> s16, b16;
        prepare_u8_book(book16, K, D, p == 0, q, s16, b16, vals);
        return;
    }
    vals.resize(static_cast<size_t>(K) * D);
    for (size_t i = 0; i < vals.size(); ++i) vals[i] = f16_to_f32(book16[i]);
}

struct SynthSource final : LayerSource {
    Desc d;
    uint64_t seed, layer;
    std::vector<uint16_t> wr, ws;
    std::vector<float> book8[3], book4[3];
    std::vector<std::vector<uint32_t>> codes;   // kept alive for returned views
    std::vector<std::vector<uint16_t>> scales;

    SynthSource(const Desc& dd, uint64_t s, uint64_t l) : d(dd), seed(s), layer(l) {
        const uint64_t cbt[3] = {T_CB_GATE, T_CB_UP, T_CB_DOWN};
        const uint64_t cb4[3] = {T_CB4_GATE, T_CB4_UP, T_CB4_DOWN};
        if (d.mixed) {
            for (int p = 0; p < 3; ++p) {
                synth_book(stream_key(seed, layer, cbt[p]), 16384, 8, true, book8[p], nullptr, nullptr, nullptr);
                synth_book(stream_key(seed, layer, cb4[p]), 256, 4, false, book4[p], nullptr, nullptr, nullptr);
            }
        } else {
            const int dims[3] = {d.gu_dim, d.gu_dim, d.down_dim};
            const int bits[3] = {d.gu_bits, d.gu_bits, d.down_bits};
            for (int p = 0; p < 3; ++p) {
                std::vector<uint16_t> raw;
                std::vector<float> fp16_vals;
                synth_book(stream_key(seed, layer, cbt[p]), 1 << bits[p], dims[p], false, fp16_vals, &raw, nullptr,
                           nullptr);
                layer_book(d, p, raw.data(), 1 << bits[p], dims[p], bits[p], book8[p]);
            }
        }
    }
    const uint16_t* router() override {
        if (wr.empty()) {
            const uint64_t key = stream_key(seed, layer, T_ROUTER);
            wr.resize(static_cast<size_t>(d.experts) * d.hidden);
            for (size_t i = 0; i < wr.size(); ++i) wr[i] = normal_bf16(key, i, 0.02);
        }
        return wr.data();
    }
    const uint16_t* wsg() override {
        if (ws.empty()) {
            const uint64_t key = stream_key(seed, layer, T_WSG);
            ws.resize(d.hidden);
            for (size_t i = 0; i < ws.size(); ++i) ws[i] = normal_bf16(key, i, 0.02);
        }
        return ws.data();
    }
    Proj make(int p, int e) {
        const int in = p < 2 ? d.hidden : d.inter, out = p < 2 ? d.inter : d.hidden;
        int dim, bits;
        const float* book;
        if (d.mixed) {
            const bool d4 = (e % 2) == 0;
            dim = d4 ? 4 : 8;
            bits = d4 ? 8 : 14;
            book = d4 ? book4[p].data() : book8[p].data();
        } else {
            dim = p < 2 ? d.gu_dim : d.down_dim;
            bits = p < 2 ? d.gu_bits : d.down_bits;
            book = book8[p].data();
        }
        const int group = p < 2 ? d.gu_group : d.down_group;
        const int nsub = in / dim;
        const int64_t words = word_count(nsub, bits);
        const uint64_t ct[3] = {T_CODES_GATE, T_CODES_UP, T_CODES_DOWN};
        const uint64_t st[3] = {T_SCALE_GATE, T_SCALE_UP, T_SCALE_DOWN};
        const uint64_t ck = stream_key(seed, layer, ct[p]);
        const uint64_t sk = stream_key(seed, layer, st[p]);
        codes.emplace_back(static_cast<size_t>(out) * words);
        auto& cw = codes.back();
        std::vector<uint32_t> raw(nsub);
        for (int o = 0; o < out; ++o) {
            for (int s = 0; s < nsub; ++s) raw[s] = code_at(ck, e, out, o, s, bits);
            pack(raw.data(), nsub, bits, cw.data() + static_cast<size_t>(o) * words);
        }
        const int ngrp = in / group;
        scales.emplace_back(static_cast<size_t>(out) * ngrp);
        auto& sv = scales.back();
        for (int o = 0; o < out; ++o)
            for (int g = 0; g < ngrp; ++g) {
                const uint64_t idx = (static_cast<uint64_t>(e) * out + o) * ngrp + g;
                sv[static_cast<size_t>(o) * ngrp + g] = uniform_f16(sk, idx, 0.005, 0.02);
            }
        return Proj{cw.data(), sv.data(), book, in, out, dim, bits, group};
    }
    ExpertWeights expert(int e) override { return {make(0, e), make(1, e), make(2, e)}; }
};

// Caches materialised experts so a second forward times arithmetic only.
struct CachingSource final : LayerSource {
    LayerSource& inner;
    std::vector<std::pair<int, ExpertWeights>> cache;
    explicit CachingSource(LayerSource& s) : inner(s) {}
    const uint16_t* router() override { return inner.router(); }
    const uint16_t* wsg() override { return inner.wsg(); }
    ExpertWeights expert(int e) override {
        for (auto& kv : cache) if (kv.first == e) return kv.second;
        cache.emplace_back(e, inner.expert(e));
        return cache.back().second;
    }
};

// Dense source: caller-provided host tensors in the product layout (uniform geometry).
struct DenseSource final : LayerSource {
    Desc d;
    const uint16_t* wr; const uint16_t* ws;
    const uint32_t* codes[3]; const uint16_t* scales[3];
    std::vector<float> book[3];
    bool has_sa = false;
    AffineExpert sa{};
    const AffineExpert* shared_affine() override { return has_sa ? &sa : nullptr; }
    DenseSource(const Desc& dd, const uint16_t* r, const uint16_t* w, const uint32_t* const* c,
                const uint16_t* const* s, const uint16_t* const* b)
        : d(dd), wr(r), ws(w) {
        const int dims[3] = {d.gu_dim, d.gu_dim, d.down_dim};
        const int bits[3] = {d.gu_bits, d.gu_bits, d.down_bits};
        for (int p = 0; p < 3; ++p) {
            codes[p] = c[p];
            scales[p] = s[p];
            layer_book(d, p, b[p], 1 << bits[p], dims[p], bits[p], book[p]);
        }
    }
    const uint16_t* router() override { return wr; }
    const uint16_t* wsg() override { return ws; }
    ExpertWeights expert(int e) override {
        Proj P[3];
        for (int p = 0; p < 3; ++p) {
            const int in = p < 2 ? d.hidden : d.inter, out = p < 2 ? d.inter : d.hidden;
            const int dim = p < 2 ? d.gu_dim : d.down_dim, bits = p < 2 ? d.gu_bits : d.down_bits;
            const int group = p < 2 ? d.gu_group : d.down_group;
            const int64_t words = word_count(in / dim, bits);
            P[p] = Proj{codes[p] + static_cast<size_t>(e) * out * words,
                        scales[p] + static_cast<size_t>(e) * out * (in / group),
                        book[p].data(), in, out, dim, bits, group};
        }
        return {P[0], P[1], P[2]};
    }
};

// RMSNorm with unit gamma: x = T(h / sqrt(mean(h^2) + eps)) (double arithmetic).
void rmsnorm(const uint16_t* h, int M, int H, double eps, uint16_t* out) {
    for (int r = 0; r < M; ++r) {
        double ss = 0.0;
        for (int c = 0; c < H; ++c) {
            const double v = bf16_to_f32(h[static_cast<size_t>(r) * H + c]);
            ss += v * v;
        }
        const double inv = 1.0 / std::sqrt(ss / H + eps);
        for (int c = 0; c < H; ++c)
            out[static_cast<size_t>(r) * H + c] =
                f32_to_bf16(static_cast<float>(bf16_to_f32(h[static_cast<size_t>(r) * H + c]) * inv));
    }
}

// ---------------------------------------------------------------- HyperConnection mixer
// HyperConnection::read / write (src/hyper_connection.cpp:309-493, 692-709) at the rounding
// points of the reference's fused read kernels (src/hc_metal_kernels.hpp:10-36 normalise,
// :85-128 rank projection + SiLU, :270-308 expansion + mix); the default MLX graph
// (src/hyper_connection.cpp:461-493) rounds to BF16 at the same points, and its injection
// (raw = T(dot), T(raw * T(1/HC)), T(sigmoid), T(x2), :481-493) is the one stated here.
// MLX affine weights: value j of a packed word at bits j*bits (LSB first), weight =
// q * scale + bias with one BF16 scale and bias per `group` inputs. Dot products are taken
// in double over exactly-widened operands and rounded once to float (a value every float
// accumulation order approximates; the device is compared within tolerance); the norm
// total likewise. Elementwise steps are float operations, as on the device.
struct HcDesc {
    int32_t hidden, streams, rank, bits, group, with_injection;
    float eps;
};

double affine_dot(const uint32_t* w, const uint16_t* s, const uint16_t* b, const float* x, int n, int bits, int group) {
    const int vpw = 32 / bits;
    const uint32_t mask = (1u << bits) - 1u;
    double acc = 0.0;
    for (int k = 0; k < n; ++k) {
        const uint32_t q = (w[k / vpw] >> (bits * (k % vpw))) & mask;
        const double wq = static_cast<double>(q) * bf16_to_f32(s[k / group]) + bf16_to_f32(b[k / group]);
        acc += static_cast<double>(x[k]) * wq;
    }
    return acc;
}

inline float sigmoid_d(float v) { return static_cast<float>(1.0 / (1.0 + std::exp(-static_cast<double>(v)))); }

void hc_read(const HcDesc& d, const uint16_t* norm, const uint32_t* dw, const uint16_t* ds, const uint16_t* db,
             const uint32_t* uw, const uint16_t* us, const uint16_t* ub, const uint32_t* iw, const uint16_t* is,
             const uint16_t* ib, const uint16_t* stream, int M, uint16_t* mixed, uint16_t* inj, uint16_t* xn_out,
             float* act_out) {
    const int H = d.hidden, HC = d.streams, R = d.rank, K = HC * H;
    const int vpw = 32 / d.bits;
    std::vector<float> xn(K), act(R);
    for (int m = 0; m < M; ++m) {
        const uint16_t* row = stream + static_cast<size_t>(m) * K;
        for (int s = 0; s < HC; ++s) {
            double ss = 0.0;
            for (int k = 0; k < H; ++k) {
                const double v = bf16_to_f32(row[s * H + k]);
                ss += v * v;
            }
            const float inv = static_cast<float>(1.0 / std::sqrt(static_cast<double>(static_cast<float>(ss)) / H + d.eps));
            for (int k = 0; k < H; ++k) {
                const float t = rbf16(bf16_to_f32(row[s * H + k]) * inv);
                const float wn = rbf16(bf16_to_f32(norm[s * H + k]) + 1.0f);
                xn[s * H + k] = rbf16(t * wn);
            }
        }
        for (int r = 0; r < R; ++r) {
            const double dot = affine_dot(dw + static_cast<size_t>(r) * (K / vpw), ds + static_cast<size_t>(r) * (K / d.group),
                                          db + static_cast<size_t>(r) * (K / d.group), xn.data(), K, d.bits, d.group);
            const float v = rbf16(static_cast<float>(dot) / static_cast<float>(HC));
            act[r] = rbf16(v * rbf16(sigmoid_d(v)));
        }
        if (d.with_injection && inj) {
            for (int c = 0; c < HC; ++c) {
                const double dot = affine_dot(iw + static_cast<size_t>(c) * (K / vpw), is + static_cast<size_t>(c) * (K / d.group),
                                              ib + static_cast<size_t>(c) * (K / d.group), xn.data(), K, d.bits, d.group);
                const float v = rbf16(rbf16(static_cast<float>(dot)) * rbf16(1.0f / static_cast<float>(HC)));
                inj[static_cast<size_t>(m) * HC + c] = f32_to_bf16(rbf16(sigmoid_d(v)) * 2.0f);
            }
        }
        for (int c = 0; c < H; ++c) {
            float sum = 0.0f;
            for (int s = 0; s < HC; ++s) {
                const size_t wr = static_cast<size_t>(s) * H + c;
                const double dot = affine_dot(uw + wr * (R / vpw), us + wr * (R / d.group), ub + wr * (R / d.group),
                                              act.data(), R, d.bits, d.group);
                const float u = rbf16(static_cast<float>(dot));
                const float gate = rbf16(sigmoid_d(u));
                sum += rbf16(gate * xn[s * H + c]);
            }
            mixed[static_cast<size_t>(m) * H + c] = f32_to_bf16(rbf16(sum) / static_cast<float>(HC));
        }
        if (xn_out)
            for (int k = 0; k < K; ++k) xn_out[static_cast<size_t>(m) * K + k] = f32_to_bf16(xn[k]);
        if (act_out)
            for (int r = 0; r < R; ++r) act_out[static_cast<size_t>(m) * R + r] = act[r];
    }
}

void hc_write(int H, int HC, int M, const uint16_t* stream, const uint16_t* block, const uint16_t* inj, uint16_t* out) {
    for (int m = 0; m < M; ++m)
        for (int s = 0; s < HC; ++s) {
            const float g = bf16_to_f32(inj[static_cast<size_t>(m) * HC + s]);
            for (int c = 0; c < H; ++c) {
                const size_t at = (static_cast<size_t>(m) * HC + s) * H + c;
                out[at] = f32_to_bf16(bf16_to_f32(stream[at]) + rbf16(bf16_to_f32(block[static_cast<size_t>(m) * H + c]) * g));
            }
        }
}

// ---------------------------------------------------------------- LM head (R12/R13)
// Reference: batched quantized_matmul over the final rows (src/model.cpp:466-492) and
// argmax_all + take (src/mtp_verifier.cpp:30-55), ties to the lowest index
// (src/mlx_backend.cpp:78-85, tests/mlx_backend_test.cpp:26-36). The build's head is
// symmetric int8 with one FP16 scale per vocab row. Logit contract (shared with the HIP
// exact pass): 64 lane partials in double, lane l adds w[v,64j+l]*h[64j+l] for j = 0..
// in order (every product is exact in double), joined by the xor butterfly, then
// logit = float(double(scale_v) * dot).
inline float head_q8_logit(const int8_t* w, const float* h, int H, uint16_t scale) {
    double part[64];
    for (int l = 0; l < 64; ++l) {
        double acc = 0.0;
        for (int j = 0; j * 64 + l < H; ++j)
            acc += static_cast<double>(w[j * 64 + l]) * static_cast<double>(h[j * 64 + l]);
        part[l] = acc;
    }
    for (int off = 32; off >= 1; off >>= 1) {
        double next[64];
        for (int l = 0; l < 64; ++l) next[l] = part[l] + part[l ^ off];
        std::memcpy(part, next, sizeof(part));
    }
    return static_cast<float>(static_cast<double>(f16_to_f32(scale)) * part[0]);
}

inline int8_t head_w_at(uint64_t key, uint64_t i) {
    return static_cast<int8_t>(static_cast<int>(((bits_at(key, i) >> 32) * 255ull) >> 32) - 127);
}
inline int8_t draft_w_at(uint64_t key, uint64_t i) {
    return static_cast<int8_t>(static_cast<int>(bits_at(key, i) >> 60) - 8);
}

// ---------------------------------------------------------------- Philox4x32-10
// Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy as 1, 2, 3" (SC'11).
inline void philox(const uint32_t ctr_in[4], const uint32_t key_in[2], uint32_t out[4]) {
    uint32_t c0 = ctr_in[0], c1 = ctr_in[1], c2 = ctr_in[2], c3 = ctr_in[3];
    uint32_t k0 = key_in[0], k1 = key_in[1];
    for (int round = 0; round < 10; ++round) {
        const uint64_t p0 = static_cast<uint64_t>(0xD2511F53u) * c0;
        const uint64_t p1 = static_cast<uint64_t>(0xCD9E8D57u) * c2;
        const uint32_t n0 = static_cast<uint32_t>(p1 >> 32) ^ c1 ^ k0;
        const uint32_t n1 = static_cast<uint32_t>(p1);
        const uint32_t n2 = static_cast<uint32_t>(p0 >> 32) ^ c3 ^ k1;
        const uint32_t n3 = static_cast<uint32_t>(p0);
        c0 = n0; c1 = n1; c2 = n2; c3 = n3;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

// Uniforms for (seed, slot, round, position): counter = {position, round lo, round hi,
// slot}, key = {seed lo, seed hi}; u = (x0 >> 8) * 2^-24 (acceptance), v = (x1 >> 8) *
// 2^-24 (residual / bonus draw).
inline void round_uniforms(uint64_t seed, uint64_t slot, uint64_t round, uint32_t pos, float* u, float* v) {
    const uint32_t ctr[4] = {pos, static_cast<uint32_t>(round), static_cast<uint32_t>(round >> 32),
                             static_cast<uint32_t>(slot)};
    const uint32_t key[2] = {static_cast<uint32_t>(seed), static_cast<uint32_t>(seed >> 32)};
    uint32_t out[4];
    philox(ctr, key, out);
    *u = static_cast<float>(out[0] >> 8) * 0x1.0p-24f;
    *v = static_cast<float>(out[1] >> 8) * 0x1.0p-24f;
}

// softmax(logits / T) in double.
void softmax_T(const float* l, int64_t V, double T, std::vector<double>& p) {
    p.resize(V);
    double mx = l[0];
    for (int64_t i = 1; i < V; ++i) mx = std::max(mx, static_cast<double>(l[i]));
    double s = 0.0;
    for (int64_t i = 0; i < V; ++i) { p[i] = std::exp((l[i] - mx) / T); s += p[i]; }
    for (int64_t i = 0; i < V; ++i) p[i] /= s;
}

// Inverse-CDF draw in index order: the smallest x with cumsum(w)[x] > v * sum(w).
int64_t draw(const std::vector<double>& w, double v) {
    double total = 0.0;
    for (double x : w) total += x;
    const double target = v * total;
    double c = 0.0;
    int64_t last = -1;
    for (int64_t i = 0; i < static_cast<int64_t>(w.size()); ++i) {
        if (w[i] > 0.0) last = i;
        c += w[i];
        if (c > target && w[i] > 0.0) return i;
    }
    return last < 0 ? 0 : last;
}


// ---------------------------------------------------------------- GatedDeltaNet verify
// GatedDeltaNet::forward_verify (src/gated_delta_net.cpp:657-834): the linear-attention half
// of a decoder layer for S rows (1..64) from an origin state, with the state after every
// row kept as that row's checkpoint. The rounding points restate the ops of that path:
//   qkv, z, b, a   T(quantized_matmul) (affine_row_dot, double accumulation)
//   conv1d         depthwise, width 4 over [origin conv rows ; qkv rows]: T(sum_j w[c][j] *
//                  in[t + j][c]) (:691-692), then silu = T(c * T(sigmoid(c))) (MlxArray::silu,
//                  src/mlx_backend.cpp:621-624)
//   q, k           rms_norm with unit weight over the head dimension (:709-710):
//                  T(x * 1/sqrt(mean(x^2) + 1e-6)), then q = T(q * bf16(1/DK)),
//                  k = T(k * bf16(1/sqrt(DK))) (:711-716); value head h reads key head
//                  h / (HV / HK) (repeat_axis, :717-719)
//   beta           T(sigmoid(b)) (:721); decay T(exp(-(exp(A_log) * softplus(T(a + dt_bias)))))
//                  with softplus = log1p(exp(.)) in float (:722-725)
//   recurrence     the bf16-sum verify kernel (src/gdn_metal_kernels.hpp:498-562): per value
//                  head and value row, 32 lanes of DK/32 state items, every product, lane sum,
//                  residual, delta, update and state rounded to bf16 as there; the 32 lanes'
//                  partial sums (simd_sum there) are added in float by an xor butterfly
//                  (lane offsets 16, 8, 4, 2, 1) and rounded once — the order is this build's
//                  contract (Metal's simd_sum order is not specified: parity unpinned there)
//   output         rms_norm(y, norm_weight, eps) = T(w * T(y * inv)) per value head
//                  (:809 / :824), gate T(sigmoid(z)) or silu T(z * T(sigmoid(z))), their product
//                  T, then T(quantized_matmul(out_proj)) (:829-833)
//   checkpoints    after row t: conv rows t+1..t+3 of [origin ; qkv] and the recurrent state
//                  (:825-831).
struct GdnDesc {
    int hidden, hk, hv, dk, dv, conv, bits, group, fmt, gate_silu;
    float eps;
};
struct GdnW {
    AffineProj qkv, z, b, a, out;
    const uint16_t* conv_w;  // [C][4] bf16
    const float* a_log;      // [HV]
    const uint16_t* dt_bias; // [HV] bf16
    const uint16_t* norm_w;  // [DV] bf16
};
int g_gdn_fault;  // planted faults (tests only): 1 = value head h reads key head h % HK
inline float tb(float v) { return bf16_to_f32(f32_to_bf16(v)); }
inline float sigmoid_t(float x) { return tb(static_cast<float>(1.0 / (1.0 + std::exp(-static_cast<double>(x))))); }

// The recurrence of S rows (the bf16-sum kernel's rounding points, above): q, k [S][HK][DK],
// v [S][HV][DV], decay / beta [S][HV] (bf16 values); state_in [HV][DV][DK] bf16 or null (zero);
// y [S][HV][DV]; the state after row t at state_rows + t * row_stride when given.
void gdn_recurrence(int HK, int HV, int DK, int DV, int S, const float* q, const float* k, const float* v,
                    const float* decay, const float* beta, const uint16_t* state_in, float* y, uint16_t* state_rows,
                    size_t row_stride) {
    const int KW = HK * DK, VW = HV * DV, rep = HV / HK, items = DK / 32;
    for (int h = 0; h < HV; ++h) {
        const int hk = g_gdn_fault == 1 ? h % HK : h / rep;
        for (int r = 0; r < DV; ++r) {
            std::vector<float> st(DK);
            for (int i = 0; i < DK; ++i)
                st[i] = state_in ? bf16_to_f32(state_in[(static_cast<size_t>(h) * DV + r) * DK + i]) : 0.0f;
            for (int t = 0; t < S; ++t) {
                const float g = decay[static_cast<size_t>(t) * HV + h], bt = beta[static_cast<size_t>(t) * HV + h];
                const float* kr = k + static_cast<size_t>(t) * KW + hk * DK;
                const float* qr = q + static_cast<size_t>(t) * KW + hk * DK;
                float part[32];
                for (int l = 0; l < 32; ++l) {
                    float acc = 0.0f;
                    for (int i = 0; i < items; ++i) {
                        const int ix = l * items + i;
                        st[ix] = tb(st[ix] * g);
                        acc = tb(acc + tb(st[ix] * kr[ix]));
                    }
                    part[l] = acc;
                }
                auto lane_sum = [&](float* pp) {
                    for (int off = 16; off > 0; off >>= 1) {
                        float nx[32];
                        for (int l = 0; l < 32; ++l) nx[l] = pp[l] + pp[l ^ off];
                        std::memcpy(pp, nx, sizeof(nx));
                    }
                    return tb(pp[0]);
                };
                const float recalled = lane_sum(part);
                const float delta = tb(tb(v[static_cast<size_t>(t) * VW + h * DV + r] - recalled) * bt);
                for (int l = 0; l < 32; ++l) {
                    float acc = 0.0f;
                    for (int i = 0; i < items; ++i) {
                        const int ix = l * items + i;
                        st[ix] = tb(st[ix] + tb(kr[ix] * delta));
                        acc = tb(acc + tb(st[ix] * qr[ix]));
                    }
                    part[l] = acc;
                }
                y[static_cast<size_t>(t) * VW + h * DV + r] = lane_sum(part);
                if (state_rows) {
                    uint16_t* cs = state_rows + static_cast<size_t>(t) * row_stride + (static_cast<size_t>(h) * DV + r) * DK;
                    for (int i = 0; i < DK; ++i) cs[i] = f32_to_bf16(st[i]);
                }
            }
        }
    }
}

// state: conv [3][C] bf16 then recurrent [HV][DV][DK] bf16
void gdn_verify(const GdnDesc& d, const GdnW& W, const uint16_t* x, int S, const uint16_t* origin, uint16_t* out,
                uint16_t* ckpt) {
    const int H = d.hidden, HK = d.hk, HV = d.hv, DK = d.dk, DV = d.dv;
    const int KW = HK * DK, VW = HV * DV, C = 2 * KW + VW;
    const size_t state_elems = static_cast<size_t>(3) * C + static_cast<size_t>(HV) * DV * DK;
    std::vector<float> xf(H), qkv(static_cast<size_t>(S + 3) * C), z(static_cast<size_t>(S) * VW),
        beta(static_cast<size_t>(S) * HV), decay(static_cast<size_t>(S) * HV), q(static_cast<size_t>(S) * KW),
        k(static_cast<size_t>(S) * KW), v(static_cast<size_t>(S) * VW), y(static_cast<size_t>(S) * VW),
        gated(static_cast<size_t>(S) * VW);
    for (int i = 0; i < 3 * C; ++i) qkv[i] = origin ? bf16_to_f32(origin[i]) : 0.0f;
    for (int t = 0; t < S; ++t) {
        for (int c = 0; c < H; ++c) xf[c] = bf16_to_f32(x[static_cast<size_t>(t) * H + c]);
        for (int c = 0; c < C; ++c) qkv[static_cast<size_t>(t + 3) * C + c] = rbf16(affine_row_dot(W.qkv, c, xf.data()));
        for (int c = 0; c < VW; ++c) z[static_cast<size_t>(t) * VW + c] = rbf16(affine_row_dot(W.z, c, xf.data()));
        for (int h = 0; h < HV; ++h) {
            const float b = rbf16(affine_row_dot(W.b, h, xf.data()));
            const float a = rbf16(affine_row_dot(W.a, h, xf.data()));
            beta[static_cast<size_t>(t) * HV + h] = sigmoid_t(b);
            const float biased = tb(a + bf16_to_f32(W.dt_bias[h]));
            const double softplus = std::log1p(std::exp(static_cast<double>(biased)));
            const double rate = std::exp(static_cast<double>(W.a_log[h]));
            decay[static_cast<size_t>(t) * HV + h] = rbf16(std::exp(-(static_cast<double>(static_cast<float>(rate)) *
                                                                        static_cast<float>(softplus))));
        }
        // conv + silu, then the q / k norms per head
        std::vector<float> act(C);
        for (int c = 0; c < C; ++c) {
            float acc = 0.0f;
            for (int j = 0; j < 4; ++j)
                acc = std::fma(bf16_to_f32(W.conv_w[static_cast<size_t>(c) * 4 + j]),
                               qkv[static_cast<size_t>(t + j) * C + c], acc);
            const float cv = tb(acc);
            act[c] = tb(cv * sigmoid_t(cv));
        }
        const float ks = tb(static_cast<float>(1.0 / std::sqrt(static_cast<double>(DK))));
        const float qs = tb(static_cast<float>(1.0 / DK));
        for (int part = 0; part < 2; ++part)
            for (int h = 0; h < HK; ++h) {
                const float* a = act.data() + part * KW + h * DK;
                double ss = 0.0;
                for (int i = 0; i < DK; ++i) ss += static_cast<double>(a[i]) * a[i];
                const float inv = static_cast<float>(1.0 / std::sqrt(ss / DK + 1e-6));
                float* dst = (part ? k.data() : q.data()) + static_cast<size_t>(t) * KW + h * DK;
                for (int i = 0; i < DK; ++i) dst[i] = tb(tb(a[i] * inv) * (part ? ks : qs));
            }
        for (int c = 0; c < VW; ++c) v[static_cast<size_t>(t) * VW + c] = act[2 * KW + c];
    }
    gdn_recurrence(HK, HV, DK, DV, S, q.data(), k.data(), v.data(), decay.data(), beta.data(),
                   origin ? origin + static_cast<size_t>(3) * C : nullptr, y.data(),
                   ckpt ? ckpt + static_cast<size_t>(3) * C : nullptr, state_elems);
    // norm and gate per (row, value head), then the output projection
    for (int t = 0; t < S; ++t) {
        for (int h = 0; h < HV; ++h) {
            const float* yr = y.data() + static_cast<size_t>(t) * VW + h * DV;
            double ss = 0.0;
            for (int i = 0; i < DV; ++i) ss += static_cast<double>(yr[i]) * yr[i];
            const float inv = static_cast<float>(1.0 / std::sqrt(ss / DV + static_cast<double>(d.eps)));
            for (int i = 0; i < DV; ++i) {
                const float nrm = tb(bf16_to_f32(W.norm_w[i]) * tb(yr[i] * inv));
                const float zz = z[static_cast<size_t>(t) * VW + h * DV + i];
                const float gate = d.gate_silu ? tb(zz * sigmoid_t(zz)) : sigmoid_t(zz);
                gated[static_cast<size_t>(t) * VW + h * DV + i] = tb(nrm * gate);
            }
        }
        for (int o = 0; o < H; ++o)
            out[static_cast<size_t>(t) * H + o] = f32_to_bf16(rbf16(affine_row_dot(W.out, o, gated.data() + static_cast<size_t>(t) * VW)));
        if (ckpt) {
            uint16_t* cc = ckpt + static_cast<size_t>(t) * state_elems;
            for (int j = 0; j < 3; ++j)
                for (int c = 0; c < C; ++c) cc[static_cast<size_t>(j) * C + c] = f32_to_bf16(qkv[static_cast<size_t>(t + 1 + j) * C + c]);
        }
    }
}
// ---- full attention, verify (SelfAttention::forward_verify, src/self_attention.cpp:1450-1720,
// on its dense path: no QSA mask, which the reference builds only once a context exceeds the
// indexer budget, :764-766, and a bf16 KV cache). The rounding points are those of the
// explicit decode path (:1240-1305), which the batched path computes in one pass:
//   projections    qg = T(q_proj x) [HQ][2 D] (per head D query values, then D gate values,
//                  :1464-1466 / :1481-1488), k = T(k_proj x), v = T(v_proj x) [HKV][D]
//   q / k norms    rms_norm per head: T(wn * T(x * inv)), inv = 1 / sqrt(mean(x^2) + eps),
//                  wn = w, or T(1 + w) with an offset norm (effective_norm_weight, :52-58)
//   RoPE           (:641-679) on the first R dims at position p: c_i, s_i = bf16 of
//                  float(cos / sin(p * theta^(-2i / R))) in double, i < R / 2, repeated for
//                  the second half; x'_j = T(T(x_j * c_j) + T(rot_j * s_j)),
//                  rot = (-x_{j + R/2} for j < R/2, x_{j - R/2} after); dims >= R unchanged
//   cache          keys / values [HKV][T][D]: the origin's T0 tokens, then the S rows
//   scores         row r, query head h (kv head h / (HQ / HKV)) over tokens t <= T0 + r:
//                  s_t = T(T(q . k_t) * T(1 / sqrt D)) (:1299-1302)
//   softmax        of the float32 scores: e_t = exp(s_t - max s), p_t = T(e_t / sum e) (:1303)
//   output         attended = T(sum_t p_t v_t), gated = T(attended * T(sigmoid(gate)))
//                  (:1321-1323), out = T(o_proj gated)
// Positions: row r of the call is at position + r (origin.position_base + token_count, :1254).
struct AttnDesc {
    int hidden, q_heads, kv_heads, head_dim, rotary_dim, bits, group, fmt, norm_offset;
    float eps;
    double rope_theta;
};
struct AttnW {
    AffineProj q, k, v, o;
    const uint16_t* q_norm;  // [D] bf16
    const uint16_t* k_norm;  // [D] bf16
};
int g_attn_fault;  // planted faults (tests only): 1 = RoPE on adjacent pairs, 2 = no causal mask within the rows

// The bf16 RoPE table of one position: c[i], s[i] for i < R / 2.
void rope_table(double theta, int R, int64_t pos, float* c, float* s) {
    for (int i = 0; i < R / 2; ++i) {
        const double freq = std::pow(theta, -2.0 * static_cast<double>(i) / static_cast<double>(R));
        const double angle = static_cast<double>(pos) * freq;
        c[i] = rbf16(static_cast<float>(std::cos(angle)));
        s[i] = rbf16(static_cast<float>(std::sin(angle)));
    }
}

// rms_norm of one head (T(wn * T(x * inv))) then RoPE at pos, in place on D values.
void attn_norm_rope(float* x, int D, int R, const float* wn, float eps, double theta, int64_t pos) {
    double ss = 0.0;
    for (int i = 0; i < D; ++i) ss += static_cast<double>(x[i]) * x[i];
    const float inv = static_cast<float>(1.0 / std::sqrt(ss / D + static_cast<double>(eps)));
    for (int i = 0; i < D; ++i) x[i] = tb(wn[i] * tb(x[i] * inv));
    std::vector<float> c(R / 2), sn(R / 2), y(R);
    rope_table(theta, R, pos, c.data(), sn.data());
    const int half = R / 2;
    for (int j = 0; j < R; ++j) {
        float rot, cj, sj;
        if (g_attn_fault == 1) {  // interleaved pairs (2i, 2i + 1), the other RoPE convention
            const int i = j / 2;
            rot = (j % 2 == 0) ? -x[j + 1] : x[j - 1];
            cj = c[i];
            sj = sn[i];
        } else {
            rot = j < half ? -x[j + half] : x[j - half];
            cj = c[j % half];
            sj = sn[j % half];
        }
        y[j] = tb(tb(x[j] * cj) + tb(rot * sj));
    }
    for (int j = 0; j < R; ++j) x[j] = y[j];
}

// keys / values: [HKV][cap][D] bf16 with the origin's T0 tokens; the S new rows are written at
// T0..T0+S-1 (the cache after the call); out [S][H].
void attn_verify(const AttnDesc& d, const AttnW& W, const uint16_t* x, int S, uint16_t* keys, uint16_t* values,
                 int64_t cap, int64_t T0, int64_t position, uint16_t* out) {
    const int H = d.hidden, HQ = d.q_heads, HKV = d.kv_heads, D = d.head_dim, R = d.rotary_dim;
    const int grp = HQ / HKV;
    std::vector<float> qn(D), kn(D);
    for (int i = 0; i < D; ++i) {
        const float qw = bf16_to_f32(W.q_norm[i]), kw = bf16_to_f32(W.k_norm[i]);
        qn[i] = d.norm_offset ? tb(1.0f + qw) : qw;
        kn[i] = d.norm_offset ? tb(1.0f + kw) : kw;
    }
    std::vector<float> xf(H), q(static_cast<size_t>(S) * HQ * D), gate(static_cast<size_t>(S) * HQ * D);
    for (int r = 0; r < S; ++r) {
        for (int c = 0; c < H; ++c) xf[c] = bf16_to_f32(x[static_cast<size_t>(r) * H + c]);
        const int64_t pos = position + r;
        for (int h = 0; h < HQ; ++h) {
            float* qh = q.data() + (static_cast<size_t>(r) * HQ + h) * D;
            for (int i = 0; i < D; ++i) {
                qh[i] = rbf16(affine_row_dot(W.q, h * 2 * D + i, xf.data()));
                gate[(static_cast<size_t>(r) * HQ + h) * D + i] =
                    sigmoid_t(rbf16(affine_row_dot(W.q, h * 2 * D + D + i, xf.data())));
            }
            attn_norm_rope(qh, D, R, qn.data(), d.eps, d.rope_theta, pos);
        }
        std::vector<float> kh(D);
        for (int g = 0; g < HKV; ++g) {
            for (int i = 0; i < D; ++i) kh[i] = rbf16(affine_row_dot(W.k, g * D + i, xf.data()));
            attn_norm_rope(kh.data(), D, R, kn.data(), d.eps, d.rope_theta, pos);
            uint16_t* kd = keys + (static_cast<size_t>(g) * cap + T0 + r) * D;
            uint16_t* vd = values + (static_cast<size_t>(g) * cap + T0 + r) * D;
            for (int i = 0; i < D; ++i) {
                kd[i] = f32_to_bf16(kh[i]);
                vd[i] = f32_to_bf16(rbf16(affine_row_dot(W.v, g * D + i, xf.data())));
            }
        }
    }
    const float scale = tb(static_cast<float>(1.0 / std::sqrt(static_cast<double>(D))));
    std::vector<float> gated(static_cast<size_t>(HQ) * D);
    for (int r = 0; r < S; ++r) {
        const int64_t T = g_attn_fault == 2 ? T0 + S : T0 + r + 1;
        for (int h = 0; h < HQ; ++h) {
            const int g = h / grp;
            const float* qh = q.data() + (static_cast<size_t>(r) * HQ + h) * D;
            std::vector<float> sc(static_cast<size_t>(T));
            float m = -INFINITY;
            for (int64_t t = 0; t < T; ++t) {
                const uint16_t* kt = keys + (static_cast<size_t>(g) * cap + t) * D;
                double dot = 0.0;
                for (int i = 0; i < D; ++i) dot += static_cast<double>(qh[i]) * bf16_to_f32(kt[i]);
                sc[t] = tb(rbf16(dot) * scale);
                m = std::max(m, sc[t]);
            }
            double sum = 0.0;
            std::vector<float> e(static_cast<size_t>(T));
            for (int64_t t = 0; t < T; ++t) {
                e[t] = static_cast<float>(std::exp(static_cast<double>(sc[t] - m)));
                sum += e[t];
            }
            std::vector<double> acc(D, 0.0);
            for (int64_t t = 0; t < T; ++t) {
                const float pt = rbf16(static_cast<double>(e[t]) / static_cast<double>(static_cast<float>(sum)));
                const uint16_t* vt = values + (static_cast<size_t>(g) * cap + t) * D;
                for (int i = 0; i < D; ++i) acc[i] += static_cast<double>(pt) * bf16_to_f32(vt[i]);
            }
            for (int i = 0; i < D; ++i)
                gated[static_cast<size_t>(h) * D + i] = tb(rbf16(acc[i]) * gate[(static_cast<size_t>(r) * HQ + h) * D + i]);
        }
        for (int o = 0; o < H; ++o)
            out[static_cast<size_t>(r) * H + o] = f32_to_bf16(rbf16(affine_row_dot(W.o, o, gated.data())));
    }
}

// ---- the decoder's MLP output map (DecoderLayer::apply_mlp_output_map,
// src/decoder_layer.cpp:198-210): out = T(y . T), or T(y + T(T(y . L) . R)) with the low-rank
// pair. MLX's bf16 matmul order is not specified (parity unpinned there); this build's contract:
// per output element, float fmaf over 128-input slices in ascending order, the slices' sums
// added in slice order, then rounded to bf16.
void map_product(const float* a, int rows, int K, const uint16_t* W, int N, float* out) {
    for (int r = 0; r < rows; ++r)
        for (int n = 0; n < N; ++n) {
            float total = 0.0f;
            for (int k0 = 0; k0 < K; k0 += 128) {
                float acc = 0.0f;
                for (int k = k0; k < std::min(K, k0 + 128); ++k)
                    acc = std::fma(a[static_cast<size_t>(r) * K + k], bf16_to_f32(W[static_cast<size_t>(k) * N + n]), acc);
                total += acc;
            }
            out[static_cast<size_t>(r) * N + n] = rbf16(total);
        }
}

} // namespace

// ======================================================================== C ABI
extern "C" {

// ---- formats
uint16_t orc_f32_to_bf16(float f) { return f32_to_bf16(f); }
uint16_t orc_f32_to_f16(float f) { return f32_to_f16(f); }
float orc_f16_to_f32(uint16_t h) { return f16_to_f32(h); }
float orc_exp_contract(float d) { return exp_contract(d); }

// ---- generator
uint64_t orc_stream_key(uint64_t seed, uint64_t layer, uint64_t tensor) { return stream_key(seed, layer, tensor); }
uint64_t orc_bits_at(uint64_t key, uint64_t i) { return bits_at(key, i); }
void orc_gen_normal(uint64_t key, uint64_t start, uint64_t count, double sd, int f16, uint16_t* out) {
    for (uint64_t i = 0; i < count; ++i) out[i] = f16 ? normal_f16(key, start + i, sd) : normal_bf16(key, start + i, sd);
}
void orc_gen_uniform_f16(uint64_t key, uint64_t start, uint64_t count, double lo, double hi, uint16_t* out) {
    for (uint64_t i = 0; i < count; ++i) out[i] = uniform_f16(key, start + i, lo, hi);
}
void orc_gen_int8(uint64_t key, uint64_t start, uint64_t count, int8_t* out) {
    for (uint64_t i = 0; i < count; ++i) out[i] = head_w_at(key, start + i);
}
void orc_gen_int4(uint64_t key, uint64_t start, uint64_t count, int8_t* out) {
    for (uint64_t i = 0; i < count; ++i) out[i] = draft_w_at(key, start + i);
}
// Packed code rows [rows, words] of expert e for rows o0..o0+nrows of a projection.
void orc_gen_code_rows(uint64_t key, int e, int out_dim, int o0, int nrows, int nsub, int bits, uint32_t* words) {
    const int64_t nw = word_count(nsub, bits);
    std::vector<uint32_t> raw(nsub);
    for (int i = 0; i < nrows; ++i) {
        for (int s = 0; s < nsub; ++s) raw[s] = code_at(key, e, out_dim, o0 + i, s, bits);
        pack(raw.data(), nsub, bits, words + static_cast<int64_t>(i) * nw);
    }
}
// Synthetic codebook as stored on the device: f16 values (int8 == 0) or int8 values + one
// f16 scale (int8 == 1).
void orc_gen_book(uint64_t key, int K, int D, int int8, uint16_t* f16_out, int8_t* i8_out, uint16_t* scale_out) {
    std::vector<float> vals;
    std::vector<uint16_t> raw;
    std::vector<int8_t> raw8;
    synth_book(key, K, D, int8 != 0, vals, &raw, &raw8, scale_out);
    if (!int8 && f16_out) std::copy(raw.begin(), raw.end(), f16_out);
    if (int8 && i8_out) std::copy(raw8.begin(), raw8.end(), i8_out);
}
// Per-dimension INT8/U8 codebook of an FP16 book: q [K*D] int32, scales/biases [D] fp16,
// decoded values [K*D] float.
void orc_prepare_u8_book(const uint16_t* book16, int K, int D, int centered, int32_t* q, uint16_t* s16, uint16_t* b16,
                         float* vals) {
    std::vector<int32_t> qv;
    std::vector<uint16_t> sv, bv;
    std::vector<float> fv;
    prepare_u8_book(book16, K, D, centered != 0, qv, sv, bv, fv);
    std::copy(qv.begin(), qv.end(), q);
    std::copy(sv.begin(), sv.end(), s16);
    std::copy(bv.begin(), bv.end(), b16);
    std::copy(fv.begin(), fv.end(), vals);
}
void orc_gen_embed(uint64_t seed, const uint32_t* tokens, int n, int H, uint16_t* out) {
    const uint64_t key = stream_key(seed, kEmbedLayer, T_EMBED);
    for (int r = 0; r < n; ++r)
        for (int c = 0; c < H; ++c)
            out[static_cast<size_t>(r) * H + c] = normal_bf16(key, static_cast<uint64_t>(tokens[r]) * H + c, 1.0);
}

// ---- geometry
int64_t orc_packed_word_count(int64_t n, int bits) { return word_count(n, bits); }
int orc_pack_row(const uint32_t* codes, int64_t n, int bits, uint32_t* words) {
    if (word_count(n, bits) < 0) return -1;
    for (int64_t i = 0; i < n; ++i) if (codes[i] >> bits) return -1;
    pack(codes, n, bits, words);
    return 0;
}
// 0 ok, -1 invalid bits, -2 buffer too short (the reference throws std::out_of_range).
int orc_unpack_code(const uint32_t* words, int64_t nwords, int64_t index, int bits, uint32_t* out) {
    const int64_t need = word_count(index + 1, bits);
    if (need < 0) return -1;
    if (nwords < need) return -2;
    *out = unpack(words, index, bits);
    return 0;
}

// ---- router
void orc_router_logits(const uint16_t* x, int M, int H, const uint16_t* W, int E, float* logits) {
    for (int r = 0; r < M; ++r)
        for (int e = 0; e < E; ++e)
            logits[static_cast<size_t>(r) * E + e] =
                rbf16(dot_contract(x + static_cast<size_t>(r) * H, W + static_cast<size_t>(e) * H, H));
}
float orc_dot_contract(const uint16_t* x, const uint16_t* w, int H) { return dot_contract(x, w, H); }
void orc_route(const float* logits, int M, int E, int k, int normalize, int32_t* experts, float* weights) {
    route_rows(logits, M, E, k, normalize, experts, weights);
}
int orc_route_plan(const int32_t* experts, int M, int k, int E, int32_t* n_unique, int32_t* uexp,
                   int32_t* uoff, int32_t* route_list, int32_t* route_pos) {
    return route_plan(experts, M, k, E, n_unique, uexp, uoff, route_list, route_pos);
}

// ---- MoE layer
int orc_moe_layer_synth(const Desc* d, uint64_t seed, int layer, const uint16_t* x, int M, uint16_t* y,
                        int32_t* experts, float* weights, float* logits, int threads) {
    SynthSource src(*d, seed, static_cast<uint64_t>(layer));
    return moe_layer(*d, src, x, M, y, experts, weights, logits, threads);
}
// Routing alone (R1 + R2) of the synthetic layer (seed, layer): logits [M, E] (BF16-rounded
// contract dot, plus the optional bias), experts / weights [M, k].
int orc_route_synth(const Desc* d, uint64_t seed, int layer, const uint16_t* x, int M, const float* bias,
                    int32_t* experts, float* weights, float* logits, int threads) {
    const int H = d->hidden, E = d->experts;
    if (H % 512 != 0 || E % 64 != 0 || d->top_k < 1 || d->top_k > E || M < 1) return -1;
    SynthSource src(*d, seed, static_cast<uint64_t>(layer));
    const uint16_t* Wr = src.router();
    std::vector<float> lg(static_cast<size_t>(M) * E);
    parallel_for(E, threads, [&](int e) {
        for (int r = 0; r < M; ++r) {
            const float v = rbf16(dot_contract(x + static_cast<size_t>(r) * H, Wr + static_cast<size_t>(e) * H, H));
            lg[static_cast<size_t>(r) * E + e] = bias ? v + bias[e] : v;
        }
    });
    route_rows(lg.data(), M, E, d->top_k, d->normalize, experts, weights);
    if (logits) std::copy(lg.begin(), lg.end(), logits);
    return 0;
}
// orc_moe_layer_synth with an additive router-logit bias (float, added to the BF16 logit).
int orc_moe_layer_synth_bias(const Desc* d, uint64_t seed, int layer, const uint16_t* x, int M, const float* bias,
                             uint16_t* y, int32_t* experts, float* weights, float* logits, int threads) {
    SynthSource src(*d, seed, static_cast<uint64_t>(layer));
    return moe_layer(*d, src, x, M, y, experts, weights, logits, threads, bias);
}
// Same as orc_moe_layer_synth, but the tensors are materialised by an untimed first pass
// and *seconds receives the wall time of a second, arithmetic-only pass (CPU baseline).
// Repeated timing of one synthetic layer: the layer's experts are generated once (untimed),
// then for each of the n_cfg thread counts, `warm` untimed passes and `reps` timed passes;
// seconds[c * reps + r] is pass r at threads[c].
int orc_moe_layer_synth_reps(const Desc* d, uint64_t seed, int layer, const uint16_t* x, int M, uint16_t* y,
                             const int* threads, int n_cfg, int warm, int reps, double* seconds) {
    SynthSource src(*d, seed, static_cast<uint64_t>(layer));
    CachingSource cs(src);
    int rc = moe_layer(*d, cs, x, M, y, nullptr, nullptr, nullptr, threads[0]);
    for (int c = 0; c < n_cfg && rc == 0; ++c) {
        for (int w = 0; w < warm && rc == 0; ++w) rc = moe_layer(*d, cs, x, M, y, nullptr, nullptr, nullptr, threads[c]);
        for (int r = 0; r < reps && rc == 0; ++r) {
            const auto t0 = std::chrono::steady_clock::now();
            rc = moe_layer(*d, cs, x, M, y, nullptr, nullptr, nullptr, threads[c]);
            seconds[c * reps + r] = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
        }
    }
    return rc;
}
// codes/scales/books: arrays of 3 pointers (gate, up, down) in the product layout
// [E(+1), OUT, words] / [E(+1), OUT, IN/G] / [K, D] fp16.
int orc_moe_layer_dense(const Desc* d, const uint16_t* router, const uint16_t* wsg,
                        const uint32_t* const* codes, const uint16_t* const* scales,
                        const uint16_t* const* books, const uint16_t* x, int M, uint16_t* y,
                        int32_t* experts, float* weights, float* logits, int threads) {
    if (d->mixed) return -1;
    DenseSource src(*d, router, wsg, codes, scales, books);
    return moe_layer(*d, src, x, M, y, experts, weights, logits, threads);
}
// orc_moe_layer_dense with the shared expert in MLX affine form: codes / scales hold the E
// routed experts only; sa_w / sa_s / sa_b: gate, up ([inter, H]) and down ([H, inter]) packed
// words, scales and biases (fmt 0 bf16, 1 fp16).
int orc_moe_layer_dense_affine_shared(const Desc* d, const uint16_t* router, const uint16_t* wsg,
                                      const uint32_t* const* codes, const uint16_t* const* scales,
                                      const uint16_t* const* books, const uint32_t* const* sa_w,
                                      const uint16_t* const* sa_s, const uint16_t* const* sa_b, int bits, int group,
                                      int inter, int fmt, const uint16_t* x, int M, uint16_t* y, int32_t* experts,
                                      float* weights, float* logits, int threads) {
    if (d->mixed || !d->has_shared || bits <= 0 || 32 % bits || group <= 0 || d->hidden % group || inter % group)
        return -1;
    DenseSource src(*d, router, wsg, codes, scales, books);
    src.has_sa = true;
    src.sa.gate = AffineProj{sa_w[0], sa_s[0], sa_b[0], d->hidden, inter, bits, group, fmt};
    src.sa.up = AffineProj{sa_w[1], sa_s[1], sa_b[1], d->hidden, inter, bits, group, fmt};
    src.sa.down = AffineProj{sa_w[2], sa_s[2], sa_b[2], inter, d->hidden, bits, group, fmt};
    return moe_layer(*d, src, x, M, y, experts, weights, logits, threads);
}
// The affine shared expert alone on rows of x: dout [M, H] = T(down) per row (no gate).
int orc_affine_expert(const uint32_t* const* sa_w, const uint16_t* const* sa_s, const uint16_t* const* sa_b, int H,
                      int inter, int bits, int group, int fmt, const uint16_t* x, int M, float* dout) {
    if (bits <= 0 || 32 % bits || group <= 0 || H % group || inter % group) return -1;
    const AffineExpert W{AffineProj{sa_w[0], sa_s[0], sa_b[0], H, inter, bits, group, fmt},
                         AffineProj{sa_w[1], sa_s[1], sa_b[1], H, inter, bits, group, fmt},
                         AffineProj{sa_w[2], sa_s[2], sa_b[2], inter, H, bits, group, fmt}};
    std::vector<float> xf(H);
    for (int r = 0; r < M; ++r) {
        for (int c = 0; c < H; ++c) xf[c] = bf16_to_f32(x[static_cast<size_t>(r) * H + c]);
        affine_expert_forward(W, xf.data(), dout + static_cast<size_t>(r) * H);
    }
    return 0;
}
// One expert applied to rows of x (no routing); dout [M, H] = T(down) per row.
int orc_expert_dense(const Desc* d, const uint32_t* const* codes, const uint16_t* const* scales,
                     const uint16_t* const* books, int e, const uint16_t* x, int M, float* dout) {
    DenseSource src(*d, nullptr, nullptr, codes, scales, books);
    const ExpertWeights W = src.expert(e);
    std::vector<float> xf(d->hidden);
    for (int r = 0; r < M; ++r) {
        for (int c = 0; c < d->hidden; ++c) xf[c] = bf16_to_f32(x[static_cast<size_t>(r) * d->hidden + c]);
        expert_forward(W, xf.data(), dout + static_cast<size_t>(r) * d->hidden);
    }
    return 0;
}
void orc_rmsnorm(const uint16_t* h, int M, int H, double eps, uint16_t* out) { rmsnorm(h, M, H, eps, out); }
void orc_residual_add(const uint16_t* h, const uint16_t* y, int64_t n, uint16_t* out) {
    for (int64_t i = 0; i < n; ++i)
        out[i] = f32_to_bf16(bf16_to_f32(h[i]) + bf16_to_f32(y[i]));
}

// ---- LM heads
// Contract logits for vocab rows [v0, v0+nv) of the synthetic Q8 head; h: [M, H] bf16.
void orc_head_q8_synth_logits(uint64_t seed, int H, int64_t v0, int64_t nv, const uint16_t* h, int M,
                              float* logits, int threads) {
    const uint64_t wk = stream_key(seed, kHeadLayer, T_HEAD_W), sk = stream_key(seed, kHeadLayer, T_HEAD_S);
    std::vector<float> hf(static_cast<size_t>(M) * H);
    for (size_t i = 0; i < hf.size(); ++i) hf[i] = bf16_to_f32(h[i]);
    const int chunks = static_cast<int>((nv + 255) / 256);
    parallel_for(chunks, threads, [&](int ch) {
        std::vector<int8_t> w(H);
        for (int64_t v = v0 + static_cast<int64_t>(ch) * 256; v < std::min(v0 + nv, v0 + static_cast<int64_t>(ch + 1) * 256); ++v) {
            for (int c = 0; c < H; ++c) w[c] = head_w_at(wk, static_cast<uint64_t>(v) * H + c);
            const uint16_t s = uniform_f16(sk, static_cast<uint64_t>(v), 1e-4, 1e-3);
            for (int r = 0; r < M; ++r)
                logits[static_cast<size_t>(r) * nv + (v - v0)] = head_q8_logit(w.data(), hf.data() + static_cast<size_t>(r) * H, H, s);
        }
    });
}
// Contract logits of an explicit head: W [V, H] int8, s [V] fp16.
void orc_head_q8_logits(const int8_t* W, const uint16_t* s, int64_t V, int H, const uint16_t* h, int M,
                        float* logits, int threads) {
    std::vector<float> hf(static_cast<size_t>(M) * H);
    for (size_t i = 0; i < hf.size(); ++i) hf[i] = bf16_to_f32(h[i]);
    const int chunks = static_cast<int>((V + 1023) / 1024);
    parallel_for(chunks, threads, [&](int ch) {
        for (int64_t v = static_cast<int64_t>(ch) * 1024; v < std::min(V, static_cast<int64_t>(ch + 1) * 1024); ++v)
            for (int r = 0; r < M; ++r)
                logits[static_cast<size_t>(r) * V + v] = head_q8_logit(W + v * H, hf.data() + static_cast<size_t>(r) * H, H, s[v]);
    });
}
// argmax with ties to the lowest index (src/mlx_backend.cpp:78-85).
void orc_argmax(const float* logits, int M, int64_t V, uint32_t* idx, float* val) {
    for (int r = 0; r < M; ++r) {
        const float* l = logits + static_cast<size_t>(r) * V;
        int64_t best = 0;
        for (int64_t v = 1; v < V; ++v) if (l[v] > l[best]) best = v;
        idx[r] = static_cast<uint32_t>(best);
        val[r] = l[best];
    }
}
// Q4 draft head logit of one vocab row (same arithmetic for explicit and synthetic weights):
// signed int4 w[c] in [-8, 7], one FP16 scale per 64 inputs, in double:
// sum_g scale[v, g] * sum_{c in g} w[c] * h[c] (groups in order, inputs in order).
inline float head_q4_logit(const int8_t* w, const float* h, int H, const uint16_t* s_row) {
    double acc = 0.0;
    for (int g = 0; g < H / 64; ++g) {
        double ga = 0.0;
        for (int c = g * 64; c < g * 64 + 64; ++c) ga += static_cast<double>(w[c]) * h[c];
        acc += static_cast<double>(f16_to_f32(s_row[g])) * ga;
    }
    return static_cast<float>(acc);
}
// Explicit Q4 head: Wp [V, H/2] bytes, input 2i in the low nibble and 2i + 1 in the high
// nibble, each a signed (two's-complement) int4; s [V, H/64] fp16. This is the device
// head's tensor contract (q38_head_create, Q38_HEAD_Q4G64).
void orc_head_q4_logits(const uint8_t* Wp, const uint16_t* s, int64_t V, int H, const uint16_t* h, int M,
                        float* logits, int threads) {
    std::vector<float> hf(static_cast<size_t>(M) * H);
    for (size_t i = 0; i < hf.size(); ++i) hf[i] = bf16_to_f32(h[i]);
    const int chunks = static_cast<int>((V + 255) / 256);
    parallel_for(chunks, threads, [&](int ch) {
        std::vector<int8_t> w(H);
        for (int64_t v = static_cast<int64_t>(ch) * 256; v < std::min(V, static_cast<int64_t>(ch + 1) * 256); ++v) {
            const uint8_t* row = Wp + v * (H / 2);
            for (int i = 0; i < H / 2; ++i) {
                w[2 * i] = static_cast<int8_t>(static_cast<int>(row[i] & 0xF) - ((row[i] & 0x8) ? 16 : 0));
                w[2 * i + 1] = static_cast<int8_t>(static_cast<int>(row[i] >> 4) - ((row[i] & 0x80) ? 16 : 0));
            }
            for (int r = 0; r < M; ++r)
                logits[static_cast<size_t>(r) * V + v] =
                    head_q4_logit(w.data(), hf.data() + static_cast<size_t>(r) * H, H, s + v * (H / 64));
        }
    });
}
// Q4 draft head with synthetic weights: w = draft_w_at (T_DRAFT_W stream), scales ~
// U(1.6e-3, 1.6e-2) (T_DRAFT_S stream, index v * H/64 + g).
void orc_head_q4_synth_logits(uint64_t seed, int H, int64_t v0, int64_t nv, const uint16_t* h, int M,
                              float* logits, int threads) {
    const uint64_t wk = stream_key(seed, kDraftLayer, T_DRAFT_W), sk = stream_key(seed, kDraftLayer, T_DRAFT_S);
    const int G = H / 64;
    std::vector<float> hf(static_cast<size_t>(M) * H);
    for (size_t i = 0; i < hf.size(); ++i) hf[i] = bf16_to_f32(h[i]);
    const int chunks = static_cast<int>((nv + 255) / 256);
    parallel_for(chunks, threads, [&](int ch) {
        std::vector<int8_t> w(H);
        std::vector<uint16_t> srow(G);
        for (int64_t v = v0 + static_cast<int64_t>(ch) * 256; v < std::min(v0 + nv, v0 + static_cast<int64_t>(ch + 1) * 256); ++v) {
            for (int c = 0; c < H; ++c) w[c] = draft_w_at(wk, static_cast<uint64_t>(v) * H + c);
            for (int g = 0; g < G; ++g) srow[g] = uniform_f16(sk, static_cast<uint64_t>(v) * G + g, 1.6e-3, 1.6e-2);
            for (int r = 0; r < M; ++r)
                logits[static_cast<size_t>(r) * nv + (v - v0)] =
                    head_q4_logit(w.data(), hf.data() + static_cast<size_t>(r) * H, H, srow.data());
        }
    });
}

// ---- acceptance (R15, R16) and commit (R17)
// decide_mtp_greedy (src/mtp_lifecycle.cpp:75-97). Returns -1 (empty drafts) or -2
// (missing bonus row) as the reference throws.
int orc_decide_greedy(const uint32_t* drafts, int64_t k, const uint32_t* target, int64_t ntarget,
                      const uint32_t* stop, int64_t nstop, int64_t* accepted, int64_t* row, uint32_t* next) {
    if (k <= 0) return -1;
    if (ntarget != k + 1) return -2;
    int64_t a = 0;
    while (a < k && drafts[a] == target[a]) {
        bool is_stop = false;
        for (int64_t s = 0; s < nstop; ++s) if (stop[s] == drafts[a]) is_stop = true;
        if (is_stop) break;
        ++a;
    }
    *accepted = a;
    *row = a;
    *next = target[a];
    return 0;
}
// plan_mtp_commit (src/mtp_lifecycle.cpp:57-73): out = {truncate_head_to,
// target_rows_to_keep, stash_rows, committed_boundary}; -1 when accepted > drafted.
int orc_plan_commit(uint64_t round_offset, uint64_t drafted, uint64_t accepted, uint64_t* out) {
    if (accepted > drafted) return -1;
    out[0] = round_offset;
    out[1] = 1 + accepted;
    out[2] = 1 + accepted;
    out[3] = round_offset + 1 + accepted;
    return 0;
}
void orc_philox4x32_10(const uint32_t* ctr, const uint32_t* key, uint32_t* out) { philox(ctr, key, out); }
void orc_round_uniforms(uint64_t seed, uint64_t slot, uint64_t round, uint32_t pos, float* u, float* v) {
    round_uniforms(seed, slot, round, pos, u, v);
}
// Speculative sampling (Leviathan et al. 2023, Chen et al. 2023): for i < k accept draft
// d_i iff u_i * q_i(d_i) < p_i(d_i); at the first rejection emit a draw from
// norm(max(0, p_i - q_i)) with v_i; if all k are accepted emit a draw from p_k with v_k.
// p = softmax(target_logits/T) [k+1, V], q = softmax(draft_logits/T) [k, V].
// Test-only fault injection for the sampler (0: none). 1: the all-accepted bonus token is
// drawn from p_{k-1} instead of p_k. 2: after a first rejection at position i >= 1 the
// residual is formed from rows i-1 instead of i. The distribution tests set it to show that
// a wrong-row draw fails them; nothing else touches it.
static int g_plant_fault = 0;
void orc_plant_fault(int code) { g_plant_fault = code; }
int orc_accept_sampled(const float* target_logits, const float* draft_logits, const uint32_t* drafts, int k,
                       int64_t V, float temperature, uint64_t seed, uint64_t slot, uint64_t round,
                       int64_t* accepted, uint32_t* next) {
    if (k <= 0 || V <= 0 || !(temperature > 0.0f)) return -1;
    std::vector<double> p, q;
    for (int i = 0; i < k; ++i) {
        if (drafts[i] >= V) return -1;
        softmax_T(target_logits + static_cast<size_t>(i) * V, V, temperature, p);
        softmax_T(draft_logits + static_cast<size_t>(i) * V, V, temperature, q);
        float u, v;
        round_uniforms(seed, slot, round, static_cast<uint32_t>(i), &u, &v);
        const double pd = p[drafts[i]], qd = q[drafts[i]];
        if (static_cast<double>(u) * qd < pd) continue;
        if (g_plant_fault == 2 && i >= 1) {
            softmax_T(target_logits + static_cast<size_t>(i - 1) * V, V, temperature, p);
            softmax_T(draft_logits + static_cast<size_t>(i - 1) * V, V, temperature, q);
        }
        std::vector<double> res(V);
        for (int64_t x = 0; x < V; ++x) res[x] = std::max(0.0, p[x] - q[x]);
        *accepted = i;
        *next = static_cast<uint32_t>(draw(res, v));
        return 0;
    }
    softmax_T(target_logits + static_cast<size_t>(g_plant_fault == 1 ? k - 1 : k) * V, V, temperature, p);
    float u, v;
    round_uniforms(seed, slot, round, static_cast<uint32_t>(k), &u, &v);
    *accepted = k;
    *next = static_cast<uint32_t>(draw(p, v));
    return 0;
}

int orc_hc_read(const HcDesc* d, const uint16_t* norm, const uint32_t* dw, const uint16_t* ds, const uint16_t* db,
                const uint32_t* uw, const uint16_t* us, const uint16_t* ub, const uint32_t* iw, const uint16_t* is,
                const uint16_t* ib, const uint16_t* stream, int M, uint16_t* mixed, uint16_t* inj, uint16_t* xn_out,
                float* act_out) {
    if (!d || d->bits <= 0 || 32 % d->bits || d->group <= 0 || d->hidden % d->group || d->rank % d->group) return -1;
    hc_read(*d, norm, dw, ds, db, uw, us, ub, iw, is, ib, stream, M, mixed, inj, xn_out, act_out);
    return 0;
}
void orc_hc_write(int H, int HC, int M, const uint16_t* stream, const uint16_t* block, const uint16_t* inj,
                  uint16_t* out) {
    hc_write(H, HC, M, stream, block, inj, out);
}


// ---- GatedDeltaNet verify (GdnDesc: hidden, hk, hv, dk, dv, conv, bits, group, fmt, gate_silu, eps)
void orc_gdn_plant_fault(int code) { g_gdn_fault = code; }
// The recurrence alone (bf16 values as floats; state_in / state_rows bf16 bits).
int orc_gdn_recurrence(int HK, int HV, int DK, int DV, int S, const float* q, const float* k, const float* v,
                       const float* decay, const float* beta, const uint16_t* state_in, float* y, uint16_t* state_rows) {
    if (HK < 1 || HV % HK || DK % 32 || S < 1) return -1;
    gdn_recurrence(HK, HV, DK, DV, S, q, k, v, decay, beta, state_in, y, state_rows,
                   static_cast<size_t>(HV) * DV * DK);
    return 0;
}
int orc_gdn_verify(const GdnDesc* d, const uint32_t* const* w, const uint16_t* const* sc, const uint16_t* const* bi,
                   const uint16_t* conv_w, const float* a_log, const uint16_t* dt_bias, const uint16_t* norm_w,
                   const uint16_t* x, int S, const uint16_t* origin, uint16_t* out, uint16_t* ckpt) {
    if (!d || S < 1 || d->conv != 4 || d->dk % 32 || d->hv % d->hk || d->bits <= 0 || 32 % d->bits || d->group <= 0)
        return -1;
    const int KW = d->hk * d->dk, VW = d->hv * d->dv, C = 2 * KW + VW;
    GdnW W{};
    const int ins[5] = {d->hidden, d->hidden, d->hidden, d->hidden, VW}, outs[5] = {C, VW, d->hv, d->hv, d->hidden};
    AffineProj* P[5] = {&W.qkv, &W.z, &W.b, &W.a, &W.out};
    for (int p = 0; p < 5; ++p) {
        if (ins[p] % d->group) return -1;
        *P[p] = AffineProj{w[p], sc[p], bi[p], ins[p], outs[p], d->bits, d->group, d->fmt};
    }
    W.conv_w = conv_w;
    W.a_log = a_log;
    W.dt_bias = dt_bias;
    W.norm_w = norm_w;
    gdn_verify(*d, W, x, S, origin, out, ckpt);
    return 0;
}

void orc_mlp_map(int H, int rank, const uint16_t* full, const uint16_t* left, const uint16_t* right,
                 const uint16_t* y, int rows, uint16_t* out) {
    std::vector<float> yf(static_cast<size_t>(rows) * H), o(static_cast<size_t>(rows) * H);
    for (size_t i = 0; i < yf.size(); ++i) yf[i] = bf16_to_f32(y[i]);
    if (rank == 0) {
        map_product(yf.data(), rows, H, full, H, o.data());
    } else {
        std::vector<float> t(static_cast<size_t>(rows) * rank);
        map_product(yf.data(), rows, H, left, rank, t.data());
        map_product(t.data(), rows, rank, right, H, o.data());
        for (size_t i = 0; i < o.size(); ++i) o[i] = rbf16(yf[i] + o[i]);
    }
    for (size_t i = 0; i < o.size(); ++i) out[i] = f32_to_bf16(o[i]);
}
void orc_attn_plant_fault(int f) { g_attn_fault = f; }
void orc_rope_table(double theta, int R, int64_t pos, float* c, float* s) { rope_table(theta, R, pos, c, s); }
int orc_attn_verify(const AttnDesc* d, const uint32_t* const* w, const uint16_t* const* sc, const uint16_t* const* bi,
                    const uint16_t* q_norm, const uint16_t* k_norm, const uint16_t* x, int S, uint16_t* keys,
                    uint16_t* values, int64_t cap, int64_t T0, int64_t position, uint16_t* out) {
    if (!d || S < 1 || d->q_heads % d->kv_heads || d->rotary_dim <= 0 || d->rotary_dim % 2 ||
        d->rotary_dim > d->head_dim || d->bits <= 0 || 32 % d->bits || d->group <= 0 || T0 < 0 || T0 + S > cap)
        return -1;
    const int QW = d->q_heads * d->head_dim, KW = d->kv_heads * d->head_dim;
    const int ins[4] = {d->hidden, d->hidden, d->hidden, QW}, outs[4] = {2 * QW, KW, KW, d->hidden};
    AttnW W{};
    AffineProj* P[4] = {&W.q, &W.k, &W.v, &W.o};
    for (int p = 0; p < 4; ++p) {
        if (ins[p] % d->group) return -1;
        *P[p] = AffineProj{w[p], sc[p], bi[p], ins[p], outs[p], d->bits, d->group, d->fmt};
    }
    W.q_norm = q_norm;
    W.k_norm = k_norm;
    attn_verify(*d, W, x, S, keys, values, cap, T0, position, out);
    return 0;
}

} // extern "C"
