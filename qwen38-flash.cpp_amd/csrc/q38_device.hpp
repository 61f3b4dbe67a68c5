// q38_device.hpp — device-side building blocks shared by the gfx950 kernels: number
// formats, the counter-based synthetic generator, the packed-VQ code reader, the exp
// contract of the router softmax, and wave64 reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace q38 {

constexpr int kWave = 64;

// ------------------------------------------------------------------ workgroup barrier
// A barrier that orders LDS only. __syncthreads() fences every address space, which on
// gfx950 waits for all of the wave's outstanding global loads (vmcnt(0)) before s_barrier
// and so drains any prefetch in flight. Kernels that share data through LDS only use this
// one; data that arrives in LDS over the direct global-to-LDS path is covered by an
// explicit vmcnt wait of the issuing wave before the barrier.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}
// The same for a phase in which direct global-to-LDS copies are still in flight: the LDS
// fence above also waits for those (they count as LDS writes), so this barrier waits only
// for the wave's own LDS instructions (lgkmcnt) and leaves the copies running. Only data
// written with ds_* instructions may be read after it.
__device__ __forceinline__ void lds_barrier_dma_pending() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// ------------------------------------------------------------------ kernel arguments
// Kernel arguments are read through the scalar cache on first use, so an argument line
// first needed deep inside a kernel costs a memory round trip at that point. This reads one
// dword of every 64-byte line of the first BYTES bytes at kernel entry: the reads are issued
// together and waited for once, and every later argument read hits.
template <int BYTES>
__device__ __forceinline__ void touch_kernargs() {
    typedef const __attribute__((address_space(4))) uint32_t karg_t;
    karg_t* ka = (karg_t*)(__builtin_amdgcn_kernarg_segment_ptr());
    constexpr int kLines = (BYTES + 63) / 64;
    uint32_t v[kLines];
#pragma unroll
    for (int i = 0; i < kLines; ++i) v[i] = ka[16 * i];
#pragma unroll
    for (int i = 0; i < kLines; ++i) asm volatile("" ::"s"(v[i]));
}

// ------------------------------------------------------------------ number formats
__device__ __forceinline__ float bf2f(uint16_t h) { return __uint_as_float(static_cast<uint32_t>(h) << 16); }
// Round to nearest even; NaN keeps its sign and top mantissa bits and becomes quiet. Written
// as a value select (no branch): every float store of the kernels goes through it.
__device__ __forceinline__ uint16_t f2bf(float f) {
    const uint32_t x = __float_as_uint(f);
    const uint32_t rounded = (x + 0x7fffu + ((x >> 16) & 1u)) >> 16;
    const uint32_t quiet = (x >> 16) | 0x40u;
    return static_cast<uint16_t>((x & 0x7fffffffu) > 0x7f800000u ? quiet : rounded);
}
__device__ __forceinline__ float rbf(float f) { return bf2f(f2bf(f)); }
__device__ __forceinline__ float h2f(uint16_t h) { return static_cast<float>(__builtin_bit_cast(_Float16, h)); }
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f)); }

// Two bf16 packed in a u32 -> floats (low half first).
__device__ __forceinline__ float bflo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bfhi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// ------------------------------------------------------------------ generator
// splitmix64 streams keyed by (seed, layer, tensor); element i = mix64(key + golden*(i+1)).
constexpr uint64_t kGolden = 0x9E3779B97F4A7C15ull;
__host__ __device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
__host__ __device__ __forceinline__ uint64_t stream_key(uint64_t seed, uint64_t layer, uint64_t tensor) {
    return mix64(mix64(mix64(seed) + kGolden * (layer + 1)) + kGolden * (tensor + 1));
}
__host__ __device__ __forceinline__ uint64_t bits_at(uint64_t key, uint64_t i) { return mix64(key + kGolden * (i + 1)); }

enum Tensor : uint64_t {
    T_ROUTER = 1, T_WSG = 2, T_CB_GATE = 3, T_CB_UP = 4, T_CB_DOWN = 5,
    T_CODES_GATE = 6, T_CODES_UP = 7, T_CODES_DOWN = 8,
    T_SCALE_GATE = 9, T_SCALE_UP = 10, T_SCALE_DOWN = 11,
    T_CB4_GATE = 12, T_CB4_UP = 13, T_CB4_DOWN = 14,
    T_X = 20, T_EMBED = 21,
    T_HEAD_W = 30, T_HEAD_S = 31, T_DRAFT_W = 32, T_DRAFT_S = 33,
};
constexpr uint64_t kEmbedLayer = 0xFFFF, kHeadLayer = 0xFFFE, kDraftLayer = 0xFFFD;

// Box-Muller in double from two stream elements.
__device__ __forceinline__ double normal_at(uint64_t key, uint64_t i) {
    const double u1 = static_cast<double>((bits_at(key, 2 * i) >> 11) + 1) * 0x1.0p-53;
    const double u2 = static_cast<double>(bits_at(key, 2 * i + 1) >> 11) * 0x1.0p-53;
    const double rad = sqrt(-2.0 * log(u1));
    const double ang = cos(6.283185307179586 * u2);
    return rad * ang;
}
__device__ __forceinline__ float uniform_f32(uint64_t key, uint64_t i, double lo, double hi) {
#pragma clang fp contract(off)
    const double u = static_cast<double>(bits_at(key, i) >> 11) * 0x1.0p-53;
    const double span = hi - lo;
    const double prod = u * span;
    const double v = lo + prod;
    return static_cast<float>(v);
}

// ------------------------------------------------------------------ packed VQ codes
// Row layout (src/quantization_geometry.cpp:50-67): 32-code blocks of BITS words,
// code q of a block at bit q*BITS, LSB-first.
template <int BITS>
__device__ __forceinline__ uint32_t code_from(const uint32_t* w, int q) {
    // w: words of the 16-code half-block (or whole block) that holds code q; bit offset
    // q*BITS is a compile-time constant after unrolling.
    const int bit = q * BITS;
    const int wi = bit >> 5, sh = bit & 31;
    uint32_t v = w[wi] >> sh;
    if (sh + BITS > 32) v |= w[wi + 1] << (32 - sh);
    return v & ((1u << BITS) - 1u);
}

// ------------------------------------------------------------------ exp contract
// Cody-Waite reduction + degree-7 Taylor polynomial, evaluated with explicit fmaf so the
// float operations are identical to the CPU restatement; results below 2^-125 flush to 0.
// Branch-free: the argument is clamped (NaN included) before the reduction and the flush
// is a final select, so a wave never splits.
__device__ __forceinline__ float exp_contract(float d) {
    const float dc = __builtin_fmaxf(d, -88.0f);
    const float kf = rintf(dc * 1.44269504088896341f);
    float r = __builtin_fmaf(kf, -0.693145751953125f, dc);
    r = __builtin_fmaf(kf, -1.42860682030941723212e-06f, r);
    float p = 1.0f / 5040.0f;
    p = __builtin_fmaf(p, r, 1.0f / 720.0f);
    p = __builtin_fmaf(p, r, 1.0f / 120.0f);
    p = __builtin_fmaf(p, r, 1.0f / 24.0f);
    p = __builtin_fmaf(p, r, 1.0f / 6.0f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    const int k = static_cast<int>(kf);
    const float v = ldexpf(p, k);
    return d > -87.0f && k >= -125 ? v : 0.0f;
}

// ------------------------------------------------------------------ wave reductions
// xor butterfly: every lane ends with the same value, equal to the pairwise tree
// ((l, l^32), then ^16, ...) that the CPU restatement reproduces.
// Value of lane l ^ M. M = 1, 2: DPP quad permutations; M = 4, 8: a row shift for the
// lanes whose bit is clear and the opposite shift for the others (bank masks select the
// lanes, every source lies in the same row); M = 16, 32: permlane swaps (no LDS round trip).
template <int M>
__device__ __forceinline__ uint32_t xor_lane(uint32_t v) {
    if constexpr (M == 1) {
        return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0xB1, 0xF, 0xF, false));
    } else if constexpr (M == 2) {
        return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x4E, 0xF, 0xF, false));
    } else if constexpr (M == 4 || M == 8) {
        constexpr int lo_banks = M == 4 ? 0x5 : 0x3;  // lanes with bit M clear: read l + M
        const int t = __builtin_amdgcn_update_dpp(static_cast<int>(v), static_cast<int>(v), 0x100 + M, 0xF, lo_banks,
                                                  false);
        return static_cast<uint32_t>(
            __builtin_amdgcn_update_dpp(t, static_cast<int>(v), 0x110 + M, 0xF, 0xF ^ lo_banks, false));
    } else {
        // M = 16, 32: the gfx950 lane swaps. With both operands v, the first result holds the
        // lower 16-lane row (32-lane half) of each pair in both rows (halves) and the second
        // the upper one, so lane l takes the one that is not its own.
        const auto r = M == 16 ? __builtin_amdgcn_permlane16_swap(v, v, false, false)
                               : __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return (threadIdx.x & M) ? r[0] : r[1];
    }
}
template <int M>
__device__ __forceinline__ float xor_lane_f(float v) {
    return __uint_as_float(xor_lane<M>(__float_as_uint(v)));
}
template <int M>
__device__ __forceinline__ double xor_lane_d(double v) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint64_t r = (static_cast<uint64_t>(xor_lane<M>(static_cast<uint32_t>(b >> 32))) << 32) |
                       xor_lane<M>(static_cast<uint32_t>(b));
    return __builtin_bit_cast(double, r);
}
// Butterfly sum (offsets 32, 16, ..., 1; v = v + v[l ^ off]): every lane ends with the
// same total, in an order the CPU restatement repeats.
__device__ __forceinline__ float wave_sum_xor(float v) {
    v = v + xor_lane_f<32>(v);
    v = v + xor_lane_f<16>(v);
    v = v + xor_lane_f<8>(v);
    v = v + xor_lane_f<4>(v);
    v = v + xor_lane_f<2>(v);
    v = v + xor_lane_f<1>(v);
    return v;
}
__device__ __forceinline__ double wave_sum_xor(double v) {
    v = v + xor_lane_d<32>(v);
    v = v + xor_lane_d<16>(v);
    v = v + xor_lane_d<8>(v);
    v = v + xor_lane_d<4>(v);
    v = v + xor_lane_d<2>(v);
    v = v + xor_lane_d<1>(v);
    return v;
}
// wave_sum_xor of N values (N a power of two, 2..16), reduced and scattered: the xor-32 step
// swaps the upper half of value i with the lower half of value i + N/2 (one lane swap and
// one add per pair), the xor-16 step does the same for 16-lane rows when two or more values
// are left, and the steps inside a row are DPP adds (row rotations by 8 and by 4, which equal
// the xor partners once the previous step has made the row's halves, quarters, equal; then
// the two quad permutations). Every add joins the same two partial sums as wave_sum_xor does
// (float addition commutes exactly), so each total is bit-identical to wave_sum_xor of that
// value. On return v[s] for s < scatter_slots<N>() holds in lane l the total of input value
// scatter_value<N>(s, l >> 4); the other entries are dead.
template <int N>
__device__ constexpr int scatter_slots() { return N >= 4 ? N / 4 : 1; }
template <int N>
__device__ constexpr int scatter_value(int s, int row) {
    return N >= 4 ? s + (row & 1) * (N / 4) + (row >> 1) * (N / 2) : (N == 2 ? (row >> 1) : 0);
}
// one lane per distinct (slot, value): the first lane of each 16-lane row (of each 32-lane
// half when N = 2; lane 0 for N = 1, a plain wave_sum_xor)
template <int N>
__device__ __forceinline__ bool scatter_leader(int lane) {
    return (lane & (N == 1 ? 63 : N == 2 ? 31 : 15)) == 0;
}
template <int N>
__device__ __forceinline__ void wave_sum_xor_scatter(float (&v)[N]) {
    static_assert(N >= 2 && N <= 16 && (N & (N - 1)) == 0, "N: a power of two in 2..16");
#pragma unroll
    for (int i = 0; i < N / 2; ++i) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[i]), __float_as_uint(v[i + N / 2]), false,
                                                        false);
        v[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    constexpr int S = scatter_slots<N>();
    if constexpr (N >= 4) {
#pragma unroll
        for (int i = 0; i < N / 4; ++i) {
            const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[i]), __float_as_uint(v[i + N / 4]), false,
                                                            false);
            v[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
        }
    } else {
        v[0] = v[0] + xor_lane_f<16>(v[0]);
    }
#pragma unroll
    for (int i = 0; i < S; ++i)
        v[i] = v[i] + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v[i]), 0x128, 0xF, 0xF, false));
#pragma unroll
    for (int i = 0; i < S; ++i)
        v[i] = v[i] + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v[i]), 0x124, 0xF, 0xF, false));
#pragma unroll
    for (int i = 0; i < S; ++i)
        v[i] = v[i] + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v[i]), 0x4E, 0xF, 0xF, false));
#pragma unroll
    for (int i = 0; i < S; ++i)
        v[i] = v[i] + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v[i]), 0xB1, 0xF, 0xF, false));
}

// wave_sum_xor of N independent values, step by step across all of them (the exchanges of
// one step are in flight together); each result equals wave_sum_xor of that value alone.
template <int N>
__device__ __forceinline__ void wave_sum_xor_n(float (&v)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = v[i] + xor_lane_f<32>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = v[i] + xor_lane_f<16>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = v[i] + xor_lane_f<8>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = v[i] + xor_lane_f<4>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = v[i] + xor_lane_f<2>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = v[i] + xor_lane_f<1>(v[i]);
}
// The same butterfly through lane permutes only (the reference form of the exchanges).
__device__ __forceinline__ float wave_sum_xor_shfl(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = v + __shfl_xor(v, off, kWave);
    return v;
}
__device__ __forceinline__ double wave_sum_xor_shfl(double v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = v + __shfl_xor(v, off, kWave);
    return v;
}
template <int WIDTH>
__device__ __forceinline__ float group_sum_xor(float v) {
#pragma unroll
    for (int off = WIDTH / 2; off >= 1; off >>= 1) v = v + __shfl_xor(v, off, kWave);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
    return v;
}
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const uint64_t o = __shfl_xor(v, off, kWave);
        v = o > v ? o : v;
    }
    return v;
}

// ------------------------------------------------------------------ Philox4x32-10
// Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy as 1, 2, 3" (SC'11).
__host__ __device__ __forceinline__ void philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
    uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3];
    uint32_t k0 = key[0], k1 = key[1];
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
// Acceptance / resample uniforms of (seed, slot, round, position): counter {position,
// round lo, round hi, slot}, key {seed lo, seed hi}; u = (x0 >> 8) 2^-24, v = (x1 >> 8) 2^-24.
__host__ __device__ __forceinline__ void round_uniforms(uint64_t seed, uint64_t slot, uint64_t round, uint32_t pos,
                                                        float* u, float* v) {
    const uint32_t ctr[4] = {pos, static_cast<uint32_t>(round), static_cast<uint32_t>(round >> 32),
                             static_cast<uint32_t>(slot)};
    const uint32_t key[2] = {static_cast<uint32_t>(seed), static_cast<uint32_t>(seed >> 32)};
    uint32_t out[4];
    philox4x32_10(ctr, key, out);
    *u = static_cast<float>(out[0] >> 8) * 0x1.0p-24f;
    *v = static_cast<float>(out[1] >> 8) * 0x1.0p-24f;
}

// Total order on float bit patterns (larger float -> larger key).
__device__ __forceinline__ uint32_t orderable(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float from_orderable(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

} // namespace q38
