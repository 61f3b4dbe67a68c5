// q38_internal.hpp — device-side layer/head descriptors and the launchers shared between
// the kernel translation units and the C ABI implementation.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace q38 {

constexpr int kMaxRows = 16;   // verify rows per MoE call (4 slots x (1 + 3 drafts))
constexpr int kMaxTopK = 16;
constexpr int kHeadCap = 256;  // exact-pass candidates kept per row before the full fallback

struct ProjDev {
    const uint32_t* codes;   // [E+1, OUT, words]
    const uint16_t* scales;  // [E+1, OUT, ngrp] fp16
    const uint16_t* book;    // [2^bits, dim] fp16
    int words, ngrp, dim, bits;
};

struct LayerDev {
    const uint16_t* router;  // [E, H] bf16
    const uint16_t* wsg;     // [H] bf16
    ProjDev p[3];            // gate, up, down
    int H, I, E, K, normalize, has_shared;
};

struct HeadDev {
    const int8_t* w;         // Q8: [V, H]; Q4: [V, H/2] packed nibbles
    const uint16_t* scales;  // Q8: [V]; Q4: [V, H/64]
    int64_t V;
    int H, kind;
    float s_max;             // max |scale| over the head (exact-pass window)
};

// MoE layer
hipError_t launch_router(const LayerDev& L, const uint16_t* hin, int M, int do_norm, float eps, uint16_t* xn,
                         float* logits, float* sgate, hipStream_t st);
hipError_t launch_topk_plan(const LayerDev& L, const float* logits, int M, int32_t* experts, float* weights,
                            int32_t* plan, hipStream_t st);
hipError_t launch_gate_up(const LayerDev& L, const uint16_t* xn, int M, const int32_t* plan, uint16_t* hbuf,
                          hipStream_t st);
hipError_t launch_down(const LayerDev& L, int M, const int32_t* plan, const uint16_t* hbuf, uint16_t* dbuf,
                       hipStream_t st);
hipError_t launch_combine(const LayerDev& L, int M, const int32_t* plan, const float* weights, const float* sgate,
                          const uint16_t* dbuf, const uint16_t* hin, uint16_t* out, hipStream_t st);
hipError_t launch_rmsnorm(const uint16_t* x, int M, int H, float eps, uint16_t* y, hipStream_t st);

// generators
hipError_t launch_gen_codes(uint64_t key, int e0, int n_experts, int out_dim, int nsub, int bits, int words,
                            uint32_t* codes, hipStream_t st);
hipError_t launch_gen_uniform_f16(uint64_t key, int64_t idx0, int64_t n, double lo, double hi, uint16_t* out,
                                  hipStream_t st);
hipError_t launch_gen_normal(uint64_t key, int64_t n, double sd, int f16, uint16_t* out, hipStream_t st);
hipError_t launch_gen_embed(uint64_t seed, const uint32_t* tokens, int n, int H, uint16_t* out, hipStream_t st);
hipError_t launch_book_to_int8(const uint16_t* book16, int n, int8_t* q8, uint16_t* scale, hipStream_t st);
hipError_t launch_gen_head(const HeadDev& hd, uint64_t seed, int8_t* w, uint16_t* scales, hipStream_t st);
hipError_t launch_scale_absmax(const uint16_t* scales, int64_t n, float* out, hipStream_t st);

// heads
struct HeadWork {
    float* fast;        // [M, V]
    uint32_t* rowmax;   // [M] orderable
    float* tsum;        // [M] sum |h|
    int32_t* cnt;       // [M]
    int32_t* cand;      // [M, kHeadCap]
    unsigned long long* best;  // [M]
};
size_t head_work_bytes(int64_t V, int M);
HeadWork head_work_carve(void* base, int64_t V, int M);
hipError_t launch_head_greedy(const HeadDev& hd, const uint16_t* h, int M, const HeadWork& w, uint32_t* argmax,
                              float* logit, hipStream_t st);
hipError_t launch_head_logits(const HeadDev& hd, const uint16_t* h, int M, float* logits, hipStream_t st);

// acceptance
hipError_t launch_accept_sampled(const float* tl, const float* dl, const uint32_t* drafts, int k, int64_t V,
                                 float T, uint64_t seed, uint64_t slot, uint64_t round, int64_t* out,
                                 hipStream_t st);

} // namespace q38
