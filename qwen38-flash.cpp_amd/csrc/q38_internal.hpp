// q38_internal.hpp — device-side layer/head descriptors and the launchers shared between
// the kernel translation units and the C ABI implementation.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <mutex>

namespace q38 {

// Kernel timing for the profiled entry points: while a timer is set, the first launch made
// through launch() records `start` at its kernel's own begin and every launch records `stop`
// at its kernel's end, so a phase of one or more kernels spans the first kernel's begin to
// the last kernel's end (the interval a kernel trace reports); the caller clears the timer
// after the phase. One timer per host thread. Every kernel launch of the library goes
// through launch().
struct KernelTimer {
    hipEvent_t start = nullptr, stop = nullptr;
};
KernelTimer& kernel_timer();

template <typename F, typename... Args>
hipError_t launch(F kernel, dim3 grid, dim3 block, size_t lds, hipStream_t st, Args... args) {
    KernelTimer& t = kernel_timer();
    if (t.stop) {
        hipExtLaunchKernelGGL(kernel, grid, block, static_cast<uint32_t>(lds), st, t.start, t.stop, 0, args...);
        t.start = nullptr;
    } else {
        hipLaunchKernelGGL(kernel, grid, block, lds, st, args...);
    }
    return hipGetLastError();
}

// Dynamic-LDS limit of kernel KERN on the current device, raised to `bytes` when a call needs
// more than any call before it (the limit only grows, so calls with smaller needs keep
// working; the raise is serialised, and the recorded size is updated only after the
// attribute call succeeded).
template <auto KERN>
hipError_t ensure_lds(size_t bytes) {
    static std::atomic<uint32_t> limit[64];
    static std::mutex mu;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    std::atomic<uint32_t>& cur = limit[dev & 63];
    if (cur.load(std::memory_order_acquire) >= bytes) return hipSuccess;
    std::lock_guard<std::mutex> lk(mu);
    if (cur.load(std::memory_order_acquire) >= bytes) return hipSuccess;
    e = hipFuncSetAttribute(reinterpret_cast<const void*>(KERN), hipFuncAttributeMaxDynamicSharedMemorySize,
                            static_cast<int>(bytes));
    if (e == hipSuccess) cur.store(static_cast<uint32_t>(bytes), std::memory_order_release);
    return e;
}

constexpr int kMaxRows = 16;   // verify rows per MoE call (4 slots x (1 + 3 drafts))
constexpr int kMaxPrefillRows = 2048;  // prefill-width rows per MoE call
constexpr int kMaxTopK = 16;
constexpr int kHeadCap = 256;  // exact-pass candidates kept per row before the full fallback

struct ProjDev {
    const uint32_t* codes;   // [experts, OUT, words]
    const uint16_t* scales;  // [experts, OUT, ngrp] fp16
    const uint16_t* book;    // [2^bits, dim] fp16 (null for an INT8 codebook)
    const uint16_t* book4;   // [dim/4, 2^bits, 4] fp16: the codebook split into 4-dim chunks
    int words, ngrp, dim, bits;
    const int8_t* book_i8;   // [2^bits, dim] int8 codebook (value = q * book_scale), or null
    float book_scale;
    // The codes again, tiled for the verify kernels (or null): 64-row tiles of the flattened
    // [experts * OUT] rows; per (tile, 32-code block) the 64 rows' BITS words are stored as
    // chunks of 4 words (the last chunk BITS % 4 wide when not 0) with the 64 rows
    // interleaved inside each chunk, so one 16-byte load per lane reads 1 KiB contiguously.
    const uint32_t* codes_t;
    // A per-dimension INT8/U8 book in the form the U8 verify kernels read (or null): [2^bits][8]
    // bytes u (the centred book's codes offset by 128, u = q + 128), and u8_sb = 16 floats,
    // the per-dimension scale s[8] then the offset b[8] (the affine book's min, -128 s for the
    // centred book), so that the decoded weight is u * s[d] + b[d].
    const uint8_t* book_u8;
    const float* u8_sb;
};

// Workspace views of one MoE call (rows <= kMaxRows).
struct MoeBufs {
    uint16_t* x;       // [M, H] bf16 normalised layer input
    uint16_t* x16;     // [M, H] fp16 copy of x (MFMA operand)
    float* logits;     // [M, E]
    float* sgate;      // [M] sigmoid(x . w_sg) rounded to bf16
    int32_t* experts;  // [M*K]
    float* weights;    // [M*K]
    int32_t* plan;     // [2 + 4*M*K]
    // Projection partial sums, one plane per codebook chunk (summed chunk 0 + chunk 1 by the
    // consumer). g / u rows in sorted route order, d rows at the route index (row * K +
    // slot); shared-expert rows last (M*K + row).
    float* g;          // [2][M*K + M, I] gate
    float* u;          // [2][M*K + M, I] up
    float* d;          // [2][M*K + M, H] down
    uint16_t* h16;     // [M*K + M, I] fp16 SwiGLU rows (prefill path; the U8 down operand)
    // [M*K + M] per-route correction of the U8 down kernel; it shares the storage of g's second
    // plane, which the U8 path (one plane) leaves unused.
    float* dcorr;
    size_t gu_plane;   // floats between the chunk planes of g and u
    size_t d_plane;    // floats between the chunk planes of d
    // Re-reads a bounded wait between workgroups of one launch makes before it gives up
    // (kWaitLimit; smaller only when a test forces the give-up path).
    int wait_limit;
};

// A projection in MLX affine form: packed values, per-group scales and biases.
struct AffineDev {
    const uint32_t* w;  // [OUT][IN * bits / 32], value j of a word at bits j * bits
    const uint16_t* s;  // [OUT][IN / group]
    const uint16_t* b;  // [OUT][IN / group]
};

struct LayerDev {
    const uint16_t* router;  // [E, H] bf16
    const uint16_t* wsg;     // [H] bf16
    ProjDev p[3];            // gate, up, down
    int H, I, E, K, normalize, has_shared;
    int gu_parts, d_parts;   // chunk planes written by the gate/up and down kernels (1 or 2)
    // Mixed geometry: pb[p][0] holds the even experts (index e/2; the shared expert E is
    // even) as d4/8-bit with an fp16 codebook, pb[p][1] the odd experts (index e/2) as
    // d8/14-bit with an INT8 codebook.
    int mixed;
    ProjDev pb[3][2];
    const float* rbias;      // [E] additive router-logit bias (device) or null
    // The call's choice of the one-launch layer kernel (k_gd4), fixed by moe_call_dev so that
    // the router (which resets the planes that kernel waits on) and the expert launch agree:
    // 0 undecided (decided from the layer on each query), 1 fused, 2 not fused.
    int fused_mode;
    // The shared expert in MLX affine form (shared_affine 1; the reference checkpoints'
    // format): gate and up [sa_inter][H], down [H][sa_inter], sa_bits-bit values, one scale and
    // bias per sa_group inputs, bf16 (sa_f16 0) or fp16. The expert kernels then take the layer
    // without a shared slot (expert_view); the router (shared gate) and the combine keep it.
    AffineDev sa[3];
    int shared_affine, sa_bits, sa_group, sa_inter, sa_f16;
    // u8_native: the three projections carry U8 books the U8 verify kernels read (d8/14-bit,
    // H 2048, I 512, per-row scales, no affine shared expert). u8_call: this call runs them
    // (moe_call_dev: 1-16 rows while they are enabled); it then writes one partial-sum plane.
    int u8_native, u8_call;
};

// The view of a layer the routed-expert kernels take: without the shared slot when the shared
// expert is affine (its down rows come from launch_shared_affine).
inline LayerDev expert_view(const LayerDev& L) {
    LayerDev v = L;
    if (L.shared_affine) v.has_shared = 0;
    return v;
}

struct HeadDev {
    const int8_t* w;         // Q8: [V, H]; Q4: [V, H/2] packed nibbles
    const uint16_t* scales;  // Q8: [V]; Q4: [V, H/64]
    int64_t V;
    int H, kind;
    float s_max;             // max |scale| over the head (exact-pass window)
};

// MoE layer (rows M <= kMaxRows)
// Router logits of the layer input: norm = false: src is x (copied to B.x / B.x16 unless it
// is B.x); norm = true: src is the residual stream h and x = RMSNorm(h) (eps) is formed
// first (the verify chain).
hipError_t launch_router(const LayerDev& L, const MoeBufs& B, int M, const uint16_t* src, bool norm, float eps,
                         hipStream_t st);
hipError_t launch_topk_plan(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st);
hipError_t launch_gate_up(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st);
// the grouped-scale (VALU) kernels of launch_gate_up / launch_down (q38_moe_grp.hip)
hipError_t launch_gate_up_grouped(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st);
hipError_t launch_down_grouped(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st);
// GatedDeltaNet verify step (q38_gdn.hip). Projections p: 0 qkv [C, H], 1 z [HV DV, H],
// 2 b [HV, H], 3 a [HV, H], 4 out [H, HV DV], MLX affine (bits, group, bf16 / fp16 scales).
// Several MLX affine projections of the same rows in one launch (k_affine_rows): weight rows
// [out, IN] (packed values, scales and biases [out][IN / group]), outputs rounded to bf16 into
// dst rows of stride dst_stride.
struct AffineRows {
    const uint32_t* w;
    const uint16_t* s;
    const uint16_t* b;
    uint16_t* dst;
    int out, dst_stride, first_block;
};
struct AffineRowSet {
    AffineRows p[4];
    int n;
};
hipError_t launch_affine_rows(const AffineRowSet& set, const uint16_t* x, int S, int IN, int G, int bits, int f16,
                              hipStream_t st);

// Full attention, verify (q38_attn.hip): geometry, the projections' tensors (q, k, v, o), the
// effective q / k norm weights [D] (1 + w formed at creation for offset norms).
struct AttnDev {
    int hidden, hq, hkv, d, rot, bits, group, f16;
    float eps;
    double theta;
    const uint32_t* w[4];
    const uint16_t* s[4];
    const uint16_t* b[4];
    const uint16_t* qn;
    const uint16_t* kn;
};
// Workspace of one call: projection outputs qg [S][2 HQ D], kr / vr [S][HKV D]; queries q and
// gates gs [S][HQ][D]; scores sc [S HQ][score stride]; per (score tile, query) max and sum
// stats; per-query max and sum; P.V partials [tiles][S HQ][D]; gated rows [S][HQ D].
struct AttnBufs {
    uint16_t *qg, *kr, *vr, *q, *gs, *sc;
    float2* stats;
    float *mx, *sm, *part;
    uint16_t* gated;
};
bool attn_geometry_ok(int hidden, int hq, int hkv, int d, int rot);
int64_t attn_score_stride(int64_t tokens);
int64_t attn_pv_tiles(int64_t tokens);
int64_t attn_score_tiles(int64_t tokens);
hipError_t launch_attn_verify(const AttnDev& A, const AttnBufs& B, int S, const uint16_t* x, uint16_t* keys,
                              uint16_t* values, int64_t cap, int64_t T0, int64_t position, uint16_t* out,
                              hipStream_t st);

// The decoder's MLP output map (q38_map.hip): rank 0 = the full map full [H][H]; otherwise
// the low-rank pair left [H][rank], right [rank][H]; bf16.
struct MlpMapDev {
    int hidden, rank;
    const uint16_t* full;
    const uint16_t* left;
    const uint16_t* right;
};
size_t mlp_map_workspace(int hidden, int rank, int rows);
hipError_t launch_mlp_map(const MlpMapDev& m, const uint16_t* y, int rows, uint16_t* out, void* ws, hipStream_t st);

struct GdnDev {
    int hidden, hk, hv, dk, dv, bits, group, f16, gate_silu;
    float eps;
    const uint32_t* w[5];
    const uint16_t* s[5];
    const uint16_t* b[5];
    const uint16_t* conv_w;   // [C][4] bf16
    const float* a_log;       // [HV]
    const uint16_t* dt_bias;  // [HV] bf16
    const uint16_t* norm_w;   // [DV] bf16
};
// Workspace views of one verify call of S rows (bf16 unless noted).
struct GdnBufs {
    uint16_t *qkv, *z, *bpr, *apr;  // projections [S][C], [S][HV DV], [S][HV] x 2
    uint16_t *q, *k, *v;            // [S][HK DK] x 2, [S][HV DV]
    float *beta, *decay;            // [S][HV] (bf16 values)
    uint16_t *y, *gated;            // [S][HV DV]
};
bool gdn_geometry_ok(const GdnDev& G);
hipError_t launch_gdn_verify(const GdnDev& G, const GdnBufs& B, int S, const uint16_t* x, const uint16_t* origin,
                             uint16_t* ckpt, uint16_t* out, hipStream_t st);

// Prefill widths (kMaxRows < M) on the grouped kernels: layouts the segmented MFMA kernels
// do not take (scale groups, d4 and d2 codes)
bool moe_supports_grouped_prefill(const LayerDev& L);
// The affine shared expert of the call's rows (q38_affine.hip): SwiGLU rows into B.h16, then
// its down outputs into the shared rows of the down planes (plane 0; plane 1 cleared). Runs
// after the router (it reads B.x) and before the combine; nothing without shared_affine.
hipError_t launch_shared_affine(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st);
hipError_t launch_down(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st);
// chain: h <- h + y (in place); otherwise out <- y. Down rows are read at the route index.
hipError_t launch_combine(const LayerDev& L, const MoeBufs& B, int M, uint16_t* h, uint16_t* out, hipStream_t st);
// The combine followed by the HyperConnection write of the layer output into hs ([M][HC][H]
// bf16, in place) with the per-row stream gates inj ([M][HC] bf16).
hipError_t launch_combine_hc(const LayerDev& L, const MoeBufs& B, int M, uint16_t* hs, const uint16_t* inj, int HC,
                             hipStream_t st);
hipError_t launch_rmsnorm(const uint16_t* x, int M, int H, float eps, uint16_t* y, hipStream_t st);
// The same with a learned weight w [H] bf16: y = T(T(x * inv_rms) * w) (MLX rms_norm's rounding).
hipError_t launch_rmsnorm_w(const uint16_t* x, int M, int H, float eps, const uint16_t* w, uint16_t* y,
                            hipStream_t st);
hipError_t launch_split_book(const uint16_t* book, int entries, int dim, uint16_t* book4, hipStream_t st);
hipError_t launch_split_book_i8(const int8_t* book, float scale, int entries, int dim, uint16_t* book4,
                                hipStream_t st);
// codes [rows, words] (rows a multiple of 64) -> the tiled layout of ProjDev::codes_t
hipError_t launch_tile_codes(const uint32_t* codes, int64_t rows, int words, int bits, uint32_t* out, hipStream_t st);
bool moe_uses_mfma(const LayerDev& L);
// The MFMA layers' geometry, whatever the scale groups.
bool moe_uses_mfma_geometry(const LayerDev& L);
// Mixed layer on the MFMA kernels (both banks prepared); the gate/up kernels of both the
// uniform and the mixed MFMA paths route and build the plan themselves.
bool moe_mixed_mfma(const LayerDev& L);
bool moe_plans_in_gate_up(const LayerDev& L, int M);
// Verify widths of up to 4 rows on the 4x4x4 MFMA kernels (q38_moe4.hip): the MFMA layers,
// and d8 layers of the same geometry with per-64-input scale groups. They write one partial-
// sum plane per codebook chunk (gu_parts / d_parts of the call: moe_call_dev).
bool moe_uses_narrow(const LayerDev& L, int M);
// The layer view of a call of M rows: the partial-sum plane counts of the kernels it takes.
LayerDev moe_call_dev(const LayerDev& L, int M);
// Verify widths (1-16 rows) of layers with U8 books on the kernels that read the books
// themselves (k_gu_u8, k_swiglu_u8, k_dn_u8), by mode: 0 never (the decoded fp16 books on the
// other verify kernels), 1 (default) at 5-16 rows and at 1-4 rows where the one-launch layer
// is not taken, 2 at every verify width.
bool moe_u8_call(const LayerDev& L, int M);
void set_u8_native(int mode);
// The U8 kernels' operands of a per-dimension book: u = q (+ 128 when centred) as bytes and
// the 16 floats s[8], b[8] (ProjDev::book_u8, u8_sb).
hipError_t launch_u8_operands(const void* q, int K, int centered, const uint16_t* s16, const uint16_t* b16,
                              uint8_t* u, float* sb, hipStream_t st);
hipError_t launch_gate_up4(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st);
hipError_t launch_down4(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st);
// The d8/14-bit, H 2048, I 512, top-10, per-row-scale layers at up to 4 rows run gate/up and
// down in one launch (k_gd4), and with h or out set the combine too (h <- h + y in place, or
// out <- y): launch_gate_up takes it without the combine, launch_down then has nothing to
// launch. The router kernel before it resets the gate/up and down planes the launch waits on.
bool moe_uses_fused(const LayerDev& L, int M);
// The one-launch kernel's workgroups wait for each other, so it is taken only while it is
// enabled (q38_set_fused_layers) and the compiled kernels fit one workgroup per CU with the
// grid no larger than the CU count (checked once per device).
void set_fused_enabled(bool on);
// Bounded waits between workgroups: re-reads before a wait gives up, and the device status
// word that a wait which gave up sets (bit 0). read_wait_status synchronises the device's
// null stream with the copy (the caller synchronises its own stream first).
constexpr int kWaitLimit = 1 << 16;
void set_wait_limit(int spins);  // < 0: kWaitLimit
int wait_limit();
hipError_t read_wait_status(uint32_t* status, bool clear);
// HC > 0: h holds the rows' HC streams, and the combine writes the output into every stream
// with the injection weights inj ([M][HC]) as k_combine_hc does.
hipError_t launch_gate_down4(const LayerDev& L, const MoeBufs& B, int M, uint16_t* h, uint16_t* out, hipStream_t st,
                             const uint16_t* inj = nullptr, int HC = 0);
int mfma_grid();  // persistent workgroups of the expert kernels (a multiple of 32)
// Prefill widths, kMaxRows < M <= kMaxPrefillRows (q38_moe_pf.hip), one kernel each:
// router logits, per-row top-k, sorted plan, segmented gate/up, SwiGLU, segmented down
// (gate/up/down write one plane each).
bool moe_supports_prefill(const LayerDev& L);
hipError_t launch_router_rows(const LayerDev& L, const MoeBufs& B, int M, const uint16_t* x, hipStream_t st);
hipError_t launch_topk_rows(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st);
hipError_t launch_plan_sort(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st);
// Partial-sum planes the prefill gate/up and down kernels write: 2 on the LDS-codebook
// kernels (one per codebook chunk), 1 on the tile kernels.
int prefill_planes(const LayerDev& L, int M);
hipError_t launch_gate_up_pf(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st);
hipError_t launch_swiglu_pf(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st);
hipError_t launch_down_pf(const LayerDev& L, const MoeBufs& B, int M, hipStream_t st);

// generators
// codes of experts e0, e0 + e_stride, ... (n_experts of them), stored contiguously
hipError_t launch_gen_codes(uint64_t key, int e0, int e_stride, int n_experts, int out_dim, int nsub, int bits,
                            int words, uint32_t* codes, hipStream_t st);
// per-row scales of experts e0, e0 + e_stride, ...: out[i * out_dim + o] = uniform at (e * out_dim + o)
hipError_t launch_gen_scales(uint64_t key, int e0, int e_stride, int n_experts, int out_dim, double lo, double hi,
                             uint16_t* out, hipStream_t st);
hipError_t launch_gen_uniform_f16(uint64_t key, int64_t idx0, int64_t n, double lo, double hi, uint16_t* out,
                                  hipStream_t st);
hipError_t launch_gen_normal(uint64_t key, int64_t n, double sd, int f16, uint16_t* out, hipStream_t st);
hipError_t launch_gen_embed(uint64_t seed, const uint32_t* tokens, int n, int H, uint16_t* out, hipStream_t st);
hipError_t launch_gen_embed_dev(uint64_t seed, const uint32_t* tokens_dev, int n, int H, uint16_t* out,
                                hipStream_t st);
hipError_t launch_book_to_int8(const uint16_t* book16, int n, int8_t* q8, uint16_t* scale, hipStream_t st);
// Per-dimension INT8 (centred) / U8 (affine) codebook of a [K, 8] fp16 book: q [K*8], scales
// and biases [8] fp16, and the decoded book [K*8] fp16.
hipError_t launch_prepare_u8(const uint16_t* book16, int K, int centered, uint8_t* q, uint16_t* s16, uint16_t* b16,
                             uint16_t* dec, hipStream_t st);
hipError_t launch_gen_head(const HeadDev& hd, uint64_t seed, int8_t* w, uint16_t* scales, hipStream_t st);
hipError_t launch_scale_absmax(const uint16_t* scales, int64_t n, float* out, hipStream_t st);

// heads
// Head workspace; the logits path uses the leading part (planes .. best) only.
struct HeadWork {
    int8_t* planes;     // [3, M, H] int8 planes of the request rows
    float* hscale;      // [M] plane scale (a power of two)
    float* res;         // [M] sum |h - plane reconstruction|
    float* tsum;        // [M] sum |h|
    uint32_t* rowmax;   // [M] orderable
    int32_t* cnt;       // [M]
    unsigned long long* best;  // [M]
    int32_t* cand;      // [M, kHeadCap] (greedy)
    float* fast;        // [M, V] (greedy)
};
constexpr int kHeadMaxRows = 16;
// The draft step's prologue (k_draft_prologue): embedding / stream rows, their RMSNorms and
// the Q8 planes of the FC projections' rows.
struct DraftPro {
    uint64_t embed_key;
    const uint32_t* toks;               // step tokens, or null: take them from best
    const unsigned long long* best;     // the previous step's argmax keys
    const unsigned long long* part;     // or (non-null) its Q4 head's partial keys [M][nparts]
    int nparts;
    uint32_t* drafts;                   // (chain) the previous step's drafts [M][depth]
    uint32_t* tokens_out;
    int depth, prev_step;
    const uint16_t* stream;             // [M][HC * H]
    int H, HC, M;
    float eps;
    const uint16_t* emb_norm;           // [H] or null
    const uint16_t* hid_norm;           // [HC * H] or null
    HeadWork we;                        // the embedding projection's rows
    HeadWork wh[4];                     // the stream projection's passes of up to 16 rows
    int mh[4];
};
hipError_t launch_draft_prologue(const DraftPro& P, hipStream_t st);
hipError_t launch_argmax_rows(const float* logits, int M, int64_t V, unsigned long long* best, hipStream_t st);
// The Q4 head's logits with each workgroup's argmax key per row in part ([M][q4_blocks(M)]
// u64), and the decode of row r's maximum of such keys into tokens / values /
// drafts[r * depth + step] (each may be null).
constexpr int kQ4MaxBlocks = 2048;
int q4_blocks(int M);
hipError_t launch_head_q4_part(const HeadDev& hd, const uint16_t* h, int M, float* logits, unsigned long long* part,
                               hipStream_t st);
hipError_t launch_argmax_part_final(const unsigned long long* part, int n, int M, uint32_t* tokens, float* values,
                                    uint32_t* drafts, int depth, int step, hipStream_t st);
hipError_t launch_head_logits_prepared(const HeadDev& hd, int M, const HeadWork& w, float* logits, hipStream_t st);
size_t head_work_bytes(const HeadDev& hd, int M, bool greedy);
HeadWork head_work_carve(void* base, const HeadDev& hd, int M, bool greedy);
hipError_t head_init_attrs();
hipError_t launch_head_greedy(const HeadDev& hd, const uint16_t* h, int M, const HeadWork& w, uint32_t* argmax,
                              float* logit, hipStream_t st);
hipError_t launch_head_logits(const HeadDev& hd, const uint16_t* h, int M, const HeadWork& w, float* logits,
                              hipStream_t st);

// draft head: x = T(T(a) + T(b)) over n values, clearing best[0..M) (best may be null)
hipError_t launch_fc_join(const float* a, const float* b, int M, int HC, int H, uint16_t* x, unsigned long long* best,
                          hipStream_t st);
// Row argmax of logits [M, V] (ties to the lowest index) into best[M] (cleared first when
// `clear`, else it must hold 0), decoded into tokens / values / drafts[r * depth + step]
// (each may be null). M <= 64.
hipError_t launch_argmax(const float* logits, int M, int64_t V, unsigned long long* best, bool clear,
                         uint32_t* tokens, float* values, uint32_t* drafts, int depth, int step, hipStream_t st);

// acceptance
// k <= 24; ws: accept_sampled_workspace(k, V) bytes.
size_t accept_sampled_workspace(int k, int64_t V);
// Softmax of rows [rows, V] float at temperature T: stats [rows][2] = (max, sum of
// exp((l - max) / T)) and, when probs is given (it may be logits), the probabilities.
// ws: softmax_rows_workspace(rows, V) bytes.
size_t softmax_rows_workspace(int rows, int64_t V);
hipError_t launch_softmax_rows(const float* logits, int rows, int64_t V, float T, float* stats, float* probs, void* ws,
                               hipStream_t st);
hipError_t launch_accept_sampled(const float* tl, const float* dl, const uint32_t* drafts, int k, int64_t V,
                                 float T, uint64_t seed, uint64_t slot, uint64_t round, int64_t* out, void* ws,
                                 hipStream_t st);

// HyperConnection mixer (streams of H values per row; MLX affine-quantised projections with
// 32 / bits values per packed word, one bf16 scale and bias per G inputs).
constexpr int kHcMaxPerThread = 16;  // H <= 4096 (H / 256 values per normalisation thread)
constexpr int kHcMaxRank = 512;
constexpr int kHcMaxStreams = 16;
struct HcDev {
    int H, HC, R, bits, G, with_inj;
    float eps;
    const uint16_t* wn;                       // [HC * H] bf16: 1 + hc_norm.weight
    const uint32_t* dw;                       // down [R][HC * H / vpw]
    const uint16_t *ds, *db;                  //      [R][HC * H / G]
    const uint32_t* uw;                       // up [HC * H][R / vpw]
    const uint16_t *us, *ub;                  //    [HC * H][R / G]
    const uint32_t* iw;                       // injection [HC][HC * H / vpw] (with_inj)
    const uint16_t *is, *ib;                  //           [HC][HC * H / G]
};
size_t hc_up_lds_max();
// xn: [M][HC * H] bf16 and act: [M][R] float of the workspace; mixed [M][H], inj [M][HC] bf16
// (inj unused without injection).
hipError_t launch_hc_read(const HcDev& D, int M, const uint16_t* stream, uint16_t* xn, float* act, uint16_t* mixed,
                          uint16_t* inj, hipStream_t st);
hipError_t launch_hc_write(int H, int HC, int M, const uint16_t* stream, const uint16_t* block_out,
                           const uint16_t* inj, uint16_t* out, hipStream_t st);
hipError_t launch_hc_tile(int H, int HC, int M, const uint16_t* emb, uint16_t* out, hipStream_t st);
hipError_t launch_hc_norm_weight(const uint16_t* raw, int n, uint16_t* wn, hipStream_t st);

} // namespace q38
