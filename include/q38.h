/* q38.h — C ABI of the MI355X (gfx950) MTP verification round.
 *
 * This is the drop-in boundary: plain C types, device pointers and sizes, no C++ or
 * torch types. The C++20 host mirror (qwen38::SparseMoe, verify/commit, run round)
 * sits on top of it; a ctypes binding sits beside it. Every entry point names the
 * reference interface it replaces (paths relative to the reference checkout).
 *
 * Conventions
 *   - Return 0 on success, a negative Q38_E* code otherwise; q38_last_error() gives a
 *     thread-local message. No C++ exception crosses this ABI. A failed validation
 *     leaves every output and state untouched.
 *   - Tensors are row-major. bf16 / fp16 values travel as uint16_t bit patterns.
 *   - Pointers documented as "device" are HBM addresses; all device work is ordered on
 *     the caller's stream (a hipStream_t passed as void*; NULL = the null stream). The
 *     only host synchronisation is where the reference reads back token ids.
 *   - Handles own the memory they allocate; callers own their I/O buffers.
 *   - One layer / head handle may be used by one stream at a time.
 */
#ifndef Q38_H
#define Q38_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    Q38_OK = 0,
    Q38_EINVAL = -1,  /* bad argument / shape                 (std::runtime_error) */
    Q38_ERANGE = -2,  /* out of range (short packed buffer)   (std::out_of_range)  */
    Q38_EHIP = -3,    /* HIP runtime failure */
    Q38_ENOMEM = -4,  /* allocation failure */
    Q38_ESTATE = -5,  /* invalid lifecycle / commit request   (std::runtime_error) */
    Q38_ESPACE = -6,  /* workspace too small */
    Q38_EWAIT = -7    /* a bounded wait between workgroups gave up (q38_ctx_synchronize) */
};

typedef struct q38_ctx q38_ctx;
typedef struct q38_moe_layer q38_moe_layer;
typedef struct q38_head q38_head;
typedef struct q38_slot q38_slot;

/* Codebook formats. Q38_CB_FP16: the FP16 books as given. Q38_CB_INT8_SCALED: the mixed
 * layout's INT8 d8 books with one FP16 scale per book. Q38_CB_U8_PERDIM: the reference's
 * verify-width books (SparseMoe::prepare_u8_codebook, src/sparse_moe.cpp:528-544, 750-804),
 * derived at layer creation from the FP16 books of the d8/14-bit projections: per-dimension
 * min/max, scale = (max - min) / 255, a centred INT8 gate book and affine U8 up/down books
 * with FP16 scale and bias per dimension, decoded as q * scale (+ bias). */
enum { Q38_CB_FP16 = 0, Q38_CB_INT8_SCALED = 1, Q38_CB_U8_PERDIM = 2 };

/* Layer description. Mirrors the SparseMoe constructor arguments
 * (include/qwen38/sparse_moe.hpp:48-55) plus the VQ geometry of the projection tensors
 * (src/sparse_moe.cpp:618-661, include/qwen38/quantization_geometry.hpp:12-17). */
typedef struct q38_moe_desc {
    int32_t hidden;        /* H, multiple of 512 (2048; 2560 in the reference family) */
    int32_t inter;         /* I, expert intermediate, multiple of 128 (512; 640)      */
    int32_t experts;       /* E routed experts, multiple of 64, <= 1024 (512)         */
    int32_t top_k;         /* experts per token, <= 16 (10)                           */
    int32_t gu_dim, gu_bits;     /* gate/up VQ geometry: (8,14) or (4,8)              */
    int32_t down_dim, down_bits; /* down VQ geometry:    (8,14) or (4,8)              */
    int32_t gu_group, down_group;/* scale group along the input; == input = per row   */
    int32_t normalize_topk;      /* normalize_topk_probability                        */
    int32_t has_shared;          /* shared expert (expert index E) + sigmoid gate     */
    int32_t mixed;               /* 1: even experts d4/8-bit FP16 books, odd experts
                                    d8/14-bit INT8 books with one FP16 scale each     */
    int32_t book_format;         /* uniform layers: Q38_CB_FP16 or Q38_CB_U8_PERDIM   */
} q38_moe_desc;

/* Device tensors of one layer (uniform geometry). The layer adopts the pointers; the
 * caller keeps them alive for the layer's lifetime. The tensors must be final when the
 * layer is created: creation copies the codebooks (re-laid in 4-dim chunks, or derived
 * per-dimension U8 books) and, for layers the <= 4-row kernels serve, the packed codes
 * (tiled); those kernels read the copies while wider calls read the originals, so a
 * later in-place change would make the two disagree. Expert index E is the shared expert.
 *   router       [E, H] bf16                      (SparseMoe::router_,  sparse_moe.hpp:201)
 *   shared_gate  [H] bf16 (w_sg)                  (shared_router_,       sparse_moe.hpp:209)
 *   codes[p]     [E+1, OUT_p, words_p] u32, words_p = ceil(IN_p/D/32)*BITS (E rows without a
 *                shared expert)
 *   scales[p]    [E+1, OUT_p, IN_p/G_p] fp16 (E rows without a shared expert)
 *   books[p]     [2^BITS, D] fp16
 * p = 0 gate, 1 up, 2 down. */
typedef struct q38_moe_weights {
    const uint16_t* router;
    const uint16_t* shared_gate;
    const uint32_t* codes[3];
    const uint16_t* scales[3];
    const uint16_t* books[3];
} q38_moe_weights;

/* Device tensors of a mixed-geometry layer (desc->mixed = 1; hidden 2048, inter 512,
 * one scale per output row). Expert e uses bank e % 2 at index e / 2; the shared expert
 * (index E, even) is the last entry of bank 0.
 *   bank 0 (even): codes_d4[p] [E/2+1, OUT_p, ceil(IN_p/4/32)*8] u32 (8-bit codes),
 *                  scales_d4[p] [E/2+1, OUT_p] fp16, books_d4[p] [256, 4] fp16
 *   bank 1 (odd):  codes_d8[p] [E/2, OUT_p, ceil(IN_p/8/32)*14] u32 (14-bit codes),
 *                  scales_d8[p] [E/2, OUT_p] fp16, books_d8[p] [16384, 8] int8 with one
 *                  fp16 scale per codebook, book_scales_d8[p] (value = q * scale)
 * (the per-expert geometry of the reference's mixed VQ v2 layers, src/sparse_moe.cpp:
 * 539-544, 2249-2258; INT8 codebooks as in SparseMoe::prepare_u8_codebook,
 * src/sparse_moe.cpp:750-804, with one scale per codebook). */
typedef struct q38_moe_mixed_weights {
    const uint16_t* router;
    const uint16_t* shared_gate;
    const uint32_t* codes_d4[3];
    const uint16_t* scales_d4[3];
    const uint16_t* books_d4[3];
    const uint32_t* codes_d8[3];
    const uint16_t* scales_d8[3];
    const int8_t* books_d8[3];
    uint16_t book_scales_d8[3];
    uint16_t reserved;
} q38_moe_mixed_weights;

/* Routing outputs (optional, device). */
typedef struct q38_route_out {
    int32_t* experts;   /* [rows*k] ids in rank order                                  */
    float* weights;     /* [rows*k]                                                    */
    float* logits;      /* [rows*E] router logits (BF16 values widened to float)       */
    int32_t* plan;      /* [1 + 4*rows*k + 1]: n_unique, uexp[rows*k], uoff[rows*k+1],
                           route_list[rows*k], route_pos[rows*k]; past n_unique, uexp
                           holds -1 and uoff rows*k (verify widths)                    */
    uint16_t* x_norm;   /* [rows*H] the normalised layer input (chain mode)            */
} q38_route_out;

/* ------------------------------------------------------------------ context */
int q38_ctx_create(int hip_device, q38_ctx** out);
void q38_ctx_destroy(q38_ctx* ctx);
const char* q38_last_error(void);
const char* q38_version(void);

/* ------------------------------------------------------------------ geometry (host)
 * packed_vq_word_count / unpack_vq_code: src/quantization_geometry.cpp:37-67.
 * supports_segmented_vq: include/qwen38/quantization_geometry.hpp:12-17. */
int64_t q38_packed_vq_word_count(int64_t code_count, int bits_per_code);
int q38_unpack_vq_code(const uint32_t* words, int64_t n_words, int64_t code_index, int bits_per_code,
                       uint32_t* out);
int q38_supports_segmented_vq(int dimension, int packed_bits);

/* ------------------------------------------------------------------ MoE layer
 * Replaces SparseMoe (include/qwen38/sparse_moe.hpp:46-214). */
int q38_moe_layer_create(q38_ctx* ctx, const q38_moe_desc* desc, const q38_moe_weights* weights,
                         q38_moe_layer** out);
/* SparseMoe(MlxTensorStore&, prefix, ...) (include/qwen38/sparse_moe.hpp:48-55) over an
 * on-disk checkpoint directory: config.json's vq_modules (src/model_manifest.cpp:210-230)
 * and safetensors tensors prefix.switch_mlp.{gate,up,down}_proj.{codes,codebook,vq_scales}
 * checked against the reference's tensor contract (src/sparse_moe.cpp:618-661), the BF16
 * router prefix.gate.weight, and a VQ shared expert (prefix.shared_expert.*_proj with the
 * routed codebook, prefix.shared_expert_gate.weight) when present. U32 packed codes
 * (pack_bits 1..31) and byte codes (pack_bits 0: d2/K256) load; top-k and normalisation
 * come from the config. The layer owns the device copies of its tensors. */
int q38_moe_layer_load(q38_ctx* ctx, const char* checkpoint_dir, const char* prefix, int32_t book_format,
                       q38_moe_layer** out);
/* The layer description a checkpoint gives for prefix, after the same checks, without
 * device work (book_format left 0). */
int q38_checkpoint_inspect(const char* checkpoint_dir, const char* prefix, q38_moe_desc* desc);
/* Mixed-geometry layer (desc->mixed = 1) over caller-owned tensors. Allocates the INT8
 * books decoded to fp16 chunks (3 x 256 KiB) for the MFMA kernels. */
int q38_moe_layer_create_mixed(q38_ctx* ctx, const q38_moe_desc* desc, const q38_moe_mixed_weights* weights,
                               q38_moe_layer** out);
/* Library-owned synthetic layer: every tensor generated from (seed, layer_index) by the
 * counter-based generator, on the device (uniform or, with desc->mixed, mixed geometry). */
int q38_moe_layer_create_synthetic(q38_ctx* ctx, const q38_moe_desc* desc, uint64_t seed,
                                   int32_t layer_index, q38_moe_layer** out);
void q38_moe_layer_destroy(q38_moe_layer* layer);
/* Device pointers of a layer's tensors (uniform geometry, as given at creation) for
 * inspection. */
int q38_moe_layer_weights(const q38_moe_layer* layer, q38_moe_weights* out);
/* The bank tensors of a mixed layer (as given to q38_moe_layer_create_mixed, or generated). */
int q38_moe_layer_mixed_weights(const q38_moe_layer* layer, q38_moe_mixed_weights* out);
/* The codebook the kernels read for projection p (0 gate, 1 up, 2 down): device [2^BITS, D]
 * fp16. With Q38_CB_U8_PERDIM and a d8/14-bit projection it is the decoded per-dimension
 * book (q * scale (+ bias) rounded to fp16, the MFMA operand type), and q (int8 centred for
 * the gate, uint8 affine otherwise, [2^BITS, D]), scales [D] and biases [D] (fp16) are the
 * derived tables (the reference's codebook_u8, codebook_u8_scales and codebook_u8_biases);
 * otherwise the FP16 book as given and null tables. Outputs may be null. */
int q38_moe_layer_codebook(const q38_moe_layer* layer, int proj, const uint16_t** book, const void** q,
                           const uint16_t** scales, const uint16_t** biases);
/* Algorithmic HBM bytes of one forward that touches n_unique routed experts. */
int64_t q38_moe_layer_bytes(const q38_moe_layer* layer, int32_t n_unique, int32_t rows);
/* Completion check of the stream's work on the context's device. The one-launch verify
 * layer (d8/14-bit, H 2048, I 512, top-10, 1-4 rows; see q38_verify_chain) passes values
 * between its workgroups, which wait for each other with bounded waits; a wait that gives up
 * (the grid was not resident at once: the device shared with other work) leaves NaN outputs
 * and sets a status bit on the device. This call synchronises `stream`, then returns
 * Q38_EWAIT if any such wait gave up on the device since the last check (and clears the
 * bit), Q38_OK otherwise. No counterpart in the reference (its Metal dispatches do not wait
 * on each other); the C++ mirror calls it wherever it reads tokens back
 * (src/mtp_verifier.cpp:47-52). */
int q38_ctx_synchronize(q38_ctx* ctx, void* stream);

/* Process-wide switch (default on): 0 makes every later call take the multi-kernel layer
 * (gate/up, down and combine as separate launches, no waits between workgroups) instead of
 * the one-launch kernel. The one-launch kernel is also taken only where the device fits its
 * grid at one workgroup per CU (checked once per device against the kernel's occupancy). */
void q38_set_fused_layers(int enable);

/* Process-wide mode for layers with Q38_CB_U8_PERDIM books whose three projections are
 * d8/14-bit with per-row scales (H 2048, I 512, no affine shared expert): which verify widths
 * run on the kernels that read the per-dimension INT8/U8 books themselves (the reference's
 * verify-width decode, src/vq_metal_kernels.hpp:564-579, which forms w = q * scale (+ bias)
 * per weight): one 8-byte entry per subvector from a book held whole in LDS, the
 * per-dimension scale applied to the inputs and the bias as a per-row sum. 0: none (the
 * decoded fp16 book on the other kernels); 1 (default): 5-16 rows, and 1-4 rows where the
 * one-launch layer kernel is not taken (it is faster at those widths); 2: 1-16 rows.
 * No counterpart in the reference. */
void q38_set_u8_native(int mode);

/* Test hook: the number of re-reads a bounded wait makes before it gives up (default 65536,
 * about 0.1 s; a negative value restores it). A limit of 0 makes a wait give up at its first
 * read of a value another workgroup has not stored yet, so tests can reach the give-up path
 * while every kernel still runs to its end. */
void q38_debug_set_wait_limit(int32_t spins);

/* Shared expert in MLX affine form: the only shared-expert format of the reference's
 * checkpoints (SparseMoe::load_projection's affine branch, src/sparse_moe.cpp:474-480,
 * 662-700, applied by SparseMoe::forward_shared, :1306-1313, through quantized_matmul).
 * Projection p = gate, up (OUT = inter, IN = hidden), down (OUT = hidden, IN = inter):
 *   weight[p]  [OUT, IN * bits / 32] u32, value j of a word at bits j * bits (LSB first)
 *   scales[p], biases[p]  [OUT, IN / group], bf16 (scale_dtype 0) or fp16 (1)
 * w[o, c] = scale[o, c / group] * q[o, c] + bias[o, c / group]. bits 2, 4 or 8; group 32, 64
 * or 128; inter <= 4096 (its own size: SparseMoe's shared_expert_intermediate_size). Device
 * pointers, adopted like q38_moe_weights. */
typedef struct q38_affine_shared {
    const uint32_t* weight[3];
    const uint16_t* scales[3];
    const uint16_t* biases[3];
    int32_t bits, group, inter, scale_dtype;
} q38_affine_shared;

/* q38_moe_layer_create for a layer whose shared expert is affine (desc->has_shared = 1):
 * weights->codes / scales hold the E routed experts only ([E, OUT, ...], no row for E), and
 * weights->shared_gate is the BF16 w_sg. The shared expert then runs as two kernels of its own
 * after the router; routing, the routed experts and the merge are those of q38_moe_layer_create
 * (SparseMoe ctor, include/qwen38/sparse_moe.hpp:48-55). */
int q38_moe_layer_create_affine_shared(q38_ctx* ctx, const q38_moe_desc* desc, const q38_moe_weights* weights,
                                       const q38_affine_shared* shared, q38_moe_layer** out);

/* Workspace bytes needed by q38_moe_forward / q38_verify_chain for up to max_rows rows
 * (1..2048). */
size_t q38_moe_workspace_size(const q38_moe_desc* desc, int32_t max_rows);

/* Router only (R1-R3): SparseMoe::route_decode_batch (src/sparse_moe.cpp:1032-1086) and
 * the gather-by-expert plan (src/sparse_moe.cpp:2260-2364), rows 1..2048. x: device
 * [rows, H] bf16. */
int q38_moe_route(q38_moe_layer* layer, const uint16_t* x, int32_t rows, const q38_route_out* routes,
                  void* workspace, size_t workspace_bytes, void* stream);

/* SparseMoe::forward_verify / forward_prefill (src/sparse_moe.cpp:1953-2171, 2199-2624):
 * y = routed + shared for rows 1..2048 of x. Rows 1..16 take the verify kernels; wider
 * calls (SparseMoe::forward_prefill, include/qwen38/sparse_moe.hpp:68, S <= 2048) take the
 * segmented-GEMM kernels, which need d8/14-bit projections with per-row scales and
 * rows * top_k <= 32768. x, y: device [rows, H] bf16 (may not alias). The expert kernels
 * take x as an fp16 MFMA operand: |x| must stay below 65504, and elements below 2^-14 lose
 * relative precision (an RMSNorm output, as in the verify chain, is bounded by sqrt(H) and
 * its small elements weigh nothing in the products). */
int q38_moe_forward(q38_moe_layer* layer, const uint16_t* x, int32_t rows, uint16_t* y,
                    const q38_route_out* routes, void* workspace, size_t workspace_bytes, void* stream);

/* q38_moe_forward for verify widths (rows 1..16) without a workspace argument and without
 * any allocation: no counterpart in the reference. It is for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Scratch is one fixed 8 MiB device array per GPU, held until the process ends; its address
 * is looked up by q38_ctx_create. Calls needing more (a layer's workspace for `rows`, see
 * q38_moe_workspace_size) return Q38_ESPACE. Every call on a GPU shares that GPU's array and
 * leaves its contents behind: calls that overlap on one GPU (two streams, two threads) race.
 * x, y: device [rows, H] bf16 (may not alias); routes optional as for q38_moe_forward. */
int q38_moe_forward_static(q38_moe_layer* layer, const uint16_t* x, int32_t rows, uint16_t* y,
                           const q38_route_out* routes, void* stream);

/* SparseMoe::forward_prefill_profiled (include/qwen38/sparse_moe.hpp:69-71) for rows
 * 17..2048: the same call as q38_moe_forward, synchronised, with the execution time of each
 * kernel in milliseconds: kernel_ms[7] = router logits, top-k, route plan, gate/up,
 * SwiGLU, down, combine. */
int q38_moe_forward_prefill_profiled(q38_moe_layer* layer, const uint16_t* x, int32_t rows, uint16_t* y,
                                     const q38_route_out* routes, void* workspace, size_t workspace_bytes,
                                     float* kernel_ms, void* stream);

/* Additive router-logit bias: logits[r, e] = T(x_r . Wr_e) + bias[e] (float), before the
 * softmax. bias: device [E] float kept by the layer (not copied), or null to clear. No
 * counterpart in the reference: it is the hook a prefill benchmark uses to skew expert
 * popularity (and a mask, with -inf entries). */
int q38_moe_layer_set_router_bias(q38_moe_layer* layer, const float* bias);

/* The verify pass through a stack of MoE layers (QwenModel::forward_verify_layer_major_
 * reference, src/model.cpp:386-441, with the HyperConnection/attention parts replaced by
 * a pre-norm residual): for each layer h <- h + MoE(RMSNorm(h)). h: device [rows, H]
 * bf16, updated in place. traces (optional): per-layer route outputs, array of n_layers.
 * At 1-4 rows on d8/14-bit H 2048 layers the experts and the combine run as one kernel whose
 * workgroups (one per CU) wait for each other: it expects the device's CUs to itself while
 * it runs. Otherwise bounded waits give up, the affected outputs are NaN, and the next
 * q38_ctx_synchronize returns Q38_EWAIT (q38_set_fused_layers(0) avoids the kernel). */
int q38_verify_chain(q38_moe_layer* const* layers, int32_t n_layers, uint16_t* h, int32_t rows,
                     float eps, const q38_route_out* traces, void* workspace, size_t workspace_bytes,
                     void* stream);

/* Phase timings of a profiled verify pass (MoeVerifyTimings, include/qwen38/sparse_moe.hpp:
 * 30-36), summed over layers, in milliseconds: the execution time of each phase's kernel,
 * from start/stop events the runtime records at the kernel's own begin and end (the
 * interval a kernel trace reports; launch gaps are not included). */
typedef struct q38_moe_timings {
    double routing_ms;   /* router logits kernel */
    double gate_up_ms;   /* gate/up projections (+ top-k + plan on the MFMA path); on layers
                            that run gate/up, down and combine in one kernel (d8/14-bit, H
                            2048, I 512, top-10, per-row scales, rows <= 4), that kernel */
    double down_ms;      /* down projection (+ SwiGLU on the narrow path); 0 on those layers */
    double merge_ms;     /* ordered route reduction + shared gate + residual; 0 on those layers */
    int32_t layers;
    int32_t reserved;
} q38_moe_timings;
int q38_verify_chain_profiled(q38_moe_layer* const* layers, int32_t n_layers, uint16_t* h, int32_t rows,
                              float eps, const q38_route_out* traces, void* workspace, size_t workspace_bytes,
                              q38_moe_timings* timings, void* stream);

/* RMSNorm with unit gamma, y = T(x / sqrt(mean(x^2) + eps)); device [rows, H] bf16. */
int q38_rmsnorm(const uint16_t* x, int32_t rows, int32_t hidden, float eps, uint16_t* y, void* stream);

/* Synthetic token embedding (stands in for QwenModel::embed, src/model.cpp:410-414):
 * row r = N(0,1) bf16 values keyed by (seed, token r). h: device [n, H]. */
int q38_embed_synthetic(uint64_t seed, const uint32_t* tokens_host, int32_t n, int32_t hidden, uint16_t* h,
                        void* stream);

/* The same embedding with the token ids in device memory (device u32 [n]), so a captured
 * graph can be replayed with new tokens. */
int q38_embed_synthetic_dev(uint64_t seed, const uint32_t* tokens, int32_t n, int32_t hidden, uint16_t* h,
                            void* stream);

/* ------------------------------------------------------------------ LM heads
 * Target head (src/model.cpp:466-492): symmetric int8 [V, H] + one FP16 scale per row.
 * Draft head (devtools/build_mtp_lm_head_q4.py:60-92): signed int4 (two per byte, low
 * nibble first) [V, H/2] + FP16 scales [V, H/64]. */
enum { Q38_HEAD_Q8 = 0, Q38_HEAD_Q4G64 = 1 };
int q38_head_create(q38_ctx* ctx, int kind, int64_t vocab, int32_t hidden, const void* weights,
                    const uint16_t* scales, q38_head** out);
int q38_head_create_synthetic(q38_ctx* ctx, int kind, int64_t vocab, int32_t hidden, uint64_t seed,
                              q38_head** out);
void q38_head_destroy(q38_head* head);
int q38_head_weights(const q38_head* head, const void** weights, const uint16_t** scales);
int64_t q38_head_bytes(const q38_head* head);
/* Device workspace bytes for q38_head_greedy / q38_head_logits with up to max_rows rows
 * (Q8: 1..16; Q4: 1..4); 0 for an invalid count. */
size_t q38_head_workspace_size(const q38_head* head, int32_t max_rows);

/* greedy_batch_from_logits (src/mtp_verifier.cpp:30-55): per row the argmax (lowest index
 * on ties) of the exact logit contract, and that logit. h: device [rows, H] bf16 (rows
 * 1..16, one pass over the weights for all rows); argmax, logit: device [rows]. Q8 heads
 * only. */
int q38_head_greedy(q38_head* head, const uint16_t* h, int32_t rows, uint32_t* argmax, float* logit,
                    void* workspace, size_t workspace_bytes, void* stream);
/* Logits of either head: device [rows, V] float. Q8: the fast pass (rows 1..16, needs the
 * workspace), the float rounding of scale * (w . h^) with h^ the int8-plane form of h (equal
 * to h for every element with |h| >= max|h| * 2^-12). Q4: rows 1..4, no workspace. */
int q38_head_logits(q38_head* head, const uint16_t* h, int32_t rows, float* logits, void* workspace,
                    size_t workspace_bytes, void* stream);

/* Softmax of the head's logits at temperature T > 0: the probabilities sampling reads
 * (logits.softmax_axis(-1), src/native_engine.cpp:116-118, at T = 1; the tempered target and
 * draft distributions of rejection sampling otherwise). Per row, stats [rows][2] = (max
 * logit, sum over the vocabulary of exp((l - max) / T)), summed in a fixed order; when probs
 * (device [rows, V] float) is given it receives exp((l - max) / T) / sum, and the logits are
 * computed into it first. Rows as for q38_head_logits (Q8: 1..16, Q4: 1..4); workspace:
 * q38_head_probs_workspace_size bytes. */
size_t q38_head_probs_workspace_size(const q38_head* head, int32_t max_rows);
int q38_head_probs(q38_head* head, const uint16_t* h, int32_t rows, float temperature, float* probs, float* stats,
                   void* workspace, size_t workspace_bytes, void* stream);

/* greedy_from_logits (src/mtp_verifier.cpp:20-55) on device logits [rows, vocab] float:
 * per row the argmax, lowest index on ties (src/mlx_backend.cpp:78-85), and its value.
 * argmax, value: device [rows] (value may be null); rows 1..64; workspace: device, at least
 * 8 * rows bytes. */
int q38_argmax_rows(const float* logits, int32_t rows, int64_t vocab, uint32_t* argmax, float* value,
                    void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------ MTP draft head
 * QwenMtpHead (include/qwen38/mtp_head.hpp:29-63) on the verify path's model: one draft step
 * (forward_decode, src/mtp_head.cpp:454-470) for rows independent requests maps the target's
 * pre-norm residual stream s (device [rows, H] bf16) and the next token t to
 *   e = embed(t)                          the target's embedding (seeded generator)
 *   x = T(T(W_e . rms(e)) + T(W_h . rms(s)))   combine_inputs (src/mtp_head.cpp:258-266):
 *                                         two H x H Q8 projections (q38_head_logits, Q8)
 *   s' = x + MoE(rms(x))                  the head's decoder block: one SparseMoe layer
 *                                         (block.mlp as layer 48, src/sparse_moe.cpp:376-381)
 *   logits = Q4 head(rms(s'))             the draft LM head (R14)
 * with rms the unit-gain RMSNorm (eps of the head). s' is the step's output stream
 * (pre_mixer_stream), the input of the next step of a draft chain. Rows 1..4 (the Q4 head's
 * row limit); hidden 2048. */
typedef struct q38_mtp_head q38_mtp_head;
typedef struct q38_hc q38_hc; /* the HyperConnection mixer (declared below) */
/* Borrowed components (kept alive by the caller): layer (hidden H), fc_embedding and
 * fc_hidden (Q8 heads, vocab = hidden = H), draft_head (Q4, hidden H). */
int q38_mtp_head_create(q38_ctx* ctx, q38_moe_layer* layer, q38_head* fc_embedding, q38_head* fc_hidden,
                        q38_head* draft_head, uint64_t embed_seed, float eps, q38_mtp_head** out);
/* Seeded random-init head: layer 48 of the seed's synthetic stack (desc), FC projections
 * from the Q8 generator with seeds seed ^ Q38_MTP_FC_EMBED_SALT / seed ^ Q38_MTP_FC_HIDDEN_SALT,
 * the Q4 draft head of the seed, the seed's embedding; eps 1e-6. */
#define Q38_MTP_FC_EMBED_SALT 0x46C0E3BEull
#define Q38_MTP_FC_HIDDEN_SALT 0x46C0411Dull
int q38_mtp_head_create_synthetic(q38_ctx* ctx, const q38_moe_desc* desc, int64_t vocab, uint64_t seed,
                                  q38_mtp_head** out);
void q38_mtp_head_destroy(q38_mtp_head* head);
/* The component handles (owned by the head when it was created synthetic). */
int q38_mtp_head_parts(const q38_mtp_head* head, q38_moe_layer** layer, q38_head** fc_embedding,
                       q38_head** fc_hidden, q38_head** draft_head);
/* HC streams (QwenMtpHead with hyper_connection_count streams, src/mtp_head.cpp:120-170,
 * 223-267, 454-470). After this call a step maps the target's pre-mixer streams s (device
 * [rows, HC * H] bf16) and the next token t to
 *   ne = T(T(rms(embed(t))) * (1 + w_e))        pre_fc_norm_embedding, over H
 *   nh = T(T(rms(s)) * (1 + w_h))               pre_fc_norm_hidden, over the row's HC * H
 *   x[s] = T(T(W_e . ne) + T(W_h . nh[s]))      the hidden projection per stream, the
 *                                               embedding projection added to every stream
 *   x' = block mixer write(x, MoE(read(x).mixed), read(x).injection)   the head's block
 *   logits = Q4 head(final mixer read(x').mixed)
 * and x' is the step's output stream [rows, HC * H]. The mixers (q38_hc_create) are borrowed:
 * the block mixer with injection weights, the final mixer without (the reference builds it
 * with with_injection false), both of the head's hidden size and one stream count. The norm
 * weights are the raw checkpoint tensors (bf16; null for zeros); 1 + w is formed once here.
 * The trace's combined rows are then [rows, HC * H] and final_mixed is the final mixer's
 * mixed row. Size workspaces after this call. A null streams argument returns to the
 * single-stream head. */
typedef struct q38_mtp_streams {
    q38_hc* block_mixer;            /* language_model.mtp.layers.0's MLP mixer          */
    q38_hc* final_mixer;            /* language_model.mtp.hyper_connection_mixer        */
    const uint16_t* embedding_norm; /* pre_fc_norm_embedding.weight [H]                 */
    const uint16_t* hidden_norm;    /* pre_fc_norm_hidden.weight [HC * H]               */
} q38_mtp_streams;
int q38_mtp_head_set_streams(q38_mtp_head* head, const q38_mtp_streams* streams);
/* The head's stream count (1 for the single-stream head). */
int q38_mtp_head_streams(const q38_mtp_head* head);
/* Device workspace bytes for up to max_rows rows (1..4); 0 for an invalid count. */
size_t q38_mtp_workspace_size(const q38_mtp_head* head, int32_t max_rows);
/* Optional intermediate rows of a step (MtpTrace, include/qwen38/mtp_head.hpp:24-28):
 * combined = x, final_mixed = rms(s'); device [rows, H] bf16 each, or null. */
typedef struct q38_mtp_trace {
    uint16_t* combined;
    uint16_t* final_mixed;
} q38_mtp_trace;
/* One draft step: tokens device u32 [rows]; logits device [rows, V] float (or null);
 * stream_out device [rows, H] bf16 (or null). */
int q38_mtp_forward_decode(q38_mtp_head* head, const uint16_t* stream_in, const uint32_t* tokens, int32_t rows,
                           float* logits, uint16_t* stream_out, const q38_mtp_trace* trace, void* workspace,
                           size_t workspace_bytes, void* stream);
/* Greedy draft chain (draft_lazy_chain, src/mtp_runner.cpp:152-211): depth steps, each
 * feeding its argmax token (q38_argmax_rows) and output stream into the next, all on the
 * device. drafts: device u32 [rows, depth]; depth 1..24; stream_out (optional) receives
 * the last step's output stream. No host synchronisation (graph-capturable). */
int q38_mtp_draft_greedy(q38_mtp_head* head, const uint16_t* stream_in, const uint32_t* tokens, int32_t rows,
                         int32_t depth, uint32_t* drafts, uint16_t* stream_out, void* workspace,
                         size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------ acceptance
 * decide_mtp_greedy (src/mtp_lifecycle.cpp:75-97), host. */
typedef struct q38_greedy_decision {
    int64_t accepted;
    int64_t correction_row;
    uint32_t next_token;
} q38_greedy_decision;
int q38_mtp_decide_greedy(const uint32_t* drafts, int64_t k, const uint32_t* target_rows, int64_t n_target,
                          const uint32_t* stop_tokens, int64_t n_stop, q38_greedy_decision* out);

/* plan_mtp_commit (src/mtp_lifecycle.cpp:57-73), host. out: {truncate_head_to,
 * target_rows_to_keep, stash_rows, committed_boundary}. */
int q38_plan_mtp_commit(uint64_t round_offset, uint64_t drafted, uint64_t accepted, uint64_t* out);

/* Rejection-sampling acceptance on the device (no counterpart in the reference, which
 * bypasses MTP when sampling: src/native_engine.cpp:943-945). target_logits [k+1, V],
 * draft_logits [k, V] (device float), drafts (device u32 [k]); uniforms from
 * Philox4x32-10 keyed by (seed; position, round, slot). out: device int64 [2] =
 * {accepted, next_token}. Four launches spread over the chip, no host synchronisation;
 * workspace: device, q38_mtp_accept_workspace_size(k, vocab) bytes. */
int q38_mtp_accept_sampled(const float* target_logits, const float* draft_logits, const uint32_t* drafts,
                           int32_t k, int64_t vocab, float temperature, uint64_t seed, uint64_t slot,
                           uint64_t round, int64_t* out, void* workspace, size_t workspace_bytes, void* stream);
/* Device workspace bytes of q38_mtp_accept_sampled (k 1..24); 0 for invalid sizes. */
size_t q38_mtp_accept_workspace_size(int32_t k, int64_t vocab);
/* Philox4x32-10 (host), for checking the device stream. */
void q38_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);

/* ------------------------------------------------------------------ per-slot state
 * The slot keeps the committed length and the committed hidden row of a request;
 * verification rows are its speculative checkpoints (MtpTargetVerification,
 * include/qwen38/mtp_verifier.hpp:15-25). */
int q38_slot_create(q38_ctx* ctx, int32_t hidden, int32_t max_rows, uint64_t token_count, q38_slot** out);
void q38_slot_destroy(q38_slot* slot);
/* Record a verification of draft_count drafts: rows = draft_count + 1 checkpoints whose
 * hidden rows are h (device [rows, H] bf16, copied on stream). draft_count 0 stages a
 * serial decode step (one row, committed with accepted = 0). */
int q38_slot_stage(q38_slot* slot, int32_t draft_count, const uint16_t* h, void* stream);
/* commit_mtp_target_verification (src/mtp_verifier.cpp:129-145): keep checkpoint
 * `accepted`; token_count becomes origin + accepted + 1; all staged rows are released.
 * Invalid counts return Q38_ESTATE and leave the slot untouched. The slot double-buffers
 * its checkpoints, so a commit moves no data (the reference moves state_after, :139). */
int q38_slot_commit(q38_slot* slot, int64_t accepted, void* stream);
/* Drop the staged rows, keeping the committed state. */
int q38_slot_rollback(q38_slot* slot);
int q38_slot_info(const q38_slot* slot, uint64_t* token_count, int32_t* staged_rows, int32_t* draft_count);
/* Committed hidden row (device [H] bf16), valid after the first commit. */
const uint16_t* q38_slot_hidden(const q38_slot* slot);
/* Generation of the staged verification: a number that every q38_slot_stage call makes
 * new (1, 2, ...), or 0 when nothing is staged. A caller that holds a verification keeps
 * the generation of its stage and commits only while the slot still reports it (the
 * reference consumes the verification's own rows, src/mtp_verifier.cpp:129-145). */
uint64_t q38_slot_generation(const q38_slot* slot);

/* ---- GatedDeltaNet verify step (the linear-attention half of a decoder layer):
 * GatedDeltaNet::forward_verify (src/gated_delta_net.cpp:657-834) for S rows
 * (1..64) from an origin state, with the state after every row as that row's checkpoint; the
 * caller commits a round by taking the checkpoint of its last accepted row as the next
 * origin (q38_gdn_commit). Weights are the reference checkpoint's tensors as stored
 * (src/gated_delta_net.cpp:138-178): in_proj_qkv [C, H], in_proj_z [HV DV, H], in_proj_b
 * [HV, H], in_proj_a [HV, H] and out_proj [H, HV DV] MLX affine-quantized (packed u32 weight,
 * scales and biases [out][in / group] bf16 or fp16), conv1d.weight [C, 4] bf16 (MLX
 * [C, 4, 1]), A_log [HV] fp32, dt_bias [HV] bf16, norm.weight [DV] bf16; C = 2 HK DK + HV DV.
 * A state (q38_gdn_state_bytes) is the convolution rows [3][C] bf16 followed by the
 * recurrent state [HV][DV][DK] bf16 (GatedDeltaNetState's convolution and recurrent arrays,
 * include/qwen38/gated_delta_net.hpp:28-37). */
typedef struct q38_gdn q38_gdn;
typedef struct q38_gdn_desc {
    int32_t hidden;        /* H: a multiple of the group and of 32                          */
    int32_t key_heads;     /* HK (linear_num_key_heads)                                     */
    int32_t value_heads;   /* HV, a multiple of HK (value head h reads key head h / (HV/HK)) */
    int32_t key_dim;       /* DK = DV: 64, 128 or 256                                       */
    int32_t value_dim;     /* DV                                                            */
    int32_t conv_kernel;   /* 4 (linear_conv_kernel_dim)                                    */
    int32_t bits;          /* 2, 4 or 8                                                     */
    int32_t group;         /* 32, 64 or 128                                                 */
    int32_t scale_dtype;   /* 0 bf16, 1 fp16 scales and biases                              */
    int32_t gate_silu;     /* output_gate_type: 0 "sigmoid", 1 "silu"                       */
    float eps;             /* rms_norm_eps of the output norm                               */
} q38_gdn_desc;
typedef struct q38_gdn_weights {
    const uint32_t* weight[5];  /* qkv, z, b, a, out                                         */
    const uint16_t* scales[5];
    const uint16_t* biases[5];
    const uint16_t* conv;       /* [C][4] bf16                                               */
    const float* a_log;         /* [HV]                                                      */
    const uint16_t* dt_bias;    /* [HV] bf16                                                 */
    const uint16_t* norm;       /* [DV] bf16                                                 */
} q38_gdn_weights;
/* GatedDeltaNet::GatedDeltaNet (src/gated_delta_net.cpp:138-178): adopts the device weight
 * pointers (they must stay alive). */
int q38_gdn_create(q38_ctx* ctx, const q38_gdn_desc* desc, const q38_gdn_weights* weights, q38_gdn** out);
void q38_gdn_destroy(q38_gdn* gdn);
/* Bytes of one state (the origin and each checkpoint). */
size_t q38_gdn_state_bytes(const q38_gdn* gdn);
size_t q38_gdn_workspace_size(const q38_gdn* gdn, int32_t max_rows);
/* GatedDeltaNet::forward_verify: x [rows, H] bf16 -> out [rows, H] bf16; origin: a state, or
 * null for the zero state of an uninitialised one; checkpoints: rows states, the state after
 * each row (may be null when not needed). */
int q38_gdn_verify(q38_gdn* gdn, const uint16_t* x, int32_t rows, const void* origin, void* checkpoints,
                   uint16_t* out, void* workspace, size_t workspace_bytes, void* stream);
/* The commit of a verify round for this layer's state (the checkpoint of the last accepted
 * row becomes the state, src/gated_delta_net.cpp:825-831 with the verifier's commit,
 * src/mtp_verifier.cpp:129-145): copies checkpoints[row] to state on the stream. */
int q38_gdn_commit(const q38_gdn* gdn, const void* checkpoints, int32_t row, void* state, void* stream);

/* ------------------------------------------------------------------ full attention (verify)
 * SelfAttention::forward_verify (src/self_attention.cpp:1450-1720) on its dense path: the
 * attention half of a full-attention decoder layer for S verify rows of one slot over the
 * slot's KV cache. The call appends the rows' keys and values to the cache at tokens
 * cache_tokens .. cache_tokens + S - 1, and row r attends tokens 0 .. cache_tokens + r. Row
 * r's checkpoint (SelfAttentionState after the row, :1595-1610) is the cache prefix of
 * cache_tokens + r + 1 tokens, so commit and rollback are the caller's token count: no
 * device work, and a rejected suffix is overwritten by the next call. The arithmetic is the
 * reference's explicit decode path (:1240-1305) with its bf16 rounding points: q_proj rows
 * per head (D query values, then D gate values), k_proj, v_proj; RMS norms of q and k per head
 * with the q_norm / k_norm weights (1 + w when norm_offset); RoPE on the first rotary_dim
 * dims (the split-half rotation, cos / sin of position * theta^(-2i / R) rounded to bf16,
 * :641-679); scores T(T(q . k) * T(1/sqrt D)); the softmax of the float32 scores rounded to
 * bf16; T(P . V); the gate T(sigmoid); the output projection. Not part of this path: the QSA
 * block selection (the reference builds its mask only once a context exceeds the indexer
 * budget, :764-766; within the budget the results agree) and the Q8 KV cache. */
typedef struct q38_attn q38_attn;
typedef struct q38_attn_desc {
    int32_t hidden;       /* H: a multiple of the group and of 32, at most 8192                */
    int32_t q_heads;      /* HQ (num_attention_heads)                                         */
    int32_t kv_heads;     /* HKV (num_key_value_heads); HQ a multiple of it                   */
    int32_t head_dim;     /* D: 64, 128 or 256                                                */
    int32_t rotary_dim;   /* R: even, 0 < R <= D (head_dim * partial_rotary_factor)            */
    int32_t bits;         /* 2, 4 or 8                                                        */
    int32_t group;        /* 32, 64 or 128                                                    */
    int32_t scale_dtype;  /* 0 bf16, 1 fp16 scales and biases                                 */
    int32_t norm_offset;  /* 1: the norms apply 1 + weight (attention_norm_has_offset)         */
    float eps;            /* rms_norm_eps                                                     */
    double rope_theta;
} q38_attn_desc;
typedef struct q38_attn_weights {
    const uint32_t* weight[4];  /* q_proj [2 HQ D][H], k_proj [HKV D][H], v_proj, o_proj [H][HQ D] */
    const uint16_t* scales[4];
    const uint16_t* biases[4];
    const uint16_t* q_norm;     /* [D] bf16                                                   */
    const uint16_t* k_norm;     /* [D] bf16                                                   */
} q38_attn_weights;
/* SelfAttention::SelfAttention (src/self_attention.cpp:460-521): adopts the device weight
 * pointers (they must stay alive); the norm weights are copied (1 + w formed when
 * norm_offset). */
int q38_attn_create(q38_ctx* ctx, const q38_attn_desc* desc, const q38_attn_weights* weights, q38_attn** out);
void q38_attn_destroy(q38_attn* attn);
/* Bytes of a KV cache of `capacity` tokens: keys [HKV][capacity][D] bf16, then values. */
size_t q38_attn_cache_bytes(const q38_attn* attn, int64_t capacity);
/* Workspace for calls of up to max_rows rows (1..64) with up to max_tokens tokens after the
 * call (cache_tokens + rows). */
size_t q38_attn_workspace_size(const q38_attn* attn, int32_t max_rows, int64_t max_tokens);
/* x [rows, H] bf16 -> out [rows, H] bf16; cache: 16-byte aligned, q38_attn_cache_bytes(capacity)
 * bytes, cache_tokens valid tokens; position: the position of row 0 (the state's position_base
 * + token_count). Q38_ERANGE when cache_tokens + rows exceeds capacity. */
int q38_attn_verify(q38_attn* attn, const uint16_t* x, int32_t rows, void* cache, int64_t capacity,
                    int64_t cache_tokens, int64_t position, uint16_t* out, void* workspace, size_t workspace_bytes,
                    void* stream);

/* ------------------------------------------------------------------ HyperConnection mixer
 * The stream mixer around a decoder block (HyperConnection, include/qwen38/hyper_connection.hpp:18-40,
 * src/hyper_connection.cpp:150-211 for the weights, :309-493 read, :692-709 write). A row's state
 * is HC residual streams of H values ([rows, HC * H] bf16, stream s at columns s H ..). read()
 * normalises each stream (RMSNorm, then the learned weight 1 + hc_norm.weight), projects the
 * flat normalised row to the rank R (input_mix_weight_down) and back to HC x H
 * (input_mix_weight_up) through x / HC, SiLU and sigmoid, and returns the block input
 * mixed = mean over streams of sigmoid(up) * normalised stream, plus per-stream injection
 * gates 2 sigmoid(block_inject_weight . normalised / HC) when the mixer has them. write() adds
 * block_output * injection[s] to every stream s. Values are rounded to bf16 at the points of
 * the reference's fused read kernels (src/hc_metal_kernels.hpp:10-36, 85-128, 270-308); the
 * dot products accumulate in float. Projections are MLX affine-quantised: weight
 * [out][in / (32 / bits)] uint32 (value j of a word at bits j*bits.., LSB first), scales and
 * biases [out][in / group] bf16, value = q * scale + bias. */
typedef struct q38_hc_desc {
    int32_t hidden;          /* H: a multiple of 256, at most 4096                       */
    int32_t streams;         /* HC: 1..16                                                 */
    int32_t rank;            /* R: rows of input_mix_weight_down, a multiple of the group
                                and of 128 / bits, at most 512                            */
    int32_t bits;            /* 4 or 8                                                    */
    int32_t group;           /* 32, 64 or 128                                             */
    int32_t with_injection;  /* 1: block_inject_weight present (the decoder mixers)       */
    float eps;               /* RMSNorm epsilon, > 0                                      */
} q38_hc_desc;
typedef struct q38_hc_weights {
    const uint16_t* norm;                                  /* hc_norm.weight [HC * H]     */
    const uint32_t* down_w; const uint16_t* down_s; const uint16_t* down_b;  /* [R][HC H] */
    const uint32_t* up_w; const uint16_t* up_s; const uint16_t* up_b;        /* [HC H][R] */
    const uint32_t* inj_w; const uint16_t* inj_s; const uint16_t* inj_b;     /* [HC][HC H] */
} q38_hc_weights;
/* HyperConnection::HyperConnection (src/hyper_connection.cpp:150-211): adopts the device
 * weight pointers (they must stay alive) and forms 1 + hc_norm.weight once (bf16). */
int q38_hc_create(q38_ctx* ctx, const q38_hc_desc* desc, const q38_hc_weights* weights, q38_hc** out);
void q38_hc_destroy(q38_hc* hc);
size_t q38_hc_workspace_size(const q38_hc_desc* desc, int32_t max_rows);
/* HyperConnection::read (src/hyper_connection.cpp:309-493; the MLX graph at :461-493): stream [rows, HC H] bf16 ->
 * mixed [rows, H] bf16 and, with injection, injection [rows, HC] bf16 (may be null
 * otherwise). rows 1..16. */
int q38_hc_read(q38_hc* hc, const uint16_t* stream, int32_t rows, uint16_t* mixed, uint16_t* injection, void* workspace,
                size_t workspace_bytes, void* hip_stream);
/* HyperConnection::write (src/hyper_connection.cpp:692-709): out = stream + block_output *
 * injection per stream, rounded to bf16 at the product and the sum; out may be stream. */
int q38_hc_write(const q38_hc* hc, const uint16_t* stream, const uint16_t* block_output, const uint16_t* injection,
                 int32_t rows, uint16_t* out, void* hip_stream);
/* The MLP half of DecoderLayer::forward_verify_dense_batched (src/decoder_layer.cpp:494-497)
 * over n_layers layers: per layer l, read = mixers[l].read(stream), y = MoE_l(read.mixed)
 * (q38_moe_forward), stream = mixers[l].write(stream, y, read.injection). stream: device
 * [rows, HC * H] bf16, updated in place; rows 1..16. Layers and mixers share H; every
 * mixer has injection weights, the same streams and rank. The decoder's optional MLP output
 * map (src/decoder_layer.cpp:198-210) is applied by q38_verify_chain_hc_mapped. Workspace:
 * q38_verify_chain_hc_workspace_size bytes for the largest layer description. */
size_t q38_verify_chain_hc_workspace_size(const q38_moe_desc* desc, const q38_hc_desc* mixer, int32_t max_rows);
int q38_verify_chain_hc(q38_moe_layer* const* layers, q38_hc* const* mixers, int32_t n_layers, uint16_t* stream,
                        int32_t rows, void* workspace, size_t workspace_bytes, void* hip_stream);
/* The decoder's optional MLP output map (DecoderLayer::apply_mlp_output_map,
 * src/decoder_layer.cpp:198-210, tensors loaded at :158-182): rank 0 takes the full map mlp.T
 * [H][H] bf16 (out = T(y . T)); rank R > 0 the low-rank pair mlp.T_delta_left [H][R] and
 * mlp.T_delta_right [R][H] bf16 (out = T(y + T(T(y . left) . right))). Each product sums in
 * float over 128-input slices in ascending order, the slices added in order. */
typedef struct q38_mlp_map {
    int32_t hidden;
    int32_t rank;          /* 0: full map                                                    */
    const uint16_t* full;  /* [H][H] bf16 (rank 0)                                           */
    const uint16_t* left;  /* [H][rank] bf16                                                 */
    const uint16_t* right; /* [rank][H] bf16                                                 */
} q38_mlp_map;
size_t q38_mlp_map_workspace_size(const q38_mlp_map* map, int32_t max_rows);
/* y [rows, H] bf16 -> out [rows, H] bf16 (out must not alias y); rows 1..16. */
int q38_mlp_output_map(const q38_mlp_map* map, const uint16_t* y, int32_t rows, uint16_t* out, void* workspace,
                       size_t workspace_bytes, void* stream);
/* q38_verify_chain_hc with the MLP output map of each layer (maps[l], or null for a layer
 * without one; maps itself may be null): per layer read, MoE, map, write
 * (src/decoder_layer.cpp:494-497). Workspace: q38_verify_chain_hc_mapped_workspace_size for
 * the largest layer description. */
size_t q38_verify_chain_hc_mapped_workspace_size(const q38_moe_desc* desc, const q38_hc_desc* mixer, int32_t max_rows);
int q38_verify_chain_hc_mapped(q38_moe_layer* const* layers, q38_hc* const* mixers, const q38_mlp_map* const* maps,
                               int32_t n_layers, uint16_t* stream, int32_t rows, void* workspace,
                               size_t workspace_bytes, void* hip_stream);
/* HyperConnection::initialize_stream (src/hyper_connection.cpp:298-307): the embedding rows
 * [rows, H] tiled to [rows, streams * H]. H a multiple of 8. */
int q38_hc_initialize_stream(const uint16_t* embedding, int32_t rows, int32_t hidden, int32_t streams, uint16_t* out,
                             void* hip_stream);

#ifdef __cplusplus
}
#endif
#endif /* Q38_H */
