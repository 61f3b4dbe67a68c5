// qwen38_verify.hpp — C++20 host interface of the MI355X MTP verification round.
//
// It mirrors the reference's interfaces for this path (same names, argument meaning and
// error behaviour) on top of the C ABI in include/q38.h:
//   SparseMoe, RouterSelection, MoeVerifyTimings   include/qwen38/sparse_moe.hpp:12-36, 46-214
//   GreedyStep                                     include/qwen38/model.hpp:24-27
//   MtpTargetVerifyRow / MtpTargetVerification      include/qwen38/mtp_verifier.hpp:15-25
//   verify_mtp_target_layer_major_reference,
//   commit_mtp_target_verification                  include/qwen38/mtp_verifier.hpp:33-47
//   MtpCommitPlan / plan_mtp_commit, MtpGreedyDecision / decide_mtp_greedy
//                                                   include/qwen38/mtp_lifecycle.hpp:38-59
//   MtpRoundStep / run_greedy_external_draft_round_reference
//                                                   include/qwen38/mtp_runner.hpp:19-60
// DeviceTensor (an owning HBM buffer with shape, dtype and stream) takes the place of
// MlxArray. Errors are thrown as std::runtime_error (std::out_of_range for packed-code
// lookups past the buffer); a failed validation leaves its arguments untouched.
#pragma once

#include "q38.h"
#include "qwen38_engine.hpp"

#include <cstddef>
#include <cstdint>
#include <memory>
#include <optional>
#include <span>
#include <string>
#include <vector>

namespace qwen38 {

// ------------------------------------------------------------------ device plumbing
class Context {
public:
    explicit Context(int hip_device = 0);
    ~Context();
    Context(const Context&) = delete;
    Context& operator=(const Context&) = delete;
    [[nodiscard]] q38_ctx* handle() const noexcept { return ctx_; }
    [[nodiscard]] void* stream() const noexcept { return stream_; }  // hipStream_t
    void synchronize() const;

private:
    q38_ctx* ctx_ = nullptr;
    void* stream_ = nullptr;
};

enum class DType { bf16, f16, f32, i32, u32 };
[[nodiscard]] std::size_t dtype_size(DType t) noexcept;

// Owning device tensor. Move-only; share() hands out another owner of the same buffer
// (as MlxArray::share does).
class DeviceTensor {
public:
    DeviceTensor() = default;
    DeviceTensor(std::vector<std::size_t> shape, DType dtype);
    DeviceTensor(DeviceTensor&&) noexcept = default;
    DeviceTensor& operator=(DeviceTensor&&) noexcept = default;
    DeviceTensor(const DeviceTensor&) = delete;
    DeviceTensor& operator=(const DeviceTensor&) = delete;

    [[nodiscard]] DeviceTensor share() const;
    [[nodiscard]] const std::vector<std::size_t>& shape() const noexcept { return shape_; }
    [[nodiscard]] DType dtype() const noexcept { return dtype_; }
    [[nodiscard]] std::size_t numel() const noexcept;
    [[nodiscard]] std::size_t nbytes() const noexcept { return numel() * dtype_size(dtype_); }
    [[nodiscard]] void* data() const noexcept { return buf_.get(); }
    [[nodiscard]] bool empty() const noexcept { return !buf_; }

    // Synchronous host transfers (the reference's readback points).
    void upload(const void* host, std::size_t bytes);
    void download(void* host, std::size_t bytes) const;
    template <typename T>
    [[nodiscard]] std::vector<T> to_host() const {
        std::vector<T> out(nbytes() / sizeof(T));
        download(out.data(), out.size() * sizeof(T));
        return out;
    }

private:
    std::shared_ptr<void> buf_;
    std::vector<std::size_t> shape_;
    DType dtype_ = DType::bf16;
};

// ------------------------------------------------------------------ sparse MoE
struct RouterSelection {
    std::vector<std::size_t> experts;
    std::vector<float> weights;
};

struct MoeVerifyTimings {
    double routing_ms{0.0};
    double gate_up_ms{0.0};
    double down_ms{0.0};
    double shared_expert_ms{0.0};  // the shared expert runs inside the projection kernels
    double merge_ms{0.0};
};

// MoePrefillTimings (include/qwen38/sparse_moe.hpp:17-28): kernel execution times of one
// prefill call in milliseconds. Gate and up run in one kernel (gate_up_ms; gate_qmm_ms and
// up_qmm_ms stay 0), the down kernel reduces nothing (down_qmm_ms; down_reduce_ms 0), and
// the route reduction, shared-expert gate and output form one kernel (merge_ms).
struct MoePrefillTimings {
    double routing_ms{0.0};
    double gate_up_ms{0.0};
    double gate_qmm_ms{0.0};
    double up_qmm_ms{0.0};
    double swiglu_ms{0.0};
    double down_reduce_ms{0.0};
    double down_qmm_ms{0.0};
    double route_reduce_ms{0.0};
    double shared_expert_ms{0.0};
    double merge_ms{0.0};
};

// VQ geometry of the projection tensors (the reference reads it from the checkpoint's
// tensor shapes, src/sparse_moe.cpp:618-661).
struct MoeGeometry {
    std::size_t hidden{2048};
    std::size_t intermediate{512};
    std::size_t gate_up_dimension{8}, gate_up_bits{14};
    std::size_t down_dimension{8}, down_bits{14};
    bool shared_expert{true};
};

class SparseMoe final {
public:
    // Adopts device tensors in the reference layout. Arguments as SparseMoe's constructor
    // (include/qwen38/sparse_moe.hpp:48-55): quantization_bits / quantization_group_size
    // describe the scale groups along the input (group size == input: one scale per row).
    SparseMoe(const Context& ctx, const q38_moe_weights& tensors, std::size_t expert_count,
              std::size_t experts_per_token, std::size_t quantization_bits, std::size_t quantization_group_size,
              bool normalize_topk_probability, const MoeGeometry& geometry = {});
    // Seeded random-init layer generated on the device.
    SparseMoe(const Context& ctx, std::uint64_t seed, int layer_index, std::size_t expert_count,
              std::size_t experts_per_token, bool normalize_topk_probability, const MoeGeometry& geometry = {});
    ~SparseMoe();
    SparseMoe(SparseMoe&&) noexcept;
    SparseMoe& operator=(SparseMoe&&) noexcept;
    SparseMoe(const SparseMoe&) = delete;
    SparseMoe& operator=(const SparseMoe&) = delete;

    // input [1, S, H] bf16 (normalised), S in 1..2048. Selections per row, read back to the
    // host.
    [[nodiscard]] RouterSelection route_decode(const DeviceTensor& input) const;
    [[nodiscard]] std::vector<RouterSelection> route_decode_batch(const DeviceTensor& input) const;
    // forward_decode (src/sparse_moe.cpp:1629-1642): one row, input [1, 1, H] bf16.
    [[nodiscard]] DeviceTensor forward_decode(const DeviceTensor& input) const;
    // forward_decode_multi (src/sparse_moe.cpp:1775-1950): one [1, 1, H] row per request,
    // routed and computed as one batch (rows 1..2048); one output per request.
    [[nodiscard]] std::vector<DeviceTensor> forward_decode_multi(const std::vector<DeviceTensor>& inputs) const;
    // forward_verify (src/sparse_moe.cpp:1953-2171): input [1, S, H] bf16, S in 1..1024
    // (src/sparse_moe.cpp:1974-1976); output the same shape and dtype. S <= 16 takes the
    // verify-width kernels, wider calls the segmented-GEMM kernels.
    [[nodiscard]] DeviceTensor forward_verify(const DeviceTensor& input) const;
    // forward_prefill (src/sparse_moe.cpp:2199-2624): input [1, S, H] bf16, S in 1..2048;
    // S > 16 takes the segmented-GEMM kernels.
    [[nodiscard]] DeviceTensor forward_prefill(const DeviceTensor& input) const;
    // forward_prefill_profiled: the same for S in 17..2048, synchronised, with kernel times.
    [[nodiscard]] DeviceTensor forward_prefill_profiled(const DeviceTensor& input, MoePrefillTimings& timings) const;
    // Additive router-logit bias (device [E] float, kept by reference, or an empty tensor to
    // clear): a benchmark hook with no counterpart in the reference.
    void set_router_bias(const DeviceTensor& bias);

    [[nodiscard]] q38_moe_layer* handle() const noexcept { return layer_; }
    [[nodiscard]] const q38_moe_desc& desc() const noexcept { return desc_; }
    [[nodiscard]] std::size_t experts_per_token() const noexcept { return static_cast<std::size_t>(desc_.top_k); }

private:
    DeviceTensor forward_rows(const DeviceTensor& input, std::size_t rows, const char* what) const;
    void reserve_workspace(std::size_t rows) const;

    const Context* ctx_ = nullptr;
    q38_moe_layer* layer_ = nullptr;
    q38_moe_desc desc_{};
    mutable DeviceTensor workspace_;
};

// ------------------------------------------------------------------ HyperConnection mixer
// HyperConnectionRead (include/qwen38/hyper_connection.hpp:12-16).
struct HyperConnectionRead {
    DeviceTensor mixed;      // [B, S, H] bf16: the block input
    DeviceTensor injection;  // [B, S, HC, 1] bf16 stream gates (empty without injection)
    bool has_injection{false};
};

// HyperConnection (include/qwen38/hyper_connection.hpp:18-71) over device tensors in the
// reference layout: hc_norm.weight [HC * H], input_mix_weight_down [R][HC * H] and
// input_mix_weight_up [HC * H][R] (and block_inject_weight [HC][HC * H] when with_injection),
// MLX affine-quantised (packed uint32 words, bf16 scales and biases per group). The reference
// reads bits and group size from the manifest; here they are arguments.
class HyperConnection final {
public:
    HyperConnection(const Context& ctx, const q38_hc_weights& tensors, std::size_t hidden_size,
                    std::size_t stream_count, std::size_t rank, std::size_t quantization_bits,
                    std::size_t quantization_group_size, float rms_norm_epsilon, bool with_injection);
    ~HyperConnection();
    HyperConnection(HyperConnection&&) noexcept;
    HyperConnection& operator=(HyperConnection&&) noexcept;
    HyperConnection(const HyperConnection&) = delete;
    HyperConnection& operator=(const HyperConnection&) = delete;

    // initialize_stream (src/hyper_connection.cpp:298-307): [B, S, H] -> [B, S, HC * H].
    [[nodiscard]] static DeviceTensor initialize_stream(const Context& ctx, const DeviceTensor& embedding,
                                                        std::size_t stream_count);
    // read (src/hyper_connection.cpp:309-493): stream [B, S, HC * H] bf16, B * S in 1..16.
    [[nodiscard]] HyperConnectionRead read(const DeviceTensor& stream) const;
    // write (src/hyper_connection.cpp:692-709): stream + block_output * injection per stream.
    [[nodiscard]] DeviceTensor write(const DeviceTensor& stream, const DeviceTensor& block_output,
                                     const DeviceTensor& injection) const;

    [[nodiscard]] q38_hc* handle() const noexcept { return hc_; }
    [[nodiscard]] const q38_hc_desc& desc() const noexcept { return desc_; }
    [[nodiscard]] const Context& context() const noexcept { return *ctx_; }

private:
    const Context* ctx_ = nullptr;
    q38_hc* hc_ = nullptr;
    q38_hc_desc desc_{};
    mutable DeviceTensor workspace_;
};

// ------------------------------------------------------------------ GatedDeltaNet (verify)
// GatedDeltaNetState (include/qwen38/gated_delta_net.hpp:28-37): the convolution rows and the
// recurrent state of one layer and slot, one device block of GatedDeltaNet::state_bytes()
// (conv [3][C] bf16, then recurrent [HV][DV][DK] bf16) at `offset` bytes into `block`; the
// checkpoints of one verify call share one block, as the reference's slices share theirs.
struct GatedDeltaNetState {
    DeviceTensor block;
    std::size_t offset{0};
    bool initialized{false};
    [[nodiscard]] void* data() const noexcept { return static_cast<char*>(block.data()) + offset; }
};

// GatedDeltaNet (include/qwen38/gated_delta_net.hpp:40-106) on the verify path: the
// reference checkpoint's tensors (q38_gdn_weights) with the manifest's geometry.
class GatedDeltaNet final {
public:
    GatedDeltaNet(const Context& ctx, const q38_gdn_weights& tensors, std::size_t hidden_size,
                  std::size_t key_head_count, std::size_t value_head_count, std::size_t key_head_dimension,
                  std::size_t value_head_dimension, std::size_t convolution_kernel_size, int quantization_bits,
                  int quantization_group_size, bool fp16_scales, const std::string& output_gate_type,
                  float rms_norm_epsilon);
    ~GatedDeltaNet();
    GatedDeltaNet(GatedDeltaNet&&) noexcept;
    GatedDeltaNet& operator=(GatedDeltaNet&&) noexcept;
    GatedDeltaNet(const GatedDeltaNet&) = delete;
    GatedDeltaNet& operator=(const GatedDeltaNet&) = delete;

    // forward_verify (src/gated_delta_net.cpp:657-834): input [1, S, hidden] bf16, S = 1..64,
    // from origin (an uninitialised origin is the zero state); checkpoints receives the S
    // states after each row. Throws on a deferred-rollback origin as the reference does (this
    // build's states never defer).
    [[nodiscard]] DeviceTensor forward_verify(const DeviceTensor& input, const GatedDeltaNetState& origin,
                                              std::vector<GatedDeltaNetState>& checkpoints) const;
    [[nodiscard]] std::size_t state_bytes() const noexcept;
    [[nodiscard]] q38_gdn* handle() const noexcept { return gdn_; }

private:
    const Context* ctx_ = nullptr;
    q38_gdn* gdn_ = nullptr;
    std::size_t hidden_ = 0;
    mutable DeviceTensor workspace_;
};

// ------------------------------------------------------------------ SelfAttention (verify)
// SelfAttentionState (include/qwen38/self_attention.hpp:12-30) on the dense path: a KV cache of
// `capacity` tokens (keys [HKV][capacity][D] bf16, then values) holding token_count tokens,
// the first at position_base. The checkpoints of a verify call share the cache and differ in
// token_count, so committing a row is adopting its checkpoint and rolling back is keeping the
// origin.
struct SelfAttentionState {
    DeviceTensor cache;
    std::size_t capacity{0};
    std::size_t token_count{0};
    std::size_t position_base{0};
};

// SelfAttention (include/qwen38/self_attention.hpp:32-128) on the verify path: the reference
// checkpoint's tensors (q38_attn_weights) with the manifest's geometry.
class SelfAttention final {
public:
    SelfAttention(const Context& ctx, const q38_attn_weights& tensors, std::size_t hidden_size,
                  std::size_t attention_heads, std::size_t key_value_heads, std::size_t head_dimension,
                  std::size_t rotary_dimension, int quantization_bits, int quantization_group_size, bool fp16_scales,
                  bool norm_has_offset, float rms_norm_epsilon, double rope_theta);
    ~SelfAttention();
    SelfAttention(SelfAttention&&) noexcept;
    SelfAttention& operator=(SelfAttention&&) noexcept;
    SelfAttention(const SelfAttention&) = delete;
    SelfAttention& operator=(const SelfAttention&) = delete;

    // An empty state with a cache of `capacity` tokens.
    [[nodiscard]] SelfAttentionState make_state(std::size_t capacity, std::size_t position_base = 0) const;
    // forward_verify (src/self_attention.cpp:1450-1720): input [1, S, hidden] bf16, S = 1..64;
    // appends the rows to origin's cache (shared with the returned checkpoints).
    [[nodiscard]] DeviceTensor forward_verify(const DeviceTensor& input, const SelfAttentionState& origin,
                                              std::vector<SelfAttentionState>& checkpoints) const;
    [[nodiscard]] q38_attn* handle() const noexcept { return attn_; }

private:
    const Context* ctx_ = nullptr;
    q38_attn* attn_ = nullptr;
    std::size_t hidden_ = 0;
    mutable DeviceTensor workspace_;
};

// ------------------------------------------------------------------ DecoderLayer (verify)
// DecoderLayerState (include/qwen38/decoder_layer.hpp): the attention half's state of one
// layer and slot, the linear-attention state or the full-attention KV cache (by layer kind).
struct DecoderLayerState {
    GatedDeltaNetState linear_attention;
    SelfAttentionState full_attention;
};

// DecoderLayer::forward_verify_dense_batched (src/decoder_layer.cpp:447-504) over one layer's
// components, referenced (the caller keeps them alive): the attention mixer, a GatedDeltaNet
// or a SelfAttention, the MLP mixer, the SparseMoe and the optional MLP output map. The
// per-layer embeddings (PLE, :457-467) are not part of this build.
class DecoderLayer final {
public:
    DecoderLayer(const HyperConnection& attention_mixer, const GatedDeltaNet& linear_attention,
                 const HyperConnection& mlp_mixer, const SparseMoe& mlp, const q38_mlp_map* output_map = nullptr);
    DecoderLayer(const HyperConnection& attention_mixer, const SelfAttention& full_attention,
                 const HyperConnection& mlp_mixer, const SparseMoe& mlp, const q38_mlp_map* output_map = nullptr);

    // streams [1, S, HC * H] bf16, S = 1..16 (the mixers' row limit): attention mixer read,
    // the attention step from origin (checkpoints receive the state after each row), the
    // attention mixer's write, then the MLP half (mixer read, MoE, output map, mixer write).
    // Returns the layer's output streams.
    [[nodiscard]] DeviceTensor forward_verify_dense_batched(const DeviceTensor& streams, const DecoderLayerState& origin,
                                                            std::vector<DecoderLayerState>& checkpoints) const;
    [[nodiscard]] bool linear() const noexcept { return linear_ != nullptr; }

private:
    const HyperConnection* attention_mixer_ = nullptr;
    const GatedDeltaNet* linear_ = nullptr;
    const SelfAttention* full_ = nullptr;
    const HyperConnection* mlp_mixer_ = nullptr;
    const SparseMoe* mlp_ = nullptr;
    const q38_mlp_map* map_ = nullptr;
    mutable DeviceTensor workspace_;
};

// ------------------------------------------------------------------ verify model
struct GreedyStep {
    std::uint32_t token{0};
    float logit{0.0F};
};

// The verify-path model: seeded embedding, a stack of SparseMoe layers applied as
// h <- h + MoE(RMSNorm(h)), a final RMSNorm and the Q8 LM head (exact greedy argmax).
class QwenModel final {
public:
    QwenModel(const Context& ctx, std::uint64_t seed, std::size_t layer_count, std::size_t vocab,
              const MoeGeometry& geometry = {}, std::size_t expert_count = 512, std::size_t experts_per_token = 10,
              float rms_eps = 1e-6F);
    ~QwenModel();
    QwenModel(const QwenModel&) = delete;
    QwenModel& operator=(const QwenModel&) = delete;

    [[nodiscard]] const Context& context() const noexcept { return *ctx_; }
    [[nodiscard]] std::size_t hidden() const noexcept { return geometry_.hidden; }
    [[nodiscard]] std::size_t vocab() const noexcept { return vocab_; }
    [[nodiscard]] std::size_t layer_count() const noexcept { return layers_.size(); }

    // Layer-major verify of the given tokens (rows 1..16): returns the final hidden rows
    // (after the final RMSNorm) and each row's greedy step.
    // pre_mixer_streams (optional): the rows' residual streams after the last layer, before
    // the final norm ([1, rows, H] bf16; the reference's pre_mixer_stream rows).
    void forward_verify_layer_major(std::span<const std::uint32_t> tokens, DeviceTensor& final_mixed,
                                    std::vector<GreedyStep>& greedy, MoeVerifyTimings* timings = nullptr,
                                    DeviceTensor* pre_mixer_streams = nullptr) const;
    [[nodiscard]] std::uint64_t seed() const noexcept { return seed_; }
    [[nodiscard]] const MoeGeometry& geometry() const noexcept { return geometry_; }

private:
    const Context* ctx_ = nullptr;
    MoeGeometry geometry_;
    std::uint64_t seed_ = 0;
    std::size_t vocab_ = 0;
    float eps_ = 1e-6F;
    std::vector<SparseMoe> layers_;
    q38_head* head_ = nullptr;
    mutable DeviceTensor moe_ws_, head_ws_, tokens_dev_, h_;
};

// Per-request decode state of the verify path: the committed length and the committed
// hidden row, with the verification rows as speculative checkpoints (a q38 slot).
class ModelDecodeState final {
public:
    ModelDecodeState(const QwenModel& model, std::size_t token_count, std::size_t max_rows = 8);
    ~ModelDecodeState();
    ModelDecodeState(const ModelDecodeState&) = delete;
    ModelDecodeState& operator=(const ModelDecodeState&) = delete;
    [[nodiscard]] std::size_t token_count() const;
    [[nodiscard]] q38_slot* slot() const noexcept { return slot_; }

private:
    q38_slot* slot_ = nullptr;
};

struct MtpTargetVerifyRow {
    GreedyStep greedy;
    DeviceTensor final_mixed;       // [1, 1, H] bf16 final hidden of the row
    DeviceTensor pre_mixer_stream;  // [1, 1, H] bf16 residual stream before the final norm
    std::size_t state_after{0};  // token count of the state after this row
};

struct MtpTargetVerification {
    std::size_t draft_count{0};
    std::vector<MtpTargetVerifyRow> rows;
    ModelDecodeState* origin = nullptr;  // the state whose slot holds the staged checkpoints
    std::uint64_t generation{0};         // the slot's staging generation of these rows
};

// The correctness oracle of the verification (include/qwen38/mtp_verifier.hpp:27-31,
// src/mtp_verifier.cpp:59-82): one target decode per row, each row's state built on the
// previous one; the rows are staged as checkpoints like the layer-major pass's. For up to
// four rows (one kernel family) its results equal the layer-major pass's bit for bit.
[[nodiscard]] MtpTargetVerification verify_mtp_target_serial_oracle(const QwenModel& model,
                                                                   std::uint32_t current_token,
                                                                   std::span<const std::uint32_t> drafts,
                                                                   ModelDecodeState& origin);

[[nodiscard]] MtpTargetVerification verify_mtp_target_layer_major_reference(const QwenModel& model,
                                                                           std::uint32_t current_token,
                                                                           std::span<const std::uint32_t> drafts,
                                                                           ModelDecodeState& origin);

// accepted = N keeps the checkpoint after current_token plus N accepted drafts. Consumes
// all verification rows on success; validation failures leave verification and
// destination intact. A verification whose checkpoints the state has since replaced (a
// later verification was staged on it) is rejected.
void commit_mtp_target_verification(MtpTargetVerification&& verification, std::size_t accepted,
                                    ModelDecodeState& destination);

// ------------------------------------------------------------------ lifecycle (host)
struct MtpCommitPlan {
    std::size_t truncate_head_to{0};
    std::size_t target_rows_to_keep{0};
    std::size_t stash_rows{0};
    std::size_t committed_boundary{0};
};
[[nodiscard]] MtpCommitPlan plan_mtp_commit(std::size_t round_offset, std::size_t drafted, std::size_t accepted);

struct MtpGreedyDecision {
    std::size_t accepted{0};
    std::size_t correction_row{0};
    std::uint32_t next_token{0};
};
[[nodiscard]] MtpGreedyDecision decide_mtp_greedy(std::span<const std::uint32_t> drafts,
                                                  std::span<const std::uint32_t> target_argmax_rows,
                                                  std::span<const std::uint32_t> stop_tokens = {});

// Packed-VQ geometry (src/quantization_geometry.cpp:37-67).
[[nodiscard]] std::size_t packed_vq_word_count(std::size_t code_count, std::size_t bits_per_code);
[[nodiscard]] std::uint32_t unpack_vq_code(std::span<const std::uint32_t> words, std::size_t code_index,
                                           std::size_t bits_per_code);
[[nodiscard]] bool supports_segmented_vq(std::size_t dimension, std::size_t packed_bits) noexcept;

// ------------------------------------------------------------------ round
struct MtpRoundStep {
    std::vector<std::uint32_t> emitted_tokens;
    std::vector<std::uint32_t> draft_tokens;
    std::size_t accepted{0};
    std::uint32_t next_current_token{0};
    std::size_t next_query_position{0};
    DeviceTensor next_target_stream;  // pre_mixer_stream of the correction row (set by the head rounds)
    double draft_ms{0.0};
    double verify_ms{0.0};
    double commit_ms{0.0};
};

// One greedy round with externally proposed drafts: verify [current, drafts...], decide,
// commit. current_token has been emitted but is not yet in target_state.
[[nodiscard]] MtpRoundStep run_greedy_external_draft_round_reference(const QwenModel& target,
                                                                     std::uint32_t current_token,
                                                                     std::size_t query_position,
                                                                     std::vector<std::uint32_t> drafts,
                                                                     ModelDecodeState& target_state,
                                                                     std::span<const std::uint32_t> stop_tokens = {});

// ------------------------------------------------------------------ MTP draft head
// MtpDecodeState (include/qwen38/mtp_head.hpp:14-18): the head's position bookkeeping. The
// verify path's head block is a SparseMoe layer without attention, so there is no per-row
// cache to hold; positions must still advance contiguously.
struct MtpDecodeState {
    std::size_t row_count{0};
    std::optional<std::size_t> position_base;
};
[[nodiscard]] MtpDecodeState snapshot_mtp_decode_state(const MtpDecodeState& state);

struct MtpDecodeStep {
    DeviceTensor logits;            // [1, 1, V] float
    DeviceTensor pre_mixer_stream;  // [1, 1, H] bf16: the step's output stream
};

// QwenMtpHead (include/qwen38/mtp_head.hpp:29-63) over q38_mtp_head (include/q38.h): the
// seeded random-init draft head of a QwenModel with the same seed and geometry.
class QwenMtpHead final {
public:
    QwenMtpHead(const Context& ctx, std::uint64_t seed, std::size_t vocab, const MoeGeometry& geometry = {},
                std::size_t expert_count = 512, std::size_t experts_per_token = 10);
    ~QwenMtpHead();
    QwenMtpHead(const QwenMtpHead&) = delete;
    QwenMtpHead& operator=(const QwenMtpHead&) = delete;

    [[nodiscard]] MtpDecodeState make_state() const { return {}; }
    [[nodiscard]] MtpDecodeState snapshot_state(const MtpDecodeState& state) const {
        return snapshot_mtp_decode_state(state);
    }
    // The reference head's HC streams (src/mtp_head.cpp:120-170, 223-267, 454-470): the
    // block's MLP mixer (with injection weights), the final mixer (without), and the raw
    // pre_fc_norm_embedding [H] and pre_fc_norm_hidden [HC * H] weights (empty: zeros).
    // Afterwards target streams are [1, 1, HC * H]. The mixers must outlive the head's use.
    void attach_streams(const HyperConnection& block_mixer, const HyperConnection& final_mixer,
                        const DeviceTensor& embedding_norm = DeviceTensor(),
                        const DeviceTensor& hidden_norm = DeviceTensor());
    [[nodiscard]] std::size_t stream_count() const noexcept { return streams_; }
    // forward_decode (src/mtp_head.cpp:454-470): target_pre_mixer_stream [1, 1, HC * H] bf16.
    [[nodiscard]] MtpDecodeStep forward_decode(const DeviceTensor& target_pre_mixer_stream, std::uint32_t next_token,
                                               std::size_t query_position, MtpDecodeState& state) const;
    // The greedy draft chain (draft_lazy_chain, src/mtp_runner.cpp:152-211): depth drafts on
    // the device, read back once; advances state by depth rows.
    [[nodiscard]] std::vector<std::uint32_t> draft_greedy(const DeviceTensor& target_pre_mixer_stream,
                                                          std::uint32_t current_token, std::size_t query_position,
                                                          std::size_t depth, MtpDecodeState& state) const;
    // Several requests' chains in one pass per step (rows 1..4): row r starts from
    // streams[r] ([1, 1, H] each) and tokens[r]; returns drafts[r] (depth each). No state.
    [[nodiscard]] std::vector<std::vector<std::uint32_t>> draft_greedy_rows(std::span<const DeviceTensor* const> streams,
                                                                            std::span<const std::uint32_t> tokens,
                                                                            std::size_t depth) const;
    // consume_decode (src/mtp_head.cpp): a committed row advances the head's positions.
    void consume_decode(const DeviceTensor& target_pre_mixer_stream, std::uint32_t next_token,
                        std::size_t query_position, MtpDecodeState& state) const;

    [[nodiscard]] q38_mtp_head* handle() const noexcept { return head_; }
    [[nodiscard]] std::size_t vocab() const noexcept { return vocab_; }

private:
    void advance(std::size_t query_position, std::size_t rows, MtpDecodeState& state) const;
    const Context* ctx_ = nullptr;
    q38_mtp_head* head_ = nullptr;
    [[nodiscard]] std::size_t width() const noexcept { return hidden_ * streams_; }
    std::size_t hidden_ = 0, vocab_ = 0, streams_ = 1;
    mutable DeviceTensor ws_, tokens_dev_, streams_dev_, drafts_dev_;
};

// run_greedy_mtp_round_reference (include/qwen38/mtp_runner.hpp:38-47,
// src/mtp_runner.cpp:355-406): draft depth (2..4) tokens with the head from the previous
// target stream, verify them layer-major, decide, commit; the head's state is restored to its
// origin before verification and advanced over the committed rows.
[[nodiscard]] MtpRoundStep run_greedy_mtp_round_reference(const QwenModel& target, const QwenMtpHead& head,
                                                          std::uint32_t current_token,
                                                          const DeviceTensor& previous_target_stream,
                                                          std::size_t query_position, std::size_t draft_depth,
                                                          ModelDecodeState& target_state, MtpDecodeState& head_state,
                                                          std::span<const std::uint32_t> stop_tokens = {});
// run_greedy_external_draft_round_reference with the reference's full signature
// (include/qwen38/mtp_runner.hpp:49-60): externally proposed drafts (2..24), the head's state
// bookkept as in the learned round.
[[nodiscard]] MtpRoundStep run_greedy_external_draft_round_reference(
    const QwenModel& target, const QwenMtpHead& head, std::uint32_t current_token,
    const DeviceTensor& previous_target_stream, std::size_t query_position, std::vector<std::uint32_t> drafts,
    ModelDecodeState& target_state, MtpDecodeState& head_state, std::span<const std::uint32_t> stop_tokens = {});

// ------------------------------------------------------------------ batched slots
// BatchVerifier on the GPU: one verification packs every slot's rows [current, drafts...]
// into one layer-major pass of the model (up to 16 rows) and stages each slot's rows as the
// checkpoints of its decode state; commit() keeps one of them (q38_slot_commit).
class QwenBatchVerifier final : public BatchVerifier {
public:
    QwenBatchVerifier(const QwenModel& model, std::vector<ModelDecodeState*> slots);
    [[nodiscard]] std::size_t max_rows() const override { return 16; }
    [[nodiscard]] std::vector<std::vector<std::uint32_t>> verify(std::span<const SlotVerifyRows> batch) override;
    void commit(std::size_t slot, std::size_t accepted) override;
    // Final hidden rows [1, rows, H] of the last verification, in batch order.
    [[nodiscard]] const DeviceTensor& last_final_mixed() const noexcept { return final_mixed_; }
    // The pre-norm stream row [1, 1, H] of the slot's last committed checkpoint (empty before
    // its first commit): the next draft chain's input.
    [[nodiscard]] const DeviceTensor& committed_stream(std::size_t slot) const;

private:
    const QwenModel& model_;
    std::vector<ModelDecodeState*> slots_;
    DeviceTensor final_mixed_, pre_mixer_;
    std::vector<std::size_t> row_of_;      // first row of each slot in the last verification
    std::vector<DeviceTensor> committed_;  // per slot
};

// LearnedDrafter over the draft head: each slot's chain starts from the pre-norm stream of its
// last committed checkpoint (none before the first commit: no drafts, a serial step), and up
// to 4 slots share each chain step.
class MtpHeadDrafter final : public LearnedDrafter {
public:
    MtpHeadDrafter(const QwenMtpHead& head, const QwenBatchVerifier& verifier) : head_(head), verifier_(verifier) {}
    [[nodiscard]] std::vector<std::uint32_t> propose(std::size_t slot, std::uint32_t current_token,
                                                     std::size_t depth) override;
    [[nodiscard]] std::vector<std::vector<std::uint32_t>> propose_batch(std::span<const DraftRequest> requests) override;

private:
    const QwenMtpHead& head_;
    const QwenBatchVerifier& verifier_;
};

} // namespace qwen38
