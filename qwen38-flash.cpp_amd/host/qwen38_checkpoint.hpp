// qwen38_checkpoint.hpp — the on-disk VQ checkpoint format of the sparse-MoE layers: the
// manifest's vq_modules metadata and safetensors tensors, read and checked on the host, then
// uploaded into a q38 layer. Host-only C++20.
//
// Format (the reference's, kept alike so that its checkpoints load unchanged):
//   config.json      "vq_modules": {module: {experts, out, in, k, dim, group, pack_bits}}
//                    (ModelManifest, src/model_manifest.cpp:210-230), the expert count and
//                    top-k in "text_config" (or the root): num_experts, num_experts_per_tok,
//                    norm_topk_prob.
//   *.safetensors    (a model.safetensors.index.json weight_map, or every *.safetensors file
//                    of the directory) with, per VQ projection `base`
//                    (SparseMoe::load_projection, src/sparse_moe.cpp:618-661):
//                      base.codes      [experts, out, width] U32 packed (pack_bits 1..31,
//                                      width = packed_vq_word_count(in/dim, pack_bits)) or
//                                      U8 one code per byte (pack_bits 0, width = in/dim)
//                      base.codebook   [k, dim] F16
//                      base.vq_scales  [experts, out, in/group] F16
//                    and per layer prefix: prefix.gate.weight [E, H] BF16 (the router,
//                    src/sparse_moe.cpp:467) and, with a shared expert,
//                    prefix.shared_expert_gate.weight [1, H] BF16 plus the MLX affine
//                    projections prefix.shared_expert.{gate,up,down}_proj (the affine branch of
//                    SparseMoe::load_projection, src/sparse_moe.cpp:662-700):
//                      base.weight     [out, in * bits / 32] U32 (values LSB-first)
//                      base.scales     [out, in / group] BF16 or F16
//                      base.biases     [out, in / group] BF16 or F16
//                    with bits inferred from the shapes (infer_affine_quantization_bits,
//                    src/quantization_geometry.cpp:9-35) and checked against the manifest's
//                    "quantization" (or "quantization_config") bits for the module, whose
//                    group_size it takes (ModelManifest::quantization_for,
//                    src/model_manifest.cpp:188-208, 470-482).
// Module and tensor names resolve as the reference's do: a name under "language_model." that
// is absent falls back to the name without it (src/model_manifest.cpp:484-500).
// Byte codes (pack_bits 0) are the 8-bit packed layout when in/dim is a multiple of 32 (four
// codes per word, lowest byte first); other widths are re-laid out into 32-code blocks.
#pragma once

#include "q38.h"

#include <cstddef>
#include <cstdint>
#include <map>
#include <memory>
#include <optional>
#include <string>
#include <string_view>
#include <variant>
#include <vector>

namespace qwen38 {

// A parsed JSON value (objects keep their keys sorted; numbers are doubles, with the exact
// integer kept when the text is an integer).
class Json {
public:
    using Object = std::map<std::string, Json, std::less<>>;
    using Array = std::vector<Json>;
    static Json parse(std::string_view text);

    [[nodiscard]] bool is_object() const noexcept { return std::holds_alternative<Object>(v_); }
    [[nodiscard]] bool is_array() const noexcept { return std::holds_alternative<Array>(v_); }
    [[nodiscard]] bool is_string() const noexcept { return std::holds_alternative<std::string>(v_); }
    [[nodiscard]] bool is_number() const noexcept { return std::holds_alternative<Number>(v_); }
    [[nodiscard]] bool is_bool() const noexcept { return std::holds_alternative<bool>(v_); }
    [[nodiscard]] bool is_null() const noexcept { return std::holds_alternative<std::nullptr_t>(v_); }
    [[nodiscard]] const Json* find(std::string_view key) const;
    [[nodiscard]] const Json& at(std::string_view key) const;
    [[nodiscard]] const Object& as_object() const;
    [[nodiscard]] const Array& as_array() const;
    [[nodiscard]] const std::string& as_string() const;
    [[nodiscard]] double as_number() const;
    [[nodiscard]] bool as_bool() const;
    // A non-negative integer (throws for fractions, negatives and values past 2^53).
    [[nodiscard]] std::uint64_t as_size(std::string_view what) const;

private:
    struct Number {
        double value;
        bool integral;
    };
    std::variant<std::nullptr_t, bool, Number, std::string, Array, Object> v_{nullptr};
    friend class JsonParser;
};

// VectorQuantizationSpec (include/qwen38/model_manifest.hpp).
struct VectorQuantizationSpec {
    std::size_t expert_count{0};
    std::size_t output_dimension{0};
    std::size_t input_dimension{0};
    std::size_t codebook_size{0};
    std::size_t vector_dimension{0};
    std::size_t group_size{0};
    std::size_t packed_bits{0};  // 0: one code per byte
};

// QuantizationSpec (include/qwen38/model_manifest.hpp): affine bits and group size.
struct QuantizationSpec {
    std::size_t bits{0};
    std::size_t group_size{0};
};

// The manifest subset the MoE layers need (config.json of a checkpoint directory).
class ModelManifest {
public:
    static ModelManifest load(const std::string& directory);
    static ModelManifest parse(std::string_view config_json);
    [[nodiscard]] std::size_t expert_count() const noexcept { return expert_count_; }
    [[nodiscard]] std::size_t experts_per_token() const noexcept { return experts_per_token_; }
    [[nodiscard]] bool normalize_topk_probability() const noexcept { return normalize_; }
    // The config's shared_expert_intermediate_size (0 when the config has none).
    [[nodiscard]] std::size_t shared_expert_intermediate_size() const noexcept { return shared_inter_; }
    [[nodiscard]] const VectorQuantizationSpec* vector_quantization_for(std::string_view module) const;
    // The module's override, else the model-wide bits and group size; throws when the config
    // carries no quantization metadata (the reference requires it of every model).
    [[nodiscard]] QuantizationSpec quantization_for(std::string_view module) const;

private:
    std::size_t expert_count_{0}, experts_per_token_{0}, shared_inter_{0};
    bool normalize_{true};
    bool has_quantization_{false};
    QuantizationSpec quantization_{};
    std::map<std::string, QuantizationSpec, std::less<>> quantization_overrides_;
    std::map<std::string, VectorQuantizationSpec, std::less<>> vq_;
};

// A tensor of a memory-mapped safetensors file (host view).
struct TensorView {
    std::string dtype;                 // "U8", "U32", "F16", "BF16", ...
    std::vector<std::int64_t> shape;
    const void* data{nullptr};
    std::size_t nbytes{0};
};

// The tensors of a checkpoint directory (memory-mapped; checked header offsets).
class TensorStore {
public:
    explicit TensorStore(const std::string& directory);
    ~TensorStore();
    TensorStore(const TensorStore&) = delete;
    TensorStore& operator=(const TensorStore&) = delete;
    [[nodiscard]] bool has(std::string_view name) const;
    [[nodiscard]] const TensorView& tensor(std::string_view name) const;  // throws when absent
    [[nodiscard]] const ModelManifest& manifest() const noexcept { return manifest_; }

private:
    struct Mapping;
    void map_file(const std::string& path);
    ModelManifest manifest_;
    std::vector<std::unique_ptr<Mapping>> files_;
    std::map<std::string, TensorView, std::less<>> tensors_;
};

// One MLX affine projection's host tensors after the reference's checks (bits inferred from
// the shapes and equal to the manifest's; scales and biases of one dtype).
struct AffineProjectionTensors {
    std::size_t bits{0}, group_size{0}, out{0}, in{0};
    const TensorView* weight{nullptr};
    const TensorView* scales{nullptr};
    const TensorView* biases{nullptr};
};
[[nodiscard]] AffineProjectionTensors load_affine_projection(const TensorStore& store, std::string_view base);

// One VQ projection's host tensors after the reference's checks.
struct VqProjectionTensors {
    VectorQuantizationSpec spec;
    const TensorView* codes{nullptr};
    const TensorView* codebook{nullptr};
    const TensorView* scales{nullptr};
};
[[nodiscard]] VqProjectionTensors load_vq_projection(const TensorStore& store, std::string_view base);

// The affine shared expert of the layer at `prefix` and its BF16 gate row.
struct SharedExpertTensors {
    AffineProjectionTensors proj[3];  // gate, up, down
    const TensorView* gate{nullptr};
};
[[nodiscard]] SharedExpertTensors checkpoint_shared_expert(const TensorStore& store, std::string_view prefix,
                                                           std::size_t hidden);

// The q38 layer description of the MoE layer at `prefix` (geometry from the VQ modules).
[[nodiscard]] q38_moe_desc checkpoint_layer_desc(const TensorStore& store, std::string_view prefix,
                                                 std::size_t experts_per_token, bool normalize_topk_probability);

} // namespace qwen38
