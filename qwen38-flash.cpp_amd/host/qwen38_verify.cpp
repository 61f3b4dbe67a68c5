// qwen38_verify.cpp — C++20 host interface of the verify round over the C ABI (q38.h).
// Every device operation goes through libq38's HIP kernels; this file only orders them,
// owns buffers and converts error codes to the reference's exception types.
#include "qwen38_verify.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstdint>
#include <mutex>
#include <stdexcept>

namespace qwen38 {
namespace {

void check(int rc, const char* what) {
    if (rc == Q38_OK) return;
    std::string msg = std::string(what) + ": " + q38_last_error();
    if (rc == Q38_ERANGE) throw std::out_of_range(msg);
    throw std::runtime_error(msg);
}
void check_hip(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

std::size_t rows_of(const DeviceTensor& t, std::size_t hidden) {
    const auto& s = t.shape();
    if (t.dtype() != DType::bf16 || s.empty() || s.back() != hidden)
        throw std::runtime_error("expected a bf16 tensor whose last dimension is the hidden size");
    std::size_t rows = 1;
    for (std::size_t i = 0; i + 1 < s.size(); ++i) rows *= s[i];
    return rows;
}

std::mutex g_ws_mutex;  // lazily sized workspaces of logically const objects

} // namespace

// ------------------------------------------------------------------ Context / tensors
Context::Context(int hip_device) {
    check(q38_ctx_create(hip_device, &ctx_), "q38_ctx_create");
    hipStream_t s = nullptr;
    const hipError_t e = hipStreamCreate(&s);  // default priority
    if (e != hipSuccess) {
        q38_ctx_destroy(ctx_);
        check_hip(e, "hipStreamCreate");
    }
    stream_ = s;
}
Context::~Context() {
    if (stream_) (void)hipStreamDestroy(static_cast<hipStream_t>(stream_));
    q38_ctx_destroy(ctx_);
}
// Every read-back of the host interface waits here: the stream's work, then the device's
// status of the one-launch layer kernel's bounded waits (a wait that gave up throws, as any
// other failed verification does, instead of passing NaN rows on).
void Context::synchronize() const { check(q38_ctx_synchronize(ctx_, stream_), "sync"); }

std::size_t dtype_size(DType t) noexcept {
    switch (t) {
        case DType::bf16:
        case DType::f16: return 2;
        default: return 4;
    }
}

DeviceTensor::DeviceTensor(std::vector<std::size_t> shape, DType dtype) : shape_(std::move(shape)), dtype_(dtype) {
    const std::size_t n = std::max<std::size_t>(nbytes(), 1);
    void* p = nullptr;
    check_hip(hipMalloc(&p, n), "hipMalloc");
    buf_ = std::shared_ptr<void>(p, [](void* q) { (void)hipFree(q); });
}
DeviceTensor DeviceTensor::share() const {
    DeviceTensor t;
    t.buf_ = buf_;
    t.shape_ = shape_;
    t.dtype_ = dtype_;
    return t;
}
std::size_t DeviceTensor::numel() const noexcept {
    std::size_t n = 1;
    for (std::size_t d : shape_) n *= d;
    return n;
}
void DeviceTensor::upload(const void* host, std::size_t bytes) {
    if (bytes > nbytes()) throw std::runtime_error("upload larger than the tensor");
    check_hip(hipMemcpy(data(), host, bytes, hipMemcpyHostToDevice), "upload");
}
void DeviceTensor::download(void* host, std::size_t bytes) const {
    if (bytes > nbytes()) throw std::runtime_error("download larger than the tensor");
    check_hip(hipMemcpy(host, data(), bytes, hipMemcpyDeviceToHost), "download");
}

// ------------------------------------------------------------------ SparseMoe
static q38_moe_desc make_desc(std::size_t experts, std::size_t top_k, bool normalize, const MoeGeometry& g,
                              std::size_t group) {
    q38_moe_desc d{};
    d.hidden = static_cast<int32_t>(g.hidden);
    d.inter = static_cast<int32_t>(g.intermediate);
    d.experts = static_cast<int32_t>(experts);
    d.top_k = static_cast<int32_t>(top_k);
    d.gu_dim = static_cast<int32_t>(g.gate_up_dimension);
    d.gu_bits = static_cast<int32_t>(g.gate_up_bits);
    d.down_dim = static_cast<int32_t>(g.down_dimension);
    d.down_bits = static_cast<int32_t>(g.down_bits);
    d.gu_group = static_cast<int32_t>(group ? group : g.hidden);
    d.down_group = static_cast<int32_t>(group ? group : g.intermediate);
    d.normalize_topk = normalize ? 1 : 0;
    d.has_shared = g.shared_expert ? 1 : 0;
    return d;
}

SparseMoe::SparseMoe(const Context& ctx, const q38_moe_weights& tensors, std::size_t expert_count,
                     std::size_t experts_per_token, std::size_t quantization_bits,
                     std::size_t quantization_group_size, bool normalize_topk_probability, const MoeGeometry& geometry)
    : ctx_(&ctx) {
    if (quantization_bits != geometry.gate_up_bits)
        throw std::runtime_error("quantization_bits must equal the gate/up VQ code width");
    desc_ = make_desc(expert_count, experts_per_token, normalize_topk_probability, geometry, quantization_group_size);
    check(q38_moe_layer_create(ctx.handle(), &desc_, &tensors, &layer_), "SparseMoe");
}
SparseMoe::SparseMoe(const Context& ctx, std::uint64_t seed, int layer_index, std::size_t expert_count,
                     std::size_t experts_per_token, bool normalize_topk_probability, const MoeGeometry& geometry)
    : ctx_(&ctx) {
    desc_ = make_desc(expert_count, experts_per_token, normalize_topk_probability, geometry, 0);
    check(q38_moe_layer_create_synthetic(ctx.handle(), &desc_, seed, layer_index, &layer_), "SparseMoe");
}
SparseMoe::~SparseMoe() { q38_moe_layer_destroy(layer_); }
SparseMoe::SparseMoe(SparseMoe&& o) noexcept
    : ctx_(o.ctx_), layer_(o.layer_), desc_(o.desc_), workspace_(std::move(o.workspace_)) {
    o.layer_ = nullptr;
}
SparseMoe& SparseMoe::operator=(SparseMoe&& o) noexcept {
    if (this != &o) {
        q38_moe_layer_destroy(layer_);
        ctx_ = o.ctx_;
        layer_ = o.layer_;
        desc_ = o.desc_;
        workspace_ = std::move(o.workspace_);
        o.layer_ = nullptr;
    }
    return *this;
}

void SparseMoe::reserve_workspace(std::size_t rows) const {
    std::lock_guard<std::mutex> lk(g_ws_mutex);
    const std::size_t need = q38_moe_workspace_size(&desc_, static_cast<int32_t>(std::max<std::size_t>(rows, 16)));
    if (workspace_.nbytes() < need) workspace_ = DeviceTensor({need}, DType::u32);
}

std::vector<RouterSelection> SparseMoe::route_decode_batch(const DeviceTensor& input) const {
    const std::size_t rows = rows_of(input, static_cast<std::size_t>(desc_.hidden));
    if (rows < 1 || rows > 2048) throw std::runtime_error("route_decode: rows must be between 1 and 2048");
    const std::size_t k = experts_per_token();
    DeviceTensor ex({rows * k}, DType::i32), wt({rows * k}, DType::f32);
    reserve_workspace(rows);
    q38_route_out r{static_cast<int32_t*>(ex.data()), static_cast<float*>(wt.data()), nullptr, nullptr, nullptr};
    check(q38_moe_route(layer_, static_cast<const uint16_t*>(input.data()), static_cast<int32_t>(rows), &r,
                        workspace_.data(), workspace_.nbytes(), ctx_->stream()),
          "route_decode");
    ctx_->synchronize();
    const auto e = ex.to_host<int32_t>();
    const auto w = wt.to_host<float>();
    std::vector<RouterSelection> out(rows);
    for (std::size_t i = 0; i < rows; ++i) {
        for (std::size_t s = 0; s < k; ++s) {
            out[i].experts.push_back(static_cast<std::size_t>(e[i * k + s]));
            out[i].weights.push_back(w[i * k + s]);
        }
    }
    return out;
}
RouterSelection SparseMoe::route_decode(const DeviceTensor& input) const {
    auto all = route_decode_batch(input);
    if (all.size() != 1) throw std::runtime_error("route_decode expects one row");
    return std::move(all.front());
}

// One q38_moe_forward over `rows` rows of input into a new tensor of the input's shape.
DeviceTensor SparseMoe::forward_rows(const DeviceTensor& input, std::size_t rows, const char* what) const {
    DeviceTensor out(input.shape(), DType::bf16);
    reserve_workspace(rows);
    std::lock_guard<std::mutex> lk(g_ws_mutex);  // the workspace is shared by the calls of this layer
    check(q38_moe_forward(layer_, static_cast<const uint16_t*>(input.data()), static_cast<int32_t>(rows),
                          static_cast<uint16_t*>(out.data()), nullptr, workspace_.data(), workspace_.nbytes(),
                          ctx_->stream()),
          what);
    return out;
}

DeviceTensor SparseMoe::forward_verify(const DeviceTensor& input) const {
    const std::size_t rows = rows_of(input, static_cast<std::size_t>(desc_.hidden));
    if (input.shape().size() != 3 || input.shape()[0] != 1 || rows < 1 || rows > 1024)
        throw std::runtime_error("MoE batch requires shape [1,S,hidden], S=1..1024");
    return forward_rows(input, rows, "forward_verify");
}

DeviceTensor SparseMoe::forward_decode(const DeviceTensor& input) const {
    const std::size_t rows = rows_of(input, static_cast<std::size_t>(desc_.hidden));
    if (rows != 1) throw std::runtime_error("MoE decode requires shape [1,1,hidden]");
    return forward_rows(input, 1, "forward_decode");
}

std::vector<DeviceTensor> SparseMoe::forward_decode_multi(const std::vector<DeviceTensor>& inputs) const {
    if (inputs.empty()) throw std::runtime_error("multi-request MoE requires at least one row");
    const std::size_t H = static_cast<std::size_t>(desc_.hidden);
    if (inputs.size() > 2048) throw std::runtime_error("multi-request MoE takes at most 2048 rows");
    for (const DeviceTensor& in : inputs)
        if (rows_of(in, H) != 1) throw std::runtime_error("multi-request MoE requires [1,1,hidden] rows");
    const std::size_t n = inputs.size();
    DeviceTensor batch({1, n, H}, DType::bf16);
    const auto st = static_cast<hipStream_t>(ctx_->stream());
    for (std::size_t i = 0; i < n; ++i)
        check_hip(hipMemcpyAsync(static_cast<char*>(batch.data()) + i * H * 2, inputs[i].data(), H * 2,
                                 hipMemcpyDeviceToDevice, st),
                  "gather rows");
    DeviceTensor out = forward_rows(batch, n, "forward_decode_multi");
    std::vector<DeviceTensor> rows;
    rows.reserve(n);
    for (std::size_t i = 0; i < n; ++i) {
        DeviceTensor r(inputs[i].shape(), DType::bf16);
        check_hip(hipMemcpyAsync(r.data(), static_cast<const char*>(out.data()) + i * H * 2, H * 2,
                                 hipMemcpyDeviceToDevice, st),
                  "scatter rows");
        rows.push_back(std::move(r));
    }
    return rows;
}

DeviceTensor SparseMoe::forward_prefill(const DeviceTensor& input) const {
    const std::size_t rows = rows_of(input, static_cast<std::size_t>(desc_.hidden));
    if (rows < 1 || rows > 2048) throw std::runtime_error("MoE prefill requires shape [1,S,hidden], S=1..2048");
    return forward_rows(input, rows, "forward_prefill");
}

DeviceTensor SparseMoe::forward_prefill_profiled(const DeviceTensor& input, MoePrefillTimings& timings) const {
    const std::size_t rows = rows_of(input, static_cast<std::size_t>(desc_.hidden));
    if (rows < 17 || rows > 2048) throw std::runtime_error("profiled MoE prefill requires S=17..2048");
    DeviceTensor out(input.shape(), DType::bf16);
    float ms[7] = {};
    reserve_workspace(rows);
    std::lock_guard<std::mutex> lk(g_ws_mutex);
    check(q38_moe_forward_prefill_profiled(layer_, static_cast<const uint16_t*>(input.data()),
                                           static_cast<int32_t>(rows), static_cast<uint16_t*>(out.data()), nullptr,
                                           workspace_.data(), workspace_.nbytes(), ms, ctx_->stream()),
          "forward_prefill_profiled");
    timings = MoePrefillTimings{};
    timings.routing_ms = static_cast<double>(ms[0]) + ms[1] + ms[2];
    timings.gate_up_ms = ms[3];
    timings.swiglu_ms = ms[4];
    timings.down_qmm_ms = ms[5];
    timings.merge_ms = ms[6];
    return out;
}

void SparseMoe::set_router_bias(const DeviceTensor& bias) {
    if (bias.empty()) {
        check(q38_moe_layer_set_router_bias(layer_, nullptr), "set_router_bias");
        return;
    }
    if (bias.dtype() != DType::f32 || bias.numel() != static_cast<std::size_t>(desc_.experts))
        throw std::runtime_error("router bias must be an f32 tensor of expert_count values");
    check(q38_moe_layer_set_router_bias(layer_, static_cast<const float*>(bias.data())), "set_router_bias");
}

// ------------------------------------------------------------------ HyperConnection mixer
HyperConnection::HyperConnection(const Context& ctx, const q38_hc_weights& tensors, std::size_t hidden_size,
                                 std::size_t stream_count, std::size_t rank, std::size_t quantization_bits,
                                 std::size_t quantization_group_size, float rms_norm_epsilon, bool with_injection)
    : ctx_(&ctx) {
    if (!(rms_norm_epsilon > 0.0F)) throw std::runtime_error("RMS norm epsilon must be positive");
    desc_ = q38_hc_desc{static_cast<int32_t>(hidden_size), static_cast<int32_t>(stream_count),
                        static_cast<int32_t>(rank), static_cast<int32_t>(quantization_bits),
                        static_cast<int32_t>(quantization_group_size), with_injection ? 1 : 0, rms_norm_epsilon};
    check(q38_hc_create(ctx.handle(), &desc_, &tensors, &hc_), "HyperConnection");
}
HyperConnection::~HyperConnection() { q38_hc_destroy(hc_); }
HyperConnection::HyperConnection(HyperConnection&& o) noexcept
    : ctx_(o.ctx_), hc_(o.hc_), desc_(o.desc_), workspace_(std::move(o.workspace_)) {
    o.hc_ = nullptr;
}
HyperConnection& HyperConnection::operator=(HyperConnection&& o) noexcept {
    if (this != &o) {
        q38_hc_destroy(hc_);
        ctx_ = o.ctx_;
        hc_ = o.hc_;
        desc_ = o.desc_;
        workspace_ = std::move(o.workspace_);
        o.hc_ = nullptr;
    }
    return *this;
}

// ------------------------------------------------------------------ GatedDeltaNet
GatedDeltaNet::GatedDeltaNet(const Context& ctx, const q38_gdn_weights& tensors, std::size_t hidden_size,
                             std::size_t key_head_count, std::size_t value_head_count, std::size_t key_head_dimension,
                             std::size_t value_head_dimension, std::size_t convolution_kernel_size,
                             int quantization_bits, int quantization_group_size, bool fp16_scales,
                             const std::string& output_gate_type, float rms_norm_epsilon)
    : ctx_(&ctx), hidden_(hidden_size) {
    if (output_gate_type != "sigmoid" && output_gate_type != "silu")
        throw std::runtime_error("unsupported output_gate_type");
    const q38_gdn_desc d{static_cast<int32_t>(hidden_size), static_cast<int32_t>(key_head_count),
                         static_cast<int32_t>(value_head_count), static_cast<int32_t>(key_head_dimension),
                         static_cast<int32_t>(value_head_dimension), static_cast<int32_t>(convolution_kernel_size),
                         quantization_bits, quantization_group_size, fp16_scales ? 1 : 0,
                         output_gate_type == "silu" ? 1 : 0, rms_norm_epsilon};
    check(q38_gdn_create(ctx.handle(), &d, &tensors, &gdn_), "GatedDeltaNet");
}
GatedDeltaNet::~GatedDeltaNet() { q38_gdn_destroy(gdn_); }
GatedDeltaNet::GatedDeltaNet(GatedDeltaNet&& o) noexcept
    : ctx_(o.ctx_), gdn_(o.gdn_), hidden_(o.hidden_), workspace_(std::move(o.workspace_)) {
    o.gdn_ = nullptr;
}
GatedDeltaNet& GatedDeltaNet::operator=(GatedDeltaNet&& o) noexcept {
    if (this != &o) {
        q38_gdn_destroy(gdn_);
        ctx_ = o.ctx_;
        gdn_ = o.gdn_;
        hidden_ = o.hidden_;
        workspace_ = std::move(o.workspace_);
        o.gdn_ = nullptr;
    }
    return *this;
}
std::size_t GatedDeltaNet::state_bytes() const noexcept { return q38_gdn_state_bytes(gdn_); }

DeviceTensor GatedDeltaNet::forward_verify(const DeviceTensor& input, const GatedDeltaNetState& origin,
                                           std::vector<GatedDeltaNetState>& checkpoints) const {
    const auto& s = input.shape();
    if (s.size() != 3 || s[0] != 1 || s[1] < 1 || s[1] > 64 || s[2] != hidden_ || input.dtype() != DType::bf16)
        throw std::runtime_error("GatedDeltaNet batch requires shape [1,S,hidden], S=1..64");
    if (origin.initialized && origin.block.empty()) throw std::runtime_error("GatedDeltaNet origin state has no data");
    const std::size_t rows = s[1], sb = state_bytes();
    DeviceTensor out({1, rows, hidden_}, DType::bf16);
    DeviceTensor block({rows * sb / 2}, DType::bf16);
    std::lock_guard<std::mutex> lk(g_ws_mutex);
    const std::size_t need = q38_gdn_workspace_size(gdn_, static_cast<int32_t>(rows));
    if (workspace_.nbytes() < need) workspace_ = DeviceTensor({need}, DType::u32);
    check(q38_gdn_verify(gdn_, static_cast<const uint16_t*>(input.data()), static_cast<int32_t>(rows),
                         origin.initialized ? origin.data() : nullptr, block.data(),
                         static_cast<uint16_t*>(out.data()), workspace_.data(), workspace_.nbytes(), ctx_->stream()),
          "GatedDeltaNet::forward_verify");
    checkpoints.clear();
    checkpoints.resize(rows);
    for (std::size_t r = 0; r < rows; ++r) {
        checkpoints[r].block = block.share();
        checkpoints[r].offset = r * sb;
        checkpoints[r].initialized = true;
    }
    return out;
}

// ------------------------------------------------------------------ SelfAttention
SelfAttention::SelfAttention(const Context& ctx, const q38_attn_weights& tensors, std::size_t hidden_size,
                             std::size_t attention_heads, std::size_t key_value_heads, std::size_t head_dimension,
                             std::size_t rotary_dimension, int quantization_bits, int quantization_group_size,
                             bool fp16_scales, bool norm_has_offset, float rms_norm_epsilon, double rope_theta)
    : ctx_(&ctx), hidden_(hidden_size) {
    const q38_attn_desc d{static_cast<int32_t>(hidden_size), static_cast<int32_t>(attention_heads),
                          static_cast<int32_t>(key_value_heads), static_cast<int32_t>(head_dimension),
                          static_cast<int32_t>(rotary_dimension), quantization_bits, quantization_group_size,
                          fp16_scales ? 1 : 0, norm_has_offset ? 1 : 0, rms_norm_epsilon, rope_theta};
    check(q38_attn_create(ctx.handle(), &d, &tensors, &attn_), "SelfAttention");
}
SelfAttention::~SelfAttention() { q38_attn_destroy(attn_); }
SelfAttention::SelfAttention(SelfAttention&& o) noexcept
    : ctx_(o.ctx_), attn_(o.attn_), hidden_(o.hidden_), workspace_(std::move(o.workspace_)) {
    o.attn_ = nullptr;
}
SelfAttention& SelfAttention::operator=(SelfAttention&& o) noexcept {
    if (this != &o) {
        q38_attn_destroy(attn_);
        ctx_ = o.ctx_;
        attn_ = o.attn_;
        hidden_ = o.hidden_;
        workspace_ = std::move(o.workspace_);
        o.attn_ = nullptr;
    }
    return *this;
}

SelfAttentionState SelfAttention::make_state(std::size_t capacity, std::size_t position_base) const {
    const std::size_t bytes = q38_attn_cache_bytes(attn_, static_cast<int64_t>(capacity));
    if (bytes == 0) throw std::runtime_error("attention cache capacity must be positive");
    SelfAttentionState s;
    s.cache = DeviceTensor({bytes / 2}, DType::bf16);
    s.capacity = capacity;
    s.position_base = position_base;
    return s;
}

DeviceTensor SelfAttention::forward_verify(const DeviceTensor& input, const SelfAttentionState& origin,
                                           std::vector<SelfAttentionState>& checkpoints) const {
    const auto& s = input.shape();
    if (s.size() != 3 || s[0] != 1 || s[1] < 1 || s[1] > 64 || s[2] != hidden_ || input.dtype() != DType::bf16)
        throw std::runtime_error("attention batch requires shape [1,S,hidden], S=1..64");
    if (origin.cache.empty()) throw std::runtime_error("attention state has no cache");
    const std::size_t rows = s[1], tokens = origin.token_count + rows;
    DeviceTensor out({1, rows, hidden_}, DType::bf16);
    std::lock_guard<std::mutex> lk(g_ws_mutex);
    const std::size_t need = q38_attn_workspace_size(attn_, static_cast<int32_t>(rows), static_cast<int64_t>(tokens));
    if (workspace_.nbytes() < need) workspace_ = DeviceTensor({(need + 3) / 4}, DType::u32);
    check(q38_attn_verify(attn_, static_cast<const uint16_t*>(input.data()), static_cast<int32_t>(rows),
                          origin.cache.data(), static_cast<int64_t>(origin.capacity),
                          static_cast<int64_t>(origin.token_count),
                          static_cast<int64_t>(origin.position_base + origin.token_count),
                          static_cast<uint16_t*>(out.data()), workspace_.data(), workspace_.nbytes(), ctx_->stream()),
          "SelfAttention::forward_verify");
    checkpoints.clear();
    checkpoints.resize(rows);
    for (std::size_t r = 0; r < rows; ++r) {
        checkpoints[r].cache = origin.cache.share();
        checkpoints[r].capacity = origin.capacity;
        checkpoints[r].token_count = origin.token_count + r + 1;
        checkpoints[r].position_base = origin.position_base;
    }
    return out;
}

DeviceTensor HyperConnection::initialize_stream(const Context& ctx, const DeviceTensor& embedding,
                                                std::size_t stream_count) {
    const auto& s = embedding.shape();
    if (s.size() != 3) throw std::runtime_error("hyper-connection embedding must have rank 3");
    if (embedding.dtype() != DType::bf16) throw std::runtime_error("hyper-connection embedding must be bf16");
    const std::size_t rows = s[0] * s[1];
    DeviceTensor out({s[0], s[1], s[2] * stream_count}, DType::bf16);
    check(q38_hc_initialize_stream(static_cast<const uint16_t*>(embedding.data()), static_cast<int32_t>(rows),
                                   static_cast<int32_t>(s[2]), static_cast<int32_t>(stream_count),
                                   static_cast<uint16_t*>(out.data()), ctx.stream()),
          "initialize_stream");
    return out;
}

HyperConnectionRead HyperConnection::read(const DeviceTensor& stream) const {
    const auto& s = stream.shape();
    const std::size_t width = static_cast<std::size_t>(desc_.hidden) * static_cast<std::size_t>(desc_.streams);
    if (s.size() != 3 || s[2] != width || stream.dtype() != DType::bf16)
        throw std::runtime_error("invalid hyper-connection stream shape");
    const std::size_t rows = s[0] * s[1];
    HyperConnectionRead out;
    out.mixed = DeviceTensor({s[0], s[1], static_cast<std::size_t>(desc_.hidden)}, DType::bf16);
    if (desc_.with_injection) {
        out.injection = DeviceTensor({s[0], s[1], static_cast<std::size_t>(desc_.streams), 1}, DType::bf16);
        out.has_injection = true;
    }
    std::lock_guard<std::mutex> lk(g_ws_mutex);
    const std::size_t need = q38_hc_workspace_size(&desc_, static_cast<int32_t>(std::min<std::size_t>(rows, 16)));
    if (workspace_.nbytes() < need) workspace_ = DeviceTensor({need}, DType::u32);
    check(q38_hc_read(hc_, static_cast<const uint16_t*>(stream.data()), static_cast<int32_t>(rows),
                      static_cast<uint16_t*>(out.mixed.data()),
                      out.has_injection ? static_cast<uint16_t*>(out.injection.data()) : nullptr, workspace_.data(),
                      workspace_.nbytes(), ctx_->stream()),
          "HyperConnection::read");
    return out;
}

DeviceTensor HyperConnection::write(const DeviceTensor& stream, const DeviceTensor& block_output,
                                    const DeviceTensor& injection) const {
    const auto& s = stream.shape();
    if (s.size() != 3) throw std::runtime_error("hyper-connection stream must have rank 3");
    const std::size_t rows = s[0] * s[1];
    if (rows_of(block_output, static_cast<std::size_t>(desc_.hidden)) != rows ||
        injection.numel() != rows * static_cast<std::size_t>(desc_.streams) ||
        s[2] != static_cast<std::size_t>(desc_.hidden) * static_cast<std::size_t>(desc_.streams))
        throw std::runtime_error("invalid hyper-connection write shapes");
    DeviceTensor out(s, DType::bf16);
    check(q38_hc_write(hc_, static_cast<const uint16_t*>(stream.data()),
                       static_cast<const uint16_t*>(block_output.data()),
                       static_cast<const uint16_t*>(injection.data()), static_cast<int32_t>(rows),
                       static_cast<uint16_t*>(out.data()), ctx_->stream()),
          "HyperConnection::write");
    return out;
}

// ------------------------------------------------------------------ DecoderLayer (verify)
DecoderLayer::DecoderLayer(const HyperConnection& attention_mixer, const GatedDeltaNet& linear_attention,
                           const HyperConnection& mlp_mixer, const SparseMoe& mlp, const q38_mlp_map* output_map)
    : attention_mixer_(&attention_mixer), linear_(&linear_attention), mlp_mixer_(&mlp_mixer), mlp_(&mlp),
      map_(output_map) {}

DecoderLayer::DecoderLayer(const HyperConnection& attention_mixer, const SelfAttention& full_attention,
                           const HyperConnection& mlp_mixer, const SparseMoe& mlp, const q38_mlp_map* output_map)
    : attention_mixer_(&attention_mixer), full_(&full_attention), mlp_mixer_(&mlp_mixer), mlp_(&mlp),
      map_(output_map) {}

DeviceTensor DecoderLayer::forward_verify_dense_batched(const DeviceTensor& streams, const DecoderLayerState& origin,
                                                        std::vector<DecoderLayerState>& checkpoints) const {
    const auto& s = streams.shape();
    if (s.size() != 3 || s[0] != 1 || s[1] < 1 || s[1] > 16)
        throw std::runtime_error("decoder batch must contain 1 to 16 matching rows");
    const std::size_t rows = s[1];
    checkpoints.clear();
    checkpoints.resize(rows);
    // attention half (src/decoder_layer.cpp:469-491)
    const HyperConnectionRead attention = attention_mixer_->read(streams);
    DeviceTensor outputs;
    if (linear_) {
        std::vector<GatedDeltaNetState> cps;
        outputs = linear_->forward_verify(attention.mixed, origin.linear_attention, cps);
        for (std::size_t r = 0; r < rows; ++r) checkpoints[r].linear_attention = std::move(cps[r]);
    } else {
        std::vector<SelfAttentionState> cps;
        outputs = full_->forward_verify(attention.mixed, origin.full_attention, cps);
        for (std::size_t r = 0; r < rows; ++r) checkpoints[r].full_attention = std::move(cps[r]);
    }
    DeviceTensor post = attention_mixer_->write(streams, outputs, attention.injection);
    // MLP half (:493-497): read, MoE, output map, write, in place on the post-attention streams
    std::lock_guard<std::mutex> lk(g_ws_mutex);
    const std::size_t need = q38_verify_chain_hc_mapped_workspace_size(&mlp_->desc(), &mlp_mixer_->desc(),
                                                                       static_cast<int32_t>(rows));
    if (need == 0) throw std::runtime_error("decoder layer: no MLP-half workspace for these shapes");
    if (workspace_.nbytes() < need) workspace_ = DeviceTensor({need}, DType::u32);
    q38_moe_layer* layer = mlp_->handle();
    q38_hc* mixer = mlp_mixer_->handle();
    const q38_mlp_map* map = map_;
    check(q38_verify_chain_hc_mapped(&layer, &mixer, &map, 1, static_cast<uint16_t*>(post.data()),
                                     static_cast<int32_t>(rows), workspace_.data(), workspace_.nbytes(),
                                     mlp_mixer_->context().stream()),
          "DecoderLayer::forward_verify_dense_batched");
    return post;
}

// ------------------------------------------------------------------ QwenModel (verify path)
QwenModel::QwenModel(const Context& ctx, std::uint64_t seed, std::size_t layer_count, std::size_t vocab,
                     const MoeGeometry& geometry, std::size_t expert_count, std::size_t experts_per_token,
                     float rms_eps)
    : ctx_(&ctx), geometry_(geometry), seed_(seed), vocab_(vocab), eps_(rms_eps) {
    if (layer_count < 1) throw std::runtime_error("QwenModel needs at least one layer");
    layers_.reserve(layer_count);
    for (std::size_t l = 0; l < layer_count; ++l)
        layers_.emplace_back(ctx, seed, static_cast<int>(l), expert_count, experts_per_token, true, geometry);
    check(q38_head_create_synthetic(ctx.handle(), Q38_HEAD_Q8, static_cast<int64_t>(vocab),
                                    static_cast<int32_t>(geometry.hidden), seed, &head_),
          "LM head");
    moe_ws_ = DeviceTensor({q38_moe_workspace_size(&layers_.front().desc(), 16)}, DType::u32);
    head_ws_ = DeviceTensor({q38_head_workspace_size(head_, 16)}, DType::u32);
    tokens_dev_ = DeviceTensor({16}, DType::u32);
    h_ = DeviceTensor({16, geometry.hidden}, DType::bf16);
}
QwenModel::~QwenModel() { q38_head_destroy(head_); }

void QwenModel::forward_verify_layer_major(std::span<const std::uint32_t> tokens, DeviceTensor& final_mixed,
                                           std::vector<GreedyStep>& greedy, MoeVerifyTimings* timings,
                                           DeviceTensor* pre_mixer_streams) const {
    const std::size_t rows = tokens.size();
    if (rows < 1 || rows > 16) throw std::runtime_error("verify rows must be between 1 and 16");
    for (std::uint32_t t : tokens)
        if (t >= vocab_) throw std::runtime_error("token id outside the vocabulary");
    void* st = ctx_->stream();
    const auto H = static_cast<int32_t>(geometry_.hidden);
    const auto n = static_cast<int32_t>(rows);
    check_hip(hipMemcpyAsync(tokens_dev_.data(), tokens.data(), rows * 4, hipMemcpyHostToDevice,
                             static_cast<hipStream_t>(st)),
              "tokens");
    check(q38_embed_synthetic_dev(seed_, static_cast<const uint32_t*>(tokens_dev_.data()), n, H,
                                  static_cast<uint16_t*>(h_.data()), st),
          "embedding");
    std::vector<q38_moe_layer*> hs;
    for (const SparseMoe& L : layers_) hs.push_back(L.handle());
    if (timings) {
        q38_moe_timings t{};
        check(q38_verify_chain_profiled(hs.data(), static_cast<int32_t>(hs.size()), static_cast<uint16_t*>(h_.data()),
                                        n, eps_, nullptr, moe_ws_.data(), moe_ws_.nbytes(), &t, st),
              "verify chain");
        *timings = MoeVerifyTimings{t.routing_ms, t.gate_up_ms, t.down_ms, 0.0, t.merge_ms};
    } else {
        check(q38_verify_chain(hs.data(), static_cast<int32_t>(hs.size()), static_cast<uint16_t*>(h_.data()), n, eps_,
                               nullptr, moe_ws_.data(), moe_ws_.nbytes(), st),
              "verify chain");
    }
    if (pre_mixer_streams) {
        *pre_mixer_streams = DeviceTensor({1, rows, geometry_.hidden}, DType::bf16);
        check_hip(hipMemcpyAsync(pre_mixer_streams->data(), h_.data(), rows * geometry_.hidden * 2,
                                 hipMemcpyDeviceToDevice, static_cast<hipStream_t>(st)),
                  "pre-mixer streams");
    }
    final_mixed = DeviceTensor({1, rows, geometry_.hidden}, DType::bf16);
    check(q38_rmsnorm(static_cast<const uint16_t*>(h_.data()), n, H, eps_, static_cast<uint16_t*>(final_mixed.data()),
                      st),
          "final norm");
    DeviceTensor am({rows}, DType::u32), lg({rows}, DType::f32);
    check(q38_head_greedy(head_, static_cast<const uint16_t*>(final_mixed.data()), n, static_cast<uint32_t*>(am.data()),
                          static_cast<float*>(lg.data()), head_ws_.data(), head_ws_.nbytes(), st),
          "LM head");
    ctx_->synchronize();
    const auto a = am.to_host<uint32_t>();
    const auto l = lg.to_host<float>();
    greedy.resize(rows);
    for (std::size_t i = 0; i < rows; ++i) greedy[i] = GreedyStep{a[i], l[i]};
}

// ------------------------------------------------------------------ decode state / verify / commit
ModelDecodeState::ModelDecodeState(const QwenModel& model, std::size_t token_count, std::size_t max_rows) {
    check(q38_slot_create(model.context().handle(), static_cast<int32_t>(model.hidden()),
                          static_cast<int32_t>(max_rows), token_count, &slot_),
          "decode state");
}
ModelDecodeState::~ModelDecodeState() { q38_slot_destroy(slot_); }
std::size_t ModelDecodeState::token_count() const {
    uint64_t tc = 0;
    int32_t staged = 0, drafts = 0;
    check(q38_slot_info(slot_, &tc, &staged, &drafts), "decode state");
    return static_cast<std::size_t>(tc);
}

MtpTargetVerification verify_mtp_target_layer_major_reference(const QwenModel& model, std::uint32_t current_token,
                                                               std::span<const std::uint32_t> drafts,
                                                               ModelDecodeState& origin) {
    if (drafts.empty()) throw std::runtime_error("MTP verification requires at least one draft");
    std::vector<std::uint32_t> tokens;
    tokens.reserve(drafts.size() + 1);
    tokens.push_back(current_token);
    tokens.insert(tokens.end(), drafts.begin(), drafts.end());
    DeviceTensor final_mixed, streams;
    std::vector<GreedyStep> greedy;
    model.forward_verify_layer_major(tokens, final_mixed, greedy, nullptr, &streams);
    const std::size_t base = origin.token_count();
    check(q38_slot_stage(origin.slot(), static_cast<int32_t>(drafts.size()),
                         static_cast<const uint16_t*>(final_mixed.data()), model.context().stream()),
          "verification checkpoints");
    MtpTargetVerification v;
    v.draft_count = drafts.size();
    v.origin = &origin;
    v.generation = q38_slot_generation(origin.slot());
    const std::size_t H = model.hidden();
    for (std::size_t i = 0; i < tokens.size(); ++i) {
        MtpTargetVerifyRow row;
        row.greedy = greedy[i];
        row.final_mixed = DeviceTensor({1, 1, H}, DType::bf16);
        check_hip(hipMemcpyAsync(row.final_mixed.data(), static_cast<const char*>(final_mixed.data()) + i * H * 2,
                                 H * 2, hipMemcpyDeviceToDevice, static_cast<hipStream_t>(model.context().stream())),
                  "verification row");
        row.pre_mixer_stream = DeviceTensor({1, 1, H}, DType::bf16);
        check_hip(hipMemcpyAsync(row.pre_mixer_stream.data(), static_cast<const char*>(streams.data()) + i * H * 2,
                                 H * 2, hipMemcpyDeviceToDevice, static_cast<hipStream_t>(model.context().stream())),
                  "verification stream row");
        row.state_after = base + i + 1;
        v.rows.push_back(std::move(row));
    }
    model.context().synchronize();
    return v;
}

MtpTargetVerification verify_mtp_target_serial_oracle(const QwenModel& model, std::uint32_t current_token,
                                                      std::span<const std::uint32_t> drafts, ModelDecodeState& origin) {
    if (drafts.empty()) throw std::runtime_error("MTP verification requires at least one draft");
    std::vector<std::uint32_t> tokens;
    tokens.reserve(drafts.size() + 1);
    tokens.push_back(current_token);
    tokens.insert(tokens.end(), drafts.begin(), drafts.end());
    const std::size_t H = model.hidden(), n = tokens.size();
    const auto st = static_cast<hipStream_t>(model.context().stream());
    DeviceTensor all({1, n, H}, DType::bf16);  // the rows' final hidden states, staged below
    MtpTargetVerification v;
    v.draft_count = drafts.size();
    v.origin = &origin;
    const std::size_t base = origin.token_count();
    for (std::size_t i = 0; i < n; ++i) {
        // (in the verify model a row's decode reads only its own token: no attention state)
        MtpTargetVerifyRow row;
        std::vector<GreedyStep> greedy;
        model.forward_verify_layer_major(std::span<const std::uint32_t>(&tokens[i], 1), row.final_mixed, greedy,
                                         nullptr, &row.pre_mixer_stream);
        row.greedy = greedy.at(0);
        check_hip(hipMemcpyAsync(static_cast<char*>(all.data()) + i * H * 2, row.final_mixed.data(), H * 2,
                                 hipMemcpyDeviceToDevice, st),
                  "serial verification row");
        row.state_after = base + i + 1;
        v.rows.push_back(std::move(row));
    }
    check(q38_slot_stage(origin.slot(), static_cast<int32_t>(drafts.size()), static_cast<const uint16_t*>(all.data()),
                         model.context().stream()),
          "verification checkpoints");
    v.generation = q38_slot_generation(origin.slot());
    model.context().synchronize();
    return v;
}

void commit_mtp_target_verification(MtpTargetVerification&& verification, std::size_t accepted,
                                    ModelDecodeState& destination) {
    if (verification.rows.size() != verification.draft_count + 1)
        throw std::runtime_error("MTP verification row count is invalid");
    if (accepted > verification.draft_count)
        throw std::runtime_error("MTP accepted count exceeds verified draft count");
    if (verification.origin != &destination)
        throw std::runtime_error("MTP verification belongs to another decode state");
    if (verification.generation == 0 || q38_slot_generation(destination.slot()) != verification.generation)
        throw std::runtime_error("MTP verification is stale: the decode state holds a newer verification");
    check(q38_slot_commit(destination.slot(), static_cast<int64_t>(accepted), nullptr), "commit");
    verification.rows.clear();
    verification.draft_count = 0;
}

// ------------------------------------------------------------------ lifecycle (host, via the ABI)
MtpCommitPlan plan_mtp_commit(std::size_t round_offset, std::size_t drafted, std::size_t accepted) {
    uint64_t out[4] = {0, 0, 0, 0};
    check(q38_plan_mtp_commit(round_offset, drafted, accepted, out), "plan_mtp_commit");
    return MtpCommitPlan{static_cast<std::size_t>(out[0]), static_cast<std::size_t>(out[1]),
                         static_cast<std::size_t>(out[2]), static_cast<std::size_t>(out[3])};
}

MtpGreedyDecision decide_mtp_greedy(std::span<const std::uint32_t> drafts,
                                    std::span<const std::uint32_t> target_argmax_rows,
                                    std::span<const std::uint32_t> stop_tokens) {
    q38_greedy_decision d{};
    check(q38_mtp_decide_greedy(drafts.data(), static_cast<int64_t>(drafts.size()), target_argmax_rows.data(),
                                static_cast<int64_t>(target_argmax_rows.size()), stop_tokens.data(),
                                static_cast<int64_t>(stop_tokens.size()), &d),
          "decide_mtp_greedy");
    return MtpGreedyDecision{static_cast<std::size_t>(d.accepted), static_cast<std::size_t>(d.correction_row),
                             d.next_token};
}

std::size_t packed_vq_word_count(std::size_t code_count, std::size_t bits_per_code) {
    const int64_t n = q38_packed_vq_word_count(static_cast<int64_t>(code_count), static_cast<int>(bits_per_code));
    if (n < 0) check(static_cast<int>(n), "packed_vq_word_count");
    return static_cast<std::size_t>(n);
}
std::uint32_t unpack_vq_code(std::span<const std::uint32_t> words, std::size_t code_index, std::size_t bits_per_code) {
    uint32_t out = 0;
    check(q38_unpack_vq_code(words.data(), static_cast<int64_t>(words.size()), static_cast<int64_t>(code_index),
                             static_cast<int>(bits_per_code), &out),
          "unpack_vq_code");
    return out;
}
bool supports_segmented_vq(std::size_t dimension, std::size_t packed_bits) noexcept {
    return q38_supports_segmented_vq(static_cast<int>(dimension), static_cast<int>(packed_bits)) != 0;
}

// ------------------------------------------------------------------ round
MtpRoundStep run_greedy_external_draft_round_reference(const QwenModel& target, std::uint32_t current_token,
                                                       std::size_t query_position, std::vector<std::uint32_t> drafts,
                                                       ModelDecodeState& target_state,
                                                       std::span<const std::uint32_t> stop_tokens) {
    if (target_state.token_count() != query_position)
        throw std::runtime_error("MTP target state is not at the query position");
    const auto t0 = std::chrono::steady_clock::now();
    MtpTargetVerification verification =
        verify_mtp_target_layer_major_reference(target, current_token, drafts, target_state);
    const auto t1 = std::chrono::steady_clock::now();
    std::vector<std::uint32_t> target_rows;
    target_rows.reserve(verification.rows.size());
    for (const MtpTargetVerifyRow& row : verification.rows) target_rows.push_back(row.greedy.token);
    const MtpGreedyDecision decision = decide_mtp_greedy(drafts, target_rows, stop_tokens);
    commit_mtp_target_verification(std::move(verification), decision.accepted, target_state);
    const std::size_t next_query_position = query_position + decision.accepted + 1;
    if (target_state.token_count() != next_query_position)
        throw std::runtime_error("MTP committed target length mismatch");
    const auto t2 = std::chrono::steady_clock::now();
    std::vector<std::uint32_t> emitted;
    emitted.reserve(decision.accepted + 1);
    for (std::size_t i = 0; i < decision.accepted; ++i) emitted.push_back(drafts[i]);
    emitted.push_back(decision.next_token);
    MtpRoundStep step;
    step.emitted_tokens = std::move(emitted);
    step.draft_tokens = std::move(drafts);
    step.accepted = decision.accepted;
    step.next_current_token = decision.next_token;
    step.next_query_position = next_query_position;
    step.verify_ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
    step.commit_ms = std::chrono::duration<double, std::milli>(t2 - t1).count();
    return step;
}

// ------------------------------------------------------------------ MTP draft head
MtpDecodeState snapshot_mtp_decode_state(const MtpDecodeState& state) { return state; }

QwenMtpHead::QwenMtpHead(const Context& ctx, std::uint64_t seed, std::size_t vocab, const MoeGeometry& geometry,
                         std::size_t expert_count, std::size_t experts_per_token)
    : ctx_(&ctx), hidden_(geometry.hidden), vocab_(vocab) {
    q38_moe_desc d{};
    d.hidden = static_cast<int32_t>(geometry.hidden);
    d.inter = static_cast<int32_t>(geometry.intermediate);
    d.experts = static_cast<int32_t>(expert_count);
    d.top_k = static_cast<int32_t>(experts_per_token);
    d.gu_dim = static_cast<int32_t>(geometry.gate_up_dimension);
    d.gu_bits = static_cast<int32_t>(geometry.gate_up_bits);
    d.down_dim = static_cast<int32_t>(geometry.down_dimension);
    d.down_bits = static_cast<int32_t>(geometry.down_bits);
    d.gu_group = d.hidden;
    d.down_group = d.inter;
    d.normalize_topk = 1;
    d.has_shared = geometry.shared_expert ? 1 : 0;
    check(q38_mtp_head_create_synthetic(ctx.handle(), &d, static_cast<int64_t>(vocab), seed, &head_), "MTP head");
    ws_ = DeviceTensor({q38_mtp_workspace_size(head_, 4)}, DType::u32);
    tokens_dev_ = DeviceTensor({4}, DType::u32);
    streams_dev_ = DeviceTensor({4, hidden_}, DType::bf16);
    drafts_dev_ = DeviceTensor({4, 24}, DType::u32);
}
QwenMtpHead::~QwenMtpHead() { q38_mtp_head_destroy(head_); }

void QwenMtpHead::attach_streams(const HyperConnection& block_mixer, const HyperConnection& final_mixer,
                                 const DeviceTensor& embedding_norm, const DeviceTensor& hidden_norm) {
    const std::size_t hc = static_cast<std::size_t>(block_mixer.desc().streams);
    if ((!embedding_norm.empty() && (embedding_norm.numel() != hidden_ || embedding_norm.dtype() != DType::bf16)) ||
        (!hidden_norm.empty() && (hidden_norm.numel() != hc * hidden_ || hidden_norm.dtype() != DType::bf16)))
        throw std::runtime_error("MTP norm weights must be bf16 of the hidden size and the stream width");
    const q38_mtp_streams s{block_mixer.handle(), final_mixer.handle(),
                            embedding_norm.empty() ? nullptr : static_cast<const uint16_t*>(embedding_norm.data()),
                            hidden_norm.empty() ? nullptr : static_cast<const uint16_t*>(hidden_norm.data())};
    check(q38_mtp_head_set_streams(head_, &s), "MTP head streams");
    streams_ = static_cast<std::size_t>(q38_mtp_head_streams(head_));
    ws_ = DeviceTensor({q38_mtp_workspace_size(head_, 4)}, DType::u32);
    streams_dev_ = DeviceTensor({4, width()}, DType::bf16);
}

void QwenMtpHead::advance(std::size_t query_position, std::size_t rows, MtpDecodeState& state) const {
    if (!state.position_base.has_value()) state.position_base = query_position;
    if (query_position != *state.position_base + state.row_count)
        throw std::runtime_error("MTP query positions must be contiguous");
    state.row_count += rows;
}

MtpDecodeStep QwenMtpHead::forward_decode(const DeviceTensor& stream, std::uint32_t next_token,
                                          std::size_t query_position, MtpDecodeState& state) const {
    if (stream.shape() != std::vector<std::size_t>{1, 1, width()} || stream.dtype() != DType::bf16)
        throw std::runtime_error("MTP target stream must have shape [1,1,stream width] bf16");
    if (next_token >= vocab_) throw std::runtime_error("MTP token id is out of range");
    MtpDecodeState next = state;
    advance(query_position, 1, next);
    const hipStream_t st = static_cast<hipStream_t>(ctx_->stream());
    check_hip(hipMemcpyAsync(tokens_dev_.data(), &next_token, 4, hipMemcpyHostToDevice, st), "MTP token");
    MtpDecodeStep out{DeviceTensor({1, 1, vocab_}, DType::f32), DeviceTensor({1, 1, width()}, DType::bf16)};
    check(q38_mtp_forward_decode(head_, static_cast<const uint16_t*>(stream.data()),
                                 static_cast<const uint32_t*>(tokens_dev_.data()), 1, static_cast<float*>(out.logits.data()),
                                 static_cast<uint16_t*>(out.pre_mixer_stream.data()), nullptr, ws_.data(), ws_.nbytes(),
                                 ctx_->stream()),
          "MTP forward_decode");
    ctx_->synchronize();
    state = next;
    return out;
}

std::vector<std::vector<std::uint32_t>> QwenMtpHead::draft_greedy_rows(std::span<const DeviceTensor* const> streams,
                                                                       std::span<const std::uint32_t> tokens,
                                                                       std::size_t depth) const {
    const std::size_t rows = tokens.size();
    if (rows < 1 || rows > 4 || streams.size() != rows)
        throw std::runtime_error("MTP draft rows must be 1..4 matching streams and tokens");
    if (depth < 1 || depth > 24) throw std::runtime_error("MTP draft depth must be between 1 and 24");
    const hipStream_t st = static_cast<hipStream_t>(ctx_->stream());
    for (std::size_t r = 0; r < rows; ++r) {
        if (streams[r] == nullptr || streams[r]->numel() != width() || streams[r]->dtype() != DType::bf16)
            throw std::runtime_error("MTP target stream must have shape [1,1,stream width] bf16");
        if (tokens[r] >= vocab_) throw std::runtime_error("MTP token id is out of range");
        check_hip(hipMemcpyAsync(static_cast<char*>(streams_dev_.data()) + r * width() * 2, streams[r]->data(),
                                 width() * 2, hipMemcpyDeviceToDevice, st),
                  "MTP streams");
    }
    check_hip(hipMemcpyAsync(tokens_dev_.data(), tokens.data(), rows * 4, hipMemcpyHostToDevice, st), "MTP tokens");
    check(q38_mtp_draft_greedy(head_, static_cast<const uint16_t*>(streams_dev_.data()),
                               static_cast<const uint32_t*>(tokens_dev_.data()), static_cast<int32_t>(rows),
                               static_cast<int32_t>(depth), static_cast<uint32_t*>(drafts_dev_.data()), nullptr,
                               ws_.data(), ws_.nbytes(), ctx_->stream()),
          "MTP draft chain");
    std::vector<std::uint32_t> flat(rows * depth);
    check_hip(hipMemcpyAsync(flat.data(), drafts_dev_.data(), flat.size() * 4, hipMemcpyDeviceToHost, st), "drafts");
    ctx_->synchronize();
    std::vector<std::vector<std::uint32_t>> out(rows);
    for (std::size_t r = 0; r < rows; ++r) out[r].assign(flat.begin() + r * depth, flat.begin() + (r + 1) * depth);
    return out;
}

std::vector<std::uint32_t> QwenMtpHead::draft_greedy(const DeviceTensor& stream, std::uint32_t current_token,
                                                     std::size_t query_position, std::size_t depth,
                                                     MtpDecodeState& state) const {
    MtpDecodeState next = state;
    advance(query_position, depth, next);
    const DeviceTensor* s[1] = {&stream};
    std::vector<std::uint32_t> d = draft_greedy_rows(s, std::span<const std::uint32_t>(&current_token, 1), depth).front();
    state = next;
    return d;
}

void QwenMtpHead::consume_decode(const DeviceTensor& stream, std::uint32_t next_token, std::size_t query_position,
                                 MtpDecodeState& state) const {
    if (stream.numel() != width()) throw std::runtime_error("MTP target stream must have shape [1,1,stream width] bf16");
    if (next_token >= vocab_) throw std::runtime_error("MTP token id is out of range");
    advance(query_position, 1, state);
}

namespace {
// finish_greedy_mtp_round (src/mtp_runner.cpp:213-340) on the verify path.
MtpRoundStep finish_head_round(const QwenModel& target, const QwenMtpHead& head, std::uint32_t current_token,
                               const DeviceTensor& previous_target_stream, std::size_t query_position,
                               std::vector<std::uint32_t> drafts, double draft_ms, MtpDecodeState head_origin,
                               ModelDecodeState& target_state, MtpDecodeState& head_state,
                               std::span<const std::uint32_t> stop_tokens) {
    if (drafts.size() < 2 || drafts.size() > 24)
        throw std::runtime_error("speculative proposal depth must be between 2 and 24");
    if (query_position != target_state.token_count())
        throw std::runtime_error("MTP query position must match target committed length");
    const auto t0 = std::chrono::steady_clock::now();
    head_state = std::move(head_origin);  // speculative head rows are never committed
    MtpTargetVerification verification =
        verify_mtp_target_layer_major_reference(target, current_token, drafts, target_state);
    const auto t1 = std::chrono::steady_clock::now();
    std::vector<std::uint32_t> target_rows;
    for (const MtpTargetVerifyRow& row : verification.rows) target_rows.push_back(row.greedy.token);
    const MtpGreedyDecision decision = decide_mtp_greedy(drafts, target_rows, stop_tokens);
    DeviceTensor next_stream = verification.rows[decision.correction_row].pre_mixer_stream.share();
    head.consume_decode(previous_target_stream, current_token, query_position, head_state);
    for (std::size_t i = 0; i < decision.accepted; ++i)
        head.consume_decode(verification.rows[i].pre_mixer_stream, drafts[i], query_position + i + 1, head_state);
    commit_mtp_target_verification(std::move(verification), decision.accepted, target_state);
    const std::size_t next_query_position = query_position + decision.accepted + 1;
    if (target_state.token_count() != next_query_position)
        throw std::runtime_error("MTP committed target length mismatch");
    const auto t2 = std::chrono::steady_clock::now();
    MtpRoundStep step;
    step.emitted_tokens.assign(drafts.begin(), drafts.begin() + static_cast<std::ptrdiff_t>(decision.accepted));
    step.emitted_tokens.push_back(decision.next_token);
    step.draft_tokens = std::move(drafts);
    step.accepted = decision.accepted;
    step.next_current_token = decision.next_token;
    step.next_query_position = next_query_position;
    step.next_target_stream = std::move(next_stream);
    step.draft_ms = draft_ms;
    step.verify_ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
    step.commit_ms = std::chrono::duration<double, std::milli>(t2 - t1).count();
    return step;
}
} // namespace

MtpRoundStep run_greedy_mtp_round_reference(const QwenModel& target, const QwenMtpHead& head,
                                            std::uint32_t current_token, const DeviceTensor& previous_target_stream,
                                            std::size_t query_position, std::size_t draft_depth,
                                            ModelDecodeState& target_state, MtpDecodeState& head_state,
                                            std::span<const std::uint32_t> stop_tokens) {
    if (draft_depth < 2 || draft_depth > 4) throw std::runtime_error("MTP draft depth must be between 2 and 4");
    MtpDecodeState head_origin = head.snapshot_state(head_state);
    const auto t0 = std::chrono::steady_clock::now();
    std::vector<std::uint32_t> drafts =
        head.draft_greedy(previous_target_stream, current_token, query_position, draft_depth, head_state);
    const double draft_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    return finish_head_round(target, head, current_token, previous_target_stream, query_position, std::move(drafts),
                             draft_ms, std::move(head_origin), target_state, head_state, stop_tokens);
}

MtpRoundStep run_greedy_external_draft_round_reference(const QwenModel& target, const QwenMtpHead& head,
                                                       std::uint32_t current_token,
                                                       const DeviceTensor& previous_target_stream,
                                                       std::size_t query_position, std::vector<std::uint32_t> drafts,
                                                       ModelDecodeState& target_state, MtpDecodeState& head_state,
                                                       std::span<const std::uint32_t> stop_tokens) {
    MtpDecodeState head_origin = head.snapshot_state(head_state);
    return finish_head_round(target, head, current_token, previous_target_stream, query_position, std::move(drafts),
                             0.0, std::move(head_origin), target_state, head_state, stop_tokens);
}

// ------------------------------------------------------------------ batched slots
QwenBatchVerifier::QwenBatchVerifier(const QwenModel& model, std::vector<ModelDecodeState*> slots)
    : model_(model), slots_(std::move(slots)) {
    for (ModelDecodeState* s : slots_)
        if (s == nullptr) throw std::runtime_error("batch verifier slot is null");
}

std::vector<std::vector<std::uint32_t>> QwenBatchVerifier::verify(std::span<const SlotVerifyRows> batch) {
    std::vector<std::uint32_t> tokens;
    for (const SlotVerifyRows& e : batch) {
        if (e.slot >= slots_.size()) throw std::runtime_error("batch verification names an unknown slot");
        tokens.push_back(e.current_token);
        tokens.insert(tokens.end(), e.drafts.begin(), e.drafts.end());
    }
    std::vector<GreedyStep> greedy;
    model_.forward_verify_layer_major(tokens, final_mixed_, greedy, nullptr, &pre_mixer_);
    const std::size_t H = model_.hidden();
    std::vector<std::vector<std::uint32_t>> out;
    out.reserve(batch.size());
    row_of_.assign(slots_.size(), SIZE_MAX);
    std::size_t row = 0;
    for (const SlotVerifyRows& e : batch) {
        row_of_[e.slot] = row;
        const std::size_t n = e.drafts.size() + 1;
        check(q38_slot_stage(slots_[e.slot]->slot(), static_cast<int32_t>(e.drafts.size()),
                             static_cast<const uint16_t*>(final_mixed_.data()) + row * H, model_.context().stream()),
              "batched verification checkpoints");
        std::vector<std::uint32_t> t(n);
        for (std::size_t i = 0; i < n; ++i) t[i] = greedy[row + i].token;
        out.push_back(std::move(t));
        row += n;
    }
    return out;
}

void QwenBatchVerifier::commit(std::size_t slot, std::size_t accepted) {
    if (slot >= slots_.size() || slot >= row_of_.size() || row_of_[slot] == SIZE_MAX)
        throw std::runtime_error("commit names a slot outside the last verification");
    check(q38_slot_commit(slots_[slot]->slot(), static_cast<int64_t>(accepted), model_.context().stream()), "commit");
    const std::size_t H = model_.hidden();
    if (committed_.size() < slots_.size()) committed_.resize(slots_.size());
    if (committed_[slot].empty()) committed_[slot] = DeviceTensor({1, 1, H}, DType::bf16);
    check_hip(hipMemcpyAsync(committed_[slot].data(),
                             static_cast<const char*>(pre_mixer_.data()) + (row_of_[slot] + accepted) * H * 2, H * 2,
                             hipMemcpyDeviceToDevice, static_cast<hipStream_t>(model_.context().stream())),
              "committed stream row");
}

const DeviceTensor& QwenBatchVerifier::committed_stream(std::size_t slot) const {
    static const DeviceTensor none;
    return slot < committed_.size() ? committed_[slot] : none;
}

std::vector<std::uint32_t> MtpHeadDrafter::propose(std::size_t slot, std::uint32_t current_token, std::size_t depth) {
    const DraftRequest r{slot, current_token, depth};
    return propose_batch(std::span<const DraftRequest>(&r, 1)).front();
}

std::vector<std::vector<std::uint32_t>> MtpHeadDrafter::propose_batch(std::span<const DraftRequest> requests) {
    std::vector<std::vector<std::uint32_t>> out(requests.size());
    std::vector<std::size_t> ready;  // requests whose slot has a committed stream
    for (std::size_t i = 0; i < requests.size(); ++i)
        if (requests[i].depth > 0 && !verifier_.committed_stream(requests[i].slot).empty()) ready.push_back(i);
    for (std::size_t first = 0; first < ready.size(); first += 4) {
        const std::size_t n = std::min<std::size_t>(4, ready.size() - first);
        std::vector<const DeviceTensor*> streams;
        std::vector<std::uint32_t> tokens;
        std::size_t depth = 0;
        for (std::size_t j = 0; j < n; ++j) {
            const DraftRequest& r = requests[ready[first + j]];
            streams.push_back(&verifier_.committed_stream(r.slot));
            tokens.push_back(r.current_token);
            depth = std::max(depth, r.depth);
        }
        std::vector<std::vector<std::uint32_t>> d = head_.draft_greedy_rows(streams, tokens, depth);
        for (std::size_t j = 0; j < n; ++j) {
            std::vector<std::uint32_t>& v = d[j];
            v.resize(std::min(v.size(), requests[ready[first + j]].depth));
            out[ready[first + j]] = std::move(v);
        }
    }
    return out;
}

} // namespace qwen38
