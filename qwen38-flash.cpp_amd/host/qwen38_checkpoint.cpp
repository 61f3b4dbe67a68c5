// qwen38_checkpoint.cpp — on-disk VQ checkpoint reader (host) and its C ABI entry points
// q38_checkpoint_inspect / q38_moe_layer_load.
#include "qwen38_checkpoint.hpp"

#include "q38_private.h"

#include <hip/hip_runtime.h>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <sstream>
#include <stdexcept>

namespace qwen38 {

// ------------------------------------------------------------------ JSON
class JsonParser {
public:
    explicit JsonParser(std::string_view t) : t_(t) {}
    Json document() {
        Json v = value(0);
        skip();
        if (i_ != t_.size()) fail("trailing characters");
        return v;
    }

private:
    [[noreturn]] void fail(const char* what) const {
        throw std::runtime_error(std::string("invalid JSON (") + what + ") at offset " + std::to_string(i_));
    }
    void skip() {
        while (i_ < t_.size() && (t_[i_] == ' ' || t_[i_] == '\n' || t_[i_] == '\r' || t_[i_] == '\t')) ++i_;
    }
    bool eat(char c) {
        skip();
        if (i_ < t_.size() && t_[i_] == c) {
            ++i_;
            return true;
        }
        return false;
    }
    void expect(char c) {
        if (!eat(c)) fail("unexpected character");
    }
    void word(std::string_view w) {
        if (t_.substr(i_, w.size()) != w) fail("bad literal");
        i_ += w.size();
    }
    static void utf8(std::string& out, std::uint32_t cp) {
        if (cp < 0x80) {
            out += static_cast<char>(cp);
        } else if (cp < 0x800) {
            out += static_cast<char>(0xC0 | (cp >> 6));
            out += static_cast<char>(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            out += static_cast<char>(0xE0 | (cp >> 12));
            out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
            out += static_cast<char>(0x80 | (cp & 0x3F));
        } else {
            out += static_cast<char>(0xF0 | (cp >> 18));
            out += static_cast<char>(0x80 | ((cp >> 12) & 0x3F));
            out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
            out += static_cast<char>(0x80 | (cp & 0x3F));
        }
    }
    std::uint32_t hex4() {
        if (i_ + 4 > t_.size()) fail("short escape");
        std::uint32_t v = 0;
        for (int k = 0; k < 4; ++k) {
            const char c = t_[i_++];
            v <<= 4;
            if (c >= '0' && c <= '9') v |= static_cast<std::uint32_t>(c - '0');
            else if (c >= 'a' && c <= 'f') v |= static_cast<std::uint32_t>(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= static_cast<std::uint32_t>(c - 'A' + 10);
            else fail("bad escape");
        }
        return v;
    }
    std::string string() {
        expect('"');
        std::string out;
        while (true) {
            if (i_ >= t_.size()) fail("unterminated string");
            const char c = t_[i_++];
            if (c == '"') return out;
            if (static_cast<unsigned char>(c) < 0x20) fail("control character in string");
            if (c != '\\') {
                out += c;
                continue;
            }
            if (i_ >= t_.size()) fail("unterminated escape");
            const char e = t_[i_++];
            switch (e) {
            case '"': out += '"'; break;
            case '\\': out += '\\'; break;
            case '/': out += '/'; break;
            case 'b': out += '\b'; break;
            case 'f': out += '\f'; break;
            case 'n': out += '\n'; break;
            case 'r': out += '\r'; break;
            case 't': out += '\t'; break;
            case 'u': {
                std::uint32_t cp = hex4();
                if (cp >= 0xD800 && cp < 0xDC00 && t_.substr(i_, 2) == "\\u") {
                    i_ += 2;
                    const std::uint32_t lo = hex4();
                    if (lo < 0xDC00 || lo >= 0xE000) fail("bad surrogate pair");
                    cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                }
                utf8(out, cp);
                break;
            }
            default: fail("bad escape");
            }
        }
    }
    Json number() {
        const std::size_t b = i_;
        if (i_ < t_.size() && t_[i_] == '-') ++i_;
        bool integral = true;
        while (i_ < t_.size() && std::isdigit(static_cast<unsigned char>(t_[i_]))) ++i_;
        if (i_ < t_.size() && t_[i_] == '.') {
            integral = false;
            ++i_;
            while (i_ < t_.size() && std::isdigit(static_cast<unsigned char>(t_[i_]))) ++i_;
        }
        if (i_ < t_.size() && (t_[i_] == 'e' || t_[i_] == 'E')) {
            integral = false;
            ++i_;
            if (i_ < t_.size() && (t_[i_] == '+' || t_[i_] == '-')) ++i_;
            while (i_ < t_.size() && std::isdigit(static_cast<unsigned char>(t_[i_]))) ++i_;
        }
        const std::string s(t_.substr(b, i_ - b));
        if (s.empty() || s == "-") fail("bad number");
        Json j;
        j.v_ = Json::Number{std::strtod(s.c_str(), nullptr), integral};
        return j;
    }
    Json value(int depth) {
        if (depth > 256) fail("nesting too deep");
        skip();
        if (i_ >= t_.size()) fail("unexpected end");
        const char c = t_[i_];
        Json j;
        if (c == '{') {
            ++i_;
            Json::Object o;
            if (!eat('}')) {
                do {
                    skip();
                    std::string k = string();
                    expect(':');
                    o.insert_or_assign(std::move(k), value(depth + 1));
                } while (eat(','));
                expect('}');
            }
            j.v_ = std::move(o);
        } else if (c == '[') {
            ++i_;
            Json::Array a;
            if (!eat(']')) {
                do a.push_back(value(depth + 1));
                while (eat(','));
                expect(']');
            }
            j.v_ = std::move(a);
        } else if (c == '"') {
            j.v_ = string();
        } else if (c == 't') {
            word("true");
            j.v_ = true;
        } else if (c == 'f') {
            word("false");
            j.v_ = false;
        } else if (c == 'n') {
            word("null");
        } else {
            return number();
        }
        return j;
    }
    std::string_view t_;
    std::size_t i_ = 0;
};

Json Json::parse(std::string_view text) { return JsonParser(text).document(); }

const Json* Json::find(std::string_view key) const {
    if (!is_object()) return nullptr;
    const Object& o = std::get<Object>(v_);
    const auto it = o.find(key);
    return it == o.end() ? nullptr : &it->second;
}
const Json& Json::at(std::string_view key) const {
    const Json* j = find(key);
    if (!j) throw std::runtime_error("missing JSON key " + std::string(key));
    return *j;
}
const Json::Object& Json::as_object() const {
    if (!is_object()) throw std::runtime_error("JSON value is not an object");
    return std::get<Object>(v_);
}
const Json::Array& Json::as_array() const {
    if (!is_array()) throw std::runtime_error("JSON value is not an array");
    return std::get<Array>(v_);
}
const std::string& Json::as_string() const {
    if (!is_string()) throw std::runtime_error("JSON value is not a string");
    return std::get<std::string>(v_);
}
double Json::as_number() const {
    if (!is_number()) throw std::runtime_error("JSON value is not a number");
    return std::get<Number>(v_).value;
}
bool Json::as_bool() const {
    if (!is_bool()) throw std::runtime_error("JSON value is not a boolean");
    return std::get<bool>(v_);
}
std::uint64_t Json::as_size(std::string_view what) const {
    if (!is_number()) throw std::runtime_error(std::string(what) + " must be a number");
    const Number n = std::get<Number>(v_);
    if (!n.integral || n.value < 0.0 || n.value > 9007199254740992.0)
        throw std::runtime_error(std::string(what) + " must be a non-negative integer");
    return static_cast<std::uint64_t>(n.value);
}

// ------------------------------------------------------------------ manifest
namespace {
std::string read_file(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("cannot open " + path);
    std::ostringstream s;
    s << f.rdbuf();
    return s.str();
}
} // namespace

ModelManifest ModelManifest::load(const std::string& directory) {
    return parse(read_file((std::filesystem::path(directory) / "config.json").string()));
}

ModelManifest ModelManifest::parse(std::string_view config_json) {
    const Json root = Json::parse(config_json);
    if (!root.is_object()) throw std::runtime_error("model config must be a JSON object");
    const Json* text = root.find("text_config");
    const Json& cfg = text ? *text : root;
    ModelManifest m;
    m.expert_count_ = cfg.at("num_experts").as_size("num_experts");
    m.experts_per_token_ = cfg.at("num_experts_per_tok").as_size("num_experts_per_tok");
    if (const Json* n = cfg.find("norm_topk_prob")) m.normalize_ = n->as_bool();
    if (const Json* n = cfg.find("shared_expert_intermediate_size"))
        m.shared_inter_ = n->as_size("shared_expert_intermediate_size");
    // quantization metadata (src/model_manifest.cpp:188-208): model-wide bits and group_size,
    // and per-module objects {bits, group_size} with bits 2..8.
    const Json* quantization = root.find("quantization");
    if (!quantization) quantization = root.find("quantization_config");
    if (quantization) {
        m.has_quantization_ = true;
        m.quantization_.bits = quantization->at("bits").as_size("quantization.bits");
        m.quantization_.group_size = quantization->at("group_size").as_size("quantization.group_size");
        for (const auto& [module, value] : quantization->as_object()) {
            if (!value.is_object()) continue;
            const Json* bits = value.find("bits");
            const Json* group = value.find("group_size");
            if (!bits || !group) continue;
            const QuantizationSpec spec{bits->as_size("quantization override bits"),
                                        group->as_size("quantization override group_size")};
            if (spec.bits < 2 || spec.bits > 8 || spec.group_size == 0)
                throw std::runtime_error("invalid quantization override for " + module);
            m.quantization_overrides_.emplace(module, spec);
        }
    }
    // vq_modules (src/model_manifest.cpp:210-230): every module must describe the model's
    // expert count, a non-empty geometry whose input splits into whole vectors and scale
    // groups, and packed codes of at most 31 bits.
    if (const Json* modules = root.find("vq_modules")) {
        for (const auto& [module, value] : modules->as_object()) {
            VectorQuantizationSpec s;
            s.expert_count = value.at("experts").as_size("vq_modules.experts");
            s.output_dimension = value.at("out").as_size("vq_modules.out");
            s.input_dimension = value.at("in").as_size("vq_modules.in");
            s.codebook_size = value.at("k").as_size("vq_modules.k");
            s.vector_dimension = value.at("dim").as_size("vq_modules.dim");
            s.group_size = value.at("group").as_size("vq_modules.group");
            if (const Json* pb = value.find("pack_bits"); pb && !pb->is_null())  // absent / null: byte codes
                s.packed_bits = pb->as_size("vq_modules.pack_bits");
            if (s.expert_count != m.expert_count_ ||
                s.output_dimension == 0 || s.input_dimension == 0 || s.codebook_size < 2 ||
                s.vector_dimension == 0 || s.group_size == 0 || s.input_dimension % s.vector_dimension != 0 ||
                s.input_dimension % s.group_size != 0 || (s.packed_bits != 0 && s.packed_bits > 31))
                throw std::runtime_error("unsupported vector quantization geometry for " + module);
            m.vq_.emplace(module, s);
        }
    }
    return m;
}

namespace {
constexpr std::string_view kWrapper = "language_model.";
// The name without the "language_model." wrapper, or empty when it has none.
std::string_view flat_name(std::string_view name) {
    return name.substr(0, kWrapper.size()) == kWrapper ? name.substr(kWrapper.size()) : std::string_view{};
}
} // namespace

const VectorQuantizationSpec* ModelManifest::vector_quantization_for(std::string_view module) const {
    auto it = vq_.find(module);
    if (it == vq_.end() && !flat_name(module).empty()) it = vq_.find(flat_name(module));
    return it == vq_.end() ? nullptr : &it->second;
}

QuantizationSpec ModelManifest::quantization_for(std::string_view module) const {
    if (!has_quantization_) throw std::runtime_error("model is missing quantization metadata");
    auto it = quantization_overrides_.find(module);
    if (it == quantization_overrides_.end() && !flat_name(module).empty())
        it = quantization_overrides_.find(flat_name(module));
    return it == quantization_overrides_.end() ? quantization_ : it->second;
}

// ------------------------------------------------------------------ safetensors
struct TensorStore::Mapping {
    void* base = MAP_FAILED;
    std::size_t size = 0;
    ~Mapping() {
        if (base != MAP_FAILED) munmap(base, size);
    }
};

namespace {
std::size_t dtype_bytes(const std::string& d) {
    if (d == "U8" || d == "I8" || d == "BOOL" || d == "F8_E4M3" || d == "F8_E5M2") return 1;
    if (d == "U16" || d == "I16" || d == "F16" || d == "BF16") return 2;
    if (d == "U32" || d == "I32" || d == "F32") return 4;
    if (d == "U64" || d == "I64" || d == "F64") return 8;
    throw std::runtime_error("unknown safetensors dtype " + d);
}
} // namespace

void TensorStore::map_file(const std::string& path) {
    const int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) throw std::runtime_error("cannot open " + path);
    struct stat st {};
    if (::fstat(fd, &st) != 0) {
        ::close(fd);
        throw std::runtime_error("cannot stat " + path);
    }
    auto m = std::make_unique<Mapping>();
    m->size = static_cast<std::size_t>(st.st_size);
    if (m->size < 8) {
        ::close(fd);
        throw std::runtime_error("safetensors file too short: " + path);
    }
    m->base = ::mmap(nullptr, m->size, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (m->base == MAP_FAILED) throw std::runtime_error("cannot map " + path);
    const auto* bytes = static_cast<const unsigned char*>(m->base);
    std::uint64_t hlen = 0;
    for (int i = 0; i < 8; ++i) hlen |= static_cast<std::uint64_t>(bytes[i]) << (8 * i);
    if (hlen > m->size - 8) throw std::runtime_error("safetensors header exceeds the file: " + path);
    const Json header = Json::parse(std::string_view(reinterpret_cast<const char*>(bytes + 8), hlen));
    const std::size_t data0 = 8 + static_cast<std::size_t>(hlen), data_size = m->size - data0;
    for (const auto& [name, spec] : header.as_object()) {
        if (name == "__metadata__") continue;
        TensorView t;
        t.dtype = spec.at("dtype").as_string();
        std::size_t numel = 1;
        for (const Json& d : spec.at("shape").as_array()) {
            const std::uint64_t v = d.as_size("safetensors shape");
            t.shape.push_back(static_cast<std::int64_t>(v));
            if (v != 0 && numel > SIZE_MAX / v) throw std::runtime_error("safetensors shape overflows: " + name);
            numel *= v;
        }
        const Json::Array& off = spec.at("data_offsets").as_array();
        if (off.size() != 2) throw std::runtime_error("safetensors data_offsets must have two entries: " + name);
        const std::uint64_t b = off[0].as_size("data_offsets"), e = off[1].as_size("data_offsets");
        if (b > e || e > data_size) throw std::runtime_error("safetensors tensor outside the file: " + name);
        if (e - b != numel * dtype_bytes(t.dtype)) throw std::runtime_error("safetensors size mismatch: " + name);
        t.data = bytes + data0 + b;
        t.nbytes = static_cast<std::size_t>(e - b);
        if (!tensors_.emplace(name, std::move(t)).second) throw std::runtime_error("duplicate tensor " + name);
    }
    files_.push_back(std::move(m));
}

TensorStore::TensorStore(const std::string& directory) : manifest_(ModelManifest::load(directory)) {
    namespace fs = std::filesystem;
    const fs::path dir(directory);
    std::vector<std::string> files;
    if (fs::exists(dir / "model.safetensors.index.json")) {
        const Json index = Json::parse(read_file((dir / "model.safetensors.index.json").string()));
        for (const auto& [name, file] : index.at("weight_map").as_object()) {
            const std::string f = file.as_string();
            if (f.find('/') != std::string::npos || f.find("..") != std::string::npos)
                throw std::runtime_error("weight_map names a file outside the checkpoint: " + f);
            if (std::find(files.begin(), files.end(), f) == files.end()) files.push_back(f);
        }
    } else {
        for (const auto& e : fs::directory_iterator(dir))
            if (e.is_regular_file() && e.path().extension() == ".safetensors")
                files.push_back(e.path().filename().string());
        std::sort(files.begin(), files.end());
    }
    if (files.empty()) throw std::runtime_error("no safetensors files in " + directory);
    for (const std::string& f : files) map_file((dir / f).string());
}
TensorStore::~TensorStore() = default;

bool TensorStore::has(std::string_view name) const {
    return tensors_.find(name) != tensors_.end() ||
           (!flat_name(name).empty() && tensors_.find(flat_name(name)) != tensors_.end());
}

const TensorView& TensorStore::tensor(std::string_view name) const {
    auto it = tensors_.find(name);
    if (it == tensors_.end() && !flat_name(name).empty()) it = tensors_.find(flat_name(name));
    if (it == tensors_.end()) throw std::runtime_error("missing tensor " + std::string(name));
    return it->second;
}

// ------------------------------------------------------------------ affine projections
// infer_affine_quantization_bits (src/quantization_geometry.cpp:9-35) on the last dimensions.
static std::size_t infer_affine_bits(const TensorView& weight, const TensorView& scales, std::size_t group,
                                     const std::string& label) {
    if (weight.shape.empty() || weight.shape.size() != scales.shape.size() || weight.shape.back() <= 0 ||
        scales.shape.back() <= 0 || group == 0)
        throw std::runtime_error("cannot infer " + label + " quantization geometry");
    const auto packed = static_cast<std::size_t>(weight.shape.back());
    const auto width = static_cast<std::size_t>(scales.shape.back()) * group;
    if (width == 0 || packed * 32 % width != 0) throw std::runtime_error("non-integral " + label + " quantization bits");
    const std::size_t bits = packed * 32 / width;
    if (bits != 2 && bits != 3 && bits != 4 && bits != 5 && bits != 6 && bits != 8)
        throw std::runtime_error(label + " projections must use affine Q2, Q3, Q4, Q5, Q6, or Q8");
    return bits;
}

AffineProjectionTensors load_affine_projection(const TensorStore& store, std::string_view name) {
    const std::string base(name);
    AffineProjectionTensors p;
    p.weight = &store.tensor(base + ".weight");
    p.scales = &store.tensor(base + ".scales");
    p.biases = &store.tensor(base + ".biases");
    const QuantizationSpec q = store.manifest().quantization_for(base);
    p.group_size = q.group_size;
    p.bits = infer_affine_bits(*p.weight, *p.scales, q.group_size, "MoE");
    // (src/sparse_moe.cpp:668-671; MTP-head modules may differ from the metadata)
    if (p.bits != q.bits && base.find("language_model.mtp.") != 0)
        throw std::runtime_error("MoE tensor disagrees with quantization metadata for " + base);
    if (p.weight->dtype != "U32" || p.weight->shape.size() != 2 || p.scales->shape != p.biases->shape ||
        p.scales->shape.size() != 2 || p.scales->shape[0] != p.weight->shape[0] ||
        (p.scales->dtype != "BF16" && p.scales->dtype != "F16") || p.biases->dtype != p.scales->dtype)
        throw std::runtime_error("invalid affine quantization tensors for " + base);
    p.out = static_cast<std::size_t>(p.weight->shape[0]);
    p.in = static_cast<std::size_t>(p.scales->shape[1]) * p.group_size;
    return p;
}

// ------------------------------------------------------------------ VQ projections
VqProjectionTensors load_vq_projection(const TensorStore& store, std::string_view name) {
    const std::string base(name);
    const VectorQuantizationSpec* vq = store.manifest().vector_quantization_for(base);
    if (!vq) throw std::runtime_error("no vq_modules entry for " + base);
    VqProjectionTensors p;
    p.spec = *vq;
    p.codes = &store.tensor(base + ".codes");
    p.codebook = &store.tensor(base + ".codebook");
    p.scales = &store.tensor(base + ".vq_scales");
    // the tensor contract of SparseMoe::load_projection (src/sparse_moe.cpp:618-661)
    const std::int64_t subvectors = static_cast<std::int64_t>(vq->input_dimension / vq->vector_dimension);
    const std::int64_t width =
        vq->packed_bits == 0 ? subvectors
                             : ((subvectors + 31) / 32) * static_cast<std::int64_t>(vq->packed_bits);
    const auto E = static_cast<std::int64_t>(vq->expert_count), O = static_cast<std::int64_t>(vq->output_dimension);
    if (p.codes->shape != std::vector<std::int64_t>{E, O, width} ||
        p.codebook->shape != std::vector<std::int64_t>{static_cast<std::int64_t>(vq->codebook_size),
                                                       static_cast<std::int64_t>(vq->vector_dimension)} ||
        p.scales->shape !=
            std::vector<std::int64_t>{E, O, static_cast<std::int64_t>(vq->input_dimension / vq->group_size)} ||
        (vq->packed_bits == 0 && p.codes->dtype != "U8") || (vq->packed_bits != 0 && p.codes->dtype != "U32") ||
        p.codebook->dtype != "F16" || p.scales->dtype != "F16")
        throw std::runtime_error("invalid vector quantization tensors for " + base);
    return p;
}

q38_moe_desc checkpoint_layer_desc(const TensorStore& store, std::string_view prefix, std::size_t experts_per_token,
                                   bool normalize) {
    const std::string pre(prefix);
    const VqProjectionTensors g = load_vq_projection(store, pre + ".switch_mlp.gate_proj");
    const VqProjectionTensors u = load_vq_projection(store, pre + ".switch_mlp.up_proj");
    const VqProjectionTensors d = load_vq_projection(store, pre + ".switch_mlp.down_proj");
    const auto bits = [](const VectorQuantizationSpec& s) { return s.packed_bits == 0 ? std::size_t{8} : s.packed_bits; };
    if (g.spec.input_dimension != u.spec.input_dimension || g.spec.output_dimension != u.spec.output_dimension ||
        g.spec.vector_dimension != u.spec.vector_dimension || bits(g.spec) != bits(u.spec) ||
        g.spec.group_size != u.spec.group_size || g.spec.codebook_size != u.spec.codebook_size)
        throw std::runtime_error("gate and up projections of " + pre + " differ in geometry");
    if (d.spec.input_dimension != g.spec.output_dimension || d.spec.output_dimension != g.spec.input_dimension)
        throw std::runtime_error("down projection of " + pre + " does not invert the gate/up shape");
    for (const VqProjectionTensors* p : {&g, &d})
        if (p->spec.codebook_size > (std::size_t{1} << bits(p->spec)))
            throw std::runtime_error("codebook of " + pre + " has more entries than its codes address");
    const TensorView& router = store.tensor(pre + ".gate.weight");
    const auto H = static_cast<std::int64_t>(g.spec.input_dimension);
    if (router.dtype != "BF16" || router.shape != std::vector<std::int64_t>{
                                                     static_cast<std::int64_t>(store.manifest().expert_count()), H})
        throw std::runtime_error("router " + pre + ".gate.weight must be BF16 [experts, hidden]");
    q38_moe_desc desc{};
    desc.hidden = static_cast<int32_t>(g.spec.input_dimension);
    desc.inter = static_cast<int32_t>(g.spec.output_dimension);
    desc.experts = static_cast<int32_t>(store.manifest().expert_count());
    desc.top_k = static_cast<int32_t>(experts_per_token);
    desc.gu_dim = static_cast<int32_t>(g.spec.vector_dimension);
    desc.gu_bits = static_cast<int32_t>(bits(g.spec));
    desc.down_dim = static_cast<int32_t>(d.spec.vector_dimension);
    desc.down_bits = static_cast<int32_t>(bits(d.spec));
    desc.gu_group = static_cast<int32_t>(g.spec.group_size);
    desc.down_group = static_cast<int32_t>(d.spec.group_size);
    desc.normalize_topk = normalize ? 1 : 0;
    // The shared expert: SparseMoe::forward_shared applies it with quantized_matmul, so the
    // reference reads it in MLX affine form only (the VQ branch of load_projection would need a
    // vq_modules entry for all routed experts).
    if (store.manifest().vector_quantization_for(pre + ".shared_expert.gate_proj"))
        throw std::runtime_error("shared expert of " + pre + " is VQ-coded; shared experts load in affine form");
    const bool any_shared = store.has(pre + ".shared_expert_gate.weight") ||
                            store.has(pre + ".shared_expert.gate_proj.weight");
    if (any_shared) (void)checkpoint_shared_expert(store, pre, g.spec.input_dimension);  // (its checks)
    desc.has_shared = any_shared ? 1 : 0;
    return desc;
}

SharedExpertTensors checkpoint_shared_expert(const TensorStore& store, std::string_view prefix, std::size_t hidden) {
    const std::string pre(prefix);
    SharedExpertTensors s;
    const char* names[3] = {".gate_proj", ".up_proj", ".down_proj"};
    for (int p = 0; p < 3; ++p) s.proj[p] = load_affine_projection(store, pre + ".shared_expert" + names[p]);
    const std::size_t Is = s.proj[0].out;
    if (s.proj[0].in != hidden || s.proj[1].in != hidden || s.proj[1].out != Is || s.proj[2].in != Is ||
        s.proj[2].out != hidden)
        throw std::runtime_error("shared expert of " + pre + ": gate/up [inter, hidden] and down [hidden, inter]");
    for (int p = 1; p < 3; ++p)
        if (s.proj[p].bits != s.proj[0].bits || s.proj[p].group_size != s.proj[0].group_size ||
            s.proj[p].scales->dtype != s.proj[0].scales->dtype)
            throw std::runtime_error("shared expert of " + pre + ": the device kernels take one bits, group size "
                                     "and scale dtype for its three projections");
    const std::size_t cfg = store.manifest().shared_expert_intermediate_size();
    if (cfg != 0 && cfg != Is)
        throw std::runtime_error("shared expert of " + pre + " disagrees with shared_expert_intermediate_size");
    s.gate = &store.tensor(pre + ".shared_expert_gate.weight");
    if (s.gate->dtype != "BF16" || s.gate->nbytes != hidden * 2)
        throw std::runtime_error("shared expert gate of " + pre + " must be BF16 [1, hidden]");
    return s;
}

} // namespace qwen38

// ====================================================================== C ABI
namespace {
thread_local std::string g_ck_error;
int ck_fail(int code, const std::string& msg) {
    g_ck_error = msg;
    q38_private_set_error(msg.c_str());
    return code;
}

// Codes of one projection into the packed q38 layout [rows, words]: U32 words as they are;
// byte codes into 8-bit words (32-code blocks of 8 words, lowest byte first).
std::vector<std::uint32_t> packed_codes(const qwen38::VqProjectionTensors& p, std::int64_t rows, int words) {
    std::vector<std::uint32_t> out(static_cast<std::size_t>(rows) * words, 0u);
    if (p.spec.packed_bits != 0) {
        std::memcpy(out.data(), p.codes->data, std::min(out.size() * 4, p.codes->nbytes));
        return out;
    }
    const auto n = static_cast<std::int64_t>(p.spec.input_dimension / p.spec.vector_dimension);
    const auto* src = static_cast<const std::uint8_t*>(p.codes->data);
    auto* dst = reinterpret_cast<std::uint8_t*>(out.data());
    for (std::int64_t r = 0; r < rows; ++r) std::memcpy(dst + r * words * 4, src + r * n, static_cast<std::size_t>(n));
    return out;
}
} // namespace

extern "C" int q38_checkpoint_inspect(const char* checkpoint, const char* prefix, q38_moe_desc* desc) {
    if (!checkpoint || !prefix || !desc) return ck_fail(Q38_EINVAL, "q38_checkpoint_inspect: null argument");
    try {
        qwen38::TensorStore store(checkpoint);
        *desc = qwen38::checkpoint_layer_desc(store, prefix, store.manifest().experts_per_token(),
                                              store.manifest().normalize_topk_probability());
        return Q38_OK;
    } catch (const std::exception& e) {
        return ck_fail(Q38_EINVAL, e.what());
    }
}

extern "C" int q38_moe_layer_load(q38_ctx* ctx, const char* checkpoint, const char* prefix, int32_t book_format,
                                  q38_moe_layer** out) {
    if (!ctx || !checkpoint || !prefix || !out) return ck_fail(Q38_EINVAL, "q38_moe_layer_load: null argument");
    try {
        qwen38::TensorStore store(checkpoint);
        const std::string pre(prefix);
        q38_moe_desc d = qwen38::checkpoint_layer_desc(store, pre, store.manifest().experts_per_token(),
                                                       store.manifest().normalize_topk_probability());
        d.book_format = book_format;
        const char* names[3] = {".gate_proj", ".up_proj", ".down_proj"};
        qwen38::VqProjectionTensors routed[3];
        for (int p = 0; p < 3; ++p) routed[p] = qwen38::load_vq_projection(store, pre + ".switch_mlp" + names[p]);
        qwen38::SharedExpertTensors shared;
        if (d.has_shared) shared = qwen38::checkpoint_shared_expert(store, pre, static_cast<std::size_t>(d.hidden));
        const int E = d.experts;
        const int dims[3] = {d.gu_dim, d.gu_dim, d.down_dim}, bits[3] = {d.gu_bits, d.gu_bits, d.down_bits};
        const int ins[3] = {d.hidden, d.hidden, d.inter}, outs[3] = {d.inter, d.inter, d.hidden};
        const int grps[3] = {d.gu_group, d.gu_group, d.down_group};
        // one device block: router, shared gate, per projection codes, scales, book, then the
        // affine shared expert's weights, scales and biases
        auto a256 = [](std::size_t v) { return (v + 255) / 256 * 256; };
        std::size_t off = 0, o_router = off;
        off += a256(static_cast<std::size_t>(E) * d.hidden * 2);
        const std::size_t o_wsg = off;
        off += a256(static_cast<std::size_t>(d.hidden) * 2);
        std::size_t o_codes[3], o_scales[3], o_book[3], words[3], o_sw[3] = {}, o_ss[3] = {}, o_sb[3] = {};
        for (int p = 0; p < 3; ++p) {
            words[p] = static_cast<std::size_t>(((ins[p] / dims[p] + 31) / 32) * bits[p]);
            o_codes[p] = off;
            off += a256(static_cast<std::size_t>(E) * outs[p] * words[p] * 4);
            o_scales[p] = off;
            off += a256(static_cast<std::size_t>(E) * outs[p] * (ins[p] / grps[p]) * 2);
            o_book[p] = off;
            off += a256((std::size_t{1} << bits[p]) * dims[p] * 2);
        }
        if (d.has_shared)
            for (int p = 0; p < 3; ++p) {
                o_sw[p] = off;
                off += a256(shared.proj[p].weight->nbytes);
                o_ss[p] = off;
                off += a256(shared.proj[p].scales->nbytes);
                o_sb[p] = off;
                off += a256(shared.proj[p].biases->nbytes);
            }
        char* base = nullptr;
        if (hipMalloc(&base, off) != hipSuccess) return ck_fail(Q38_ENOMEM, "hipMalloc failed for checkpoint tensors");
        auto up = [&](std::size_t o, const void* src, std::size_t n) {
            if (hipMemcpy(base + o, src, n, hipMemcpyHostToDevice) != hipSuccess)
                throw std::runtime_error("upload of checkpoint tensors failed");
        };
        try {
            if (hipMemset(base, 0, off) != hipSuccess) throw std::runtime_error("clearing checkpoint tensors failed");
            up(o_router, store.tensor(pre + ".gate.weight").data, static_cast<std::size_t>(E) * d.hidden * 2);
            for (int p = 0; p < 3; ++p) {
                const std::int64_t rows = static_cast<std::int64_t>(E) * outs[p];
                const std::vector<std::uint32_t> c = packed_codes(routed[p], rows, static_cast<int>(words[p]));
                up(o_codes[p], c.data(), c.size() * 4);
                up(o_scales[p], routed[p].scales->data, routed[p].scales->nbytes);
                up(o_book[p], routed[p].codebook->data, routed[p].codebook->nbytes);  // unused entries stay 0
            }
            q38_moe_weights w{};
            w.router = reinterpret_cast<const uint16_t*>(base + o_router);
            for (int p = 0; p < 3; ++p) {
                w.codes[p] = reinterpret_cast<const uint32_t*>(base + o_codes[p]);
                w.scales[p] = reinterpret_cast<const uint16_t*>(base + o_scales[p]);
                w.books[p] = reinterpret_cast<const uint16_t*>(base + o_book[p]);
            }
            q38_moe_layer* layer = nullptr;
            int rc = Q38_OK;
            if (d.has_shared) {
                up(o_wsg, shared.gate->data, shared.gate->nbytes);
                w.shared_gate = reinterpret_cast<const uint16_t*>(base + o_wsg);
                q38_affine_shared a{};
                for (int p = 0; p < 3; ++p) {
                    up(o_sw[p], shared.proj[p].weight->data, shared.proj[p].weight->nbytes);
                    up(o_ss[p], shared.proj[p].scales->data, shared.proj[p].scales->nbytes);
                    up(o_sb[p], shared.proj[p].biases->data, shared.proj[p].biases->nbytes);
                    a.weight[p] = reinterpret_cast<const uint32_t*>(base + o_sw[p]);
                    a.scales[p] = reinterpret_cast<const uint16_t*>(base + o_ss[p]);
                    a.biases[p] = reinterpret_cast<const uint16_t*>(base + o_sb[p]);
                }
                a.bits = static_cast<int32_t>(shared.proj[0].bits);
                a.group = static_cast<int32_t>(shared.proj[0].group_size);
                a.inter = static_cast<int32_t>(shared.proj[0].out);
                a.scale_dtype = shared.proj[0].scales->dtype == "F16" ? 1 : 0;
                rc = q38_moe_layer_create_affine_shared(ctx, &d, &w, &a, &layer);
            } else {
                rc = q38_moe_layer_create(ctx, &d, &w, &layer);
            }
            if (rc) {
                (void)hipFree(base);
                return rc;  // the create call set the message
            }
            q38_private_layer_adopt(layer, base);
            *out = layer;
            return Q38_OK;
        } catch (...) {
            (void)hipFree(base);
            throw;
        }
    } catch (const std::exception& e) {
        return ck_fail(Q38_EINVAL, e.what());
    }
}

