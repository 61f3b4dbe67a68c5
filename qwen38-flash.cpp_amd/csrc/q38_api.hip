// q38_api.hip — the C ABI (include/q38.h): handle lifetime, validation, workspace
// carving and kernel launches. No exception crosses the ABI; every failure returns a
// Q38_E* code and leaves outputs untouched.
#include "q38.h"

#include <cmath>

#include "q38_device.hpp"
#include "q38_internal.hpp"
#include "q38_private.h"

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

using namespace q38;

namespace {

thread_local std::string g_error;

int fail(int code, const std::string& msg) {
    g_error = msg;
    return code;
}
int hip_fail(hipError_t e, const char* where) {
    g_error = std::string(where) + ": " + hipGetErrorString(e);
    return Q38_EHIP;
}
#define Q38_HIP(expr)                                   \
    do {                                                \
        const hipError_t e_ = (expr);                   \
        if (e_ != hipSuccess) return hip_fail(e_, #expr); \
    } while (0)

size_t align256(size_t v) { return (v + 255) / 256 * 256; }

// Scratch of the allocation-free forward (q38_moe_forward_static): one fixed array per GPU,
// allocated with the code object and held until the process ends. Host code never passes
// the array's name to a kernel: it passes the device address that hipGetSymbolAddress
// returns for the current device, kept per device in g_scratch.
constexpr size_t kScratchBytes = size_t{8} << 20;
__device__ __align__(256) unsigned char scratch[kScratchBytes];
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch[kMaxDevices] = {};

// With `dev` current: look the array's address up once for this device.
int scratch_init(int dev) {
    if (dev < 0 || dev >= kMaxDevices) {
        g_error = "q38: device index beyond the scratch table";
        return Q38_EINVAL;
    }
    std::lock_guard<std::mutex> lk(g_scratch_mutex);
    if (g_scratch[dev]) return Q38_OK;
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
        g_error = std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e);
        return Q38_EHIP;
    }
    g_scratch[dev] = ptr;
    return Q38_OK;
}

int64_t words_for(int64_t n, int bits) { return ((n + 31) / 32) * bits; }

} // namespace

struct q38_ctx {
    int device;
};

struct q38_moe_layer {
    q38_ctx* ctx;
    q38_moe_desc desc;
    LayerDev dev;
    void* owned = nullptr;      // synthetic tensors
    size_t owned_bytes = 0;
    void* prepared = nullptr;   // codebooks split into 4-dim chunks (+ tiled codes, derived books)
    const uint16_t* books_in[3] = {nullptr, nullptr, nullptr};  // the FP16 books as given
    // per-dimension INT8/U8 books (Q38_CB_U8_PERDIM) of d8/14-bit projections, else null
    const void* u8q[3] = {nullptr, nullptr, nullptr};
    const uint16_t* u8s[3] = {nullptr, nullptr, nullptr};
    const uint16_t* u8b[3] = {nullptr, nullptr, nullptr};
    q38_moe_mixed_weights mixed_in{};  // a mixed layer's bank tensors as given
};

struct q38_head {
    q38_ctx* ctx;
    HeadDev dev;
    void* owned = nullptr;
    size_t owned_bytes = 0;
};

struct q38_slot {
    q38_ctx* ctx;
    int hidden, max_rows;
    uint64_t token_count;
    int staged_rows = 0;
    int draft_count = 0;
    bool has_hidden = false;
    uint16_t* rows[2] = {nullptr, nullptr};  // two [max_rows, H] checkpoint buffers
    int stage_buf = 0;                       // buffer the next stage writes
    const uint16_t* committed = nullptr;     // row of the committed checkpoint
    uint64_t stages = 0;                     // verifications staged so far
};

extern "C" {

const char* q38_last_error(void) { return g_error.c_str(); }
const char* q38_version(void) { return "q38 0.1 gfx950"; }

int q38_ctx_create(int hip_device, q38_ctx** out) {
    if (!out) return fail(Q38_EINVAL, "q38_ctx_create: null output");
    int n = 0;
    Q38_HIP(hipGetDeviceCount(&n));
    if (hip_device < 0 || hip_device >= n) return fail(Q38_EINVAL, "q38_ctx_create: no such HIP device");
    Q38_HIP(hipSetDevice(hip_device));
    if (int rc = scratch_init(hip_device)) return rc;
    *out = new q38_ctx{hip_device};
    return Q38_OK;
}
void q38_ctx_destroy(q38_ctx* ctx) { delete ctx; }

int q38_ctx_synchronize(q38_ctx* ctx, void* stream) {
    if (!ctx) return fail(Q38_EINVAL, "q38_ctx_synchronize: null context");
    int prev = 0;
    Q38_HIP(hipGetDevice(&prev));
    if (prev != ctx->device) Q38_HIP(hipSetDevice(ctx->device));
    hipError_t e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
    uint32_t status = 0;
    if (e == hipSuccess) e = read_wait_status(&status, true);
    if (prev != ctx->device) (void)hipSetDevice(prev);
    if (e != hipSuccess) return hip_fail(e, "q38_ctx_synchronize");
    if (status)
        return fail(Q38_EWAIT, "a bounded wait between workgroups of the one-launch verify layer gave up: the "
                               "outputs of the calls since the last check are invalid (is the device shared?)");
    return Q38_OK;
}

void q38_set_fused_layers(int enable) { set_fused_enabled(enable != 0); }
void q38_set_u8_native(int mode) { set_u8_native(mode); }

void q38_debug_set_wait_limit(int32_t spins) { set_wait_limit(spins); }

// ------------------------------------------------------------------ geometry
int64_t q38_packed_vq_word_count(int64_t code_count, int bits) {
    if (bits <= 0 || bits > 31 || code_count < 0) {
        g_error = "packed VQ codes must use 1 to 31 bits";
        return Q38_EINVAL;
    }
    return words_for(code_count, bits);
}
int q38_unpack_vq_code(const uint32_t* words, int64_t n_words, int64_t index, int bits, uint32_t* out) {
    if (bits <= 0 || bits > 31 || index < 0 || !out || (!words && n_words > 0))
        return fail(Q38_EINVAL, "packed VQ codes must use 1 to 31 bits");
    if (n_words < words_for(index + 1, bits)) return fail(Q38_ERANGE, "packed VQ code is out of range");
    const int64_t bit = (index % 32) * bits;
    const int64_t w = (index / 32) * bits + bit / 32;
    const int sh = static_cast<int>(bit % 32);
    uint64_t v = static_cast<uint64_t>(words[w]) >> sh;
    if (sh + bits > 32) v |= static_cast<uint64_t>(words[w + 1]) << (32 - sh);
    *out = static_cast<uint32_t>(v & ((uint64_t{1} << bits) - 1));
    return Q38_OK;
}
int q38_supports_segmented_vq(int d, int bits) {
    return (d == 2 && bits == 0) || (d == 4 && bits == 8) || (d == 8 && bits == 14);
}

// ------------------------------------------------------------------ MoE layer
static int validate_desc(const q38_moe_desc* d) {
    if (!d) return fail(Q38_EINVAL, "null layer description");
    if (d->hidden <= 0 || d->hidden % 512) return fail(Q38_EINVAL, "hidden size must be a positive multiple of 512");
    if (d->inter <= 0 || d->inter % 128) return fail(Q38_EINVAL, "expert intermediate size must be a positive multiple of 128");
    if (d->experts < 64 || d->experts > 1024 || d->experts % 64)
        return fail(Q38_EINVAL, "routed expert count must be a multiple of 64 in [64, 1024]");
    if (d->top_k < 1 || d->top_k > kMaxTopK || d->top_k > d->experts)
        return fail(Q38_EINVAL, "experts per token must be in [1, 16]");
    if (d->book_format != Q38_CB_FP16 && (d->mixed || d->book_format != Q38_CB_U8_PERDIM))
        return fail(Q38_EINVAL, "codebook format must be Q38_CB_FP16, or Q38_CB_U8_PERDIM for a uniform layer");
    if (d->mixed) {
        if (d->hidden != 2048 || d->inter != 512)
            return fail(Q38_EINVAL, "mixed VQ layers need hidden 2048 and expert intermediate 512");
        if (d->gu_group != d->hidden || d->down_group != d->inter)
            return fail(Q38_EINVAL, "mixed VQ layers use one scale per output row");
        if (d->experts % 2) return fail(Q38_EINVAL, "mixed VQ layers need an even expert count");
        return Q38_OK;
    }
    const int geo[2][2] = {{d->gu_dim, d->gu_bits}, {d->down_dim, d->down_bits}};
    for (auto& g : geo)
        if (!((g[0] == 8 && g[1] == 14) || (g[0] == 4 && g[1] == 8) || (g[0] == 2 && g[1] == 8)))
            return fail(Q38_EINVAL, "VQ geometry must be d8/14-bit, d4/8-bit or d2/8-bit (byte codes)");
    // scale groups: one per row, or groups whose codes tile 16-code lane spans (or are
    // whole multiples of them)
    const int ins[2] = {d->hidden, d->inter};
    const int grp[2] = {d->gu_group, d->down_group};
    for (int p = 0; p < 2; ++p) {
        const int G = grp[p], D = geo[p][0];
        if (G <= 0 || ins[p] % G) return fail(Q38_EINVAL, "scale group must divide the projection input");
        if (G != ins[p] && (G % D || (16 % (G / D) && (G / D) % 16))) return fail(Q38_EINVAL, "unsupported scale group size");
    }
    // the grouped kernels cover a row with at most 64 lanes of 16 codes
    if (d->hidden / d->gu_dim > 1024 || d->inter / d->down_dim > 1024)
        return fail(Q38_EINVAL, "more than 1024 codes per projection row");
    return Q38_OK;
}

static void fill_dev(q38_moe_layer* L, const q38_moe_weights* w) {
    const q38_moe_desc& d = L->desc;
    LayerDev& v = L->dev;
    for (int p = 0; p < 3; ++p) L->books_in[p] = w->books[p];
    v.router = w->router;
    v.wsg = w->shared_gate;
    v.H = d.hidden;
    v.I = d.inter;
    v.E = d.experts;
    v.K = d.top_k;
    v.normalize = d.normalize_topk;
    v.has_shared = d.has_shared;
    for (int p = 0; p < 3; ++p) {
        const int in = p < 2 ? d.hidden : d.inter;
        const int dim = p < 2 ? d.gu_dim : d.down_dim;
        const int bits = p < 2 ? d.gu_bits : d.down_bits;
        const int grp = p < 2 ? d.gu_group : d.down_group;
        v.p[p].codes = w->codes[p];
        v.p[p].scales = w->scales[p];
        v.p[p].book = w->books[p];
        v.p[p].words = static_cast<int>(words_for(in / dim, bits));
        v.p[p].ngrp = in / grp;
        v.p[p].dim = dim;
        v.p[p].bits = bits;
    }
    const bool mfma = moe_uses_mfma(v);
    v.gu_parts = mfma ? d.gu_dim / 4 : 1;
    v.d_parts = mfma ? d.down_dim / 4 : 1;
}

// Codebooks split into 4-dim chunks ([dim/4][entries][4]) for the LDS-resident MFMA path,
// and, for layers the four-row verify kernels serve, the codes in the tiled layout those
// kernels load from (one more copy of the codes: HBM traded for coalesced loads).
// With Q38_CB_U8_PERDIM, the d8/14-bit projections first get their per-dimension INT8/U8
// books (q, scales, biases) and the decoded book, which every kernel then reads in place of
// the FP16 book (SparseMoe::prepare_u8_codebook runs at load time too, src/sparse_moe.cpp:
// 528-544): the gate book centred, up and down affine.
static int prepare_layer(q38_moe_layer* L) {
    size_t total = 0, off[3], toff[3], uoff[3];
    const bool tiled = moe_uses_narrow(L->dev, 1);
    bool u8[3];
    for (int p = 0; p < 3; ++p) {
        off[p] = total;
        total += align256((static_cast<size_t>(1) << L->dev.p[p].bits) * L->dev.p[p].dim * 2);
        u8[p] = L->desc.book_format == Q38_CB_U8_PERDIM && L->dev.p[p].dim == 8 && L->dev.p[p].bits == 14;
        uoff[p] = total;
        // q, scales + biases, the decoded book, then the U8 kernels' operands (u, 16 floats)
        if (u8[p]) total += align256(size_t{16384} * 8) + 256 + align256(size_t{16384} * 8 * 2) +
                            align256(size_t{16384} * 8) + 256;
    }
    int64_t rows[3] = {0, 0, 0};
    for (int p = 0; p < 3 && tiled; ++p) {
        // (the routed experts and the VQ shared expert E: the tensors hold no row E otherwise)
        const int experts = L->desc.experts + (L->desc.has_shared && !L->dev.shared_affine ? 1 : 0);
        rows[p] = static_cast<int64_t>(experts) * (p < 2 ? L->desc.inter : L->desc.hidden);
        toff[p] = total;
        total += align256(static_cast<size_t>(rows[p]) * L->dev.p[p].words * 4);
    }
    char* base = nullptr;
    if (hipMalloc(&base, total) != hipSuccess) return fail(Q38_ENOMEM, "hipMalloc failed for prepared codebooks");
    hipError_t e = hipSuccess;
    for (int p = 0; p < 3 && e == hipSuccess; ++p) {
        if (!u8[p]) continue;
        auto* q = reinterpret_cast<uint8_t*>(base + uoff[p]);
        auto* sb = reinterpret_cast<uint16_t*>(base + uoff[p] + align256(size_t{16384} * 8));
        auto* dec = reinterpret_cast<uint16_t*>(base + uoff[p] + align256(size_t{16384} * 8) + 256);
        e = launch_prepare_u8(L->dev.p[p].book, 16384, p == 0 ? 1 : 0, q, sb, sb + 8, dec, nullptr);
        char* ops = base + uoff[p] + align256(size_t{16384} * 8) + 256 + align256(size_t{16384} * 8 * 2);
        if (e == hipSuccess)
            e = launch_u8_operands(q, 16384, p == 0 ? 1 : 0, sb, sb + 8, reinterpret_cast<uint8_t*>(ops),
                                   reinterpret_cast<float*>(ops + align256(size_t{16384} * 8)), nullptr);
        L->dev.p[p].book_u8 = reinterpret_cast<const uint8_t*>(ops);
        L->dev.p[p].u8_sb = reinterpret_cast<const float*>(ops + align256(size_t{16384} * 8));
        L->u8q[p] = q;
        L->u8s[p] = sb;
        L->u8b[p] = sb + 8;
        L->dev.p[p].book = dec;
    }
    for (int p = 0; p < 3 && e == hipSuccess; ++p) {
        auto* dst = reinterpret_cast<uint16_t*>(base + off[p]);
        // 4-dim chunks feed the MFMA kernels (d8, d4); d2 books are read whole
        if (L->dev.p[p].dim % 4 == 0) {
            e = launch_split_book(L->dev.p[p].book, 1 << L->dev.p[p].bits, L->dev.p[p].dim, dst, nullptr);
            L->dev.p[p].book4 = dst;
        } else {
            L->dev.p[p].book4 = nullptr;
        }
        L->dev.p[p].codes_t = nullptr;
        if (tiled && e == hipSuccess) {
            auto* ct = reinterpret_cast<uint32_t*>(base + toff[p]);
            e = launch_tile_codes(L->dev.p[p].codes, rows[p], L->dev.p[p].words, L->dev.p[p].bits, ct, nullptr);
            L->dev.p[p].codes_t = ct;
        }
    }
    if (e == hipSuccess) e = hipStreamSynchronize(nullptr);
    if (e != hipSuccess) {
        (void)hipFree(base);
        return hip_fail(e, "codebook preparation");
    }
    L->prepared = base;
    // the U8 verify kernels: all three books U8, H 2048, I 512, per-row scales
    L->dev.u8_native = u8[0] && u8[1] && u8[2] && !L->dev.mixed && L->dev.H == 2048 && L->dev.I == 512 &&
                       L->dev.p[0].ngrp == 1 && L->dev.p[1].ngrp == 1 && L->dev.p[2].ngrp == 1;
    return Q38_OK;
}

int q38_moe_layer_create(q38_ctx* ctx, const q38_moe_desc* desc, const q38_moe_weights* weights,
                         q38_moe_layer** out) {
    if (!ctx || !out || !weights) return fail(Q38_EINVAL, "q38_moe_layer_create: null argument");
    if (desc && desc->mixed)
        return fail(Q38_EINVAL, "q38_moe_layer_create: a mixed-geometry layer (desc->mixed = 1) takes per-bank "
                                "tensors; use q38_moe_layer_create_mixed");
    if (int rc = validate_desc(desc)) return rc;
    if (!weights->router || (desc->has_shared && !weights->shared_gate))
        return fail(Q38_EINVAL, "router / shared gate tensors are required");
    for (int p = 0; p < 3; ++p)
        if (!weights->codes[p] || !weights->scales[p] || !weights->books[p])
            return fail(Q38_EINVAL, "every projection needs codes, scales and a codebook");
    auto* L = new q38_moe_layer{ctx, *desc, {}, nullptr, 0, nullptr};
    fill_dev(L, weights);
    if (int rc = prepare_layer(L)) {
        delete L;
        return rc;
    }
    *out = L;
    return Q38_OK;
}

int q38_moe_layer_create_affine_shared(q38_ctx* ctx, const q38_moe_desc* desc, const q38_moe_weights* weights,
                                       const q38_affine_shared* shared, q38_moe_layer** out) {
    if (!ctx || !out || !weights || !shared || !desc)
        return fail(Q38_EINVAL, "q38_moe_layer_create_affine_shared: null argument");
    if (desc->mixed || !desc->has_shared)
        return fail(Q38_EINVAL, "q38_moe_layer_create_affine_shared: a uniform layer with a shared expert "
                                "(has_shared = 1, mixed = 0)");
    if (int rc = validate_desc(desc)) return rc;
    const int bits = shared->bits, G = shared->group, Is = shared->inter;
    if (bits != 2 && bits != 4 && bits != 8)
        return fail(Q38_EINVAL, "affine shared expert: bits must be 2, 4 or 8 (values whole in 32-bit words)");
    if (G != 32 && G != 64 && G != 128) return fail(Q38_EINVAL, "affine shared expert: group must be 32, 64 or 128");
    if (Is < G || Is % G || desc->hidden % G || Is > 4096 || desc->hidden > 4096)
        return fail(Q38_EINVAL, "affine shared expert: the group must divide hidden and inter (both <= 4096)");
    if (static_cast<int64_t>(Is) > static_cast<int64_t>(desc->top_k + 1) * desc->inter)
        return fail(Q38_EINVAL, "affine shared expert: its intermediate size may be at most (top_k + 1) x inter");
    if (shared->scale_dtype != 0 && shared->scale_dtype != 1)
        return fail(Q38_EINVAL, "affine shared expert: scale_dtype 0 (bf16) or 1 (fp16)");
    if (!weights->router || !weights->shared_gate) return fail(Q38_EINVAL, "router / shared gate tensors are required");
    for (int p = 0; p < 3; ++p) {
        if (!weights->codes[p] || !weights->scales[p] || !weights->books[p])
            return fail(Q38_EINVAL, "every projection needs codes, scales and a codebook");
        if (!shared->weight[p] || !shared->scales[p] || !shared->biases[p])
            return fail(Q38_EINVAL, "affine shared expert: every projection needs weight, scales and biases");
    }
    auto* L = new q38_moe_layer{ctx, *desc, {}, nullptr, 0, nullptr};
    fill_dev(L, weights);
    LayerDev& v = L->dev;
    v.shared_affine = 1;
    v.sa_bits = bits;
    v.sa_group = G;
    v.sa_inter = Is;
    v.sa_f16 = shared->scale_dtype;
    for (int p = 0; p < 3; ++p) v.sa[p] = AffineDev{shared->weight[p], shared->scales[p], shared->biases[p]};
    if (int rc = prepare_layer(L)) {
        delete L;
        return rc;
    }
    *out = L;
    return Q38_OK;
}

struct SynthLayout {
    size_t router, wsg, book[3], codes[3], scales[3], total;
};
static SynthLayout synth_layout(const q38_moe_desc& d) {
    SynthLayout s{};
    size_t off = 0;
    const int E1 = d.experts + 1;
    s.router = off; off += align256(static_cast<size_t>(d.experts) * d.hidden * 2);
    s.wsg = off; off += align256(static_cast<size_t>(d.hidden) * 2);
    for (int p = 0; p < 3; ++p) {
        const int in = p < 2 ? d.hidden : d.inter, outd = p < 2 ? d.inter : d.hidden;
        const int dim = p < 2 ? d.gu_dim : d.down_dim, bits = p < 2 ? d.gu_bits : d.down_bits;
        const int grp = p < 2 ? d.gu_group : d.down_group;
        s.book[p] = off; off += align256((static_cast<size_t>(1) << bits) * dim * 2);
        s.codes[p] = off; off += align256(static_cast<size_t>(E1) * outd * words_for(in / dim, bits) * 4);
        s.scales[p] = off; off += align256(static_cast<size_t>(E1) * outd * (in / grp) * 2);
    }
    s.total = off;
    return s;
}

static int create_synthetic_mixed(q38_ctx* ctx, const q38_moe_desc& d, uint64_t seed, int32_t layer_index,
                                  q38_moe_layer** out);

int q38_moe_layer_create_synthetic(q38_ctx* ctx, const q38_moe_desc* desc, uint64_t seed, int32_t layer_index,
                                   q38_moe_layer** out) {
    if (!ctx || !out) return fail(Q38_EINVAL, "q38_moe_layer_create_synthetic: null argument");
    if (int rc = validate_desc(desc)) return rc;
    if (desc->mixed) return create_synthetic_mixed(ctx, *desc, seed, layer_index, out);
    const q38_moe_desc& d = *desc;
    const SynthLayout s = synth_layout(d);
    char* base = nullptr;
    if (hipMalloc(&base, s.total) != hipSuccess) return fail(Q38_ENOMEM, "hipMalloc failed for a synthetic layer");
    const hipStream_t st = nullptr;
    const uint64_t layer = static_cast<uint64_t>(layer_index);
    auto* r = reinterpret_cast<uint16_t*>(base + s.router);
    auto* ws = reinterpret_cast<uint16_t*>(base + s.wsg);
    hipError_t e = launch_gen_normal(stream_key(seed, layer, T_ROUTER), static_cast<int64_t>(d.experts) * d.hidden,
                                     0.02, 0, r, st);
    if (e == hipSuccess) e = launch_gen_normal(stream_key(seed, layer, T_WSG), d.hidden, 0.02, 0, ws, st);
    const uint64_t tb[3] = {T_CB_GATE, T_CB_UP, T_CB_DOWN};
    const uint64_t tc[3] = {T_CODES_GATE, T_CODES_UP, T_CODES_DOWN};
    const uint64_t ts[3] = {T_SCALE_GATE, T_SCALE_UP, T_SCALE_DOWN};
    q38_moe_weights w{};
    w.router = r;
    w.shared_gate = ws;
    for (int p = 0; p < 3 && e == hipSuccess; ++p) {
        const int in = p < 2 ? d.hidden : d.inter, outd = p < 2 ? d.inter : d.hidden;
        const int dim = p < 2 ? d.gu_dim : d.down_dim, bits = p < 2 ? d.gu_bits : d.down_bits;
        const int grp = p < 2 ? d.gu_group : d.down_group;
        auto* book = reinterpret_cast<uint16_t*>(base + s.book[p]);
        auto* codes = reinterpret_cast<uint32_t*>(base + s.codes[p]);
        auto* scales = reinterpret_cast<uint16_t*>(base + s.scales[p]);
        e = launch_gen_normal(stream_key(seed, layer, tb[p]), (int64_t{1} << bits) * dim, 1.0, 1, book, st);
        if (e == hipSuccess)
            e = launch_gen_codes(stream_key(seed, layer, tc[p]), 0, 1, d.experts + 1, outd, in / dim, bits,
                                 static_cast<int>(words_for(in / dim, bits)), codes, st);
        if (e == hipSuccess)
            e = launch_gen_uniform_f16(stream_key(seed, layer, ts[p]), 0,
                                       static_cast<int64_t>(d.experts + 1) * outd * (in / grp), 0.005, 0.02, scales,
                                       st);
        w.codes[p] = codes;
        w.scales[p] = scales;
        w.books[p] = book;
    }
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) {
        (void)hipFree(base);
        return hip_fail(e, "synthetic layer generation");
    }
    auto* L = new q38_moe_layer{ctx, d, {}, base, s.total, nullptr};
    fill_dev(L, &w);
    if (int rc = prepare_layer(L)) {
        (void)hipFree(base);
        delete L;
        return rc;
    }
    *out = L;
    return Q38_OK;
}

// ------------------------------------------------------------------ mixed geometry
static float h2f_host(uint16_t h) {
    _Float16 v;
    std::memcpy(&v, &h, 2);
    return static_cast<float>(v);
}

static void fill_dev_mixed(q38_moe_layer* L, const q38_moe_mixed_weights* w) {
    const q38_moe_desc& d = L->desc;
    LayerDev& v = L->dev;
    L->mixed_in = *w;
    v = LayerDev{};
    v.router = w->router;
    v.wsg = w->shared_gate;
    v.H = d.hidden;
    v.I = d.inter;
    v.E = d.experts;
    v.K = d.top_k;
    v.normalize = d.normalize_topk;
    v.has_shared = d.has_shared;
    v.mixed = 1;
    for (int p = 0; p < 3; ++p) {
        const int in = p < 2 ? d.hidden : d.inter;
        ProjDev a{};
        a.codes = w->codes_d4[p];
        a.scales = w->scales_d4[p];
        a.book = w->books_d4[p];
        a.words = static_cast<int>(words_for(in / 4, 8));
        a.ngrp = 1;
        a.dim = 4;
        a.bits = 8;
        ProjDev b{};
        b.codes = w->codes_d8[p];
        b.scales = w->scales_d8[p];
        b.book_i8 = w->books_d8[p];
        b.book_scale = h2f_host(w->book_scales_d8[p]);
        b.words = static_cast<int>(words_for(in / 8, 14));
        b.ngrp = 1;
        b.dim = 8;
        b.bits = 14;
        v.pb[p][0] = a;
        v.pb[p][1] = b;
        v.p[p] = b;
    }
    // the odd bank (two codebook chunks) writes two partial-sum planes, the even bank writes
    // one and clears the second
    v.gu_parts = v.d_parts = 2;
}

// Chunked fp16 codebooks of a mixed layer for the MFMA kernels: the d4 books are already in
// the chunk layout ([1][256][4]); the INT8 d8 books are decoded (q * scale) into
// [2][16384][4] fp16.
static int prepare_mixed(q38_moe_layer* L) {
    const size_t per = align256(static_cast<size_t>(16384) * 8 * 2);
    char* base = nullptr;
    if (hipMalloc(&base, 3 * per) != hipSuccess) return fail(Q38_ENOMEM, "hipMalloc failed for prepared codebooks");
    hipError_t e = hipSuccess;
    LayerDev& v = L->dev;
    for (int p = 0; p < 3 && e == hipSuccess; ++p) {
        auto* dst = reinterpret_cast<uint16_t*>(base + p * per);
        e = launch_split_book_i8(v.pb[p][1].book_i8, v.pb[p][1].book_scale, 1 << v.pb[p][1].bits, v.pb[p][1].dim, dst,
                                 nullptr);
        v.pb[p][0].book4 = v.pb[p][0].book;
        v.pb[p][1].book4 = dst;
        v.p[p] = v.pb[p][1];
    }
    if (e == hipSuccess) e = hipStreamSynchronize(nullptr);
    if (e != hipSuccess) {
        (void)hipFree(base);
        return hip_fail(e, "mixed codebook preparation");
    }
    L->prepared = base;
    return Q38_OK;
}

int q38_moe_layer_create_mixed(q38_ctx* ctx, const q38_moe_desc* desc, const q38_moe_mixed_weights* w,
                               q38_moe_layer** out) {
    if (!ctx || !out || !w) return fail(Q38_EINVAL, "q38_moe_layer_create_mixed: null argument");
    if (!desc || !desc->mixed) return fail(Q38_EINVAL, "q38_moe_layer_create_mixed: desc->mixed must be 1");
    if (int rc = validate_desc(desc)) return rc;
    if (!w->router || (desc->has_shared && !w->shared_gate))
        return fail(Q38_EINVAL, "router / shared gate tensors are required");
    for (int p = 0; p < 3; ++p)
        if (!w->codes_d4[p] || !w->scales_d4[p] || !w->books_d4[p] || !w->codes_d8[p] || !w->scales_d8[p] ||
            !w->books_d8[p])
            return fail(Q38_EINVAL, "mixed layer tensors are required for all three projections");
    auto* L = new q38_moe_layer{ctx, *desc, {}, nullptr, 0, nullptr};
    fill_dev_mixed(L, w);
    if (int rc = prepare_mixed(L)) {
        delete L;
        return rc;
    }
    *out = L;
    return Q38_OK;
}

static int create_synthetic_mixed(q38_ctx* ctx, const q38_moe_desc& d, uint64_t seed, int32_t layer_index,
                                  q38_moe_layer** out) {
    const int nA = d.experts / 2 + 1, nB = d.experts / 2;  // bank 0 holds the shared expert
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t at = off;
        off += align256(bytes);
        return at;
    };
    const size_t o_router = take(static_cast<size_t>(d.experts) * d.hidden * 2), o_wsg = take(d.hidden * 2);
    size_t o_bA[3], o_cA[3], o_sA[3], o_b16[3], o_bB[3], o_bs[3], o_cB[3], o_sB[3];
    for (int p = 0; p < 3; ++p) {
        const int in = p < 2 ? d.hidden : d.inter, outd = p < 2 ? d.inter : d.hidden;
        o_bA[p] = take(256 * 4 * 2);
        o_cA[p] = take(static_cast<size_t>(nA) * outd * words_for(in / 4, 8) * 4);
        o_sA[p] = take(static_cast<size_t>(nA) * outd * 2);
        o_b16[p] = take(16384 * 8 * 2);
        o_bB[p] = take(16384 * 8);
        o_bs[p] = take(2);
        o_cB[p] = take(static_cast<size_t>(nB) * outd * words_for(in / 8, 14) * 4);
        o_sB[p] = take(static_cast<size_t>(nB) * outd * 2);
    }
    char* base = nullptr;
    if (hipMalloc(&base, off) != hipSuccess) return fail(Q38_ENOMEM, "hipMalloc failed for a synthetic layer");
    const hipStream_t st = nullptr;
    const uint64_t layer = static_cast<uint64_t>(layer_index);
    q38_moe_mixed_weights w{};
    w.router = reinterpret_cast<uint16_t*>(base + o_router);
    w.shared_gate = reinterpret_cast<uint16_t*>(base + o_wsg);
    hipError_t e = launch_gen_normal(stream_key(seed, layer, T_ROUTER), static_cast<int64_t>(d.experts) * d.hidden,
                                     0.02, 0, const_cast<uint16_t*>(w.router), st);
    if (e == hipSuccess)
        e = launch_gen_normal(stream_key(seed, layer, T_WSG), d.hidden, 0.02, 0, const_cast<uint16_t*>(w.shared_gate),
                              st);
    const uint64_t tb[3] = {T_CB_GATE, T_CB_UP, T_CB_DOWN}, tb4[3] = {T_CB4_GATE, T_CB4_UP, T_CB4_DOWN};
    const uint64_t tc[3] = {T_CODES_GATE, T_CODES_UP, T_CODES_DOWN};
    const uint64_t ts[3] = {T_SCALE_GATE, T_SCALE_UP, T_SCALE_DOWN};
    for (int p = 0; p < 3 && e == hipSuccess; ++p) {
        const int in = p < 2 ? d.hidden : d.inter, outd = p < 2 ? d.inter : d.hidden;
        auto* bA = reinterpret_cast<uint16_t*>(base + o_bA[p]);
        auto* cA = reinterpret_cast<uint32_t*>(base + o_cA[p]);
        auto* sA = reinterpret_cast<uint16_t*>(base + o_sA[p]);
        auto* b16 = reinterpret_cast<uint16_t*>(base + o_b16[p]);
        auto* bB = reinterpret_cast<int8_t*>(base + o_bB[p]);
        auto* bs = reinterpret_cast<uint16_t*>(base + o_bs[p]);
        auto* cB = reinterpret_cast<uint32_t*>(base + o_cB[p]);
        auto* sB = reinterpret_cast<uint16_t*>(base + o_sB[p]);
        e = launch_gen_normal(stream_key(seed, layer, tb4[p]), 256 * 4, 1.0, 1, bA, st);
        if (e == hipSuccess) e = launch_gen_normal(stream_key(seed, layer, tb[p]), 16384 * 8, 1.0, 1, b16, st);
        if (e == hipSuccess) e = launch_book_to_int8(b16, 16384 * 8, bB, bs, st);
        if (e == hipSuccess)
            e = launch_gen_codes(stream_key(seed, layer, tc[p]), 0, 2, nA, outd, in / 4, 8,
                                 static_cast<int>(words_for(in / 4, 8)), cA, st);
        if (e == hipSuccess)
            e = launch_gen_codes(stream_key(seed, layer, tc[p]), 1, 2, nB, outd, in / 8, 14,
                                 static_cast<int>(words_for(in / 8, 14)), cB, st);
        if (e == hipSuccess) e = launch_gen_scales(stream_key(seed, layer, ts[p]), 0, 2, nA, outd, 0.005, 0.02, sA, st);
        if (e == hipSuccess) e = launch_gen_scales(stream_key(seed, layer, ts[p]), 1, 2, nB, outd, 0.005, 0.02, sB, st);
        if (e == hipSuccess) e = hipMemcpyAsync(&w.book_scales_d8[p], bs, 2, hipMemcpyDeviceToHost, st);
        w.codes_d4[p] = cA;
        w.scales_d4[p] = sA;
        w.books_d4[p] = bA;
        w.codes_d8[p] = cB;
        w.scales_d8[p] = sB;
        w.books_d8[p] = bB;
    }
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) {
        (void)hipFree(base);
        return hip_fail(e, "synthetic mixed layer generation");
    }
    auto* L = new q38_moe_layer{ctx, d, {}, base, off, nullptr};
    fill_dev_mixed(L, &w);
    if (int rc = prepare_mixed(L)) {
        (void)hipFree(base);
        delete L;
        return rc;
    }
    *out = L;
    return Q38_OK;
}

// ------------------------------------------------------------------ GatedDeltaNet verify
struct q38_gdn {
    q38_ctx* ctx;
    q38_gdn_desc desc;
    GdnDev dev;
    size_t state_elems;
};

int q38_gdn_create(q38_ctx* ctx, const q38_gdn_desc* desc, const q38_gdn_weights* w, q38_gdn** out) {
    if (!ctx || !desc || !w || !out) return fail(Q38_EINVAL, "q38_gdn_create: null argument");
    const q38_gdn_desc& d = *desc;
    // the reference's own checks (src/gated_delta_net.cpp:169-177), then what the kernels take
    if (d.key_heads <= 0 || d.value_heads <= 0 || d.key_dim <= 0 || d.value_dim <= 0 || d.hidden <= 0)
        return fail(Q38_EINVAL, "GatedDeltaNet dimensions must be positive");
    if (d.value_heads % d.key_heads != 0) return fail(Q38_EINVAL, "value heads must be divisible by key heads");
    if (d.conv_kernel != 4)
        return fail(Q38_EINVAL, "the retained Qwen3.8 checkpoint requires convolution width 4");
    if (d.bits != 2 && d.bits != 4 && d.bits != 8) return fail(Q38_EINVAL, "GatedDeltaNet projections: bits must be 2, 4 or 8");
    if (d.group != 32 && d.group != 64 && d.group != 128)
        return fail(Q38_EINVAL, "GatedDeltaNet projections: group must be 32, 64 or 128");
    if (d.scale_dtype != 0 && d.scale_dtype != 1) return fail(Q38_EINVAL, "scale_dtype must be 0 (bf16) or 1 (fp16)");
    if (d.gate_silu != 0 && d.gate_silu != 1) return fail(Q38_EINVAL, "gate_silu must be 0 (sigmoid) or 1 (silu)");
    if (!(d.eps > 0.0f)) return fail(Q38_EINVAL, "eps must be positive");
    const int VW = d.value_heads * d.value_dim;
    if (d.hidden % d.group || VW % d.group || d.hidden % 32 || d.hidden > 8192 || VW > 16384)
        return fail(Q38_EINVAL, "hidden and HV * DV must be multiples of the group (hidden <= 8192, HV * DV <= 16384)");
    GdnDev G{};
    G.hidden = d.hidden;
    G.hk = d.key_heads;
    G.hv = d.value_heads;
    G.dk = d.key_dim;
    G.dv = d.value_dim;
    G.bits = d.bits;
    G.group = d.group;
    G.f16 = d.scale_dtype;
    G.gate_silu = d.gate_silu;
    G.eps = d.eps;
    if (!gdn_geometry_ok(G)) return fail(Q38_EINVAL, "GatedDeltaNet: key_dim = value_dim of 64, 128 or 256");
    for (int p = 0; p < 5; ++p) {
        if (!w->weight[p] || !w->scales[p] || !w->biases[p]) return fail(Q38_EINVAL, "q38_gdn_create: null projection");
        G.w[p] = w->weight[p];
        G.s[p] = w->scales[p];
        G.b[p] = w->biases[p];
    }
    if (!w->conv || !w->a_log || !w->dt_bias || !w->norm) return fail(Q38_EINVAL, "q38_gdn_create: null tensor");
    G.conv_w = w->conv;
    G.a_log = w->a_log;
    G.dt_bias = w->dt_bias;
    G.norm_w = w->norm;
    const size_t C = 2 * static_cast<size_t>(d.key_heads) * d.key_dim + static_cast<size_t>(VW);
    *out = new q38_gdn{ctx, d, G, 3 * C + static_cast<size_t>(VW) * d.key_dim};
    return Q38_OK;
}

void q38_gdn_destroy(q38_gdn* gdn) { delete gdn; }

size_t q38_gdn_state_bytes(const q38_gdn* gdn) { return gdn ? gdn->state_elems * 2 : 0; }

static size_t gdn_ws(const q38_gdn* g, int S, GdnBufs* b, void* base) {
    const q38_gdn_desc& d = g->desc;
    const size_t KW = static_cast<size_t>(d.key_heads) * d.key_dim, VW = static_cast<size_t>(d.value_heads) * d.value_dim;
    const size_t C = 2 * KW + VW, HV = static_cast<size_t>(d.value_heads);
    size_t off = 0;
    char* p = static_cast<char*>(base);
    auto take = [&](size_t bytes) {
        char* q = p ? p + off : nullptr;
        off += align256(bytes);
        return q;
    };
    GdnBufs t{};
    t.qkv = reinterpret_cast<uint16_t*>(take(S * C * 2));
    t.z = reinterpret_cast<uint16_t*>(take(S * VW * 2));
    t.bpr = reinterpret_cast<uint16_t*>(take(S * HV * 2));
    t.apr = reinterpret_cast<uint16_t*>(take(S * HV * 2));
    t.q = reinterpret_cast<uint16_t*>(take(S * KW * 2));
    t.k = reinterpret_cast<uint16_t*>(take(S * KW * 2));
    t.v = reinterpret_cast<uint16_t*>(take(S * VW * 2));
    t.beta = reinterpret_cast<float*>(take(S * HV * 4));
    t.decay = reinterpret_cast<float*>(take(S * HV * 4));
    t.y = reinterpret_cast<uint16_t*>(take(S * VW * 2));
    t.gated = reinterpret_cast<uint16_t*>(take(S * VW * 2));
    if (b) *b = t;
    return off;
}

size_t q38_gdn_workspace_size(const q38_gdn* gdn, int32_t max_rows) {
    if (!gdn || max_rows < 1 || max_rows > 64) return 0;
    return gdn_ws(gdn, max_rows, nullptr, nullptr);
}

int q38_gdn_verify(q38_gdn* gdn, const uint16_t* x, int32_t rows, const void* origin, void* checkpoints,
                   uint16_t* out, void* ws, size_t ws_bytes, void* stream) {
    if (!gdn || !x || !out) return fail(Q38_EINVAL, "q38_gdn_verify: null argument");
    if (rows < 1 || rows > 64) return fail(Q38_EINVAL, "GatedDeltaNet batch requires shape [1,S,hidden], S=1..64");
    GdnBufs b{};
    if (!ws || ws_bytes < gdn_ws(gdn, rows, &b, ws)) return fail(Q38_ESPACE, "workspace too small");
    Q38_HIP(launch_gdn_verify(gdn->dev, b, rows, x, static_cast<const uint16_t*>(origin),
                              static_cast<uint16_t*>(checkpoints), out, static_cast<hipStream_t>(stream)));
    return Q38_OK;
}

int q38_gdn_commit(const q38_gdn* gdn, const void* checkpoints, int32_t row, void* state, void* stream) {
    if (!gdn || !checkpoints || !state) return fail(Q38_EINVAL, "q38_gdn_commit: null argument");
    if (row < 0 || row >= 64) return fail(Q38_EINVAL, "q38_gdn_commit: row must be 0..63");
    const size_t bytes = gdn->state_elems * 2;
    Q38_HIP(hipMemcpyAsync(state, static_cast<const char*>(checkpoints) + bytes * static_cast<size_t>(row), bytes,
                           hipMemcpyDeviceToDevice, static_cast<hipStream_t>(stream)));
    return Q38_OK;
}

// ------------------------------------------------------------------ full attention verify
struct q38_attn {
    q38_ctx* ctx;
    q38_attn_desc desc;
    AttnDev dev;
    uint16_t* norms;  // effective q and k norm weights [2][D] (owned)
};

int q38_attn_create(q38_ctx* ctx, const q38_attn_desc* desc, const q38_attn_weights* w, q38_attn** out) {
    if (!ctx || !desc || !w || !out) return fail(Q38_EINVAL, "q38_attn_create: null argument");
    const q38_attn_desc& d = *desc;
    // the reference's check (src/self_attention.cpp:515-520), then what the kernels take
    if (d.hidden <= 0 || d.q_heads <= 0 || d.kv_heads <= 0 || d.head_dim <= 0)
        return fail(Q38_EINVAL, "attention dimensions must be positive");
    if (d.q_heads % d.kv_heads != 0 || d.rotary_dim <= 0 || d.rotary_dim % 2 != 0 || d.rotary_dim > d.head_dim)
        return fail(Q38_EINVAL, "unsupported attention head/rotary configuration");
    if (!attn_geometry_ok(d.hidden, d.q_heads, d.kv_heads, d.head_dim, d.rotary_dim))
        return fail(Q38_EINVAL, "attention head dimension must be 64, 128 or 256");
    if (d.bits != 2 && d.bits != 4 && d.bits != 8) return fail(Q38_EINVAL, "attention projections: bits must be 2, 4 or 8");
    if (d.group != 32 && d.group != 64 && d.group != 128)
        return fail(Q38_EINVAL, "attention projections: group must be 32, 64 or 128");
    if (d.scale_dtype != 0 && d.scale_dtype != 1) return fail(Q38_EINVAL, "scale_dtype must be 0 (bf16) or 1 (fp16)");
    if (d.norm_offset != 0 && d.norm_offset != 1) return fail(Q38_EINVAL, "norm_offset must be 0 or 1");
    if (!(d.eps > 0.0f) || !(d.rope_theta > 0.0)) return fail(Q38_EINVAL, "eps and rope_theta must be positive");
    const int QW = d.q_heads * d.head_dim;
    if (d.hidden % d.group || QW % d.group || d.hidden % 32 || d.hidden > 8192 || QW > 16384)
        return fail(Q38_EINVAL, "hidden and HQ * D must be multiples of the group (hidden <= 8192, HQ * D <= 16384)");
    AttnDev A{};
    A.hidden = d.hidden;
    A.hq = d.q_heads;
    A.hkv = d.kv_heads;
    A.d = d.head_dim;
    A.rot = d.rotary_dim;
    A.bits = d.bits;
    A.group = d.group;
    A.f16 = d.scale_dtype;
    A.eps = d.eps;
    A.theta = d.rope_theta;
    for (int p = 0; p < 4; ++p) {
        if (!w->weight[p] || !w->scales[p] || !w->biases[p]) return fail(Q38_EINVAL, "q38_attn_create: null projection");
        A.w[p] = w->weight[p];
        A.s[p] = w->scales[p];
        A.b[p] = w->biases[p];
    }
    if (!w->q_norm || !w->k_norm) return fail(Q38_EINVAL, "q38_attn_create: null norm weight");
    uint16_t* norms = nullptr;
    const size_t D = static_cast<size_t>(d.head_dim);
    if (hipMalloc(&norms, 2 * D * 2) != hipSuccess) return fail(Q38_ENOMEM, "hipMalloc failed for the attention norms");
    hipError_t e = hipSuccess;
    if (d.norm_offset) {
        e = launch_hc_norm_weight(w->q_norm, static_cast<int>(D), norms, nullptr);
        if (e == hipSuccess) e = launch_hc_norm_weight(w->k_norm, static_cast<int>(D), norms + D, nullptr);
    } else {
        e = hipMemcpy(norms, w->q_norm, D * 2, hipMemcpyDeviceToDevice);
        if (e == hipSuccess) e = hipMemcpy(norms + D, w->k_norm, D * 2, hipMemcpyDeviceToDevice);
    }
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        (void)hipFree(norms);
        return hip_fail(e, "attention norm weights");
    }
    A.qn = norms;
    A.kn = norms + D;
    *out = new q38_attn{ctx, d, A, norms};
    return Q38_OK;
}

void q38_attn_destroy(q38_attn* a) {
    if (!a) return;
    (void)hipFree(a->norms);
    delete a;
}

size_t q38_attn_cache_bytes(const q38_attn* a, int64_t capacity) {
    if (!a || capacity < 1) return 0;
    return 2 * static_cast<size_t>(a->desc.kv_heads) * static_cast<size_t>(capacity) * a->desc.head_dim * 2;
}

static size_t attn_ws(const q38_attn* a, int S, int64_t tokens, AttnBufs* b, void* base) {
    const q38_attn_desc& d = a->desc;
    const size_t QW = static_cast<size_t>(d.q_heads) * d.head_dim, KW = static_cast<size_t>(d.kv_heads) * d.head_dim;
    const size_t NQ = static_cast<size_t>(S) * d.q_heads;
    size_t off = 0;
    char* p = static_cast<char*>(base);
    auto take = [&](size_t bytes) {
        char* q = p ? p + off : nullptr;
        off += align256(bytes);
        return q;
    };
    AttnBufs t{};
    t.qg = reinterpret_cast<uint16_t*>(take(S * 2 * QW * 2));
    t.kr = reinterpret_cast<uint16_t*>(take(S * KW * 2));
    t.vr = reinterpret_cast<uint16_t*>(take(S * KW * 2));
    t.q = reinterpret_cast<uint16_t*>(take(S * QW * 2));
    t.gs = reinterpret_cast<uint16_t*>(take(S * QW * 2));
    t.sc = reinterpret_cast<uint16_t*>(take(NQ * static_cast<size_t>(attn_score_stride(tokens)) * 2));
    t.stats = reinterpret_cast<float2*>(take(static_cast<size_t>(attn_score_tiles(tokens)) * NQ * 8));
    t.mx = reinterpret_cast<float*>(take(NQ * 4));
    t.sm = reinterpret_cast<float*>(take(NQ * 4));
    t.part = reinterpret_cast<float*>(take(static_cast<size_t>(attn_pv_tiles(tokens)) * NQ * d.head_dim * 4));
    t.gated = reinterpret_cast<uint16_t*>(take(S * QW * 2));
    if (b) *b = t;
    return off;
}

size_t q38_attn_workspace_size(const q38_attn* a, int32_t max_rows, int64_t max_tokens) {
    if (!a || max_rows < 1 || max_rows > 64 || max_tokens < max_rows) return 0;
    return attn_ws(a, max_rows, max_tokens, nullptr, nullptr);
}

int q38_attn_verify(q38_attn* a, const uint16_t* x, int32_t rows, void* cache, int64_t capacity, int64_t cache_tokens,
                    int64_t position, uint16_t* out, void* ws, size_t ws_bytes, void* stream) {
    if (!a || !x || !cache || !out || !ws) return fail(Q38_EINVAL, "q38_attn_verify: null argument");
    if (rows < 1 || rows > 64) return fail(Q38_EINVAL, "attention batch requires shape [1,S,hidden], S=1..64");
    if (cache_tokens < 0 || position < 0 || capacity < 1)
        return fail(Q38_EINVAL, "attention cache tokens and position must not be negative");
    if (cache_tokens + rows > capacity) return fail(Q38_ERANGE, "attention cache capacity exceeded");
    if (reinterpret_cast<uintptr_t>(cache) % 16) return fail(Q38_EINVAL, "q38_attn_verify: cache must be 16-byte aligned");
    AttnBufs b{};
    if (ws_bytes < attn_ws(a, rows, cache_tokens + rows, &b, ws)) return fail(Q38_ESPACE, "workspace too small");
    uint16_t* keys = static_cast<uint16_t*>(cache);
    uint16_t* values = keys + static_cast<size_t>(a->desc.kv_heads) * static_cast<size_t>(capacity) * a->desc.head_dim;
    Q38_HIP(launch_attn_verify(a->dev, b, rows, x, keys, values, capacity, cache_tokens, position, out,
                               static_cast<hipStream_t>(stream)));
    return Q38_OK;
}

void q38_moe_layer_destroy(q38_moe_layer* layer) {
    if (!layer) return;
    if (layer->owned) (void)hipFree(layer->owned);
    if (layer->prepared) (void)hipFree(layer->prepared);
    delete layer;
}

int q38_moe_layer_weights(const q38_moe_layer* L, q38_moe_weights* out) {
    if (!L || !out) return fail(Q38_EINVAL, "null argument");
    if (L->dev.mixed) return fail(Q38_EINVAL, "a mixed layer has per-bank tensors (q38_moe_mixed_weights)");
    out->router = L->dev.router;
    out->shared_gate = L->dev.wsg;
    for (int p = 0; p < 3; ++p) {
        out->codes[p] = L->dev.p[p].codes;
        out->scales[p] = L->dev.p[p].scales;
        out->books[p] = L->books_in[p];
    }
    return Q38_OK;
}

int q38_moe_layer_mixed_weights(const q38_moe_layer* L, q38_moe_mixed_weights* out) {
    if (!L || !out) return fail(Q38_EINVAL, "null argument");
    if (!L->dev.mixed) return fail(Q38_EINVAL, "a uniform layer has one set of tensors (q38_moe_weights)");
    *out = L->mixed_in;
    return Q38_OK;
}

int q38_moe_layer_codebook(const q38_moe_layer* L, int proj, const uint16_t** book, const void** q,
                           const uint16_t** scales, const uint16_t** biases) {
    if (!L || proj < 0 || proj > 2) return fail(Q38_EINVAL, "q38_moe_layer_codebook: bad arguments");
    if (L->dev.mixed) return fail(Q38_EINVAL, "a mixed layer has per-bank codebooks");
    if (book) *book = L->dev.p[proj].book;
    if (q) *q = L->u8q[proj];
    if (scales) *scales = L->u8s[proj];
    if (biases) *biases = L->u8b[proj];
    return Q38_OK;
}

int64_t q38_moe_layer_bytes(const q38_moe_layer* L, int32_t n_unique, int32_t rows) {
    if (!L) return Q38_EINVAL;
    const LayerDev& v = L->dev;
    if (v.mixed) {  // half the routed experts of each geometry on average; shared expert d4
        int64_t pe[2] = {0, 0}, books = 0;
        for (int b = 0; b < 2; ++b)
            for (int p = 0; p < 3; ++p) {
                const int outd = p < 2 ? v.I : v.H;
                pe[b] += static_cast<int64_t>(outd) * v.pb[p][b].words * 4 + static_cast<int64_t>(outd) * 2;
            }
        books = 3 * (256 * 4 * 2 + 16384 * 8);
        return static_cast<int64_t>(n_unique) * (pe[0] + pe[1]) / 2 + (v.has_shared ? pe[0] : 0) + books +
               static_cast<int64_t>(v.E) * v.H * 2 + (v.has_shared ? v.H * 2 : 0) +
               static_cast<int64_t>(2) * rows * v.H * 2;
    }
    int64_t per_expert = 0, books = 0;
    for (int p = 0; p < 3; ++p) {
        const int outd = p < 2 ? v.I : v.H;
        per_expert += static_cast<int64_t>(outd) * v.p[p].words * 4 + static_cast<int64_t>(outd) * v.p[p].ngrp * 2;
        books += (int64_t{1} << v.p[p].bits) * v.p[p].dim * 2;
    }
    const int64_t experts = static_cast<int64_t>(n_unique) + (v.has_shared && !v.shared_affine ? 1 : 0);
    // an affine shared expert: 3 projections of sa_inter x H values, a scale and a bias per group
    const int64_t sa = v.shared_affine ? 3 * (static_cast<int64_t>(v.sa_inter) * v.H * v.sa_bits / 8 +
                                              static_cast<int64_t>(v.sa_inter) * v.H / v.sa_group * 4)
                                       : 0;
    return experts * per_expert + sa + books + static_cast<int64_t>(v.E) * v.H * 2 + (v.has_shared ? v.H * 2 : 0) +
           static_cast<int64_t>(2) * rows * v.H * 2;
}

static size_t moe_ws(const q38_moe_desc& d, int M, MoeBufs* w, void* base) {
    const int MK = M * d.top_k;
    size_t off = 0;
    char* b = static_cast<char*>(base);
    auto take = [&](size_t bytes) {
        char* p = b ? b + off : nullptr;
        off += align256(bytes);
        return p;
    };
    MoeBufs t{};
    t.x = reinterpret_cast<uint16_t*>(take(static_cast<size_t>(M) * d.hidden * 2));
    t.x16 = reinterpret_cast<uint16_t*>(take(static_cast<size_t>(M) * d.hidden * 2));
    t.logits = reinterpret_cast<float*>(take(static_cast<size_t>(M) * d.experts * 4));
    t.sgate = reinterpret_cast<float*>(take(static_cast<size_t>(M) * 4));
    t.experts = reinterpret_cast<int32_t*>(take(static_cast<size_t>(MK) * 4));
    t.weights = reinterpret_cast<float*>(take(static_cast<size_t>(MK) * 4));
    t.plan = reinterpret_cast<int32_t*>(take(static_cast<size_t>(2 + 4 * MK) * 4));
    const size_t gu = static_cast<size_t>(MK + M) * d.inter, dn = static_cast<size_t>(MK + M) * d.hidden;
    t.g = reinterpret_cast<float*>(take(2 * gu * 4));
    t.u = reinterpret_cast<float*>(take(2 * gu * 4));
    t.d = reinterpret_cast<float*>(take(2 * dn * 4));
    t.h16 = reinterpret_cast<uint16_t*>(take(gu * 2));
    t.dcorr = t.g ? t.g + gu : nullptr;  // (g's second plane: unused by the U8 kernels' calls)
    t.gu_plane = gu;
    t.d_plane = dn;
    t.wait_limit = wait_limit();
    if (w) *w = t;
    return off;
}

size_t q38_moe_workspace_size(const q38_moe_desc* desc, int32_t max_rows) {
    if (!desc || max_rows < 1 || max_rows > kMaxPrefillRows) return 0;
    return moe_ws(*desc, max_rows, nullptr, nullptr);
}

static int check_rows(int rows) {
    if (rows < 1 || rows > kMaxRows) return fail(Q38_EINVAL, "verify rows must be between 1 and 16");
    return Q38_OK;
}

static int copy_routes(const q38_moe_layer* L, int M, const MoeBufs& w, const q38_route_out* r, hipStream_t st) {
    if (!r) return Q38_OK;
    const int MK = M * L->desc.top_k;
    if (r->experts) Q38_HIP(hipMemcpyAsync(r->experts, w.experts, MK * 4, hipMemcpyDeviceToDevice, st));
    if (r->weights) Q38_HIP(hipMemcpyAsync(r->weights, w.weights, MK * 4, hipMemcpyDeviceToDevice, st));
    if (r->logits)
        Q38_HIP(hipMemcpyAsync(r->logits, w.logits, static_cast<size_t>(M) * L->desc.experts * 4,
                               hipMemcpyDeviceToDevice, st));
    if (r->plan) Q38_HIP(hipMemcpyAsync(r->plan, w.plan, (2 + 4 * MK) * 4, hipMemcpyDeviceToDevice, st));
    if (r->x_norm)
        Q38_HIP(hipMemcpyAsync(r->x_norm, w.x, static_cast<size_t>(M) * L->desc.hidden * 2,
                               hipMemcpyDeviceToDevice, st));
    return Q38_OK;
}

// Rows beyond the verify width take the prefill kernels (one plane per projection).
static int check_forward_rows(const q38_moe_layer* L, int rows) {
    if (rows >= 1 && rows <= kMaxRows) return Q38_OK;
    if (rows < 1 || rows > kMaxPrefillRows) return fail(Q38_EINVAL, "rows must be between 1 and 2048");
    if (L->desc.top_k * rows > 32768) return fail(Q38_EINVAL, "rows x top_k must not exceed 32768");
    if (!moe_supports_prefill(L->dev) && !moe_supports_grouped_prefill(L->dev))
        return fail(Q38_EINVAL, "prefill widths (rows > 16) need a uniform layer of d8/14, d4/8 or d2/8 codes");
    return Q38_OK;
}

static int route_prefill(const q38_moe_layer* L, const MoeBufs& w, int rows, const uint16_t* x, hipStream_t st,
                         hipEvent_t* ev) {
    KernelTimer& kt = kernel_timer();
    if (ev) kt = {ev[0], ev[1]};
    Q38_HIP(launch_router_rows(L->dev, w, rows, x, st));
    if (ev) kt = {ev[2], ev[3]};
    Q38_HIP(launch_topk_rows(L->dev, w, rows, st));
    if (ev) kt = {ev[4], ev[5]};
    Q38_HIP(launch_plan_sort(L->dev, w, rows, st));
    return Q38_OK;
}

int q38_moe_route(q38_moe_layer* L, const uint16_t* x, int32_t rows, const q38_route_out* routes, void* ws,
                  size_t ws_bytes, void* stream) {
    if (!L || !x) return fail(Q38_EINVAL, "q38_moe_route: null argument");
    if (int rc = check_forward_rows(L, rows)) return rc;
    MoeBufs w{};
    if (!ws || ws_bytes < moe_ws(L->desc, rows, &w, ws)) return fail(Q38_ESPACE, "workspace too small");
    const hipStream_t st = static_cast<hipStream_t>(stream);
    if (rows > kMaxRows) {
        if (int rc = route_prefill(L, w, rows, x, st, nullptr)) return rc;
    } else {
        Q38_HIP(launch_router(L->dev, w, rows, x, false, 0.0f, st));
        Q38_HIP(launch_topk_plan(expert_view(L->dev), w, rows, st));
    }
    return copy_routes(L, rows, w, routes, st);
}

// Prefill widths (SparseMoe::forward_prefill_impl, src/sparse_moe.cpp:2252-2505): logits,
// top-k, sorted plan, segmented gate/up, SwiGLU, segmented down, combine. ev, when given,
// holds 14 events: start/stop of each of the 7 kernels in that order.
static int run_prefill(q38_moe_layer* L, const MoeBufs& w, int rows, const uint16_t* x, uint16_t* y,
                       const q38_route_out* trace, hipEvent_t* ev, hipStream_t st) {
    if (int rc = route_prefill(L, w, rows, x, st, ev)) return rc;
    Q38_HIP(launch_shared_affine(L->dev, w, rows, st));
    LayerDev one = expert_view(L->dev);  // partial-sum planes of the prefill kernels
    KernelTimer& kt = kernel_timer();
    if (!moe_supports_prefill(L->dev)) {
        // scale groups, d4 and d2 codes: the grouped kernels over 16-route passes of each slot
        // (one partial-sum plane; SwiGLU inside the down kernel)
        one.gu_parts = one.d_parts = 1;
        if (ev) kt = {ev[6], ev[7]};
        Q38_HIP(launch_gate_up_grouped(one, w, rows, st));
        kt = {};
        if (trace)
            if (int rc = copy_routes(L, rows, w, trace, st)) return rc;
        if (ev) {
            Q38_HIP(hipEventRecord(ev[8], st));
            Q38_HIP(hipEventRecord(ev[9], st));
            kt = {ev[10], ev[11]};
        }
        Q38_HIP(launch_down_grouped(one, w, rows, st));
        if (ev) kt = {ev[12], ev[13]};
        one.has_shared = L->dev.has_shared;
        Q38_HIP(launch_combine(one, w, rows, nullptr, y, st));
        kt = {};
        return Q38_OK;
    }
    one.gu_parts = one.d_parts = prefill_planes(L->dev, rows);
    if (ev) kt = {ev[6], ev[7]};
    Q38_HIP(launch_gate_up_pf(one, w, rows, st));
    if (trace)
        if (int rc = copy_routes(L, rows, w, trace, st)) return rc;
    if (ev) kt = {ev[8], ev[9]};
    Q38_HIP(launch_swiglu_pf(one, w, rows, st));
    if (ev) kt = {ev[10], ev[11]};
    Q38_HIP(launch_down_pf(one, w, rows, st));
    if (ev) kt = {ev[12], ev[13]};
    one.has_shared = L->dev.has_shared;  // (the combine adds the shared expert, affine or not)
    Q38_HIP(launch_combine(one, w, rows, nullptr, y, st));
    kt = {};
    return Q38_OK;
}

// One layer: router logits (with the layer-input RMSNorm of h when norm is set), routing
// plan (fused into the MFMA gate/up kernels, a separate kernel otherwise), gate/up, down,
// combine. Chain mode (h_chain): src is h_chain, and the combine adds the residual to it in
// place; otherwise src is x and y receives the layer output. ev, when given, holds 5
// events recorded around the phases.
static int run_layer(q38_moe_layer* L, const MoeBufs& w, int rows, const uint16_t* src, bool norm, float eps,
                     uint16_t* h_chain, uint16_t* y, const q38_route_out* trace, hipEvent_t* ev, hipStream_t st) {
    const LayerDev dev = moe_call_dev(L->dev, rows);
    const LayerDev ex = expert_view(dev);  // (without the shared slot when it is affine)
    if (ev) Q38_HIP(hipEventRecord(ev[0], st));
    Q38_HIP(launch_router(dev, w, rows, src, norm, eps, st));
    Q38_HIP(launch_shared_affine(dev, w, rows, st));
    if (!moe_plans_in_gate_up(ex, rows)) Q38_HIP(launch_topk_plan(ex, w, rows, st));
    if (ev) Q38_HIP(hipEventRecord(ev[1], st));
    if (moe_uses_fused(ex, rows)) {  // gate/up, down and combine in one launch
        if (dev.shared_affine) {  // (the combine, with the affine shared rows, as its own kernel)
            Q38_HIP(launch_gate_down4(ex, w, rows, nullptr, nullptr, st));
            Q38_HIP(launch_combine(dev, w, rows, h_chain, y, st));
        } else {
            Q38_HIP(launch_gate_down4(ex, w, rows, h_chain, h_chain ? nullptr : y, st));
        }
        if (ev)
            for (int i = 2; i <= 4; ++i) Q38_HIP(hipEventRecord(ev[i], st));
        return copy_routes(L, rows, w, trace, st);
    }
    Q38_HIP(launch_gate_up(ex, w, rows, st));
    if (ev) Q38_HIP(hipEventRecord(ev[2], st));
    if (trace)
        if (int rc = copy_routes(L, rows, w, trace, st)) return rc;
    Q38_HIP(launch_down(ex, w, rows, st));
    if (ev) Q38_HIP(hipEventRecord(ev[3], st));
    Q38_HIP(launch_combine(dev, w, rows, h_chain, y, st));
    if (ev) Q38_HIP(hipEventRecord(ev[4], st));
    return Q38_OK;
}

int q38_moe_forward(q38_moe_layer* L, const uint16_t* x, int32_t rows, uint16_t* y, const q38_route_out* routes,
                    void* ws, size_t ws_bytes, void* stream) {
    if (!L || !x || !y) return fail(Q38_EINVAL, "q38_moe_forward: null argument");
    if (x == y) return fail(Q38_EINVAL, "q38_moe_forward: input and output must not alias");
    if (int rc = check_forward_rows(L, rows)) return rc;
    MoeBufs w{};
    if (!ws || ws_bytes < moe_ws(L->desc, rows, &w, ws)) return fail(Q38_ESPACE, "workspace too small");
    if (rows > kMaxRows) return run_prefill(L, w, rows, x, y, routes, nullptr, static_cast<hipStream_t>(stream));
    return run_layer(L, w, rows, x, false, 0.0f, nullptr, y, routes, nullptr, static_cast<hipStream_t>(stream));
}

int q38_moe_forward_static(q38_moe_layer* L, const uint16_t* x, int32_t rows, uint16_t* y, const q38_route_out* routes,
                           void* stream) {
    if (!L || !x || !y) return fail(Q38_EINVAL, "q38_moe_forward_static: null argument");
    if (x == y) return fail(Q38_EINVAL, "q38_moe_forward_static: input and output must not alias");
    if (int rc = check_rows(rows)) return rc;
    const size_t need = moe_ws(L->desc, rows, nullptr, nullptr);
    if (need > kScratchBytes)
        return fail(Q38_ESPACE, "q38_moe_forward_static: the layer needs " + std::to_string(need) +
                                    " bytes of scratch for this many rows; the fixed scratch holds " +
                                    std::to_string(kScratchBytes));
    void* base = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_scratch_mutex);
        const int dev = L->ctx->device;
        base = dev >= 0 && dev < kMaxDevices ? g_scratch[dev] : nullptr;
    }
    if (!base) return fail(Q38_ESTATE, "q38_moe_forward_static: no scratch on the layer's device");
    MoeBufs w{};
    moe_ws(L->desc, rows, &w, base);
    return run_layer(L, w, rows, x, false, 0.0f, nullptr, y, routes, nullptr, static_cast<hipStream_t>(stream));
}

int q38_moe_forward_prefill_profiled(q38_moe_layer* L, const uint16_t* x, int32_t rows, uint16_t* y,
                                     const q38_route_out* routes, void* ws, size_t ws_bytes, float* kernel_ms,
                                     void* stream) {
    if (!L || !x || !y || !kernel_ms) return fail(Q38_EINVAL, "q38_moe_forward_prefill_profiled: null argument");
    if (x == y) return fail(Q38_EINVAL, "q38_moe_forward_prefill_profiled: input and output must not alias");
    if (rows <= kMaxRows) return fail(Q38_EINVAL, "profiled prefill needs rows > 16");
    if (int rc = check_forward_rows(L, rows)) return rc;
    MoeBufs w{};
    if (!ws || ws_bytes < moe_ws(L->desc, rows, &w, ws)) return fail(Q38_ESPACE, "workspace too small");
    const hipStream_t st = static_cast<hipStream_t>(stream);
    hipEvent_t ev[14] = {};
    int rc = Q38_OK;
    for (auto& e : ev)
        if (rc == Q38_OK && hipEventCreate(&e) != hipSuccess) rc = fail(Q38_EHIP, "hipEventCreate failed");
    if (rc == Q38_OK) rc = run_prefill(L, w, rows, x, y, routes, ev, st);
    kernel_timer() = {};
    if (rc == Q38_OK) {
        hipError_t e = hipStreamSynchronize(st);
        for (int k = 0; k < 7 && e == hipSuccess; ++k) e = hipEventElapsedTime(&kernel_ms[k], ev[2 * k], ev[2 * k + 1]);
        if (e != hipSuccess) rc = hip_fail(e, "profiled prefill timings");
    }
    for (auto& e : ev)
        if (e) (void)hipEventDestroy(e);
    return rc;
}

int q38_moe_layer_set_router_bias(q38_moe_layer* L, const float* bias) {
    if (!L) return fail(Q38_EINVAL, "q38_moe_layer_set_router_bias: null layer");
    L->dev.rbias = bias;
    return Q38_OK;
}

static int chain_check(q38_moe_layer* const* layers, int32_t n_layers, uint16_t* h, int32_t rows, void* ws,
                       size_t ws_bytes) {
    if (!layers || n_layers < 1 || !h) return fail(Q38_EINVAL, "verify chain: bad arguments");
    if (int rc = check_rows(rows)) return rc;
    size_t need = 0;
    for (int l = 0; l < n_layers; ++l) {
        if (!layers[l]) return fail(Q38_EINVAL, "verify chain: null layer");
        if (layers[l]->desc.hidden != layers[0]->desc.hidden)
            return fail(Q38_EINVAL, "verify chain: layers disagree on the hidden size");
        need = std::max(need, moe_ws(layers[l]->desc, rows, nullptr, nullptr));
    }
    if (!ws || ws_bytes < need) return fail(Q38_ESPACE, "workspace too small");
    return Q38_OK;
}

int q38_verify_chain(q38_moe_layer* const* layers, int32_t n_layers, uint16_t* h, int32_t rows, float eps,
                     const q38_route_out* traces, void* ws, size_t ws_bytes, void* stream) {
    if (int rc = chain_check(layers, n_layers, h, rows, ws, ws_bytes)) return rc;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    for (int l = 0; l < n_layers; ++l) {
        MoeBufs w{};
        moe_ws(layers[l]->desc, rows, &w, ws);
        if (int rc = run_layer(layers[l], w, rows, h, true, eps, h, nullptr, traces ? &traces[l] : nullptr, nullptr, st))
            return rc;
    }
    return Q38_OK;
}

int q38_verify_chain_profiled(q38_moe_layer* const* layers, int32_t n_layers, uint16_t* h, int32_t rows, float eps,
                              const q38_route_out* traces, void* ws, size_t ws_bytes, q38_moe_timings* tm,
                              void* stream) {
    if (!tm) return fail(Q38_EINVAL, "q38_verify_chain_profiled: null timings");
    if (int rc = chain_check(layers, n_layers, h, rows, ws, ws_bytes)) return rc;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    // per layer and phase (router, gate/up, down, combine): start/stop of the phase's kernel
    std::vector<hipEvent_t> ev(static_cast<size_t>(n_layers) * 8, nullptr);
    int rc = Q38_OK;
    for (auto& e : ev)
        if (hipEventCreate(&e) != hipSuccess) rc = fail(Q38_EHIP, "hipEventCreate failed");
    KernelTimer& kt = kernel_timer();
    for (int l = 0; l < n_layers && rc == Q38_OK; ++l) {
        MoeBufs w{};
        moe_ws(layers[l]->desc, rows, &w, ws);
        hipEvent_t* E = &ev[static_cast<size_t>(l) * 8];
        const q38_moe_layer* L = layers[l];
        const LayerDev dev = moe_call_dev(L->dev, rows);
        hipError_t e = hipSuccess;
        const LayerDev ex = expert_view(dev);
        kt = {E[0], E[1]};
        e = launch_router(dev, w, rows, h, true, eps, st);
        if (e == hipSuccess) e = launch_shared_affine(dev, w, rows, st);
        if (e == hipSuccess && !moe_plans_in_gate_up(ex, rows)) e = launch_topk_plan(ex, w, rows, st);
        // (gate/up, down and combine in one launch; with an affine shared expert the combine is
        // a kernel of its own)
        const bool fused = moe_uses_fused(ex, rows), split_combine = !fused || dev.shared_affine;
        if (e == hipSuccess) {
            kt = {E[2], E[3]};
            e = fused ? launch_gate_down4(ex, w, rows, dev.shared_affine ? nullptr : h, nullptr, st)
                      : launch_gate_up(ex, w, rows, st);
        }
        if (e == hipSuccess && traces)
            if (copy_routes(L, rows, w, &traces[l], st) != Q38_OK) e = hipErrorUnknown;
        if (e == hipSuccess) {
            if (fused) {  // down (and the combine) ran in the gate/up launch (down_ms 0)
                kt = {};
                for (int i = 4; i < (split_combine ? 6 : 8) && e == hipSuccess; ++i) e = hipEventRecord(E[i], st);
            } else {
                kt = {E[4], E[5]};
                e = launch_down(ex, w, rows, st);
            }
        }
        if (e == hipSuccess && split_combine) {
            kt = {E[6], E[7]};
            e = launch_combine(dev, w, rows, h, nullptr, st);
        }
        kt = {};
        if (e != hipSuccess) rc = hip_fail(e, "profiled verify chain");
    }
    if (rc == Q38_OK) {
        hipError_t e = hipStreamSynchronize(st);
        q38_moe_timings t{};
        for (int l = 0; l < n_layers && e == hipSuccess; ++l) {
            hipEvent_t* E = &ev[static_cast<size_t>(l) * 8];
            float ms[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            // (a fused layer's down and combine phases ran inside its gate/up kernel: 0; with an
            // affine shared expert its combine is timed)
            const LayerDev lv = moe_call_dev(layers[l]->dev, rows);
            const bool fz = moe_uses_fused(expert_view(lv), rows);
            for (int i = 0; i < 4 && e == hipSuccess; ++i)
                if (!fz || i < 2 || (i == 3 && lv.shared_affine)) e = hipEventElapsedTime(&ms[i], E[2 * i], E[2 * i + 1]);
            t.routing_ms += ms[0];
            t.gate_up_ms += ms[1];
            t.down_ms += ms[2];
            t.merge_ms += ms[3];
        }
        t.layers = n_layers;
        uint32_t status = 0;
        if (e == hipSuccess) e = read_wait_status(&status, true);
        if (e != hipSuccess) rc = hip_fail(e, "profiled chain timing");
        else if (status) rc = fail(Q38_EWAIT, "q38_verify_chain_profiled: a wait between workgroups gave up");
        else *tm = t;
    }
    for (auto& e : ev)
        if (e) (void)hipEventDestroy(e);
    return rc;
}

int q38_rmsnorm(const uint16_t* x, int32_t rows, int32_t hidden, float eps, uint16_t* y, void* stream) {
    if (!x || !y || rows < 1 || hidden < 1) return fail(Q38_EINVAL, "q38_rmsnorm: bad arguments");
    Q38_HIP(launch_rmsnorm(x, rows, hidden, eps, y, static_cast<hipStream_t>(stream)));
    return Q38_OK;
}

int q38_embed_synthetic_dev(uint64_t seed, const uint32_t* tokens, int32_t n, int32_t hidden, uint16_t* h,
                            void* stream) {
    if (!tokens || !h || n < 1 || hidden < 1) return fail(Q38_EINVAL, "q38_embed_synthetic_dev: bad arguments");
    Q38_HIP(launch_gen_embed_dev(seed, tokens, n, hidden, h, static_cast<hipStream_t>(stream)));
    return Q38_OK;
}

int q38_embed_synthetic(uint64_t seed, const uint32_t* tokens, int32_t n, int32_t hidden, uint16_t* h,
                        void* stream) {
    if (!tokens || !h || n < 1 || hidden < 1) return fail(Q38_EINVAL, "q38_embed_synthetic: bad arguments");
    for (int r = 0; r < n; r += 32)  // token ids travel as kernel arguments, 32 per launch
        Q38_HIP(launch_gen_embed(seed, tokens + r, std::min(32, n - r), hidden, h + static_cast<size_t>(r) * hidden,
                                 static_cast<hipStream_t>(stream)));
    return Q38_OK;
}

// ------------------------------------------------------------------ heads
static int head_validate(int kind, int64_t vocab, int hidden) {
    if (kind != Q38_HEAD_Q8 && kind != Q38_HEAD_Q4G64) return fail(Q38_EINVAL, "unknown head kind");
    if (vocab < 1 || vocab > (int64_t{1} << 31) - 2) return fail(Q38_EINVAL, "vocab out of range");
    if (kind == Q38_HEAD_Q8 && hidden != 1024 && hidden != 2048 && hidden != 2560)
        return fail(Q38_EINVAL, "Q8 head hidden size must be 1024, 2048 or 2560");
    if (kind == Q38_HEAD_Q4G64 && hidden != 2048) return fail(Q38_EINVAL, "Q4 head hidden size must be 2048");
    return Q38_OK;
}

static int head_finish(q38_head* hd) {
    Q38_HIP(head_init_attrs());
    float* d = nullptr;
    Q38_HIP(hipMalloc(&d, sizeof(float)));
    const int64_t ns = hd->dev.kind == 0 ? hd->dev.V : hd->dev.V * (hd->dev.H / 64);
    hipError_t e = launch_scale_absmax(hd->dev.scales, ns, d, nullptr);
    if (e == hipSuccess) e = hipMemcpy(&hd->dev.s_max, d, sizeof(float), hipMemcpyDeviceToHost);
    (void)hipFree(d);
    if (e != hipSuccess) return hip_fail(e, "head scale scan");
    return Q38_OK;
}

int q38_head_create(q38_ctx* ctx, int kind, int64_t vocab, int32_t hidden, const void* weights,
                    const uint16_t* scales, q38_head** out) {
    if (!ctx || !out || !weights || !scales) return fail(Q38_EINVAL, "q38_head_create: null argument");
    if (int rc = head_validate(kind, vocab, hidden)) return rc;
    auto* hd = new q38_head{ctx, {}, nullptr, 0};
    hd->dev = HeadDev{static_cast<const int8_t*>(weights), scales, vocab, hidden, kind, 0.0f};
    if (int rc = head_finish(hd)) {
        delete hd;
        return rc;
    }
    *out = hd;
    return Q38_OK;
}

int q38_head_create_synthetic(q38_ctx* ctx, int kind, int64_t vocab, int32_t hidden, uint64_t seed, q38_head** out) {
    if (!ctx || !out) return fail(Q38_EINVAL, "q38_head_create_synthetic: null argument");
    if (int rc = head_validate(kind, vocab, hidden)) return rc;
    const size_t wbytes = kind == 0 ? static_cast<size_t>(vocab) * hidden : static_cast<size_t>(vocab) * hidden / 2;
    const size_t sbytes = kind == 0 ? static_cast<size_t>(vocab) * 2 : static_cast<size_t>(vocab) * (hidden / 64) * 2;
    char* base = nullptr;
    if (hipMalloc(&base, align256(wbytes) + align256(sbytes)) != hipSuccess)
        return fail(Q38_ENOMEM, "hipMalloc failed for a synthetic head");
    auto* w = reinterpret_cast<int8_t*>(base);
    auto* s = reinterpret_cast<uint16_t*>(base + align256(wbytes));
    auto* hd = new q38_head{ctx, HeadDev{w, s, vocab, hidden, kind, 0.0f}, base, align256(wbytes) + align256(sbytes)};
    hipError_t e = launch_gen_head(hd->dev, seed, w, s, nullptr);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        (void)hipFree(base);
        delete hd;
        return hip_fail(e, "synthetic head generation");
    }
    if (int rc = head_finish(hd)) {
        (void)hipFree(base);
        delete hd;
        return rc;
    }
    *out = hd;
    return Q38_OK;
}

void q38_head_destroy(q38_head* hd) {
    if (!hd) return;
    if (hd->owned) (void)hipFree(hd->owned);
    delete hd;
}

int q38_head_weights(const q38_head* hd, const void** weights, const uint16_t** scales) {
    if (!hd) return fail(Q38_EINVAL, "null head");
    if (weights) *weights = hd->dev.w;
    if (scales) *scales = hd->dev.scales;
    return Q38_OK;
}

int64_t q38_head_bytes(const q38_head* hd) {
    if (!hd) return Q38_EINVAL;
    if (hd->dev.kind == 0) return hd->dev.V * hd->dev.H + hd->dev.V * 2;
    return hd->dev.V * hd->dev.H / 2 + hd->dev.V * (hd->dev.H / 64) * 2;
}

size_t q38_head_workspace_size(const q38_head* hd, int32_t max_rows) {
    if (!hd || max_rows < 1 || max_rows > kHeadMaxRows) return 0;
    if (hd->dev.kind != Q38_HEAD_Q8) return max_rows <= 4 ? 256 : 0;
    return head_work_bytes(hd->dev, max_rows, true);
}

int q38_head_greedy(q38_head* hd, const uint16_t* h, int32_t rows, uint32_t* argmax, float* logit, void* ws,
                    size_t ws_bytes, void* stream) {
    if (!hd || !h || !argmax || !logit) return fail(Q38_EINVAL, "q38_head_greedy: null argument");
    if (hd->dev.kind != Q38_HEAD_Q8) return fail(Q38_EINVAL, "greedy argmax needs a Q8 head");
    if (rows < 1 || rows > kHeadMaxRows) return fail(Q38_EINVAL, "head rows must be between 1 and 16 per call");
    if (!ws || ws_bytes < head_work_bytes(hd->dev, rows, true)) return fail(Q38_ESPACE, "workspace too small");
    const HeadWork w = head_work_carve(ws, hd->dev, rows, true);
    Q38_HIP(launch_head_greedy(hd->dev, h, rows, w, argmax, logit, static_cast<hipStream_t>(stream)));
    return Q38_OK;
}

int q38_head_logits(q38_head* hd, const uint16_t* h, int32_t rows, float* logits, void* ws, size_t ws_bytes,
                    void* stream) {
    if (!hd || !h || !logits) return fail(Q38_EINVAL, "q38_head_logits: null argument");
    HeadWork w{};
    if (hd->dev.kind == Q38_HEAD_Q8) {
        if (rows < 1 || rows > kHeadMaxRows) return fail(Q38_EINVAL, "head rows must be between 1 and 16 per call");
        if (!ws || ws_bytes < head_work_bytes(hd->dev, rows, false)) return fail(Q38_ESPACE, "workspace too small");
        w = head_work_carve(ws, hd->dev, rows, false);
    } else if (rows < 1 || rows > 4) {
        return fail(Q38_EINVAL, "Q4 head rows must be between 1 and 4 per call");
    }
    Q38_HIP(launch_head_logits(hd->dev, h, rows, w, logits, static_cast<hipStream_t>(stream)));
    return Q38_OK;
}

// q38_head_probs: [head logits workspace | logits (when probs is null) | softmax partials]
static size_t head_probs_layout(const q38_head* hd, int rows, size_t* logits_off, size_t* part_off) {
    const size_t hw = align256(q38_head_workspace_size(hd, rows));
    const size_t lg = align256(static_cast<size_t>(rows) * static_cast<size_t>(hd->dev.V) * 4);
    if (logits_off) *logits_off = hw;
    if (part_off) *part_off = hw + lg;
    return hw + lg + softmax_rows_workspace(rows, hd->dev.V);
}

size_t q38_head_probs_workspace_size(const q38_head* hd, int32_t max_rows) {
    if (!hd || max_rows < 1 || q38_head_workspace_size(hd, max_rows) == 0) return 0;
    return head_probs_layout(hd, max_rows, nullptr, nullptr);
}

int q38_head_probs(q38_head* hd, const uint16_t* h, int32_t rows, float temperature, float* probs, float* stats,
                   void* ws, size_t ws_bytes, void* stream) {
    if (!hd || !h || !stats) return fail(Q38_EINVAL, "q38_head_probs: null argument");
    if (!(temperature > 0.0f) || !std::isfinite(temperature))
        return fail(Q38_EINVAL, "q38_head_probs: temperature must be positive and finite");
    if (q38_head_workspace_size(hd, rows) == 0)
        return fail(Q38_EINVAL, hd->dev.kind == Q38_HEAD_Q8 ? "head rows must be between 1 and 16 per call"
                                                            : "Q4 head rows must be between 1 and 4 per call");
    size_t lo = 0, po = 0;
    const size_t need = head_probs_layout(hd, rows, &lo, &po);
    if (!ws || ws_bytes < need) return fail(Q38_ESPACE, "workspace too small");
    char* base = static_cast<char*>(ws);
    float* logits = probs ? probs : reinterpret_cast<float*>(base + lo);
    if (int rc = q38_head_logits(hd, h, rows, logits, ws, lo, stream)) return rc;
    Q38_HIP(launch_softmax_rows(logits, rows, hd->dev.V, temperature, stats, probs, base + po,
                                static_cast<hipStream_t>(stream)));
    return Q38_OK;
}

int q38_argmax_rows(const float* logits, int32_t rows, int64_t vocab, uint32_t* argmax, float* value, void* ws,
                    size_t ws_bytes, void* stream) {
    if (!logits || !argmax) return fail(Q38_EINVAL, "q38_argmax_rows: null argument");
    if (rows < 1 || rows > 64 || vocab < 1 || vocab > (int64_t{1} << 31) - 2)
        return fail(Q38_EINVAL, "q38_argmax_rows: rows must be 1..64 and vocab positive");
    if (!ws || ws_bytes < static_cast<size_t>(rows) * 8) return fail(Q38_ESPACE, "workspace too small");
    Q38_HIP(launch_argmax(logits, rows, vocab, static_cast<unsigned long long*>(ws), true, argmax, value, nullptr, 1,
                          0, static_cast<hipStream_t>(stream)));
    return Q38_OK;
}

// ------------------------------------------------------------------ MTP draft head
struct q38_hc {
    q38_ctx* ctx;
    q38_hc_desc desc;
    HcDev dev;
    uint16_t* wn;  // 1 + hc_norm.weight (owned)
};

struct q38_mtp_head {
    q38_ctx* ctx;
    q38_moe_layer* layer;
    q38_head* fc_e;
    q38_head* fc_h;
    q38_head* draft;
    uint64_t embed_seed;
    float eps;
    bool owned;
    // HC streams (q38_mtp_head_set_streams); streams == 1 and no mixers: the single-stream head
    int streams = 1;
    q38_hc* block_hc = nullptr;
    q38_hc* final_hc = nullptr;
    uint16_t* emb_norm = nullptr;  // 1 + pre_fc_norm_embedding.weight [H] (owned; null: gain 1)
    uint16_t* hid_norm = nullptr;  // 1 + pre_fc_norm_hidden.weight [HC * H] (owned; null: gain 1)
};

namespace {
constexpr int kMtpMaxRows = 4;

struct MtpWork {
    uint16_t *x, *f;
    float *pe, *ph, *logits;
    unsigned long long* best;
    unsigned long long* part;  // the Q4 draft head's partial argmax keys [rows][nparts]
    int nparts;
    uint32_t* tokens;
    HeadWork we, wh[4];  // the FC projections' prepared rows (the stream projection in passes)
    int mh[4], passes;
    void* moe_ws;
    size_t moe_ws_bytes;
};

size_t mtp_layout(const q38_mtp_head* m, int rows, MtpWork* w, void* base) {
    const size_t H = static_cast<size_t>(m->layer->desc.hidden);
    const size_t V = static_cast<size_t>(m->draft->dev.V);
    char* b = static_cast<char*>(base);
    size_t off = 0;
    auto take = [&](size_t bytes) {
        char* p = b ? b + off : nullptr;
        off += align256(bytes);
        return p;
    };
    const size_t HC = static_cast<size_t>(m->streams);
    MtpWork t{};
    t.x = reinterpret_cast<uint16_t*>(take(rows * HC * H * 2));
    t.f = reinterpret_cast<uint16_t*>(take(rows * H * 2));
    t.pe = reinterpret_cast<float*>(take(rows * H * 4));
    t.ph = reinterpret_cast<float*>(take(rows * HC * H * 4));
    t.logits = reinterpret_cast<float*>(take(rows * V * 4));
    t.best = reinterpret_cast<unsigned long long*>(take(rows * 8));
    t.part = reinterpret_cast<unsigned long long*>(take(static_cast<size_t>(rows) * kQ4MaxBlocks * 8));
    t.nparts = b ? q4_blocks(rows) : 0;
    t.tokens = reinterpret_cast<uint32_t*>(take(rows * 4));
    t.we = head_work_carve(take(head_work_bytes(m->fc_e->dev, rows, false)), m->fc_e->dev, rows, false);
    const int nrows = rows * m->streams;  // the stream projection's rows, in passes of up to 16
    t.passes = (nrows + kHeadMaxRows - 1) / kHeadMaxRows;
    for (int p = 0; p < t.passes; ++p) {
        t.mh[p] = std::min(kHeadMaxRows, nrows - p * kHeadMaxRows);
        t.wh[p] = head_work_carve(take(head_work_bytes(m->fc_h->dev, t.mh[p], false)), m->fc_h->dev, t.mh[p], false);
    }
    t.moe_ws_bytes = q38_moe_workspace_size(&m->layer->desc, rows);
    if (m->block_hc) {
        t.moe_ws_bytes = std::max(t.moe_ws_bytes, q38_verify_chain_hc_workspace_size(&m->layer->desc,
                                                                                     &m->block_hc->desc, rows));
        t.moe_ws_bytes = std::max(t.moe_ws_bytes, q38_hc_workspace_size(&m->final_hc->desc, rows));
    }
    t.moe_ws = take(t.moe_ws_bytes);
    if (w) *w = t;
    return off;
}

int mtp_validate(q38_moe_layer* layer, q38_head* fe, q38_head* fh, q38_head* dh) {
    if (!layer || !fe || !fh || !dh) return fail(Q38_EINVAL, "q38_mtp_head_create: null component");
    const int H = layer->desc.hidden;
    if (H != 2048) return fail(Q38_EINVAL, "MTP draft head hidden size must be 2048");
    for (const q38_head* fc : {fe, fh})
        if (fc->dev.kind != Q38_HEAD_Q8 || fc->dev.V != H || fc->dev.H != H)
            return fail(Q38_EINVAL, "MTP FC projections must be Q8 heads with vocab = hidden = the layer's hidden");
    if (dh->dev.kind != Q38_HEAD_Q4G64 || dh->dev.H != H)
        return fail(Q38_EINVAL, "MTP draft LM head must be a Q4 head of the layer's hidden size");
    return Q38_OK;
}

// One draft step on rows (<= 4) requests; logits into `logits`, the output stream in w.x.
// With HC streams (combine_inputs, src/mtp_head.cpp:258-266; forward_decode, :454-470): the
// hidden norm runs over the row's HC * H values, the hidden projection over each stream, the
// embedding projection is added to every stream, the block is the mixer read -> MoE ->
// mixer write, and the final mixer's read gives the LM head's input.
// tokens: the step's tokens, or null in a chain: the previous step's argmax keys in w.best,
// whose tokens the prologue also records as drafts[., prev_step].
int mtp_step(q38_mtp_head* m, const MtpWork& w, const uint16_t* stream_in, const uint32_t* tokens, uint32_t* drafts,
             int depth, int prev_step, int rows, float* logits, const q38_mtp_trace* trace, hipStream_t st,
             bool argmax = false) {
    const int H = m->layer->desc.hidden, HC = m->streams;
    DraftPro P{};
    P.embed_key = stream_key(m->embed_seed, kEmbedLayer, T_EMBED);
    P.toks = tokens;
    P.best = w.best;
    // (a chain step after the first takes its token from the previous Q4 head's partial keys)
    P.part = m->draft->dev.kind != Q38_HEAD_Q8 ? w.part : nullptr;
    P.nparts = w.nparts;
    P.drafts = drafts;
    P.tokens_out = w.tokens;
    P.depth = depth;
    P.prev_step = prev_step;
    P.stream = stream_in;
    P.H = H;
    P.HC = HC;
    P.M = rows;
    P.eps = m->eps;
    P.emb_norm = m->emb_norm;
    P.hid_norm = m->hid_norm;
    P.we = w.we;
    for (int p = 0; p < w.passes; ++p) {
        P.wh[p] = w.wh[p];
        P.mh[p] = w.mh[p];
    }
    Q38_HIP(launch_draft_prologue(P, st));
    Q38_HIP(launch_head_logits_prepared(m->fc_e->dev, rows, w.we, w.pe, st));
    for (int p = 0; p < w.passes; ++p)
        Q38_HIP(launch_head_logits_prepared(m->fc_h->dev, w.mh[p], w.wh[p],
                                            w.ph + static_cast<size_t>(p) * kHeadMaxRows * H, st));
    Q38_HIP(launch_fc_join(w.pe, w.ph, rows, HC, H, w.x, w.best, st));
    if (trace && trace->combined)
        Q38_HIP(hipMemcpyAsync(trace->combined, w.x, static_cast<size_t>(rows) * HC * H * 2, hipMemcpyDeviceToDevice,
                               st));
    q38_moe_layer* layers[1] = {m->layer};
    if (m->block_hc) {
        q38_hc* mixers[1] = {m->block_hc};
        if (int rc = q38_verify_chain_hc(layers, mixers, 1, w.x, rows, w.moe_ws, w.moe_ws_bytes, st)) return rc;
        if (int rc = q38_hc_read(m->final_hc, w.x, rows, w.f, nullptr, w.moe_ws, w.moe_ws_bytes, st)) return rc;
    } else {
        if (int rc = q38_verify_chain(layers, 1, w.x, rows, m->eps, nullptr, w.moe_ws, w.moe_ws_bytes, st)) return rc;
        Q38_HIP(launch_rmsnorm(w.x, rows, H, m->eps, w.f, st));
    }
    if (trace && trace->final_mixed)
        Q38_HIP(hipMemcpyAsync(trace->final_mixed, w.f, static_cast<size_t>(rows) * H * 2, hipMemcpyDeviceToDevice,
                               st));
    // (argmax: a Q4 draft head also forms its workgroups' argmax keys in w.part)
    if (argmax && m->draft->dev.kind != Q38_HEAD_Q8) {
        Q38_HIP(launch_head_q4_part(m->draft->dev, w.f, rows, logits, w.part, st));
        return Q38_OK;
    }
    return q38_head_logits(m->draft, w.f, rows, logits, nullptr, 0, st);
}
} // namespace

int q38_mtp_head_create(q38_ctx* ctx, q38_moe_layer* layer, q38_head* fc_embedding, q38_head* fc_hidden,
                        q38_head* draft_head, uint64_t embed_seed, float eps, q38_mtp_head** out) {
    if (!ctx || !out) return fail(Q38_EINVAL, "q38_mtp_head_create: null argument");
    if (int rc = mtp_validate(layer, fc_embedding, fc_hidden, draft_head)) return rc;
    if (!(eps > 0.0f)) return fail(Q38_EINVAL, "q38_mtp_head_create: eps must be positive");
    *out = new q38_mtp_head{ctx, layer, fc_embedding, fc_hidden, draft_head, embed_seed, eps, false};
    return Q38_OK;
}

int q38_mtp_head_create_synthetic(q38_ctx* ctx, const q38_moe_desc* desc, int64_t vocab, uint64_t seed,
                                  q38_mtp_head** out) {
    if (!ctx || !desc || !out) return fail(Q38_EINVAL, "q38_mtp_head_create_synthetic: null argument");
    if (desc->hidden != 2048) return fail(Q38_EINVAL, "MTP draft head hidden size must be 2048");
    q38_moe_layer* layer = nullptr;
    q38_head *fe = nullptr, *fh = nullptr, *dh = nullptr;
    int rc = q38_moe_layer_create_synthetic(ctx, desc, seed, 48, &layer);
    if (rc == Q38_OK)
        rc = q38_head_create_synthetic(ctx, Q38_HEAD_Q8, desc->hidden, desc->hidden, seed ^ Q38_MTP_FC_EMBED_SALT, &fe);
    if (rc == Q38_OK)
        rc = q38_head_create_synthetic(ctx, Q38_HEAD_Q8, desc->hidden, desc->hidden, seed ^ Q38_MTP_FC_HIDDEN_SALT, &fh);
    if (rc == Q38_OK) rc = q38_head_create_synthetic(ctx, Q38_HEAD_Q4G64, vocab, desc->hidden, seed, &dh);
    if (rc == Q38_OK) rc = mtp_validate(layer, fe, fh, dh);
    if (rc != Q38_OK) {
        const std::string msg = g_error;
        q38_head_destroy(dh);
        q38_head_destroy(fh);
        q38_head_destroy(fe);
        q38_moe_layer_destroy(layer);
        return fail(rc, msg);
    }
    *out = new q38_mtp_head{ctx, layer, fe, fh, dh, seed, 1e-6f, true};
    return Q38_OK;
}

static void mtp_free_norms(q38_mtp_head* m) {
    (void)hipFree(m->emb_norm);
    (void)hipFree(m->hid_norm);
    m->emb_norm = m->hid_norm = nullptr;
}

int q38_mtp_head_set_streams(q38_mtp_head* m, const q38_mtp_streams* s) {
    if (!m) return fail(Q38_EINVAL, "q38_mtp_head_set_streams: null head");
    const int H = m->layer->desc.hidden;
    if (!s) {
        mtp_free_norms(m);
        m->streams = 1;
        m->block_hc = m->final_hc = nullptr;
        return Q38_OK;
    }
    if (!s->block_mixer || !s->final_mixer) return fail(Q38_EINVAL, "MTP streams need the block and final mixers");
    const q38_hc_desc &b = s->block_mixer->desc, &f = s->final_mixer->desc;
    if (b.hidden != H || f.hidden != H || b.streams != f.streams)
        return fail(Q38_EINVAL, "MTP mixers must share the head's hidden size and stream count");
    if (!b.with_injection) return fail(Q38_EINVAL, "the MTP block mixer carries injection weights");
    if (f.with_injection) return fail(Q38_EINVAL, "the MTP final mixer is read without injection");
    const int HC = b.streams;
    uint16_t *en = nullptr, *hn = nullptr;
    hipError_t e = hipSuccess;
    if (s->embedding_norm && e == hipSuccess) e = hipMalloc(&en, static_cast<size_t>(H) * 2);
    if (s->hidden_norm && e == hipSuccess) e = hipMalloc(&hn, static_cast<size_t>(HC) * H * 2);
    if (e == hipSuccess && en) e = launch_hc_norm_weight(s->embedding_norm, H, en, nullptr);
    if (e == hipSuccess && hn) e = launch_hc_norm_weight(s->hidden_norm, HC * H, hn, nullptr);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        (void)hipFree(en);
        (void)hipFree(hn);
        return hip_fail(e, "MTP stream norm weights");
    }
    mtp_free_norms(m);
    m->streams = HC;
    m->block_hc = s->block_mixer;
    m->final_hc = s->final_mixer;
    m->emb_norm = en;
    m->hid_norm = hn;
    return Q38_OK;
}

int q38_mtp_head_streams(const q38_mtp_head* m) { return m ? m->streams : 0; }

void q38_mtp_head_destroy(q38_mtp_head* m) {
    if (!m) return;
    mtp_free_norms(m);
    if (m->owned) {
        q38_head_destroy(m->draft);
        q38_head_destroy(m->fc_h);
        q38_head_destroy(m->fc_e);
        q38_moe_layer_destroy(m->layer);
    }
    delete m;
}

int q38_mtp_head_parts(const q38_mtp_head* m, q38_moe_layer** layer, q38_head** fc_embedding, q38_head** fc_hidden,
                       q38_head** draft_head) {
    if (!m) return fail(Q38_EINVAL, "null MTP head");
    if (layer) *layer = m->layer;
    if (fc_embedding) *fc_embedding = m->fc_e;
    if (fc_hidden) *fc_hidden = m->fc_h;
    if (draft_head) *draft_head = m->draft;
    return Q38_OK;
}

size_t q38_mtp_workspace_size(const q38_mtp_head* m, int32_t max_rows) {
    if (!m || max_rows < 1 || max_rows > kMtpMaxRows) return 0;
    return mtp_layout(m, max_rows, nullptr, nullptr);
}

int q38_mtp_forward_decode(q38_mtp_head* m, const uint16_t* stream_in, const uint32_t* tokens, int32_t rows,
                           float* logits, uint16_t* stream_out, const q38_mtp_trace* trace, void* ws,
                           size_t ws_bytes, void* stream) {
    if (!m || !stream_in || !tokens) return fail(Q38_EINVAL, "q38_mtp_forward_decode: null argument");
    if (rows < 1 || rows > kMtpMaxRows) return fail(Q38_EINVAL, "MTP draft rows must be between 1 and 4 per call");
    if (!ws || ws_bytes < mtp_layout(m, rows, nullptr, nullptr)) return fail(Q38_ESPACE, "workspace too small");
    MtpWork w{};
    mtp_layout(m, rows, &w, ws);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    if (int rc = mtp_step(m, w, stream_in, tokens, nullptr, 0, 0, rows, logits ? logits : w.logits, trace, st))
        return rc;
    if (stream_out)
        Q38_HIP(hipMemcpyAsync(stream_out, w.x, static_cast<size_t>(rows) * m->streams * m->layer->desc.hidden * 2,
                               hipMemcpyDeviceToDevice, st));
    return Q38_OK;
}

int q38_mtp_draft_greedy(q38_mtp_head* m, const uint16_t* stream_in, const uint32_t* tokens, int32_t rows,
                         int32_t depth, uint32_t* drafts, uint16_t* stream_out, void* ws, size_t ws_bytes,
                         void* stream) {
    if (!m || !stream_in || !tokens || !drafts) return fail(Q38_EINVAL, "q38_mtp_draft_greedy: null argument");
    if (rows < 1 || rows > kMtpMaxRows) return fail(Q38_EINVAL, "MTP draft rows must be between 1 and 4 per call");
    if (depth < 1 || depth > 24) return fail(Q38_EINVAL, "MTP draft depth must be between 1 and 24");
    if (!ws || ws_bytes < mtp_layout(m, rows, nullptr, nullptr)) return fail(Q38_ESPACE, "workspace too small");
    MtpWork w{};
    mtp_layout(m, rows, &w, ws);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const uint16_t* s_in = stream_in;
    const uint32_t* t_in = tokens;
    for (int step = 0; step < depth; ++step) {
        // the step's join clears w.best; its argmax keys feed the next step's prologue (which
        // records this step's drafts), the last step's are finished here
        const bool fused = m->draft->dev.kind != Q38_HEAD_Q8;  // (the Q4 head merges the keys itself)
        if (int rc = mtp_step(m, w, s_in, step == 0 ? t_in : nullptr, drafts, depth, step - 1, rows, w.logits, nullptr,
                              st, true))
            return rc;
        if (step + 1 == depth) {
            if (fused)
                Q38_HIP(launch_argmax_part_final(w.part, w.nparts, rows, w.tokens, nullptr, drafts, depth, step, st));
            else
                Q38_HIP(launch_argmax(w.logits, rows, m->draft->dev.V, w.best, false, w.tokens, nullptr, drafts,
                                      depth, step, st));
        } else if (!fused) {
            Q38_HIP(launch_argmax_rows(w.logits, rows, m->draft->dev.V, w.best, st));
        }
        s_in = w.x;
    }
    if (stream_out)
        Q38_HIP(hipMemcpyAsync(stream_out, w.x, static_cast<size_t>(rows) * m->streams * m->layer->desc.hidden * 2,
                               hipMemcpyDeviceToDevice, st));
    return Q38_OK;
}

// ------------------------------------------------------------------ acceptance
int q38_mtp_decide_greedy(const uint32_t* drafts, int64_t k, const uint32_t* target, int64_t n_target,
                          const uint32_t* stop, int64_t n_stop, q38_greedy_decision* out) {
    if (!out) return fail(Q38_EINVAL, "null output");
    if (k <= 0 || !drafts) return fail(Q38_EINVAL, "MTP verification requires at least one draft");
    if (n_target != k + 1 || !target) return fail(Q38_EINVAL, "MTP target verification must include the bonus row");
    if (n_stop > 0 && !stop) return fail(Q38_EINVAL, "null stop-token list");
    int64_t a = 0;
    while (a < k && drafts[a] == target[a]) {
        bool is_stop = false;
        for (int64_t s = 0; s < n_stop; ++s) is_stop |= stop[s] == drafts[a];
        if (is_stop) break;
        ++a;
    }
    out->accepted = a;
    out->correction_row = a;
    out->next_token = target[a];
    return Q38_OK;
}

int q38_plan_mtp_commit(uint64_t round_offset, uint64_t drafted, uint64_t accepted, uint64_t* out) {
    if (!out) return fail(Q38_EINVAL, "null output");
    if (accepted > drafted) return fail(Q38_ESTATE, "MTP accepted count exceeds drafted count");
    if (accepted == UINT64_MAX || round_offset > UINT64_MAX - (accepted + 1))
        return fail(Q38_ESTATE, "MTP committed boundary overflow");
    out[0] = round_offset;
    out[1] = 1 + accepted;
    out[2] = 1 + accepted;
    out[3] = round_offset + 1 + accepted;
    return Q38_OK;
}

void q38_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
    philox4x32_10(ctr, key, out);
}

size_t q38_mtp_accept_workspace_size(int32_t k, int64_t vocab) {
    if (k < 1 || k > 24 || vocab < 1 || vocab > (int64_t{1} << 31) - 2) return 0;
    return accept_sampled_workspace(k, vocab);
}

int q38_mtp_accept_sampled(const float* tl, const float* dl, const uint32_t* drafts, int32_t k, int64_t vocab,
                           float temperature, uint64_t seed, uint64_t slot, uint64_t round, int64_t* out, void* ws,
                           size_t ws_bytes, void* stream) {
    if (!tl || !dl || !drafts || !out) return fail(Q38_EINVAL, "q38_mtp_accept_sampled: null argument");
    if (k < 1 || k > 24 || vocab < 1 || vocab > (int64_t{1} << 31) - 2)
        return fail(Q38_EINVAL, "q38_mtp_accept_sampled: bad sizes");
    if (!(temperature > 0.0f)) return fail(Q38_EINVAL, "temperature must be positive");
    if (!ws || ws_bytes < accept_sampled_workspace(k, vocab)) return fail(Q38_ESPACE, "workspace too small");
    Q38_HIP(launch_accept_sampled(tl, dl, drafts, k, vocab, temperature, seed, slot, round, out, ws,
                                  static_cast<hipStream_t>(stream)));
    return Q38_OK;
}

// ------------------------------------------------------------------ private hooks
void q38_private_set_error(const char* msg) { g_error = msg ? msg : ""; }
void q38_private_layer_adopt(q38_moe_layer* layer, void* block) {
    if (layer && !layer->owned) layer->owned = block;
}

// ------------------------------------------------------------------ slots
int q38_slot_create(q38_ctx* ctx, int32_t hidden, int32_t max_rows, uint64_t token_count, q38_slot** out) {
    if (!ctx || !out || hidden < 1 || max_rows < 2 || max_rows > 25)
        return fail(Q38_EINVAL, "q38_slot_create: bad arguments");
    auto* s = new q38_slot{ctx, hidden, max_rows, token_count};
    for (auto& r : s->rows)
        if (hipMalloc(&r, static_cast<size_t>(max_rows) * hidden * 2) != hipSuccess) {
            for (auto& q : s->rows) (void)hipFree(q);
            delete s;
            return fail(Q38_ENOMEM, "hipMalloc failed for a slot");
        }
    *out = s;
    return Q38_OK;
}
void q38_slot_destroy(q38_slot* s) {
    if (!s) return;
    for (auto& r : s->rows) (void)hipFree(r);
    delete s;
}
// Stages into the buffer that does not hold the committed row, so commit is a pointer
// update and the committed checkpoint survives a later stage + rollback.
int q38_slot_stage(q38_slot* s, int32_t draft_count, const uint16_t* h, void* stream) {
    if (!s || !h) return fail(Q38_EINVAL, "q38_slot_stage: null argument");
    if (draft_count < 0 || draft_count + 1 > s->max_rows)
        return fail(Q38_EINVAL, "staged verification exceeds the slot's row capacity");
    Q38_HIP(hipMemcpyAsync(s->rows[s->stage_buf], h, static_cast<size_t>(draft_count + 1) * s->hidden * 2,
                           hipMemcpyDeviceToDevice, static_cast<hipStream_t>(stream)));
    s->staged_rows = draft_count + 1;
    s->draft_count = draft_count;
    s->stages += 1;
    return Q38_OK;
}
int q38_slot_commit(q38_slot* s, int64_t accepted, void* stream) {
    (void)stream;
    if (!s) return fail(Q38_EINVAL, "null slot");
    if (s->staged_rows == 0 || s->staged_rows != s->draft_count + 1)
        return fail(Q38_ESTATE, "MTP verification row count is invalid");
    if (accepted < 0 || accepted > s->draft_count)
        return fail(Q38_ESTATE, "MTP accepted count exceeds verified draft count");
    s->committed = s->rows[s->stage_buf] + static_cast<size_t>(accepted) * s->hidden;
    s->stage_buf ^= 1;
    s->token_count += static_cast<uint64_t>(accepted) + 1;
    s->staged_rows = 0;
    s->draft_count = 0;
    s->has_hidden = true;
    return Q38_OK;
}
int q38_slot_rollback(q38_slot* s) {
    if (!s) return fail(Q38_EINVAL, "null slot");
    s->staged_rows = 0;
    s->draft_count = 0;
    return Q38_OK;
}
int q38_slot_info(const q38_slot* s, uint64_t* token_count, int32_t* staged_rows, int32_t* draft_count) {
    if (!s) return fail(Q38_EINVAL, "null slot");
    if (token_count) *token_count = s->token_count;
    if (staged_rows) *staged_rows = s->staged_rows;
    if (draft_count) *draft_count = s->draft_count;
    return Q38_OK;
}
const uint16_t* q38_slot_hidden(const q38_slot* s) { return s && s->has_hidden ? s->committed : nullptr; }
uint64_t q38_slot_generation(const q38_slot* s) { return s && s->staged_rows > 0 ? s->stages : 0; }

// ------------------------------------------------------------------ HyperConnection mixer
static int hc_validate(const q38_hc_desc* d) {
    if (!d) return fail(Q38_EINVAL, "null HyperConnection description");
    if (d->hidden <= 0 || d->hidden % 256 || d->hidden > 256 * kHcMaxPerThread)
        return fail(Q38_EINVAL, "HyperConnection hidden size must be a positive multiple of 256, at most 4096");
    if (d->streams < 1 || d->streams > kHcMaxStreams) return fail(Q38_EINVAL, "HyperConnection stream count must be 1..16");
    if (d->bits != 4 && d->bits != 8) return fail(Q38_EINVAL, "HyperConnection projections must be 4- or 8-bit affine");
    if (d->group != 32 && d->group != 64 && d->group != 128)
        return fail(Q38_EINVAL, "HyperConnection quantization group must be 32, 64 or 128");
    if (d->rank <= 0 || d->rank > kHcMaxRank || d->rank % d->group || d->rank % (128 / d->bits))
        return fail(Q38_EINVAL, "HyperConnection rank must be a multiple of the group and of 128 / bits, at most 512");
    if (!(d->eps > 0.0f)) return fail(Q38_EINVAL, "RMS norm epsilon must be positive");
    return Q38_OK;
}

int q38_hc_create(q38_ctx* ctx, const q38_hc_desc* d, const q38_hc_weights* w, q38_hc** out) {
    if (!ctx || !w || !out) return fail(Q38_EINVAL, "q38_hc_create: null argument");
    if (int rc = hc_validate(d)) return rc;
    if (!w->norm || !w->down_w || !w->down_s || !w->down_b || !w->up_w || !w->up_s || !w->up_b)
        return fail(Q38_EINVAL, "q38_hc_create: norm, down and up tensors are required");
    if (d->with_injection && (!w->inj_w || !w->inj_s || !w->inj_b))
        return fail(Q38_EINVAL, "q38_hc_create: a mixer with injection needs block_inject_weight tensors");
    const uintptr_t a = reinterpret_cast<uintptr_t>(w->up_w);
    if (a % 16) return fail(Q38_EINVAL, "q38_hc_create: input_mix_weight_up must be 16-byte aligned");
    const int n = d->streams * d->hidden;
    uint16_t* wn = nullptr;
    if (hipMalloc(&wn, static_cast<size_t>(n) * 2) != hipSuccess)
        return fail(Q38_ENOMEM, "hipMalloc failed for the HyperConnection norm weight");
    hipError_t e = launch_hc_norm_weight(w->norm, n, wn, nullptr);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        (void)hipFree(wn);
        return hip_fail(e, "HyperConnection norm weight");
    }
    auto* hc = new q38_hc{ctx, *d, {}, wn};
    hc->dev = HcDev{d->hidden, d->streams, d->rank, d->bits, d->group, d->with_injection ? 1 : 0, d->eps, wn,
                    w->down_w, w->down_s, w->down_b, w->up_w, w->up_s, w->up_b,
                    d->with_injection ? w->inj_w : nullptr, d->with_injection ? w->inj_s : nullptr,
                    d->with_injection ? w->inj_b : nullptr};
    *out = hc;
    return Q38_OK;
}

void q38_hc_destroy(q38_hc* hc) {
    if (!hc) return;
    (void)hipFree(hc->wn);
    delete hc;
}

static size_t hc_workspace(const q38_hc_desc& d, int rows) {
    return align256(static_cast<size_t>(rows) * d.streams * d.hidden * 2) + align256(static_cast<size_t>(rows) * d.rank * 4);
}

size_t q38_hc_workspace_size(const q38_hc_desc* d, int32_t max_rows) {
    if (hc_validate(d) || max_rows < 1 || max_rows > kMaxRows) return 0;
    return hc_workspace(*d, max_rows);
}

int q38_hc_read(q38_hc* hc, const uint16_t* stream, int32_t rows, uint16_t* mixed, uint16_t* injection, void* ws,
                size_t ws_bytes, void* st) {
    if (!hc || !stream || !mixed || !ws) return fail(Q38_EINVAL, "q38_hc_read: null argument");
    if (rows < 1 || rows > kMaxRows) return fail(Q38_EINVAL, "q38_hc_read: rows must be 1..16");
    if (hc->desc.with_injection && !injection) return fail(Q38_EINVAL, "q38_hc_read: this mixer returns an injection");
    const size_t need = hc_workspace(hc->desc, rows);
    if (ws_bytes < need) return fail(Q38_ESPACE, "q38_hc_read: workspace too small");
    if (reinterpret_cast<uintptr_t>(stream) % 16) return fail(Q38_EINVAL, "q38_hc_read: stream must be 16-byte aligned");
    auto* xn = static_cast<uint16_t*>(ws);
    auto* act = reinterpret_cast<float*>(static_cast<char*>(ws) +
                                         align256(static_cast<size_t>(rows) * hc->desc.streams * hc->desc.hidden * 2));
    Q38_HIP(launch_hc_read(hc->dev, rows, stream, xn, act, mixed, injection, static_cast<hipStream_t>(st)));
    return Q38_OK;
}

int q38_hc_write(const q38_hc* hc, const uint16_t* stream, const uint16_t* block_output, const uint16_t* injection,
                 int32_t rows, uint16_t* out, void* st) {
    if (!hc || !stream || !block_output || !injection || !out) return fail(Q38_EINVAL, "q38_hc_write: null argument");
    if (rows < 1 || rows > kMaxPrefillRows) return fail(Q38_EINVAL, "q38_hc_write: rows must be 1..2048");
    if ((reinterpret_cast<uintptr_t>(stream) | reinterpret_cast<uintptr_t>(block_output) |
         reinterpret_cast<uintptr_t>(out)) % 16)
        return fail(Q38_EINVAL, "q38_hc_write: stream, block output and out must be 16-byte aligned");
    Q38_HIP(launch_hc_write(hc->desc.hidden, hc->desc.streams, rows, stream, block_output, injection, out,
                            static_cast<hipStream_t>(st)));
    return Q38_OK;
}

// Workspace of the mixer chain: the largest layer's MoE workspace, then the mixer's (xn,
// act), the block input and the injection gates (the layer output goes straight into the
// streams).
static size_t chain_hc_ws(size_t moe_bytes, const q38_hc_desc& hd, int rows, char* base, uint16_t** mixed,
                          uint16_t** inj, void** hcws) {
    size_t off = align256(moe_bytes);
    if (hcws) *hcws = base + off;
    off += hc_workspace(hd, rows);
    if (mixed) *mixed = reinterpret_cast<uint16_t*>(base + off);
    off += align256(static_cast<size_t>(rows) * hd.hidden * 2);
    if (inj) *inj = reinterpret_cast<uint16_t*>(base + off);
    off += align256(static_cast<size_t>(rows) * hd.streams * 2);
    return off;
}

size_t q38_verify_chain_hc_workspace_size(const q38_moe_desc* d, const q38_hc_desc* hd, int32_t max_rows) {
    if (!d || hc_validate(hd) || max_rows < 1 || max_rows > kMaxRows) return 0;
    return chain_hc_ws(moe_ws(*d, max_rows, nullptr, nullptr), *hd, max_rows, nullptr, nullptr, nullptr, nullptr);
}

int q38_verify_chain_hc(q38_moe_layer* const* layers, q38_hc* const* mixers, int32_t n_layers, uint16_t* stream,
                        int32_t rows, void* ws, size_t ws_bytes, void* hip_stream) {
    if (!layers || !mixers || n_layers < 1 || !stream || !ws) return fail(Q38_EINVAL, "q38_verify_chain_hc: bad arguments");
    if (int rc = check_rows(rows)) return rc;
    if (reinterpret_cast<uintptr_t>(stream) % 16) return fail(Q38_EINVAL, "q38_verify_chain_hc: stream must be 16-byte aligned");
    size_t moe_need = 0;
    for (int l = 0; l < n_layers; ++l) {
        if (!layers[l] || !mixers[l]) return fail(Q38_EINVAL, "q38_verify_chain_hc: null layer or mixer");
        const q38_hc_desc& hd = mixers[l]->desc;
        if (layers[l]->desc.hidden != hd.hidden || hd.hidden != mixers[0]->desc.hidden ||
            hd.streams != mixers[0]->desc.streams || hd.rank != mixers[0]->desc.rank)
            return fail(Q38_EINVAL, "q38_verify_chain_hc: layers and mixers disagree on the hidden size, streams or rank");
        if (!hd.with_injection) return fail(Q38_EINVAL, "q38_verify_chain_hc: a decoder mixer carries injection weights");
        moe_need = std::max(moe_need, moe_ws(layers[l]->desc, rows, nullptr, nullptr));
    }
    char* base = static_cast<char*>(ws);
    uint16_t *mixed = nullptr, *inj = nullptr;
    void* hcws = nullptr;
    if (ws_bytes < chain_hc_ws(moe_need, mixers[0]->desc, rows, base, &mixed, &inj, &hcws))
        return fail(Q38_ESPACE, "workspace too small");
    const hipStream_t st = static_cast<hipStream_t>(hip_stream);
    const q38_hc_desc& hd0 = mixers[0]->desc;
    auto* xn = static_cast<uint16_t*>(hcws);
    auto* act = reinterpret_cast<float*>(static_cast<char*>(hcws) +
                                         align256(static_cast<size_t>(rows) * hd0.streams * hd0.hidden * 2));
    for (int l = 0; l < n_layers; ++l) {
        Q38_HIP(launch_hc_read(mixers[l]->dev, rows, stream, xn, act, mixed, inj, st));
        MoeBufs w{};
        moe_ws(layers[l]->desc, rows, &w, ws);
        // the MoE layer on the block input; its combine writes the output into the streams
        const LayerDev dev = moe_call_dev(layers[l]->dev, rows);
        const LayerDev ex = expert_view(dev);
        Q38_HIP(launch_router(dev, w, rows, mixed, false, 0.0f, st));
        Q38_HIP(launch_shared_affine(dev, w, rows, st));
        if (!moe_plans_in_gate_up(ex, rows)) Q38_HIP(launch_topk_plan(ex, w, rows, st));
        if (moe_uses_fused(ex, rows) && !dev.shared_affine) {
            // gate/up, down and the combine into the streams in one launch
            Q38_HIP(launch_gate_down4(ex, w, rows, stream, nullptr, st, inj, hd0.streams));
            continue;
        }
        Q38_HIP(launch_gate_up(ex, w, rows, st));
        Q38_HIP(launch_down(ex, w, rows, st));
        Q38_HIP(launch_combine_hc(dev, w, rows, stream, inj, hd0.streams, st));
    }
    return Q38_OK;
}

static int map_check(const q38_mlp_map* m, int hidden) {
    if (!m) return fail(Q38_EINVAL, "null MLP output map");
    if (m->hidden != hidden || hidden <= 0) return fail(Q38_EINVAL, "MLP output map hidden size mismatch");
    if (m->rank < 0 || m->rank > hidden) return fail(Q38_EINVAL, "invalid Niwaki low-rank map geometry");
    if (m->rank == 0 ? !m->full : (!m->left || !m->right)) return fail(Q38_EINVAL, "incomplete Niwaki low-rank map pair");
    return Q38_OK;
}
static MlpMapDev map_dev(const q38_mlp_map* m) { return MlpMapDev{m->hidden, m->rank, m->full, m->left, m->right}; }

size_t q38_mlp_map_workspace_size(const q38_mlp_map* map, int32_t max_rows) {
    if (!map || max_rows < 1 || max_rows > kMaxRows || map->hidden <= 0 || map->rank < 0 || map->rank > map->hidden)
        return 0;
    return mlp_map_workspace(map->hidden, map->rank, max_rows);
}

int q38_mlp_output_map(const q38_mlp_map* map, const uint16_t* y, int32_t rows, uint16_t* out, void* ws,
                       size_t ws_bytes, void* stream) {
    if (!map || !y || !out || !ws) return fail(Q38_EINVAL, "q38_mlp_output_map: null argument");
    if (int rc = map_check(map, map->hidden)) return rc;
    if (int rc = check_rows(rows)) return rc;
    if (out == y) return fail(Q38_EINVAL, "q38_mlp_output_map: out must not alias y");
    if (ws_bytes < mlp_map_workspace(map->hidden, map->rank, rows)) return fail(Q38_ESPACE, "workspace too small");
    Q38_HIP(launch_mlp_map(map_dev(map), y, rows, out, ws, static_cast<hipStream_t>(stream)));
    return Q38_OK;
}

size_t q38_verify_chain_hc_mapped_workspace_size(const q38_moe_desc* d, const q38_hc_desc* hd, int32_t max_rows) {
    const size_t base = q38_verify_chain_hc_workspace_size(d, hd, max_rows);
    if (!base) return 0;
    // the MoE output, the mapped output and the map's scratch (a full map is the largest)
    const size_t H = static_cast<size_t>(hd->hidden), R = static_cast<size_t>(max_rows);
    return base + 2 * align256(R * H * 2) + mlp_map_workspace(hd->hidden, 0, max_rows);
}

int q38_verify_chain_hc_mapped(q38_moe_layer* const* layers, q38_hc* const* mixers, const q38_mlp_map* const* maps,
                               int32_t n_layers, uint16_t* stream, int32_t rows, void* ws, size_t ws_bytes,
                               void* hip_stream) {
    if (!maps) return q38_verify_chain_hc(layers, mixers, n_layers, stream, rows, ws, ws_bytes, hip_stream);
    if (!layers || !mixers || n_layers < 1 || !stream || !ws) return fail(Q38_EINVAL, "q38_verify_chain_hc: bad arguments");
    if (int rc = check_rows(rows)) return rc;
    if (!mixers[0] || !layers[0]) return fail(Q38_EINVAL, "q38_verify_chain_hc: null layer or mixer");
    for (int l = 0; l < n_layers; ++l)
        if (maps[l])
            if (int rc = map_check(maps[l], mixers[0]->desc.hidden)) return rc;
    const size_t need = q38_verify_chain_hc_mapped_workspace_size(&layers[0]->desc, &mixers[0]->desc, rows);
    size_t chain_need = 0;
    for (int l = 0; l < n_layers; ++l) {
        if (!layers[l]) return fail(Q38_EINVAL, "q38_verify_chain_hc: null layer or mixer");
        chain_need = std::max(chain_need, q38_verify_chain_hc_workspace_size(&layers[l]->desc, &mixers[0]->desc, rows));
    }
    const size_t H = static_cast<size_t>(mixers[0]->desc.hidden);
    const size_t extra = 2 * align256(static_cast<size_t>(rows) * H * 2) + mlp_map_workspace(static_cast<int>(H), 0, rows);
    if (ws_bytes < std::max(need, chain_need + extra)) return fail(Q38_ESPACE, "workspace too small");
    char* base = static_cast<char*>(ws);
    const size_t chain_bytes = align256(chain_need);
    uint16_t* y = reinterpret_cast<uint16_t*>(base + chain_bytes);
    uint16_t* ym = reinterpret_cast<uint16_t*>(base + chain_bytes + align256(static_cast<size_t>(rows) * H * 2));
    void* mws = base + chain_bytes + 2 * align256(static_cast<size_t>(rows) * H * 2);
    const hipStream_t st = static_cast<hipStream_t>(hip_stream);
    for (int l = 0; l < n_layers; ++l) {
        if (!maps[l]) {  // the fused path for this layer
            if (int rc = q38_verify_chain_hc(layers + l, mixers + l, 1, stream, rows, ws, chain_bytes, hip_stream))
                return rc;
            continue;
        }
        if (!mixers[l]) return fail(Q38_EINVAL, "q38_verify_chain_hc: null layer or mixer");
        const q38_hc_desc& hd = mixers[l]->desc;
        if (layers[l]->desc.hidden != hd.hidden || hd.hidden != mixers[0]->desc.hidden ||
            hd.streams != mixers[0]->desc.streams || hd.rank != mixers[0]->desc.rank || !hd.with_injection)
            return fail(Q38_EINVAL, "q38_verify_chain_hc: layers and mixers disagree on the hidden size, streams or rank");
        uint16_t *mixed = nullptr, *inj = nullptr;
        void* hcws = nullptr;
        const size_t moe_need = moe_ws(layers[l]->desc, rows, nullptr, nullptr);
        chain_hc_ws(moe_need, hd, rows, base, &mixed, &inj, &hcws);
        auto* xn = static_cast<uint16_t*>(hcws);
        auto* act = reinterpret_cast<float*>(static_cast<char*>(hcws) +
                                             align256(static_cast<size_t>(rows) * hd.streams * hd.hidden * 2));
        Q38_HIP(launch_hc_read(mixers[l]->dev, rows, stream, xn, act, mixed, inj, st));
        MoeBufs w{};
        moe_ws(layers[l]->desc, rows, &w, ws);
        const LayerDev dev = moe_call_dev(layers[l]->dev, rows);
        const LayerDev ex = expert_view(dev);
        Q38_HIP(launch_router(dev, w, rows, mixed, false, 0.0f, st));
        Q38_HIP(launch_shared_affine(dev, w, rows, st));
        if (!moe_plans_in_gate_up(ex, rows)) Q38_HIP(launch_topk_plan(ex, w, rows, st));
        Q38_HIP(launch_gate_up(ex, w, rows, st));
        Q38_HIP(launch_down(ex, w, rows, st));
        Q38_HIP(launch_combine(dev, w, rows, nullptr, y, st));
        Q38_HIP(launch_mlp_map(map_dev(maps[l]), y, rows, ym, mws, st));
        Q38_HIP(launch_hc_write(hd.hidden, hd.streams, rows, stream, ym, inj, stream, st));
    }
    return Q38_OK;
}

int q38_hc_initialize_stream(const uint16_t* embedding, int32_t rows, int32_t hidden, int32_t streams, uint16_t* out,
                             void* st) {
    if (!embedding || !out || rows < 1 || rows > kMaxPrefillRows || hidden < 8 || hidden % 8 || streams < 1 ||
        streams > kHcMaxStreams)
        return fail(Q38_EINVAL, "q38_hc_initialize_stream: bad arguments");
    if ((reinterpret_cast<uintptr_t>(embedding) | reinterpret_cast<uintptr_t>(out)) % 16)
        return fail(Q38_EINVAL, "q38_hc_initialize_stream: embedding and out must be 16-byte aligned");
    Q38_HIP(launch_hc_tile(hidden, streams, rows, embedding, out, static_cast<hipStream_t>(st)));
    return Q38_OK;
}

} // extern "C"

#ifdef Q38_TRACE
// Phase stamps of the Q38_TRACE build (see q38_moe_dev.hpp).
namespace q38 {
__device__ unsigned long long g_trace[32768];
}
extern "C" int q38_trace_read(unsigned long long* out) {
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(q38::g_trace), sizeof(unsigned long long) * 32768) == hipSuccess
               ? 0
               : -1;
}
#endif
