// ref_shim.cpp — C entry points over the reference's own model-free sources, compiled
// directly from /root/reference (src/quantization_geometry.cpp, src/mtp_lifecycle.cpp)
// into oracle/_ref/libq38_ref.so. TEST INFRASTRUCTURE ONLY: tests use it to pin the CPU
// restatement in q38_oracle.cpp against the reference's compiled code.
#include "qwen38/mtp_lifecycle.hpp"
#include "qwen38/quantization_geometry.hpp"

#include <cstdint>
#include <span>
#include <stdexcept>

extern "C" {

int64_t ref_packed_vq_word_count(int64_t n, int bits) {
    try {
        return static_cast<int64_t>(qwen38::packed_vq_word_count(static_cast<std::size_t>(n),
                                                                 static_cast<std::size_t>(bits)));
    } catch (const std::exception&) {
        return -1;
    }
}

// 0 ok, -1 runtime_error, -2 out_of_range (short buffer).
int ref_unpack_vq_code(const uint32_t* words, int64_t nwords, int64_t index, int bits, uint32_t* out) {
    try {
        *out = qwen38::unpack_vq_code(std::span<const uint32_t>(words, static_cast<std::size_t>(nwords)),
                                      static_cast<std::size_t>(index), static_cast<std::size_t>(bits));
        return 0;
    } catch (const std::out_of_range&) {
        return -2;
    } catch (const std::exception&) {
        return -1;
    }
}

int ref_supports_segmented_vq(int dim, int bits) { return qwen38::supports_segmented_vq(dim, bits) ? 1 : 0; }

int ref_decide_greedy(const uint32_t* drafts, int64_t k, const uint32_t* target, int64_t ntarget,
                      const uint32_t* stop, int64_t nstop, int64_t* accepted, int64_t* row, uint32_t* next) {
    try {
        const auto d = qwen38::decide_mtp_greedy(
            std::span<const uint32_t>(drafts, static_cast<std::size_t>(k)),
            std::span<const uint32_t>(target, static_cast<std::size_t>(ntarget)),
            std::span<const uint32_t>(stop, static_cast<std::size_t>(nstop)));
        *accepted = static_cast<int64_t>(d.accepted);
        *row = static_cast<int64_t>(d.correction_row);
        *next = d.next_token;
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

int ref_plan_commit(uint64_t round_offset, uint64_t drafted, uint64_t accepted, uint64_t* out) {
    try {
        const auto p = qwen38::plan_mtp_commit(round_offset, drafted, accepted);
        out[0] = p.truncate_head_to;
        out[1] = p.target_rows_to_keep;
        out[2] = p.stash_rows;
        out[3] = p.committed_boundary;
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

} // extern "C"
