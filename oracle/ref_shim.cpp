// ref_shim.cpp — C entry points over the reference's own model-free sources, compiled
// directly from /root/reference (src/quantization_geometry.cpp, src/mtp_lifecycle.cpp,
// src/mtp_depth_policy.cpp, src/history_draft.cpp and the header-only
// include/qwen38/mtp_profitability.hpp) into oracle/_ref/libq38_ref.so. TEST
// INFRASTRUCTURE ONLY: tests use it to pin the CPU restatement in q38_oracle.cpp and the
// host round policy against the reference's compiled code.
#include "qwen38/history_draft.hpp"
#include "qwen38/mtp_depth_policy.hpp"
#include "qwen38/mtp_lifecycle.hpp"
#include "qwen38/mtp_profitability.hpp"
#include "qwen38/quantization_geometry.hpp"

#include <vector>

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

// ---- round policy (trajectories: the observable state after construction and each call)

// out[(i + 1) * 4 + {0..3}] = depth, promotions, demotions, probing after observation i;
// out[0..3] after construction. Returns 0, -1 when the constructor throws, or -(2 + i) when
// observation i throws.
int ref_depth_policy_run(uint64_t max_depth, uint64_t prompt_tokens, int adaptive4, const uint64_t* proposed,
                         const uint64_t* accepted, int64_t n, uint64_t* out) {
    try {
        qwen38::MtpDepthPolicy p(max_depth, prompt_tokens, adaptive4 != 0);
        auto put = [&](int64_t i) {
            out[i * 4 + 0] = p.depth();
            out[i * 4 + 1] = p.promotions();
            out[i * 4 + 2] = p.demotions();
            out[i * 4 + 3] = p.probing() ? 1 : 0;
        };
        put(0);
        for (int64_t i = 0; i < n; ++i) {
            try {
                p.observe(proposed[i], accepted[i]);
            } catch (const std::exception&) {
                return static_cast<int>(-(2 + i));
            }
            put(i + 1);
        }
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

// out[i * 5 + {0..4}] = rounds, total_accepted, window_accepted, zero_accept_streak,
// should_fallback(streak) after observation i.
int ref_guard_run(const uint64_t* accepted, int64_t n, uint64_t streak, uint64_t* out) {
    qwen38::MtpProfitabilityGuard g;
    for (int64_t i = 0; i < n; ++i) {
        g.observe(accepted[i]);
        out[i * 5 + 0] = g.rounds();
        out[i * 5 + 1] = g.total_accepted();
        out[i * 5 + 2] = g.window_accepted();
        out[i * 5 + 3] = g.zero_accept_streak();
        out[i * 5 + 4] = g.should_fallback(streak) ? 1 : 0;
    }
    return 0;
}

int ref_should_fallback_mtp(uint64_t streak, uint64_t fallback_streak, uint64_t rounds, uint64_t accepted) {
    return qwen38::should_fallback_mtp(streak, fallback_streak, rounds, accepted) ? 1 : 0;
}
int ref_cache_mtp_as_profitable(uint64_t rounds, uint64_t accepted, uint64_t fallbacks) {
    return qwen38::cache_mtp_as_profitable(rounds, accepted, fallbacks) ? 1 : 0;
}

// mode 0 disabled, 1 adaptive, 2 forced; kind[i] 0 = observe_learned, 1 = observe_history.
// out[i * 4 + {0..3}] = should_try, exhausted, activations, deactivations after call i.
// Returns 0, or -(1 + i) when call i throws.
int ref_history_policy_run(int mode, const int* kind, const uint64_t* proposed, const uint64_t* accepted,
                           int64_t n, uint64_t* out) {
    const qwen38::HistoryDraftMode m = mode == 0 ? qwen38::HistoryDraftMode::disabled
                                       : mode == 1 ? qwen38::HistoryDraftMode::adaptive
                                                   : qwen38::HistoryDraftMode::forced;
    qwen38::HistoryDraftPolicy p(m);
    for (int64_t i = 0; i < n; ++i) {
        try {
            if (kind[i] == 0) p.observe_learned(proposed[i], accepted[i]);
            else p.observe_history(proposed[i], accepted[i]);
        } catch (const std::exception&) {
            return static_cast<int>(-(1 + i));
        }
        out[i * 4 + 0] = p.should_try() ? 1 : 0;
        out[i * 4 + 1] = p.exhausted() ? 1 : 0;
        out[i * 4 + 2] = p.activations();
        out[i * 4 + 3] = p.deactivations();
    }
    return 0;
}

// After appending tokens[i], propose(max_tokens[i]): counts[i] tokens at out[i * cap].
// Returns 0, or -1 when the constructor throws.
int ref_history_cache_run(uint64_t min_order, uint64_t max_order, const uint32_t* tokens, int64_t n,
                          const uint64_t* max_tokens, uint64_t cap, uint32_t* out, uint64_t* counts) {
    try {
        qwen38::HistoryDraftCache c(min_order, max_order);
        for (int64_t i = 0; i < n; ++i) {
            c.append(tokens[i]);
            const std::vector<uint32_t> p = c.propose(max_tokens[i]);
            counts[i] = p.size();
            for (std::size_t j = 0; j < p.size() && j < cap; ++j) out[i * cap + j] = p[j];
        }
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

// ContextCopyCache(prompt, min, max).propose(history, max_tokens) (completion = 0) or
// .propose_completion(history, max_tokens) (completion = 1). Returns 0 or -1 (constructor).
int ref_context_copy(const uint32_t* prompt, int64_t np, uint64_t min_order, uint64_t max_order,
                     const uint32_t* history, int64_t nh, uint64_t max_tokens, int completion, uint64_t cap,
                     uint32_t* out, uint64_t* count, uint64_t* extension) {
    try {
        qwen38::ContextCopyCache c(std::span<const uint32_t>(prompt, static_cast<std::size_t>(np)), min_order,
                                   max_order);
        const std::span<const uint32_t> h(history, static_cast<std::size_t>(nh));
        const qwen38::ContextCopyProposal p = completion ? c.propose_completion(h, max_tokens) : c.propose(h, max_tokens);
        *count = p.tokens.size();
        *extension = p.match_extension;
        for (std::size_t j = 0; j < p.tokens.size() && j < cap; ++j) out[j] = p.tokens[j];
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

} // extern "C"
