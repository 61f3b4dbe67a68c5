// qwen38_policy.hpp — engine-side policy of the MTP round: how deep to draft, when drafting
// stops paying, and where non-learned drafts come from. Host-only C++20 (no device code).
//
// Same names, argument meaning and error behaviour as the reference's interfaces:
//   MtpDepthPolicy                              include/qwen38/mtp_depth_policy.hpp:7-37
//                                               (behaviour src/mtp_depth_policy.cpp:9-140)
//   should_fallback_mtp, cache_mtp_as_profitable,
//   MtpProfitabilityGuard                       include/qwen38/mtp_profitability.hpp:12-72
//   HistoryDraftMode, HistoryDraftPolicy,
//   HistoryDraftCache, ContextCopyProposal,
//   ContextCopyCache                            include/qwen38/history_draft.hpp:10-105
//                                               (behaviour src/history_draft.cpp:1-266)
// Environment switches read by the reference at the same points are read here too:
// QWEN38_MTP_ADAPTIVE_DEPTH4 (construction), QWEN38_MTP_DEMOTION and
// QWEN38_MTP_EARLY_DEMOTION (each observation).
#pragma once

#include <array>
#include <cstddef>
#include <cstdint>
#include <span>
#include <unordered_map>
#include <vector>

namespace qwen38 {

// Draft depth of the learned MTP drafter, adapted to measured acceptance. Depth 3 starts at
// 2 and probes for 8 rounds (promotion to 3 at >= 10 accepted tokens) on prompts of at most
// 2048 tokens; depth 3 is watched in 12-round windows (two losing windows in a row demote to
// 2); an adaptive depth 4 is watched in 4-round probation and 8-round windows on how often
// all four drafts were accepted (demotion to 3).
class MtpDepthPolicy final {
public:
    MtpDepthPolicy(std::size_t maximum_depth, std::size_t prompt_tokens, bool adaptive_depth_four = false);

    [[nodiscard]] std::size_t depth() const noexcept { return depth_; }
    [[nodiscard]] std::size_t promotions() const noexcept { return promotions_; }
    [[nodiscard]] std::size_t demotions() const noexcept { return demotions_; }
    [[nodiscard]] bool probing() const noexcept { return phase_ == Phase::probing; }

    // One learned round: `proposed` drafts verified, `accepted` of them kept.
    void observe(std::size_t proposed, std::size_t accepted);

private:
    enum class Phase : std::uint8_t { fixed, probing, watch_four, watch_three };
    struct Window {
        std::size_t rounds{0}, proposed{0}, accepted{0}, all_four{0};
        void clear() noexcept { *this = Window{}; }
    };
    void observe_probe(std::size_t accepted);
    void observe_four(std::size_t proposed, std::size_t accepted);
    void observe_three(std::size_t proposed, std::size_t accepted);
    void demote_to(std::size_t depth, Phase next) noexcept;

    std::size_t maximum_depth_{0};
    std::size_t depth_{0};
    Phase phase_{Phase::fixed};
    Window probe_{}, window_{};
    bool four_probation_passed_{false};
    bool three_probation_passed_{false};
    std::size_t losing_windows_{0};
    std::size_t promotions_{0};
    std::size_t demotions_{0};
};

// True when a zero-accept streak of at least `fallback_streak` rounds is evidence of a losing
// drafter: the request has not reached one accepted token per round on average.
[[nodiscard]] inline bool should_fallback_mtp(std::size_t zero_accept_streak, std::size_t fallback_streak,
                                              std::size_t rounds, std::size_t accepted) noexcept {
    if (zero_accept_streak < fallback_streak) return false;
    return accepted < rounds;
}

// Whether a completed request's MTP use is remembered as profitable for an exact-prefix
// replay: it never fell back, or it accepted at least one token per round overall.
[[nodiscard]] inline bool cache_mtp_as_profitable(std::size_t rounds, std::size_t accepted,
                                                  std::size_t fallbacks) noexcept {
    if (fallbacks == 0) return true;
    return rounds != 0 && accepted >= rounds;
}

// Break-even guard on the learned drafter: before 16 rounds have been seen it falls back on
// a zero-accept streak (should_fallback_mtp); afterwards when the last 16 rounds accepted
// fewer than 16 tokens.
class MtpProfitabilityGuard final {
public:
    static constexpr std::size_t window_size = 16;

    void observe(std::size_t accepted) noexcept;
    [[nodiscard]] bool should_fallback(std::size_t fallback_streak) const noexcept;

    [[nodiscard]] std::size_t rounds() const noexcept { return rounds_; }
    [[nodiscard]] std::size_t total_accepted() const noexcept { return total_; }
    [[nodiscard]] std::size_t window_accepted() const noexcept { return window_sum_; }
    [[nodiscard]] std::size_t zero_accept_streak() const noexcept { return streak_; }

private:
    std::array<std::size_t, window_size> ring_{};
    std::size_t rounds_{0}, total_{0}, window_sum_{0}, streak_{0};
};

enum class HistoryDraftMode {
    disabled,
    adaptive,
    forced,
};

// Admission of history (n-gram) drafts: in adaptive mode they are tried once 8 learned
// rounds accepted less than half of what they proposed, and withdrawn for good once 2
// history rounds do the same. Forced mode always tries them; disabled never does.
class HistoryDraftPolicy final {
public:
    explicit HistoryDraftPolicy(HistoryDraftMode mode = HistoryDraftMode::adaptive)
        : mode_(mode), active_(mode == HistoryDraftMode::forced) {}

    [[nodiscard]] bool enabled() const noexcept { return mode_ != HistoryDraftMode::disabled; }
    [[nodiscard]] bool should_try() const noexcept { return active_; }
    [[nodiscard]] bool exhausted() const noexcept { return rejected_; }
    void observe_learned(std::size_t proposed, std::size_t accepted);
    void observe_history(std::size_t proposed, std::size_t accepted);

    [[nodiscard]] std::size_t activations() const noexcept { return activations_; }
    [[nodiscard]] std::size_t deactivations() const noexcept { return deactivations_; }

private:
    struct Tally {
        std::size_t rounds{0}, proposed{0}, accepted{0};
        // Adds one round; true (and cleared) when `limit` rounds are in and fewer than half of
        // the proposed tokens were accepted; cleared without verdict otherwise.
        bool add(std::size_t p, std::size_t a, std::size_t limit) noexcept;
    };
    HistoryDraftMode mode_;
    bool active_{false};
    bool rejected_{false};
    Tally learned_{}, history_{};
    std::size_t activations_{0};
    std::size_t deactivations_{0};
};

// Request-local suffix index of the token history for exact speculative proposals: after
// every appended token, each suffix of order min..max that ends just before it is recorded
// with the position it started at (latest wins), so a lookup never points at the suffix
// being queried. propose() takes the longest order whose current suffix was seen before and
// returns what followed it.
class HistoryDraftCache final {
public:
    explicit HistoryDraftCache(std::size_t minimum_order = 2, std::size_t maximum_order = 5);

    void append(std::uint32_t token);
    void append(std::span<const std::uint32_t> tokens);

    [[nodiscard]] std::vector<std::uint32_t> propose(std::size_t maximum_tokens) const;
    [[nodiscard]] std::size_t size() const noexcept { return tokens_.size(); }

private:
    [[nodiscard]] std::uint64_t suffix_key(std::size_t start, std::size_t order) const noexcept;
    [[nodiscard]] bool same_as_tail(std::size_t start, std::size_t order) const noexcept;

    std::size_t min_order_;
    std::size_t max_order_;
    std::vector<std::uint32_t> tokens_;
    std::unordered_map<std::uint64_t, std::size_t> last_start_;
};

struct ContextCopyProposal {
    std::vector<std::uint32_t> tokens;
    std::size_t match_extension{0};
};

// Prompt-only index for long exact copies: every prompt position p >= min is filed under
// the min-token window ending at p. A proposal continues the prompt after the most recent
// (of at most 32) windows equal to the history's last min tokens, preferring the one whose
// left context agrees with the history for longest (up to max - min extra tokens).
class ContextCopyCache final {
public:
    explicit ContextCopyCache(std::span<const std::uint32_t> prompt, std::size_t minimum_order = 6,
                              std::size_t maximum_order = 10);

    [[nodiscard]] ContextCopyProposal propose(std::span<const std::uint32_t> history,
                                              std::size_t maximum_tokens) const;
    // The same, with the history = prompt followed by `completion`.
    [[nodiscard]] ContextCopyProposal propose_completion(std::span<const std::uint32_t> completion,
                                                         std::size_t maximum_tokens) const;

private:
    template <typename TokenAt>
    [[nodiscard]] ContextCopyProposal lookup(std::size_t history_size, TokenAt&& at, std::size_t maximum_tokens) const;

    std::size_t min_order_;
    std::size_t max_order_;
    std::vector<std::uint32_t> prompt_;
    std::unordered_map<std::uint64_t, std::vector<std::size_t>> ends_;
};

} // namespace qwen38
