// qwen38_engine.hpp — engine-side MTP round driver for several requests (slots) at once.
//
// Each round, every unfinished slot picks its proposal the way the reference engine's
// greedy generation loop does (src/native_engine.cpp:1404-1680): a serial decode row once
// MTP stopped paying (or with one token left), else a prompt context copy (opt-in), else
// history drafts while HistoryDraftPolicy admits them, else the learned drafter at
// MtpDepthPolicy's depth. Unlike the reference, which runs one request's round at a time and
// batches only serial decode rows across requests (src/native_engine.cpp:725-771), all slots'
// verify rows [current, drafts...] are packed into one batched verification (up to the
// verifier's row width, 16 on the MI355X verify kernels), so one pass over the expert weights
// serves every slot. After the pass each slot decides (decide_mtp_greedy), commits its own
// checkpoint and feeds its policies exactly as the reference loop does.
//
// Host-only C++20; the device side is behind BatchVerifier (QwenBatchVerifier in
// qwen38_verify.hpp verifies on the GPU).
#pragma once

#include "qwen38_policy.hpp"

#include <cstddef>
#include <cstdint>
#include <optional>
#include <span>
#include <string>
#include <vector>

namespace qwen38 {

// One slot's rows of a batched verification: [current_token, drafts...] (drafts may be
// empty: a serial decode row).
struct SlotVerifyRows {
    std::size_t slot{0};
    std::uint32_t current_token{0};
    std::vector<std::uint32_t> drafts;
};

// Verifies several slots' rows in one pass. verify() stages each slot's checkpoints and
// returns, per entry of `batch`, the greedy target token of each of its rows (drafts + 1);
// commit() keeps checkpoint `accepted` of that slot's last verification.
class BatchVerifier {
public:
    virtual ~BatchVerifier() = default;
    [[nodiscard]] virtual std::size_t max_rows() const = 0;
    [[nodiscard]] virtual std::vector<std::vector<std::uint32_t>> verify(std::span<const SlotVerifyRows> batch) = 0;
    virtual void commit(std::size_t slot, std::size_t accepted) = 0;
};

struct DraftRequest {
    std::size_t slot{0};
    std::uint32_t current_token{0};
    std::size_t depth{0};
};

// The learned drafter (the MTP draft head's role): up to `depth` drafts following
// current_token for the slot. propose_batch serves every learned slot of a round at once
// (by default one propose() per request).
class LearnedDrafter {
public:
    virtual ~LearnedDrafter() = default;
    [[nodiscard]] virtual std::vector<std::uint32_t> propose(std::size_t slot, std::uint32_t current_token,
                                                             std::size_t depth) = 0;
    [[nodiscard]] virtual std::vector<std::vector<std::uint32_t>> propose_batch(std::span<const DraftRequest> requests) {
        std::vector<std::vector<std::uint32_t>> out;
        out.reserve(requests.size());
        for (const DraftRequest& r : requests) out.push_back(propose(r.slot, r.current_token, r.depth));
        return out;
    }
};

enum class DraftSourceKind { serial, learned, history, context_copy };

struct MtpSchedulerOptions {
    std::size_t mtp_depth{3};                  // 0 or 2..4 (MtpDepthPolicy)
    bool adaptive_depth_four{false};
    HistoryDraftMode history_mode{HistoryDraftMode::adaptive};
    bool context_copy{false};                  // prompt copies (opt-in, as QWEN38_CONTEXT_COPY=1)
    std::size_t context_copy_max_tokens{16};   // 4..24
    bool long_history_depth_four{true};        // history drafts of 4 once the context holds 512 tokens
    std::size_t zero_accept_fallback_rounds{2};
    bool economic_fallback{true};              // MtpProfitabilityGuard (else the zero-accept streak alone)
    std::vector<std::uint32_t> stop_tokens;
};

struct SlotStats {
    std::size_t mtp_rounds{0}, mtp_proposed{0}, mtp_accepted{0}, mtp_fallbacks{0};
    std::size_t serial_steps{0};
    std::size_t history_draft_rounds{0}, history_draft_proposed{0}, history_draft_accepted{0};
    std::size_t history_draft_activations{0}, history_draft_deactivations{0};
    std::size_t context_copy_rounds{0}, context_copy_proposed{0}, context_copy_accepted{0};
    std::size_t context_copy_suspensions{0};
    std::size_t mtp_final_depth{0}, mtp_promotions{0}, mtp_demotions{0};
    std::string finish_reason;                 // "", "stop" or "length"
};

struct SlotRound {
    std::size_t slot{0};
    DraftSourceKind source{DraftSourceKind::serial};
    std::vector<std::uint32_t> draft_tokens;
    std::size_t accepted{0};
    std::vector<std::uint32_t> emitted_tokens;  // as committed (before max-token / stop truncation)
};

class MtpSlotScheduler final {
public:
    MtpSlotScheduler(BatchVerifier& verifier, LearnedDrafter* drafter, MtpSchedulerOptions options);

    // A request prefilled into the verifier's slot `slot`: the slot's state holds
    // query_position tokens and the prompt's last token is the current token, not yet in the
    // state (src/native_engine.cpp:1232). Returns the scheduler's index of the request.
    std::size_t add_request(std::size_t slot, std::span<const std::uint32_t> prompt, std::size_t query_position,
                            std::size_t max_tokens);

    // One round over every unfinished request (one or more batched verifications).
    std::vector<SlotRound> step();
    [[nodiscard]] bool done() const noexcept;

    [[nodiscard]] const std::vector<std::uint32_t>& tokens(std::size_t request) const { return at(request).tokens; }
    [[nodiscard]] const SlotStats& stats(std::size_t request) const { return at(request).stats; }
    [[nodiscard]] std::uint32_t current_token(std::size_t request) const { return at(request).current; }
    [[nodiscard]] std::size_t query_position(std::size_t request) const { return at(request).position; }
    [[nodiscard]] std::size_t batches() const noexcept { return batches_; }

private:
    struct Request {
        std::size_t slot{0};
        std::uint32_t current{0};
        std::size_t position{0};
        std::size_t max_tokens{0};
        std::vector<std::uint32_t> tokens;
        bool finished{false};
        bool mtp_profitable{true};
        MtpDepthPolicy depth;
        MtpProfitabilityGuard guard;
        HistoryDraftPolicy history_policy;
        HistoryDraftCache history;
        std::optional<ContextCopyCache> copy;
        std::size_t copy_seen{0}, copy_perfect{0}, copy_suspend_until{0}, copy_backoff{64};
        double copy_ema{0.5};
        SlotStats stats;
        Request(std::size_t max_depth, std::size_t prompt_tokens, bool adaptive_four, HistoryDraftMode mode)
            : depth(max_depth, prompt_tokens, adaptive_four), history_policy(mode) {}
    };
    struct Plan {
        std::size_t request;
        DraftSourceKind source;
        std::vector<std::uint32_t> drafts;
        bool wants_learned{false};  // learned drafts to be filled in by the round's batch request
    };

    [[nodiscard]] const Request& at(std::size_t request) const;
    Plan plan(std::size_t request);
    SlotRound finish(const Plan& p, std::span<const std::uint32_t> targets);
    [[nodiscard]] bool is_stop(std::uint32_t token) const noexcept;

    BatchVerifier& verifier_;
    LearnedDrafter* drafter_;
    MtpSchedulerOptions opt_;
    std::vector<Request> requests_;
    std::size_t batches_{0};
};

} // namespace qwen38
