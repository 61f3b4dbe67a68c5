// qwen38_engine.cpp — batched multi-slot MTP round driver (host only).
#include "qwen38_engine.hpp"

#include "qwen38_verify.hpp"

#include <algorithm>
#include <array>
#include <cstdlib>
#include <stdexcept>
#include <string_view>

namespace qwen38 {
namespace {

constexpr std::size_t kLongHistory = 512;  // context length from which history drafts go 4 deep
// Context-copy block length by match extension (extra left-context tokens that agree).
constexpr std::array<std::size_t, 5> kCopyBlock{8, 12, 16, 24, 24};

bool long_history_enabled() {
    const char* v = std::getenv("QWEN38_LONG_HISTORY_DEPTH4");
    return v == nullptr || std::string_view(v) != "0";
}

} // namespace

MtpSlotScheduler::MtpSlotScheduler(BatchVerifier& verifier, LearnedDrafter* drafter, MtpSchedulerOptions options)
    : verifier_(verifier), drafter_(drafter), opt_(std::move(options)) {
    if (opt_.context_copy && (opt_.context_copy_max_tokens < 4 || opt_.context_copy_max_tokens > 24))
        throw std::runtime_error("QWEN38_CONTEXT_COPY_MAX_TOKENS must be an integer from 4 to 24");
    if (verifier_.max_rows() < 1) throw std::runtime_error("batch verifier has no rows");
}

const MtpSlotScheduler::Request& MtpSlotScheduler::at(std::size_t request) const {
    if (request >= requests_.size()) throw std::out_of_range("unknown request");
    return requests_[request];
}

bool MtpSlotScheduler::is_stop(std::uint32_t token) const noexcept {
    return std::find(opt_.stop_tokens.begin(), opt_.stop_tokens.end(), token) != opt_.stop_tokens.end();
}

std::size_t MtpSlotScheduler::add_request(std::size_t slot, std::span<const std::uint32_t> prompt,
                                          std::size_t query_position, std::size_t max_tokens) {
    if (prompt.empty()) throw std::runtime_error("request prompt is empty");
    for (const Request& r : requests_)
        if (!r.finished && r.slot == slot) throw std::runtime_error("slot already holds an unfinished request");
    Request r(opt_.mtp_depth, prompt.size(), opt_.adaptive_depth_four, opt_.history_mode);
    r.slot = slot;
    r.current = prompt.back();
    r.position = query_position;
    r.max_tokens = max_tokens;
    r.mtp_profitable = drafter_ != nullptr && opt_.mtp_depth != 0;
    if (r.history_policy.enabled()) r.history.append(prompt);
    if (opt_.context_copy) r.copy.emplace(prompt);
    r.stats.mtp_final_depth = r.depth.depth();
    if (max_tokens == 0) {
        r.finished = true;
        r.stats.finish_reason = "length";
    }
    requests_.push_back(std::move(r));
    return requests_.size() - 1;
}

bool MtpSlotScheduler::done() const noexcept {
    return std::all_of(requests_.begin(), requests_.end(), [](const Request& r) { return r.finished; });
}

MtpSlotScheduler::Plan MtpSlotScheduler::plan(std::size_t index) {
    Request& r = requests_[index];
    Plan p{index, DraftSourceKind::serial, {}};
    const std::size_t remaining = r.max_tokens - r.tokens.size();
    if (!r.mtp_profitable || remaining == 1) return p;
    const std::size_t width = verifier_.max_rows() - 1;  // drafts that fit one verification
    if (width == 0) return p;
    const std::span<const std::uint32_t> completion(r.tokens);
    if (r.copy && r.tokens.size() >= r.copy_suspend_until) {
        const std::size_t cap =
            r.copy_perfect >= 2 && r.copy_ema >= 0.75 ? opt_.context_copy_max_tokens : std::size_t{4};
        ContextCopyProposal prop = r.copy->propose_completion(completion, std::min(cap, remaining));
        const std::size_t block = std::min(cap, kCopyBlock[std::min(prop.match_extension, kCopyBlock.size() - 1)]);
        if (prop.tokens.size() > block) prop.tokens.resize(block);
        if (prop.match_extension >= 2 && prop.tokens.size() >= 2) {
            if (prop.tokens.size() > width) prop.tokens.resize(width);
            p.source = DraftSourceKind::context_copy;
            p.drafts = std::move(prop.tokens);
            if (p.drafts.size() >= 2) return p;
            p.source = DraftSourceKind::serial;
            p.drafts.clear();
        }
    }
    if (r.history_policy.should_try()) {
        const bool four = opt_.long_history_depth_four && r.position >= kLongHistory && long_history_enabled();
        const std::size_t depth = four ? 4 : r.depth.depth();
        std::vector<std::uint32_t> prop = r.history.propose(std::min(depth, remaining));
        if (prop.size() < 2 && four) prop = r.history.propose(std::min(r.depth.depth(), remaining));
        if (prop.size() >= 2) {
            if (prop.size() > width) prop.resize(width);
            p.source = DraftSourceKind::history;
            p.drafts = std::move(prop);
            return p;
        }
    }
    p.wants_learned = true;  // filled in by step(), one drafter call for all learned slots
    return p;
}

SlotRound MtpSlotScheduler::finish(const Plan& p, std::span<const std::uint32_t> targets) {
    Request& r = requests_[p.request];
    if (targets.size() != p.drafts.size() + 1) throw std::runtime_error("batch verifier returned a wrong row count");
    SlotRound out;
    out.slot = r.slot;
    out.source = p.source;
    out.draft_tokens = p.drafts;
    if (p.drafts.empty()) {
        out.accepted = 0;
        out.emitted_tokens = {targets[0]};
    } else {
        const MtpGreedyDecision d = decide_mtp_greedy(p.drafts, targets, opt_.stop_tokens);
        out.accepted = d.accepted;
        out.emitted_tokens.assign(p.drafts.begin(), p.drafts.begin() + static_cast<std::ptrdiff_t>(d.accepted));
        out.emitted_tokens.push_back(d.next_token);
    }
    verifier_.commit(r.slot, out.accepted);
    r.position += out.accepted + 1;
    r.current = out.emitted_tokens.back();

    SlotStats& s = r.stats;
    const std::size_t proposed = p.drafts.size();
    switch (p.source) {
    case DraftSourceKind::serial:
        s.serial_steps += 1;
        break;
    case DraftSourceKind::context_copy: {
        s.mtp_rounds += 1;
        s.mtp_proposed += proposed;
        s.mtp_accepted += out.accepted;
        s.context_copy_rounds += 1;
        s.context_copy_proposed += proposed;
        s.context_copy_accepted += out.accepted;
        const double ratio = static_cast<double>(out.accepted) / static_cast<double>(proposed);
        r.copy_ema = 0.7 * r.copy_ema + 0.3 * ratio;
        r.copy_seen += 1;
        r.copy_perfect = out.accepted == proposed ? r.copy_perfect + 1 : 0;
        if (ratio >= 0.5) r.copy_backoff = 64;
        if (r.copy_seen >= 3 && r.copy_ema < 0.35) {
            // Stop copying for a while; the pause doubles each time (up to 4096 tokens).
            r.copy_suspend_until = r.tokens.size() + r.copy_backoff;
            r.copy_backoff = std::min<std::size_t>(r.copy_backoff * 2, 4096);
            r.copy_ema = 0.5;
            r.copy_seen = 0;
            r.copy_perfect = 0;
            s.context_copy_suspensions += 1;
        }
        break;
    }
    case DraftSourceKind::history:
        s.mtp_rounds += 1;
        s.mtp_proposed += proposed;
        s.mtp_accepted += out.accepted;
        s.history_draft_rounds += 1;
        s.history_draft_proposed += proposed;
        s.history_draft_accepted += out.accepted;
        r.history_policy.observe_history(proposed, out.accepted);
        break;
    case DraftSourceKind::learned:
        s.mtp_rounds += 1;
        s.mtp_proposed += proposed;
        s.mtp_accepted += out.accepted;
        r.depth.observe(proposed, out.accepted);
        r.guard.observe(out.accepted);
        r.history_policy.observe_learned(proposed, out.accepted);
        break;
    }
    s.history_draft_activations = r.history_policy.activations();
    s.history_draft_deactivations = r.history_policy.deactivations();
    s.mtp_final_depth = r.depth.depth();
    s.mtp_promotions = r.depth.promotions();
    s.mtp_demotions = r.depth.demotions();

    for (const std::uint32_t t : out.emitted_tokens) {
        if (r.tokens.size() == r.max_tokens) break;
        if (is_stop(t)) {
            r.finished = true;
            s.finish_reason = "stop";
            break;
        }
        r.tokens.push_back(t);
        if (r.history_policy.enabled()) r.history.append(t);
    }
    if (!r.finished && r.tokens.size() >= r.max_tokens) {
        r.finished = true;
        s.finish_reason = "length";
    }
    if (p.source == DraftSourceKind::learned && !r.finished) {
        const bool fall_back = opt_.economic_fallback
                                   ? r.guard.should_fallback(opt_.zero_accept_fallback_rounds)
                                   : r.guard.zero_accept_streak() >= opt_.zero_accept_fallback_rounds;
        if (fall_back && r.mtp_profitable) {
            r.mtp_profitable = false;
            s.mtp_fallbacks += 1;
        }
    }
    return out;
}

std::vector<SlotRound> MtpSlotScheduler::step() {
    std::vector<Plan> plans;
    for (std::size_t i = 0; i < requests_.size(); ++i)
        if (!requests_[i].finished) plans.push_back(plan(i));
    std::vector<DraftRequest> asks;
    for (const Plan& p : plans)
        if (p.wants_learned) {
            const Request& r = requests_[p.request];
            asks.push_back(DraftRequest{r.slot, r.current, r.depth.depth()});
        }
    if (!asks.empty()) {
        std::vector<std::vector<std::uint32_t>> got = drafter_->propose_batch(asks);
        if (got.size() != asks.size()) throw std::runtime_error("learned drafter returned a wrong request count");
        std::size_t j = 0;
        const std::size_t width = verifier_.max_rows() - 1;
        for (Plan& p : plans) {
            if (!p.wants_learned) continue;
            std::vector<std::uint32_t>& d = got[j];
            const std::size_t cap = std::min(asks[j].depth, width);
            if (d.size() > cap) d.resize(cap);
            ++j;
            if (d.empty()) continue;  // the drafter had nothing: a serial step
            p.source = DraftSourceKind::learned;
            p.drafts = std::move(d);
        }
    }
    std::vector<SlotRound> rounds;
    rounds.reserve(plans.size());
    const std::size_t width = verifier_.max_rows();
    std::size_t first = 0;
    while (first < plans.size()) {
        // Pack consecutive plans while their rows fit one verification.
        std::size_t last = first, rows = 0;
        std::vector<SlotVerifyRows> batch;
        while (last < plans.size() && rows + plans[last].drafts.size() + 1 <= width) {
            const Plan& p = plans[last];
            rows += p.drafts.size() + 1;
            batch.push_back(SlotVerifyRows{requests_[p.request].slot, requests_[p.request].current, p.drafts});
            ++last;
        }
        const std::vector<std::vector<std::uint32_t>> targets = verifier_.verify(batch);
        batches_ += 1;
        if (targets.size() != batch.size()) throw std::runtime_error("batch verifier returned a wrong slot count");
        for (std::size_t j = first; j < last; ++j) rounds.push_back(finish(plans[j], targets[j - first]));
        first = last;
    }
    return rounds;
}

} // namespace qwen38
