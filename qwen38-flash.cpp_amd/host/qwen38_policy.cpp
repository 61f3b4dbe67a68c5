// qwen38_policy.cpp — engine-side MTP round policy (host only).
#include "qwen38_policy.hpp"

#include <algorithm>
#include <cstdlib>
#include <stdexcept>
#include <string_view>

namespace qwen38 {
namespace {

constexpr std::size_t kShortPrompt = 2048;        // probing / adaptive depth 4 only up to here
constexpr std::size_t kProbeRounds = 8;
constexpr std::size_t kProbePromote = 10;         // accepted tokens over the probe to promote
constexpr std::size_t kThreeProbation = 4;
constexpr std::size_t kThreeWindow = 12;
constexpr std::size_t kThreeLosingWindows = 2;
constexpr std::size_t kFourProbation = 4;
constexpr std::size_t kFourWindow = 8;
constexpr std::size_t kLearnedTrial = 8;          // learned rounds before history drafts may start
constexpr std::size_t kHistoryTrial = 2;          // history rounds before they may be withdrawn

bool env_equals(const char* name, std::string_view value) {
    const char* v = std::getenv(name);
    return v != nullptr && std::string_view(v) == value;
}
bool demotion_enabled() { return !env_equals("QWEN38_MTP_DEMOTION", "0"); }
bool early_demotion_enabled() { return env_equals("QWEN38_MTP_EARLY_DEMOTION", "1"); }

// Token-window key: a multiply-xorshift mix seeded with the window length. Every match is
// confirmed against the tokens themselves, so the key only has to spread windows out.
struct WindowKey {
    std::uint64_t h;
    explicit WindowKey(std::size_t length) noexcept : h(0x243F6A8885A308D3ULL ^ static_cast<std::uint64_t>(length)) {}
    void add(std::uint32_t token) noexcept {
        h = (h ^ token) * 0x9E3779B97F4A7C15ULL;
        h ^= h >> 29;
    }
};

} // namespace

// ------------------------------------------------------------------ MtpDepthPolicy
MtpDepthPolicy::MtpDepthPolicy(std::size_t maximum_depth, std::size_t prompt_tokens, bool adaptive_depth_four)
    : maximum_depth_(maximum_depth), depth_(maximum_depth) {
    if (maximum_depth != 0 && (maximum_depth < 2 || maximum_depth > 4))
        throw std::runtime_error("MTP policy depth must be 0 or between 2 and 4");
    const bool short_prompt = prompt_tokens <= kShortPrompt;
    if (maximum_depth == 4) {
        if (adaptive_depth_four && short_prompt) phase_ = Phase::watch_four;
    } else if (maximum_depth == 3) {
        const bool four = adaptive_depth_four || env_equals("QWEN38_MTP_ADAPTIVE_DEPTH4", "1");
        if (four && short_prompt) {
            depth_ = 4;
            phase_ = Phase::watch_four;
        } else {
            depth_ = 2;
            phase_ = short_prompt ? Phase::probing : Phase::fixed;
        }
    }
}

void MtpDepthPolicy::demote_to(std::size_t depth, Phase next) noexcept {
    depth_ = depth;
    phase_ = next;
    ++demotions_;
}

void MtpDepthPolicy::observe(std::size_t proposed, std::size_t accepted) {
    if (accepted > proposed) throw std::runtime_error("MTP accepted count exceeds proposals");
    if (depth_ == 0 || proposed == 0) return;
    switch (phase_) {
    case Phase::probing:
        observe_probe(accepted);
        break;
    case Phase::watch_four:
        if (demotion_enabled()) observe_four(proposed, accepted);
        break;
    case Phase::watch_three:
        if (demotion_enabled()) observe_three(proposed, accepted);
        break;
    case Phase::fixed:
        break;
    }
}

void MtpDepthPolicy::observe_probe(std::size_t accepted) {
    probe_.rounds += 1;
    probe_.accepted += accepted;
    if (probe_.rounds < kProbeRounds) return;
    if (probe_.accepted >= kProbePromote) {
        depth_ = maximum_depth_;
        phase_ = Phase::watch_three;
        ++promotions_;
    } else {
        phase_ = Phase::fixed;
    }
}

void MtpDepthPolicy::observe_four(std::size_t proposed, std::size_t accepted) {
    Window& w = window_;
    w.rounds += 1;
    w.proposed += proposed;
    w.accepted += accepted;
    if (accepted >= 4) w.all_four += 1;
    // Probation: fewer than half of the first 4 rounds with all four drafts accepted.
    if (!four_probation_passed_ && w.rounds == kFourProbation && 2 * w.all_four < kFourProbation) {
        demote_to(3, Phase::watch_three);
        w.clear();
        return;
    }
    if (w.rounds == kFourProbation) four_probation_passed_ = true;
    if (w.rounds == kFourWindow) {
        if (2 * w.all_four < kFourWindow) demote_to(3, Phase::watch_three);
        w.clear();
    }
}

void MtpDepthPolicy::observe_three(std::size_t proposed, std::size_t accepted) {
    Window& w = window_;
    w.rounds += 1;
    w.proposed += proposed;
    w.accepted += accepted;
    const bool losing = 2 * w.accepted < w.proposed;
    if (!three_probation_passed_ && w.rounds == kThreeProbation && losing && early_demotion_enabled()) {
        demote_to(2, Phase::fixed);
        return;
    }
    if (w.rounds == kThreeProbation) three_probation_passed_ = true;
    if (w.rounds == kThreeWindow) {
        if (!losing) {
            losing_windows_ = 0;
        } else if (++losing_windows_ == kThreeLosingWindows) {
            demote_to(2, Phase::fixed);
        }
        w.clear();
    }
}

// ------------------------------------------------------------------ MtpProfitabilityGuard
void MtpProfitabilityGuard::observe(std::size_t accepted) noexcept {
    streak_ = accepted == 0 ? streak_ + 1 : 0;
    const std::size_t slot = rounds_ % window_size;  // the oldest entry once the ring is full
    if (rounds_ >= window_size) window_sum_ -= ring_[slot];
    ring_[slot] = accepted;
    window_sum_ += accepted;
    rounds_ += 1;
    total_ += accepted;
}

bool MtpProfitabilityGuard::should_fallback(std::size_t fallback_streak) const noexcept {
    if (rounds_ < window_size) return should_fallback_mtp(streak_, fallback_streak, rounds_, total_);
    return window_sum_ < window_size;
}

// ------------------------------------------------------------------ HistoryDraftPolicy
namespace {
void check_observation(std::size_t proposed, std::size_t accepted) {
    if (accepted > proposed) throw std::runtime_error("draft acceptance exceeds proposed tokens");
}
} // namespace

bool HistoryDraftPolicy::Tally::add(std::size_t p, std::size_t a, std::size_t limit) noexcept {
    rounds += 1;
    proposed += p;
    accepted += a;
    if (rounds < limit) return false;
    const bool losing = 2 * accepted < proposed;
    *this = Tally{};
    return losing;
}

void HistoryDraftPolicy::observe_learned(std::size_t proposed, std::size_t accepted) {
    check_observation(proposed, accepted);
    if (mode_ != HistoryDraftMode::adaptive || active_ || rejected_ || proposed == 0) return;
    if (learned_.add(proposed, accepted, kLearnedTrial)) {
        active_ = true;
        ++activations_;
    }
}

void HistoryDraftPolicy::observe_history(std::size_t proposed, std::size_t accepted) {
    check_observation(proposed, accepted);
    if (mode_ != HistoryDraftMode::adaptive || !active_ || proposed == 0) return;
    if (history_.add(proposed, accepted, kHistoryTrial)) {
        active_ = false;
        rejected_ = true;
        ++deactivations_;
    }
}

// ------------------------------------------------------------------ HistoryDraftCache
HistoryDraftCache::HistoryDraftCache(std::size_t minimum_order, std::size_t maximum_order)
    : min_order_(minimum_order), max_order_(maximum_order) {
    if (min_order_ == 0 || min_order_ > max_order_) throw std::runtime_error("invalid history draft order range");
}

std::uint64_t HistoryDraftCache::suffix_key(std::size_t start, std::size_t order) const noexcept {
    WindowKey k(order);
    for (std::size_t i = 0; i < order; ++i) k.add(tokens_[start + i]);
    return k.h;
}

bool HistoryDraftCache::same_as_tail(std::size_t start, std::size_t order) const noexcept {
    const std::size_t n = tokens_.size();
    if (order > n || start + order >= n) return false;  // the tail itself never matches
    return std::equal(tokens_.begin() + static_cast<std::ptrdiff_t>(start),
                      tokens_.begin() + static_cast<std::ptrdiff_t>(start + order),
                      tokens_.end() - static_cast<std::ptrdiff_t>(order));
}

void HistoryDraftCache::append(std::uint32_t token) {
    tokens_.push_back(token);
    const std::size_t n = tokens_.size();
    // The windows that end just before the new token now have a known continuation.
    for (std::size_t order = min_order_; order <= max_order_ && order + 1 <= n; ++order) {
        const std::size_t start = n - 1 - order;
        last_start_.insert_or_assign(suffix_key(start, order), start);
    }
}

void HistoryDraftCache::append(std::span<const std::uint32_t> tokens) {
    tokens_.reserve(tokens_.size() + tokens.size());
    for (const std::uint32_t t : tokens) append(t);
}

std::vector<std::uint32_t> HistoryDraftCache::propose(std::size_t maximum_tokens) const {
    if (maximum_tokens == 0) return {};
    const std::size_t n = tokens_.size();
    for (std::size_t order = max_order_ + 1; order-- > min_order_;) {
        if (order > n) continue;
        const auto hit = last_start_.find(suffix_key(n - order, order));
        if (hit == last_start_.end() || !same_as_tail(hit->second, order)) continue;
        const std::size_t from = hit->second + order;
        const std::size_t count = std::min(maximum_tokens, n - from);
        return {tokens_.begin() + static_cast<std::ptrdiff_t>(from),
                tokens_.begin() + static_cast<std::ptrdiff_t>(from + count)};
    }
    return {};
}

// ------------------------------------------------------------------ ContextCopyCache
namespace {
constexpr std::size_t kCopyCandidates = 32;  // most recent prompt matches examined
}

ContextCopyCache::ContextCopyCache(std::span<const std::uint32_t> prompt, std::size_t minimum_order,
                                   std::size_t maximum_order)
    : min_order_(minimum_order), max_order_(maximum_order), prompt_(prompt.begin(), prompt.end()) {
    if (min_order_ == 0 || min_order_ > max_order_) throw std::runtime_error("invalid context-copy order range");
    ends_.reserve(prompt_.size());
    for (std::size_t end = min_order_; end < prompt_.size(); ++end) {
        WindowKey k(min_order_);
        for (std::size_t i = end - min_order_; i < end; ++i) k.add(prompt_[i]);
        ends_[k.h].push_back(end);
    }
}

template <typename TokenAt>
ContextCopyProposal ContextCopyCache::lookup(std::size_t history_size, TokenAt&& at, std::size_t maximum_tokens) const {
    if (maximum_tokens == 0 || history_size < min_order_) return {};
    const std::size_t tail = history_size - min_order_;
    WindowKey k(min_order_);
    for (std::size_t i = tail; i < history_size; ++i) k.add(at(i));
    const auto hit = ends_.find(k.h);
    if (hit == ends_.end()) return {};
    const std::vector<std::size_t>& ends = hit->second;
    const std::size_t cap = max_order_ - min_order_;
    const std::size_t oldest = ends.size() > kCopyCandidates ? ends.size() - kCopyCandidates : 0;
    bool found = false;
    std::size_t best = 0, best_ext = 0;
    for (std::size_t c = ends.size(); c-- > oldest;) {
        const std::size_t end = ends[c];
        if (end >= prompt_.size()) continue;
        bool equal = true;
        for (std::size_t i = 0; i < min_order_ && equal; ++i) equal = prompt_[end - min_order_ + i] == at(tail + i);
        if (!equal) continue;  // a key collision
        // How far the agreement reaches further left.
        std::size_t ext = 0;
        while (ext < cap && end > min_order_ + ext && history_size > min_order_ + ext &&
               prompt_[end - min_order_ - ext - 1] == at(tail - ext - 1))
            ++ext;
        if (!found || ext > best_ext) {
            found = true;
            best = end;
            best_ext = ext;
            if (ext == cap) break;
        }
    }
    if (!found) return {};
    const std::size_t count = std::min(maximum_tokens, prompt_.size() - best);
    ContextCopyProposal out;
    out.tokens.assign(prompt_.begin() + static_cast<std::ptrdiff_t>(best),
                      prompt_.begin() + static_cast<std::ptrdiff_t>(best + count));
    out.match_extension = best_ext;
    return out;
}

ContextCopyProposal ContextCopyCache::propose(std::span<const std::uint32_t> history,
                                              std::size_t maximum_tokens) const {
    return lookup(history.size(), [&](std::size_t i) { return history[i]; }, maximum_tokens);
}

ContextCopyProposal ContextCopyCache::propose_completion(std::span<const std::uint32_t> completion,
                                                         std::size_t maximum_tokens) const {
    const std::size_t np = prompt_.size();
    return lookup(np + completion.size(), [&](std::size_t i) { return i < np ? prompt_[i] : completion[i - np]; },
                  maximum_tokens);
}

} // namespace qwen38
