// policy_test.cpp — CPU tests of the engine-side MTP round policy (host/qwen38_policy.hpp) and
// of the batched multi-slot round driver (host/qwen38_engine.hpp). No GPU calls.
//
//   1. Known answers restated from the reference's own tests:
//      tests/mtp_depth_policy_test.cpp:8-148 and tests/history_draft_test.cpp:6-67.
//   2. Random call sequences run through these classes and through the reference's sources
//      compiled into oracle/_ref/libq38_ref.so (argument 1; skipped when absent): the
//      observable state after every call must be identical, including where errors are thrown
//      and the environment switches the reference reads.
//   3. The scheduler over an exact fake verifier (targets are a fixed token map): whatever the
//      drafts, each request's output equals serial greedy decoding; batches stay within the
//      verifier's rows; fallback, history drafts, context copies and stop tokens behave as the
//      reference's engine loop specifies; replaying each request's learned rounds into a fresh
//      policy (and the reference's) reproduces the reported depth statistics.
// Usage: policy_test [path/to/libq38_ref.so]
#include "qwen38_engine.hpp"
#include "qwen38_policy.hpp"

#include <dlfcn.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <functional>
#include <random>
#include <set>
#include <stdexcept>
#include <string>
#include <vector>

using namespace qwen38;

static int g_fail = 0;
static int g_checks = 0;
#define CHECK(c)                                                                \
    do {                                                                        \
        ++g_checks;                                                             \
        if (!(c)) {                                                             \
            ++g_fail;                                                           \
            std::fprintf(stderr, "FAIL %s:%d: %s\n", __FILE__, __LINE__, #c);   \
        }                                                                       \
    } while (0)

template <typename F>
static std::string thrown(F&& f) {
    try {
        f();
    } catch (const std::exception& e) {
        return e.what();
    }
    return {};
}

static void clear_env() {
    for (const char* v : {"QWEN38_MTP_DEMOTION", "QWEN38_MTP_EARLY_DEMOTION", "QWEN38_MTP_ADAPTIVE_DEPTH4",
                          "QWEN38_LONG_HISTORY_DEPTH4"})
        unsetenv(v);
}

// ------------------------------------------------------------------ 1. known answers
static void feed(MtpDepthPolicy& p, int rounds, std::size_t proposed, std::size_t accepted) {
    for (int i = 0; i < rounds; ++i) p.observe(proposed, accepted);
}

static void known_answers_depth() {
    clear_env();
    {   // depth 2 never moves
        MtpDepthPolicy p(2, 10);
        feed(p, 16, 2, 2);
        CHECK(p.depth() == 2 && p.promotions() == 0);
    }
    {   // long prompts skip the probe
        MtpDepthPolicy p(3, 2049);
        feed(p, 16, 2, 2);
        CHECK(p.depth() == 2 && !p.probing());
    }
    {   // probe: 10 accepted in 8 rounds promotes; then two losing 12-round windows demote
        MtpDepthPolicy p(3, 32);
        feed(p, 5, 2, 2);
        feed(p, 3, 2, 0);
        CHECK(p.depth() == 3 && p.promotions() == 1);
        for (int r = 0; r < 11; ++r) p.observe(3, r < 5 ? 2 : 1);
        CHECK(p.depth() == 3);
        p.observe(3, 0);
        CHECK(p.depth() == 3);
        feed(p, 12, 3, 0);
        CHECK(p.depth() == 2 && p.demotions() == 1);
    }
    {   // 8 accepted in the probe: no promotion
        MtpDepthPolicy p(3, 32);
        feed(p, 4, 2, 2);
        feed(p, 4, 2, 0);
        CHECK(p.depth() == 2 && p.promotions() == 0);
    }
    {   // a winning window in between resets the losing count
        MtpDepthPolicy p(3, 32);
        feed(p, 8, 2, 2);
        feed(p, 12, 3, 1);
        feed(p, 12, 3, 2);
        feed(p, 12, 3, 1);
        CHECK(p.depth() == 3 && p.demotions() == 0);
    }
    {   // exactly half accepted is not losing
        MtpDepthPolicy p(3, 32);
        feed(p, 8, 2, 2);
        for (int r = 0; r < 12; ++r) p.observe(3, r < 6 ? 3 : 0);
        CHECK(p.depth() == 3 && p.demotions() == 0);
    }
    {   // QWEN38_MTP_DEMOTION=0 keeps depth 3
        setenv("QWEN38_MTP_DEMOTION", "0", 1);
        MtpDepthPolicy p(3, 32);
        feed(p, 8, 2, 2);
        feed(p, 24, 3, 0);
        CHECK(p.depth() == 3 && p.promotions() == 1 && p.demotions() == 0);
        unsetenv("QWEN38_MTP_DEMOTION");
    }
    {   // early demotion after a losing 4-round probation
        setenv("QWEN38_MTP_EARLY_DEMOTION", "1", 1);
        MtpDepthPolicy p(3, 32);
        feed(p, 8, 2, 2);
        feed(p, 3, 3, 1);
        CHECK(p.depth() == 3);
        p.observe(3, 1);
        CHECK(p.depth() == 2 && p.demotions() == 1);
        MtpDepthPolicy q(3, 32);
        feed(q, 8, 2, 2);
        feed(q, 12, 3, 2);
        feed(q, 4, 3, 0);
        CHECK(q.depth() == 3);
        unsetenv("QWEN38_MTP_EARLY_DEMOTION");
    }
    {   // explicit depth 4 is fixed; adaptive depth 4 watches how often all four are accepted
        MtpDepthPolicy p(4, 100000);
        CHECK(p.depth() == 4);
        feed(p, 8, 4, 0);
        CHECK(p.depth() == 4 && p.demotions() == 0);
        MtpDepthPolicy a(4, 32, true);
        CHECK(a.depth() == 4);
        a.observe(4, 4);
        feed(a, 3, 4, 3);
        CHECK(a.depth() == 3 && a.demotions() == 1);
        MtpDepthPolicy l(4, 2049, true);
        CHECK(l.depth() == 4);
    }
    {   // QWEN38_MTP_ADAPTIVE_DEPTH4=1 turns depth 3 into an adaptive depth 4
        setenv("QWEN38_MTP_ADAPTIVE_DEPTH4", "1", 1);
        MtpDepthPolicy p(3, 32);
        CHECK(p.depth() == 4);
        feed(p, 4, 4, 4);
        feed(p, 4, 4, 2);
        CHECK(p.depth() == 4);
        MtpDepthPolicy q(3, 32);
        feed(q, 3, 4, 4);
        feed(q, 5, 4, 3);
        CHECK(q.depth() == 3 && q.demotions() == 1);
        MtpDepthPolicy e(3, 32);
        e.observe(4, 4);
        feed(e, 3, 4, 3);
        CHECK(e.depth() == 3 && e.demotions() == 1);
        MtpDepthPolicy l(3, 2049);
        CHECK(l.depth() == 2 && !l.probing());
        unsetenv("QWEN38_MTP_ADAPTIVE_DEPTH4");
    }
    CHECK(thrown([] { MtpDepthPolicy p(1, 10); }) == "MTP policy depth must be 0 or between 2 and 4");
    CHECK(thrown([] { MtpDepthPolicy p(5, 10); }) == "MTP policy depth must be 0 or between 2 and 4");
    CHECK(thrown([] { MtpDepthPolicy p(3, 10); p.observe(2, 3); }) == "MTP accepted count exceeds proposals");
    {
        MtpDepthPolicy z(0, 10);
        z.observe(3, 3);
        CHECK(z.depth() == 0);
    }
}

static void known_answers_profitability() {
    CHECK(should_fallback_mtp(2, 2, 2, 0));
    CHECK(should_fallback_mtp(2, 2, 11, 10));
    CHECK(!should_fallback_mtp(1, 2, 2, 0));
    CHECK(!should_fallback_mtp(2, 2, 28, 39));
    CHECK(!should_fallback_mtp(2, 2, 11, 11));
    CHECK(!cache_mtp_as_profitable(2, 0, 1));
    CHECK(!cache_mtp_as_profitable(4, 3, 1));
    CHECK(cache_mtp_as_profitable(47, 59, 1));
    CHECK(cache_mtp_as_profitable(59, 70, 0));
    MtpProfitabilityGuard early;
    early.observe(0);
    CHECK(!early.should_fallback(2));
    early.observe(0);
    CHECK(early.should_fallback(2));
    MtpProfitabilityGuard profitable;
    for (int r = 0; r < 6; ++r) profitable.observe(2);
    profitable.observe(0);
    profitable.observe(0);
    CHECK(!profitable.should_fallback(2));
    MtpProfitabilityGuard even;
    for (std::size_t r = 0; r < MtpProfitabilityGuard::window_size; ++r) even.observe(1);
    CHECK(!even.should_fallback(2));
    MtpProfitabilityGuard losing;
    for (std::size_t r = 0; r < MtpProfitabilityGuard::window_size; ++r) losing.observe(r < 15 ? 1 : 0);
    CHECK(losing.should_fallback(2));
    // The window slides: 16 more rounds of 1 after a bad start recover.
    MtpProfitabilityGuard slide;
    for (int r = 0; r < 16; ++r) slide.observe(0);
    CHECK(slide.should_fallback(100));
    for (int r = 0; r < 16; ++r) slide.observe(1);
    CHECK(!slide.should_fallback(100) && slide.window_accepted() == 16 && slide.total_accepted() == 16);
}

static void known_answers_history() {
    HistoryDraftPolicy adaptive;
    CHECK(!adaptive.should_try());
    for (int r = 0; r < 7; ++r) {
        adaptive.observe_learned(2, r == 0 ? 1 : 0);
        CHECK(!adaptive.should_try());
    }
    adaptive.observe_learned(2, 1);
    CHECK(adaptive.should_try() && adaptive.activations() == 1);
    for (int r = 0; r < 2; ++r) adaptive.observe_history(3, 1);
    CHECK(!adaptive.should_try() && adaptive.exhausted() && adaptive.deactivations() == 1);
    for (int r = 0; r < 8; ++r) adaptive.observe_learned(2, 0);
    CHECK(!adaptive.should_try() && adaptive.activations() == 1);

    HistoryDraftPolicy strong;
    for (int r = 0; r < 8; ++r) strong.observe_learned(2, r % 2 == 0 ? 2 : 1);
    CHECK(!strong.should_try() && strong.activations() == 0);

    HistoryDraftPolicy forced(HistoryDraftMode::forced);
    CHECK(forced.enabled() && forced.should_try() && !forced.exhausted());
    for (int r = 0; r < 2; ++r) forced.observe_history(3, 0);
    CHECK(forced.should_try() && !forced.exhausted());

    HistoryDraftPolicy disabled(HistoryDraftMode::disabled);
    CHECK(!disabled.enabled() && !disabled.should_try() && !disabled.exhausted());
    CHECK(thrown([] { HistoryDraftPolicy p; p.observe_learned(1, 2); }) == "draft acceptance exceeds proposed tokens");

    HistoryDraftCache cache(2, 4);
    const std::vector<std::uint32_t> hist{1, 2, 3, 4, 9, 1, 2, 3, 4};
    cache.append(hist);
    CHECK(cache.propose(4) == (std::vector<std::uint32_t>{9, 1, 2, 3}));
    cache.append(9);
    CHECK(cache.propose(3) == (std::vector<std::uint32_t>{1, 2, 3}));
    CHECK(cache.propose(0).empty());
    HistoryDraftCache miss;
    miss.append(std::vector<std::uint32_t>{10, 11, 12, 13, 14});
    CHECK(miss.propose(4).empty());
    CHECK(thrown([] { HistoryDraftCache c(0, 3); }) == "invalid history draft order range");
    CHECK(thrown([] { HistoryDraftCache c(4, 3); }) == "invalid history draft order range");

    const std::vector<std::uint32_t> prompt{10, 11, 12, 13, 14, 15, 16, 17, 18, 30, 31, 12, 13, 14, 15, 16, 17, 40};
    ContextCopyCache copy(prompt, 3, 6);
    const std::vector<std::uint32_t> tail{90, 11, 12, 13, 14, 15, 16};
    const ContextCopyProposal got = copy.propose(tail, 8);
    CHECK(got.tokens == (std::vector<std::uint32_t>{17, 18, 30, 31, 12, 13, 14, 15}));
    CHECK(got.match_extension == 3);
    CHECK(copy.propose(std::vector<std::uint32_t>{99, 98, 97, 96}, 8).tokens.empty());
    const ContextCopyProposal comp = copy.propose_completion(std::vector<std::uint32_t>{11, 12, 13, 14, 15, 16}, 8);
    CHECK(comp.tokens == got.tokens && comp.match_extension == got.match_extension);
    CHECK(thrown([&] { ContextCopyCache c(prompt, 7, 6); }) == "invalid context-copy order range");
}

// ------------------------------------------------------------------ 2. differential vs the reference
struct Ref {
    void* h = nullptr;
    int (*depth_run)(uint64_t, uint64_t, int, const uint64_t*, const uint64_t*, int64_t, uint64_t*) = nullptr;
    int (*guard_run)(const uint64_t*, int64_t, uint64_t, uint64_t*) = nullptr;
    int (*fallback)(uint64_t, uint64_t, uint64_t, uint64_t) = nullptr;
    int (*profitable)(uint64_t, uint64_t, uint64_t) = nullptr;
    int (*hpolicy_run)(int, const int*, const uint64_t*, const uint64_t*, int64_t, uint64_t*) = nullptr;
    int (*hcache_run)(uint64_t, uint64_t, const uint32_t*, int64_t, const uint64_t*, uint64_t, uint32_t*,
                      uint64_t*) = nullptr;
    int (*copy)(const uint32_t*, int64_t, uint64_t, uint64_t, const uint32_t*, int64_t, uint64_t, int, uint64_t,
                uint32_t*, uint64_t*, uint64_t*) = nullptr;
    bool load(const char* path) {
        h = dlopen(path, RTLD_NOW | RTLD_LOCAL | RTLD_DEEPBIND);  // its qwen38:: classes are its own
        if (!h) return false;
        auto sym = [&](auto& fn, const char* name) { fn = reinterpret_cast<std::remove_reference_t<decltype(fn)>>(dlsym(h, name)); return fn != nullptr; };
        return sym(depth_run, "ref_depth_policy_run") && sym(guard_run, "ref_guard_run") &&
               sym(fallback, "ref_should_fallback_mtp") && sym(profitable, "ref_cache_mtp_as_profitable") &&
               sym(hpolicy_run, "ref_history_policy_run") && sym(hcache_run, "ref_history_cache_run") &&
               sym(copy, "ref_context_copy");
    }
};

static int depth_run_mine(uint64_t max_depth, uint64_t prompt, int adaptive4, const std::vector<uint64_t>& prop,
                          const std::vector<uint64_t>& acc, std::vector<uint64_t>& out) {
    out.assign((prop.size() + 1) * 4, 0);
    try {
        MtpDepthPolicy p(max_depth, prompt, adaptive4 != 0);
        auto put = [&](std::size_t i) {
            out[i * 4 + 0] = p.depth();
            out[i * 4 + 1] = p.promotions();
            out[i * 4 + 2] = p.demotions();
            out[i * 4 + 3] = p.probing() ? 1 : 0;
        };
        put(0);
        for (std::size_t i = 0; i < prop.size(); ++i) {
            try {
                p.observe(prop[i], acc[i]);
            } catch (const std::exception&) {
                return static_cast<int>(-(2 + static_cast<int64_t>(i)));
            }
            put(i + 1);
        }
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

static void differential(const Ref& ref) {
    std::mt19937_64 rng(20260);
    auto uni = [&](uint64_t lo, uint64_t hi) { return std::uniform_int_distribution<uint64_t>(lo, hi)(rng); };
    int cases = 0;
    // Depth policy: every depth / prompt / mode / environment combination, random acceptance.
    const char* envs[][3] = {{nullptr, nullptr, nullptr}, {"0", nullptr, nullptr}, {nullptr, "1", nullptr},
                             {nullptr, nullptr, "1"}, {nullptr, "1", "1"}, {"0", "1", "1"}};
    for (const auto& env : envs) {
        clear_env();
        if (env[0]) setenv("QWEN38_MTP_DEMOTION", env[0], 1);
        if (env[1]) setenv("QWEN38_MTP_EARLY_DEMOTION", env[1], 1);
        if (env[2]) setenv("QWEN38_MTP_ADAPTIVE_DEPTH4", env[2], 1);
        for (uint64_t depth : {0, 1, 2, 3, 4, 5})
            for (uint64_t prompt : {1, 2048, 2049})
                for (int a4 : {0, 1})
                    for (int rep = 0; rep < 12; ++rep) {
                        const std::size_t n = 40 + uni(0, 40);
                        std::vector<uint64_t> p(n), a(n);
                        const uint64_t skew = uni(0, 4);  // acceptance level of this sequence
                        for (std::size_t i = 0; i < n; ++i) {
                            p[i] = uni(0, 4);
                            a[i] = p[i] == 0 ? 0 : std::min<uint64_t>(p[i], uni(0, p[i]) + (uni(0, 4) < skew ? p[i] : 0));
                            if (uni(0, 199) == 0) a[i] = p[i] + 1;  // an invalid observation
                        }
                        std::vector<uint64_t> mine, theirs((n + 1) * 4, 0);
                        const int rm = depth_run_mine(depth, prompt, a4, p, a, mine);
                        const int rr = ref.depth_run(depth, prompt, a4, p.data(), a.data(), static_cast<int64_t>(n),
                                                     theirs.data());
                        CHECK(rm == rr);
                        CHECK(mine == theirs);
                        ++cases;
                    }
    }
    clear_env();
    // Profitability guard and its two predicates.
    for (int rep = 0; rep < 300; ++rep) {
        const std::size_t n = 1 + uni(0, 60);
        const uint64_t streak = uni(0, 4);
        std::vector<uint64_t> a(n);
        const uint64_t zero_bias = uni(0, 9);
        for (auto& v : a) v = uni(0, 9) < zero_bias ? 0 : uni(0, 4);
        std::vector<uint64_t> theirs(n * 5);
        ref.guard_run(a.data(), static_cast<int64_t>(n), streak, theirs.data());
        MtpProfitabilityGuard g;
        bool same = true;
        for (std::size_t i = 0; i < n; ++i) {
            g.observe(a[i]);
            same &= theirs[i * 5 + 0] == g.rounds() && theirs[i * 5 + 1] == g.total_accepted() &&
                    theirs[i * 5 + 2] == g.window_accepted() && theirs[i * 5 + 3] == g.zero_accept_streak() &&
                    theirs[i * 5 + 4] == (g.should_fallback(streak) ? 1u : 0u);
        }
        CHECK(same);
        ++cases;
    }
    for (uint64_t s = 0; s < 5; ++s)
        for (uint64_t f = 0; f < 5; ++f)
            for (uint64_t r = 0; r < 6; ++r)
                for (uint64_t a = 0; a < 8; ++a) {
                    CHECK((ref.fallback(s, f, r, a) != 0) == should_fallback_mtp(s, f, r, a));
                    CHECK((ref.profitable(r, a, f) != 0) == cache_mtp_as_profitable(r, a, f));
                }
    // History draft policy.
    for (int mode = 0; mode < 3; ++mode)
        for (int rep = 0; rep < 100; ++rep) {
            const std::size_t n = 1 + uni(0, 50);
            std::vector<int> kind(n);
            std::vector<uint64_t> p(n), a(n);
            for (std::size_t i = 0; i < n; ++i) {
                kind[i] = static_cast<int>(uni(0, 1));
                p[i] = uni(0, 4);
                a[i] = p[i] == 0 ? 0 : uni(0, p[i]);
                if (uni(0, 99) == 0) a[i] = p[i] + 1;
            }
            std::vector<uint64_t> theirs(n * 4, 0), mine(n * 4, 0);
            const int rr = ref.hpolicy_run(mode, kind.data(), p.data(), a.data(), static_cast<int64_t>(n), theirs.data());
            HistoryDraftPolicy hp(mode == 0 ? HistoryDraftMode::disabled
                                            : mode == 1 ? HistoryDraftMode::adaptive : HistoryDraftMode::forced);
            int rm = 0;
            for (std::size_t i = 0; i < n && rm == 0; ++i) {
                try {
                    if (kind[i] == 0) hp.observe_learned(p[i], a[i]);
                    else hp.observe_history(p[i], a[i]);
                } catch (const std::exception&) {
                    rm = static_cast<int>(-(1 + static_cast<int64_t>(i)));
                    break;
                }
                mine[i * 4 + 0] = hp.should_try();
                mine[i * 4 + 1] = hp.exhausted();
                mine[i * 4 + 2] = hp.activations();
                mine[i * 4 + 3] = hp.deactivations();
            }
            CHECK(rm == rr);
            CHECK(mine == theirs);
            ++cases;
        }
    // History cache: small alphabets so suffixes recur.
    const std::size_t cap = 8;
    for (uint64_t lo : {0, 1, 2, 3})
        for (uint64_t hi : {2, 3, 5, 6})
            for (int rep = 0; rep < 20; ++rep) {
                const std::size_t n = 1 + uni(0, 120);
                const uint32_t alpha = static_cast<uint32_t>(2 + uni(0, 6));
                std::vector<uint32_t> t(n);
                for (auto& v : t) v = static_cast<uint32_t>(uni(0, alpha - 1));
                std::vector<uint64_t> mt(n);
                for (auto& v : mt) v = uni(0, 7);
                std::vector<uint32_t> theirs(n * cap, 0);
                std::vector<uint64_t> counts(n, 0);
                const int rr = ref.hcache_run(lo, hi, t.data(), static_cast<int64_t>(n), mt.data(), cap, theirs.data(),
                                              counts.data());
                int rm = 0;
                bool same = true;
                try {
                    HistoryDraftCache c(lo, hi);
                    for (std::size_t i = 0; i < n; ++i) {
                        c.append(t[i]);
                        const std::vector<uint32_t> p = c.propose(mt[i]);
                        same &= p.size() == counts[i];
                        for (std::size_t j = 0; j < p.size() && j < cap; ++j) same &= p[j] == theirs[i * cap + j];
                    }
                } catch (const std::exception&) {
                    rm = -1;
                }
                CHECK(rm == rr);
                if (rr == 0) CHECK(same);
                ++cases;
            }
    // Context copy: prompts with planted repeats; histories cut from the prompt plus noise.
    for (int rep = 0; rep < 600; ++rep) {
        const uint64_t lo = 1 + uni(0, 6), hi = lo + uni(0, 5) - (uni(0, 20) == 0 ? 6 : 0);
        const uint32_t alpha = static_cast<uint32_t>(2 + uni(0, 5));
        std::vector<uint32_t> prompt(uni(0, 80));
        for (auto& v : prompt) v = static_cast<uint32_t>(uni(0, alpha - 1));
        if (prompt.size() > 20 && uni(0, 1)) {  // plant a copy of an earlier span
            const std::size_t len = uni(4, 12), from = uni(0, prompt.size() / 2), to = uni(prompt.size() / 2, prompt.size() - 1);
            for (std::size_t i = 0; i < len && to + i < prompt.size() && from + i < prompt.size(); ++i)
                prompt[to + i] = prompt[from + i];
        }
        std::vector<uint32_t> hist;
        if (!prompt.empty() && uni(0, 2) != 0) {
            const std::size_t b = uni(0, prompt.size() - 1), e = uni(b, prompt.size());
            for (std::size_t i = 0; i < uni(0, 3); ++i) hist.push_back(static_cast<uint32_t>(uni(0, alpha)));
            hist.insert(hist.end(), prompt.begin() + static_cast<std::ptrdiff_t>(b),
                        prompt.begin() + static_cast<std::ptrdiff_t>(e));
        } else {
            hist.resize(uni(0, 20));
            for (auto& v : hist) v = static_cast<uint32_t>(uni(0, alpha));
        }
        const uint64_t mt = uni(0, 30);
        for (int completion : {0, 1}) {
            std::vector<uint32_t> theirs(64, 0);
            uint64_t count = 0, ext = 0;
            const int rr = ref.copy(prompt.data(), static_cast<int64_t>(prompt.size()), lo, hi, hist.data(),
                                    static_cast<int64_t>(hist.size()), mt, completion, 64, theirs.data(), &count, &ext);
            int rm = 0;
            ContextCopyProposal mine;
            try {
                ContextCopyCache c(prompt, lo, hi);
                mine = completion ? c.propose_completion(hist, mt) : c.propose(hist, mt);
            } catch (const std::exception&) {
                rm = -1;
            }
            CHECK(rm == rr);
            if (rr == 0) {
                theirs.resize(std::min<uint64_t>(count, 64));
                CHECK(mine.tokens == theirs && mine.match_extension == ext);
            }
            ++cases;
        }
    }
    std::printf("differential: %d random cases against the reference's compiled policy\n", cases);
}

// ------------------------------------------------------------------ 3. scheduler
// Exact fake target: the greedy token after t is next(t); checkpoints are counted per slot.
struct FakeVerifier final : BatchVerifier {
    std::function<std::uint32_t(std::uint32_t)> next;
    std::size_t width = 16;
    std::vector<std::size_t> staged, committed;
    std::size_t calls = 0, max_rows_seen = 0;
    bool bad = false;
    explicit FakeVerifier(std::size_t slots) : staged(slots, 0), committed(slots, 0) {}
    std::size_t max_rows() const override { return width; }
    std::vector<std::vector<std::uint32_t>> verify(std::span<const SlotVerifyRows> batch) override {
        calls += 1;
        std::size_t rows = 0;
        std::set<std::size_t> seen;
        std::vector<std::vector<std::uint32_t>> out;
        for (const SlotVerifyRows& e : batch) {
            bad |= !seen.insert(e.slot).second || e.slot >= staged.size();
            rows += e.drafts.size() + 1;
            std::vector<std::uint32_t> t{next(e.current_token)};
            for (const std::uint32_t d : e.drafts) t.push_back(next(d));
            staged[e.slot] = e.drafts.size() + 1;
            out.push_back(std::move(t));
        }
        max_rows_seen = std::max(max_rows_seen, rows);
        bad |= rows > width;
        return out;
    }
    void commit(std::size_t slot, std::size_t accepted) override {
        bad |= staged[slot] == 0 || accepted >= staged[slot];
        committed[slot] += accepted + 1;
        staged[slot] = 0;
    }
};

// Proposes the true continuation with probability p per position (else a wrong token).
struct NoisyDrafter final : LearnedDrafter {
    std::function<std::uint32_t(std::uint32_t)> next;
    double p;
    std::mt19937_64 rng;
    NoisyDrafter(std::function<std::uint32_t(std::uint32_t)> f, double prob, uint64_t seed)
        : next(std::move(f)), p(prob), rng(seed) {}
    std::vector<std::uint32_t> propose(std::size_t, std::uint32_t cur, std::size_t depth) override {
        std::vector<std::uint32_t> d;
        std::uniform_real_distribution<double> u(0.0, 1.0);
        for (std::size_t i = 0; i < depth; ++i) {
            const std::uint32_t truth = next(cur);
            cur = u(rng) < p ? truth : truth + 1000;  // off-vocabulary of the fake target: never accepted
            d.push_back(cur);
        }
        return d;
    }
};

static std::vector<std::uint32_t> greedy_reference(const std::function<std::uint32_t(std::uint32_t)>& next,
                                                   std::uint32_t cur, std::size_t max_tokens,
                                                   const std::vector<std::uint32_t>& stop) {
    std::vector<std::uint32_t> out;
    while (out.size() < max_tokens) {
        cur = next(cur);
        if (std::find(stop.begin(), stop.end(), cur) != stop.end()) break;
        out.push_back(cur);
    }
    return out;
}

struct Run {
    std::vector<std::vector<SlotRound>> per_request;
};

static Run drive(MtpSlotScheduler& s, std::size_t requests, std::size_t max_steps = 1000) {
    Run run;
    run.per_request.resize(requests);
    for (std::size_t step = 0; step < max_steps && !s.done(); ++step)
        for (const SlotRound& r : s.step()) run.per_request[r.slot].push_back(r);
    return run;
}

static void scheduler_tests(const Ref* ref) {
    clear_env();
    // A permutation on 0..96 made of one long cycle: greedy text repeats with period 97.
    const auto next = [](std::uint32_t t) -> std::uint32_t { return (t * 5 + 3) % 97; };
    {   // 5 requests at depth 4 (25 rows per round > 16): several batches, output = greedy
        FakeVerifier v(5);
        v.next = next;
        NoisyDrafter d(next, 0.8, 7);
        MtpSchedulerOptions o;
        o.mtp_depth = 4;
        o.history_mode = HistoryDraftMode::disabled;
        MtpSlotScheduler s(v, &d, o);
        std::vector<std::vector<std::uint32_t>> prompts;
        for (std::size_t i = 0; i < 5; ++i) {
            prompts.push_back({static_cast<std::uint32_t>(3 + i), static_cast<std::uint32_t>(40 + 7 * i)});
            s.add_request(i, prompts.back(), 1, 30 + i);
        }
        const Run run = drive(s, 5);
        CHECK(s.done() && !v.bad && v.max_rows_seen <= 16);
        CHECK(s.batches() > run.per_request[0].size());  // rounds needed more than one batch
        for (std::size_t i = 0; i < 5; ++i) {
            CHECK(s.tokens(i) == greedy_reference(next, prompts[i].back(), 30 + i, {}));
            CHECK(s.stats(i).finish_reason == "length");
            CHECK(v.committed[i] + 1 == s.query_position(i));
            std::size_t accepted = 0;
            for (const SlotRound& r : run.per_request[i]) accepted += r.accepted;
            CHECK(accepted == s.stats(i).mtp_accepted && accepted > 0);
        }
    }
    {   // a drafter that is always wrong: two zero-accept learned rounds, then serial decoding
        FakeVerifier v(2);
        v.next = next;
        NoisyDrafter d(next, 0.0, 8);
        MtpSchedulerOptions o;
        o.history_mode = HistoryDraftMode::disabled;
        MtpSlotScheduler s(v, &d, o);
        const std::vector<std::uint32_t> prompt{5, 6, 7};
        s.add_request(0, prompt, 2, 20);
        s.add_request(1, prompt, 2, 20);
        const Run run = drive(s, 2);
        for (std::size_t i = 0; i < 2; ++i) {
            CHECK(s.tokens(i) == greedy_reference(next, 7, 20, {}));
            CHECK(s.stats(i).mtp_rounds == 2 && s.stats(i).mtp_fallbacks == 1 && s.stats(i).mtp_accepted == 0);
            CHECK(s.stats(i).serial_steps == 18);
            CHECK(run.per_request[i][0].source == DraftSourceKind::learned);
            CHECK(run.per_request[i][0].draft_tokens.size() == 2);  // depth 3 probes at 2
            CHECK(run.per_request[i].back().source == DraftSourceKind::serial);
        }
        CHECK(!v.bad);
    }
    {   // forced history drafts on a repeating text: they are exact once the period has been seen
        FakeVerifier v(1);
        v.next = next;
        NoisyDrafter d(next, 0.0, 9);
        MtpSchedulerOptions o;
        o.history_mode = HistoryDraftMode::forced;
        o.zero_accept_fallback_rounds = 1000;
        o.economic_fallback = false;
        MtpSlotScheduler s(v, &d, o);
        std::vector<std::uint32_t> prompt{11};
        for (int i = 0; i < 120; ++i) prompt.push_back(next(prompt.back()));  // more than one period
        s.add_request(0, prompt, prompt.size() - 1, 60);
        drive(s, 1);
        CHECK(s.tokens(0) == greedy_reference(next, prompt.back(), 60, {}));
        CHECK(s.stats(0).history_draft_rounds > 0 && s.stats(0).history_draft_accepted > 0);
        CHECK(s.stats(0).history_draft_accepted == s.stats(0).history_draft_proposed);
        CHECK(!v.bad);
    }
    {   // context copies from the prompt (opt-in): capped to the verifier width
        FakeVerifier v(1);
        v.next = next;
        NoisyDrafter d(next, 0.5, 10);
        MtpSchedulerOptions o;
        o.context_copy = true;
        o.context_copy_max_tokens = 24;
        o.history_mode = HistoryDraftMode::disabled;
        MtpSlotScheduler s(v, &d, o);
        std::vector<std::uint32_t> prompt{17};
        for (int i = 0; i < 150; ++i) prompt.push_back(next(prompt.back()));
        s.add_request(0, prompt, prompt.size() - 1, 80);
        const Run run = drive(s, 1);
        CHECK(s.tokens(0) == greedy_reference(next, prompt.back(), 80, {}));
        CHECK(s.stats(0).context_copy_rounds > 0 && s.stats(0).context_copy_accepted > 0);
        std::size_t longest = 0;
        for (const SlotRound& r : run.per_request[0]) longest = std::max(longest, r.draft_tokens.size());
        CHECK(longest <= 15 && !v.bad && v.max_rows_seen <= 16);
    }
    {   // a stop token inside the greedy text ends the request before it
        FakeVerifier v(1);
        v.next = next;
        NoisyDrafter d(next, 0.9, 11);
        MtpSchedulerOptions o;
        const std::vector<std::uint32_t> truth = greedy_reference(next, 4, 50, {});
        o.stop_tokens = {truth[9]};
        MtpSlotScheduler s(v, &d, o);
        s.add_request(0, std::vector<std::uint32_t>{4}, 0, 50);
        drive(s, 1);
        CHECK(s.tokens(0) == greedy_reference(next, 4, 50, o.stop_tokens));
        CHECK(s.tokens(0).size() == 9 && s.stats(0).finish_reason == "stop");
    }
    {   // replaying each request's learned rounds into a fresh policy reproduces its statistics
        FakeVerifier v(3);
        v.next = next;
        NoisyDrafter d(next, 0.55, 12);
        MtpSchedulerOptions o;
        o.history_mode = HistoryDraftMode::disabled;
        o.zero_accept_fallback_rounds = 1000;
        o.economic_fallback = false;
        MtpSlotScheduler s(v, &d, o);
        for (std::size_t i = 0; i < 3; ++i) s.add_request(i, std::vector<std::uint32_t>{static_cast<std::uint32_t>(i)}, 0, 200);
        const Run run = drive(s, 3);
        for (std::size_t i = 0; i < 3; ++i) {
            CHECK(s.tokens(i) == greedy_reference(next, static_cast<std::uint32_t>(i), 200, {}));
            std::vector<uint64_t> p, a;
            MtpDepthPolicy replay(3, 1);
            for (const SlotRound& r : run.per_request[i])
                if (r.source == DraftSourceKind::learned) {
                    replay.observe(r.draft_tokens.size(), r.accepted);
                    p.push_back(r.draft_tokens.size());
                    a.push_back(r.accepted);
                }
            CHECK(replay.depth() == s.stats(i).mtp_final_depth && replay.promotions() == s.stats(i).mtp_promotions &&
                  replay.demotions() == s.stats(i).mtp_demotions);
            if (ref) {
                std::vector<uint64_t> theirs((p.size() + 1) * 4);
                CHECK(ref->depth_run(3, 1, 0, p.data(), a.data(), static_cast<int64_t>(p.size()), theirs.data()) == 0);
                CHECK(theirs[p.size() * 4 + 0] == s.stats(i).mtp_final_depth &&
                      theirs[p.size() * 4 + 1] == s.stats(i).mtp_promotions &&
                      theirs[p.size() * 4 + 2] == s.stats(i).mtp_demotions);
            }
        }
    }
    {   // one token left: a serial step; no drafter: serial decoding throughout
        FakeVerifier v(2);
        v.next = next;
        MtpSlotScheduler s(v, nullptr, MtpSchedulerOptions{});
        s.add_request(0, std::vector<std::uint32_t>{8}, 0, 1);
        s.add_request(1, std::vector<std::uint32_t>{9}, 0, 5);
        const Run run = drive(s, 2);
        CHECK(s.tokens(0) == greedy_reference(next, 8, 1, {}) && s.tokens(1) == greedy_reference(next, 9, 5, {}));
        CHECK(run.per_request[1].size() == 5 && s.stats(1).serial_steps == 5 && s.batches() == 5);
        CHECK(thrown([&] { s.add_request(1, std::vector<std::uint32_t>{}, 0, 3); }) == "request prompt is empty");
    }
    {   // a slot can hold one unfinished request at a time
        FakeVerifier v(1);
        v.next = next;
        MtpSlotScheduler s(v, nullptr, MtpSchedulerOptions{});
        s.add_request(0, std::vector<std::uint32_t>{1}, 0, 3);
        CHECK(thrown([&] { s.add_request(0, std::vector<std::uint32_t>{2}, 0, 3); }) ==
              "slot already holds an unfinished request");
    }
}

int main(int argc, char** argv) {
    known_answers_depth();
    known_answers_profitability();
    known_answers_history();
    Ref ref;
    const bool have_ref = argc > 1 && ref.load(argv[1]);
    if (have_ref) differential(ref);
    else std::printf("differential: SKIPPED (no reference library%s%s)\n", argc > 1 ? " at " : "", argc > 1 ? argv[1] : "");
    scheduler_tests(have_ref ? &ref : nullptr);
    std::printf("%d checks, %d failures\n", g_checks, g_fail);
    return g_fail == 0 ? 0 : 1;
}
