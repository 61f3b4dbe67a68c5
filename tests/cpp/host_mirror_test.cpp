// host_mirror_test.cpp — tests of the C++20 host interface (qwen38-flash.cpp_amd/host/),
// written like the reference's own tests:
//   host section   KATs restated from tests/quantization_geometry_test.cpp:48-84 and
//                  tests/mtp_lifecycle_test.cpp:39-71, and the exception types of
//                  include/qwen38/mtp_verifier.hpp:39-47 / quantization_geometry.hpp.
//   --gpu section  a verify model on the device: SparseMoe routes and outputs through the
//                  C++ interface equal the C ABI's, a verify + commit round keeps the
//                  reference's lifecycle (rows = k + 1, accepted <= k, token_count =
//                  q + accepted + 1, failed validation leaves state intact).
// Prints one line per section and exits non-zero on the first failed check.
#include "qwen38_verify.hpp"

#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <algorithm>
#include <cstring>
#include <memory>
#include <optional>
#include <stdexcept>
#include <vector>

#define CHECK(cond)                                                             \
    do {                                                                        \
        if (!(cond)) {                                                          \
            std::fprintf(stderr, "check failed %s:%d: %s\n", __FILE__, __LINE__, #cond); \
            std::exit(1);                                                       \
        }                                                                       \
    } while (0)

template <typename E, typename F>
bool throws(F&& f) {
    try {
        f();
    } catch (const E&) {
        return true;
    } catch (...) {
        return false;
    }
    return false;
}

static void host_tests() {
    // packed-VQ geometry (tests/quantization_geometry_test.cpp:48-84)
    constexpr std::size_t bits = 14;
    std::vector<std::uint32_t> expected(67);
    for (std::size_t i = 0; i < expected.size(); ++i) expected[i] = static_cast<std::uint32_t>((i * 997 + 17) & 0x3FFF);
    std::vector<std::uint32_t> packed(qwen38::packed_vq_word_count(expected.size(), bits), 0);
    for (std::size_t i = 0; i < expected.size(); ++i) {
        const std::size_t off = (i % 32) * bits, word = (i / 32) * bits + off / 32, sh = off % 32;
        const std::uint64_t v = static_cast<std::uint64_t>(expected[i]) << sh;
        packed[word] |= static_cast<std::uint32_t>(v);
        if (sh + bits > 32) packed[word + 1] |= static_cast<std::uint32_t>(v >> 32);
    }
    CHECK(packed.size() == 42);
    for (std::size_t i = 0; i < expected.size(); ++i) CHECK(qwen38::unpack_vq_code(packed, i, bits) == expected[i]);
    CHECK(throws<std::out_of_range>([&] {
        (void)qwen38::unpack_vq_code(std::span<const std::uint32_t>(packed.data(), 13), 31, bits);
    }));
    std::vector<std::uint32_t> packed8(qwen38::packed_vq_word_count(160, 8));
    for (std::size_t i = 0; i < 160; ++i)
        packed8[i / 4] |= static_cast<std::uint32_t>((i * 17 + 255) % 256) << ((i % 4) * 8);
    CHECK(packed8.size() == 40);
    for (std::size_t i = 0; i < 160; ++i) CHECK(qwen38::unpack_vq_code(packed8, i, 8) == (i * 17 + 255) % 256);
    CHECK(qwen38::supports_segmented_vq(8, 14) && qwen38::supports_segmented_vq(4, 8));

    // lifecycle (tests/mtp_lifecycle_test.cpp:39-71)
    const auto partial = qwen38::plan_mtp_commit(12, 3, 1);
    CHECK(partial.truncate_head_to == 12 && partial.target_rows_to_keep == 2 && partial.stash_rows == 2 &&
          partial.committed_boundary == 14);
    CHECK(throws<std::runtime_error>([] { (void)qwen38::plan_mtp_commit(0, 1, 2); }));
    const std::vector<std::uint32_t> drafts{10, 20, 30};
    const auto zero = qwen38::decide_mtp_greedy(drafts, std::vector<std::uint32_t>{11, 20, 30, 40});
    CHECK(zero.accepted == 0 && zero.correction_row == 0 && zero.next_token == 11);
    const auto part = qwen38::decide_mtp_greedy(drafts, std::vector<std::uint32_t>{10, 20, 31, 40});
    CHECK(part.accepted == 2 && part.correction_row == 2 && part.next_token == 31);
    const auto full = qwen38::decide_mtp_greedy(drafts, std::vector<std::uint32_t>{10, 20, 30, 40});
    CHECK(full.accepted == 3 && full.correction_row == 3 && full.next_token == 40);
    const auto stopped = qwen38::decide_mtp_greedy(drafts, std::vector<std::uint32_t>{10, 20, 30, 40},
                                                   std::vector<std::uint32_t>{20, 99});
    CHECK(stopped.accepted == 1 && stopped.correction_row == 1 && stopped.next_token == 20);
    CHECK(throws<std::runtime_error>(
        [&] { (void)qwen38::decide_mtp_greedy(drafts, std::vector<std::uint32_t>{10, 20, 30}); }));
    std::printf("host section: ok\n");
}

// The engine-side round driver over the GPU: 3 requests share each batched verification.
// Every recorded batch is recomputed row by row in the same kernel family (a row alone when
// the batch had at most 4 rows, else the row with 4 fixed companions: rows of a batch are
// independent within a family), so the greedy tokens and logits must match exactly; each
// state's committed length and hidden row follow the scheduler's commits.
static void batched_slot_tests(const qwen38::Context& ctx, const qwen38::QwenModel& model) {
    struct Recording final : qwen38::BatchVerifier {
        qwen38::QwenBatchVerifier& inner;
        std::vector<std::vector<qwen38::SlotVerifyRows>> batches;
        std::vector<std::vector<std::vector<std::uint32_t>>> targets;
        std::vector<std::vector<std::size_t>> accepted;
        explicit Recording(qwen38::QwenBatchVerifier& v) : inner(v) {}
        std::size_t max_rows() const override { return inner.max_rows(); }
        std::vector<std::vector<std::uint32_t>> verify(std::span<const qwen38::SlotVerifyRows> b) override {
            auto t = inner.verify(b);
            batches.emplace_back(b.begin(), b.end());
            targets.push_back(t);
            accepted.emplace_back();
            return t;
        }
        void commit(std::size_t slot, std::size_t a) override {
            inner.commit(slot, a);
            accepted.back().push_back(a);
        }
    };
    // Drafts from the (token -> target) pairs seen so far; unseen tokens get a made-up successor.
    struct MemoDrafter final : qwen38::LearnedDrafter {
        Recording* rec = nullptr;
        std::size_t vocab = 0;
        std::vector<std::uint32_t> propose(std::size_t, std::uint32_t cur, std::size_t depth) override {
            std::vector<std::uint32_t> d;
            for (std::size_t i = 0; i < depth; ++i) {
                std::uint32_t nxt = static_cast<std::uint32_t>((cur * 31u + 7u) % vocab);
                for (std::size_t b = 0; b < rec->batches.size(); ++b)
                    for (std::size_t e = 0; e < rec->batches[b].size(); ++e) {
                        const auto& rows = rec->batches[b][e];
                        if (rows.current_token == cur) nxt = rec->targets[b][e][0];
                        for (std::size_t j = 0; j < rows.drafts.size(); ++j)
                            if (rows.drafts[j] == cur) nxt = rec->targets[b][e][j + 1];
                    }
                d.push_back(nxt);
                cur = nxt;
            }
            return d;
        }
    };
    std::vector<std::unique_ptr<qwen38::ModelDecodeState>> states;
    std::vector<qwen38::ModelDecodeState*> ptrs;
    for (std::size_t i = 0; i < 3; ++i) {
        states.push_back(std::make_unique<qwen38::ModelDecodeState>(model, 10 + i, 16));
        ptrs.push_back(states.back().get());
    }
    qwen38::QwenBatchVerifier gpu(model, ptrs);
    Recording rec(gpu);
    MemoDrafter drafter;
    drafter.rec = &rec;
    drafter.vocab = model.vocab();
    qwen38::MtpSchedulerOptions opt;
    opt.zero_accept_fallback_rounds = 1000;
    opt.economic_fallback = false;
    qwen38::MtpSlotScheduler sched(rec, &drafter, opt);
    for (std::size_t i = 0; i < 3; ++i) {
        const std::vector<std::uint32_t> prompt{static_cast<std::uint32_t>(100 + i), static_cast<std::uint32_t>(200 + 3 * i)};
        sched.add_request(i, prompt, 10 + i, 20);
    }
    std::size_t rounds = 0;
    while (!sched.done() && rounds < 100) {
        (void)sched.step();
        ++rounds;
        // the last verification's committed rows are the slots' committed hidden rows
        const auto& b = rec.batches.back();
        const qwen38::DeviceTensor& fm = gpu.last_final_mixed();
        const std::size_t H = model.hidden();
        std::vector<std::uint16_t> all(fm.numel()), mine(H);
        fm.download(all.data(), all.size() * 2);
        std::size_t row = 0;
        for (std::size_t e = 0; e < b.size(); ++e) {
            const std::size_t a = rec.accepted.back()[e];
            CHECK(hipMemcpy(mine.data(), q38_slot_hidden(ptrs[b[e].slot]->slot()), H * 2, hipMemcpyDeviceToHost) ==
                  hipSuccess);
            CHECK(std::equal(mine.begin(), mine.end(), all.begin() + static_cast<std::ptrdiff_t>((row + a) * H)));
            row += b[e].drafts.size() + 1;
        }
    }
    CHECK(sched.done());
    std::size_t recomputed = 0, wide = 0, accepted_total = 0;
    const std::vector<std::uint32_t> companions{3, 1, 4, 1};
    for (std::size_t bi = 0; bi < rec.batches.size(); ++bi) {
        std::size_t rows = 0;
        for (const auto& e : rec.batches[bi]) rows += e.drafts.size() + 1;
        wide += rows > 4;
        for (std::size_t e = 0; e < rec.batches[bi].size(); ++e) {
            const auto& rs = rec.batches[bi][e];
            std::vector<std::uint32_t> toks{rs.current_token};
            toks.insert(toks.end(), rs.drafts.begin(), rs.drafts.end());
            accepted_total += rec.accepted[bi][e];
            for (std::size_t j = 0; j < toks.size(); ++j) {
                std::vector<std::uint32_t> alone{toks[j]};
                if (rows > 4) alone.insert(alone.end(), companions.begin(), companions.end());
                qwen38::DeviceTensor f1;
                std::vector<qwen38::GreedyStep> g1;
                model.forward_verify_layer_major(alone, f1, g1);
                CHECK(g1[0].token == rec.targets[bi][e][j]);
                ++recomputed;
            }
        }
    }
    for (std::size_t i = 0; i < 3; ++i) {
        CHECK(sched.tokens(i).size() == 20 && sched.stats(i).finish_reason == "length");
        CHECK(states[i]->token_count() == sched.query_position(i));
    }
    CHECK(wide > 0 && accepted_total > 0);
    std::printf("batched slots: ok (%zu rounds, %zu verifications, %zu wide, %zu rows recomputed, %zu accepted)\n",
                rounds, rec.batches.size(), wide, recomputed, accepted_total);
}

// The MTP draft head and the learned-draft round (run_greedy_mtp_round_reference): drafts
// equal the head's chain on the previous target stream and a host replay of single steps;
// the round keeps the reference's lifecycle (target length q + accepted + 1, head positions
// advanced over the committed rows only, next stream = the correction row's pre-norm stream);
// bad depths and positions throw with both states intact; the batched scheduler drafts
// with the head once a slot has a committed stream.
// HyperConnection mirror: initialize_stream tiles the embedding; read and write give the C
// ABI's results bit for bit (one kernel family); shape errors throw as the reference does.
static void hyper_connection_tests(const qwen38::Context& ctx) {
    const std::size_t H = 2048, HC = 4, R = 256, G = 64, K = H * HC, M = 4;
    std::uint64_t st = 0x9E3779B97F4A7C15ull;
    auto next = [&] { st = st * 6364136223846793005ull + 1442695040888963407ull; return static_cast<std::uint32_t>(st >> 32); };
    auto bf16 = [](float f) { std::uint32_t u; std::memcpy(&u, &f, 4); return static_cast<std::uint16_t>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16); };
    auto unit = [&] { return (static_cast<float>(next() >> 8) / 16777216.0f) - 0.5f; };
    auto upload_u32 = [&](std::size_t n) {
        std::vector<std::uint32_t> h(n);
        for (auto& v : h) v = next();
        qwen38::DeviceTensor t({n}, qwen38::DType::u32);
        t.upload(h.data(), n * 4);
        return t;
    };
    auto upload_bf16 = [&](std::size_t n, float scale, float offset) {
        std::vector<std::uint16_t> h(n);
        for (auto& v : h) v = bf16(offset + scale * unit());
        qwen38::DeviceTensor t({n}, qwen38::DType::bf16);
        t.upload(h.data(), n * 2);
        return t;
    };
    // centred 4-bit groups: weight = q * s + b with b ~ -7.5 s
    auto norm = upload_bf16(K, 0.2f, 0.0f);
    auto dw = upload_u32(R * K / 8), ds = upload_bf16(R * K / G, 0.004f, 0.006f), db = upload_bf16(R * K / G, 0.002f, -0.045f);
    auto uw = upload_u32(K * R / 8), us = upload_bf16(K * R / G, 0.004f, 0.006f), ub = upload_bf16(K * R / G, 0.002f, -0.045f);
    auto iw = upload_u32(HC * K / 8), is = upload_bf16(HC * K / G, 0.004f, 0.006f), ib = upload_bf16(HC * K / G, 0.002f, -0.045f);
    auto u16 = [](const qwen38::DeviceTensor& t) { return static_cast<const std::uint16_t*>(t.data()); };
    auto u32 = [](const qwen38::DeviceTensor& t) { return static_cast<const std::uint32_t*>(t.data()); };
    const q38_hc_weights w{u16(norm), u32(dw), u16(ds), u16(db), u32(uw), u16(us), u16(ub), u32(iw), u16(is), u16(ib)};
    qwen38::HyperConnection hc(ctx, w, H, HC, R, 4, G, 1e-6f, true);

    auto emb = upload_bf16(M * H, 2.0f, 0.0f);
    qwen38::DeviceTensor emb3({1, M, H}, qwen38::DType::bf16);
    CHECK(hipMemcpy(emb3.data(), emb.data(), M * H * 2, hipMemcpyDeviceToDevice) == hipSuccess);
    const qwen38::DeviceTensor stream = qwen38::HyperConnection::initialize_stream(ctx, emb3, HC);
    ctx.synchronize();
    CHECK(stream.shape() == (std::vector<std::size_t>{1, M, K}));
    {
        const auto e = emb3.to_host<std::uint16_t>();
        const auto s = stream.to_host<std::uint16_t>();
        for (std::size_t r = 0; r < M; ++r)
            for (std::size_t h = 0; h < HC; ++h)
                CHECK(std::equal(e.begin() + static_cast<std::ptrdiff_t>(r * H), e.begin() + static_cast<std::ptrdiff_t>((r + 1) * H),
                                 s.begin() + static_cast<std::ptrdiff_t>(r * K + h * H)));
    }
    const qwen38::HyperConnectionRead rd = hc.read(stream);
    CHECK(rd.has_injection && rd.mixed.shape() == (std::vector<std::size_t>{1, M, H}) &&
          rd.injection.shape() == (std::vector<std::size_t>{1, M, HC, 1}));
    // the same read through the C ABI
    qwen38::DeviceTensor mixed2({M, H}, qwen38::DType::bf16), inj2({M, HC}, qwen38::DType::bf16);
    const std::size_t wsb = q38_hc_workspace_size(&hc.desc(), static_cast<int32_t>(M));
    qwen38::DeviceTensor ws({wsb}, qwen38::DType::u32);
    CHECK(q38_hc_read(hc.handle(), u16(stream), static_cast<int32_t>(M), static_cast<std::uint16_t*>(mixed2.data()),
                      static_cast<std::uint16_t*>(inj2.data()), ws.data(), ws.nbytes(), ctx.stream()) == Q38_OK);
    ctx.synchronize();
    CHECK(rd.mixed.to_host<std::uint16_t>() == mixed2.to_host<std::uint16_t>());
    CHECK(rd.injection.to_host<std::uint16_t>() == inj2.to_host<std::uint16_t>());
    // write with the block input standing in for the block output
    const qwen38::DeviceTensor out = hc.write(stream, rd.mixed, rd.injection);
    qwen38::DeviceTensor out2({M, K}, qwen38::DType::bf16);
    CHECK(q38_hc_write(hc.handle(), u16(stream), u16(rd.mixed), u16(rd.injection), static_cast<int32_t>(M),
                       static_cast<std::uint16_t*>(out2.data()), ctx.stream()) == Q38_OK);
    ctx.synchronize();
    CHECK(out.to_host<std::uint16_t>() == out2.to_host<std::uint16_t>());
    CHECK(out.to_host<std::uint16_t>() != stream.to_host<std::uint16_t>());
    // shape and argument errors
    qwen38::DeviceTensor bad({1, M, K - 8}, qwen38::DType::bf16);
    CHECK(throws<std::runtime_error>([&] { (void)hc.read(bad); }));
    CHECK(throws<std::runtime_error>([&] { (void)hc.write(stream, rd.injection, rd.injection); }));
    CHECK(throws<std::runtime_error>([&] {
        qwen38::HyperConnection bad_eps(ctx, w, H, HC, R, 4, G, 0.0f, true);
    }));
    CHECK(throws<std::runtime_error>([&] {
        qwen38::HyperConnection bad_rank(ctx, w, H, HC, 100, 4, G, 1e-6f, true);
    }));
    std::printf("hyper connection: ok\n");
}

// GatedDeltaNet mirror: forward_verify equals the C ABI call bit for bit (outputs and the
// checkpoint block); S rows equal S one-row calls each from the previous call's last
// checkpoint; shape and geometry errors throw with the reference's messages.
static void gated_delta_net_tests(const qwen38::Context& ctx) {
    const std::size_t H = 512, HK = 2, HV = 4, D = 128, C = 2 * HK * D + HV * D, VW = HV * D, S = 4, G = 64;
    std::uint64_t st = 0x2545F4914F6CDD1Dull;
    auto next = [&] { st = st * 6364136223846793005ull + 1442695040888963407ull; return static_cast<std::uint32_t>(st >> 32); };
    auto bf16 = [](float f) { std::uint32_t u; std::memcpy(&u, &f, 4); return static_cast<std::uint16_t>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16); };
    auto unit = [&] { return (static_cast<float>(next() >> 8) / 16777216.0f) - 0.5f; };
    auto upload_u32 = [&](std::size_t n) {
        std::vector<std::uint32_t> h(n);
        for (auto& v : h) v = next();
        qwen38::DeviceTensor t({n}, qwen38::DType::u32);
        t.upload(h.data(), n * 4);
        return t;
    };
    auto upload_bf16 = [&](std::size_t n, float scale, float offset) {
        std::vector<std::uint16_t> h(n);
        for (auto& v : h) v = bf16(offset + scale * unit());
        qwen38::DeviceTensor t({n}, qwen38::DType::bf16);
        t.upload(h.data(), n * 2);
        return t;
    };
    const std::size_t outs[5] = {C, VW, HV, HV, H}, ins[5] = {H, H, H, H, VW};
    std::vector<qwen38::DeviceTensor> keep;
    q38_gdn_weights w{};
    for (int p = 0; p < 5; ++p) {  // 8-bit, centred: weight = q * s + b with b ~ -127.5 s
        keep.push_back(upload_u32(outs[p] * ins[p] / 4));
        keep.push_back(upload_bf16(outs[p] * ins[p] / G, 0.0001f, 0.00015f));
        keep.push_back(upload_bf16(outs[p] * ins[p] / G, 0.002f, -0.019f));
        w.weight[p] = static_cast<const std::uint32_t*>(keep[keep.size() - 3].data());
        w.scales[p] = static_cast<const std::uint16_t*>(keep[keep.size() - 2].data());
        w.biases[p] = static_cast<const std::uint16_t*>(keep[keep.size() - 1].data());
    }
    keep.push_back(upload_bf16(C * 4, 1.0f, 0.0f));
    w.conv = static_cast<const std::uint16_t*>(keep.back().data());
    std::vector<float> alog(HV, 0.5f);
    qwen38::DeviceTensor alog_t({HV}, qwen38::DType::f32);
    alog_t.upload(alog.data(), HV * 4);
    w.a_log = static_cast<const float*>(alog_t.data());
    keep.push_back(upload_bf16(HV, 1.0f, 0.0f));
    w.dt_bias = static_cast<const std::uint16_t*>(keep.back().data());
    keep.push_back(upload_bf16(D, 0.5f, 1.0f));
    w.norm = static_cast<const std::uint16_t*>(keep.back().data());
    qwen38::GatedDeltaNet gdn(ctx, w, H, HK, HV, D, D, 4, 8, static_cast<int>(G), false, "sigmoid", 1e-6f);
    const std::size_t sb = gdn.state_bytes();
    CHECK(sb == (3 * C + VW * D) * 2);

    auto x = upload_bf16(S * H, 2.0f, 0.0f);
    qwen38::DeviceTensor x3({1, S, H}, qwen38::DType::bf16);
    CHECK(hipMemcpy(x3.data(), x.data(), S * H * 2, hipMemcpyDeviceToDevice) == hipSuccess);
    qwen38::GatedDeltaNetState origin;
    origin.block = upload_bf16(sb / 2, 0.1f, 0.0f);
    origin.initialized = true;
    std::vector<qwen38::GatedDeltaNetState> ck;
    const qwen38::DeviceTensor out = gdn.forward_verify(x3, origin, ck);
    CHECK(ck.size() == S && out.shape() == (std::vector<std::size_t>{1, S, H}));
    // the same call through the C ABI
    qwen38::DeviceTensor out2({S, H}, qwen38::DType::bf16), blk2({S * sb / 2}, qwen38::DType::bf16);
    qwen38::DeviceTensor ws({q38_gdn_workspace_size(gdn.handle(), static_cast<int32_t>(S))}, qwen38::DType::u32);
    CHECK(q38_gdn_verify(gdn.handle(), static_cast<const std::uint16_t*>(x3.data()), static_cast<int32_t>(S),
                         origin.data(), blk2.data(), static_cast<std::uint16_t*>(out2.data()), ws.data(), ws.nbytes(),
                         ctx.stream()) == Q38_OK);
    ctx.synchronize();
    CHECK(out.to_host<std::uint16_t>() == out2.to_host<std::uint16_t>());
    CHECK(ck[0].block.to_host<std::uint16_t>() == blk2.to_host<std::uint16_t>());
    // row by row from the previous call's checkpoint
    qwen38::GatedDeltaNetState state;
    state.block = origin.block.share();
    state.initialized = true;
    const auto want = out.to_host<std::uint16_t>();
    for (std::size_t r = 0; r < S; ++r) {
        qwen38::DeviceTensor xr({1, 1, H}, qwen38::DType::bf16);
        CHECK(hipMemcpy(xr.data(), static_cast<const char*>(x3.data()) + r * H * 2, H * 2, hipMemcpyDeviceToDevice) ==
              hipSuccess);
        std::vector<qwen38::GatedDeltaNetState> c1;
        const qwen38::DeviceTensor o1 = gdn.forward_verify(xr, state, c1);
        ctx.synchronize();
        const auto got = o1.to_host<std::uint16_t>();
        CHECK(std::equal(got.begin(), got.end(), want.begin() + static_cast<std::ptrdiff_t>(r * H)));
        state = std::move(c1[0]);
    }
    {
        std::vector<std::uint16_t> a(sb / 2), b(sb / 2);
        CHECK(hipMemcpy(a.data(), state.data(), sb, hipMemcpyDeviceToHost) == hipSuccess);
        CHECK(hipMemcpy(b.data(), ck[S - 1].data(), sb, hipMemcpyDeviceToHost) == hipSuccess);
        CHECK(a == b);
    }
    // errors
    qwen38::DeviceTensor bad({1, 65, H}, qwen38::DType::bf16);
    CHECK(throws<std::runtime_error>([&] { (void)gdn.forward_verify(bad, origin, ck); }));
    CHECK(throws<std::runtime_error>([&] {
        qwen38::GatedDeltaNet g3(ctx, w, H, HK, HV, D, D, 3, 8, static_cast<int>(G), false, "sigmoid", 1e-6f);
    }));
    CHECK(throws<std::runtime_error>([&] {
        qwen38::GatedDeltaNet gx(ctx, w, H, HK, HV, D, D, 4, 8, static_cast<int>(G), false, "tanh", 1e-6f);
    }));
    std::printf("gated delta net: ok\n");
}

// SelfAttention mirror: forward_verify equals the C ABI call bit for bit (outputs and cache),
// the checkpoints share the cache with token counts origin + r + 1, S rows equal S one-row
// calls chained through the checkpoints, and a full cache throws std::out_of_range.
static void self_attention_tests(const qwen38::Context& ctx) {
    const std::size_t H = 512, HQ = 4, HKV = 2, D = 128, R = 32, G = 64, QW = HQ * D, KW = HKV * D, S = 4, CAP = 40;
    std::uint64_t st = 0x6A09E667F3BCC909ull;
    auto next = [&] { st = st * 6364136223846793005ull + 1442695040888963407ull; return static_cast<std::uint32_t>(st >> 32); };
    auto bf16 = [](float f) { std::uint32_t u; std::memcpy(&u, &f, 4); return static_cast<std::uint16_t>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16); };
    auto unit = [&] { return (static_cast<float>(next() >> 8) / 16777216.0f) - 0.5f; };
    std::vector<qwen38::DeviceTensor> keep;
    keep.reserve(16);
    auto u32t = [&](std::size_t n) {
        std::vector<std::uint32_t> h(n);
        for (auto& v : h) v = next();
        keep.emplace_back(std::vector<std::size_t>{n}, qwen38::DType::u32);
        keep.back().upload(h.data(), n * 4);
        return static_cast<const std::uint32_t*>(keep.back().data());
    };
    auto bft = [&](std::size_t n, float scale, float offset) {
        std::vector<std::uint16_t> h(n);
        for (auto& v : h) v = bf16(offset + scale * unit());
        keep.emplace_back(std::vector<std::size_t>{n}, qwen38::DType::bf16);
        keep.back().upload(h.data(), n * 2);
        return static_cast<const std::uint16_t*>(keep.back().data());
    };
    const std::size_t outs[4] = {2 * QW, KW, KW, H}, ins[4] = {H, H, H, QW};
    q38_attn_weights w{};
    for (int p = 0; p < 4; ++p) {  // 8-bit, centred: weight = q * s + b with b ~ -127.5 s
        w.weight[p] = u32t(outs[p] * ins[p] / 4);
        w.scales[p] = bft(outs[p] * ins[p] / G, 0.0001f, 0.00015f);
        w.biases[p] = bft(outs[p] * ins[p] / G, 0.002f, -0.019f);
    }
    w.q_norm = bft(D, 0.5f, 1.0f);
    w.k_norm = bft(D, 0.5f, 1.0f);
    qwen38::SelfAttention attn(ctx, w, H, HQ, HKV, D, R, 8, static_cast<int>(G), false, false, 1e-6f, 1e6);
    // an origin holding 20 tokens (random cache contents), at position 100
    qwen38::SelfAttentionState origin = attn.make_state(CAP, 100);
    {
        std::vector<std::uint16_t> h(origin.cache.numel());
        for (auto& v : h) v = bf16(unit());
        origin.cache.upload(h.data(), h.size() * 2);
        origin.token_count = 20;
    }
    auto copy_state = [&](const qwen38::SelfAttentionState& a) {
        qwen38::SelfAttentionState b = attn.make_state(a.capacity, a.position_base);
        CHECK(hipMemcpy(b.cache.data(), a.cache.data(), a.cache.nbytes(), hipMemcpyDeviceToDevice) == hipSuccess);
        b.token_count = a.token_count;
        return b;
    };
    const qwen38::SelfAttentionState base = copy_state(origin);
    auto x = bft(S * H, 2.0f, 0.0f);
    qwen38::DeviceTensor x3({1, S, H}, qwen38::DType::bf16);
    CHECK(hipMemcpy(x3.data(), x, S * H * 2, hipMemcpyDeviceToDevice) == hipSuccess);
    std::vector<qwen38::SelfAttentionState> ck;
    const qwen38::DeviceTensor out = attn.forward_verify(x3, origin, ck);
    ctx.synchronize();
    CHECK(ck.size() == S);
    for (std::size_t r = 0; r < S; ++r)
        CHECK(ck[r].token_count == 21 + r && ck[r].cache.data() == origin.cache.data() && ck[r].position_base == 100);
    {   // the C ABI on a copy of the origin
        qwen38::SelfAttentionState o2 = copy_state(base);
        qwen38::DeviceTensor out2({S, H}, qwen38::DType::bf16);
        qwen38::DeviceTensor ws({q38_attn_workspace_size(attn.handle(), S, CAP)}, qwen38::DType::u32);
        CHECK(q38_attn_verify(attn.handle(), static_cast<const std::uint16_t*>(x3.data()), S, o2.cache.data(), CAP, 20,
                              120, static_cast<std::uint16_t*>(out2.data()), ws.data(), ws.nbytes(), ctx.stream()) == Q38_OK);
        ctx.synchronize();
        CHECK(out.to_host<std::uint16_t>() == out2.to_host<std::uint16_t>());
        CHECK(origin.cache.to_host<std::uint16_t>() == o2.cache.to_host<std::uint16_t>());
    }
    {   // row by row through the checkpoints
        qwen38::SelfAttentionState s = copy_state(base);
        const auto want = out.to_host<std::uint16_t>();
        for (std::size_t r = 0; r < S; ++r) {
            qwen38::DeviceTensor xr({1, 1, H}, qwen38::DType::bf16);
            CHECK(hipMemcpy(xr.data(), static_cast<const char*>(x3.data()) + r * H * 2, H * 2,
                            hipMemcpyDeviceToDevice) == hipSuccess);
            std::vector<qwen38::SelfAttentionState> c1;
            const qwen38::DeviceTensor o1 = attn.forward_verify(xr, s, c1);
            ctx.synchronize();
            const auto got = o1.to_host<std::uint16_t>();
            CHECK(std::equal(got.begin(), got.end(), want.begin() + static_cast<std::ptrdiff_t>(r * H)));
            s = std::move(c1[0]);
        }
        CHECK(s.token_count == 24 && s.cache.to_host<std::uint16_t>() == origin.cache.to_host<std::uint16_t>());
    }
    // a full cache
    qwen38::SelfAttentionState full = copy_state(base);
    full.token_count = CAP - 2;
    CHECK(throws<std::out_of_range>([&] { (void)attn.forward_verify(x3, full, ck); }));
    qwen38::DeviceTensor bad({1, 65, H}, qwen38::DType::bf16);
    CHECK(throws<std::runtime_error>([&] { (void)attn.forward_verify(bad, origin, ck); }));
    CHECK(throws<std::runtime_error>([&] {
        qwen38::SelfAttention a3(ctx, w, H, 3, HKV, D, R, 8, static_cast<int>(G), false, false, 1e-6f, 1e6);
    }));
    std::printf("self attention: ok\n");
}

// DecoderLayer mirror (forward_verify_dense_batched) on a linear-attention layer and a
// full-attention layer: the output equals the C ABI composition (mixer read, attention step,
// mixer write, then the MLP half through q38_verify_chain_hc_mapped) bit for bit, the
// checkpoints are the attention step's, and rows split over two calls chained through a
// checkpoint equal the rows of one call.
static void decoder_layer_tests(const qwen38::Context& ctx) {
    const std::size_t H = 512, HCN = 4, R = 64, G = 64, K = H * HCN, S = 4;
    std::uint64_t st = 0xBB67AE8584CAA73Bull;
    auto next = [&] { st = st * 6364136223846793005ull + 1442695040888963407ull; return static_cast<std::uint32_t>(st >> 32); };
    auto bf16 = [](float f) { std::uint32_t u; std::memcpy(&u, &f, 4); return static_cast<std::uint16_t>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16); };
    auto unit = [&] { return (static_cast<float>(next() >> 8) / 16777216.0f) - 0.5f; };
    std::vector<qwen38::DeviceTensor> keep;
    keep.reserve(64);
    auto u32t = [&](std::size_t n) {
        std::vector<std::uint32_t> h(n);
        for (auto& v : h) v = next();
        keep.emplace_back(std::vector<std::size_t>{n}, qwen38::DType::u32);
        keep.back().upload(h.data(), n * 4);
        return static_cast<const std::uint32_t*>(keep.back().data());
    };
    auto bft = [&](std::size_t n, float scale, float offset) {
        std::vector<std::uint16_t> h(n);
        for (auto& v : h) v = bf16(offset + scale * unit());
        keep.emplace_back(std::vector<std::size_t>{n}, qwen38::DType::bf16);
        keep.back().upload(h.data(), n * 2);
        return static_cast<const std::uint16_t*>(keep.back().data());
    };
    auto mixer_weights = [&] {  // 4-bit centred groups, as in the mixer test
        return q38_hc_weights{bft(K, 0.2f, 0.0f),
                              u32t(R * K / 8), bft(R * K / G, 0.004f, 0.006f), bft(R * K / G, 0.002f, -0.045f),
                              u32t(K * R / 8), bft(K * R / G, 0.004f, 0.006f), bft(K * R / G, 0.002f, -0.045f),
                              u32t(HCN * K / 8), bft(HCN * K / G, 0.004f, 0.006f), bft(HCN * K / G, 0.002f, -0.045f)};
    };
    const q38_hc_weights aw = mixer_weights(), mw = mixer_weights();
    qwen38::HyperConnection amix(ctx, aw, H, HCN, R, 4, G, 1e-6f, true);
    qwen38::HyperConnection mmix(ctx, mw, H, HCN, R, 4, G, 1e-6f, true);
    qwen38::MoeGeometry g;
    g.hidden = H;
    g.intermediate = 128;
    qwen38::SparseMoe moe(ctx, 0x5EEDull, 7, 64, 4, true, g);
    // a linear-attention block (the GatedDeltaNet test's geometry)
    const std::size_t HK = 2, HV = 4, D = 128, C = 2 * HK * D + HV * D, VW = HV * D;
    q38_gdn_weights gw{};
    {
        const std::size_t outs[5] = {C, VW, HV, HV, H}, ins[5] = {H, H, H, H, VW};
        for (int p = 0; p < 5; ++p) {
            gw.weight[p] = u32t(outs[p] * ins[p] / 4);
            gw.scales[p] = bft(outs[p] * ins[p] / G, 0.0001f, 0.00015f);
            gw.biases[p] = bft(outs[p] * ins[p] / G, 0.002f, -0.019f);
        }
        gw.conv = bft(C * 4, 1.0f, 0.0f);
        gw.dt_bias = bft(HV, 1.0f, 0.0f);
        gw.norm = bft(D, 0.5f, 1.0f);
    }
    std::vector<float> alog(HV, 0.5f);
    qwen38::DeviceTensor alog_t({HV}, qwen38::DType::f32);
    alog_t.upload(alog.data(), HV * 4);
    gw.a_log = static_cast<const float*>(alog_t.data());
    qwen38::GatedDeltaNet gdn(ctx, gw, H, HK, HV, D, D, 4, 8, static_cast<int>(G), false, "sigmoid", 1e-6f);
    // a full-attention block (the SelfAttention test's geometry)
    const std::size_t HQ = 4, HKV = 2, RD = 32, QW = HQ * D, KW = HKV * D, CAP = 40;
    q38_attn_weights tw{};
    {
        const std::size_t outs[4] = {2 * QW, KW, KW, H}, ins[4] = {H, H, H, QW};
        for (int p = 0; p < 4; ++p) {
            tw.weight[p] = u32t(outs[p] * ins[p] / 4);
            tw.scales[p] = bft(outs[p] * ins[p] / G, 0.0001f, 0.00015f);
            tw.biases[p] = bft(outs[p] * ins[p] / G, 0.002f, -0.019f);
        }
        tw.q_norm = bft(D, 0.5f, 1.0f);
        tw.k_norm = bft(D, 0.5f, 1.0f);
    }
    qwen38::SelfAttention attn(ctx, tw, H, HQ, HKV, D, RD, 8, static_cast<int>(G), false, false, 1e-6f, 1e6);

    // streams of S rows
    const std::uint16_t* emb = bft(S * H, 2.0f, 0.0f);
    qwen38::DeviceTensor emb3({1, S, H}, qwen38::DType::bf16);
    CHECK(hipMemcpy(emb3.data(), emb, S * H * 2, hipMemcpyDeviceToDevice) == hipSuccess);
    const qwen38::DeviceTensor streams = qwen38::HyperConnection::initialize_stream(ctx, emb3, HCN);
    auto rows_of = [&](const qwen38::DeviceTensor& t, std::size_t r0, std::size_t n) {
        qwen38::DeviceTensor o({1, n, K}, qwen38::DType::bf16);
        CHECK(hipMemcpy(o.data(), static_cast<const char*>(t.data()) + r0 * K * 2, n * K * 2,
                        hipMemcpyDeviceToDevice) == hipSuccess);
        return o;
    };
    // the MLP half through the C ABI, in place
    auto mlp_half = [&](qwen38::DeviceTensor& x, std::size_t rows) {
        qwen38::DeviceTensor ws({q38_verify_chain_hc_mapped_workspace_size(&moe.desc(), &mmix.desc(),
                                                                            static_cast<int32_t>(rows))},
                                qwen38::DType::u32);
        q38_moe_layer* l = moe.handle();
        q38_hc* m = mmix.handle();
        CHECK(q38_verify_chain_hc_mapped(&l, &m, nullptr, 1, static_cast<std::uint16_t*>(x.data()),
                                         static_cast<int32_t>(rows), ws.data(), ws.nbytes(), ctx.stream()) == Q38_OK);
    };

    {   // linear-attention layer
        qwen38::DecoderLayer layer(amix, gdn, mmix, moe);
        CHECK(layer.linear());
        qwen38::DecoderLayerState origin;
        origin.linear_attention.block = qwen38::DeviceTensor({gdn.state_bytes() / 2}, qwen38::DType::bf16);
        {
            std::vector<std::uint16_t> h(gdn.state_bytes() / 2);
            for (auto& v : h) v = bf16(0.1f * unit());
            origin.linear_attention.block.upload(h.data(), h.size() * 2);
        }
        origin.linear_attention.initialized = true;
        std::vector<qwen38::DecoderLayerState> ck;
        const qwen38::DeviceTensor out = layer.forward_verify_dense_batched(streams, origin, ck);
        ctx.synchronize();
        CHECK(ck.size() == S && out.shape() == streams.shape());
        // the composition through the components and the C ABI
        const qwen38::HyperConnectionRead rd = amix.read(streams);
        std::vector<qwen38::GatedDeltaNetState> gck;
        const qwen38::DeviceTensor go = gdn.forward_verify(rd.mixed, origin.linear_attention, gck);
        qwen38::DeviceTensor post = amix.write(streams, go, rd.injection);
        mlp_half(post, S);
        ctx.synchronize();
        const auto want = post.to_host<std::uint16_t>();
        CHECK(out.to_host<std::uint16_t>() == want);
        CHECK(out.to_host<std::uint16_t>() != streams.to_host<std::uint16_t>());
        for (std::size_t r = 0; r < S; ++r) {
            std::vector<std::uint16_t> a(gdn.state_bytes() / 2), b(gdn.state_bytes() / 2);
            CHECK(hipMemcpy(a.data(), ck[r].linear_attention.data(), gdn.state_bytes(), hipMemcpyDeviceToHost) ==
                  hipSuccess);
            CHECK(hipMemcpy(b.data(), gck[r].data(), gdn.state_bytes(), hipMemcpyDeviceToHost) == hipSuccess);
            CHECK(a == b);
        }
        // rows 0-1, then rows 2-3 from the checkpoint of row 1
        std::vector<qwen38::DecoderLayerState> c1, c2;
        const qwen38::DeviceTensor o1 = layer.forward_verify_dense_batched(rows_of(streams, 0, 2), origin, c1);
        const qwen38::DeviceTensor o2 = layer.forward_verify_dense_batched(rows_of(streams, 2, 2), c1[1], c2);
        ctx.synchronize();
        const auto a1 = o1.to_host<std::uint16_t>(), a2 = o2.to_host<std::uint16_t>();
        CHECK(std::equal(a1.begin(), a1.end(), want.begin()));
        CHECK(std::equal(a2.begin(), a2.end(), want.begin() + static_cast<std::ptrdiff_t>(2 * K)));
    }
    {   // full-attention layer over a cache holding 20 tokens at position 100
        qwen38::DecoderLayer layer(amix, attn, mmix, moe);
        CHECK(!layer.linear());
        auto fresh = [&] {
            qwen38::DecoderLayerState o;
            o.full_attention = attn.make_state(CAP, 100);
            std::uint64_t s2 = 0x3C6EF372FE94F82Bull;
            std::vector<std::uint16_t> h(o.full_attention.cache.numel());
            for (auto& v : h) {
                s2 = s2 * 6364136223846793005ull + 1442695040888963407ull;
                v = bf16(static_cast<float>(static_cast<std::uint32_t>(s2 >> 40)) / 16777216.0f - 0.5f);
            }
            o.full_attention.cache.upload(h.data(), h.size() * 2);
            o.full_attention.token_count = 20;
            return o;
        };
        qwen38::DecoderLayerState origin = fresh();
        std::vector<qwen38::DecoderLayerState> ck;
        const qwen38::DeviceTensor out = layer.forward_verify_dense_batched(streams, origin, ck);
        ctx.synchronize();
        CHECK(ck.size() == S);
        for (std::size_t r = 0; r < S; ++r) CHECK(ck[r].full_attention.token_count == 21 + r);
        qwen38::DecoderLayerState o2 = fresh();
        const qwen38::HyperConnectionRead rd = amix.read(streams);
        std::vector<qwen38::SelfAttentionState> ack;
        const qwen38::DeviceTensor ao = attn.forward_verify(rd.mixed, o2.full_attention, ack);
        qwen38::DeviceTensor post = amix.write(streams, ao, rd.injection);
        mlp_half(post, S);
        ctx.synchronize();
        const auto want = post.to_host<std::uint16_t>();
        CHECK(out.to_host<std::uint16_t>() == want);
        CHECK(origin.full_attention.cache.to_host<std::uint16_t>() == o2.full_attention.cache.to_host<std::uint16_t>());
        // rows 0-1, then rows 2-3 from the checkpoint of row 1
        qwen38::DecoderLayerState o3 = fresh();
        std::vector<qwen38::DecoderLayerState> c1, c2;
        const qwen38::DeviceTensor p1 = layer.forward_verify_dense_batched(rows_of(streams, 0, 2), o3, c1);
        const qwen38::DeviceTensor p2 = layer.forward_verify_dense_batched(rows_of(streams, 2, 2), c1[1], c2);
        ctx.synchronize();
        const auto a1 = p1.to_host<std::uint16_t>(), a2 = p2.to_host<std::uint16_t>();
        CHECK(std::equal(a1.begin(), a1.end(), want.begin()));
        CHECK(std::equal(a2.begin(), a2.end(), want.begin() + static_cast<std::ptrdiff_t>(2 * K)));
        CHECK(c2[1].full_attention.token_count == 24);
    }
    qwen38::DeviceTensor bad({1, 17, K}, qwen38::DType::bf16);
    std::vector<qwen38::DecoderLayerState> ck;
    qwen38::DecoderLayerState none;
    CHECK(throws<std::runtime_error>([&] {
        (void)qwen38::DecoderLayer(amix, gdn, mmix, moe).forward_verify_dense_batched(bad, none, ck);
    }));
    std::printf("decoder layer: ok\n");
}

// The draft head on HC streams (5 streams of the model's hidden size): forward_decode equals
// the C ABI step bit for bit, the greedy chain equals a replay of single steps, and a
// single-stream row is refused.
static void mtp_stream_tests(const qwen38::Context& ctx, const qwen38::QwenModel& model) {
    const std::size_t H = model.hidden(), HC = 5, R = 256, G = 64, K = H * HC;
    std::uint64_t st = 0xD1B54A32D192ED03ull;
    auto next = [&] { st = st * 6364136223846793005ull + 1442695040888963407ull; return static_cast<std::uint32_t>(st >> 32); };
    auto bf16 = [](float f) { std::uint32_t u; std::memcpy(&u, &f, 4); return static_cast<std::uint16_t>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16); };
    auto unit = [&] { return (static_cast<float>(next() >> 8) / 16777216.0f) - 0.5f; };
    std::vector<qwen38::DeviceTensor> keep;
    auto u32t = [&](std::size_t n) {
        std::vector<std::uint32_t> h(n);
        for (auto& v : h) v = next();
        keep.emplace_back(std::vector<std::size_t>{n}, qwen38::DType::u32);
        keep.back().upload(h.data(), n * 4);
        return static_cast<const std::uint32_t*>(keep.back().data());
    };
    auto bft = [&](std::size_t n, float scale, float offset) {
        std::vector<std::uint16_t> h(n);
        for (auto& v : h) v = bf16(offset + scale * unit());
        keep.emplace_back(std::vector<std::size_t>{n}, qwen38::DType::bf16);
        keep.back().upload(h.data(), n * 2);
        return static_cast<const std::uint16_t*>(keep.back().data());
    };
    keep.reserve(32);
    auto mixer = [&](bool inj) {
        q38_hc_weights w{};
        w.norm = bft(K, 0.2f, 0.0f);
        w.down_w = u32t(R * K / 8), w.down_s = bft(R * K / G, 0.004f, 0.006f), w.down_b = bft(R * K / G, 0.002f, -0.045f);
        w.up_w = u32t(K * R / 8), w.up_s = bft(K * R / G, 0.004f, 0.006f), w.up_b = bft(K * R / G, 0.002f, -0.045f);
        if (inj) w.inj_w = u32t(HC * K / 8), w.inj_s = bft(HC * K / G, 0.004f, 0.006f), w.inj_b = bft(HC * K / G, 0.002f, -0.045f);
        return qwen38::HyperConnection(ctx, w, H, HC, R, 4, G, 1e-6f, inj);
    };
    qwen38::HyperConnection block = mixer(true), final_mixer = mixer(false);
    qwen38::DeviceTensor en({H}, qwen38::DType::bf16), hn({K}, qwen38::DType::bf16);
    CHECK(hipMemcpy(en.data(), bft(H, 0.2f, 0.0f), H * 2, hipMemcpyDeviceToDevice) == hipSuccess);
    CHECK(hipMemcpy(hn.data(), bft(K, 0.2f, 0.0f), K * 2, hipMemcpyDeviceToDevice) == hipSuccess);
    qwen38::MoeGeometry g;
    qwen38::QwenMtpHead head(ctx, model.seed(), model.vocab(), g);
    head.attach_streams(block, final_mixer, en, hn);
    CHECK(head.stream_count() == HC);
    // target streams: a verified row tiled over the streams
    qwen38::DeviceTensor fm, rows;
    std::vector<qwen38::GreedyStep> gs;
    model.forward_verify_layer_major(std::vector<std::uint32_t>{321}, fm, gs, nullptr, &rows);
    qwen38::DeviceTensor one({1, 1, H}, qwen38::DType::bf16);
    CHECK(hipMemcpy(one.data(), rows.data(), H * 2, hipMemcpyDeviceToDevice) == hipSuccess);
    const qwen38::DeviceTensor prev = qwen38::HyperConnection::initialize_stream(ctx, one, HC);
    CHECK(prev.shape() == (std::vector<std::size_t>{1, 1, K}));
    const std::uint32_t cur = gs[0].token;
    qwen38::MtpDecodeState rs = head.make_state();
    const qwen38::MtpDecodeStep s0 = head.forward_decode(prev, cur, 10, rs);
    CHECK(s0.pre_mixer_stream.shape() == (std::vector<std::size_t>{1, 1, K}));
    {   // the same step through the C ABI
        qwen38::DeviceTensor lg({1, model.vocab()}, qwen38::DType::f32), so({1, K}, qwen38::DType::bf16);
        qwen38::DeviceTensor tok({1}, qwen38::DType::u32), ws({q38_mtp_workspace_size(head.handle(), 1)}, qwen38::DType::u32);
        tok.upload(&cur, 4);
        CHECK(q38_mtp_forward_decode(head.handle(), static_cast<const std::uint16_t*>(prev.data()),
                                     static_cast<const std::uint32_t*>(tok.data()), 1, static_cast<float*>(lg.data()),
                                     static_cast<std::uint16_t*>(so.data()), nullptr, ws.data(), ws.nbytes(),
                                     ctx.stream()) == Q38_OK);
        ctx.synchronize();
        CHECK(lg.to_host<float>() == s0.logits.to_host<float>());
        CHECK(so.to_host<std::uint16_t>() == s0.pre_mixer_stream.to_host<std::uint16_t>());
    }
    qwen38::MtpDecodeState cs = head.make_state();
    const auto d = head.draft_greedy(prev, cur, 10, 3, cs);
    qwen38::MtpDecodeState ps = head.make_state();
    qwen38::DeviceTensor s = prev.share();
    std::uint32_t t = cur;
    for (std::size_t k = 0; k < 3; ++k) {
        qwen38::MtpDecodeStep step = head.forward_decode(s, t, 10 + k, ps);
        const auto lg = step.logits.to_host<float>();
        t = static_cast<std::uint32_t>(std::max_element(lg.begin(), lg.end()) - lg.begin());
        CHECK(t == d[k]);
        s = std::move(step.pre_mixer_stream);
    }
    CHECK(throws<std::runtime_error>([&] { (void)head.forward_decode(one, cur, 13, ps); }));
    std::printf("mtp streams: ok\n");
}

static void draft_head_tests(const qwen38::Context& ctx, const qwen38::QwenModel& model) {
    qwen38::MoeGeometry g;
    qwen38::QwenMtpHead head(ctx, model.seed(), model.vocab(), g);
    // a previous target stream: the pre-norm row of verifying one token
    qwen38::DeviceTensor fm, streams;
    std::vector<qwen38::GreedyStep> gs;
    model.forward_verify_layer_major(std::vector<std::uint32_t>{321}, fm, gs, nullptr, &streams);
    qwen38::DeviceTensor prev({1, 1, model.hidden()}, qwen38::DType::bf16);
    CHECK(hipMemcpy(prev.data(), streams.data(), model.hidden() * 2, hipMemcpyDeviceToDevice) == hipSuccess);
    std::uint32_t cur = gs[0].token;
    // chain = replay of single steps with a host argmax
    {
        qwen38::MtpDecodeState st = head.make_state();
        const auto d = head.draft_greedy(prev, cur, 50, 3, st);
        CHECK(d.size() == 3 && st.row_count == 3 && st.position_base == std::optional<std::size_t>(50));
        qwen38::MtpDecodeState rs = head.make_state();
        qwen38::DeviceTensor s = prev.share();
        std::uint32_t t = cur;
        for (std::size_t k = 0; k < 3; ++k) {
            qwen38::MtpDecodeStep step = head.forward_decode(s, t, 50 + k, rs);
            const auto lg = step.logits.to_host<float>();
            t = static_cast<std::uint32_t>(std::max_element(lg.begin(), lg.end()) - lg.begin());
            CHECK(t == d[k]);
            s = std::move(step.pre_mixer_stream);
        }
        CHECK(throws<std::runtime_error>([&] { (void)head.forward_decode(s, t, 99, rs); }));  // not contiguous
        CHECK(rs.row_count == 3);
    }
    qwen38::ModelDecodeState state(model, 100, 8);
    qwen38::MtpDecodeState hs = head.make_state();
    std::size_t q = 100, learned_accepted = 0;
    CHECK(throws<std::runtime_error>(
        [&] { (void)qwen38::run_greedy_mtp_round_reference(model, head, cur, prev, q, 1, state, hs); }));
    CHECK(state.token_count() == 100 && hs.row_count == 0);
    // A query position that does not match the target is found after drafting, as in the
    // reference (src/mtp_runner.cpp:227-245 run before the head state is restored): the target
    // state is intact, the head state holds the speculative rows.
    CHECK(throws<std::runtime_error>(
        [&] { (void)qwen38::run_greedy_mtp_round_reference(model, head, cur, prev, q + 1, 3, state, hs); }));
    CHECK(state.token_count() == 100 && hs.row_count == 3);
    hs = head.make_state();
    for (int round = 0; round < 4; ++round) {
        const std::size_t rows_before = hs.row_count;
        std::vector<std::uint32_t> expect;
        {
            const qwen38::DeviceTensor* s1[1] = {&prev};
            expect = head.draft_greedy_rows(s1, std::span<const std::uint32_t>(&cur, 1), 3).front();
        }
        qwen38::MtpRoundStep step = qwen38::run_greedy_mtp_round_reference(model, head, cur, prev, q, 3, state, hs);
        CHECK(step.draft_tokens == expect);
        CHECK(state.token_count() == q + step.accepted + 1 && step.next_query_position == q + step.accepted + 1);
        CHECK(hs.row_count == rows_before + step.accepted + 1);
        CHECK(step.emitted_tokens.size() == step.accepted + 1 && step.emitted_tokens.back() == step.next_current_token);
        // the next stream is the correction row's pre-norm stream of [cur, drafts]
        std::vector<std::uint32_t> toks{cur};
        toks.insert(toks.end(), expect.begin(), expect.end());
        qwen38::DeviceTensor fm2, st2;
        std::vector<qwen38::GreedyStep> g2;
        model.forward_verify_layer_major(toks, fm2, g2, nullptr, &st2);
        std::vector<std::uint16_t> a(model.hidden()), b = step.next_target_stream.to_host<std::uint16_t>();
        CHECK(hipMemcpy(a.data(), static_cast<const char*>(st2.data()) + step.accepted * model.hidden() * 2,
                        model.hidden() * 2, hipMemcpyDeviceToHost) == hipSuccess);
        CHECK(a == b && g2[step.accepted].token == step.next_current_token);
        learned_accepted += step.accepted;
        q = step.next_query_position;
        cur = step.next_current_token;
        prev = std::move(step.next_target_stream);
    }
    // the batched scheduler with the head as its learned drafter
    std::vector<std::unique_ptr<qwen38::ModelDecodeState>> states;
    std::vector<qwen38::ModelDecodeState*> ptrs;
    for (std::size_t i = 0; i < 2; ++i) {
        states.push_back(std::make_unique<qwen38::ModelDecodeState>(model, 7, 16));
        ptrs.push_back(states.back().get());
    }
    qwen38::QwenBatchVerifier verifier(model, ptrs);
    qwen38::MtpHeadDrafter drafter(head, verifier);
    qwen38::MtpSchedulerOptions opt;
    opt.zero_accept_fallback_rounds = 1000;
    opt.economic_fallback = false;
    opt.history_mode = qwen38::HistoryDraftMode::disabled;
    qwen38::MtpSlotScheduler sched(verifier, &drafter, opt);
    sched.add_request(0, std::vector<std::uint32_t>{5, 6}, 7, 12);
    sched.add_request(1, std::vector<std::uint32_t>{8, 9}, 7, 12);
    std::size_t learned = 0, first_serial = 0;
    for (int r = 0; r < 40 && !sched.done(); ++r)
        for (const qwen38::SlotRound& sr : sched.step()) {
            learned += sr.source == qwen38::DraftSourceKind::learned;
            if (r == 0) first_serial += sr.source == qwen38::DraftSourceKind::serial;
            if (sr.source == qwen38::DraftSourceKind::learned)
                CHECK(sr.draft_tokens.size() == 2 || sr.draft_tokens.size() == 3);  // probe depth, then promoted
        }
    CHECK(sched.done() && learned > 0 && first_serial == 2);
    for (std::size_t i = 0; i < 2; ++i)
        CHECK(sched.tokens(i).size() == 12 && states[i]->token_count() == sched.query_position(i));
    std::printf("draft head: ok (learned rounds accepted %zu; scheduler learned rounds %zu)\n", learned_accepted,
                learned);
}

static void gpu_tests() {
    qwen38::Context ctx(0);
    const std::uint64_t seed = 0x51A5EED;
    qwen38::MoeGeometry g;  // config-0 shapes
    // one layer through the C++ interface against the C ABI on the same input
    qwen38::SparseMoe moe(ctx, seed, 0, 512, 10, true, g);
    qwen38::DeviceTensor x({1, 4, 2048}, qwen38::DType::bf16);
    {
        const std::uint32_t toks[4] = {1, 2, 3, 4};
        qwen38::DeviceTensor h({4, 2048}, qwen38::DType::bf16);
        CHECK(q38_embed_synthetic(seed, toks, 4, 2048, static_cast<uint16_t*>(h.data()), ctx.stream()) == Q38_OK);
        CHECK(q38_rmsnorm(static_cast<const uint16_t*>(h.data()), 4, 2048, 1e-6F, static_cast<uint16_t*>(x.data()),
                          ctx.stream()) == Q38_OK);
        ctx.synchronize();
    }
    const auto sel = moe.route_decode_batch(x);
    CHECK(sel.size() == 4);
    std::vector<int32_t> ex(40);
    {
        qwen38::DeviceTensor ed({40}, qwen38::DType::i32), ws({q38_moe_workspace_size(&moe.desc(), 4)},
                                                              qwen38::DType::u32);
        q38_route_out r{static_cast<int32_t*>(ed.data()), nullptr, nullptr, nullptr, nullptr};
        CHECK(q38_moe_route(moe.handle(), static_cast<const uint16_t*>(x.data()), 4, &r, ws.data(), ws.nbytes(),
                            ctx.stream()) == Q38_OK);
        ctx.synchronize();
        ed.download(ex.data(), ex.size() * 4);
    }
    for (std::size_t r = 0; r < 4; ++r) {
        CHECK(sel[r].experts.size() == 10 && sel[r].weights.size() == 10);
        float wsum = 0.0F;
        for (std::size_t s = 0; s < 10; ++s) {
            CHECK(sel[r].experts[s] == static_cast<std::size_t>(ex[r * 10 + s]));
            wsum += sel[r].weights[s];
        }
        CHECK(wsum > 0.999F && wsum < 1.001F);
    }
    const auto y1 = moe.forward_verify(x).to_host<std::uint16_t>();
    const auto y2 = moe.forward_verify(x).to_host<std::uint16_t>();
    CHECK(y1 == y2);  // deterministic
    CHECK(throws<std::runtime_error>([&] {
        qwen38::DeviceTensor bad({1, 1025, 2048}, qwen38::DType::bf16);
        (void)moe.forward_verify(bad);
    }));
    // forward_decode / forward_decode_multi: one-row requests batched through one pass equal
    // the rows of the same batch verified together
    {
        std::vector<qwen38::DeviceTensor> reqs;
        for (std::size_t r = 0; r < 4; ++r) {
            qwen38::DeviceTensor t({1, 1, 2048}, qwen38::DType::bf16);
            CHECK(hipMemcpy(t.data(), static_cast<const char*>(x.data()) + r * 4096, 4096, hipMemcpyDeviceToDevice) ==
                  hipSuccess);
            reqs.push_back(std::move(t));
        }
        const auto outs = moe.forward_decode_multi(reqs);
        CHECK(outs.size() == 4);
        for (std::size_t r = 0; r < 4; ++r) {
            const auto o = outs[r].to_host<std::uint16_t>();
            CHECK(std::equal(o.begin(), o.end(), y1.begin() + r * 2048));
        }
        const auto d0 = moe.forward_decode(reqs[0]).to_host<std::uint16_t>();
        std::vector<qwen38::DeviceTensor> one;
        one.push_back(reqs[0].share());
        const auto m0 = moe.forward_decode_multi(one);
        CHECK(d0 == m0[0].to_host<std::uint16_t>());
        CHECK(throws<std::runtime_error>([&] { (void)moe.forward_decode(x); }));
        CHECK(throws<std::runtime_error>([&] { (void)moe.forward_decode_multi({}); }));
    }
    // prefill widths: S <= 16 is the verify call, S = 64 the segmented kernels, profiled or not
    CHECK(moe.forward_prefill(x).to_host<std::uint16_t>() == y1);
    {
        std::vector<std::uint32_t> toks(64);
        for (std::size_t i = 0; i < toks.size(); ++i) toks[i] = static_cast<std::uint32_t>(1000 + 7 * i);
        qwen38::DeviceTensor h({64, 2048}, qwen38::DType::bf16), xp({1, 64, 2048}, qwen38::DType::bf16);
        CHECK(q38_embed_synthetic(seed, toks.data(), 64, 2048, static_cast<uint16_t*>(h.data()), ctx.stream()) ==
              Q38_OK);
        CHECK(q38_rmsnorm(static_cast<const uint16_t*>(h.data()), 64, 2048, 1e-6F, static_cast<uint16_t*>(xp.data()),
                          ctx.stream()) == Q38_OK);
        const auto p1 = moe.forward_prefill(xp).to_host<std::uint16_t>();
        qwen38::MoePrefillTimings t;
        const auto p2 = moe.forward_prefill_profiled(xp, t).to_host<std::uint16_t>();
        CHECK(p1 == p2 && p1.size() == 64 * 2048);
        CHECK(t.routing_ms > 0.0 && t.gate_up_ms > 0.0 && t.swiglu_ms > 0.0 && t.down_qmm_ms > 0.0 && t.merge_ms > 0.0);
        CHECK(throws<std::runtime_error>([&] { (void)moe.forward_prefill_profiled(x, t); }));
        // a bias of +100 on experts 0..9 routes every row to exactly those experts
        std::vector<float> b(512, 0.0F);
        for (int e = 0; e < 10; ++e) b[e] = 100.0F;
        qwen38::DeviceTensor bias({512}, qwen38::DType::f32);
        bias.upload(b.data(), b.size() * 4);
        moe.set_router_bias(bias);
        for (const auto& s : moe.route_decode_batch(x))
            for (std::size_t e : s.experts) CHECK(e < 10);
        moe.set_router_bias(qwen38::DeviceTensor{});
        CHECK(moe.forward_verify(x).to_host<std::uint16_t>() == y1);
    }
    // forward_verify accepts S = 1..1024 (src/sparse_moe.cpp:1974-1976): S = 17 and 1024 take
    // the segmented kernels and equal the C ABI call; route_decode_batch agrees with q38_moe_route
    for (const std::size_t S : {std::size_t{17}, std::size_t{1024}}) {
        std::vector<std::uint32_t> toks(S);
        for (std::size_t i = 0; i < S; ++i) toks[i] = static_cast<std::uint32_t>(3 + 11 * i);
        qwen38::DeviceTensor h({S, 2048}, qwen38::DType::bf16), xs({1, S, 2048}, qwen38::DType::bf16);
        CHECK(q38_embed_synthetic(seed, toks.data(), static_cast<int32_t>(S), 2048, static_cast<uint16_t*>(h.data()),
                                  ctx.stream()) == Q38_OK);
        CHECK(q38_rmsnorm(static_cast<const uint16_t*>(h.data()), static_cast<int32_t>(S), 2048, 1e-6F,
                          static_cast<uint16_t*>(xs.data()), ctx.stream()) == Q38_OK);
        const auto yv = moe.forward_verify(xs).to_host<std::uint16_t>();
        qwen38::DeviceTensor yc({S, 2048}, qwen38::DType::bf16), ed({S * 10}, qwen38::DType::i32);
        qwen38::DeviceTensor ws({q38_moe_workspace_size(&moe.desc(), static_cast<int32_t>(S))}, qwen38::DType::u32);
        q38_route_out r{static_cast<int32_t*>(ed.data()), nullptr, nullptr, nullptr, nullptr};
        CHECK(q38_moe_forward(moe.handle(), static_cast<const uint16_t*>(xs.data()), static_cast<int32_t>(S),
                              static_cast<uint16_t*>(yc.data()), &r, ws.data(), ws.nbytes(), ctx.stream()) == Q38_OK);
        ctx.synchronize();
        CHECK(yv == yc.to_host<std::uint16_t>());
        const auto exs = ed.to_host<int32_t>();
        const auto sels = moe.route_decode_batch(xs);
        CHECK(sels.size() == S);
        for (std::size_t i = 0; i < S; ++i)
            for (std::size_t k = 0; k < 10; ++k) CHECK(sels[i].experts[k] == static_cast<std::size_t>(exs[i * 10 + k]));
    }
    CHECK(throws<std::runtime_error>([&] {
        qwen38::DeviceTensor bad({1, 2049, 2048}, qwen38::DType::bf16);
        (void)moe.forward_prefill(bad);
    }));

    // verify round + commit lifecycle on a 2-layer model with a small vocabulary
    qwen38::QwenModel model(ctx, seed, 2, 4096, g);
    qwen38::ModelDecodeState state(model, 100);
    const std::vector<std::uint32_t> drafts{7, 8, 9};
    auto v = qwen38::verify_mtp_target_layer_major_reference(model, 5, drafts, state);
    CHECK(v.draft_count == 3 && v.rows.size() == 4);
    for (std::size_t i = 0; i < 4; ++i) CHECK(v.rows[i].state_after == 101 + i && v.rows[i].greedy.token < 4096);
    // the same tokens through the model directly give the same greedy rows
    qwen38::DeviceTensor fm;
    std::vector<qwen38::GreedyStep> gs;
    const std::vector<std::uint32_t> toks{5, 7, 8, 9};
    model.forward_verify_layer_major(toks, fm, gs);
    for (std::size_t i = 0; i < 4; ++i)
        CHECK(gs[i].token == v.rows[i].greedy.token && gs[i].logit == v.rows[i].greedy.logit);
    // validation failures leave the verification and the state intact
    CHECK(throws<std::runtime_error>([&] { qwen38::commit_mtp_target_verification(std::move(v), 4, state); }));
    CHECK(v.rows.size() == 4 && state.token_count() == 100);
    // a second verification staged on the same state makes the first one stale: committing
    // it is rejected with the state intact, the newer one commits
    {
        auto v2 = qwen38::verify_mtp_target_layer_major_reference(model, 5, std::vector<std::uint32_t>{7, 8}, state);
        CHECK(v2.generation > v.generation);
        CHECK(throws<std::runtime_error>([&] { qwen38::commit_mtp_target_verification(std::move(v), 1, state); }));
        CHECK(v.rows.size() == 4 && state.token_count() == 100);
        qwen38::commit_mtp_target_verification(std::move(v2), 1, state);
        CHECK(v2.rows.empty() && state.token_count() == 102);
        CHECK(throws<std::runtime_error>([&] { qwen38::commit_mtp_target_verification(std::move(v), 1, state); }));
        CHECK(state.token_count() == 102);
    }
    auto v3 = qwen38::verify_mtp_target_layer_major_reference(model, 5, drafts, state);
    qwen38::commit_mtp_target_verification(std::move(v3), 2, state);
    CHECK(v3.rows.empty() && state.token_count() == 105);

    // the serial oracle (one decode per row) gives the layer-major rows bit for bit (up to
    // four rows: one kernel family) and stages checkpoints that commit the same way
    {
        auto lm = qwen38::verify_mtp_target_layer_major_reference(model, 5, drafts, state);
        auto so = qwen38::verify_mtp_target_serial_oracle(model, 5, drafts, state);
        CHECK(so.draft_count == 3 && so.rows.size() == 4 && so.generation > lm.generation);
        for (std::size_t i = 0; i < 4; ++i) {
            CHECK(so.rows[i].greedy.token == lm.rows[i].greedy.token);
            CHECK(so.rows[i].greedy.logit == lm.rows[i].greedy.logit);
            CHECK(so.rows[i].state_after == lm.rows[i].state_after);
            CHECK(so.rows[i].final_mixed.to_host<std::uint16_t>() == lm.rows[i].final_mixed.to_host<std::uint16_t>());
            CHECK(so.rows[i].pre_mixer_stream.to_host<std::uint16_t>() ==
                  lm.rows[i].pre_mixer_stream.to_host<std::uint16_t>());
        }
        CHECK(throws<std::runtime_error>([&] {
            (void)qwen38::verify_mtp_target_serial_oracle(model, 5, std::vector<std::uint32_t>{}, state);
        }));
        qwen38::commit_mtp_target_verification(std::move(so), 1, state);
        CHECK(state.token_count() == 107);
    }

    // a full external-draft round with the target's own greedy continuation as drafts
    const std::uint32_t cur = 11;
    std::vector<std::uint32_t> greedy_drafts;
    std::uint32_t prev = cur;
    for (int i = 0; i < 3; ++i) {
        qwen38::DeviceTensor f1;
        std::vector<qwen38::GreedyStep> g1;
        model.forward_verify_layer_major(std::vector<std::uint32_t>{prev}, f1, g1);
        greedy_drafts.push_back(g1[0].token);
        prev = g1[0].token;
    }
    const std::size_t q = state.token_count();
    const auto step = qwen38::run_greedy_external_draft_round_reference(model, cur, q, greedy_drafts, state);
    CHECK(step.emitted_tokens.size() == step.accepted + 1);
    CHECK(step.next_query_position == q + step.accepted + 1 && state.token_count() == step.next_query_position);
    CHECK(step.emitted_tokens.back() == step.next_current_token);
    std::printf("gpu section: ok (accepted %zu of 3 self-drafts)\n", step.accepted);
    batched_slot_tests(ctx, model);
    draft_head_tests(ctx, model);
    hyper_connection_tests(ctx);
    gated_delta_net_tests(ctx);
    mtp_stream_tests(ctx, model);
    self_attention_tests(ctx);
    decoder_layer_tests(ctx);
}

int main(int argc, char** argv) {
    host_tests();
    if (argc > 1 && std::strcmp(argv[1], "--gpu") == 0) gpu_tests();
    return 0;
}
