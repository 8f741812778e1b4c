// The engine's page logic (mini_engine.hpp) driving the real HIP backend,
// created through ember::create_backend("hip") from a model directory and
// linked from libember_hip.so: the GPU-path counterpart of the reference's
// read-back engine tests (tests/test_engine.cpp:91-230).
//
// Every request has a fixed continuation: a recording Backend wrapper returns
// it from sample() (teacher forcing) and records the logits of every row whose
// context is that request's own sequence. Each request is first run alone (its
// prompt in one chunk, a roomy cache); then all of them together on a cache too
// small for them (preemption and re-prefill, 40-token prompt chunks, a shared
// prompt prefix served from the prefix cache), then with speculative verify of
// 4 drafts, one in four wrong (rollback). A page handed to the wrong sequence,
// a stale slot or a wrong table shows up as logits far from the alone run's;
// the different kernel paths (decode runs, prefill tiles, chunk boundaries)
// only move them by rounding. Usage: hip_engine_test <model_dir> [dump]: with a
// dump path, the alone runs' sequences and logit rows are written there for the
// Python side to check against the oracle (int32 requests, then per request
// int32 prompt length, int32 length and its tokens; int32 rows, int32 vocab,
// then per row int32 request, int32 position sampled, float logits[vocab]).
#include <cmath>
#include <cstdio>
#include <map>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

#include "backend/backend.hpp"
#include "kvcache/block_manager.hpp"
#include "mini_engine.hpp"

using namespace ember;

namespace {

class Recording final : public Backend {
public:
    Recording(Backend &inner, const std::vector<std::vector<int32_t>> &full, const std::vector<int> &prompt_len)
        : in_(inner), full_(full), prompt_len_(prompt_len) {}

    std::string name() const override { return in_.name(); }
    const ModelConfig &config() const override { return in_.config(); }
    const BackendOptions &options() const override { return in_.options(); }
    int num_kv_blocks() const override { return in_.num_kv_blocks(); }
    MemoryInfo memory() const override { return in_.memory(); }
    void forward(const StepBatch &b) override {
        in_.forward(b);
        batch_ = b;
    }
    // Request id = params.seed; a row's next position = counter.
    void sample(std::span<const SampleRequest> reqs, std::span<int32_t> out) override {
        std::vector<float> lg(static_cast<size_t>(config().vocab_size));
        for (size_t i = 0; i < reqs.size(); i++) {
            const int id = static_cast<int>(reqs[i].params.seed);
            const size_t next = static_cast<size_t>(reqs[i].counter);
            const std::vector<int32_t> &seq = full_[static_cast<size_t>(id)];
            if (next >= seq.size()) {  // a verify row past the request's end: never appended
                out[i] = 3;
                continue;
            }
            out[i] = seq[next];
            // the row's context is the request's own sequence iff every batch token of its run up to the row is
            const int row = batch_.logit_rows[i];
            int s = 0;
            while (batch_.query_start[static_cast<size_t>(s) + 1] <= row) s++;
            bool own = true;
            for (int t = batch_.query_start[static_cast<size_t>(s)]; t <= row; t++) {
                const size_t p = static_cast<size_t>(batch_.positions[static_cast<size_t>(t)]);
                own = own && p < seq.size() && batch_.tokens[static_cast<size_t>(t)] == seq[p];
            }
            if (!own) continue;
            in_.logits(static_cast<int>(i), lg);
            auto &slot = rec[{id, static_cast<int>(next)}];
            if (slot.empty()) {
                slot = lg;
            } else {  // computed again (re-prefill after a preemption, or a verify row): compare
                recomputed++;
                worst_repeat = std::max(worst_repeat, rel(lg, slot));
            }
        }
    }
    void token_probs(std::span<const SampleRequest>, std::span<const int32_t>, std::span<const int32_t>,
                     std::span<float>) override {}
    void logits(int row, std::span<float> out) override { in_.logits(row, out); }
    void set_capture_hidden(bool on) override { in_.set_capture_hidden(on); }
    std::vector<float> captured_hidden() override { return in_.captured_hidden(); }

    static double rel(const std::vector<float> &a, const std::vector<float> &b) {
        double d = 0, m = 0;
        for (size_t i = 0; i < a.size(); i++) {
            d = std::max(d, std::fabs(static_cast<double>(a[i]) - b[i]));
            m = std::max(m, std::fabs(static_cast<double>(b[i])));
        }
        return m > 0 ? d / m : d;
    }

    std::map<std::pair<int, int>, std::vector<float>> rec;
    int recomputed = 0;
    double worst_repeat = 0;

private:
    Backend &in_;
    const std::vector<std::vector<int32_t>> &full_;
    const std::vector<int> &prompt_len_;
    StepBatch batch_;
};

struct Result {
    std::map<std::pair<int, int>, std::vector<float>> rec;
    int steps = 0, preemptions = 0, spec_steps = 0, accepted = 0, proposed = 0;
    uint64_t hit_tokens = 0;
};

Result run(Backend &be, const std::vector<std::vector<int32_t>> &full, const std::vector<int> &prompt_len,
           const std::vector<int> &ids, testing::MiniOptions opt, bool prefix_caching, int pages, int &failures) {
    Recording rec(be, full, prompt_len);
    BlockManager bm(pages, prefix_caching);
    testing::MiniEngine engine(rec, bm, opt);
    for (int id : ids) {
        testing::MiniRequest r;
        r.prompt.assign(full[static_cast<size_t>(id)].begin(), full[static_cast<size_t>(id)].begin() + prompt_len[static_cast<size_t>(id)]);
        r.max_tokens = static_cast<int>(full[static_cast<size_t>(id)].size()) - prompt_len[static_cast<size_t>(id)];
        r.sampling.seed = static_cast<uint64_t>(id);
        engine.submit(std::move(r));
    }
    engine.run([&] {
        if (!bm.check().empty()) {
            std::fprintf(stderr, "block accounting: %s\n", bm.check().c_str());
            failures++;
        }
    });
    for (const auto &s : engine.sequences()) {
        const auto &want = full[static_cast<size_t>(ids[static_cast<size_t>(s->id)])];
        if (s->out != std::vector<int32_t>(want.begin() + prompt_len[static_cast<size_t>(ids[static_cast<size_t>(s->id)])], want.end())) {
            std::fprintf(stderr, "request %d: tokens differ from its forced continuation\n", s->id);
            failures++;
        }
    }
    if (bm.used() != 0) {
        std::fprintf(stderr, "%d pages still held after every request finished\n", bm.used());
        failures++;
    }
    if (rec.worst_repeat > 2e-2) {
        std::fprintf(stderr, "a recomputed row's logits moved by %.3e\n", rec.worst_repeat);
        failures++;
    }
    Result r;
    r.rec = std::move(rec.rec);
    r.steps = engine.steps;
    r.preemptions = engine.preemptions;
    r.spec_steps = engine.spec_steps;
    r.accepted = engine.accepted;
    r.proposed = engine.proposed;
    r.hit_tokens = bm.hit_tokens();
    return r;
}

double compare(const Result &ref, const Result &got, const char *what, int &failures) {
    double worst = 0;
    size_t n = 0;
    for (const auto &[key, lg] : ref.rec) {
        auto it = got.rec.find(key);
        if (it == got.rec.end()) {
            std::fprintf(stderr, "%s: request %d position %d was never computed on its own context\n", what, key.first,
                         key.second);
            failures++;
            continue;
        }
        worst = std::max(worst, Recording::rel(it->second, lg));
        n++;
    }
    std::printf("%s: %zu logit rows, worst relative difference to the alone runs %.3e\n", what, n, worst);
    if (worst > 2e-2) failures++;
    return worst;
}

}  // namespace

int main(int argc, char **argv) {
    if (argc < 2) {
        std::fprintf(stderr, "usage: %s <model_dir> [dump]\n", argv[0]);
        return 2;
    }
    int failures = 0;
    try {
        BackendOptions opt;
        opt.device = "hip";
        opt.max_batch_tokens = 512;
        opt.max_seqs = 12;
        opt.max_logit_rows = 64;  // a verify step asks for 5 rows per sequence
        opt.kv_cache_tokens = 256 * kBlockSize;
        auto be = create_backend(argv[1], opt);
        const int V = be->config().vocab_size;
        std::printf("backend %s: %s, %d KV blocks\n", be->name().c_str(), be->config().describe().c_str(),
                    be->num_kv_blocks());
        // 10 requests: prompts of 20..200 tokens (four start with one 64-token system prompt), 24 forced tokens each
        std::mt19937 rng(20261005);
        std::uniform_int_distribution<int32_t> tok(3, V - 1);
        std::vector<int32_t> system(64);
        for (auto &t : system) t = tok(rng);
        std::vector<std::vector<int32_t>> full;
        std::vector<int> prompt_len, ids;
        for (int i = 0; i < 10; i++) {
            std::vector<int32_t> s;
            if (i % 3 == 0) s = system;
            const int n = std::uniform_int_distribution<int>(20, 200)(rng);
            for (int j = 0; j < n; j++) s.push_back(tok(rng));
            prompt_len.push_back(static_cast<int>(s.size()));
            for (int j = 0; j < 24; j++) s.push_back(tok(rng));
            full.push_back(std::move(s));
            ids.push_back(i);
        }
        // alone: one request at a time, the whole prompt in one chunk
        Result ref;
        for (int id : ids) {
            testing::MiniOptions o;
            o.max_batch_tokens = 512;
            o.max_prefill_chunk = 512;
            o.max_seqs = 1;
            Result one = run(*be, full, prompt_len, {id}, o, false, be->num_kv_blocks(), failures);
            ref.rec.insert(one.rec.begin(), one.rec.end());
        }
        if (argc > 2) {
            std::FILE *f = std::fopen(argv[2], "wb");
            if (!f) throw std::runtime_error(std::string("cannot write ") + argv[2]);
            auto put = [&](const void *p, size_t bytes) {
                if (std::fwrite(p, 1, bytes, f) != bytes) throw std::runtime_error("short write of the dump");
            };
            const int32_t nreq = static_cast<int32_t>(full.size());
            put(&nreq, 4);
            for (size_t i = 0; i < full.size(); i++) {
                const int32_t pl = prompt_len[i], n = static_cast<int32_t>(full[i].size());
                put(&pl, 4);
                put(&n, 4);
                put(full[i].data(), full[i].size() * 4);
            }
            const int32_t rows = static_cast<int32_t>(ref.rec.size()), vocab = V;
            put(&rows, 4);
            put(&vocab, 4);
            for (const auto &[key, lg] : ref.rec) {
                const int32_t id = key.first, pos = key.second;
                put(&id, 4);
                put(&pos, 4);
                put(lg.data(), lg.size() * 4);
            }
            std::fclose(f);
        }
        // together on 24 pages (384 tokens for ~1,400 of context): preemption, 40-token chunks, the prefix cache
        testing::MiniOptions o;
        o.max_batch_tokens = 96;
        o.max_prefill_chunk = 40;
        o.max_seqs = 8;
        Result busy = run(*be, full, prompt_len, ids, o, true, 24, failures);
        std::printf("engine: %d steps, %d preemptions, %llu prefix-cache hit tokens\n", busy.steps, busy.preemptions,
                    static_cast<unsigned long long>(busy.hit_tokens));
        if (busy.preemptions == 0 || busy.hit_tokens == 0) {
            std::fprintf(stderr, "the busy run did not preempt or hit the prefix cache\n");
            failures++;
        }
        compare(ref, busy, "engine", failures);
        // speculative verify: 4 drafts per step from the forced continuation, one in four corrupted
        testing::MiniOptions so;
        so.max_batch_tokens = 512;
        so.max_seqs = 10;
        so.spec_k = 4;
        std::mt19937 draft_rng(7);
        so.draft = [&](const std::vector<int32_t> &ctx, int k) {
            std::vector<int32_t> d;
            const std::vector<int32_t> *seq = nullptr;  // the request whose sequence starts with ctx
            for (const auto &f : full)
                if (f.size() > ctx.size() && std::equal(ctx.begin(), ctx.end(), f.begin())) seq = &f;
            for (int i = 0; i < k; i++) {
                const size_t p = ctx.size() + static_cast<size_t>(i);
                int32_t t = seq && p < seq->size() ? (*seq)[p] : 3;
                if (draft_rng() % 4 == 0) t = 3 + (t + 11) % (V - 3);
                d.push_back(t);
            }
            return d;
        };
        Result spec = run(*be, full, prompt_len, ids, so, false, be->num_kv_blocks(), failures);
        std::printf("speculative: %d verify steps, %d of %d drafts accepted\n", spec.spec_steps, spec.accepted,
                    spec.proposed);
        if (spec.spec_steps == 0 || spec.accepted == 0 || spec.accepted == spec.proposed) {
            std::fprintf(stderr, "the speculative run did not both accept and reject drafts\n");
            failures++;
        }
        compare(ref, spec, "speculative", failures);
    } catch (const std::exception &e) {
        std::fprintf(stderr, "error: %s\n", e.what());
        return 1;
    }
    if (failures) {
        std::fprintf(stderr, "%d failures\n", failures);
        return 1;
    }
    std::printf("hip engine ok\n");
    return 0;
}
