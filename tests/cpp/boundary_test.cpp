// The C++ boundary, compiled with g++ from the product headers alone
// (backend/backend.hpp, kvcache/block_manager.hpp, model/config.hpp,
// model/safetensors.hpp, common/json.hpp) and linked with the product's host
// sources: no HIP, no GPU.
//
//   1. The reference's block-manager unit test (tests/test_engine.cpp:47-78)
//      with its expected values.
//   2. ModelConfig::from_json / parameters / describe on Qwen3-0.6B's
//      config.json values: 0.44B non-embedding and 0.60B total parameters, the
//      counts the Qwen3 model card gives.
//   3. The JSON parser on escapes, surrogate pairs, numbers and errors.
//   4. A Backend subclass whose "model" reads each context back from its paged
//      cache (the reference's FakeBackend idea, tests/fake_backend.hpp:31-99),
//      driven by the engine's block-table logic (mini_engine.hpp) over the
//      product BlockManager: concurrent requests on a tiny cache (preemption,
//      chunked prefill, prefix sharing) and speculative verify with a draft that
//      is sometimes wrong. Every request must produce what it produces alone.
//   5. Given a model directory (argv[1]): SafeTensors::open_dir and
//      ModelConfig::load read it; the tensors are printed for the caller to check.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <random>
#include <string>
#include <vector>

#include "backend/backend.hpp"
#include "common/error.hpp"
#include "common/json.hpp"
#include "kvcache/block_manager.hpp"
#include "mini_engine.hpp"
#include "model/config.hpp"
#include "model/safetensors.hpp"

using namespace ember;

namespace {

int g_failures = 0;

#define EXPECT(cond)                                                               \
    do {                                                                           \
        if (!(cond)) {                                                             \
            std::fprintf(stderr, "%s:%d: EXPECT(%s) failed\n", __FILE__, __LINE__, #cond); \
            g_failures++;                                                          \
        }                                                                          \
    } while (0)

template <class F>
bool throws(F f) {
    try {
        f();
    } catch (const Error &) {
        return true;
    }
    return false;
}

// ---- 1. the reference's block-manager unit test ---------------------------

void block_manager_unit() {
    BlockManager bm(8, true);
    std::vector<int32_t> toks(40);
    for (int i = 0; i < 40; i++) toks[static_cast<size_t>(i)] = 100 + i;
    std::vector<int> mine;
    uint64_t chain = 0;
    for (int b = 0; b < 2; b++) {
        mine.push_back(bm.allocate());
        chain = bm.seal(mine.back(), chain, std::span<const int32_t>(toks).subspan(static_cast<size_t>(b) * kBlockSize, kBlockSize));
    }
    EXPECT(bm.available() == 6);
    auto hit = bm.match_prefix(toks);
    EXPECT(hit.size() == 2u && hit[0] == mine[0] && hit[1] == mine[1] && bm.refcount(mine[0]) == 2);
    bm.release_all(hit);
    bm.release_all(mine);
    EXPECT(bm.available() == 8 && bm.cached() == 2);
    auto again = bm.match_prefix(toks);
    EXPECT(again.size() == 2u);
    bm.release_all(again);
    std::vector<int32_t> other(toks);
    other[3] = 7;
    EXPECT(bm.match_prefix(other).empty());
    std::vector<int> all;
    for (int i = 0; i < 8; i++) all.push_back(bm.allocate());
    EXPECT(bm.allocate() == -1 && bm.cached() == 0 && bm.check().empty());
    bm.release_all(all);
    EXPECT(bm.check().empty() && bm.available() == 8);
}

// ---- 2. ModelConfig ----------------------------------------------------------

const char *kQwen3_06B = R"({
  "architectures": ["Qwen3ForCausalLM"], "model_type": "qwen3", "vocab_size": 151936, "hidden_size": 1024,
  "intermediate_size": 3072, "num_hidden_layers": 28, "num_attention_heads": 16, "num_key_value_heads": 8,
  "head_dim": 128, "rms_norm_eps": 1e-06, "rope_theta": 1000000, "max_position_embeddings": 40960,
  "tie_word_embeddings": true, "attention_bias": false, "rope_scaling": null, "eos_token_id": 151645,
  "torch_dtype": "bfloat16"
})";

void model_config() {
    const json::Value c = json::Value::parse(kQwen3_06B);
    const json::Value gen = json::Value::parse(R"({"eos_token_id": [151645, 151643], "do_sample": true})");
    ModelConfig m = ModelConfig::from_json(c, &gen);
    EXPECT(m.arch == "qwen3" && m.hidden == 1024 && m.n_layers == 28 && m.group() == 2 && m.head_dim == 128);
    EXPECT(m.qk_norm && !m.qkv_bias && m.tie_embeddings && m.max_position == 40960);
    EXPECT(std::fabs(m.rms_eps - 1e-6f) < 1e-12f && m.rope_theta == 1e6);
    EXPECT((m.eos_ids == std::vector<int>{151645, 151643}));  // generation_config wins
    EXPECT(ModelConfig::from_json(c, nullptr).eos_ids == std::vector<int>{151645});
    // 0.44B without the embedding, 0.60B in all (Qwen3-0.6B's model card)
    const int64_t embedding = 151936LL * 1024;
    EXPECT(m.parameters() == 596049920LL);
    EXPECT(m.parameters() - embedding - 1024 == 440466432LL);
    EXPECT(m.describe().find("0.60B") != std::string::npos);
    EXPECT(m.kv_bytes_per_token(2) == 28LL * 2 * 1024 * 2);  // 112 KiB at 1.7B's 28 layers x 8 kv heads x 128
    json::Value bad = c;
    bad.set("model_type", "llama");
    EXPECT(throws([&] { ModelConfig::from_json(bad, nullptr); }));
    json::Value scaled = c;
    scaled.set("rope_scaling", json::Value::parse(R"({"type": "yarn", "factor": 4})"));
    EXPECT(throws([&] { ModelConfig::from_json(scaled, nullptr); }));
    json::Value odd = c;
    odd.set("num_key_value_heads", 5);
    EXPECT(throws([&] { ModelConfig::from_json(odd, nullptr); }));
}

// ---- 3. JSON -----------------------------------------------------------------

void json_parser() {
    const json::Value v = json::Value::parse(
        R"( {"a": [1, -2.5e3, true, null, "x\"y\\z\n\u00e9\ud83d\ude00"], "b": {"c": 9007199254740993}, "d": 0.5} )");
    EXPECT(v["a"].size() == 5 && v["a"][0].as_int() == 1 && v["a"][1].as_number() == -2500.0);
    EXPECT(v["a"][2].as_bool() && v["a"][3].is_null());
    EXPECT(v["a"][4].as_string() == "x\"y\\z\n\xc3\xa9\xf0\x9f\x98\x80");  // é and U+1F600 in UTF-8
    EXPECT(v["b"]["c"].as_int() == 9007199254740993LL);                  // exact past 2^53
    EXPECT(v.get_number("d", 0) == 0.5 && v.get_int("missing", 7) == 7 && !v.contains("zz"));
    EXPECT(throws([&] { (void)v["d"].as_int(); }));                      // 0.5 is not an integer
    EXPECT(throws([&] { (void)v["a"].as_string(); }));
    EXPECT(json::Value::parse(v.dump()).dump() == v.dump());             // round trip
    EXPECT(json::Value::parse("[2.0, 1e3, -4E0]").dump() == "[2,1000,-4]");  // doubles print with %.17g
    EXPECT(json::Value::parse("1e3").as_int() == 1000 && json::Value::parse("-4E0").as_int() == -4);
    EXPECT(json::Value(uint64_t{18446744073709551615ULL}).as_number() == 18446744073709551616.0);
    EXPECT(throws([&] { (void)json::Value(uint64_t{18446744073709551615ULL}).as_int(); }));  // past int64
    EXPECT(json::Value(std::string("a\x0b\x01\"\\\t")).dump() == "\"a\\u000b\\u0001\\\"\\\\\\t\"");
    json::Value obj;
    obj.set("k", 1);
    obj.set("j", "x");
    obj.set("k", 2);  // replaces in place, keeps document order
    EXPECT(obj.dump() == "{\"k\":2,\"j\":\"x\"}" && obj.size() == 2);
    json::Value list;
    list.push(true);
    list.push(json::Value());
    EXPECT(list.dump() == "[true,null]" && throws([&] { (void)list[2]; }) && throws([&] { (void)json::Value(1).size(); }));
    for (const char *bad : {"{", "[1,]", "{\"a\" 1}", "\"\\ud800\"", "01x", "nul", "\"a\tb\"", "[1] 2"})
        EXPECT(throws([&] { json::Value::parse(bad); }));
    try {
        json::Value::parse("{\n  \"a\": ?\n}");
        EXPECT(false);
    } catch (const Error &e) {
        EXPECT(std::strstr(e.what(), "line 2") != nullptr);
    }
}

// ---- 4. the engine's page logic over the product BlockManager -------------

constexpr int kVocab = 1000, kEos = 1;

// The next token after a context: a hash of every token (EOS now and then when allowed).
int32_t next_token(const std::vector<int32_t> &ctx, bool allow_eos) {
    uint64_t h = 0x84222325cbf29ce4ull;
    for (int32_t t : ctx) h = (h ^ static_cast<uint32_t>(t)) * 0x100000001b3ull + (h >> 29);
    int32_t tok = static_cast<int32_t>(2 + (h >> 21) % (kVocab - 2));
    if (allow_eos && (h >> 9) % 29 == 0) tok = kEos;
    return tok;
}

// Its model reads every context back from the paged cache, through the block
// tables: a page given to the wrong sequence, a slot written twice or a stale
// slot read changes the tokens it produces.
class ReadBackBackend final : public Backend {
public:
    ReadBackBackend(int blocks, int max_batch_tokens, int max_seqs, bool eos) : blocks_(blocks), eos_(eos) {
        cfg_.arch = "qwen3";
        cfg_.vocab_size = kVocab;
        cfg_.hidden = cfg_.head_dim = 8;
        cfg_.n_layers = cfg_.n_heads = cfg_.n_kv_heads = 1;
        cfg_.max_position = 1 << 20;
        cfg_.eos_ids = {kEos};
        opt_.device = "readback";
        opt_.max_batch_tokens = max_batch_tokens;
        opt_.max_seqs = max_seqs;
        cache_.assign(static_cast<size_t>(blocks) * kBlockSize, -1);
    }
    std::string name() const override { return "readback"; }
    const ModelConfig &config() const override { return cfg_; }
    const BackendOptions &options() const override { return opt_; }
    int num_kv_blocks() const override { return blocks_; }
    MemoryInfo memory() const override { return {}; }

    void forward(const StepBatch &b) override {
        if (b.num_tokens() > opt_.max_batch_tokens || b.num_seqs() > opt_.max_seqs) throw Error("batch over its limits");
        for (int s = 0; s < b.num_seqs(); s++)  // every new token into its slot first, as the real backends do
            for (int t = b.query_start[static_cast<size_t>(s)]; t < b.query_start[static_cast<size_t>(s) + 1]; t++)
                cache_[slot(b, s, b.positions[static_cast<size_t>(t)])] = b.tokens[static_cast<size_t>(t)];
        next_.clear();
        for (int32_t row : b.logit_rows) {
            int s = 0;
            while (b.query_start[static_cast<size_t>(s) + 1] <= row) s++;
            std::vector<int32_t> ctx;
            for (int p = 0; p <= b.positions[static_cast<size_t>(row)]; p++) ctx.push_back(cache_[slot(b, s, p)]);
            next_.push_back(next_token(ctx, eos_));
        }
    }
    void sample(std::span<const SampleRequest> reqs, std::span<int32_t> out) override {
        if (reqs.size() != next_.size() || out.size() != next_.size()) throw Error("sample: rows do not match");
        std::copy(next_.begin(), next_.end(), out.begin());
    }
    void token_probs(std::span<const SampleRequest>, std::span<const int32_t>, std::span<const int32_t>,
                     std::span<float>) override {}
    void logits(int, std::span<float>) override {}
    void set_capture_hidden(bool) override {}
    std::vector<float> captured_hidden() override { return {}; }

private:
    size_t slot(const StepBatch &b, int s, int pos) const {
        const int block = b.block_tables[static_cast<size_t>(s) * b.max_blocks + pos / kBlockSize];
        if (block < 0 || block >= blocks_) throw Error(format("block {} outside the cache", block));
        return static_cast<size_t>(block) * kBlockSize + pos % kBlockSize;
    }
    ModelConfig cfg_;
    BackendOptions opt_;
    std::vector<int32_t> cache_, next_;
    int blocks_;
    bool eos_;
};

std::vector<int32_t> alone(std::vector<int32_t> ctx, int max_tokens, bool eos) {
    std::vector<int32_t> out;
    for (int i = 0; i < max_tokens; i++) {
        const int32_t t = next_token(ctx, eos);
        if (t == kEos) break;
        out.push_back(t);
        ctx.push_back(t);
    }
    return out;
}

void engine_pages(uint32_t seed) {
    // 40 pages (640 tokens) for 48 requests of up to ~300 tokens: preemption and chunked prefill;
    // one third of the prompts share a 64-token system prefix (prefix cache hits).
    std::mt19937 rng(seed);
    std::uniform_int_distribution<int32_t> tok(2, kVocab - 1);
    std::vector<int32_t> system(64);
    for (auto &t : system) t = tok(rng);
    ReadBackBackend be(40, 96, 12, true);
    BlockManager bm(40, true);
    testing::MiniOptions o;
    o.max_batch_tokens = 96;
    o.max_prefill_chunk = 40;
    o.max_seqs = 12;
    o.eos_ids = {kEos};
    testing::MiniEngine engine(be, bm, o);
    std::vector<std::vector<int32_t>> want;
    for (int i = 0; i < 48; i++) {
        testing::MiniRequest r;
        if (i % 3 == 0) r.prompt = system;
        const int n = std::uniform_int_distribution<int>(1, 200)(rng);
        for (int j = 0; j < n; j++) r.prompt.push_back(tok(rng));
        r.max_tokens = std::uniform_int_distribution<int>(1, 80)(rng);
        want.push_back(alone(r.prompt, r.max_tokens, true));
        engine.submit(std::move(r));
    }
    engine.run([&] { EXPECT(bm.check().empty()); });
    for (const auto &s : engine.sequences()) EXPECT(s->out == want[static_cast<size_t>(s->id)]);
    EXPECT(engine.preemptions > 0);
    EXPECT(bm.used() == 0 && bm.check().empty());
    EXPECT(bm.hit_tokens() > 0);  // the shared system prompt was served from the cache
}

void engine_speculative(uint32_t seed) {
    // Drafts of 4 tokens that are right most of the time: accepted prefixes, rejected slots rolled back.
    std::mt19937 rng(seed);
    std::uniform_int_distribution<int32_t> tok(2, kVocab - 1);
    ReadBackBackend be(256, 512, 16, false);
    BlockManager bm(256, true);
    testing::MiniOptions o;
    o.max_batch_tokens = 512;
    o.max_seqs = 16;
    o.spec_k = 4;
    std::mt19937 draft_rng(seed + 1);
    o.draft = [&](const std::vector<int32_t> &ctx, int k) {
        std::vector<int32_t> c = ctx, d;
        for (int i = 0; i < k; i++) {
            int32_t t = next_token(c, false);
            if (draft_rng() % 5 == 0) t = 2 + (t + 7) % (kVocab - 2);  // a wrong guess
            d.push_back(t);
            c.push_back(t);
        }
        return d;
    };
    testing::MiniEngine engine(be, bm, o);
    std::vector<std::vector<int32_t>> want;
    for (int i = 0; i < 12; i++) {
        testing::MiniRequest r;
        const int n = std::uniform_int_distribution<int>(5, 120)(rng);
        for (int j = 0; j < n; j++) r.prompt.push_back(tok(rng));
        r.max_tokens = 60;
        want.push_back(alone(r.prompt, r.max_tokens, false));
        engine.submit(std::move(r));
    }
    engine.run([&] { EXPECT(bm.check().empty()); });
    for (const auto &s : engine.sequences()) EXPECT(s->out == want[static_cast<size_t>(s->id)]);
    EXPECT(engine.spec_steps > 0 && engine.accepted > 0 && engine.accepted < engine.proposed);
    EXPECT(bm.used() == 0);
}

// ---- 5. a model directory ----------------------------------------------------

void model_dir(const char *dir) {
    const ModelConfig m = ModelConfig::load(dir);
    std::printf("config %s %d %d %d %d %d\n", m.arch.c_str(), m.hidden, m.n_layers, m.n_heads, m.n_kv_heads,
                static_cast<int>(m.eos_ids.size()));
    const SafeTensors st = SafeTensors::open_dir(dir);
    for (const auto &[name, t] : st.all()) {
        double sum = 0;
        for (int64_t i = 0; i < t.numel(); i++) {
            if (t.dtype == DType::f32) sum += static_cast<const float *>(t.data)[i];
            else if (t.dtype == DType::i32) sum += static_cast<const int32_t *>(t.data)[i];
        }
        std::printf("tensor %s %s %s %.9g\n", name.c_str(), dtype_name(t.dtype), t.shape_str().c_str(), sum);
    }
    EXPECT(throws([&] { (void)st.get("no.such.tensor"); }));
}

}  // namespace

int main(int argc, char **argv) {
    block_manager_unit();
    model_config();
    json_parser();
    for (uint32_t seed : {1u, 2u, 3u}) engine_pages(seed);
    engine_speculative(7);
    if (argc > 1) model_dir(argv[1]);
    if (g_failures) {
        std::fprintf(stderr, "%d failures\n", g_failures);
        return 1;
    }
    std::printf("boundary ok\n");
    return 0;
}
