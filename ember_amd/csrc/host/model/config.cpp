// ModelConfig from a Hugging Face config.json (and generation_config.json).
// Behaviour follows the reference's loader (src/model/config.cpp:10-67): the
// Qwen3 and Qwen2 families, the same keys with the same defaults, the same
// refusals (rope_scaling, dimensions that cannot form the attention layout) and
// eos ids taken from generation_config.json first.
#include "model/config.hpp"

#include <cstdio>

#include "common/error.hpp"
#include "common/mmap_file.hpp"

namespace ember {

namespace {

// What the architecture name fixes about the attention layer.
struct Family {
    const char *model_type;
    bool qk_norm;   // RMSNorm on every q / k head vector before RoPE
    bool qkv_bias;  // biases on the q / k / v projections
};

constexpr Family kFamilies[] = {
    {"qwen3", true, false},
    {"qwen2", false, true},
};

const Family &family_of(const std::string &model_type) {
    for (const Family &f : kFamilies)
        if (model_type == f.model_type) return f;
    fail("config.json: model_type \"{}\" is not one this backend runs (it runs qwen3 and qwen2)", model_type);
}

// An integer member that must be present.
int need_int(const json::Value &doc, const char *key) {
    const json::Value *v = doc.find(key);
    if (v == nullptr || v->is_null()) fail("config.json: \"{}\" is missing", key);
    return static_cast<int>(v->as_int());
}

int int_or(const json::Value &doc, const char *key, int64_t fallback) {
    return static_cast<int>(doc.get_int(key, fallback));
}

// eos_token_id is either one id or a list of ids.
void append_ids(const json::Value *field, std::vector<int> &ids) {
    if (field == nullptr || field->is_null()) return;
    if (!field->is_array()) {
        ids.push_back(static_cast<int>(field->as_int()));
        return;
    }
    for (size_t i = 0; i < field->size(); ++i) ids.push_back(static_cast<int>((*field)[i].as_int()));
}

// The shape checks the attention path needs: positive sizes, whole GQA groups, and a RoPE split into two halves.
void validate(const ModelConfig &m) {
    const int sizes[] = {m.vocab_size, m.hidden, m.intermediate, m.n_layers, m.n_heads, m.n_kv_heads, m.head_dim};
    for (const int v : sizes)
        if (v <= 0) fail("config.json: every model dimension must be positive ({})", m.describe());
    if (m.n_heads % m.n_kv_heads != 0)
        fail("config.json: {} query heads do not divide into groups of {} kv heads", m.n_heads, m.n_kv_heads);
    if (m.head_dim % 2 != 0 || m.head_dim > 256)
        fail("config.json: head_dim {} is not supported (it must be even and no larger than 256)", m.head_dim);
}

}  // namespace

int64_t ModelConfig::parameters() const {
    const int64_t H = hidden, I = intermediate, Q = q_dim(), KV = kv_dim();
    const int64_t per_layer = H * (Q + 2 * KV) + Q * H  // attention projections
                              + 3 * H * I               // gate, up, down
                              + 2 * H                   // input and post-attention norms
                              + (qk_norm ? 2LL * head_dim : 0);
    const int64_t embedding = static_cast<int64_t>(vocab_size) * H;
    return n_layers * per_layer + embedding * (tie_embeddings ? 1 : 2) + H;  // + the final norm
}

ModelConfig ModelConfig::from_json(const json::Value &doc, const json::Value *generation) {
    ModelConfig m;
    m.arch = doc.get_string("model_type", "");
    const Family &family = family_of(m.arch);
    if (const json::Value *scaling = doc.find("rope_scaling"); scaling != nullptr && !scaling->is_null())
        fail("config.json: rope_scaling is set, and scaled RoPE is not implemented");

    // Sizes.
    m.vocab_size = need_int(doc, "vocab_size");
    m.hidden = need_int(doc, "hidden_size");
    m.intermediate = need_int(doc, "intermediate_size");
    m.n_layers = need_int(doc, "num_hidden_layers");
    m.n_heads = need_int(doc, "num_attention_heads");
    m.n_kv_heads = int_or(doc, "num_key_value_heads", m.n_heads);  // absent: plain multi-head attention
    m.head_dim = int_or(doc, "head_dim", m.n_heads > 0 ? m.hidden / m.n_heads : 0);
    m.max_position = int_or(doc, "max_position_embeddings", 4096);

    // Numerics and layout switches.
    m.rms_eps = static_cast<float>(doc.get_number("rms_norm_eps", 1e-6));
    m.rope_theta = doc.get_number("rope_theta", 10000.0);
    m.tie_embeddings = doc.get_bool("tie_word_embeddings", false);
    m.qk_norm = family.qk_norm;
    m.qkv_bias = family.qkv_bias || doc.get_bool("attention_bias", false);
    validate(m);

    // Stop tokens: generation_config.json, when it names any, overrides config.json.
    append_ids(generation != nullptr ? generation->find("eos_token_id") : nullptr, m.eos_ids);
    if (m.eos_ids.empty()) append_ids(doc.find("eos_token_id"), m.eos_ids);
    return m;
}

ModelConfig ModelConfig::load(const std::string &dir) {
    const json::Value doc = json::Value::parse(read_file(dir + "/config.json"));
    const std::string generation_path = dir + "/generation_config.json";
    if (!file_exists(generation_path)) return from_json(doc, nullptr);
    const json::Value generation = json::Value::parse(read_file(generation_path));
    return from_json(doc, &generation);
}

std::string ModelConfig::describe() const {
    char buf[256];
    std::snprintf(buf, sizeof buf, "%s with %.2fB parameters: %d layers, d=%d, %d heads (%d kv) x %d, mlp %d, vocab %d",
                  arch.c_str(), static_cast<double>(parameters()) / 1e9, n_layers, hidden, n_heads, n_kv_heads, head_dim,
                  intermediate, vocab_size);
    return buf;
}

}  // namespace ember
