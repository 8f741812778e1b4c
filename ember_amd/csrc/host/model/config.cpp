// ModelConfig from a Hugging Face config.json: the fields and checks the
// reference reads (src/model/config.cpp:10-67), for the Qwen3 / Qwen2 families.
#include "model/config.hpp"

#include <cstdio>

#include "common/error.hpp"
#include "common/mmap_file.hpp"

namespace ember {

int64_t ModelConfig::parameters() const {
    const int64_t H = hidden, I = intermediate, Q = q_dim(), KV = kv_dim();
    const int64_t per_layer = H * (Q + 2 * KV) + Q * H  // attention projections
                              + 3 * H * I               // gate, up, down
                              + 2 * H                   // input and post-attention norms
                              + (qk_norm ? 2LL * head_dim : 0);
    const int64_t embedding = static_cast<int64_t>(vocab_size) * H;
    return n_layers * per_layer + embedding * (tie_embeddings ? 1 : 2) + H;  // + the final norm
}

ModelConfig ModelConfig::from_json(const json::Value &c, const json::Value *gen) {
    ModelConfig m;
    m.arch = c.get_string("model_type", "");
    EMBER_CHECK(m.arch == "qwen3" || m.arch == "qwen2", "unsupported model_type \"{}\" (supported: qwen3, qwen2)", m.arch);
    m.vocab_size = static_cast<int>(c["vocab_size"].as_int());
    m.hidden = static_cast<int>(c["hidden_size"].as_int());
    m.intermediate = static_cast<int>(c["intermediate_size"].as_int());
    m.n_layers = static_cast<int>(c["num_hidden_layers"].as_int());
    m.n_heads = static_cast<int>(c["num_attention_heads"].as_int());
    m.n_kv_heads = static_cast<int>(c.get_int("num_key_value_heads", m.n_heads));
    m.head_dim = static_cast<int>(c.get_int("head_dim", m.n_heads > 0 ? m.hidden / m.n_heads : 0));
    m.rms_eps = static_cast<float>(c.get_number("rms_norm_eps", 1e-6));
    m.rope_theta = c.get_number("rope_theta", 10000.0);
    m.max_position = static_cast<int>(c.get_int("max_position_embeddings", 4096));
    m.tie_embeddings = c.get_bool("tie_word_embeddings", false);
    m.qk_norm = m.arch == "qwen3";
    m.qkv_bias = m.arch == "qwen2" || c.get_bool("attention_bias", false);
    if (const json::Value *rs = c.find("rope_scaling"); rs && !rs->is_null()) fail("rope_scaling is not supported");
    EMBER_CHECK(m.hidden > 0 && m.n_layers > 0 && m.n_heads > 0 && m.n_kv_heads > 0 && m.head_dim > 0 &&
                    m.vocab_size > 0 && m.intermediate > 0,
                "config.json has non-positive dimensions");
    EMBER_CHECK(m.n_heads % m.n_kv_heads == 0, "num_attention_heads must be a multiple of num_key_value_heads");
    EMBER_CHECK(m.head_dim % 2 == 0 && m.head_dim <= 256, "head_dim must be even and at most 256");

    // eos: generation_config.json's eos_token_id wins over config.json's; either may be one id or a list.
    auto eos_from = [&m](const json::Value *v) {
        if (!v || v->is_null()) return;
        if (v->is_array()) {
            for (const json::Value &e : v->as_array()) m.eos_ids.push_back(static_cast<int>(e.as_int()));
        } else {
            m.eos_ids.push_back(static_cast<int>(v->as_int()));
        }
    };
    eos_from(gen ? gen->find("eos_token_id") : nullptr);
    if (m.eos_ids.empty()) eos_from(c.find("eos_token_id"));
    return m;
}

ModelConfig ModelConfig::load(const std::string &dir) {
    const json::Value config = json::Value::parse(read_file(dir + "/config.json"));
    const std::string gen_path = dir + "/generation_config.json";
    if (!file_exists(gen_path)) return from_json(config, nullptr);
    const json::Value gen = json::Value::parse(read_file(gen_path));
    return from_json(config, &gen);
}

std::string ModelConfig::describe() const {
    char buf[256];
    std::snprintf(buf, sizeof buf, "%s with %.2fB parameters: %d layers, d=%d, %d heads (%d kv) x %d, mlp %d, vocab %d",
                  arch.c_str(), static_cast<double>(parameters()) / 1e9, n_layers, hidden, n_heads, n_kv_heads, head_dim,
                  intermediate, vocab_size);
    return buf;
}

}  // namespace ember
