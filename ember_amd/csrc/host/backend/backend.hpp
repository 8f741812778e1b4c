// The engine <-> hardware boundary, kept declaration-for-declaration equal to
// the reference's src/backend/backend.hpp:23-137 so that the engine and a
// backend built on this path stay interchangeable with Ember's.
//
// A step is a ragged batch: S sequences, each contributing a contiguous run of
// new tokens (a prompt chunk, one decode token, or the k + 1 tokens of a
// speculative check). The KV cache is split into blocks of kBlockSize tokens;
// the engine owns each sequence's block table, the backend only reads it.
#pragma once

#include <cstdint>
#include <memory>
#include <span>
#include <string>
#include <vector>

#include "model/config.hpp"

namespace ember {

constexpr int kBlockSize = 16;

enum class WeightFormat { f16, int8, int4 };
const char *weight_format_name(WeightFormat f);
WeightFormat parse_weight_format(const std::string &s);

struct SamplingParams {
    float temperature = 1.0f;  // 0 = greedy
    float top_p = 1.0f;
    int top_k = 0;             // 0 = no limit
    float min_p = 0.0f;
    uint64_t seed = 0;
};

struct BackendOptions {
    std::string device = "cuda";
    WeightFormat weights = WeightFormat::f16;
    std::string quant_mix;
    int threads = 0;
    int max_batch_tokens = 2048;
    int max_seqs = 64;
    int max_logit_rows = 0;
    double memory_fraction = 0.92;
    int64_t kv_cache_bytes = 0;
    int kv_cache_tokens = 0;
    bool cuda_graphs = true;
    int gpu = 0;
};

// One forward step. Arrays indexed by token have T entries, by sequence S.
struct StepBatch {
    std::vector<int32_t> tokens;        // [T]
    std::vector<int32_t> positions;     // [T] position of each token in its sequence
    std::vector<int32_t> query_start;   // [S+1] sequence s owns tokens [query_start[s], query_start[s+1])
    std::vector<int32_t> context_len;   // [S] tokens in the cache after this step
    std::vector<int32_t> block_tables;  // [S * max_blocks]
    int max_blocks = 0;
    std::vector<int32_t> logit_rows;    // tokens whose logits are wanted, in output order

    int num_tokens() const { return static_cast<int>(tokens.size()); }
    int num_seqs() const { return static_cast<int>(context_len.size()); }
    void clear() {
        tokens.clear();
        positions.clear();
        query_start.assign(1, 0);
        context_len.clear();
        block_tables.clear();
        max_blocks = 0;
        logit_rows.clear();
    }
};

struct SampleRequest {
    SamplingParams params;
    uint64_t counter = 0;
};

struct MemoryInfo {
    int64_t weights = 0;
    int64_t kv_cache = 0;
    int64_t activations = 0;
    int64_t device_total = 0;
    int64_t device_free = 0;
};

class Backend {
public:
    virtual ~Backend() = default;

    virtual std::string name() const = 0;
    virtual const ModelConfig &config() const = 0;
    virtual const BackendOptions &options() const = 0;
    virtual int num_kv_blocks() const = 0;
    virtual MemoryInfo memory() const = 0;

    // Appends the new tokens' keys and values to the cache and computes the
    // logits of batch.logit_rows (kept on the device).
    virtual void forward(const StepBatch &batch) = 0;
    virtual void sample(std::span<const SampleRequest> requests, std::span<int32_t> out) = 0;
    virtual void token_probs(std::span<const SampleRequest> requests, std::span<const int32_t> rows,
                             std::span<const int32_t> tokens, std::span<float> out) = 0;
    virtual void logits(int row, std::span<float> out) = 0;
    virtual void set_capture_hidden(bool on) = 0;
    virtual std::vector<float> captured_hidden() = 0;
};

std::unique_ptr<Backend> create_backend(const std::string &model_dir, const BackendOptions &options);
int64_t estimate_weight_bytes(const std::string &model_dir, const BackendOptions &options);
int64_t gpu_free_memory();
int64_t plan_kv_split(const std::string &target_dir, const std::string &draft_dir, const BackendOptions &target,
                      const BackendOptions &draft);
bool cuda_available();

}  // namespace ember
