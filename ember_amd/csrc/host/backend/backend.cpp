// The backend factory and the free functions backend.hpp declares
// (src/backend/backend.cpp:1-89), for a build whose one device is "hip" (an
// MI355X). create_backend dispatches on BackendOptions::device exactly as the
// reference's does; "cpu" and "cuda" name backends this build does not contain.
#include "backend/backend.hpp"

#include <hip/hip_runtime.h>

#include "common/error.hpp"

namespace ember {

std::unique_ptr<Backend> create_hip_backend(const std::string &dir, const BackendOptions &opt);

const char *weight_format_name(WeightFormat f) {
    switch (f) {
        case WeightFormat::f16: return "f16";
        case WeightFormat::int8: return "int8";
        case WeightFormat::int4: return "int4";
    }
    return "?";
}

WeightFormat parse_weight_format(const std::string &s) {
    if (s == "f16" || s == "fp16") return WeightFormat::f16;
    if (s == "int8" || s == "q8") return WeightFormat::int8;
    if (s == "int4" || s == "q4") return WeightFormat::int4;
    fail("unknown weight format \"{}\" (use f16, int8 or int4)", s);
}

int64_t estimate_weight_bytes(const std::string &dir, const BackendOptions &opt) {
    EMBER_CHECK(opt.weights == WeightFormat::f16, "the hip backend takes f16 weights");
    const ModelConfig c = ModelConfig::load(dir);
    const int64_t H = c.hidden, I = c.intermediate;
    const int64_t per_layer = (c.q_dim() + 2LL * c.kv_dim()) * H + H * c.q_dim() + 2 * I * H + H * I;
    const int64_t head = static_cast<int64_t>(c.vocab_size) * H;
    // The hip backend keeps the embedding table and a packed LM head, tied or not.
    return 2 * (c.n_layers * per_layer + head * 2);
}

int64_t gpu_free_memory() {
    size_t free = 0, total = 0;
    if (hipMemGetInfo(&free, &total) != hipSuccess) return 0;
    return static_cast<int64_t>(free);
}

int64_t plan_kv_split(const std::string &target_dir, const std::string &draft_dir, const BackendOptions &opt,
                      const BackendOptions &draft) {
    const int64_t free = gpu_free_memory();
    const int64_t weights = estimate_weight_bytes(target_dir, opt) + estimate_weight_bytes(draft_dir, draft);
    const int64_t logit_rows = opt.max_logit_rows > 0 ? opt.max_logit_rows : opt.max_seqs;
    const int64_t buffers = (500LL << 20) + logit_rows * ModelConfig::load(target_dir).vocab_size * 4;
    const int64_t keep = static_cast<int64_t>((1.0 - opt.memory_fraction) * static_cast<double>(free)) + (128LL << 20);
    const int64_t left = free - weights - buffers - keep;
    EMBER_CHECK(left >= (128LL << 20), "not enough GPU memory for both models ({} MiB free, {} MiB of weights)",
                free >> 20, weights >> 20);
    return left / 2;
}

bool cuda_available() { return false; }  // this build drives HIP devices only

std::unique_ptr<Backend> create_backend(const std::string &dir, const BackendOptions &opt) {
    if (opt.device == "hip") return create_hip_backend(dir, opt);
    if (opt.device == "cpu" || opt.device == "cuda")
        fail("this build of Ember has no {} backend; use --device hip", opt.device);
    fail("unknown device \"{}\" (use hip)", opt.device);
}

}  // namespace ember
