// Test infrastructure, not product code: a C ABI over the reference's own host
// sampler (src/backend/sampling_host.cpp, src/backend/sampling_rng.hpp) and its
// AVX2 dot product (src/backend/cpu/cpu_kernels_avx2.cpp), compiled by
// oracle/Makefile from the sources where they lie under the reference tree into
// oracle/_ref/libember_ref.so. Tests check the oracle's restatements against it.
// Nothing here is restated: every function calls the reference's.
#include <cstdint>

#include "backend/cpu/cpu_kernels.hpp"
#include "backend/sampling_host.hpp"
#include "backend/sampling_rng.hpp"

namespace {

ember::SamplingParams params(float temperature, float top_p, int top_k, float min_p, uint64_t seed) {
    ember::SamplingParams p;
    p.temperature = temperature;
    p.top_p = top_p;
    p.top_k = top_k;
    p.min_p = min_p;
    p.seed = seed;
    return p;
}

}  // namespace

extern "C" {

uint64_t ember_ref_rng_mix(uint64_t z) { return ember::rng_mix(z); }

float ember_ref_gumbel_noise(uint64_t seed, uint64_t counter, uint32_t id) {
    return ember::gumbel_noise(seed, counter, id);
}

double ember_ref_sample_uniform(uint64_t seed, uint64_t counter) { return ember::sample_uniform(seed, counter); }

// The kept (token, probability) pairs, most likely first; returns how many.
int ember_ref_sampling_distribution(const float *logits, int vocab, float temperature, float top_p, int top_k,
                                    float min_p, int32_t *tokens, float *probs) {
    const auto d = ember::sampling_distribution(logits, vocab, params(temperature, top_p, top_k, min_p, 0));
    for (size_t i = 0; i < d.size(); i++) {
        tokens[i] = d[i].first;
        probs[i] = d[i].second;
    }
    return static_cast<int>(d.size());
}

int32_t ember_ref_sample_host(const float *logits, int vocab, float temperature, float top_p, int top_k, float min_p,
                              uint64_t seed, uint64_t counter) {
    ember::SampleRequest r;
    r.params = params(temperature, top_p, top_k, min_p, seed);
    r.counter = counter;
    return ember::sample_host(logits, vocab, r);
}

float ember_ref_dot_avx2(const float *a, const float *b, int n) { return ember::cpu::avx2::dot(a, b, n); }

}  // extern "C"
