// oracle.cpp - CPU restatement of the reference's paged-KV path.
//
// TEST INFRASTRUCTURE ONLY. This is the checker: tests/, __graft_entry__.smoke()
// and bench.py's cpu_baseline leg use it; the product never does.
//
// Compiled with -ffp-contract=off so that every float expression rounds the way
// the reference's CPU backend does (that file is built without -mfma, so no
// multiply-add is fused); only the dot product uses fused multiply-adds, as the
// reference's AVX2 kernel does.
#include "oracle.h"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <condition_variable>
#include <cstdio>
#include <cstring>
#include <functional>
#include <list>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#if defined(__x86_64__)
#include <immintrin.h>
#endif

namespace {

constexpr int kPage = 16;  // tokens per block (src/backend/backend.hpp:25)

// ---- f16 <-> f32 (src/common/fp16.hpp:25-71) --------------------------------

uint32_t bits_of(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return u;
}

float float_of(uint32_t u) {
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

float half_to_float(uint16_t h) {
    const uint32_t sign = (h & 0x8000u) << 16;
    const int exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ffu;
    if (exp == 0x1f) return float_of(sign | 0x7f800000u | (man << 13));  // inf / nan
    if (exp == 0) {
        // zero or subnormal: man * 2^-24, exact in f32
        const float mag = static_cast<float>(man) * 5.9604644775390625e-08f;
        return sign ? -mag : mag;
    }
    return float_of(sign | (static_cast<uint32_t>(exp - 15 + 127) << 23) | (man << 13));
}

uint16_t float_to_half(float f) {
    const uint32_t u = bits_of(f);
    const uint16_t sign = static_cast<uint16_t>((u >> 16) & 0x8000u);
    const uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return static_cast<uint16_t>(sign | 0x7e00u);  // nan (quiet)
    if (a == 0x7f800000u) return static_cast<uint16_t>(sign | 0x7c00u);
    const int e = static_cast<int>(a >> 23) - 127;  // unbiased exponent
    if (e >= 16) return static_cast<uint16_t>(sign | 0x7c00u);  // >= 65536: inf
    uint32_t mant = (a & 0x7fffffu) | 0x800000u;  // 24-bit significand (normal inputs)
    int shift;                                    // bits to drop from the 24-bit significand
    uint32_t base;                                // exponent field of the result before rounding
    if (e >= -14) {
        shift = 13;
        base = static_cast<uint32_t>(e + 15) << 10;
        mant &= 0x7fffffu;  // implicit bit is carried by the exponent field
        mant |= 0;          // (kept explicit: rounding may carry into the exponent)
    } else {
        if (a < 0x00800000u) return sign;  // f32 subnormals are far below half's range
        shift = 13 + (-14 - e);            // subnormal half: fewer significand bits survive
        if (shift > 24) return sign;
        base = 0;
    }
    const uint32_t kept = mant >> shift;
    const uint32_t rest = mant & ((1u << shift) - 1u);
    const uint32_t half_ulp = 1u << (shift - 1);
    uint32_t r = base + kept;
    if (rest > half_ulp || (rest == half_ulp && (kept & 1u))) r += 1;  // may carry into the exponent / to inf
    return static_cast<uint16_t>(sign | r);
}

// ---- threads: the reference pool's chunking (src/common/thread_pool.cpp:57-82) ----

class Pool {
public:
    explicit Pool(int threads) {
        for (int i = 1; i < threads; i++) workers_.emplace_back([this] { loop(); });
        size_ = threads;
    }
    ~Pool() {
        {
            std::lock_guard<std::mutex> g(mu_);
            stop_ = true;
        }
        cv_.notify_all();
        for (auto &t : workers_) t.join();
    }
    int size() const { return size_; }

    // fn(begin, end) over [0, n) in chunks of max(grain, ceil(n / (4 * threads))).
    void run(size_t n, size_t grain, const std::function<void(size_t, size_t)> &fn) {
        if (n == 0) return;
        grain = std::max<size_t>(grain, 1);
        if (workers_.empty() || n <= grain) {
            fn(0, n);
            return;
        }
        const size_t threads = static_cast<size_t>(size_);
        const size_t chunk = std::max(grain, (n + 4 * threads - 1) / (4 * threads));
        {
            std::lock_guard<std::mutex> g(mu_);
            job_ = &fn;
            n_ = n;
            chunk_ = chunk;
            next_.store(0);
            pending_ = (n + chunk - 1) / chunk;
            gen_++;
        }
        cv_.notify_all();
        work();
        std::unique_lock<std::mutex> lk(mu_);
        done_.wait(lk, [&] { return pending_ == 0; });
        job_ = nullptr;
    }

private:
    void work() {
        for (;;) {
            const std::function<void(size_t, size_t)> *job;
            size_t n, chunk;
            {
                std::lock_guard<std::mutex> g(mu_);
                job = job_;
                n = n_;
                chunk = chunk_;
            }
            if (!job) return;
            const size_t b = next_.fetch_add(chunk);
            if (b >= n) return;
            (*job)(b, std::min(n, b + chunk));
            std::lock_guard<std::mutex> g(mu_);
            if (--pending_ == 0) done_.notify_all();
        }
    }
    void loop() {
        uint64_t seen = 0;
        std::unique_lock<std::mutex> lk(mu_);
        for (;;) {
            cv_.wait(lk, [&] { return stop_ || gen_ != seen; });
            if (stop_) return;
            seen = gen_;
            lk.unlock();
            work();
            lk.lock();
        }
    }

    std::vector<std::thread> workers_;
    int size_ = 1;
    std::mutex mu_;
    std::condition_variable cv_, done_;
    const std::function<void(size_t, size_t)> *job_ = nullptr;
    size_t n_ = 0, chunk_ = 1, pending_ = 0;
    std::atomic<size_t> next_{0};
    uint64_t gen_ = 0;
    bool stop_ = false;
};

Pool &pool_for(int threads) {
    static std::mutex mu;
    static std::unique_ptr<Pool> pool;
    std::lock_guard<std::mutex> g(mu);
    if (threads <= 0) threads = static_cast<int>(std::max(1u, std::thread::hardware_concurrency()));
    if (!pool || pool->size() != threads) {
        pool.reset();
        pool = std::make_unique<Pool>(threads);
    }
    return *pool;
}

// ---- the dot product (cpu_kernels.cpp:74-79, cpu_kernels_avx2.cpp:27-33, :58-69) ----

float dot_scalar(const float *a, const float *b, int n) {
    float s = 0;
    for (int i = 0; i < n; i++) s += a[i] * b[i];
    return s;
}

#if defined(__x86_64__)
__attribute__((target("avx2,fma"))) float dot_avx2(const float *a, const float *b, int n) {
    __m256 even = _mm256_setzero_ps(), odd = _mm256_setzero_ps();
    int i = 0;
    for (; i + 16 <= n; i += 16) {
        even = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), even);
        odd = _mm256_fmadd_ps(_mm256_loadu_ps(a + i + 8), _mm256_loadu_ps(b + i + 8), odd);
    }
    if (i + 8 <= n) {
        even = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), even);
        i += 8;
    }
    // Horizontal sum in the reference's order: lanes (j, j+4), then (j, j+2), then (0, 1).
    const __m256 v = _mm256_add_ps(even, odd);
    __m128 q = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
    q = _mm_add_ps(q, _mm_movehl_ps(q, q));
    q = _mm_add_ss(q, _mm_shuffle_ps(q, q, 0x55));
    float s = _mm_cvtss_f32(q);
    for (; i < n; i++) s += a[i] * b[i];
    return s;
}

bool have_avx2_fma() {
    static const bool ok = __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
    return ok;
}
#endif

float dot(const float *a, const float *b, int n) {
#if defined(__x86_64__)
    if (have_avx2_fma()) return dot_avx2(a, b, n);
#endif
    return dot_scalar(a, b, n);
}

// ---- norm and rotary (cpu_backend.cpp:34-39, :262-272) ----------------------------

void rmsnorm(const float *x, const float *w, int n, float eps, float *out) {
    double ss = 0;
    for (int i = 0; i < n; i++) ss += static_cast<double>(x[i]) * x[i];
    const float scale = static_cast<float>(1.0 / std::sqrt(ss / n + eps));
    for (int i = 0; i < n; i++) out[i] = w[i] * (x[i] * scale);
}

void rope(float *x, int D, int pos, const float *inv_freq) {
    const int half = D / 2;
    for (int i = 0; i < half; i++) {
        const float angle = static_cast<float>(pos) * inv_freq[i];
        const float c = std::cos(angle), s = std::sin(angle);
        const float lo = x[i], hi = x[i + half];
        x[i] = lo * c - hi * s;
        x[i + half] = hi * c + lo * s;
    }
}

int64_t offset(const int32_t *tables, int max_blocks, int num_blocks, int n_kv, int D, int seq, int layer, int kvh,
               int pos) {
    const int block = tables[static_cast<int64_t>(seq) * max_blocks + pos / kPage];
    return ((static_cast<int64_t>(layer) * num_blocks + block) * n_kv + kvh) * kPage * D +
           static_cast<int64_t>(pos % kPage) * D;
}

std::vector<int> seq_of_tokens(const int32_t *query_start, int S, int T) {
    std::vector<int> seq(static_cast<size_t>(T), -1);
    for (int s = 0; s < S; s++)
        for (int t = query_start[s]; t < query_start[s + 1] && t < T; t++) seq[static_cast<size_t>(t)] = s;
    return seq;
}

float clamp_half(float x) { return std::fmin(std::fmax(x, -65504.0f), 65504.0f); }

// ---- block manager (src/kvcache/block_manager.cpp:9-139) -------------------------

struct OracleBlock {
    int refs = 0;
    bool sealed = false;
    uint64_t hash = 0, parent = 0;
    std::vector<int32_t> tokens;
    std::list<int>::iterator lru;
};

}  // namespace

struct EmberOracleBM {
    std::vector<OracleBlock> blocks;
    std::vector<int> free_stack;  // never-sealed free blocks; back() is handed out next
    std::list<int> lru;           // sealed, unreferenced, oldest first
    std::unordered_map<uint64_t, int> index;
    bool caching = true;
    uint64_t hits = 0, lookups = 0;

    void unseal(int b) {
        OracleBlock &k = blocks[static_cast<size_t>(b)];
        if (!k.sealed) return;
        auto it = index.find(k.hash);
        if (it != index.end() && it->second == b) index.erase(it);
        k.sealed = false;
        k.hash = 0;
        k.tokens.clear();
    }
    int allocate() {
        int b;
        if (!free_stack.empty()) {
            b = free_stack.back();
            free_stack.pop_back();
        } else if (!lru.empty()) {
            b = lru.front();
            lru.pop_front();
            unseal(b);
        } else {
            return -1;
        }
        blocks[static_cast<size_t>(b)].refs = 1;
        return b;
    }
    int release(int b) {
        if (b < 0 || b >= static_cast<int>(blocks.size())) return -1;
        OracleBlock &k = blocks[static_cast<size_t>(b)];
        if (k.refs <= 0) return -1;
        if (--k.refs > 0) return 0;
        auto it = index.find(k.hash);
        if (k.sealed && caching && it != index.end() && it->second == b) {
            lru.push_back(b);
            k.lru = std::prev(lru.end());
        } else {
            unseal(b);
            free_stack.push_back(b);
        }
        return 0;
    }
};

extern "C" {

float ember_oracle_f16_to_f32(uint16_t h) { return half_to_float(h); }
uint16_t ember_oracle_f32_to_f16(float f) { return float_to_half(f); }

void ember_oracle_f16_to_f32_n(const uint16_t *src, float *dst, int64_t n) {
    for (int64_t i = 0; i < n; i++) dst[i] = half_to_float(src[i]);
}

void ember_oracle_f32_to_f16_n(const float *src, uint16_t *dst, int64_t n) {
    for (int64_t i = 0; i < n; i++) dst[i] = float_to_half(src[i]);
}

void ember_oracle_inv_freq(double theta, int32_t D, float *out) {
    for (int i = 0; i < D / 2; i++)
        out[i] = 1.0f / std::pow(static_cast<float>(theta), static_cast<float>(2 * i) / static_cast<float>(D));
}

void ember_oracle_rmsnorm(const float *x, const float *w, int32_t n, float eps, float *out) { rmsnorm(x, w, n, eps, out); }

void ember_oracle_rope(float *x, int32_t D, int32_t pos, const float *inv_freq) { rope(x, D, pos, inv_freq); }

void ember_oracle_linear(const uint16_t *A, const uint16_t *W, int32_t M, int32_t N, int32_t K, int32_t epilogue,
                         float *C, int32_t ldc) {
    std::vector<float> a(static_cast<size_t>(K)), w(static_cast<size_t>(K));
    std::vector<float> v(static_cast<size_t>(N));
    for (int32_t m = 0; m < M; m++) {
        for (int32_t k = 0; k < K; k++) a[static_cast<size_t>(k)] = ember_oracle_f16_to_f32(A[static_cast<size_t>(m) * K + k]);
        for (int32_t n = 0; n < N; n++) {
            double s = 0.0;
            for (int32_t k = 0; k < K; k++)
                s += static_cast<double>(a[static_cast<size_t>(k)]) *
                     ember_oracle_f16_to_f32(W[static_cast<size_t>(n) * K + k]);
            v[static_cast<size_t>(n)] = static_cast<float>(s);
        }
        float *row = C + static_cast<size_t>(m) * ldc;
        if (epilogue == 3) {
            for (int32_t j = 0; j < N / 2; j++) {
                const float g = v[static_cast<size_t>(2 * j)], u = v[static_cast<size_t>(2 * j + 1)];
                row[j] = g / (1.0f + std::exp(-g)) * u;
            }
        } else if (epilogue == 2) {
            for (int32_t n = 0; n < N; n++) row[n] += v[static_cast<size_t>(n)];
        } else {
            for (int32_t n = 0; n < N; n++) row[n] = v[static_cast<size_t>(n)];
        }
    }
}

// The same linear layer with the rows of W converted once and the (token,
// feature) outputs spread over threads; every output is the same double sum in
// k order, so the results are bit-identical to ember_oracle_linear's.
void ember_oracle_linear_mt(const uint16_t *A, const uint16_t *W, int32_t M, int32_t N, int32_t K, int32_t epilogue,
                            float *C, int32_t ldc, int32_t threads) {
    std::vector<float> a(static_cast<size_t>(M) * K), w(static_cast<size_t>(N) * K), v(static_cast<size_t>(M) * N);
    for (size_t i = 0; i < a.size(); i++) a[i] = ember_oracle_f16_to_f32(A[i]);
    for (size_t i = 0; i < w.size(); i++) w[i] = ember_oracle_f16_to_f32(W[i]);
    const int nt = std::max(1, std::min<int>(threads, 64));
    std::vector<std::thread> pool;
    for (int th = 0; th < nt; th++)
        pool.emplace_back([&, th] {
            for (int64_t i = th; i < static_cast<int64_t>(M) * N; i += nt) {
                const float *ar = &a[static_cast<size_t>(i / N) * K], *wr = &w[static_cast<size_t>(i % N) * K];
                double s = 0.0;
                for (int32_t k = 0; k < K; k++) s += static_cast<double>(ar[k]) * wr[k];
                v[static_cast<size_t>(i)] = static_cast<float>(s);
            }
        });
    for (auto &t : pool) t.join();
    for (int32_t m = 0; m < M; m++) {
        const float *vr = &v[static_cast<size_t>(m) * N];
        float *row = C + static_cast<size_t>(m) * ldc;
        if (epilogue == 3) {
            for (int32_t j = 0; j < N / 2; j++) row[j] = vr[2 * j] / (1.0f + std::exp(-vr[2 * j])) * vr[2 * j + 1];
        } else if (epilogue == 2) {
            for (int32_t n = 0; n < N; n++) row[n] += vr[n];
        } else {
            for (int32_t n = 0; n < N; n++) row[n] = vr[n];
        }
    }
}

// ---- sampling: src/backend/sampling_host.cpp:20-87, sampling_rng.hpp:22-33 ----

uint64_t ember_oracle_rng_mix(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

float ember_oracle_gumbel(uint64_t seed, uint64_t counter, uint32_t id) {
    const uint64_t h = ember_oracle_rng_mix(seed ^ ember_oracle_rng_mix(counter * 0x632BE59BD9B4E019ull + id));
    const float u = (static_cast<float>(h >> 40) + 0.5f) * (1.0f / 16777216.0f);
    return -std::log(-std::log(u));
}

// The kept tokens and their probabilities, most likely first: temperature,
// then top-k (ties to the lower id), top-p over the top-k set's normalized
// mass (the first prefix reaching top_p), then min-p against the top token;
// greedy params give the first largest logit with p = 1. Returns how many.
int32_t ember_oracle_sampling_distribution(const float *logits, int32_t vocab, float temperature, float top_p,
                                           int32_t top_k, float min_p, int32_t *out_tokens, float *out_probs) {
    if (temperature <= 1e-5f) {
        int best = 0;
        for (int i = 1; i < vocab; i++)
            if (logits[i] > logits[best]) best = i;
        out_tokens[0] = best;
        out_probs[0] = 1.0f;
        return 1;
    }
    std::vector<std::pair<float, int32_t>> cand(static_cast<size_t>(vocab));
    for (int i = 0; i < vocab; i++) cand[static_cast<size_t>(i)] = {logits[i] / temperature, i};
    auto higher = [](const std::pair<float, int32_t> &a, const std::pair<float, int32_t> &b) {
        return a.first > b.first || (a.first == b.first && a.second < b.second);
    };
    if (top_k > 0 && top_k < vocab) {
        std::nth_element(cand.begin(), cand.begin() + (top_k - 1), cand.end(), higher);
        cand.resize(static_cast<size_t>(top_k));
    }
    std::sort(cand.begin(), cand.end(), higher);
    std::vector<double> p(cand.size());
    double total = 0.0;
    for (size_t i = 0; i < cand.size(); i++) total += p[i] = std::exp(static_cast<double>(cand[i].first) - cand[0].first);
    for (double &x : p) x /= total;
    size_t n = cand.size();
    if (top_p < 1.0f) {
        double cum = 0.0;
        for (size_t i = 0; i < n; i++) {
            cum += p[i];
            if (cum >= top_p) {
                n = i + 1;
                break;
            }
        }
    }
    if (min_p > 0.0f) {
        size_t m = 1;
        while (m < n && p[m] >= min_p * p[0]) m++;
        n = m;
    }
    double kept = 0.0;
    for (size_t i = 0; i < n; i++) kept += p[i];
    for (size_t i = 0; i < n; i++) {
        out_tokens[i] = cand[i].second;
        out_probs[i] = static_cast<float>(p[i] / kept);
    }
    return static_cast<int32_t>(n);
}

// One draw: the kept set's argmax of logit / temperature + Gumbel noise.
int32_t ember_oracle_sample(const float *logits, int32_t vocab, float temperature, float top_p, int32_t top_k,
                            float min_p, uint64_t seed, uint64_t counter) {
    std::vector<int32_t> toks(static_cast<size_t>(vocab));
    std::vector<float> probs(static_cast<size_t>(vocab));
    const int n = ember_oracle_sampling_distribution(logits, vocab, temperature, top_p, top_k, min_p, toks.data(),
                                                     probs.data());
    if (n == 1) return toks[0];
    int32_t best = toks[0];
    float best_score = -INFINITY;
    for (int i = 0; i < n; i++) {
        const int32_t t = toks[static_cast<size_t>(i)];
        const float score = logits[t] / temperature + ember_oracle_gumbel(seed, counter, static_cast<uint32_t>(t));
        if (score > best_score) {
            best_score = score;
            best = t;
        }
    }
    return best;
}

float ember_oracle_dot(const float *a, const float *b, int32_t n) { return dot(a, b, n); }

int64_t ember_oracle_cache_offset(const int32_t *tables, int32_t max_blocks, int32_t num_blocks, int32_t n_kv,
                                  int32_t D, int32_t seq, int32_t layer, int32_t kvh, int32_t pos) {
    return offset(tables, max_blocks, num_blocks, n_kv, D, seq, layer, kvh, pos);
}

int32_t ember_oracle_append_layer(const float *qkv, int32_t T, int32_t H, int32_t KVH, int32_t D, const float *q_norm,
                                  const float *k_norm, const float *bias, float eps, const float *inv_freq,
                                  const int32_t *positions, const int32_t *query_start, int32_t S,
                                  const int32_t *tables, int32_t max_blocks, float *q_out, void *k_cache, void *v_cache,
                                  int32_t num_blocks, int32_t kv_f16) {
    const int row = (H + 2 * KVH) * D;
    const std::vector<int> seq = seq_of_tokens(query_start, S, T);
    std::vector<float> k(static_cast<size_t>(D)), v(static_cast<size_t>(D));
    const bool norm = q_norm && k_norm;
    for (int t = 0; t < T; t++) {
        const float *src = qkv + static_cast<int64_t>(t) * row;
        const int pos = positions[t];
        if (seq[static_cast<size_t>(t)] < 0 || pos < 0 || pos / kPage >= max_blocks) return -1;
        for (int h = 0; h < H; h++) {
            float *q = q_out + (static_cast<int64_t>(t) * H + h) * D;
            // The bias is added only when there is one (cpu_backend.cpp:146-154): x + 0.0f would turn a
            // -0.0 input into +0.0, and the reference stores such a V as it came (the memcpy at :169).
            for (int d = 0; d < D; d++) q[d] = bias ? src[h * D + d] + bias[h * D + d] : src[h * D + d];
            if (norm) rmsnorm(q, q_norm, D, eps, q);
            rope(q, D, pos, inv_freq);
        }
        for (int h = 0; h < KVH; h++) {
            const int ko = (H + h) * D, vo = (H + KVH + h) * D;
            for (int d = 0; d < D; d++) {
                k[static_cast<size_t>(d)] = bias ? src[ko + d] + bias[ko + d] : src[ko + d];
                v[static_cast<size_t>(d)] = bias ? src[vo + d] + bias[vo + d] : src[vo + d];
            }
            if (norm) rmsnorm(k.data(), k_norm, D, eps, k.data());
            rope(k.data(), D, pos, inv_freq);
            const int block = tables[static_cast<int64_t>(seq[static_cast<size_t>(t)]) * max_blocks + pos / kPage];
            if (block < 0 || block >= num_blocks) return -1;
            const int64_t off = offset(tables, max_blocks, num_blocks, KVH, D, seq[static_cast<size_t>(t)], 0, h, pos);
            if (kv_f16) {
                uint16_t *kc = static_cast<uint16_t *>(k_cache) + off, *vc = static_cast<uint16_t *>(v_cache) + off;
                for (int d = 0; d < D; d++) {
                    kc[d] = float_to_half(clamp_half(k[static_cast<size_t>(d)]));
                    vc[d] = float_to_half(clamp_half(v[static_cast<size_t>(d)]));
                }
            } else {
                std::memcpy(static_cast<float *>(k_cache) + off, k.data(), sizeof(float) * static_cast<size_t>(D));
                std::memcpy(static_cast<float *>(v_cache) + off, v.data(), sizeof(float) * static_cast<size_t>(D));
            }
        }
    }
    return 0;
}

int32_t ember_oracle_attention_layer(const float *q, int32_t T, int32_t H, int32_t KVH, int32_t D,
                                     const int32_t *positions, const int32_t *query_start, int32_t S,
                                     const int32_t *tables, int32_t max_blocks, const void *k_cache,
                                     const void *v_cache, int32_t num_blocks, int32_t kv_f16, int32_t q_f16,
                                     float *out, int32_t threads) {
    if (H % KVH != 0) return -1;
    const int G = H / KVH;
    const std::vector<int> seq = seq_of_tokens(query_start, S, T);
    for (int t = 0; t < T; t++) {
        if (seq[static_cast<size_t>(t)] < 0 || positions[t] < 0 || positions[t] / kPage >= max_blocks) return -1;
        for (int p = 0; p <= positions[t]; p += kPage) {
            const int b = tables[static_cast<int64_t>(seq[static_cast<size_t>(t)]) * max_blocks + p / kPage];
            if (b < 0 || b >= num_blocks) return -1;
        }
    }
    const float scale = 1.0f / std::sqrt(static_cast<float>(D));
    Pool &pool = pool_for(threads);
    pool.run(static_cast<size_t>(T) * H, 4, [&](size_t i0, size_t i1) {
        std::vector<float> scores, qv(static_cast<size_t>(D)), kv(static_cast<size_t>(D));
        for (size_t i = i0; i < i1; i++) {
            const int t = static_cast<int>(i / H), h = static_cast<int>(i % H);
            const int s = seq[static_cast<size_t>(t)], kvh = h / G, ctx = positions[t] + 1;
            const float *qs = q + (static_cast<int64_t>(t) * H + h) * D;
            for (int d = 0; d < D; d++) qv[static_cast<size_t>(d)] = q_f16 ? half_to_float(float_to_half(qs[d])) : qs[d];
            scores.resize(static_cast<size_t>(ctx));
            float mx = -INFINITY;
            for (int j = 0; j < ctx; j++) {
                const int64_t off = offset(tables, max_blocks, num_blocks, KVH, D, s, 0, kvh, j);
                const float *krow;
                if (kv_f16) {
                    const uint16_t *kh = static_cast<const uint16_t *>(k_cache) + off;
                    for (int d = 0; d < D; d++) kv[static_cast<size_t>(d)] = half_to_float(kh[d]);
                    krow = kv.data();
                } else {
                    krow = static_cast<const float *>(k_cache) + off;
                }
                const float sc = dot(qv.data(), krow, D) * scale;
                scores[static_cast<size_t>(j)] = sc;
                mx = std::max(mx, sc);
            }
            double sum = 0;
            for (int j = 0; j < ctx; j++) sum += scores[static_cast<size_t>(j)] = std::exp(scores[static_cast<size_t>(j)] - mx);
            float *o = out + (static_cast<int64_t>(t) * H + h) * D;
            std::fill_n(o, D, 0.0f);
            for (int j = 0; j < ctx; j++) {
                const float w = static_cast<float>(scores[static_cast<size_t>(j)] / sum);
                const int64_t off = offset(tables, max_blocks, num_blocks, KVH, D, s, 0, kvh, j);
                if (kv_f16) {
                    const uint16_t *vh = static_cast<const uint16_t *>(v_cache) + off;
                    for (int d = 0; d < D; d++) o[d] += w * half_to_float(vh[d]);
                } else {
                    const float *vr = static_cast<const float *>(v_cache) + off;
                    for (int d = 0; d < D; d++) o[d] += w * vr[d];
                }
            }
        }
    });
    return 0;
}

// ---- block manager -----------------------------------------------------------------

EmberOracleBM *ember_oracle_bm_create(int32_t num_blocks, int32_t prefix_caching) {
    if (num_blocks <= 0) return nullptr;
    auto *bm = new EmberOracleBM;
    bm->blocks.resize(static_cast<size_t>(num_blocks));
    bm->caching = prefix_caching != 0;
    for (int b = num_blocks - 1; b >= 0; b--) bm->free_stack.push_back(b);  // low ids handed out first
    return bm;
}

void ember_oracle_bm_destroy(EmberOracleBM *bm) { delete bm; }
int32_t ember_oracle_bm_num_blocks(const EmberOracleBM *bm) { return static_cast<int32_t>(bm->blocks.size()); }
int32_t ember_oracle_bm_available(const EmberOracleBM *bm) {
    return static_cast<int32_t>(bm->free_stack.size() + bm->lru.size());
}
int32_t ember_oracle_bm_cached(const EmberOracleBM *bm) { return static_cast<int32_t>(bm->index.size()); }
int32_t ember_oracle_bm_allocate(EmberOracleBM *bm) { return bm->allocate(); }
int32_t ember_oracle_bm_release(EmberOracleBM *bm, int32_t b) { return bm->release(b); }

int32_t ember_oracle_bm_release_all(EmberOracleBM *bm, const int32_t *blocks, int32_t n) {
    for (int i = n - 1; i >= 0; i--)  // last blocks first: they become the first evicted
        if (bm->release(blocks[i]) != 0) return -1;
    return 0;
}

uint64_t ember_oracle_fnv1a_words(uint64_t parent, const int32_t *tokens, int32_t n) {
    uint64_t h = 0xcbf29ce484222325ull ^ parent;
    for (int i = 0; i < n; i++) {
        h ^= static_cast<uint32_t>(tokens[i]);
        h *= 0x100000001b3ull;
    }
    return h;
}

uint64_t ember_oracle_fmix64(uint64_t h) {
    h ^= h >> 33;
    h *= 0xff51afd7ed558ccdull;
    h ^= h >> 33;
    h *= 0xc4ceb9fe1a85ec53ull;
    h ^= h >> 33;
    return h;
}

uint64_t ember_oracle_bm_block_hash(uint64_t parent, const int32_t *tokens, int32_t n) {
    const uint64_t h = ember_oracle_fmix64(ember_oracle_fnv1a_words(parent, tokens, n));
    return h ? h : 1;  // 0 stands for "no parent"
}

int32_t ember_oracle_bm_match_prefix(EmberOracleBM *bm, const int32_t *tokens, int32_t n, int32_t *out) {
    if (!bm->caching) return 0;
    bm->lookups += static_cast<uint64_t>(n);
    uint64_t parent = 0;
    int found = 0;
    for (int i = 0; i < n / kPage; i++) {
        const int32_t *chunk = tokens + i * kPage;
        const uint64_t h = ember_oracle_bm_block_hash(parent, chunk, kPage);
        auto it = bm->index.find(h);
        if (it == bm->index.end()) break;
        OracleBlock &k = bm->blocks[static_cast<size_t>(it->second)];
        if (k.parent != parent || !std::equal(chunk, chunk + kPage, k.tokens.begin())) break;  // a collision
        if (k.refs == 0) bm->lru.erase(k.lru);
        k.refs++;
        out[found++] = it->second;
        parent = h;
    }
    bm->hits += static_cast<uint64_t>(found) * kPage;
    return found;
}

uint64_t ember_oracle_bm_seal(EmberOracleBM *bm, int32_t b, uint64_t parent, const int32_t *tokens, int32_t n) {
    if (n != kPage || b < 0 || b >= static_cast<int>(bm->blocks.size())) return 0;
    const uint64_t h = ember_oracle_bm_block_hash(parent, tokens, n);
    if (!bm->caching) return h;
    OracleBlock &k = bm->blocks[static_cast<size_t>(b)];
    if (k.sealed) return k.hash;
    if (bm->index.count(h)) return h;  // an identical block is cached already: this one stays private
    k.sealed = true;
    k.hash = h;
    k.parent = parent;
    k.tokens.assign(tokens, tokens + n);
    bm->index[h] = b;
    return h;
}

int32_t ember_oracle_bm_refcount(const EmberOracleBM *bm, int32_t b) { return bm->blocks[static_cast<size_t>(b)].refs; }
uint64_t ember_oracle_bm_hit_tokens(const EmberOracleBM *bm) { return bm->hits; }
uint64_t ember_oracle_bm_lookup_tokens(const EmberOracleBM *bm) { return bm->lookups; }

int32_t ember_oracle_bm_check(const EmberOracleBM *bm, char *buf, int32_t buflen) {
    std::string problem;
    std::vector<int> seen(bm->blocks.size(), 0);
    for (int b : bm->free_stack) {
        const OracleBlock &k = bm->blocks[static_cast<size_t>(b)];
        if (k.refs != 0 || k.sealed) {
            problem = "free block " + std::to_string(b) + " is referenced or sealed";
            break;
        }
        seen[static_cast<size_t>(b)]++;
    }
    if (problem.empty())
        for (int b : bm->lru) {
            const OracleBlock &k = bm->blocks[static_cast<size_t>(b)];
            if (k.refs != 0 || !k.sealed) {
                problem = "evictable block " + std::to_string(b) + " is in use or unsealed";
                break;
            }
            seen[static_cast<size_t>(b)]++;
        }
    if (problem.empty())
        for (size_t b = 0; b < bm->blocks.size(); b++) {
            if (bm->blocks[b].refs > 0) seen[b]++;
            if (seen[b] != 1) {
                problem = "block " + std::to_string(b) + " is accounted for " + std::to_string(seen[b]) + " times";
                break;
            }
        }
    if (problem.empty())
        for (const auto &kv : bm->index) {
            const OracleBlock &k = bm->blocks[static_cast<size_t>(kv.second)];
            if (!k.sealed || k.hash != kv.first) {
                problem = "hash index points to block " + std::to_string(kv.second) + " with a different hash";
                break;
            }
        }
    if (buf && buflen > 0) std::snprintf(buf, static_cast<size_t>(buflen), "%s", problem.c_str());
    return problem.empty() ? 0 : 1;
}

void ember_oracle_bm_states(const EmberOracleBM *bm, uint8_t *out) {
    for (size_t b = 0; b < bm->blocks.size(); b++) out[b] = bm->blocks[b].refs > 0 ? 2 : 0;
    for (int b : bm->lru) out[b] = 1;
}

int32_t ember_oracle_bm_share(EmberOracleBM *bm, const int32_t *blocks, int32_t n) {
    for (int i = 0; i < n; i++)
        if (blocks[i] < 0 || blocks[i] >= static_cast<int>(bm->blocks.size()) || bm->blocks[static_cast<size_t>(blocks[i])].refs <= 0)
            return -1;
    for (int i = 0; i < n; i++) bm->blocks[static_cast<size_t>(blocks[i])].refs++;
    return 0;
}

int32_t ember_oracle_bm_copy_on_write(EmberOracleBM *bm, int32_t b) {
    if (b < 0 || b >= static_cast<int>(bm->blocks.size()) || bm->blocks[static_cast<size_t>(b)].refs <= 0) return -1;
    if (bm->blocks[static_cast<size_t>(b)].refs == 1) return b;
    const int fresh = bm->allocate();
    if (fresh < 0) return -1;
    bm->blocks[static_cast<size_t>(b)].refs--;
    return fresh;
}

}  // extern "C"
