// Token sampling on gfx950, one work-group (16 waves) per row of logits.
//
// Replaces the reference's sample_kernel / prob_kernel
// (src/backend/cuda/k_sampling.cu:149-198) with the distribution its host
// sampler defines (src/backend/sampling_host.cpp:20-66), in that order:
// temperature, top-k, top-p over the top-k set's mass, then min-p relative to
// the most likely token. Each cut keeps a prefix of the order the host sorts
// by (scaled logit v = x / temperature descending, token id ascending): a
// threshold theta and the last id kept at it (kept iff v > theta, or v ==
// theta and id <= id_cut), so tokens tied at a boundary are kept lowest id
// first, as many as the count or mass asks for. Min-p keeps exp(v - max) >=
// min_p. The token is argmax over the kept set of v + Gumbel noise (the Gumbel-max trick,
// sampling_rng.hpp:20-33: the noise depends only on (seed, counter, token id),
// so a row draws the same token in any batch). Greedy rows (temperature <=
// 1e-5) take the first largest logit.
//
// Thresholds come from a radix selection over order-preserving uint32 keys of
// v, 8 bits per pass from the top. Its histograms sum integers: counts for
// top-k, and exp(v - max) in 2^-40 fixed point for top-p, so every bin's sum
// is the same whatever order the LDS atomics land in, and the kept set is a
// deterministic function of the logits (float atomics would make it depend on
// scheduling at the boundary).
#include <cstdint>

#include "device.hpp"
#include "kernels.hpp"

namespace ember::hip {
namespace {

constexpr int kSampleThreads = 1024;
constexpr int kSampleWaves = kSampleThreads / kWave;
constexpr double kFix = 1099511627776.0;  // 2^40: exp weights in (0, 1] as fixed point, V * 2^40 < 2^64

__device__ __forceinline__ uint32_t order_key(float f) {  // ascending floats -> ascending keys
    const uint32_t b = __float_as_uint(f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float key_value(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// SplitMix64's output function (sampling_rng.hpp:22-27) and the Gumbel(0, 1)
// noise of token `id` at draw `counter` (:30-33).
__device__ __forceinline__ uint64_t rng_mix(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
__device__ __forceinline__ float gumbel_noise(uint64_t seed, uint64_t counter, uint32_t id) {
    const uint64_t h = rng_mix(seed ^ rng_mix(counter * 0x632BE59BD9B4E019ull + id));
    const float u = (static_cast<float>(h >> 40) + 0.5f) * (1.0f / 16777216.0f);  // in (0, 1)
    return -logf(-logf(u));
}

struct SampleLds {
    unsigned long long hist[256];
    unsigned long long wsum[kSampleWaves];
    float wmax[kSampleWaves];
    int widx[kSampleWaves];
    uint32_t prefix, mask;
    unsigned long long above, at;  // after a selection: the weight above the found key, and at it
};

// A prefix of the (v descending, id ascending) order.
struct Cut {
    float theta = -INFINITY;
    int id_cut = 0x7fffffff;
    __device__ bool keeps(float v, int i) const { return v > theta || (v == theta && i <= id_cut); }
};

__device__ __forceinline__ float scaled(const float *x, int i, float t) { return x[i] / t; }

// Calls f(i, x[i]) for this thread's elements of a row (i = tid, tid + 1024,
// ..., ascending), with the loads of kRowBatch elements issued together: one
// memory round trip per batch instead of one per element (a 151,936-logit row
// is 148 elements per thread).
constexpr int kRowBatch = 16;
template <class F>
__device__ __forceinline__ void for_row(const float *x, int V, F f) {
    int i = static_cast<int>(threadIdx.x);
    for (; i + (kRowBatch - 1) * kSampleThreads < V; i += kRowBatch * kSampleThreads) {
        float v[kRowBatch];
#pragma unroll
        for (int u = 0; u < kRowBatch; u++) v[u] = x[i + u * kSampleThreads];
#pragma unroll
        for (int u = 0; u < kRowBatch; u++) f(i + u * kSampleThreads, v[u]);
    }
    for (; i < V; i += kSampleThreads) f(i, x[i]);
}

__device__ float block_max(float v, SampleLds &sh) {
#pragma unroll
    for (int o = kWave / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    const int wave = static_cast<int>(threadIdx.x) / kWave;
    __syncthreads();
    if (threadIdx.x % kWave == 0) sh.wmax[wave] = v;
    __syncthreads();
    float m = sh.wmax[0];
    for (int w = 1; w < kSampleWaves; w++) m = fmaxf(m, sh.wmax[w]);
    return m;
}

__device__ unsigned long long block_sum_u64(unsigned long long v, SampleLds &sh) {
#pragma unroll
    for (int o = kWave / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    const int wave = static_cast<int>(threadIdx.x) / kWave;
    __syncthreads();
    if (threadIdx.x % kWave == 0) sh.wsum[wave] = v;
    __syncthreads();
    unsigned long long s = 0;
    for (int w = 0; w < kSampleWaves; w++) s += sh.wsum[w];
    return s;
}

// First largest score(i, x[i]) over i < V (ties to the lowest index).
template <class F>
__device__ int block_argmax(const float *x, int V, F score, SampleLds &sh) {
    float best = -INFINITY;
    int idx = 0x7fffffff;
    for_row(x, V, [&](int i, float xi) {
        const float v = score(i, xi);
        if (v > best) {  // i ascends per thread: the first of equal values is kept
            best = v;
            idx = i;
        }
    });
#pragma unroll
    for (int o = kWave / 2; o > 0; o >>= 1) {
        const float ob = __shfl_xor(best, o, kWave);
        const int oi = __shfl_xor(idx, o, kWave);
        if (ob > best || (ob == best && oi < idx)) {
            best = ob;
            idx = oi;
        }
    }
    const int wave = static_cast<int>(threadIdx.x) / kWave;
    __syncthreads();
    if (threadIdx.x % kWave == 0) {
        sh.wmax[wave] = best;
        sh.widx[wave] = idx;
    }
    __syncthreads();
    best = sh.wmax[0];
    idx = sh.widx[0];
    for (int w = 1; w < kSampleWaves; w++)
        if (sh.wmax[w] > best || (sh.wmax[w] == best && sh.widx[w] < idx)) {
            best = sh.wmax[w];
            idx = sh.widx[w];
        }
    return idx == 0x7fffffff ? 0 : idx;
}

// The largest key K such that the weight of the elements with key >= K (among
// those `within` keeps) reaches `target`; weight 1 (prob = false) or
// exp(v - mx) in fixed point (prob = true). Returns the value of K; sh.above
// and sh.at then hold the weight above K and at K.
__device__ float radix_threshold(const float *x, int V, float t, const Cut &within, float mx, bool prob,
                                 unsigned long long target, SampleLds &sh) {
    const int tid = static_cast<int>(threadIdx.x);
    if (tid == 0) {
        sh.prefix = 0;
        sh.mask = 0;
        sh.above = 0;
    }
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (int i = tid; i < 256; i += kSampleThreads) sh.hist[i] = 0;
        __syncthreads();
        const uint32_t prefix = sh.prefix, mask = sh.mask;
        for_row(x, V, [&](int i, float xi) {
            const float v = xi / t;
            if (!within.keeps(v, i)) return;
            const uint32_t k = order_key(v);
            if ((k & mask) != prefix) return;
            const unsigned long long w =
                prob ? static_cast<unsigned long long>(static_cast<double>(expf(v - mx)) * kFix) : 1ull;
            atomicAdd(&sh.hist[(k >> shift) & 255u], w);
        });
        __syncthreads();
        if (tid < kWave) {  // wave 0 finds the digit: lane l holds bins 255 - 4l .. 252 - 4l
            unsigned long long mine = 0;
            for (int j = 0; j < 4; j++) mine += sh.hist[255 - 4 * tid - j];
            // inclusive scan from the top bins down (lane 0 first)
            unsigned long long incl = mine;
#pragma unroll
            for (int o = 1; o < kWave; o <<= 1) {
                const unsigned long long up = __shfl_up(incl, o, kWave);
                if (tid >= o) incl += up;
            }
            const unsigned long long above = sh.above;
            const unsigned long long before = incl - mine;  // weight of the higher lanes' bins
            // the first lane whose cumulative weight reaches the target (or the last lane)
            const bool hit = above + incl >= target;
            const unsigned long long ballot = __ballot(hit);
            const int first = ballot ? __ffsll(static_cast<long long>(ballot)) - 1 : kWave - 1;
            if (tid == first) {
                unsigned long long cum = above + before;
                int d = 255 - 4 * tid;
                for (int j = 0; j < 3; j++, d--) {
                    if (cum + sh.hist[d] >= target) break;
                    cum += sh.hist[d];
                }
                sh.above = cum;
                sh.at = sh.hist[d];
                sh.prefix = prefix | (static_cast<uint32_t>(d) << shift);
                sh.mask = mask | (255u << shift);
            }
        }
        __syncthreads();
    }
    return key_value(sh.prefix);
}

// The r-th lowest id (r >= 1) among the elements `within` keeps whose v equals
// theta: a radix selection over the ids, 8 bits per pass from the top, counting
// from the lowest bin up.
__device__ int kth_tied_id(const float *x, int V, float t, const Cut &within, float theta, unsigned long long r,
                           SampleLds &sh) {
    const int tid = static_cast<int>(threadIdx.x);
    if (tid == 0) {
        sh.prefix = 0;
        sh.mask = 0;
        sh.above = 0;  // here: the count below the bins looked at so far
    }
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (int i = tid; i < 256; i += kSampleThreads) sh.hist[i] = 0;
        __syncthreads();
        const uint32_t prefix = sh.prefix, mask = sh.mask;
        for_row(x, V, [&](int i, float xi) {
            const float v = xi / t;
            if (v != theta || !within.keeps(v, i) || (static_cast<uint32_t>(i) & mask) != prefix) return;
            atomicAdd(&sh.hist[(static_cast<uint32_t>(i) >> shift) & 255u], 1ull);
        });
        __syncthreads();
        if (tid < kWave) {  // wave 0 finds the digit: lane l holds bins 4l .. 4l + 3
            unsigned long long mine = 0;
            for (int j = 0; j < 4; j++) mine += sh.hist[4 * tid + j];
            unsigned long long incl = mine;
#pragma unroll
            for (int o = 1; o < kWave; o <<= 1) {
                const unsigned long long up = __shfl_up(incl, o, kWave);
                if (tid >= o) incl += up;
            }
            const unsigned long long below = sh.above;
            const bool hit = below + incl >= r;
            const unsigned long long ballot = __ballot(hit);
            const int first = ballot ? __ffsll(static_cast<long long>(ballot)) - 1 : kWave - 1;
            if (tid == first) {
                unsigned long long cum = below + (incl - mine);
                int d = 4 * tid;
                for (int j = 0; j < 3; j++, d++) {
                    if (cum + sh.hist[d] >= r) break;
                    cum += sh.hist[d];
                }
                sh.above = cum;
                sh.prefix = prefix | (static_cast<uint32_t>(d) << shift);
                sh.mask = mask | (255u << shift);
            }
        }
        __syncthreads();
    }
    return static_cast<int>(sh.prefix);
}

// The cut at the key radix_threshold just found (in sh): when the weight at
// that key holds more tied tokens than the target still needs, only the lowest
// ids that reach it are kept. w_each: the weight of one token at the key.
__device__ Cut cut_at(const float *x, int V, float t, const Cut &within, float theta, unsigned long long target,
                      unsigned long long w_each, SampleLds &sh) {
    Cut c;
    c.theta = theta;
    const unsigned long long above = sh.above, at = sh.at;
    __syncthreads();  // every thread has read sh before it is reused
    if (w_each == 0 || target <= above) return c;
    const unsigned long long need = (target - above + w_each - 1) / w_each, ties = at / w_each;
    if (need < ties) c.id_cut = kth_tied_id(x, V, t, within, theta, need, sh);
    return c;
}

struct Dist {
    bool greedy;
    float t, mx, min_w;
    Cut k, p;              // the top-k and top-p cuts (the top-p one lies inside the top-k one)
    unsigned long long z;  // fixed-point mass of the kept set
    __device__ bool keeps(float v, int i) const { return k.keeps(v, i) && p.keeps(v, i) && expf(v - mx) >= min_w; }
};

__device__ __forceinline__ unsigned long long fixed_weight(float v, float mx) {
    return static_cast<unsigned long long>(static_cast<double>(expf(v - mx)) * kFix);
}

// The kept set of one row, in the host sampler's order.
__device__ Dist distribution(const float *x, int V, const EmberSampleParams &p, SampleLds &sh) {
    Dist d{};
    d.greedy = !(p.temperature > 1e-5f);
    if (d.greedy) return d;
    d.t = p.temperature;
    float m = -INFINITY;
    for_row(x, V, [&](int, float xi) { m = fmaxf(m, xi / d.t); });
    d.mx = block_max(m, sh);
    const Cut all;
    d.k = all;
    d.p = all;
    if (p.top_k > 0 && p.top_k < V) {
        const auto target = static_cast<unsigned long long>(p.top_k);
        const float theta = radix_threshold(x, V, d.t, all, d.mx, false, target, sh);
        d.k = cut_at(x, V, d.t, all, theta, target, 1ull, sh);
    }
    if (p.top_p < 1.0f) {
        unsigned long long s = 0;
        for_row(x, V, [&](int i, float xi) {
            const float v = xi / d.t;
            if (d.k.keeps(v, i)) s += fixed_weight(v, d.mx);
        });
        const unsigned long long zk = block_sum_u64(s, sh);
        const double want = ceil(static_cast<double>(p.top_p) * static_cast<double>(zk));
        const unsigned long long target = want < 1.0 ? 1ull : static_cast<unsigned long long>(want);
        const float theta = radix_threshold(x, V, d.t, d.k, d.mx, true, target, sh);
        d.p = cut_at(x, V, d.t, d.k, theta, target, fixed_weight(theta, d.mx), sh);
    }
    d.min_w = p.min_p > 0.0f ? p.min_p : 0.0f;
    // the kept set's mass (min-p applied), for token probabilities
    unsigned long long s = 0;
    for_row(x, V, [&](int i, float xi) {
        const float v = xi / d.t;
        if (d.keeps(v, i)) s += fixed_weight(v, d.mx);
    });
    d.z = block_sum_u64(s, sh);
    return d;
}

__global__ void __launch_bounds__(kSampleThreads) sample_kernel(const float *__restrict__ logits, int V,
                                                                const EmberSampleParams *__restrict__ params,
                                                                int32_t *__restrict__ out) {
    __shared__ SampleLds sh;
    const int r = static_cast<int>(blockIdx.x);
    const float *x = logits + static_cast<int64_t>(r) * V;
    const EmberSampleParams p = params[r];
    const Dist d = distribution(x, V, p, sh);
    int tok;
    if (d.greedy) {
        tok = block_argmax(x, V, [](int, float xi) { return xi; }, sh);
    } else {
        tok = block_argmax(x, V, [&](int i, float xi) {
            const float v = xi / d.t;
            return d.keeps(v, i) ? v + gumbel_noise(p.seed, p.counter, static_cast<uint32_t>(i)) : -INFINITY;
        }, sh);
    }
    if (threadIdx.x == 0) out[r] = tok;
}

__global__ void __launch_bounds__(kSampleThreads) prob_kernel(const float *__restrict__ logits, int V, int R,
                                                              const EmberSampleParams *__restrict__ params,
                                                              const int32_t *__restrict__ rows,
                                                              const int32_t *__restrict__ tokens,
                                                              float *__restrict__ out) {
    __shared__ SampleLds sh;
    const int q = static_cast<int>(blockIdx.x), r = rows[q], tok = tokens[q];
    if (r < 0 || r >= R || tok < 0 || tok >= V) {  // uniform per work-group
        if (threadIdx.x == 0) out[q] = 0.0f;
        return;
    }
    const float *x = logits + static_cast<int64_t>(r) * V;
    const EmberSampleParams p = params[r];
    const Dist d = distribution(x, V, p, sh);
    float prob;
    if (d.greedy) {
        prob = block_argmax(x, V, [](int, float xi) { return xi; }, sh) == tok ? 1.0f : 0.0f;
    } else {
        const float v = scaled(x, tok, d.t);
        const float w = expf(v - d.mx);
        prob = d.keeps(v, tok) && d.z ? static_cast<float>(static_cast<double>(w) * kFix / static_cast<double>(d.z)) : 0.0f;
    }
    if (threadIdx.x == 0) out[q] = prob;
}

constexpr int kEmbedThreads = 256;

// out[t] = the f16 embedding row of tokens[t], as f32 (k_elementwise.cu's embed_tokens).
__global__ void __launch_bounds__(kEmbedThreads) embed_kernel(const int32_t *__restrict__ tokens, int vocab,
                                                              const f16 *__restrict__ table, int hidden,
                                                              float *__restrict__ out) {
    const int t = static_cast<int>(blockIdx.x);
    const int tok = tokens[t];
    float *o = out + static_cast<int64_t>(t) * hidden;
    if (tok < 0 || tok >= vocab) {  // an id outside the table embeds as zeros (checked on the host)
        for (int i = static_cast<int>(threadIdx.x); i < hidden; i += kEmbedThreads) o[i] = 0.0f;
        return;
    }
    const f16 *row = table + static_cast<int64_t>(tok) * hidden;
    for (int i = 8 * static_cast<int>(threadIdx.x); i < hidden; i += 8 * kEmbedThreads) {
        const f16x8 v = *reinterpret_cast<const f16x8 *>(row + i);
#pragma unroll
        for (int j = 0; j < 8; j++) o[i + j] = static_cast<float>(v[j]);
    }
}

}  // namespace

hipError_t launch_sample(const EmberSampleArgs &a, hipStream_t stream) {
    hipLaunchKernelGGL(sample_kernel, dim3(static_cast<unsigned>(a.R)), dim3(kSampleThreads), 0, stream, a.logits,
                       a.vocab, a.params, a.out);
    return hipGetLastError();
}

hipError_t launch_token_probs(const EmberProbArgs &a, hipStream_t stream) {
    hipLaunchKernelGGL(prob_kernel, dim3(static_cast<unsigned>(a.n)), dim3(kSampleThreads), 0, stream, a.logits,
                       a.vocab, a.R, a.params, a.rows, a.tokens, a.out);
    return hipGetLastError();
}

hipError_t launch_embed(const EmberEmbedArgs &a, hipStream_t stream) {
    hipLaunchKernelGGL(embed_kernel, dim3(static_cast<unsigned>(a.T)), dim3(kEmbedThreads), 0, stream, a.tokens,
                       a.vocab, static_cast<const f16 *>(a.table), a.hidden, a.out);
    return hipGetLastError();
}

}  // namespace ember::hip
