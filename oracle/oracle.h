/*
 * oracle.h - CPU restatement of the reference's paged-KV path. TEST
 * INFRASTRUCTURE ONLY: the checker that tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg call. Nothing in the product (ember_amd/,
 * include/) links, loads or calls it.
 *
 * Each function restates one piece of YUStulinu/Ember's CPU backend or block
 * manager and cites the lines it follows (paths under the reference's root).
 * How each is pinned (checked against something other than itself) is noted
 * per function; see tests/test_oracle_*.py.
 */
#ifndef EMBER_ORACLE_H
#define EMBER_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* IEEE half <-> float, round to nearest even, overflow to inf
 * (src/common/fp16.hpp:25-71). Pinned: numpy.float16, exhaustively / on
 * random and edge values. */
float ember_oracle_f16_to_f32(uint16_t h);
uint16_t ember_oracle_f32_to_f16(float f);
void ember_oracle_f16_to_f32_n(const uint16_t *src, float *dst, int64_t n);
void ember_oracle_f32_to_f16_n(const float *src, uint16_t *dst, int64_t n);

/* inv_freq[i] = 1 / powf(theta, 2i / D) in f32 (src/backend/cpu/cpu_backend.cpp:85-88).
 * Pinned: transformers' Qwen3RotaryEmbedding frequencies. */
void ember_oracle_inv_freq(double theta, int32_t head_dim, float *out);

/* RMSNorm with a double sum of squares (cpu_backend.cpp:34-39). In place is allowed.
 * Pinned: transformers' Qwen3RMSNorm; unit-weight outputs have unit RMS. */
void ember_oracle_rmsnorm(const float *x, const float *w, int32_t n, float eps, float *out);

/* C[M, N] = A[M, K] . W[N, K]^T from f16 bits, each dot product summed in double,
 * then an epilogue (0 store: C = v; 1 store f32: C = v; 2 add f32: C += v;
 * 3 silu_mul: C[m, j] = silu(v[m, 2j]) * v[m, 2j+1], N even), all in f32 after
 * the double sum. Restates the reference's GEMM test reference
 * (tests/test_cuda.cpp:27-47) and epilogues (src/backend/cuda/kernels.cuh:25-30).
 * C is f32 [M, ldc] in every case (the caller rounds f16 outputs).
 * Pinned: numpy float64 matmul, the identity weight, silu's closed form. */
void ember_oracle_linear(const uint16_t *A, const uint16_t *W, int32_t M, int32_t N, int32_t K, int32_t epilogue,
                         float *C, int32_t ldc);
/* The same on `threads` threads; bit-identical results (each output is the
 * same double sum in k order). Pinned: equality with ember_oracle_linear. */
void ember_oracle_linear_mt(const uint16_t *A, const uint16_t *W, int32_t M, int32_t N, int32_t K, int32_t epilogue,
                            float *C, int32_t ldc, int32_t threads);

/* Sampling (src/backend/sampling_host.cpp:20-87, src/backend/sampling_rng.hpp:22-33).
 * Every function here is pinned bit for bit against the reference's own
 * sampler, compiled from its sources into oracle/_ref (oracle/Makefile `ref`;
 * tests/test_oracle_vs_reference.py), including tied logits at the cuts.
 * rng_mix: SplitMix64's output step, also pinned by its published first outputs.
 * gumbel: -log(-log(u)) of a 24-bit uniform from (seed, counter, id); also
 * checked by the Gumbel(0, 1) mean (Euler-Mascheroni) and variance (pi^2 / 6).
 * sampling_distribution: the kept tokens, most likely first, with their
 * probabilities; also checked by numpy restatements of each filter on their
 * own (greedy argmax, top-k by sort, top-p cumulative, min-p ratio) and by the
 * probabilities summing to 1. sample: argmax of logit / T + gumbel over the
 * kept set; also checked by its frequencies against the distribution. */
uint64_t ember_oracle_rng_mix(uint64_t z);
float ember_oracle_gumbel(uint64_t seed, uint64_t counter, uint32_t id);
int32_t ember_oracle_sampling_distribution(const float *logits, int32_t vocab, float temperature, float top_p,
                                           int32_t top_k, float min_p, int32_t *out_tokens, float *out_probs);
int32_t ember_oracle_sample(const float *logits, int32_t vocab, float temperature, float top_p, int32_t top_k,
                            float min_p, uint64_t seed, uint64_t counter);

/* Rotate-half RoPE of one head vector in place (cpu_backend.cpp:262-272).
 * Pinned: transformers' apply_rotary_pos_emb; pos 0 is the identity; pair norms kept. */
void ember_oracle_rope(float *x, int32_t head_dim, int32_t pos, const float *inv_freq);

/* The f32 dot product of the CPU kernels: two 8-wide FMA accumulators over
 * 16-element strides, then a fixed horizontal sum (cpu_kernels_avx2.cpp:27-33,
 * :58-69); the scalar loop of cpu_kernels.cpp:74-79 without AVX2+FMA.
 * Pinned: float64 dot within f32 rounding, and bit for bit against the
 * reference's own AVX2 dot (oracle/_ref) at lengths that are multiples of 8.
 * Other lengths end in a scalar tail whose rounding is the compiler's (the
 * reference's GCC -O3 -mfma build vectorizes it, partly fused); the path never
 * takes it (head_dim 128). */
float ember_oracle_dot(const float *a, const float *b, int32_t n);

/* Offset of (seq, layer, kv_head, pos) in a pool of num_blocks blocks per
 * layer (cpu_backend.cpp:256-260). Pinned: brute-force enumeration of slots. */
int64_t ember_oracle_cache_offset(const int32_t *block_tables, int32_t max_blocks, int32_t num_blocks, int32_t n_kv,
                                  int32_t head_dim, int32_t seq, int32_t layer, int32_t kv_head, int32_t pos);

/* One layer's QK-norm + RoPE + cache store (cpu_backend.cpp:146-172).
 * qkv: [T, (n_heads + 2 n_kv) D] f32 (the q/k/v projections), bias optional.
 * q_out: [T, n_heads, D] f32 after norm + rope.
 * k_cache/v_cache: THIS layer's pools [num_blocks][n_kv][16][D]; f32, or f16
 * bits when kv_f16 (then values are clamped to +-65504 and rounded, as the
 * reference's CUDA store does, k_elementwise.cu:125).
 * Returns 0, or -1 when a slot falls outside the pool. */
int32_t ember_oracle_append_layer(const float *qkv, int32_t T, int32_t n_heads, int32_t n_kv, int32_t head_dim,
                                  const float *q_norm, const float *k_norm, const float *bias, float eps,
                                  const float *inv_freq, const int32_t *positions, const int32_t *query_start,
                                  int32_t num_seqs, const int32_t *block_tables, int32_t max_blocks, float *q_out,
                                  void *k_cache, void *v_cache, int32_t num_blocks, int32_t kv_f16);

/* Causal attention of every token over its sequence's cache, token t seeing
 * positions 0..positions[t] (cpu_backend.cpp:173-198): scores by
 * ember_oracle_dot times 1/sqrt(D), max, exp in f32 summed in double, weights
 * cast to f32, out += w * v. q is [T, n_heads, D] f32 (rounded to f16 first
 * when q_f16, modelling an f16 q buffer). Runs on `threads` threads with the
 * reference pool's chunking (src/common/thread_pool.cpp:57-82).
 * Pinned: float64 textbook softmax(q K^T / sqrt(D)) V (numpy), torch SDPA, and
 * closed forms (ctx 1 -> V0, equal keys -> mean of V). */
int32_t ember_oracle_attention_layer(const float *q, int32_t T, int32_t n_heads, int32_t n_kv, int32_t head_dim,
                                     const int32_t *positions, const int32_t *query_start, int32_t num_seqs,
                                     const int32_t *block_tables, int32_t max_blocks, const void *k_cache,
                                     const void *v_cache, int32_t num_blocks, int32_t kv_f16, int32_t q_f16,
                                     float *out, int32_t threads);

/* ---- block manager (src/kvcache/block_manager.cpp:9-139) ----
 * Pinned: the reference's own unit test (tests/test_engine.cpp:47-78, as a
 * fixture), published FNV-1a 64 vectors and the published inverse of the
 * MurmurHash3 finalizer, check() invariants. */
typedef struct EmberOracleBM EmberOracleBM;
EmberOracleBM *ember_oracle_bm_create(int32_t num_blocks, int32_t prefix_caching);
void ember_oracle_bm_destroy(EmberOracleBM *bm);
int32_t ember_oracle_bm_num_blocks(const EmberOracleBM *bm);
int32_t ember_oracle_bm_available(const EmberOracleBM *bm);
int32_t ember_oracle_bm_cached(const EmberOracleBM *bm);
int32_t ember_oracle_bm_allocate(EmberOracleBM *bm);
int32_t ember_oracle_bm_release(EmberOracleBM *bm, int32_t block);
int32_t ember_oracle_bm_release_all(EmberOracleBM *bm, const int32_t *blocks, int32_t n);
uint64_t ember_oracle_bm_block_hash(uint64_t parent, const int32_t *tokens, int32_t n);
/* The two stages of block_hash, for pinning each against published vectors. */
uint64_t ember_oracle_fnv1a_words(uint64_t parent, const int32_t *tokens, int32_t n);
uint64_t ember_oracle_fmix64(uint64_t h);
int32_t ember_oracle_bm_match_prefix(EmberOracleBM *bm, const int32_t *tokens, int32_t n, int32_t *out_blocks);
uint64_t ember_oracle_bm_seal(EmberOracleBM *bm, int32_t block, uint64_t parent, const int32_t *tokens, int32_t n);
int32_t ember_oracle_bm_refcount(const EmberOracleBM *bm, int32_t block);
uint64_t ember_oracle_bm_hit_tokens(const EmberOracleBM *bm);
uint64_t ember_oracle_bm_lookup_tokens(const EmberOracleBM *bm);
int32_t ember_oracle_bm_check(const EmberOracleBM *bm, char *buf, int32_t buflen);
void ember_oracle_bm_states(const EmberOracleBM *bm, uint8_t *out);
/* The additive fork / copy-on-write semantics (no reference counterpart):
 * share() takes one more reference on each held block; copy_on_write(b)
 * returns b when its refcount is 1, else drops one reference and returns
 * allocate() (or -1). Pinned: invariants only (parity unpinned vs Ember,
 * which has no such call). */
int32_t ember_oracle_bm_share(EmberOracleBM *bm, const int32_t *blocks, int32_t n);
int32_t ember_oracle_bm_copy_on_write(EmberOracleBM *bm, int32_t block);

#ifdef __cplusplus
}
#endif

#endif /* EMBER_ORACLE_H */
