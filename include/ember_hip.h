/*
 * ember_hip.h - C ABI of the MI355X (gfx950) paged-KV hot path.
 *
 * Three layers, all plain C (pointers, sizes, ints; no C++ or torch types):
 *
 *   1. Kernel launchers. Each enqueues work on `stream` (a hipStream_t passed
 *      as void*; NULL = the null stream) and returns immediately. They replace
 *      the CUDA launchers of the reference's kernel seam
 *      (src/backend/cuda/kernels.cuh:74-120) field for field, plus a few
 *      documented additions (pool size for bounds guards, element type, query
 *      runs).
 *   2. The KV block manager (src/kvcache/block_manager.hpp:25-67) behind an
 *      opaque handle, plus two additive calls (share, copy_on_write) that the
 *      reference does not have.
 *   3. The paged-KV path: the KV pool, the step plan (packing, routing,
 *      splits) and the per-layer append + attention that the reference's
 *      CudaBackend::forward / enqueue perform
 *      (src/backend/cuda/cuda_backend.cu:134-205, :288-374).
 *
 * Every function returns EMBER_OK (0), EMBER_ERR_INVALID (-1: a bad argument
 * or unsupported shape; no work was enqueued) or a positive hipError_t. None
 * throws. ember_hip_last_error() describes the last failure on the calling
 * thread.
 *
 * Layout of a layer's K (and, separately, V) pool, identical to the
 * reference's (src/backend/cpu/cpu_backend.cpp:256-260, :290):
 *   [block][kv_head][slot 0..15][head_dim]
 * token at position `pos` of sequence `s` lives in
 *   block = block_tables[s * max_blocks + pos / 16], slot = pos % 16.
 */
#ifndef EMBER_HIP_H
#define EMBER_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define EMBER_ABI_VERSION 7
#define EMBER_BLOCK_SIZE 16  /* tokens per page; kBlockSize, src/backend/backend.hpp:25 */
#define EMBER_PREFILL_TILE 64 /* query tokens per prefill tile; kPrefillTile, kernels.cuh:108 */
#define EMBER_MAX_RUN 8      /* query tokens one decode work-group reads a page for */
#define EMBER_MAX_SPLIT_LEN 1024 /* keys per decode split at most: a split's block ids fit one 64-lane register */

#define EMBER_OK 0
#define EMBER_ERR_INVALID (-1)

/* Element type of q/k/v activations and of the KV pool. f16 is the serving
 * path; f32 is the parity path checked against the f32 CPU backend. */
#define EMBER_DTYPE_F16 0
#define EMBER_DTYPE_F32 1

/* ---- 1. kernel launchers ------------------------------------------------ */

/* Replaces cuda::QkvArgs (kernels.cuh:74-84). */
typedef struct EmberQkvArgs {
    const void *qkv;              /* [T, (n_heads + 2 * n_kv) * head_dim]: q heads, k heads, v heads */
    void *q_out;                  /* [T, n_heads * head_dim] */
    void *k_cache, *v_cache;      /* this layer's pools, [num_blocks][n_kv][16][head_dim] */
    const float *q_norm, *k_norm; /* [head_dim], or NULL: no QK-RMSNorm */
    const float *bias;            /* [(n_heads + 2 * n_kv) * head_dim], or NULL */
    const float *inv_freq;        /* [head_dim / 2] rotary frequencies */
    const int32_t *positions;     /* [T] */
    const int32_t *token_seq;     /* [T] sequence of each token */
    const int32_t *block_tables;  /* [S * max_blocks] */
    int32_t max_blocks, T, n_heads, n_kv, head_dim;
    float eps;
    /* additions */
    int32_t num_blocks;           /* blocks in this layer's pool; a slot in any other block is not written */
    int32_t dtype;                /* EMBER_DTYPE_*: qkv, q_out and the pools */
} EmberQkvArgs;

/* QK-RMSNorm, rotate-half RoPE and the K/V cache write, fused.
 * Replaces cuda::qk_norm_rope_store (kernels.cuh:85-86; k_elementwise.cu:159-171).
 * head_dim must be 128; n_heads and n_kv at most 64; qkv, q_out and the
 * pools 16-byte aligned (the kernel moves 8 elements per access). */
int ember_hip_kv_append(const EmberQkvArgs *args, void *stream);

/* Replaces cuda::AttentionArgs (kernels.cuh:88-101). */
typedef struct EmberAttnArgs {
    const int32_t *token_index;   /* [T] tokens to process, or NULL = 0..T-1 */
    const void *q;                /* [*, n_heads, head_dim] */
    const void *k_cache, *v_cache;
    const int32_t *positions, *token_seq, *block_tables;
    int32_t max_blocks, T, n_heads, n_kv, head_dim;
    float scale;
    void *out;                    /* [*, n_heads, head_dim] */
    int32_t num_splits;           /* context chunks per token: 1 = no split */
    int32_t split_len;            /* keys per chunk, a multiple of 16, at most EMBER_MAX_SPLIT_LEN */
    float *part_acc;              /* [T, n_heads, num_splits, head_dim], indexed by list position 0..T-1 */
    float *part_ml;               /* [T, n_heads, num_splits, 2] */
    /* additions */
    int32_t num_blocks;           /* blocks in this layer's pool; a table entry outside it reads as a page of
                                   * zeros (its loads are bounds-checked and touch no memory) */
    int32_t dtype;                /* EMBER_DTYPE_* of q, out and the pools */
    /* Query runs: list entries [run_first[r], run_first[r] + run_count[r]) are
     * consecutive tokens of one sequence; one work-group reads each page once
     * for all of them. Each token's result is bit-identical to processing it
     * alone. NULL = every listed token is its own run. */
    const int32_t *run_first, *run_count;
    int32_t num_runs;
    int32_t max_run;              /* upper bound of run_count, 1..EMBER_MAX_RUN */
    /* Optional work list: num_work (run, split) pairs, [2 * num_work] ints,
     * each split of each run listed once (splits holding none of the run's
     * keys may be left out). One work-group per (item, kv head), dispatched in
     * list order, so a list with the longest items first balances the tail.
     * NULL = every (run, split < num_splits) pair, splits beyond a run's
     * context finishing at once. */
    const int32_t *work;
    int32_t num_work;
    /* Optional in-kernel split merge: [num_runs * n_kv] counters, zero on
     * entry and left zero. The last work-group of each (run, kv head) to
     * finish merges that run's splits, with the same arithmetic and order as
     * the merge kernel, so no second launch is needed. NULL = a separate
     * merge kernel when num_splits > 1. */
    uint32_t *merge_counters;
    /* Optional, with `work`: what the plan already knows of each item, 16
     * ints per item, [16 * num_work]:
     *   0 run, 1 split, 2 run_first[run], 3 run_count[run], 4 sequence of the
     *   run, 5 lowest position, 6 highest position,
     *   7 token_index[run_first[run]] if the run's entries name tokens t, t+1,
     *     ... at positions lowest, lowest+1, ... (else -1),
     *   8..15 block ids of the split's pages 0..7 (split * split_len / 16 + i
     *     of the sequence's table; -1 past the split's last page).
     * A work-group then issues its first page loads right after one
     * descriptor load, instead of after the chain run -> run_first ->
     * token_index -> token_seq / positions -> table. It must agree with the
     * other arrays (not checked). NULL = looked up as above. */
    const int32_t *work_desc;
} EmberAttnArgs;

/* Paged attention for short runs (decode, speculative verify): one work-group
 * per (run, kv head, context split), all G = n_heads / n_kv query heads of the
 * kv head together, online softmax, then a fixed-order merge of the splits.
 * Replaces cuda::paged_attention (kernels.cuh:102; k_attention.cu:401-415).
 * head_dim must be 128; G in 1..8. */
int ember_hip_paged_decode(const EmberAttnArgs *args, void *stream);

/* Limits of ember_hip_paged_decode_static's scratch (per GPU, held until the
 * process ends): (token, head, split) partials of 130 floats each, and
 * (run, kv head) merge counters. */
#define EMBER_STATIC_MAX_PARTIALS 49152
#define EMBER_STATIC_MAX_COUNTERS 16384
#define EMBER_STATIC_SCRATCH_BYTES (4 * EMBER_STATIC_MAX_COUNTERS + 4 * 130 * EMBER_STATIC_MAX_PARTIALS)

/* No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). ember_hip_paged_decode with its scratch (split partials
 * and merge counters) taken from a static device array of the library instead
 * of args->part_acc / part_ml / merge_counters, which must be NULL; the splits
 * are merged in the kernel, with the merge kernel's arithmetic and order, so
 * the results are bit-identical to ember_hip_paged_decode's. Allocates
 * nothing. Rejects (EMBER_ERR_INVALID) a call needing more than
 * EMBER_STATIC_MAX_PARTIALS partials (T * n_heads * num_splits) or
 * EMBER_STATIC_MAX_COUNTERS counters (runs * n_kv). Every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU (other streams or
 * host threads) race. */
int ember_hip_paged_decode_static(const EmberAttnArgs *args, void *stream);

/* Append + attention in one launch, for a step in which every sequence's new
 * tokens form one decode run (decode: 1 token; speculative verify: k + 1 <= 8)
 * with consecutive positions. Each work-group computes its rows' q
 * (QK-RMSNorm + RoPE) from qkv->qkv, and the K/V of the new tokens that fall
 * in its split: those are stored to the pools and used in place of the page
 * slots they overwrite, so no work-group waits for another. attn->q and
 * qkv->q_out are not used. Every token of qkv must be listed in attn.
 * Results (pools and attention) are bit-identical to ember_hip_kv_append
 * followed by ember_hip_paged_decode. No counterpart in the reference, which
 * launches qk_norm_rope_store and paged_attention separately
 * (src/backend/cuda/cuda_backend.cu:357-360). */
int ember_hip_decode_step(const EmberQkvArgs *qkv, const EmberAttnArgs *attn, void *stream);

/* Replaces cuda::PrefillArgs (kernels.cuh:109-119). */
typedef struct EmberPrefillArgs {
    const void *q;                /* [T, n_heads, head_dim] */
    const void *k_cache, *v_cache;
    const int32_t *tile_start;    /* [num_tiles] first token of the tile */
    const int32_t *tile_end;      /* [num_tiles] one past its last token (at most 64 tokens) */
    const int32_t *tile_seq;      /* [num_tiles] sequence of the tile */
    const int32_t *positions, *block_tables;
    int32_t num_tiles, max_blocks, n_heads, n_kv, head_dim;
    float scale;
    void *out;                    /* [T, n_heads, head_dim] */
    /* additions */
    int32_t num_blocks;
    int32_t dtype;                /* must be EMBER_DTYPE_F16 (MFMA path) */
    /* Query heads per work-group (no counterpart in the reference): 0 lets
     * the launcher choose (2 when G is even, else 1); 1 gives each query head
     * its own work-group; 2 needs an even G. A row's result is the same bits
     * either way, so a planner may pick per launch. */
    int32_t heads_per_group;
} EmberPrefillArgs;

/* Causal attention of query tiles (up to 64 consecutive tokens of one
 * sequence, each attending to keys 0..its position) over the paged cache on
 * MFMA (v_mfma_f32_16x16x32_f16), two query heads of a kv head per work-group
 * (one when G is odd), so a K/V block is read once for both. f16 only; head_dim
 * 128, G 1..8. Replaces cuda::prefill_attention (kernels.cuh:120;
 * k_attention.cu:390-399). */
int ember_hip_prefill_attn(const EmberPrefillArgs *args, void *stream);

/* No counterpart in the reference: the device half of copy-on-write. */
typedef struct EmberCopyArgs {
    void *k_cache, *v_cache;      /* layer 0's pools; layer l starts layer_stride elements later */
    const int32_t *src_blocks;    /* [n] device array */
    const int32_t *dst_blocks;    /* [n] device array */
    int32_t n;                    /* page pairs */
    int32_t n_layers;
    int64_t layer_stride;         /* elements between consecutive layers' pools */
    int32_t n_kv, head_dim;
    int32_t num_blocks;           /* blocks per layer pool; pairs naming others are skipped */
    int32_t dtype;
} EmberCopyArgs;

/* Copies whole pages (every layer, K and V, every kv head) from src to dst. */
int ember_hip_copy_pages(const EmberCopyArgs *args, void *stream);

/* The layer either side of the path: the input RMSNorm and the decode-sized
 * linear layers (qkv projection into the append, output projection into the
 * residual), in the reference's order (cuda_backend.cu:350-362). */

/* Epilogues of ember_hip_gemv; the values of cuda::Epilogue (kernels.cuh:25-30). */
#define EMBER_EPILOGUE_STORE_F16 0 /* C half [M, ldc], clamped to +-65504 */
#define EMBER_EPILOGUE_STORE_F32 1 /* C float [M, ldc] */
#define EMBER_EPILOGUE_ADD_F32 2   /* C float [M, ldc] += the product (the residual stream) */
#define EMBER_EPILOGUE_SILU_MUL 3  /* W rows interleave gate/up; C half [M, ldc], C[m][j] = silu(gate j) * up j */

/* The arguments of cuda::gemm (kernels.cuh:40-41), decode-sized. */
typedef struct EmberGemvArgs {
    const void *A;                /* f16 [M, lda] activations; 16-byte aligned rows */
    int32_t lda;
    const void *W;                /* f16 [N, K] weights, one output feature per row */
    int32_t M, N, K;              /* M 1..64; K a multiple of 32 */
    void *C;                      /* [M, ldc], f16 or f32 by epilogue */
    int32_t ldc;
    int32_t epilogue;             /* EMBER_EPILOGUE_* */
    /* Optional scratch for splitting K over work-groups when N alone gives
     * too few of them (no counterpart in the reference; its gemv_tc does not
     * split). NULL, or fewer bytes than ember_hip_gemv_workspace_bytes(M, N,
     * K), means no split. Zero-filled by the caller once after allocation;
     * every launch leaves it reusable. Launches that overlap in time must
     * not share one. */
    void *workspace;
    int64_t workspace_bytes;
    /* 0: W is row-major [N, K]. 1: W was laid out by ember_hip_gemv_pack
     * (no counterpart in the reference): the same product, the same bits, with
     * every load of W one contiguous KiB. */
    int32_t w_packed;
} EmberGemvArgs;

/* C[M, N] = A[M, K] . W[N, K]^T, f16 in, f32 accumulation, then the epilogue
 * (silu_mul: N even, C has N / 2 columns). MFMA tiles of 16 features x 16
 * tokens, 8 waves splitting K; with a workspace, few features and K beyond
 * 4096, 2 or 4 work-groups per 16 features each take a K slice, and the last to finish
 * adds the slices in slice order (deterministic; the split depends on N and
 * K only, so a token's result does not depend on the batch). Replaces
 * cuda::gemm with GemmKernel::gemv_tc (kernels.cuh:40-41; k_gemm.cu:302-425,
 * :462-485). */
int ember_hip_gemv(const EmberGemvArgs *args, void *stream);

/* Bytes of workspace ember_hip_gemv uses for this shape (0: it would not
 * split). No counterpart in the reference. */
int64_t ember_hip_gemv_workspace_bytes(int32_t M, int32_t N, int32_t K);

/* Bytes of a packed copy of an f16 [N, K] weight (N rounded up to 16 rows). No
 * counterpart in the reference. */
int64_t ember_hip_gemv_packed_bytes(int32_t N, int32_t K);

/* Lays out W (f16 [N, K], K a multiple of 32, 16-byte aligned) for
 * ember_hip_gemv with w_packed = 1: for each 16-row tile and 32-wide k step, the
 * 64 lanes' 16-byte operand pieces in lane order (lane 16 g + c: row 16 t + c,
 * columns 32 s + 8 g ..); rows past N are zero. out holds
 * ember_hip_gemv_packed_bytes(N, K). A backend packs once, at weight load. */
int ember_hip_gemv_pack(const void *W, int32_t N, int32_t K, void *out, void *stream);

/* The arguments of cuda::rmsnorm_rows (kernels.cuh:70-72). */
typedef struct EmberNormArgs {
    const float *x;               /* f32 [*, hidden] */
    const int32_t *rows;          /* [R] rows of x, or NULL = rows 0..R-1 */
    int32_t R, hidden;
    const float *w;               /* [hidden] */
    float eps;
    void *out;                    /* f16 [R, hidden] */
} EmberNormArgs;

/* out[r] = w * (x[row r] * scale), scale = 1 / sqrt(sum of squares / hidden +
 * eps), as f16 clamped to +-65504. The sum of squares is taken in double and
 * the scale rounded once to f32, as the CPU backend does
 * (cpu_backend.cpp:34-39). Replaces cuda::rmsnorm_rows (kernels.cuh:70-72;
 * k_elementwise.cu:52-65). */
int ember_hip_rmsnorm_rows(const EmberNormArgs *args, void *stream);

/* The arguments of cuda::embed_tokens (kernels.cuh:68). */
typedef struct EmberEmbedArgs {
    const int32_t *tokens;        /* [T] device */
    int32_t T;
    const void *table;            /* f16 [vocab, hidden], rows 16-byte aligned */
    int32_t vocab, hidden;        /* hidden a multiple of 8 */
    float *out;                   /* f32 [T, hidden] */
} EmberEmbedArgs;

/* out[t] = table[tokens[t]] as f32 (the residual stream's start); a token id
 * outside the table embeds as zeros. Replaces cuda::embed_tokens
 * (kernels.cuh:68; k_elementwise.cu). */
int ember_hip_embed(const EmberEmbedArgs *args, void *stream);

/* cuda::DeviceSampleParams (kernels.cuh:124-128), one per row of logits. */
typedef struct EmberSampleParams {
    float temperature, top_p, min_p;   /* temperature <= 1e-5: greedy */
    int32_t top_k;                     /* 0: no limit */
    uint64_t seed, counter;            /* the Gumbel noise's inputs */
} EmberSampleParams;

/* The arguments of cuda::sample_tokens (kernels.cuh:130). */
typedef struct EmberSampleArgs {
    const float *logits;          /* [R, vocab] device */
    int32_t R, vocab;
    const EmberSampleParams *params; /* [R] device */
    int32_t *out;                 /* [R] device */
} EmberSampleArgs;

/* One token per row: greedy rows take the first largest logit; the others
 * keep v = logit / temperature within top-k, then top-p of the top-k set's
 * mass, then min-p relative to the most likely token (the host sampler's
 * sampling_distribution, src/backend/sampling_host.cpp:20-66), and take the
 * argmax of v + Gumbel(seed, counter, token id) over the kept set
 * (sampling_rng.hpp:20-33). Replaces cuda::sample_tokens (kernels.cuh:130;
 * k_sampling.cu:149-170). */
int ember_hip_sample(const EmberSampleArgs *args, void *stream);

/* The arguments of cuda::token_probabilities (kernels.cuh:132-133). */
typedef struct EmberProbArgs {
    const float *logits;          /* [R, vocab] device */
    int32_t vocab;
    const EmberSampleParams *params; /* [R] per logit row, device */
    const int32_t *rows, *tokens; /* [n] device */
    int32_t n;
    float *out;                   /* [n] device */
    /* addition */
    int32_t R;                    /* rows of logits; a query naming another row, or a token outside the
                                   * vocabulary, gets probability 0 */
} EmberProbArgs;

/* out[i] = the probability of tokens[i] in row rows[i]'s sampling
 * distribution (1 or 0 for greedy rows). Replaces cuda::token_probabilities
 * (kernels.cuh:132-133; k_sampling.cu:172-186). */
int ember_hip_token_probs(const EmberProbArgs *args, void *stream);

/* Description of the last failure on this thread ("" if none). */
const char *ember_hip_last_error(void);
int ember_hip_abi_version(void);
/* sizeof of each argument struct, for FFI bindings to check their layouts:
 * 0 EmberQkvArgs, 1 EmberAttnArgs, 2 EmberPrefillArgs, 3 EmberCopyArgs,
 * 4 EmberKvConfig, 5 EmberStepBatch, 6 EmberLayerIo, 7 EmberGemvArgs,
 * 8 EmberNormArgs, 9 EmberEmbedArgs, 10 EmberSampleParams, 11 EmberSampleArgs,
 * 12 EmberProbArgs, 13 EmberBackendOptions, 14 EmberModelInfo; -1 otherwise. */
int32_t ember_hip_sizeof(int32_t which);

/* ---- 2. KV block manager ------------------------------------------------- */

/* Opaque handle to ember::BlockManager (src/kvcache/block_manager.hpp:25-87). */
typedef struct EmberBlockManager EmberBlockManager;

/* BlockManager(num_blocks, prefix_caching) (block_manager.hpp:27); NULL on error. */
EmberBlockManager *ember_bm_create(int32_t num_blocks, int32_t prefix_caching);
void ember_bm_destroy(EmberBlockManager *bm);
int32_t ember_bm_num_blocks(const EmberBlockManager *bm);  /* :29 */
int32_t ember_bm_available(const EmberBlockManager *bm);   /* :31 */
int32_t ember_bm_used(const EmberBlockManager *bm);        /* :32 */
int32_t ember_bm_cached(const EmberBlockManager *bm);      /* :33 */
/* allocate (:37): a fresh block, or -1 when none is available. */
int32_t ember_bm_allocate(EmberBlockManager *bm);
/* release (:39): EMBER_ERR_INVALID when the block is free (the reference throws). */
int32_t ember_bm_release(EmberBlockManager *bm, int32_t block);
/* release_all (:40): releases blocks[n-1] first. */
int32_t ember_bm_release_all(EmberBlockManager *bm, const int32_t *blocks, int32_t n);
/* block_hash (:43). */
uint64_t ember_bm_block_hash(uint64_t parent, const int32_t *tokens, int32_t n);
/* match_prefix (:47): writes up to n / 16 blocks to out_blocks, returns how many. */
int32_t ember_bm_match_prefix(EmberBlockManager *bm, const int32_t *tokens, int32_t n, int32_t *out_blocks);
/* seal (:52): returns the block's hash; 0 (never a valid hash) on error. */
uint64_t ember_bm_seal(EmberBlockManager *bm, int32_t block, uint64_t parent, const int32_t *tokens, int32_t n);
int32_t ember_bm_prefix_caching(const EmberBlockManager *bm); /* :54 */
int32_t ember_bm_refcount(const EmberBlockManager *bm, int32_t block); /* :55 */
uint64_t ember_bm_hit_tokens(const EmberBlockManager *bm);    /* :58 */
uint64_t ember_bm_lookup_tokens(const EmberBlockManager *bm); /* :59 */
/* check (:64): copies the first problem (or "") into buf; returns 0 if consistent, 1 if not. */
int32_t ember_bm_check(const EmberBlockManager *bm, char *buf, int32_t buflen);
/* states (:67): one byte per block, 0 free, 1 cached, 2 in use. */
void ember_bm_states(const EmberBlockManager *bm, uint8_t *out);
/* No counterpart in the reference: takes one more reference on each of n
 * blocks held by a sequence being forked, partial last page included. */
int32_t ember_bm_share(EmberBlockManager *bm, const int32_t *blocks, int32_t n);
/* No counterpart in the reference: before writing into `block`, a holder calls
 * this. Returns `block` itself when the caller is its only holder; otherwise
 * drops the caller's reference and returns a fresh private block (the caller
 * copies the page into it), or -1 when none is available (the reference is
 * kept then). -2 when `block` is not held. */
int32_t ember_bm_copy_on_write(EmberBlockManager *bm, int32_t block);

/* ---- 3. the paged-KV path -------------------------------------------------- */

typedef struct EmberKvConfig {
    int32_t n_layers, n_heads, n_kv_heads, head_dim;
    float rms_eps;
    double rope_theta;
    int32_t max_position;     /* bounds the block-table width */
    int32_t num_blocks;       /* blocks the engine may hand out; one spare block per layer is added */
    int32_t max_batch_tokens; /* tokens per step */
    int32_t max_seqs;         /* sequences per step */
    int32_t dtype;            /* EMBER_DTYPE_* of activations and pools */
    int32_t qk_norm;          /* nonzero: q_norm / k_norm weights are given per layer */
    int32_t split_len;        /* keys per decode split, multiple of 16 up to EMBER_MAX_SPLIT_LEN (0 = 512) */
} EmberKvConfig;

/* Replaces ember::StepBatch (src/backend/backend.hpp:56-76); host arrays. */
typedef struct EmberStepBatch {
    const int32_t *tokens;        /* [num_tokens] */
    const int32_t *positions;     /* [num_tokens] */
    const int32_t *query_start;   /* [num_seqs + 1] */
    const int32_t *context_len;   /* [num_seqs] */
    const int32_t *block_tables;  /* [num_seqs * max_blocks] */
    int32_t num_tokens, num_seqs, max_blocks;
} EmberStepBatch;

typedef struct EmberPagedKv EmberPagedKv;

/* Allocates the pools (zeroed), rotary table, q buffer, split scratch and
 * step buffers on the current device; all work goes to `stream`. NULL on error. */
EmberPagedKv *ember_kv_create(const EmberKvConfig *cfg, void *stream);
void ember_kv_destroy(EmberPagedKv *kv);
/* Packs the step's integers, routes runs of >= 16 new tokens to prefill tiles
 * and the rest to decode runs, fixes the splits and uploads the plan with one
 * host-to-device copy (cuda_backend.cu:153-205). The copy runs on a side
 * stream once the kernels of the plan before the previous one are done; the
 * call returns when it has landed (so it blocks while the GPU is more than a
 * step behind), and the stream then needs no cross-stream wait. */
int32_t ember_kv_plan(EmberPagedKv *kv, const EmberStepBatch *batch);
/* One layer of the planned step: append K/V of every new token, then attention
 * for every token into out [num_tokens, n_heads, head_dim] (cuda_backend.cu:357-361).
 * qkv must be 16-byte aligned. */
int32_t ember_kv_layer(EmberPagedKv *kv, int32_t layer, const void *qkv, const float *q_norm, const float *k_norm,
                       const float *bias, void *out);
/* One layer's buffers for a decode step replayed as a graph. */
typedef struct EmberLayerIo {
    const void *qkv;              /* [token_bucket(T), (n_heads + 2 * n_kv) * head_dim]; rows past T are padding */
    const float *q_norm, *k_norm; /* [head_dim], or NULL */
    const float *bias;            /* or NULL */
    void *out;                    /* [token_bucket(T), n_heads, head_dim] */
} EmberLayerIo;

/* A pure decode step (every sequence one new token, at most 64 tokens) planned
 * and run for all n_layers layers as one replayed hipGraph, as the reference's
 * decode graphs do (src/backend/cuda/cuda_backend.cu:376-454). The step is
 * padded to a token bucket {1, 2, 3, 4, 6, 8, 12, 16, 24, 32, 40, 48, 56, 64}
 * and a block-table width bucket (16 * 4^k blocks); padding tokens are
 * sequences of one token at position 0 whose table is the spare block, so they
 * write only there, and the splits follow the width bucket. Graphs are kept per
 * bucket pair and captured again when the layer buffers change; the buffers
 * must hold token_bucket(T) rows (64 suffice). Results equal plan + layer
 * bit for bit. Returns EMBER_OK, 1 when the step does not qualify (nothing was
 * enqueued: use ember_kv_plan + ember_kv_layer), or an error. */
int32_t ember_kv_decode_graph(EmberPagedKv *kv, const EmberStepBatch *batch, const EmberLayerIo *layers,
                              int32_t n_layers);
/* Graphs ember_kv_decode_graph has captured so far on this path (launches of a
 * kept graph do not count); -1 for a NULL handle. No counterpart in the
 * reference: a diagnostic for tests and benchmarks. */
int64_t ember_kv_graph_captures(const EmberPagedKv *kv);
/* Device copies of whole pages, src[i] -> dst[i] (host arrays of n blocks), all layers. */
int32_t ember_kv_copy_blocks(EmberPagedKv *kv, const int32_t *src, const int32_t *dst, int32_t n);
void *ember_kv_k_pool(EmberPagedKv *kv, int32_t layer);
void *ember_kv_v_pool(EmberPagedKv *kv, int32_t layer);
int64_t ember_kv_layer_stride(const EmberPagedKv *kv); /* elements between layers' pools */
int32_t ember_kv_spare_block(const EmberPagedKv *kv);  /* the block padding rows write to */
/* What the current plan launches per layer: decode runs, prefill tiles,
 * splits, and whether append and attention share one launch (every
 * sequence's new tokens form one run: ember_hip_decode_step). */
int32_t ember_kv_plan_info(const EmberPagedKv *kv, int32_t *decode_runs, int32_t *prefill_tiles, int32_t *num_splits,
                           int32_t *fused);
/* Kernel timing for benchmarks: while on, every layer() records HIP events on
 * the path's stream right before and right after the paged-decode kernel
 * (before the split merge) and the prefill-tile kernel. ember_kv_timing waits
 * for the paged-decode ones and returns the number of timed launches and their
 * total duration in ms, then starts over. */
int32_t ember_kv_set_timing(EmberPagedKv *kv, int32_t on);
int32_t ember_kv_timing(EmberPagedKv *kv, int32_t *launches, double *total_ms);
/* The same for the prefill-tile kernel's launches (timed while timing is on). */
int32_t ember_kv_prefill_timing(EmberPagedKv *kv, int32_t *launches, double *total_ms);

/* ---- 4. the backend ---------------------------------------------------------
 * ember::Backend (src/backend/backend.hpp:94-123) with device "hip", behind
 * an opaque handle: create_backend(model_dir, options) (backend.hpp:125;
 * backend.cpp:77-87) over a Hugging Face model directory (config.json,
 * generation_config.json, model.safetensors or its index), then forward /
 * sample / token_probs / logits per step. C++ callers use the classes in
 * ember_amd/csrc/host directly; these calls are the same for other FFIs. */

/* The BackendOptions fields a HIP backend reads (backend.hpp:35-48). */
typedef struct EmberBackendOptions {
    int32_t max_batch_tokens;     /* tokens per forward */
    int32_t max_seqs;             /* sequences per forward */
    int32_t max_logit_rows;       /* logit rows per forward (0 = max_seqs) */
    int64_t kv_cache_bytes;       /* K + V cache size, or 0 */
    int32_t kv_cache_tokens;      /* or the cache in tokens, or 0 (then memory_fraction of free memory) */
    double memory_fraction;       /* 0 = the default (0.92) */
    int32_t gpu;                  /* device index */
    int32_t graphs;               /* BackendOptions::cuda_graphs: 1 on, -1 off, 0 the default (on) */
} EmberBackendOptions;

typedef struct EmberModelInfo {
    int32_t vocab_size, hidden, intermediate, n_layers, n_heads, n_kv_heads, head_dim;
    int32_t num_kv_blocks;        /* Backend::num_kv_blocks(): blocks the engine may hand out */
    int32_t max_logit_rows;
} EmberModelInfo;

typedef struct EmberBackend EmberBackend;

/* NULL on error (ember_hip_last_error() says why). */
EmberBackend *ember_backend_create(const char *model_dir, const EmberBackendOptions *options);
void ember_backend_destroy(EmberBackend *backend);
int32_t ember_backend_info(const EmberBackend *backend, EmberModelInfo *out);
/* Whole-step decode graphs replayed so far by every backend of the process
 * (no counterpart in the reference; a diagnostic for tests and benchmarks). */
int64_t ember_backend_graph_replays(void);
/* Whole-step decode graphs captured and instantiated so far by every backend
 * of the process: one per planned layout (token bucket, table-width bucket). */
int64_t ember_backend_graph_captures(void);
/* Backend::forward (backend.hpp:104-106): appends every token's K/V and keeps
 * the logits of the n_rows tokens logit_rows[] on the device. */
int32_t ember_backend_forward(EmberBackend *backend, const EmberStepBatch *batch, const int32_t *logit_rows,
                              int32_t n_rows);
/* Backend::sample: one token per logit row, params[i] (with its counter) for row i. */
int32_t ember_backend_sample(EmberBackend *backend, const EmberSampleParams *params, int32_t n, int32_t *out);
/* Backend::token_probs: out[i] = P(tokens[i]) in row rows[i]'s distribution; n_params covers every row. */
int32_t ember_backend_token_probs(EmberBackend *backend, const EmberSampleParams *params, int32_t n_params,
                                  const int32_t *rows, const int32_t *tokens, int32_t n, float *out);
/* Backend::logits: row `row`'s logits into out[0..n), n >= vocab_size. */
int32_t ember_backend_logits(EmberBackend *backend, int32_t row, float *out, int32_t n);
int32_t ember_backend_set_capture_hidden(EmberBackend *backend, int32_t on);
/* Backend::captured_hidden: the last token's residual after the embedding and
 * each layer, [(n_layers + 1) * hidden]; returns the count written. */
int32_t ember_backend_captured_hidden(EmberBackend *backend, float *out, int32_t n);

#ifdef __cplusplus
}
#endif

#endif /* EMBER_HIP_H */
