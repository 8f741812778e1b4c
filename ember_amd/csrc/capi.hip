// C ABI of the kernel launchers (include/ember_hip.h, part 1): argument
// validation, instance selection, error reporting. Nothing here throws; every
// failure is a return code plus a per-thread message.
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <string>

#include "capi_errors.hpp"
#include "device.hpp"
#include "ember_hip.h"
#include "kernels.hpp"

namespace ember::hip {

namespace {
thread_local std::string g_last_error;
}

int set_error(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int hip_status(hipError_t e, const char *what) {
    if (e == hipSuccess) return EMBER_OK;
    return set_error(static_cast<int>(e), "%s: %s", what, hipGetErrorString(e));
}

namespace {

bool valid_dtype(int d) { return d == EMBER_DTYPE_F16 || d == EMBER_DTYPE_F32; }

int check_heads(const char *who, int head_dim, int n_heads, int n_kv) {
    if (head_dim != kHeadDim) return set_error(EMBER_ERR_INVALID, "%s: head_dim %d is not supported (128)", who, head_dim);
    if (n_kv <= 0 || n_heads <= 0 || n_heads % n_kv != 0)
        return set_error(EMBER_ERR_INVALID, "%s: %d query heads do not group over %d kv heads", who, n_heads, n_kv);
    return EMBER_OK;
}

}  // namespace
}  // namespace ember::hip

using namespace ember::hip;

extern "C" {

const char *ember_hip_last_error(void) { return g_last_error.c_str(); }

int ember_hip_abi_version(void) { return EMBER_ABI_VERSION; }

int32_t ember_hip_sizeof(int32_t which) {
    switch (which) {
        case 0: return sizeof(EmberQkvArgs);
        case 1: return sizeof(EmberAttnArgs);
        case 2: return sizeof(EmberPrefillArgs);
        case 3: return sizeof(EmberCopyArgs);
        case 4: return sizeof(EmberKvConfig);
        case 5: return sizeof(EmberStepBatch);
        case 6: return sizeof(EmberLayerIo);
        case 7: return sizeof(EmberGemvArgs);
        case 8: return sizeof(EmberNormArgs);
        case 9: return sizeof(EmberEmbedArgs);
        case 10: return sizeof(EmberSampleParams);
        case 11: return sizeof(EmberSampleArgs);
        case 12: return sizeof(EmberProbArgs);
        case 13: return sizeof(EmberBackendOptions);
        case 14: return sizeof(EmberModelInfo);
        default: return -1;
    }
}

int ember_hip_kv_append(const EmberQkvArgs *a, void *stream) {
    g_last_error.clear();
    if (!a) return set_error(EMBER_ERR_INVALID, "kv_append: null arguments");
    if (int e = check_heads("kv_append", a->head_dim, a->n_heads, a->n_kv)) return e;
    if (a->n_heads > 64 || a->n_kv > 64)
        return set_error(EMBER_ERR_INVALID, "kv_append: at most 64 query and 64 kv heads (got %d, %d)", a->n_heads, a->n_kv);
    if (!valid_dtype(a->dtype)) return set_error(EMBER_ERR_INVALID, "kv_append: unknown dtype %d", a->dtype);
    if (a->T < 0 || a->max_blocks <= 0 || a->num_blocks <= 0)
        return set_error(EMBER_ERR_INVALID, "kv_append: bad sizes (T %d, max_blocks %d, num_blocks %d)", a->T, a->max_blocks,
                         a->num_blocks);
    if (a->T == 0) return EMBER_OK;
    if (!a->qkv || !a->q_out || !a->k_cache || !a->v_cache || !a->inv_freq || !a->positions || !a->token_seq ||
        !a->block_tables)
        return set_error(EMBER_ERR_INVALID, "kv_append: a required pointer is null");
    if ((a->q_norm == nullptr) != (a->k_norm == nullptr))
        return set_error(EMBER_ERR_INVALID, "kv_append: q_norm and k_norm go together");
    if ((reinterpret_cast<uintptr_t>(a->qkv) | reinterpret_cast<uintptr_t>(a->q_out) |
         reinterpret_cast<uintptr_t>(a->k_cache) | reinterpret_cast<uintptr_t>(a->v_cache)) % 16 != 0)
        return set_error(EMBER_ERR_INVALID, "kv_append: qkv, q_out and the pools must be 16-byte aligned");
    return hip_status(launch_kv_append(*a, static_cast<hipStream_t>(stream)), "kv_append");
}

int ember_hip_paged_decode(const EmberAttnArgs *a, void *stream) {
    return paged_decode(a, static_cast<hipStream_t>(stream), nullptr, nullptr);
}

int ember_hip_decode_step(const EmberQkvArgs *qkv, const EmberAttnArgs *attn, void *stream) {
    if (!qkv) return set_error(EMBER_ERR_INVALID, "decode_step: null qkv arguments");
    return paged_decode(attn, static_cast<hipStream_t>(stream), nullptr, nullptr, qkv);
}

}  // extern "C"

int ember::hip::prefill_attn(const EmberPrefillArgs *a, hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
    g_last_error.clear();
    if (!a) return set_error(EMBER_ERR_INVALID, "prefill_attn: null arguments");
    if (int e = check_heads("prefill_attn", a->head_dim, a->n_heads, a->n_kv)) return e;
    const int G = a->n_heads / a->n_kv;
    if (G > 8) return set_error(EMBER_ERR_INVALID, "prefill_attn: query heads per kv head must be 1..8 (got %d)", G);
    if (a->dtype != EMBER_DTYPE_F16) return set_error(EMBER_ERR_INVALID, "prefill_attn: the MFMA path takes f16 only");
    if (a->num_tiles < 0 || a->max_blocks <= 0 || a->num_blocks <= 0)
        return set_error(EMBER_ERR_INVALID, "prefill_attn: bad sizes");
    if (!(a->scale > 0.0f) || !std::isfinite(a->scale))  // the block max is taken before scaling
        return set_error(EMBER_ERR_INVALID, "prefill_attn: scale must be positive and finite");
    if (a->heads_per_group < 0 || a->heads_per_group > 2 || (a->heads_per_group == 2 && G % 2 != 0))
        return set_error(EMBER_ERR_INVALID, "prefill_attn: heads_per_group is 0, 1 or 2 (2 only for an even G; got %d)",
                         a->heads_per_group);
    if (a->num_tiles == 0) return EMBER_OK;
    if (!a->q || !a->k_cache || !a->v_cache || !a->tile_start || !a->tile_end || !a->tile_seq || !a->positions ||
        !a->block_tables || !a->out)
        return set_error(EMBER_ERR_INVALID, "prefill_attn: a required pointer is null");
    return hip_status(launch_prefill(*a, stream, start, stop), "prefill_attn");
}

int ember::hip::decode_rows(int G, int max_run) {
    for (int r : kDecodeRowInstances)
        if (r >= G * max_run) return r;
    return 0;
}

int ember::hip::paged_decode(const EmberAttnArgs *a, hipStream_t stream, hipEvent_t start, hipEvent_t stop,
                             const EmberQkvArgs *qkv) {
    g_last_error.clear();
    if (!a) return set_error(EMBER_ERR_INVALID, "paged_decode: null arguments");
    if (qkv) {  // the fused form: both argument sets describe the same step
        if (qkv->n_heads != a->n_heads || qkv->n_kv != a->n_kv || qkv->head_dim != a->head_dim ||
            qkv->dtype != a->dtype || qkv->max_blocks != a->max_blocks || qkv->num_blocks != a->num_blocks ||
            qkv->positions != a->positions || qkv->token_seq != a->token_seq || qkv->block_tables != a->block_tables)
            return set_error(EMBER_ERR_INVALID, "decode_step: the qkv and attention arguments describe different steps");
        if (!qkv->qkv || !qkv->inv_freq || (qkv->q_norm == nullptr) != (qkv->k_norm == nullptr))
            return set_error(EMBER_ERR_INVALID, "decode_step: qkv, inv_freq (and q_norm with k_norm) are required");
        if (a->run_first && a->max_run > EMBER_MAX_RUN)
            return set_error(EMBER_ERR_INVALID, "decode_step: a run holds at most %d tokens", EMBER_MAX_RUN);
        if (qkv->T != a->T)
            return set_error(EMBER_ERR_INVALID, "decode_step: every token of qkv (%d) must be listed (%d)", qkv->T, a->T);
    }
    if (int e = check_heads("paged_decode", a->head_dim, a->n_heads, a->n_kv)) return e;
    const int G = a->n_heads / a->n_kv;
    if (G > 8) return set_error(EMBER_ERR_INVALID, "paged_decode: query heads per kv head must be 1..8 (got %d)", G);
    if (!valid_dtype(a->dtype)) return set_error(EMBER_ERR_INVALID, "paged_decode: unknown dtype %d", a->dtype);
    if (a->T < 0 || a->max_blocks <= 0 || a->num_blocks <= 0)
        return set_error(EMBER_ERR_INVALID, "paged_decode: bad sizes");
    if (a->num_splits < 1 || a->num_splits > 65535 || a->split_len < kPage || a->split_len % kPage != 0 ||
        a->split_len > EMBER_MAX_SPLIT_LEN)
        return set_error(EMBER_ERR_INVALID, "paged_decode: split_len must be a multiple of 16 in 16..%d (got %d x %d)",
                         EMBER_MAX_SPLIT_LEN, a->num_splits, a->split_len);
    if (a->T == 0) return EMBER_OK;
    if ((!a->q && !qkv) || !a->k_cache || !a->v_cache || !a->positions || !a->token_seq || !a->block_tables || !a->out)
        return set_error(EMBER_ERR_INVALID, "paged_decode: a required pointer is null");
    if (a->num_splits > 1 && (!a->part_acc || !a->part_ml))
        return set_error(EMBER_ERR_INVALID, "paged_decode: split scratch is required when num_splits > 1");
    int max_run = 1;
    if (a->run_first) {
        if (!a->run_count || a->num_runs < 0 || a->num_runs > a->T)
            return set_error(EMBER_ERR_INVALID, "paged_decode: run_first needs run_count and 0 <= num_runs <= T");
        if (a->max_run < 1 || a->max_run > EMBER_MAX_RUN)
            return set_error(EMBER_ERR_INVALID, "paged_decode: max_run must be 1..%d (got %d)", EMBER_MAX_RUN, a->max_run);
        max_run = a->max_run;
    }
    if (a->work) {
        const long long runs = a->run_first ? a->num_runs : a->T;
        if (a->num_work < 0 || a->num_work > runs * a->num_splits ||
            static_cast<long long>(a->num_work) * a->n_kv > 0x7fffffffLL)
            return set_error(EMBER_ERR_INVALID, "paged_decode: num_work %d out of range", a->num_work);
    }
    const int rows = decode_rows(G, max_run);
    if (!rows) return set_error(EMBER_ERR_INVALID, "paged_decode: %d query rows per work-group exceed 16", G * max_run);
    if (qkv) return hip_status(launch_decode_step(*qkv, *a, rows, stream, start, stop), "decode_step");
    return hip_status(launch_paged_decode(*a, rows, stream, start, stop), "paged_decode");
}

extern "C" {

int ember_hip_prefill_attn(const EmberPrefillArgs *a, void *stream) {
    return prefill_attn(a, static_cast<hipStream_t>(stream), nullptr, nullptr);
}

int ember_hip_copy_pages(const EmberCopyArgs *a, void *stream) {
    g_last_error.clear();
    if (!a) return set_error(EMBER_ERR_INVALID, "copy_pages: null arguments");
    if (!valid_dtype(a->dtype)) return set_error(EMBER_ERR_INVALID, "copy_pages: unknown dtype %d", a->dtype);
    if (a->n < 0 || a->n_layers < 0 || a->n_kv <= 0 || a->head_dim <= 0 || a->num_blocks <= 0 || a->layer_stride < 0)
        return set_error(EMBER_ERR_INVALID, "copy_pages: bad sizes");
    if (a->n == 0 || a->n_layers == 0) return EMBER_OK;
    const long long elem = a->dtype == EMBER_DTYPE_F16 ? 2 : 4;
    if ((static_cast<long long>(a->n_kv) * kPage * a->head_dim * elem) % 16 != 0)
        return set_error(EMBER_ERR_INVALID, "copy_pages: a page must be a multiple of 16 bytes");
    if (a->layer_stride < static_cast<long long>(a->num_blocks) * a->n_kv * kPage * a->head_dim)
        return set_error(EMBER_ERR_INVALID, "copy_pages: layer_stride is smaller than a layer's pool");
    if (!a->k_cache || !a->v_cache || !a->src_blocks || !a->dst_blocks)
        return set_error(EMBER_ERR_INVALID, "copy_pages: a required pointer is null");
    return hip_status(launch_copy_pages(*a, static_cast<hipStream_t>(stream)), "copy_pages");
}

int ember_hip_gemv(const EmberGemvArgs *a, void *stream) {
    g_last_error.clear();
    if (!a) return set_error(EMBER_ERR_INVALID, "gemv: null arguments");
    if (a->M < 1 || a->M > 64) return set_error(EMBER_ERR_INVALID, "gemv: M must be 1..64 (got %d)", a->M);
    if (a->N < 1 || a->K < 32 || a->K % 32 != 0)
        return set_error(EMBER_ERR_INVALID, "gemv: N >= 1 and K a positive multiple of 32 (got N %d, K %d)", a->N, a->K);
    if (a->epilogue < EMBER_EPILOGUE_STORE_F16 || a->epilogue > EMBER_EPILOGUE_SILU_MUL)
        return set_error(EMBER_ERR_INVALID, "gemv: unknown epilogue %d", a->epilogue);
    if (a->epilogue == EMBER_EPILOGUE_SILU_MUL && a->N % 2 != 0)
        return set_error(EMBER_ERR_INVALID, "gemv: silu_mul needs an even N (got %d)", a->N);
    const int cols = a->epilogue == EMBER_EPILOGUE_SILU_MUL ? a->N / 2 : a->N;
    if (a->lda < a->K || a->lda % 8 != 0 || a->ldc < cols)
        return set_error(EMBER_ERR_INVALID, "gemv: lda must be >= K and a multiple of 8, ldc >= %d (got %d, %d)", cols,
                         a->lda, a->ldc);
    if (!a->A || !a->W || !a->C) return set_error(EMBER_ERR_INVALID, "gemv: a required pointer is null");
    if (reinterpret_cast<uintptr_t>(a->A) % 16 != 0 || reinterpret_cast<uintptr_t>(a->W) % 16 != 0)
        return set_error(EMBER_ERR_INVALID, "gemv: A and W must be 16-byte aligned");
    if (a->w_packed != 0 && a->w_packed != 1) return set_error(EMBER_ERR_INVALID, "gemv: w_packed is 0 or 1");
    if (a->workspace_bytes < 0 || reinterpret_cast<uintptr_t>(a->workspace) % 16 != 0)
        return set_error(EMBER_ERR_INVALID, "gemv: the workspace must be 16-byte aligned with a size >= 0");
    return hip_status(launch_gemv(*a, static_cast<hipStream_t>(stream)), "gemv");
}

int64_t ember_hip_gemv_packed_bytes(int32_t N, int32_t K) {
    if (N < 1 || K < 32 || K % 32 != 0) return 0;
    return gemv_packed_bytes(N, K);
}

int ember_hip_gemv_pack(const void *W, int32_t N, int32_t K, void *out, void *stream) {
    g_last_error.clear();
    if (N < 1 || K < 32 || K % 32 != 0)
        return set_error(EMBER_ERR_INVALID, "gemv_pack: N >= 1 and K a positive multiple of 32 (got N %d, K %d)", N, K);
    if (!W || !out) return set_error(EMBER_ERR_INVALID, "gemv_pack: a required pointer is null");
    if (reinterpret_cast<uintptr_t>(W) % 16 != 0 || reinterpret_cast<uintptr_t>(out) % 16 != 0)
        return set_error(EMBER_ERR_INVALID, "gemv_pack: W and out must be 16-byte aligned");
    return hip_status(launch_gemv_pack(W, N, K, out, static_cast<hipStream_t>(stream)), "gemv_pack");
}

int64_t ember_hip_gemv_workspace_bytes(int32_t M, int32_t N, int32_t K) {
    if (M < 1 || M > 64 || N < 1 || K < 32 || K % 32 != 0) return 0;
    return gemv_workspace_bytes(M, N, K);
}

int ember_hip_embed(const EmberEmbedArgs *a, void *stream) {
    g_last_error.clear();
    if (!a) return set_error(EMBER_ERR_INVALID, "embed: null arguments");
    if (a->T < 0 || a->vocab < 1 || a->hidden < 8 || a->hidden % 8 != 0)
        return set_error(EMBER_ERR_INVALID, "embed: bad sizes (T %d, vocab %d, hidden %d: a multiple of 8)", a->T,
                         a->vocab, a->hidden);
    if (a->T == 0) return EMBER_OK;
    if (!a->tokens || !a->table || !a->out) return set_error(EMBER_ERR_INVALID, "embed: a required pointer is null");
    if (reinterpret_cast<uintptr_t>(a->table) % 16 != 0)
        return set_error(EMBER_ERR_INVALID, "embed: the table must be 16-byte aligned");
    return hip_status(launch_embed(*a, static_cast<hipStream_t>(stream)), "embed");
}

int ember_hip_sample(const EmberSampleArgs *a, void *stream) {
    g_last_error.clear();
    if (!a) return set_error(EMBER_ERR_INVALID, "sample: null arguments");
    if (a->R < 0 || a->vocab < 1 || a->vocab > (1 << 24))
        return set_error(EMBER_ERR_INVALID, "sample: bad sizes (R %d, vocab %d: 1..2^24)", a->R, a->vocab);
    if (a->R == 0) return EMBER_OK;
    if (!a->logits || !a->params || !a->out) return set_error(EMBER_ERR_INVALID, "sample: a required pointer is null");
    return hip_status(launch_sample(*a, static_cast<hipStream_t>(stream)), "sample");
}

int ember_hip_token_probs(const EmberProbArgs *a, void *stream) {
    g_last_error.clear();
    if (!a) return set_error(EMBER_ERR_INVALID, "token_probs: null arguments");
    if (a->n < 0 || a->R < 0 || a->vocab < 1 || a->vocab > (1 << 24))
        return set_error(EMBER_ERR_INVALID, "token_probs: bad sizes (n %d, R %d, vocab %d: 1..2^24)", a->n, a->R,
                         a->vocab);
    if (a->n == 0) return EMBER_OK;
    if (!a->logits || !a->params || !a->rows || !a->tokens || !a->out)
        return set_error(EMBER_ERR_INVALID, "token_probs: a required pointer is null");
    return hip_status(launch_token_probs(*a, static_cast<hipStream_t>(stream)), "token_probs");
}

int ember_hip_rmsnorm_rows(const EmberNormArgs *a, void *stream) {
    g_last_error.clear();
    if (!a) return set_error(EMBER_ERR_INVALID, "rmsnorm_rows: null arguments");
    if (a->R < 0 || a->hidden < 1) return set_error(EMBER_ERR_INVALID, "rmsnorm_rows: bad sizes");
    if (a->R == 0) return EMBER_OK;
    if (!a->x || !a->w || !a->out) return set_error(EMBER_ERR_INVALID, "rmsnorm_rows: a required pointer is null");
    return hip_status(launch_rmsnorm_rows(*a, static_cast<hipStream_t>(stream)), "rmsnorm_rows");
}

}  // extern "C"
