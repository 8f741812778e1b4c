// C ABI of the host-side pieces (include/ember_hip.h, parts 2 and 3): the
// block manager and the paged-KV path behind opaque handles. C++ exceptions
// (ember::Error, allocation failures) stop here and become return codes.
#include <algorithm>
#include <cstring>
#include <exception>
#include <memory>
#include <new>
#include <span>
#include <vector>

#include "backend/backend.hpp"
#include "backend/hip_paged_kv.hpp"
#include "capi_errors.hpp"

namespace ember {
int64_t hip_backend_graph_replays();  // hip_backend.cpp
int64_t hip_backend_graph_captures();  // hip_backend.cpp
}
#include "common/error.hpp"
#include "ember_hip.h"
#include "kvcache/block_manager.hpp"

struct EmberBlockManager {
    ember::BlockManager bm;
    EmberBlockManager(int n, bool caching) : bm(n, caching) {}
};

struct EmberPagedKv {
    ember::HipPagedKv kv;
    EmberPagedKv(const ember::ModelConfig &c, const ember::PagedKvOptions &o, hipStream_t s) : kv(c, o, s) {}
};

struct EmberBackend {
    std::unique_ptr<ember::Backend> be;
};

using ember::hip::set_error;

namespace {

template <class F>
int32_t guarded(const char *who, F &&f) {
    try {
        return f();
    } catch (const std::exception &e) {
        return set_error(EMBER_ERR_INVALID, "%s: %s", who, e.what());
    } catch (...) {
        return set_error(EMBER_ERR_INVALID, "%s: unknown failure", who);
    }
}

}  // namespace

extern "C" {

// ---- block manager ----

EmberBlockManager *ember_bm_create(int32_t num_blocks, int32_t prefix_caching) {
    try {
        return new EmberBlockManager(num_blocks, prefix_caching != 0);
    } catch (const std::exception &e) {
        set_error(EMBER_ERR_INVALID, "bm_create: %s", e.what());
        return nullptr;
    }
}

void ember_bm_destroy(EmberBlockManager *h) { delete h; }
int32_t ember_bm_num_blocks(const EmberBlockManager *h) { return h->bm.num_blocks(); }
int32_t ember_bm_available(const EmberBlockManager *h) { return h->bm.available(); }
int32_t ember_bm_used(const EmberBlockManager *h) { return h->bm.used(); }
int32_t ember_bm_cached(const EmberBlockManager *h) { return h->bm.cached(); }
int32_t ember_bm_allocate(EmberBlockManager *h) { return h->bm.allocate(); }

int32_t ember_bm_release(EmberBlockManager *h, int32_t block) {
    return guarded("bm_release", [&] {
        h->bm.release(block);
        return EMBER_OK;
    });
}

int32_t ember_bm_release_all(EmberBlockManager *h, const int32_t *blocks, int32_t n) {
    return guarded("bm_release_all", [&] {
        h->bm.release_all(std::span<const int>(blocks, static_cast<size_t>(n < 0 ? 0 : n)));
        return EMBER_OK;
    });
}

uint64_t ember_bm_block_hash(uint64_t parent, const int32_t *tokens, int32_t n) {
    return ember::BlockManager::block_hash(parent, std::span<const int32_t>(tokens, static_cast<size_t>(n < 0 ? 0 : n)));
}

int32_t ember_bm_match_prefix(EmberBlockManager *h, const int32_t *tokens, int32_t n, int32_t *out_blocks) {
    return guarded("bm_match_prefix", [&] {
        const auto got = h->bm.match_prefix(std::span<const int32_t>(tokens, static_cast<size_t>(n < 0 ? 0 : n)));
        for (size_t i = 0; i < got.size(); i++) out_blocks[i] = got[i];
        return static_cast<int32_t>(got.size());
    });
}

uint64_t ember_bm_seal(EmberBlockManager *h, int32_t block, uint64_t parent, const int32_t *tokens, int32_t n) {
    try {
        return h->bm.seal(block, parent, std::span<const int32_t>(tokens, static_cast<size_t>(n < 0 ? 0 : n)));
    } catch (const std::exception &e) {
        set_error(EMBER_ERR_INVALID, "bm_seal: %s", e.what());
        return 0;
    }
}

int32_t ember_bm_prefix_caching(const EmberBlockManager *h) { return h->bm.prefix_caching() ? 1 : 0; }

int32_t ember_bm_refcount(const EmberBlockManager *h, int32_t block) {
    if (block < 0 || block >= h->bm.num_blocks()) return set_error(EMBER_ERR_INVALID, "bm_refcount: block %d of %d", block, h->bm.num_blocks());
    return h->bm.refcount(block);
}

uint64_t ember_bm_hit_tokens(const EmberBlockManager *h) { return h->bm.hit_tokens(); }
uint64_t ember_bm_lookup_tokens(const EmberBlockManager *h) { return h->bm.lookup_tokens(); }

int32_t ember_bm_check(const EmberBlockManager *h, char *buf, int32_t buflen) {
    const std::string problem = h->bm.check();
    if (buf && buflen > 0) {
        const size_t n = std::min(problem.size(), static_cast<size_t>(buflen - 1));
        std::memcpy(buf, problem.data(), n);
        buf[n] = 0;
    }
    return problem.empty() ? 0 : 1;
}

void ember_bm_states(const EmberBlockManager *h, uint8_t *out) {
    const auto s = h->bm.states();
    std::memcpy(out, s.data(), s.size());
}

int32_t ember_bm_share(EmberBlockManager *h, const int32_t *blocks, int32_t n) {
    return guarded("bm_share", [&] {
        h->bm.share(std::span<const int>(blocks, static_cast<size_t>(n < 0 ? 0 : n)));
        return EMBER_OK;
    });
}

int32_t ember_bm_copy_on_write(EmberBlockManager *h, int32_t block) {
    try {
        return static_cast<int32_t>(h->bm.copy_on_write(block));
    } catch (const std::exception &e) {
        set_error(EMBER_ERR_INVALID, "bm_copy_on_write: %s", e.what());
        return -2;  // -1 means "no block available"
    }
}

// ---- the paged-KV path ----

EmberPagedKv *ember_kv_create(const EmberKvConfig *cfg, void *stream) {
    if (!cfg) {
        set_error(EMBER_ERR_INVALID, "kv_create: null config");
        return nullptr;
    }
    try {
        ember::ModelConfig c;
        c.arch = "qwen3";
        c.n_layers = cfg->n_layers;
        c.n_heads = cfg->n_heads;
        c.n_kv_heads = cfg->n_kv_heads;
        c.head_dim = cfg->head_dim;
        c.rms_eps = cfg->rms_eps;
        c.rope_theta = cfg->rope_theta;
        c.max_position = cfg->max_position;
        c.qk_norm = cfg->qk_norm != 0;
        ember::PagedKvOptions o;
        o.num_blocks = cfg->num_blocks;
        o.max_batch_tokens = cfg->max_batch_tokens;
        o.max_seqs = cfg->max_seqs;
        o.dtype = cfg->dtype;
        o.split_len = cfg->split_len;
        return new EmberPagedKv(c, o, static_cast<hipStream_t>(stream));
    } catch (const std::exception &e) {
        set_error(EMBER_ERR_INVALID, "kv_create: %s", e.what());
        return nullptr;
    }
}

void ember_kv_destroy(EmberPagedKv *h) { delete h; }

static ember::StepBatch step_batch(const EmberStepBatch *b) {
    EMBER_CHECK(b && b->num_tokens > 0 && b->num_seqs > 0 && b->max_blocks > 0, "empty or malformed batch");
    ember::StepBatch sb;
    const size_t T = static_cast<size_t>(b->num_tokens), S = static_cast<size_t>(b->num_seqs);
    sb.tokens.assign(b->tokens, b->tokens + T);
    sb.positions.assign(b->positions, b->positions + T);
    sb.query_start.assign(b->query_start, b->query_start + S + 1);
    sb.context_len.assign(b->context_len, b->context_len + S);
    sb.max_blocks = b->max_blocks;
    sb.block_tables.assign(b->block_tables, b->block_tables + S * static_cast<size_t>(b->max_blocks));
    return sb;
}

int32_t ember_kv_plan(EmberPagedKv *h, const EmberStepBatch *b) {
    return guarded("kv_plan", [&] {
        h->kv.plan(step_batch(b));
        return EMBER_OK;
    });
}

int32_t ember_kv_decode_graph(EmberPagedKv *h, const EmberStepBatch *b, const EmberLayerIo *layers, int32_t n_layers) {
    return guarded("kv_decode_graph", [&] {
        EMBER_CHECK(layers && n_layers > 0, "no layer buffers");
        std::vector<ember::HipPagedKv::LayerIo> io(static_cast<size_t>(n_layers));
        for (int l = 0; l < n_layers; l++) {
            const EmberLayerIo &x = layers[l];
            EMBER_CHECK(x.qkv && x.out, "layer {}: null qkv or out", l);
            io[static_cast<size_t>(l)] = {x.qkv, x.q_norm, x.k_norm, x.bias, x.out};
        }
        return h->kv.decode_graph(step_batch(b), io) ? EMBER_OK : 1;
    });
}

int64_t ember_kv_graph_captures(const EmberPagedKv *h) { return h ? h->kv.graph_captures() : -1; }

int32_t ember_kv_layer(EmberPagedKv *h, int32_t layer, const void *qkv, const float *q_norm, const float *k_norm,
                       const float *bias, void *out) {
    return guarded("kv_layer", [&] {
        h->kv.layer(layer, qkv, q_norm, k_norm, bias, out);
        return EMBER_OK;
    });
}

int32_t ember_kv_copy_blocks(EmberPagedKv *h, const int32_t *src, const int32_t *dst, int32_t n) {
    return guarded("kv_copy_blocks", [&] {
        const size_t m = static_cast<size_t>(n < 0 ? 0 : n);
        h->kv.copy_blocks(std::span<const int32_t>(src, m), std::span<const int32_t>(dst, m));
        return EMBER_OK;
    });
}

void *ember_kv_k_pool(EmberPagedKv *h, int32_t layer) {
    try {
        return h->kv.k_pool(layer);
    } catch (const std::exception &e) {
        set_error(EMBER_ERR_INVALID, "kv_k_pool: %s", e.what());
        return nullptr;
    }
}

void *ember_kv_v_pool(EmberPagedKv *h, int32_t layer) {
    try {
        return h->kv.v_pool(layer);
    } catch (const std::exception &e) {
        set_error(EMBER_ERR_INVALID, "kv_v_pool: %s", e.what());
        return nullptr;
    }
}

int64_t ember_kv_layer_stride(const EmberPagedKv *h) { return h->kv.layer_stride(); }
int32_t ember_kv_spare_block(const EmberPagedKv *h) { return h->kv.spare_block(); }

int32_t ember_kv_plan_info(const EmberPagedKv *h, int32_t *decode_runs, int32_t *prefill_tiles, int32_t *num_splits,
                           int32_t *fused) {
    if (decode_runs) *decode_runs = h->kv.decode_runs();
    if (prefill_tiles) *prefill_tiles = h->kv.prefill_tiles();
    if (num_splits) *num_splits = h->kv.num_splits();
    if (fused) *fused = h->kv.fused() ? 1 : 0;
    return EMBER_OK;
}

int32_t ember_kv_set_timing(EmberPagedKv *h, int32_t on) {
    h->kv.set_timing(on != 0);
    return EMBER_OK;
}

int32_t ember_kv_timing(EmberPagedKv *h, int32_t *launches, double *total_ms) {
    return guarded("kv_timing", [&] {
        const int n = h->kv.collect_timing(total_ms);
        if (launches) *launches = n;
        return EMBER_OK;
    });
}

int32_t ember_kv_prefill_timing(EmberPagedKv *h, int32_t *launches, double *total_ms) {
    return guarded("kv_prefill_timing", [&] {
        const int n = h->kv.collect_prefill_timing(total_ms);
        if (launches) *launches = n;
        return EMBER_OK;
    });
}

// ---- the backend ----

EmberBackend *ember_backend_create(const char *model_dir, const EmberBackendOptions *o) {
    try {
        EMBER_CHECK(model_dir && o, "backend_create: null arguments");
        ember::BackendOptions opt;
        opt.device = "hip";
        opt.max_batch_tokens = o->max_batch_tokens;
        opt.max_seqs = o->max_seqs;
        opt.max_logit_rows = o->max_logit_rows;
        opt.kv_cache_bytes = o->kv_cache_bytes;
        opt.kv_cache_tokens = o->kv_cache_tokens;
        if (o->memory_fraction > 0.0) opt.memory_fraction = o->memory_fraction;
        opt.gpu = o->gpu;
        if (o->graphs != 0) opt.cuda_graphs = o->graphs > 0;
        return new EmberBackend{ember::create_backend(model_dir, opt)};
    } catch (const std::exception &e) {
        set_error(EMBER_ERR_INVALID, "backend_create: %s", e.what());
        return nullptr;
    }
}

void ember_backend_destroy(EmberBackend *h) { delete h; }

int64_t ember_backend_graph_replays(void) { return ember::hip_backend_graph_replays(); }
int64_t ember_backend_graph_captures(void) { return ember::hip_backend_graph_captures(); }

int32_t ember_backend_info(const EmberBackend *h, EmberModelInfo *out) {
    return guarded("backend_info", [&] {
        EMBER_CHECK(h && out, "null arguments");
        const ember::ModelConfig &c = h->be->config();
        *out = EmberModelInfo{c.vocab_size, c.hidden, c.intermediate, c.n_layers, c.n_heads, c.n_kv_heads,
                              c.head_dim, h->be->num_kv_blocks(), h->be->options().max_logit_rows};
        return EMBER_OK;
    });
}

int32_t ember_backend_forward(EmberBackend *h, const EmberStepBatch *b, const int32_t *logit_rows, int32_t n_rows) {
    return guarded("backend_forward", [&] {
        EMBER_CHECK(h && n_rows >= 0 && (n_rows == 0 || logit_rows), "null arguments");
        ember::StepBatch sb = step_batch(b);
        sb.logit_rows.assign(logit_rows, logit_rows + n_rows);
        h->be->forward(sb);
        return EMBER_OK;
    });
}

static std::vector<ember::SampleRequest> sample_requests(const EmberSampleParams *p, int32_t n) {
    EMBER_CHECK(n >= 0 && (n == 0 || p), "null sampling parameters");
    std::vector<ember::SampleRequest> reqs(static_cast<size_t>(n));
    for (int32_t i = 0; i < n; i++) {
        ember::SamplingParams &s = reqs[static_cast<size_t>(i)].params;
        s.temperature = p[i].temperature;
        s.top_p = p[i].top_p;
        s.min_p = p[i].min_p;
        s.top_k = p[i].top_k;
        s.seed = p[i].seed;
        reqs[static_cast<size_t>(i)].counter = p[i].counter;
    }
    return reqs;
}

int32_t ember_backend_sample(EmberBackend *h, const EmberSampleParams *params, int32_t n, int32_t *out) {
    return guarded("backend_sample", [&] {
        EMBER_CHECK(h && (n == 0 || out), "null arguments");
        const auto reqs = sample_requests(params, n);
        h->be->sample(reqs, std::span<int32_t>(out, static_cast<size_t>(n)));
        return EMBER_OK;
    });
}

int32_t ember_backend_token_probs(EmberBackend *h, const EmberSampleParams *params, int32_t n_params,
                                  const int32_t *rows, const int32_t *tokens, int32_t n, float *out) {
    return guarded("backend_token_probs", [&] {
        EMBER_CHECK(h && n >= 0 && (n == 0 || (rows && tokens && out)), "null arguments");
        const auto reqs = sample_requests(params, n_params);
        const size_t m = static_cast<size_t>(n);
        h->be->token_probs(reqs, std::span<const int32_t>(rows, m), std::span<const int32_t>(tokens, m),
                           std::span<float>(out, m));
        return EMBER_OK;
    });
}

int32_t ember_backend_logits(EmberBackend *h, int32_t row, float *out, int32_t n) {
    return guarded("backend_logits", [&] {
        EMBER_CHECK(h && out && n > 0, "null arguments");
        h->be->logits(row, std::span<float>(out, static_cast<size_t>(n)));
        return EMBER_OK;
    });
}

int32_t ember_backend_set_capture_hidden(EmberBackend *h, int32_t on) {
    return guarded("backend_set_capture_hidden", [&] {
        EMBER_CHECK(h, "null backend");
        h->be->set_capture_hidden(on != 0);
        return EMBER_OK;
    });
}

int32_t ember_backend_captured_hidden(EmberBackend *h, float *out, int32_t n) {
    return guarded("backend_captured_hidden", [&] {
        EMBER_CHECK(h && out, "null arguments");
        const std::vector<float> v = h->be->captured_hidden();
        EMBER_CHECK(static_cast<size_t>(n) >= v.size(), "captured_hidden: {} floats needed", v.size());
        std::copy(v.begin(), v.end(), out);
        return static_cast<int32_t>(v.size());
    });
}

}  // extern "C"
