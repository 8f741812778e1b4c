// The paged-KV hot path of a HIP backend: what the reference's CudaBackend
// does around its attention kernels (src/backend/cuda/cuda_backend.cu:134-205
// forward: packing, routing, splits, one upload; :288-374 enqueue: the
// per-layer append + attention; :757-780 the KV pool), on MI355X.
//
// Pools: K and V separately, each [layer][block][kv_head][slot][head_dim]
// with num_blocks + 1 blocks per layer; the last one is a spare block the
// engine never hands out (padding rows of captured decode steps write there).
// Pools are zeroed at creation, so slots never written read as 0.
//
// Routing: a sequence with >= 16 new tokens goes to 64-token MFMA prefill
// tiles (f16 pools: the MFMA path); every other run, and every run of an f32
// pool, is cut into runs of at most min(8, 16 / G) tokens for the paged decode
// kernel, which reads each page once per run for its G x run query rows. Decode splits are fixed 512-key chunks ([0, 512), [512, 1024), ...)
// at every batch size, so a token's result never depends on its batch.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <map>
#include <span>
#include <vector>

#include "backend/backend.hpp"
#include "ember_hip.h"

namespace ember {

struct PagedKvOptions {
    int num_blocks = 0;         // blocks the engine may hand out
    int max_batch_tokens = 2048;
    int max_seqs = 64;
    int dtype = EMBER_DTYPE_F16;
    int split_len = 512;
    bool use_prefill_kernel = true;   // route runs of >= 16 tokens to MFMA tiles (f16 pools; f32 always decodes)
};

class HipPagedKv {
public:
    static constexpr int kFlashMinTokens = 16;  // a run this long uses prefill tiles (cuda_backend.cu:257)
    static constexpr int kMaxDecodeRows = 16;   // query rows (G heads x run tokens) of the widest decode instance

    HipPagedKv(const ModelConfig &cfg, const PagedKvOptions &opt, hipStream_t stream);
    ~HipPagedKv();
    HipPagedKv(const HipPagedKv &) = delete;
    HipPagedKv &operator=(const HipPagedKv &) = delete;

    // Packs and uploads the step's integers and decides the launches.
    void plan(const StepBatch &b) { plan(b, 0); }
    // Layer `layer` of the planned step: K/V of every new token into the
    // pools, then attention of every token into out [T, n_heads, head_dim].
    void layer(int layer, const void *qkv, const float *q_norm, const float *k_norm, const float *bias, void *out);
    // Per-layer buffers of a captured decode step.
    struct LayerIo {
        const void *qkv;
        const float *q_norm, *k_norm, *bias;
        void *out;
    };
    static constexpr int kGraphMaxTokens = 64;
    static constexpr int kDescInts = 16;  // ints per work descriptor (EmberAttnArgs::work_desc)
    static constexpr int kDecodeWgPerCu = 4;  // decode work-groups a CU holds at once (f16, up to 10 rows)
    // A pure decode step (every sequence one new token, at most 64) as one
    // replayed hipGraph of all layers' launches (cuda_backend.cu:376-454): the
    // step is padded to a token bucket and a block-table width bucket, padding
    // tokens are sequences of length 1 at position 0 on the spare block, and the
    // splits follow the width bucket, so a replay always matches its capture.
    // qkv and out of every layer must hold token_bucket(T) rows (64 suffice);
    // rows past T are padding. Graphs are kept per bucket pair and captured
    // again when the layer buffers change. Returns false, with nothing
    // enqueued, when the step is not a pure decode step of <= 64 tokens.
    bool decode_graph(const StepBatch &b, std::span<const LayerIo> io);
    // The planning half of decode_graph, for a caller that captures more than
    // the attention layers (a backend's whole model step): the token bucket
    // the step pads to, or 0 when it is not a pure decode step of <= 64 tokens.
    int graph_bucket(const StepBatch &b) const;
    // Validates, pads and plans the step as decode_graph does; returns its
    // token bucket (the planned step's tokens, rows past T padding), or 0 with
    // nothing planned. graph_key() then names the planned layout: layer()
    // launches of two plans with the same key take the same arguments, so one
    // captured graph replays either.
    int plan_graph(const StepBatch &b);
    uint64_t graph_key() const;
    // Graphs decode_graph has captured (and instantiated) so far; a launch of a
    // kept graph does not count.
    int64_t graph_captures() const { return graph_captures_; }
    static int token_bucket(int T);
    int width_bucket(int w) const;

    // Device copies of whole pages, src[i] -> dst[i], all layers, K and V.
    void copy_blocks(std::span<const int32_t> src, std::span<const int32_t> dst);

    void *k_pool(int layer) const;
    void *v_pool(int layer) const;
    int64_t layer_stride() const { return layer_elems_; }
    int spare_block() const { return opt_.num_blocks; }
    int decode_runs() const { return decode_runs_; }
    bool fused() const { return fused_; }
    int prefill_tiles() const { return tiles_; }
    int num_splits() const { return splits_; }
    hipStream_t stream() const { return stream_; }
    // The planned step's token ids (null when the batch carried none) and
    // logit rows on the device, uploaded with the rest of the plan.
    const int32_t *d_tokens() const { return d_tokens_; }
    const int32_t *d_logit_rows() const { return d_logit_rows_; }
    const int32_t *d_positions() const { return d_positions_; }

    // Benchmark timing of the paged-decode and prefill kernels (events around each launch).
    void set_timing(bool on) { timing_ = on; }
    // Waits for the recorded paged-decode launches; returns their count and total ms, then starts over.
    int collect_timing(double *total_ms);
    // The same for the prefill-tile launches.
    int collect_prefill_timing(double *total_ms);

private:
    // graph_splits > 0: a graph step's plan, with num_splits fixed to it and the
    // work list padded to T * graph_splits items (padding items do nothing), so
    // every array has the same size for the same buckets.
    void plan(const StepBatch &b, int graph_splits);

    struct GraphEntry {
        hipGraphExec_t exec = nullptr;
        std::vector<LayerIo> io;
    };
    std::map<uint64_t, GraphEntry> graphs_;
    hipStream_t capture_stream_ = nullptr;  // graphs are captured here (the path's stream may be the null stream)

    ModelConfig cfg_;
    PagedKvOptions opt_;
    hipStream_t stream_;
    size_t elem_ = 2;
    int64_t layer_elems_ = 0;       // elements of one layer's K (or V) pool
    int max_blocks_per_seq_ = 0;
    int max_splits_ = 0;
    int decode_cap_ = 0;            // decode tokens a step can hold (the split scratch is sized for it)

    void *k_ = nullptr, *v_ = nullptr, *q_ = nullptr;
    float *inv_freq_ = nullptr, *part_acc_ = nullptr, *part_ml_ = nullptr;
    uint32_t *merge_counters_ = nullptr;  // [max_batch_tokens * n_kv], zero between launches
    // A step's integers in a ring of kStages buffers: plan() packs them into
    // pinned staging and copies them up on upload_stream_, so the copy overlaps
    // earlier steps' kernels instead of sitting between the steps on stream_. A
    // buffer is reused kStages plans later, so the host can run kStages - 1
    // steps ahead of the GPU. Every kMarkEvery-th plan records a mark on
    // stream_ (all kernels of the earlier plans); an upload waits for the first
    // mark recorded after its buffer's previous plan.
    static constexpr int kStages = 8, kMarkEvery = 4, kMarks = 4;
    static_assert(kStages >= kMarkEvery && kMarks * kMarkEvery > kStages, "a mark must cover each reuse");
    int32_t *dev_ints_[kStages] = {};
    int32_t *host_ints_[kStages] = {};  // pinned staging, one per dev_ints_ buffer
    hipEvent_t staged_[kStages] = {};   // the upload into each buffer has run
    hipEvent_t consumed_[kMarks] = {};  // the marks, a ring: plan m's mark in (m / kMarkEvery) % kMarks
    hipStream_t upload_stream_ = nullptr;
    int stage_ = 0;
    int64_t plans_ = 0;
    int graph_tb_ = 0, graph_wb_ = 0;  // the last plan_graph's buckets
    // A graph plan's kernels read their integers from this one block, not from
    // the staging ring: the plan copies its stage here on stream_ (so after
    // every earlier graph launch has read it), and one graph per bucket pair
    // replays whatever stage the ring gave the step.
    int32_t *graph_ints_ = nullptr;
    int64_t graph_captures_ = 0;
    // copy_blocks' pair lists, double-buffered: pinned staging, the device list
    // the copy kernel reads, and an event recorded after that kernel.
    static constexpr int kCowPairs = 4096;
    int32_t *cow_host_[2] = {nullptr, nullptr};
    int32_t *cow_dev_[2] = {nullptr, nullptr};
    hipEvent_t cow_done_[2] = {nullptr, nullptr};
    int cow_stage_ = 0;
    size_t ints_capacity_ = 0;

    // The current plan (device addresses into dev_ints_[stage_]).
    int T_ = 0, decode_count_ = 0, decode_runs_ = 0, max_run_ = 1, tiles_ = 0, splits_ = 1, max_blocks_ = 0;
    int prefill_hg_ = 0;   // EmberPrefillArgs::heads_per_group of the planned step
    int cu_count_ = 256;   // the device's CUs (the constructor asks)
    bool fused_ = false;  // every sequence's new tokens form one run: append + attention in one launch
    const int32_t *d_positions_ = nullptr, *d_token_seq_ = nullptr, *d_tables_ = nullptr, *d_decode_ = nullptr,
                  *d_run_first_ = nullptr, *d_run_count_ = nullptr, *d_tile_start_ = nullptr, *d_tile_end_ = nullptr,
                  *d_tile_seq_ = nullptr, *d_work_ = nullptr, *d_work_desc_ = nullptr;
    std::vector<int32_t> token_seq_, decode_, run_first_, run_count_, run_ctx_, tile_start_, tile_end_, tile_seq_, work_,
        work_desc_;
    int num_work_ = 0;
    const int32_t *d_tokens_ = nullptr, *d_logit_rows_ = nullptr;

    bool timing_ = false;
    struct Timing {  // start/stop pairs, reused after collection
        std::vector<hipEvent_t> events;
        size_t used = 0;
        void next(hipEvent_t *start, hipEvent_t *stop);
        int collect(double *total_ms);
    };
    Timing decode_timing_, prefill_timing_;
};

}  // namespace ember
