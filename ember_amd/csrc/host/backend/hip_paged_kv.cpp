// The paged-KV path's host side: pool allocation, the step plan and the
// per-layer launches through the C ABI.
#include "backend/hip_paged_kv.hpp"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <functional>
#include <queue>
#include <utility>

#include "common/error.hpp"
#include "kernels.hpp"

#define EMBER_HIP_CHECK(expr)                                                                       \
    do {                                                                                            \
        hipError_t err_ = (expr);                                                                   \
        if (err_ != hipSuccess) ::ember::fail("{} failed: {}", #expr, hipGetErrorString(err_));       \
    } while (0)

namespace ember {

namespace {

void check_abi(int code, const char *what) {
    if (code != EMBER_OK) fail("{}: {}", what, ember_hip_last_error());
}

template <class T>
T *device_alloc(size_t count) {
    void *p = nullptr;
    EMBER_HIP_CHECK(hipMalloc(&p, std::max<size_t>(count, 1) * sizeof(T)));
    return static_cast<T *>(p);
}

size_t pad32(size_t n) { return (n + 31) & ~size_t(31); }

}  // namespace

HipPagedKv::HipPagedKv(const ModelConfig &cfg, const PagedKvOptions &opt, hipStream_t stream)
    : cfg_(cfg), opt_(opt), stream_(stream) {
    EMBER_CHECK(cfg_.head_dim == 128, "the paged-KV path needs head_dim 128 (got {})", cfg_.head_dim);
    EMBER_CHECK(cfg_.n_layers > 0 && cfg_.n_kv_heads > 0 && cfg_.n_heads % cfg_.n_kv_heads == 0 &&
                    cfg_.group() >= 1 && cfg_.group() <= 8,
                "unsupported head layout: {} query heads over {} kv heads", cfg_.n_heads, cfg_.n_kv_heads);
    EMBER_CHECK(opt_.num_blocks > 0, "the KV cache has no blocks");
    EMBER_CHECK(opt_.dtype == EMBER_DTYPE_F16 || opt_.dtype == EMBER_DTYPE_F32, "unknown dtype {}", opt_.dtype);
    if (opt_.split_len <= 0) opt_.split_len = 512;
    {
        int dev = 0, cus = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cus > 0)
            cu_count_ = cus;
    }
    EMBER_CHECK(opt_.split_len % kBlockSize == 0 && opt_.split_len <= EMBER_MAX_SPLIT_LEN,
                "split_len {} is not a multiple of {} up to {}", opt_.split_len, kBlockSize, EMBER_MAX_SPLIT_LEN);
    EMBER_CHECK(opt_.max_batch_tokens > 0 && opt_.max_seqs > 0, "bad batch limits");
    EMBER_CHECK(cfg_.max_position > 0, "max_position must be set");
    elem_ = opt_.dtype == EMBER_DTYPE_F16 ? 2 : 4;

    const int64_t block_elems = static_cast<int64_t>(cfg_.n_kv_heads) * kBlockSize * cfg_.head_dim;
    layer_elems_ = block_elems * (opt_.num_blocks + 1);  // + the spare block
    const size_t pool_bytes = static_cast<size_t>(layer_elems_) * cfg_.n_layers * elem_;
    EMBER_HIP_CHECK(hipMalloc(&k_, pool_bytes));
    EMBER_HIP_CHECK(hipMalloc(&v_, pool_bytes));
    EMBER_HIP_CHECK(hipMemsetAsync(k_, 0, pool_bytes, stream_));  // unwritten slots read as 0
    EMBER_HIP_CHECK(hipMemsetAsync(v_, 0, pool_bytes, stream_));

    const size_t T = static_cast<size_t>(opt_.max_batch_tokens);
    EMBER_HIP_CHECK(hipMalloc(&q_, T * cfg_.n_heads * cfg_.head_dim * elem_));
    max_blocks_per_seq_ = (cfg_.max_position + kBlockSize - 1) / kBlockSize;
    max_splits_ = (max_blocks_per_seq_ * kBlockSize + opt_.split_len - 1) / opt_.split_len;
    // Split scratch serves decode tokens only. With f16 pools a sequence's run of 16 or more new tokens
    // goes to prefill tiles, so at most 15 tokens per sequence are decode tokens.
    decode_cap_ = static_cast<int>(opt_.dtype == EMBER_DTYPE_F16 && opt_.use_prefill_kernel
                                       ? std::min<size_t>(T, static_cast<size_t>(kFlashMinTokens - 1) * opt_.max_seqs)
                                       : T);
    const size_t part_rows = static_cast<size_t>(decode_cap_) * cfg_.n_heads * static_cast<size_t>(max_splits_);
    part_acc_ = device_alloc<float>(part_rows * cfg_.head_dim);
    part_ml_ = device_alloc<float>(part_rows * 2);
    const size_t counters = static_cast<size_t>(decode_cap_) * cfg_.n_kv_heads;  // per (run, kv head); runs <= tokens
    merge_counters_ = device_alloc<uint32_t>(counters);
    EMBER_HIP_CHECK(hipMemsetAsync(merge_counters_, 0, counters * sizeof(uint32_t), stream_));

    std::vector<float> inv(static_cast<size_t>(cfg_.head_dim / 2));
    for (int i = 0; i < cfg_.head_dim / 2; i++)  // f32, as the reference computes it (cpu_backend.cpp:85-88)
        inv[static_cast<size_t>(i)] = 1.0f / std::pow(static_cast<float>(cfg_.rope_theta),
                                                      static_cast<float>(2 * i) / static_cast<float>(cfg_.head_dim));
    inv_freq_ = device_alloc<float>(inv.size());
    EMBER_HIP_CHECK(hipMemcpyAsync(inv_freq_, inv.data(), inv.size() * sizeof(float), hipMemcpyHostToDevice, stream_));

    // Step integers: positions, token_seq, decode list, runs (2), tiles (3), tables, work items and their
    // descriptors (kDescInts each, 128-byte aligned like every array here). Work items exist for decode
    // runs only, at most one per (decode token, split).
    const size_t items = static_cast<size_t>(decode_cap_) * max_splits_;
    ints_capacity_ = 4 * pad32(T) + 4 * pad32(T) + 3 * pad32(T / 16 + static_cast<size_t>(opt_.max_seqs)) +
                     static_cast<size_t>(opt_.max_seqs) * max_blocks_per_seq_ + pad32(2 * items) +
                     pad32(static_cast<size_t>(kDescInts) * items) + 64;
    for (int i = 0; i < kStages; i++) {
        dev_ints_[i] = device_alloc<int32_t>(ints_capacity_);
        EMBER_HIP_CHECK(hipHostMalloc(reinterpret_cast<void **>(&host_ints_[i]), ints_capacity_ * sizeof(int32_t), 0));
        EMBER_HIP_CHECK(hipEventCreateWithFlags(&staged_[i], hipEventDisableTiming));
    }
    graph_ints_ = device_alloc<int32_t>(ints_capacity_);
    for (int i = 0; i < kMarks; i++) EMBER_HIP_CHECK(hipEventCreateWithFlags(&consumed_[i], hipEventDisableTiming));
    EMBER_HIP_CHECK(hipStreamCreateWithFlags(&upload_stream_, hipStreamNonBlocking));  // default priority
    for (int i = 0; i < 2; i++) {  // copy-on-write pair lists: kCowPairs (src, dst) pairs per buffer
        cow_dev_[i] = device_alloc<int32_t>(2 * static_cast<size_t>(kCowPairs));
        EMBER_HIP_CHECK(hipHostMalloc(reinterpret_cast<void **>(&cow_host_[i]), 2 * kCowPairs * sizeof(int32_t), 0));
        EMBER_HIP_CHECK(hipEventCreateWithFlags(&cow_done_[i], hipEventDisableTiming));
    }
    // every event starts out recorded, so the first plans wait on nothing pending
    for (int i = 0; i < kStages; i++) EMBER_HIP_CHECK(hipEventRecord(staged_[i], stream_));
    for (int i = 0; i < kMarks; i++) EMBER_HIP_CHECK(hipEventRecord(consumed_[i], stream_));
    for (int i = 0; i < 2; i++) EMBER_HIP_CHECK(hipEventRecord(cow_done_[i], stream_));
    EMBER_HIP_CHECK(hipStreamSynchronize(stream_));
}

HipPagedKv::~HipPagedKv() {
    (void)hipStreamSynchronize(stream_);
    for (auto &[key, g] : graphs_) (void)hipGraphExecDestroy(g.exec);
    if (capture_stream_) (void)hipStreamDestroy(capture_stream_);
    if (upload_stream_) {
        (void)hipStreamSynchronize(upload_stream_);
        (void)hipStreamDestroy(upload_stream_);
    }
    for (const Timing *t : {&decode_timing_, &prefill_timing_})
        for (hipEvent_t e : t->events) (void)hipEventDestroy(e);
    for (int i = 0; i < kStages; i++) {
        if (staged_[i]) (void)hipEventDestroy(staged_[i]);
        if (i < kMarks && consumed_[i]) (void)hipEventDestroy(consumed_[i]);
        if (host_ints_[i]) (void)hipHostFree(host_ints_[i]);
        if (dev_ints_[i]) (void)hipFree(dev_ints_[i]);
    }
    for (int i = 0; i < 2; i++) {
        if (cow_done_[i]) (void)hipEventDestroy(cow_done_[i]);
        if (cow_host_[i]) (void)hipHostFree(cow_host_[i]);
        if (cow_dev_[i]) (void)hipFree(cow_dev_[i]);
    }
    for (void *p : {k_, v_, q_, static_cast<void *>(graph_ints_), static_cast<void *>(inv_freq_), static_cast<void *>(part_acc_),
                    static_cast<void *>(part_ml_), static_cast<void *>(merge_counters_)})
        if (p) (void)hipFree(p);
}

void *HipPagedKv::k_pool(int layer) const {
    EMBER_CHECK(layer >= 0 && layer < cfg_.n_layers, "layer {} out of range", layer);
    return static_cast<char *>(k_) + static_cast<size_t>(layer) * layer_elems_ * elem_;
}

void *HipPagedKv::v_pool(int layer) const {
    EMBER_CHECK(layer >= 0 && layer < cfg_.n_layers, "layer {} out of range", layer);
    return static_cast<char *>(v_) + static_cast<size_t>(layer) * layer_elems_ * elem_;
}

void HipPagedKv::plan(const StepBatch &b, int graph_splits) {
    const int T = b.num_tokens(), S = b.num_seqs();
    EMBER_CHECK(T > 0 && T <= opt_.max_batch_tokens, "batch of {} tokens (limit {})", T, opt_.max_batch_tokens);
    EMBER_CHECK(S > 0 && S <= opt_.max_seqs, "batch of {} sequences (limit {})", S, opt_.max_seqs);
    EMBER_CHECK(static_cast<int>(b.query_start.size()) == S + 1 && b.query_start[0] == 0 && b.query_start[S] == T,
                "malformed query_start");
    EMBER_CHECK(static_cast<int>(b.positions.size()) == T, "malformed positions");
    EMBER_CHECK(b.max_blocks > 0 && b.max_blocks <= max_blocks_per_seq_ &&
                    static_cast<int64_t>(b.block_tables.size()) == static_cast<int64_t>(S) * b.max_blocks,
                "malformed block tables ({} x {}, at most {} blocks per sequence)", S, b.max_blocks, max_blocks_per_seq_);

    token_seq_.assign(static_cast<size_t>(T), 0);
    decode_.clear();
    run_first_.clear();
    run_count_.clear();
    run_ctx_.clear();
    tile_start_.clear();
    tile_end_.clear();
    tile_seq_.clear();
    int max_ctx = 0;
    max_run_ = 1;
    fused_ = true;
    // A decode work-group holds at most 16 query rows (G heads x run tokens), so
    // the run length shrinks as the group grows: 8 at G <= 2, 5 at G = 3, 4 at G = 4, 2 at G = 8.
    const int run_cap = std::max(1, std::min(EMBER_MAX_RUN, kMaxDecodeRows / cfg_.group()));
    for (int s = 0; s < S; s++) {
        const int q0 = b.query_start[static_cast<size_t>(s)], q1 = b.query_start[static_cast<size_t>(s) + 1];
        EMBER_CHECK(q0 <= q1, "malformed query_start");
        int ctx = 0;
        for (int t = q0; t < q1; t++) {
            token_seq_[static_cast<size_t>(t)] = s;
            const int pos = b.positions[static_cast<size_t>(t)];
            EMBER_CHECK(pos >= 0 && pos < b.max_blocks * kBlockSize, "token {} at position {} is beyond its block table", t,
                        pos);
            ctx = std::max(ctx, pos + 1);
            if (t > q0 && pos != b.positions[static_cast<size_t>(t) - 1] + 1) fused_ = false;
        }
        if (q1 - q0 > run_cap) fused_ = false;  // one run per sequence, or runs would read each other's new slots
        // Every page a token of this sequence reads must be a real block (or the spare).
        const int32_t *row = &b.block_tables[static_cast<size_t>(s) * b.max_blocks];
        for (int p = 0; p * kBlockSize < ctx; p++)
            EMBER_CHECK(row[p] >= 0 && row[p] <= opt_.num_blocks, "sequence {} page {} names block {} (pool of {})", s, p,
                        row[p], opt_.num_blocks);
        if (q1 - q0 >= kFlashMinTokens && opt_.use_prefill_kernel && opt_.dtype == EMBER_DTYPE_F16) {
            for (int t = q0; t < q1; t += EMBER_PREFILL_TILE) {
                tile_start_.push_back(t);
                tile_end_.push_back(std::min(q1, t + EMBER_PREFILL_TILE));
                tile_seq_.push_back(s);
            }
        } else {
            for (int t = q0; t < q1; t += run_cap) {
                const int n = std::min(run_cap, q1 - t);
                int run_ctx = 0;
                for (int i = 0; i < n; i++) run_ctx = std::max(run_ctx, b.positions[static_cast<size_t>(t + i)] + 1);
                run_first_.push_back(static_cast<int32_t>(decode_.size()));
                run_count_.push_back(n);
                run_ctx_.push_back(run_ctx);
                max_run_ = std::max(max_run_, n);
                for (int i = 0; i < n; i++) decode_.push_back(t + i);
            }
            if (q1 > q0) max_ctx = std::max(max_ctx, ctx);
        }
    }
    T_ = T;
    max_blocks_ = b.max_blocks;
    decode_count_ = static_cast<int>(decode_.size());
    EMBER_CHECK(decode_count_ <= decode_cap_, "internal: {} decode tokens exceed the split scratch ({})", decode_count_,
                decode_cap_);
    decode_runs_ = static_cast<int>(run_first_.size());
    tiles_ = static_cast<int>(tile_start_.size());
    // A launch whose tiles fit one round of work-groups at one per CU (tiles x
    // head pairs <= CUs) lasts as long as its longest tile. There each query
    // head gets its own work-group instead (twice the work-groups, two per
    // CU), and the list below pairs long tiles with short ones on a CU. A
    // row's result is the same bits with one or two heads per work-group.
    const int G = cfg_.group();
    prefill_hg_ = G % 2 == 0 && static_cast<int64_t>(tiles_) * cfg_.n_heads <= 2LL * cu_count_ ? 1 : 0;
    // Prefill tiles are dispatched longest first (keys read: the tile's last
    // position + 1; ties keep list order): a launch of several rounds of
    // work-groups, one per CU, then ends on its shortest tiles instead of on
    // whichever long tile the list happened to put last. A tile's arithmetic
    // does not depend on its place in the list.
    if (tiles_ > 1) {
        std::vector<int> order(static_cast<size_t>(tiles_));
        std::vector<int> keys(static_cast<size_t>(tiles_));
        for (int i = 0; i < tiles_; i++) {
            order[static_cast<size_t>(i)] = i;
            int k = 0;
            for (int t = tile_start_[static_cast<size_t>(i)]; t < tile_end_[static_cast<size_t>(i)]; t++)
                k = std::max(k, b.positions[static_cast<size_t>(t)] + 1);
            keys[static_cast<size_t>(i)] = k;
        }
        std::stable_sort(order.begin(), order.end(),
                         [&](int x, int y) { return keys[static_cast<size_t>(x)] > keys[static_cast<size_t>(y)]; });
        if (prefill_hg_ == 1) {
            // Work-groups b and b + CUs share a CU (b = tile x heads + head), so
            // tile i shares with tile i + CUs / heads: every other run of that
            // many tiles is reversed, pairing the longest with the shortest.
            const int per = cu_count_ / cfg_.n_heads;
            for (int g0 = per; per > 0 && g0 < tiles_; g0 += 2 * per)
                std::reverse(order.begin() + g0, order.begin() + std::min(tiles_, g0 + per));
        }
        std::vector<int32_t> start(order.size()), end(order.size()), seq(order.size());
        for (size_t i = 0; i < order.size(); i++) {
            start[i] = tile_start_[static_cast<size_t>(order[i])];
            end[i] = tile_end_[static_cast<size_t>(order[i])];
            seq[i] = tile_seq_[static_cast<size_t>(order[i])];
        }
        tile_start_.swap(start);
        tile_end_.swap(end);
        tile_seq_.swap(seq);
    }
    fused_ = fused_ && tiles_ == 0 && decode_count_ == T;
    splits_ = graph_splits > 0 ? graph_splits : std::max(1, (max_ctx + opt_.split_len - 1) / opt_.split_len);

    // Decode work items (run, split), longest first (every full split, then
    // the partial last splits), in an order that balances the keys each CU
    // reads. The launch's first kDecodeWgPerCu x CUs work-groups start at
    // once, work-group b on CU b mod CUs, so with the kv heads of an item
    // side by side, item i lands on CU group i mod groups (groups = CUs /
    // n_kv): those items are dealt to the group with the fewest keys so far,
    // longest first, and later items follow longest first. Within a group
    // the shortest item takes the first slot: a CU's earliest work-group wins
    // the memory arbitration and finishes first, so the lightest CUs free a
    // slot first and take the later items.
    work_.clear();
    {
        struct Item {
            int keys, run, split;
        };
        std::vector<Item> items, partial;
        for (int r = 0; r < decode_runs_; r++) {
            const int ctx = run_ctx_[static_cast<size_t>(r)];
            const int full = ctx / opt_.split_len;
            for (int s = 0; s < full; s++) items.push_back({opt_.split_len, r, s});
            if (ctx % opt_.split_len) partial.push_back({ctx % opt_.split_len, r, full});
        }
        std::stable_sort(partial.begin(), partial.end(), [](const Item &a, const Item &b) { return a.keys > b.keys; });
        items.insert(items.end(), partial.begin(), partial.end());
        const int n = static_cast<int>(items.size());
        const int groups = std::max(1, cu_count_ / cfg_.n_kv_heads);
        std::vector<Item> order(items);
        if (n >= groups * kDecodeWgPerCu) {
            // (keys so far, group) of the groups with a free slot, least keys
            // first, then the lowest group
            std::priority_queue<std::pair<int64_t, int>, std::vector<std::pair<int64_t, int>>, std::greater<>> open;
            for (int g = 0; g < groups; g++) open.emplace(0, g);
            std::vector<std::vector<Item>> dealt(static_cast<size_t>(groups));
            for (int i = 0; i < groups * kDecodeWgPerCu; i++) {
                const auto [load, g] = open.top();
                open.pop();
                dealt[static_cast<size_t>(g)].push_back(items[static_cast<size_t>(i)]);
                if (static_cast<int>(dealt[static_cast<size_t>(g)].size()) < kDecodeWgPerCu)
                    open.emplace(load + items[static_cast<size_t>(i)].keys, g);
            }
            for (int g = 0; g < groups; g++) {
                std::reverse(dealt[static_cast<size_t>(g)].begin(), dealt[static_cast<size_t>(g)].end());
                for (int k = 0; k < kDecodeWgPerCu; k++)
                    order[static_cast<size_t>(k * groups + g)] = dealt[static_cast<size_t>(g)][static_cast<size_t>(k)];
            }
        }
        for (const Item &it : order) {
            work_.push_back(it.run);
            work_.push_back(it.split);
        }
    }
    if (graph_splits > 0) {  // the graph's fixed-length list: padding items name no run
        EMBER_CHECK(static_cast<int>(work_.size() / 2) <= decode_runs_ * graph_splits, "internal: graph work list");
        work_.resize(2 * static_cast<size_t>(decode_runs_) * graph_splits, -1);
    }
    num_work_ = static_cast<int>(work_.size() / 2);
    // The kernel's view of each item (EmberAttnArgs::work_desc): everything it
    // would otherwise look up in a chain before its first page loads.
    work_desc_.assign(static_cast<size_t>(num_work_) * kDescInts, -1);
    for (int i = 0; i < num_work_; i++) {
        const int r = work_[2 * static_cast<size_t>(i)];
        if (r < 0) continue;  // padding: run -1
        const int split = work_[2 * static_cast<size_t>(i) + 1];
        const int first = run_first_[static_cast<size_t>(r)], count = run_count_[static_cast<size_t>(r)];
        const int t0 = decode_[static_cast<size_t>(first)];
        int lo = INT32_MAX, hi = -1;
        bool counting = true;
        for (int k = 0; k < count; k++) {
            const int t = decode_[static_cast<size_t>(first + k)];
            const int pos = b.positions[static_cast<size_t>(t)];
            lo = std::min(lo, pos);
            hi = std::max(hi, pos);
            counting = counting && t == t0 + k && pos == b.positions[static_cast<size_t>(t0)] + k;
        }
        const int seq = token_seq_[static_cast<size_t>(t0)];
        int32_t *d = &work_desc_[kDescInts * static_cast<size_t>(i)];
        d[0] = r;
        d[1] = split;
        d[2] = first;
        d[3] = count;
        d[4] = seq;
        d[5] = lo;
        d[6] = hi;
        d[7] = counting ? t0 : -1;
        const int ctx = std::min(hi + 1, b.max_blocks * kBlockSize);
        const int p0 = split * opt_.split_len / kBlockSize;
        const int p_last = (std::min(ctx, (split + 1) * opt_.split_len) - 1) / kBlockSize;
        const int32_t *row = b.block_tables.data() + static_cast<size_t>(seq) * b.max_blocks;
        for (int j = 0; j < 8 && p0 + j <= p_last; j++) d[8 + j] = row[p0 + j];
    }

    // Pack into the staging buffer (wait until its previous upload has run), then one copy.
    // Everything enqueued on stream_ so far reads earlier plans' buffers. A mark
    // on stream_ every kMarkEvery plans records that point: a mark between two
    // steps idles the GPU for about 5 us, so there is not one per plan.
    const int64_t n = plans_++;
    if (n % kMarkEvery == 0) EMBER_HIP_CHECK(hipEventRecord(consumed_[(n / kMarkEvery) % kMarks], stream_));
    stage_ = static_cast<int>(n % kStages);
    EMBER_HIP_CHECK(hipEventSynchronize(staged_[stage_]));  // its staging buffer is free again
    int32_t *hp = host_ints_[stage_];
    int32_t *dp = dev_ints_[stage_];
    size_t off = 0;
    std::vector<size_t> at;
    auto put = [&](const int32_t *src, size_t n) {
        at.push_back(off);
        if (n) std::memcpy(hp + off, src, n * sizeof(int32_t));
        off += pad32(n);
    };
    put(b.positions.data(), static_cast<size_t>(T));
    put(token_seq_.data(), static_cast<size_t>(T));
    put(b.block_tables.data(), b.block_tables.size());
    put(decode_.data(), decode_.size());
    put(run_first_.data(), run_first_.size());
    put(run_count_.data(), run_count_.size());
    put(tile_start_.data(), tile_start_.size());
    put(tile_end_.data(), tile_end_.size());
    put(tile_seq_.data(), tile_seq_.size());
    put(work_.data(), work_.size());
    put(work_desc_.data(), work_desc_.size());
    // The step's token ids and logit rows ride along for a backend's embedding and final norm.
    put(b.tokens.size() == static_cast<size_t>(T) ? b.tokens.data() : nullptr,
        b.tokens.size() == static_cast<size_t>(T) ? static_cast<size_t>(T) : 0);
    EMBER_CHECK(b.logit_rows.size() <= static_cast<size_t>(T), "{} logit rows for {} tokens", b.logit_rows.size(), T);
    put(b.logit_rows.data(), b.logit_rows.size());
    EMBER_CHECK(off <= ints_capacity_, "internal: step buffer too small ({} > {})", off, ints_capacity_);
    // The copy waits for the kernels that last read this buffer (kStages plans
    // ago), then runs beside stream_'s work. The host, not stream_, waits for
    // it: the host is normally steps ahead, so the wait costs it little, while a
    // cross-stream wait on stream_ idles the GPU for about 10 us per step.
    if (n >= kStages) {
        // This buffer's previous plan, n - kStages, had its kernels enqueued
        // before plan n - kStages + 1; the first mark after it, at plan m
        // (at most n - kMarkEvery), covers them, and its ring slot is not
        // recorded again before plan m + kMarks * kMarkEvery > n.
        const int64_t m = ((n - kStages) / kMarkEvery + 1) * kMarkEvery;
        EMBER_HIP_CHECK(hipStreamWaitEvent(upload_stream_, consumed_[(m / kMarkEvery) % kMarks], 0));
    }
    EMBER_HIP_CHECK(hipMemcpyAsync(dp, hp, off * sizeof(int32_t), hipMemcpyHostToDevice, upload_stream_));
    EMBER_HIP_CHECK(hipEventRecord(staged_[stage_], upload_stream_));
    EMBER_HIP_CHECK(hipEventSynchronize(staged_[stage_]));
    if (graph_splits > 0) {
        // A graph plan: the kernels read the fixed graph block, refreshed on stream_ behind the launches of
        // earlier plans (the upload it copies has completed: the host waited for it above).
        EMBER_HIP_CHECK(hipMemcpyAsync(graph_ints_, dp, off * sizeof(int32_t), hipMemcpyDeviceToDevice, stream_));
        dp = graph_ints_;
    }
    d_positions_ = dp + at[0];
    d_token_seq_ = dp + at[1];
    d_tables_ = dp + at[2];
    d_decode_ = dp + at[3];
    d_run_first_ = dp + at[4];
    d_run_count_ = dp + at[5];
    d_tile_start_ = dp + at[6];
    d_tile_end_ = dp + at[7];
    d_tile_seq_ = dp + at[8];
    d_work_ = dp + at[9];
    d_work_desc_ = dp + at[10];
    d_tokens_ = b.tokens.size() == static_cast<size_t>(T) ? dp + at[11] : nullptr;
    d_logit_rows_ = dp + at[12];
}

void HipPagedKv::layer(int l, const void *qkv, const float *q_norm, const float *k_norm, const float *bias, void *out) {
    EMBER_CHECK(T_ > 0, "layer() before plan()");
    EMBER_CHECK(qkv && out, "layer(): null qkv or out");
    EMBER_CHECK(reinterpret_cast<uintptr_t>(qkv) % 16 == 0, "layer(): qkv must be 16-byte aligned");
    void *kc = k_pool(l), *vc = v_pool(l);

    EmberQkvArgs qa{};
    qa.qkv = qkv;
    qa.q_out = q_;
    qa.k_cache = kc;
    qa.v_cache = vc;
    qa.q_norm = q_norm;
    qa.k_norm = k_norm;
    qa.bias = bias;
    qa.inv_freq = inv_freq_;
    qa.positions = d_positions_;
    qa.token_seq = d_token_seq_;
    qa.block_tables = d_tables_;
    qa.max_blocks = max_blocks_;
    qa.T = T_;
    qa.n_heads = cfg_.n_heads;
    qa.n_kv = cfg_.n_kv_heads;
    qa.head_dim = cfg_.head_dim;
    qa.eps = cfg_.rms_eps;
    qa.num_blocks = opt_.num_blocks + 1;
    qa.dtype = opt_.dtype;
    if (!fused_) check_abi(ember_hip_kv_append(&qa, stream_), "kv_append");

    const float scale = 1.0f / std::sqrt(static_cast<float>(cfg_.head_dim));
    if (decode_runs_ > 0) {
        EmberAttnArgs at{};
        at.token_index = d_decode_;
        at.q = q_;
        at.k_cache = kc;
        at.v_cache = vc;
        at.positions = d_positions_;
        at.token_seq = d_token_seq_;
        at.block_tables = d_tables_;
        at.max_blocks = max_blocks_;
        at.T = decode_count_;
        at.n_heads = cfg_.n_heads;
        at.n_kv = cfg_.n_kv_heads;
        at.head_dim = cfg_.head_dim;
        at.scale = scale;
        at.out = out;
        at.num_splits = splits_;
        at.split_len = opt_.split_len;
        at.part_acc = part_acc_;
        at.part_ml = part_ml_;
        at.num_blocks = opt_.num_blocks + 1;
        at.dtype = opt_.dtype;
        at.run_first = d_run_first_;
        at.run_count = d_run_count_;
        at.num_runs = decode_runs_;
        at.max_run = max_run_;
        at.work = d_work_;
        at.num_work = num_work_;
        at.work_desc = d_work_desc_;
        at.merge_counters = merge_counters_;
        hipEvent_t start = nullptr, stop = nullptr;
        if (timing_) decode_timing_.next(&start, &stop);  // the kernel's own dispatch (hipExtLaunchKernel), not the gap before it
        check_abi(hip::paged_decode(&at, stream_, start, stop, fused_ ? &qa : nullptr), "paged_decode");
    }
    if (tiles_ > 0) {
        EmberPrefillArgs pa{};
        pa.q = q_;
        pa.k_cache = kc;
        pa.v_cache = vc;
        pa.tile_start = d_tile_start_;
        pa.tile_end = d_tile_end_;
        pa.tile_seq = d_tile_seq_;
        pa.positions = d_positions_;
        pa.block_tables = d_tables_;
        pa.num_tiles = tiles_;
        pa.max_blocks = max_blocks_;
        pa.n_heads = cfg_.n_heads;
        pa.n_kv = cfg_.n_kv_heads;
        pa.head_dim = cfg_.head_dim;
        pa.scale = scale;
        pa.out = out;
        pa.num_blocks = opt_.num_blocks + 1;
        pa.dtype = opt_.dtype;
        pa.heads_per_group = prefill_hg_;
        hipEvent_t start = nullptr, stop = nullptr;
        if (timing_) prefill_timing_.next(&start, &stop);
        check_abi(hip::prefill_attn(&pa, stream_, start, stop), "prefill_attn");
    }
}

void HipPagedKv::Timing::next(hipEvent_t *start, hipEvent_t *stop) {
    if (used + 2 > events.size())
        for (int i = 0; i < 2; i++) {
            hipEvent_t e;
            EMBER_HIP_CHECK(hipEventCreate(&e));
            events.push_back(e);
        }
    *start = events[used];
    *stop = events[used + 1];
    used += 2;
}

int HipPagedKv::Timing::collect(double *total_ms) {
    double ms = 0;
    for (size_t i = 0; i + 1 < used; i += 2) {
        EMBER_HIP_CHECK(hipEventSynchronize(events[i + 1]));
        float one = 0;
        EMBER_HIP_CHECK(hipEventElapsedTime(&one, events[i], events[i + 1]));
        ms += one;
    }
    const int launches = static_cast<int>(used / 2);
    used = 0;
    if (total_ms) *total_ms = ms;
    return launches;
}

int HipPagedKv::collect_timing(double *total_ms) { return decode_timing_.collect(total_ms); }

int HipPagedKv::collect_prefill_timing(double *total_ms) { return prefill_timing_.collect(total_ms); }

int HipPagedKv::token_bucket(int T) {
    static const int buckets[] = {1, 2, 3, 4, 6, 8, 12, 16, 24, 32, 40, 48, 56, 64};
    for (int b : buckets)
        if (T <= b) return b;
    return kGraphMaxTokens;
}

int HipPagedKv::width_bucket(int w) const {
    int b = 16;
    while (b < w) b *= 4;
    return std::min(b, max_blocks_per_seq_);
}

bool HipPagedKv::decode_graph(const StepBatch &b, std::span<const LayerIo> io) {
    EMBER_CHECK(static_cast<int>(io.size()) == cfg_.n_layers, "decode_graph: {} layer buffers for {} layers", io.size(),
                cfg_.n_layers);
    if (plan_graph(b) == 0) return false;
    const uint64_t key = graph_key();
    auto it = graphs_.find(key);
    auto same_io = [&](const std::vector<LayerIo> &kept) {
        for (size_t l = 0; l < io.size(); l++)
            if (std::memcmp(&kept[l], &io[l], sizeof(LayerIo)) != 0) return false;
        return true;
    };
    if (it == graphs_.end() || !same_io(it->second.io)) {
        if (it != graphs_.end()) {
            EMBER_HIP_CHECK(hipStreamSynchronize(stream_));
            (void)hipGraphExecDestroy(it->second.exec);
            graphs_.erase(it);
        }
        GraphEntry e;
        e.io.assign(io.begin(), io.end());
        // Capture on a private stream (the path's stream may be the legacy null
        // stream, which cannot capture); the graph is launched on stream_.
        if (!capture_stream_) EMBER_HIP_CHECK(hipStreamCreateWithFlags(&capture_stream_, hipStreamNonBlocking));
        hipGraph_t graph = nullptr;
        const hipStream_t path_stream = stream_;
        EMBER_HIP_CHECK(hipStreamBeginCapture(capture_stream_, hipStreamCaptureModeThreadLocal));
        stream_ = capture_stream_;
        try {
            for (int l = 0; l < cfg_.n_layers; l++) {
                const LayerIo &x = io[static_cast<size_t>(l)];
                layer(l, x.qkv, x.q_norm, x.k_norm, x.bias, x.out);
            }
        } catch (...) {
            stream_ = path_stream;
            (void)hipStreamEndCapture(capture_stream_, &graph);
            if (graph) (void)hipGraphDestroy(graph);
            throw;
        }
        stream_ = path_stream;
        EMBER_HIP_CHECK(hipStreamEndCapture(capture_stream_, &graph));
        const hipError_t inst = hipGraphInstantiate(&e.exec, graph, nullptr, nullptr, 0);
        (void)hipGraphDestroy(graph);
        EMBER_HIP_CHECK(inst);
        it = graphs_.emplace(key, std::move(e)).first;
        graph_captures_++;
    }
    EMBER_HIP_CHECK(hipGraphLaunch(it->second.exec, stream_));
    return true;
}

int HipPagedKv::graph_bucket(const StepBatch &b) const {
    const int T = b.num_tokens(), S = b.num_seqs();
    if (T < 1 || T > kGraphMaxTokens || S != T || static_cast<int>(b.query_start.size()) != S + 1) return 0;
    for (int s = 0; s <= S; s++)
        if (b.query_start[static_cast<size_t>(s)] != s) return 0;  // one new token per sequence
    const int TB = token_bucket(T), WB = width_bucket(std::max(b.max_blocks, 1));
    if (TB > opt_.max_batch_tokens || TB > opt_.max_seqs || b.max_blocks > WB) return 0;
    return TB;
}

uint64_t HipPagedKv::graph_key() const {
    // Within a bucket pair every array of the plan has the same length, so the same offsets in the graph block.
    return (static_cast<uint64_t>(graph_tb_) << 32) | static_cast<uint64_t>(graph_wb_);
}

int HipPagedKv::plan_graph(const StepBatch &b) {
    const int TB = graph_bucket(b);
    if (TB == 0) return 0;
    const int T = b.num_tokens(), S = b.num_seqs();
    const int WB = width_bucket(std::max(b.max_blocks, 1));
    EMBER_CHECK(!timing_, "decode_graph: kernel timing is not available inside a graph");
    EMBER_CHECK(static_cast<int64_t>(b.block_tables.size()) == static_cast<int64_t>(S) * b.max_blocks &&
                    static_cast<int>(b.positions.size()) == T,
                "decode_graph: malformed batch");
    // The real rows are checked as plan() checks them, before padding widens
    // their tables with the spare block: a position past the caller's own
    // table would otherwise land in the spare block instead of failing.
    for (int t = 0; t < T; t++) {
        const int pos = b.positions[static_cast<size_t>(t)];
        EMBER_CHECK(pos >= 0 && pos < b.max_blocks * kBlockSize, "token {} at position {} is beyond its block table", t,
                    pos);
        const int32_t *row = &b.block_tables[static_cast<size_t>(t) * b.max_blocks];
        for (int p = 0; p <= pos / kBlockSize; p++)
            EMBER_CHECK(row[p] >= 0 && row[p] <= opt_.num_blocks, "sequence {} page {} names block {} (pool of {})", t, p,
                        row[p], opt_.num_blocks);
    }

    // The padded step: real rows keep their table and continue with the spare
    // block; padding rows are sequences of one token at position 0 whose whole
    // table is the spare block.
    StepBatch p;
    p.max_blocks = WB;
    p.tokens.assign(static_cast<size_t>(TB), 0);
    p.positions.assign(static_cast<size_t>(TB), 0);
    p.query_start.resize(static_cast<size_t>(TB) + 1);
    p.context_len.assign(static_cast<size_t>(TB), 1);
    p.block_tables.assign(static_cast<size_t>(TB) * WB, spare_block());
    for (int t = 0; t <= TB; t++) p.query_start[static_cast<size_t>(t)] = t;
    for (int t = 0; t < T; t++) {
        p.tokens[static_cast<size_t>(t)] = b.tokens.empty() ? 0 : b.tokens[static_cast<size_t>(t)];
        p.positions[static_cast<size_t>(t)] = b.positions[static_cast<size_t>(t)];
        p.context_len[static_cast<size_t>(t)] = b.positions[static_cast<size_t>(t)] + 1;
        std::copy_n(b.block_tables.begin() + static_cast<ptrdiff_t>(t) * b.max_blocks, b.max_blocks,
                    p.block_tables.begin() + static_cast<ptrdiff_t>(t) * WB);
    }
    const int splits = (WB * kBlockSize + opt_.split_len - 1) / opt_.split_len;
    plan(p, splits);
    graph_tb_ = TB;
    graph_wb_ = WB;
    return TB;
}

void HipPagedKv::copy_blocks(std::span<const int32_t> src, std::span<const int32_t> dst) {
    EMBER_CHECK(src.size() == dst.size(), "copy_blocks: {} sources for {} destinations", src.size(), dst.size());
    if (src.empty()) return;
    for (size_t i = 0; i < src.size(); i++)
        EMBER_CHECK(src[i] >= 0 && src[i] <= opt_.num_blocks && dst[i] >= 0 && dst[i] <= opt_.num_blocks,
                    "copy_blocks: pair {} ({} -> {}) is outside the pool", i, src[i], dst[i]);
    // The pair list goes up through one of two pinned staging buffers into the
    // matching preallocated device list, on stream_, ahead of the copy kernel.
    // A buffer is reused once the copy kernel that read it has run (its event;
    // normally long done), so nothing is allocated and the host does not wait
    // for the stream.
    for (size_t at = 0; at < src.size(); at += kCowPairs) {
        const size_t n = std::min(src.size() - at, static_cast<size_t>(kCowPairs));
        cow_stage_ ^= 1;
        EMBER_HIP_CHECK(hipEventSynchronize(cow_done_[cow_stage_]));
        int32_t *hp = cow_host_[cow_stage_], *dp = cow_dev_[cow_stage_];
        std::copy_n(src.begin() + static_cast<ptrdiff_t>(at), n, hp);
        std::copy_n(dst.begin() + static_cast<ptrdiff_t>(at), n, hp + n);
        EMBER_HIP_CHECK(hipMemcpyAsync(dp, hp, 2 * n * sizeof(int32_t), hipMemcpyHostToDevice, stream_));
        EmberCopyArgs ca{};
        ca.k_cache = k_;
        ca.v_cache = v_;
        ca.src_blocks = dp;
        ca.dst_blocks = dp + n;
        ca.n = static_cast<int32_t>(n);
        ca.n_layers = cfg_.n_layers;
        ca.layer_stride = layer_elems_;
        ca.n_kv = cfg_.n_kv_heads;
        ca.head_dim = cfg_.head_dim;
        ca.num_blocks = opt_.num_blocks + 1;
        ca.dtype = opt_.dtype;
        const int code = ember_hip_copy_pages(&ca, stream_);
        EMBER_HIP_CHECK(hipEventRecord(cow_done_[cow_stage_], stream_));
        check_abi(code, "copy_pages");
    }
}

}  // namespace ember
