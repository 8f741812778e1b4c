// A test driver that plays the reference engine's block-table logic against
// any ember::Backend and the product ember::BlockManager, compiled from the
// product headers alone (backend/backend.hpp, kvcache/block_manager.hpp).
//
// It restates what the engine does with pages (src/engine/engine.cpp):
//   - admission: match_prefix(tokens[0 .. n-1)) hands out cached pages, the
//     last token is always computed (:303-313);
//   - ensure_blocks (:176-184): pages up to the chunk's end, preempting the
//     newest running sequence (from the back, never one already in this step)
//     when the pool runs dry, or the sequence itself (:268-289);
//   - seal_full_blocks (:186-193): every full computed page sealed, chained;
//   - preempt (:195-205): pages released, the sequence computed again later;
//   - decodes scheduled before prompt chunks, chunks capped (:256-296);
//   - speculative verify (:578-641): [last token, drafts] in one run per
//     sequence, one logit row per position, the matching prefix accepted, the
//     rejected slots left to be overwritten (computed = n + accepted).
// Outputs are compared with what each request produces on its own, so any
// page or slot mistake shows up as a different token.
#pragma once

#include <algorithm>
#include <cstdint>
#include <deque>
#include <functional>
#include <memory>
#include <span>
#include <string>
#include <vector>

#include "backend/backend.hpp"
#include "common/error.hpp"
#include "kvcache/block_manager.hpp"

namespace ember::testing {

struct MiniRequest {
    std::vector<int32_t> prompt;
    int max_tokens = 16;
    SamplingParams sampling{};  // default: temperature 1 (set 0 for greedy)
};

struct MiniSeq {
    int id = 0;
    MiniRequest req;
    std::vector<int32_t> tokens;  // prompt + generated
    std::vector<int32_t> out;     // generated
    std::vector<int> blocks;
    int computed = 0, sealed = 0;
    uint64_t chain = 0;
    bool finished = false;
};

struct MiniOptions {
    int max_batch_tokens = 256;
    int max_prefill_chunk = 512;
    int max_seqs = 16;
    std::vector<int32_t> eos_ids;
    // Speculative verify: when set, pure-decode steps propose k drafts per
    // sequence with this function (given the sequence's tokens) and verify them.
    int spec_k = 0;
    std::function<std::vector<int32_t>(const std::vector<int32_t> &, int k)> draft;
};

class MiniEngine {
public:
    MiniEngine(Backend &be, BlockManager &bm, MiniOptions opt) : be_(be), bm_(bm), opt_(std::move(opt)) {}

    void submit(MiniRequest r) {
        auto s = std::make_unique<MiniSeq>();
        s->id = static_cast<int>(all_.size());
        s->tokens = r.prompt;
        s->req = std::move(r);
        waiting_.push_back(s.get());
        all_.push_back(std::move(s));
    }

    // Runs steps until every request finishes; `audit` runs after each step.
    void run(const std::function<void()> &audit = {}) {
        for (int guard = 0; guard < 100000 && !all_done(); guard++) {
            step();
            if (audit) audit();
        }
        if (!all_done()) throw Error("mini engine: requests did not finish");
    }

    const std::vector<std::unique_ptr<MiniSeq>> &sequences() const { return all_; }
    int steps = 0, preemptions = 0, spec_steps = 0, accepted = 0, proposed = 0;

private:
    bool all_done() const {
        for (const auto &s : all_)
            if (!s->finished) return false;
        return true;
    }

    bool ensure_blocks(MiniSeq &s, int upto) {
        const size_t need = static_cast<size_t>((upto + kBlockSize - 1) / kBlockSize);
        while (s.blocks.size() < need) {
            const int b = bm_.allocate();
            if (b < 0) return false;
            s.blocks.push_back(b);
        }
        return true;
    }

    void seal_full_blocks(MiniSeq &s) {
        if (!bm_.prefix_caching()) return;
        for (; (s.sealed + 1) * kBlockSize <= s.computed; s.sealed++) {
            std::span<const int32_t> page(s.tokens.data() + static_cast<size_t>(s.sealed) * kBlockSize, kBlockSize);
            s.chain = bm_.seal(s.blocks[static_cast<size_t>(s.sealed)], s.chain, page);
        }
    }

    void preempt(MiniSeq &s) {
        bm_.release_all(s.blocks);
        s.blocks.clear();
        s.computed = s.sealed = 0;
        s.chain = 0;
        preemptions++;
    }

    void finish(MiniSeq &s) {
        bm_.release_all(s.blocks);
        s.blocks.clear();
        s.finished = true;
    }

    // Appends a sampled token; true when the request is complete.
    bool append(MiniSeq &s, int32_t tok) {
        s.tokens.push_back(tok);
        if (std::find(opt_.eos_ids.begin(), opt_.eos_ids.end(), tok) != opt_.eos_ids.end()) return true;
        s.out.push_back(tok);
        return static_cast<int>(s.out.size()) >= s.req.max_tokens;
    }

    void drop_finished() {
        running_.erase(std::remove_if(running_.begin(), running_.end(), [](MiniSeq *s) { return s->finished; }),
                       running_.end());
    }

    void step() {
        steps++;
        if (opt_.spec_k > 0 && waiting_.empty() && !running_.empty()) {
            bool all_decode = true;
            for (MiniSeq *s : running_) all_decode = all_decode && static_cast<int>(s->tokens.size()) - s->computed == 1;
            if (all_decode && spec_step()) return;
        }
        StepBatch b;
        b.clear();
        std::vector<MiniSeq *> seqs;
        std::vector<int> counts;
        int budget = opt_.max_batch_tokens;
        auto add = [&](MiniSeq &s, int n) {
            for (int i = 0; i < n; i++) {
                b.tokens.push_back(s.tokens[static_cast<size_t>(s.computed + i)]);
                b.positions.push_back(s.computed + i);
            }
            b.query_start.push_back(static_cast<int32_t>(b.tokens.size()));
            b.context_len.push_back(s.computed + n);
            seqs.push_back(&s);
            counts.push_back(n);
            budget -= n;
        };
        bool preempted = false;
        for (int pass = 0; pass < 2; pass++) {  // decodes first, then prompt chunks
            for (size_t i = 0; i < running_.size() && budget > 0;) {
                MiniSeq &s = *running_[i];
                const int need = static_cast<int>(s.tokens.size()) - s.computed;
                if ((need == 1) != (pass == 0) || need <= 0) {
                    i++;
                    continue;
                }
                const int n = std::min({need, budget, opt_.max_prefill_chunk});
                bool ok = ensure_blocks(s, s.computed + n);
                while (!ok) {
                    MiniSeq &victim = *running_.back();
                    if (&victim == &s || std::find(seqs.begin(), seqs.end(), &victim) != seqs.end()) break;
                    preempt(victim);
                    waiting_.push_front(&victim);
                    running_.pop_back();
                    preempted = true;
                    ok = ensure_blocks(s, s.computed + n);
                }
                if (!ok) {
                    preempt(s);
                    waiting_.push_front(&s);
                    running_.erase(running_.begin() + static_cast<ptrdiff_t>(i));
                    preempted = true;
                    continue;
                }
                add(s, n);
                i++;
            }
        }
        while (!preempted && !waiting_.empty() && budget > 0 && static_cast<int>(running_.size()) < opt_.max_seqs) {
            MiniSeq &s = *waiting_.front();
            if (s.computed == 0 && s.blocks.empty()) {
                // cached pages for all but the last token, whose logits are needed
                s.blocks = bm_.match_prefix(std::span<const int32_t>(s.tokens.data(), s.tokens.size() - 1));
                s.sealed = static_cast<int>(s.blocks.size());
                s.computed = s.sealed * kBlockSize;
                s.chain = 0;
                for (int p = 0; p < s.sealed; p++)
                    s.chain = BlockManager::block_hash(
                        s.chain, std::span<const int32_t>(s.tokens.data() + static_cast<size_t>(p) * kBlockSize, kBlockSize));
            }
            const int n = std::min({static_cast<int>(s.tokens.size()) - s.computed, budget, opt_.max_prefill_chunk});
            if (!ensure_blocks(s, s.computed + n)) {
                bm_.release_all(s.blocks);
                s.blocks.clear();
                s.computed = s.sealed = 0;
                s.chain = 0;
                break;
            }
            add(s, n);
            running_.push_back(&s);
            waiting_.pop_front();
        }
        if (seqs.empty()) return;
        fill_tables(b, seqs);
        std::vector<SampleRequest> reqs;
        for (size_t i = 0; i < seqs.size(); i++) {
            if (seqs[i]->computed + counts[i] != static_cast<int>(seqs[i]->tokens.size())) continue;
            b.logit_rows.push_back(b.query_start[i + 1] - 1);
            SampleRequest r;
            r.params = seqs[i]->req.sampling;
            r.counter = seqs[i]->tokens.size();
            reqs.push_back(r);
        }
        be_.forward(b);
        std::vector<int32_t> toks(reqs.size());
        be_.sample(reqs, toks);
        size_t r = 0;
        for (size_t i = 0; i < seqs.size(); i++) {
            MiniSeq &s = *seqs[i];
            const bool wants = s.computed + counts[i] == static_cast<int>(s.tokens.size());
            s.computed += counts[i];
            bool done = false;
            if (wants) done = append(s, toks[r++]);
            seal_full_blocks(s);
            if (done) finish(s);
        }
        drop_finished();
    }

    // Verify k drafts per running sequence in one step (every sequence decoding).
    bool spec_step() {
        const int k = opt_.spec_k;
        std::vector<std::vector<int32_t>> ext;
        for (MiniSeq *s : running_) {
            std::vector<int32_t> e = s->tokens;
            auto d = opt_.draft(e, k);
            e.insert(e.end(), d.begin(), d.end());
            if (!ensure_blocks(*s, static_cast<int>(e.size()))) return false;  // the plain path preempts
            ext.push_back(std::move(e));
        }
        StepBatch b;
        b.clear();
        std::vector<SampleRequest> reqs;
        for (size_t i = 0; i < running_.size(); i++) {
            MiniSeq &s = *running_[i];
            const int n = static_cast<int>(s.tokens.size());
            for (int p = n - 1; p <= n - 1 + k; p++) {
                b.tokens.push_back(ext[i][static_cast<size_t>(p)]);
                b.positions.push_back(p);
                b.logit_rows.push_back(static_cast<int32_t>(b.tokens.size()) - 1);
                SampleRequest r;
                r.params = s.req.sampling;
                r.counter = static_cast<uint64_t>(p + 1);
                reqs.push_back(r);
            }
            b.query_start.push_back(static_cast<int32_t>(b.tokens.size()));
            b.context_len.push_back(n + k);
        }
        std::vector<MiniSeq *> seqs(running_.begin(), running_.end());
        fill_tables(b, seqs);
        be_.forward(b);
        std::vector<int32_t> toks(reqs.size());
        be_.sample(reqs, toks);
        spec_steps++;
        for (size_t i = 0; i < seqs.size(); i++) {
            MiniSeq &s = *seqs[i];
            const int32_t *t = &toks[i * static_cast<size_t>(k + 1)];
            const int n = static_cast<int>(s.tokens.size());
            int m = 0;
            while (m < k && t[m] == ext[i][static_cast<size_t>(n + m)]) m++;
            proposed += k;
            accepted += m;
            bool done = false;
            int appended = 0;
            for (int j = 0; j <= m && !done; j++, appended++) done = append(s, t[j]);
            // the cache holds valid entries for the inputs that matched: positions n-1 .. n-1+m
            s.computed = n + std::min(m, appended - 1);
            seal_full_blocks(s);
            if (done) finish(s);
        }
        drop_finished();
        return true;
    }

    void fill_tables(StepBatch &b, const std::vector<MiniSeq *> &seqs) const {
        int mb = 0;
        for (MiniSeq *s : seqs) mb = std::max(mb, static_cast<int>(s->blocks.size()));
        b.max_blocks = mb;
        b.block_tables.assign(seqs.size() * static_cast<size_t>(mb), 0);
        for (size_t i = 0; i < seqs.size(); i++)
            std::copy(seqs[i]->blocks.begin(), seqs[i]->blocks.end(),
                      b.block_tables.begin() + static_cast<ptrdiff_t>(i * static_cast<size_t>(mb)));
    }

    Backend &be_;
    BlockManager &bm_;
    MiniOptions opt_;
    std::vector<std::unique_ptr<MiniSeq>> all_;
    std::deque<MiniSeq *> waiting_;
    std::vector<MiniSeq *> running_;
};

}  // namespace ember::testing
