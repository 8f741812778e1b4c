// Allocation of KV-cache blocks with automatic prefix caching.
//
// The public interface is declaration-for-declaration the reference's
// (src/kvcache/block_manager.hpp:25-67), so the engine builds against either.
// Two calls are added after it (share, copy_on_write) for forked sequences
// that hold a partial last page in common; nothing existing changes meaning.
//
// A block completely filled with tokens can be sealed: registered under a
// hash of its tokens chained with the previous block's hash. A later prompt
// with the same start finds and shares those blocks. When the last holder of
// a sealed block lets go it stays findable in an LRU list until the space is
// needed.
//
// The implementation is built for pools of 10^5-10^6 blocks (a 288 GB device
// holds 131,072 pages of a 28-layer model): flat per-block arrays, an
// intrusive doubly-linked LRU list and an open-addressing hash index, so no
// call allocates after construction (match_prefix's result aside).
#pragma once

#include <cstdint>
#include <span>
#include <string>
#include <vector>

#include "backend/backend.hpp"

namespace ember {

class BlockManager {
public:
    BlockManager(int num_blocks, bool prefix_caching);

    int num_blocks() const { return static_cast<int>(refs_.size()); }
    // Blocks that can be handed out now: free, or cached but unused.
    int available() const { return static_cast<int>(free_.size()) + lru_count_; }
    int used() const { return num_blocks() - available(); }
    int cached() const { return cached_; }

    // A fresh block, or -1 when none is available. Evicts the least recently
    // used cached block when no block is free.
    int allocate();
    // Drops one reference; at zero the block becomes free (or evictable if sealed).
    void release(int block);
    // Releases blocks from the last to the first, so a sequence's tail pages are evicted first.
    void release_all(std::span<const int> blocks);

    // Hash of a full block of tokens after a prefix with hash `parent` (0 for the first block).
    static uint64_t block_hash(uint64_t parent, std::span<const int32_t> tokens);

    // The longest run of cached blocks matching the start of `tokens` (whole
    // blocks only); takes a reference to each.
    std::vector<int> match_prefix(std::span<const int32_t> tokens);

    // Declares `block` full with `tokens` after a prefix with hash `parent`;
    // returns the block's hash. If an identical block is cached already,
    // nothing changes (this one stays private).
    uint64_t seal(int block, uint64_t parent, std::span<const int32_t> tokens);

    bool prefix_caching() const { return prefix_caching_; }
    int refcount(int block) const { return refs_[static_cast<size_t>(block)]; }

    uint64_t hit_tokens() const { return hit_tokens_; }
    uint64_t lookup_tokens() const { return lookup_tokens_; }

    // Every block is exactly one of free / evictable / referenced, and the hash
    // index agrees with the blocks. The first problem, or "".
    std::string check() const;

    // Per block: 0 free, 1 cached (unused), 2 in use.
    std::vector<uint8_t> states() const;

    // ---- additions (no counterpart in the reference) ----

    // One more reference on each block (all must be held already): a forked
    // sequence shares its parent's pages, the partial last page included.
    void share(std::span<const int> blocks);
    // Before a holder writes into `block`: returns `block` when the caller is
    // its only holder; otherwise drops the caller's reference and returns a
    // fresh private block that the caller must fill with a copy of the page
    // (device side: ember_hip_copy_pages), or -1 when no block is available
    // (the reference stays held then).
    int copy_on_write(int block);

private:
    static constexpr int32_t kNone = -1;

    void unseal(int block);
    void lru_push_back(int block);
    void lru_remove(int block);
    int index_find(uint64_t hash) const;
    void index_insert(uint64_t hash, int block);
    void index_erase(uint64_t hash);

    // Per block.
    std::vector<int32_t> refs_;
    std::vector<uint8_t> sealed_;
    std::vector<uint64_t> hash_, parent_;
    std::vector<int32_t> tokens_;              // [num_blocks * kBlockSize], a sealed block's tokens
    std::vector<int32_t> lru_prev_, lru_next_; // links while in the LRU list

    std::vector<int32_t> free_;                // never-sealed free blocks; back() goes out next
    int32_t lru_head_ = kNone, lru_tail_ = kNone, lru_count_ = 0;

    struct Slot {
        uint64_t hash;  // 0 = empty (block_hash never returns 0)
        int32_t block;
    };
    std::vector<Slot> index_;                  // open addressing, linear probing, load <= 1/2
    uint64_t index_mask_ = 0;
    int cached_ = 0;

    bool prefix_caching_;
    uint64_t hit_tokens_ = 0, lookup_tokens_ = 0;
};

}  // namespace ember
