// Block manager: same observable behaviour as the reference's
// src/kvcache/block_manager.cpp:9-139 (which block each call hands out, in
// which order cached blocks are evicted, what is found and shared), on flat
// arrays instead of node-based containers.
#include "kvcache/block_manager.hpp"

#include <algorithm>

#include "common/error.hpp"

namespace ember {

BlockManager::BlockManager(int num_blocks, bool prefix_caching) : prefix_caching_(prefix_caching) {
    EMBER_CHECK(num_blocks > 0, "the KV cache has no blocks");
    const size_t n = static_cast<size_t>(num_blocks);
    refs_.assign(n, 0);
    sealed_.assign(n, 0);
    hash_.assign(n, 0);
    parent_.assign(n, 0);
    tokens_.assign(n * kBlockSize, 0);
    lru_prev_.assign(n, kNone);
    lru_next_.assign(n, kNone);
    // A stack whose top is block 0: low ids are handed out first (block_manager.cpp:12).
    free_.resize(n);
    for (size_t i = 0; i < n; i++) free_[i] = static_cast<int32_t>(n - 1 - i);
    size_t cap = 16;
    while (cap < 2 * n) cap <<= 1;
    index_.assign(cap, Slot{0, kNone});
    index_mask_ = cap - 1;
}

uint64_t BlockManager::block_hash(uint64_t parent, std::span<const int32_t> tokens) {
    // FNV-1a over 32-bit token words, seeded with the parent's hash, then the
    // MurmurHash3 64-bit finalizer (block_manager.cpp:15-28). 0 is reserved.
    uint64_t h = 0xcbf29ce484222325ull ^ parent;
    for (int32_t t : tokens) {
        h ^= static_cast<uint32_t>(t);
        h *= 0x100000001b3ull;
    }
    h ^= h >> 33;
    h *= 0xff51afd7ed558ccdull;
    h ^= h >> 33;
    h *= 0xc4ceb9fe1a85ec53ull;
    h ^= h >> 33;
    return h ? h : 1;
}

// ---- LRU list of sealed, unreferenced blocks (oldest at the head) ----

void BlockManager::lru_push_back(int b) {
    lru_prev_[static_cast<size_t>(b)] = lru_tail_;
    lru_next_[static_cast<size_t>(b)] = kNone;
    if (lru_tail_ != kNone) lru_next_[static_cast<size_t>(lru_tail_)] = b;
    else lru_head_ = b;
    lru_tail_ = b;
    lru_count_++;
}

void BlockManager::lru_remove(int b) {
    const int32_t p = lru_prev_[static_cast<size_t>(b)], n = lru_next_[static_cast<size_t>(b)];
    if (p != kNone) lru_next_[static_cast<size_t>(p)] = n;
    else lru_head_ = n;
    if (n != kNone) lru_prev_[static_cast<size_t>(n)] = p;
    else lru_tail_ = p;
    lru_prev_[static_cast<size_t>(b)] = lru_next_[static_cast<size_t>(b)] = kNone;
    lru_count_--;
}

// ---- hash index: the hash values are already mixed, so the low bits serve as the home slot ----

int BlockManager::index_find(uint64_t h) const {
    for (uint64_t i = h & index_mask_;; i = (i + 1) & index_mask_) {
        const Slot &s = index_[i];
        if (s.hash == 0) return kNone;
        if (s.hash == h) return s.block;
    }
}

void BlockManager::index_insert(uint64_t h, int b) {
    uint64_t i = h & index_mask_;
    while (index_[i].hash != 0) i = (i + 1) & index_mask_;
    index_[i] = Slot{h, b};
    cached_++;
}

void BlockManager::index_erase(uint64_t h) {
    uint64_t i = h & index_mask_;
    while (index_[i].hash != h) {
        if (index_[i].hash == 0) return;
        i = (i + 1) & index_mask_;
    }
    // Backward-shift deletion: pull later members of the probe run into the hole.
    for (uint64_t j = (i + 1) & index_mask_; index_[j].hash != 0; j = (j + 1) & index_mask_) {
        const uint64_t home = index_[j].hash & index_mask_;
        const bool movable = i <= j ? (home <= i || home > j) : (home <= i && home > j);
        if (movable) {
            index_[i] = index_[j];
            i = j;
        }
    }
    index_[i] = Slot{0, kNone};
    cached_--;
}

// ---- allocation ----

int BlockManager::allocate() {
    int b;
    if (!free_.empty()) {
        b = free_.back();
        free_.pop_back();
    } else if (lru_head_ != kNone) {
        b = lru_head_;
        lru_remove(b);
        unseal(b);
    } else {
        return -1;
    }
    refs_[static_cast<size_t>(b)] = 1;
    return b;
}

void BlockManager::unseal(int b) {
    if (!sealed_[static_cast<size_t>(b)]) return;
    const uint64_t h = hash_[static_cast<size_t>(b)];
    if (index_find(h) == b) index_erase(h);
    sealed_[static_cast<size_t>(b)] = 0;
    hash_[static_cast<size_t>(b)] = 0;
}

void BlockManager::release(int b) {
    EMBER_CHECK(b >= 0 && b < num_blocks(), "internal: releasing block {} of {}", b, num_blocks());
    int32_t &refs = refs_[static_cast<size_t>(b)];
    EMBER_CHECK(refs > 0, "internal: releasing free block {}", b);
    if (--refs > 0) return;
    // A sealed block is always the one its hash is indexed under (seal never
    // indexes a second block with the same hash).
    if (sealed_[static_cast<size_t>(b)] && prefix_caching_) {
        lru_push_back(b);
    } else {
        unseal(b);
        free_.push_back(b);
    }
}

void BlockManager::release_all(std::span<const int> blocks) {
    for (size_t i = blocks.size(); i-- > 0;) release(blocks[i]);
}

// ---- prefix cache ----

std::vector<int> BlockManager::match_prefix(std::span<const int32_t> tokens) {
    std::vector<int> out;
    if (!prefix_caching_) return out;
    lookup_tokens_ += tokens.size();
    uint64_t parent = 0;
    const size_t full = tokens.size() / kBlockSize;
    for (size_t i = 0; i < full; i++) {
        const auto chunk = tokens.subspan(i * kBlockSize, kBlockSize);
        const uint64_t h = block_hash(parent, chunk);
        const int b = index_find(h);
        if (b == kNone) break;
        const int32_t *stored = &tokens_[static_cast<size_t>(b) * kBlockSize];
        if (parent_[static_cast<size_t>(b)] != parent || !std::equal(chunk.begin(), chunk.end(), stored)) break;  // collision
        if (refs_[static_cast<size_t>(b)] == 0) lru_remove(b);
        refs_[static_cast<size_t>(b)]++;
        out.push_back(b);
        parent = h;
    }
    hit_tokens_ += out.size() * kBlockSize;
    return out;
}

uint64_t BlockManager::seal(int b, uint64_t parent, std::span<const int32_t> tokens) {
    EMBER_CHECK(tokens.size() == static_cast<size_t>(kBlockSize), "internal: sealing a block with {} tokens", tokens.size());
    const uint64_t h = block_hash(parent, tokens);
    if (!prefix_caching_) return h;
    EMBER_CHECK(b >= 0 && b < num_blocks(), "internal: sealing block {} of {}", b, num_blocks());
    if (sealed_[static_cast<size_t>(b)]) return hash_[static_cast<size_t>(b)];
    if (index_find(h) != kNone) return h;  // an identical block is cached: this one stays private
    sealed_[static_cast<size_t>(b)] = 1;
    hash_[static_cast<size_t>(b)] = h;
    parent_[static_cast<size_t>(b)] = parent;
    std::copy(tokens.begin(), tokens.end(), tokens_.begin() + static_cast<ptrdiff_t>(b) * kBlockSize);
    index_insert(h, b);
    return h;
}

// ---- audit ----

std::string BlockManager::check() const {
    const size_t n = refs_.size();
    std::vector<int> seen(n, 0);
    for (int b : free_) {
        if (refs_[static_cast<size_t>(b)] != 0) return format("free block {} has references", b);
        if (sealed_[static_cast<size_t>(b)]) return format("free block {} is sealed", b);
        seen[static_cast<size_t>(b)]++;
    }
    int walked = 0;
    for (int b = lru_head_; b != kNone; b = lru_next_[static_cast<size_t>(b)]) {
        if (refs_[static_cast<size_t>(b)] != 0 || !sealed_[static_cast<size_t>(b)])
            return format("evictable block {} is in use or unsealed", b);
        seen[static_cast<size_t>(b)]++;
        if (++walked > lru_count_) return format("the LRU list is longer than its count {}", lru_count_);
    }
    if (walked != lru_count_) return format("the LRU list holds {} blocks, its count says {}", walked, lru_count_);
    for (size_t b = 0; b < n; b++) {
        if (refs_[b] > 0) seen[b]++;
        if (seen[b] != 1) return format("block {} is accounted for {} times", b, seen[b]);
    }
    int indexed = 0;
    for (const Slot &s : index_) {
        if (s.hash == 0) continue;
        indexed++;
        if (s.block < 0 || static_cast<size_t>(s.block) >= n || !sealed_[static_cast<size_t>(s.block)] ||
            hash_[static_cast<size_t>(s.block)] != s.hash)
            return format("hash index points to block {} with a different hash", s.block);
    }
    if (indexed != cached_) return format("the hash index holds {} entries, its count says {}", indexed, cached_);
    return {};
}

std::vector<uint8_t> BlockManager::states() const {
    std::vector<uint8_t> s(refs_.size(), 0);
    for (size_t b = 0; b < refs_.size(); b++) s[b] = refs_[b] > 0 ? 2 : 0;
    for (int b = lru_head_; b != kNone; b = lru_next_[static_cast<size_t>(b)]) s[static_cast<size_t>(b)] = 1;
    return s;
}

// ---- additions ----

void BlockManager::share(std::span<const int> blocks) {
    for (int b : blocks)
        EMBER_CHECK(b >= 0 && b < num_blocks() && refs_[static_cast<size_t>(b)] > 0, "share: block {} is not held", b);
    for (int b : blocks) refs_[static_cast<size_t>(b)]++;
}

int BlockManager::copy_on_write(int b) {
    EMBER_CHECK(b >= 0 && b < num_blocks() && refs_[static_cast<size_t>(b)] > 0, "copy_on_write: block {} is not held", b);
    if (refs_[static_cast<size_t>(b)] == 1) return b;
    const int fresh = allocate();
    if (fresh < 0) return -1;
    refs_[static_cast<size_t>(b)]--;
    return fresh;
}

}  // namespace ember
