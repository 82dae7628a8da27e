// Host-side paged block manager (src/paged_attention.rs:89-381).
#include "paged_attention.hpp"

#include "status.hpp"

namespace airkv {

BlockAllocator::BlockAllocator(int64_t capacity, int32_t block_size, const uint32_t *free_order)
    : blocks_((size_t)capacity), ref_counts_((size_t)capacity, 0u), total_blocks_(capacity),
      block_size_(block_size) {
    for (int64_t i = 0; i < capacity; ++i) blocks_[(size_t)i].id = (uint32_t)i;
    for (int64_t i = 0; i < capacity; ++i)
        free_blocks_.push_back(free_order ? free_order[i] : (uint32_t)i);
}

bool BlockAllocator::allocate(uint32_t *out) {      // :115-121
    if (free_blocks_.empty()) return false;
    uint32_t id = free_blocks_.front();
    free_blocks_.pop_front();
    ref_counts_[id] = 1;
    blocks_[id].num_tokens = 0;
    blocks_[id].is_full = false;
    *out = id;
    return true;
}

int BlockAllocator::share(uint32_t id) {            // :124-126
    if (!valid(id)) return fail(AIR_KV_E_INVALID_ARG, "share: block %u outside the pool", id);
    ref_counts_[id] += 1;
    return AIR_KV_OK;
}

int BlockAllocator::release(uint32_t id) {          // :129-135
    if (!valid(id)) return fail(AIR_KV_E_INVALID_ARG, "release: block %u outside the pool", id);
    if (ref_counts_[id] == 0)
        return fail(AIR_KV_E_STATE, "release: block %u is already free (double release)", id);
    ref_counts_[id] -= 1;
    if (ref_counts_[id] == 0) free_blocks_.push_back(id);
    return AIR_KV_OK;
}

bool BlockAllocator::cow_write(uint32_t id, uint32_t *out) {   // :155-167
    if (ref_counts_[id] <= 1) { *out = id; return true; }
    uint32_t nid;
    if (!allocate(&nid)) return false;
    blocks_[nid].num_tokens = blocks_[id].num_tokens;
    blocks_[nid].is_full = blocks_[id].is_full;
    release(id);
    *out = nid;
    return true;
}

int BlockAllocator::append_token(uint32_t id, bool *is_full) {  // :170-178
    if (!valid(id)) return fail(AIR_KV_E_INVALID_ARG, "append_token: block %u outside the pool", id);
    PhysicalBlock &b = blocks_[id];
    if (b.is_full) return fail(AIR_KV_E_STATE, "cannot append to a full block (%u)", id);
    b.num_tokens += 1;
    if (b.num_tokens == block_size_) b.is_full = true;
    *is_full = b.is_full;
    return AIR_KV_OK;
}

uint32_t SequenceManager::create_sequence() {       // :260-265
    uint32_t id = next_seq_id_++;
    BlockTable t;
    t.seq_id = id;
    tables_[id] = std::move(t);
    return id;
}

int SequenceManager::append_token(uint32_t seq, uint32_t *block) {   // :269-286
    auto it = tables_.find(seq);
    if (it == tables_.end()) return fail(AIR_KV_E_NOT_FOUND, "sequence not found (%u)", seq);
    BlockTable &t = it->second;
    const int32_t bs = block_size();
    bool needs_new = t.physical_blocks.empty() || (t.last_block_offset(bs) == 0 && t.num_tokens > 0);
    uint32_t active;
    if (needs_new) {
        if (!allocator_.allocate(&active))
            return fail(AIR_KV_E_OOM, "out of memory — no free blocks");
        t.physical_blocks.push_back(active);
    } else {
        active = t.physical_blocks.back();
    }
    bool full;
    int rc = allocator_.append_token(active, &full);
    if (rc) return rc;
    t.num_tokens += 1;
    *block = active;
    return AIR_KV_OK;
}

int SequenceManager::fork_sequence(uint32_t parent, uint32_t *child) {   // :290-310
    auto it = tables_.find(parent);
    if (it == tables_.end()) return fail(AIR_KV_E_NOT_FOUND, "parent sequence not found (%u)", parent);
    std::vector<uint32_t> blocks = it->second.physical_blocks;
    int64_t ntok = it->second.num_tokens;
    for (uint32_t b : blocks) allocator_.share(b);
    uint32_t id = next_seq_id_++;
    BlockTable t;
    t.seq_id = id;
    t.physical_blocks = std::move(blocks);
    t.num_tokens = ntok;
    tables_[id] = std::move(t);
    *child = id;
    return AIR_KV_OK;
}

void SequenceManager::free_sequence(uint32_t seq) {   // :313-319
    auto it = tables_.find(seq);
    if (it == tables_.end()) return;
    std::vector<uint32_t> blocks = std::move(it->second.physical_blocks);
    tables_.erase(it);
    for (uint32_t b : blocks) allocator_.release(b);
}

const BlockTable *SequenceManager::table(uint32_t seq) const {   // :322-324
    auto it = tables_.find(seq);
    return it == tables_.end() ? nullptr : &it->second;
}

int SequenceManager::cow_last_block(uint32_t seq, uint32_t *old_block, uint32_t *new_block) {
    // :327-335
    auto it = tables_.find(seq);
    if (it == tables_.end()) return fail(AIR_KV_E_NOT_FOUND, "sequence not found (%u)", seq);
    if (it->second.physical_blocks.empty())
        return fail(AIR_KV_E_NOT_FOUND, "sequence %u has no blocks", seq);
    uint32_t last = it->second.physical_blocks.back(), nid;
    if (!allocator_.cow_write(last, &nid)) return fail(AIR_KV_E_OOM, "out of memory — cow_write");
    if (nid != last) {
        it->second.physical_blocks.back() = nid;
        set_own_fill(it->second, it->second.physical_blocks.size() - 1);
    }
    *old_block = last;
    *new_block = nid;
    return AIR_KV_OK;
}

// The private block that copy-on-write puts at table index `idx` holds this
// sequence's tokens of that block, whatever the shared block's fill said: a
// sequence truncated into a block it shares sees fewer tokens there than the
// other owners (whose fill the shared block keeps), and so does one whose
// co-owner appended into the shared block.  The reference copies the shared
// block's metadata (src/paged_attention.rs:159-164); that agrees with this
// whenever the sequence's own count equals the shared fill, which is every
// case its own call sequences produce without truncation or a co-owner's
// append into a shared block.
void SequenceManager::set_own_fill(const BlockTable &t, size_t idx) {
    const int64_t bs = block_size();
    const int64_t own = t.num_tokens - (int64_t)idx * bs;
    allocator_.set_fill(t.physical_blocks[idx], (int32_t)(own < 0 ? 0 : own > bs ? bs : own));
}

void SequenceManager::undo_cow(uint32_t seq, size_t idx, uint32_t old_block, uint32_t new_block) {
    auto it = tables_.find(seq);
    if (it == tables_.end() || idx >= it->second.physical_blocks.size()) return;
    if (old_block == new_block || it->second.physical_blocks[idx] != new_block) return;
    it->second.physical_blocks[idx] = old_block;
    allocator_.share(old_block);
    allocator_.release(new_block);
}

int SequenceManager::truncate(uint32_t seq, int64_t n_tokens) {
    auto it = tables_.find(seq);
    if (it == tables_.end()) return fail(AIR_KV_E_NOT_FOUND, "sequence not found (%u)", seq);
    if (n_tokens < 0) return fail(AIR_KV_E_INVALID_ARG, "truncate: negative length");
    BlockTable &t = it->second;
    if (n_tokens >= t.num_tokens) return AIR_KV_OK;
    const int32_t bs = block_size();
    const size_t keep = (size_t)BlockAllocator::num_blocks_for_tokens(n_tokens, bs);
    if (keep > t.physical_blocks.size())
        return fail(AIR_KV_E_STATE, "sequence %u holds fewer blocks than its length needs", seq);
    for (size_t i = keep; i < t.physical_blocks.size(); ++i) allocator_.release(t.physical_blocks[i]);
    t.physical_blocks.resize(keep);
    t.num_tokens = n_tokens;
    if (keep > 0) {
        const uint32_t last = t.physical_blocks.back();
        if (allocator_.ref_count(last) == 1)
            allocator_.set_fill(last, (int32_t)(n_tokens - (int64_t)(keep - 1) * bs));
    }
    return AIR_KV_OK;
}

int SequenceManager::cow_block(uint32_t seq, int64_t index, uint32_t *old_block, uint32_t *new_block) {
    auto it = tables_.find(seq);
    if (it == tables_.end()) return fail(AIR_KV_E_NOT_FOUND, "sequence not found (%u)", seq);
    std::vector<uint32_t> &blocks = it->second.physical_blocks;
    if (index < 0 || index >= (int64_t)blocks.size())
        return fail(AIR_KV_E_INVALID_ARG, "cow_block: index %lld outside the table", (long long)index);
    const uint32_t b = blocks[(size_t)index];
    uint32_t nid;
    if (!allocator_.cow_write(b, &nid)) return fail(AIR_KV_E_OOM, "out of memory — cow_write");
    blocks[(size_t)index] = nid;
    if (nid != b) set_own_fill(it->second, (size_t)index);
    *old_block = b;
    *new_block = nid;
    return AIR_KV_OK;
}

int SequenceManager::swap_out(uint32_t seq, std::vector<uint32_t> *blocks) {   // :353-362
    auto it = tables_.find(seq);
    if (it == tables_.end()) return fail(AIR_KV_E_NOT_FOUND, "sequence not found (%u)", seq);
    *blocks = it->second.physical_blocks;
    for (uint32_t b : *blocks) allocator_.release(b);
    it->second.physical_blocks.clear();
    return AIR_KV_OK;
}

int SequenceManager::swap_in(uint32_t seq, int32_t n_blocks, std::vector<uint32_t> *blocks) {
    // :369-381 (capacity is checked before the sequence, as in the reference)
    if (n_blocks < 0) return fail(AIR_KV_E_INVALID_ARG, "swap_in: negative block count");
    if (!allocator_.can_allocate(n_blocks)) return fail(AIR_KV_E_OOM, "out of memory — cannot swap in");
    auto it = tables_.find(seq);
    if (it == tables_.end()) return fail(AIR_KV_E_NOT_FOUND, "sequence not found (%u)", seq);
    blocks->clear();
    for (int32_t i = 0; i < n_blocks; ++i) {
        uint32_t b;
        allocator_.allocate(&b);
        blocks->push_back(b);
    }
    it->second.physical_blocks = *blocks;
    return AIR_KV_OK;
}

}  // namespace airkv
