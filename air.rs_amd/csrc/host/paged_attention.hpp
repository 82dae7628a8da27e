// Host-side paged block manager: the C++ counterpart of the reference's
// BlockAllocator / BlockTable / SequenceManager (src/paged_attention.rs:89-381).
//
// Semantics follow the reference call for call (FIFO free list with
// pop_front / push_back, refcounts, copy-on-write metadata, allocate on a block
// boundary), so block tables come out identical for identical call sequences.
// Differences, all on paths where the reference panics or corrupts state:
//  * the page size is a runtime value (the reference's BLOCK_SIZE const, :40);
//  * release of a block whose refcount is already 0 is rejected (the
//    reference pushes the id onto the free list a second time, :129-135);
//  * append to a full block returns an error (the reference asserts, :172);
//  * the private block copy-on-write makes for a sequence gets that
//    sequence's own fill, not the shared block's (set_own_fill);
//  * ids outside the pool are rejected (the reference indexes out of bounds).
#pragma once

#include <cstddef>
#include <cstdint>
#include <deque>
#include <unordered_map>
#include <vector>

namespace airkv {

struct PhysicalBlock {       // src/paged_attention.rs:63-69
    uint32_t id = 0;
    int32_t num_tokens = 0;
    bool is_full = false;
};

class BlockAllocator {       // src/paged_attention.rs:89-196
public:
    BlockAllocator(int64_t capacity, int32_t block_size, const uint32_t *free_order);

    bool allocate(uint32_t *out);                 // pop_front; false = None (OOM)
    int share(uint32_t id);                        // AIR_KV_OK / AIR_KV_E_INVALID_ARG
    int release(uint32_t id);                      // ... / AIR_KV_E_STATE on rc == 0
    uint32_t ref_count(uint32_t id) const { return ref_counts_[id]; }
    int64_t num_free_blocks() const { return (int64_t)free_blocks_.size(); }
    int64_t num_used_blocks() const { return total_blocks_ - (int64_t)free_blocks_.size(); }
    // cow_write: 1 = ok (out set), 0 = OOM
    bool cow_write(uint32_t id, uint32_t *out);
    int append_token(uint32_t id, bool *is_full);  // AIR_KV_E_STATE when already full
    bool can_allocate(int64_t n) const { return (int64_t)free_blocks_.size() >= n; }
    static int64_t num_blocks_for_tokens(int64_t n, int32_t bs) { return (n + bs - 1) / bs; }
    float utilization() const { return (float)num_used_blocks() / (float)total_blocks_; }

    // Fill metadata of a block this caller owns alone (truncation of a sequence).
    void set_fill(uint32_t id, int32_t num_tokens) {
        blocks_[id].num_tokens = num_tokens;
        blocks_[id].is_full = num_tokens == block_size_;
    }

    bool valid(uint32_t id) const { return (int64_t)id < total_blocks_; }
    const PhysicalBlock &block(uint32_t id) const { return blocks_[id]; }
    int64_t total_blocks() const { return total_blocks_; }
    int32_t block_size() const { return block_size_; }

private:
    std::vector<PhysicalBlock> blocks_;
    std::vector<uint32_t> ref_counts_;
    std::deque<uint32_t> free_blocks_;
    int64_t total_blocks_;
    int32_t block_size_;
};

struct BlockTable {          // src/paged_attention.rs:202-235
    uint32_t seq_id = 0;
    std::vector<uint32_t> physical_blocks;
    int64_t num_tokens = 0;
    int64_t last_block_offset(int32_t bs) const { return num_tokens % bs; }
};

class SequenceManager {      // src/paged_attention.rs:243-382
public:
    SequenceManager(int64_t capacity, int32_t block_size, const uint32_t *free_order)
        : allocator_(capacity, block_size, free_order) {}

    BlockAllocator &allocator() { return allocator_; }
    const BlockAllocator &allocator() const { return allocator_; }
    int32_t block_size() const { return allocator_.block_size(); }

    uint32_t create_sequence();
    int append_token(uint32_t seq, uint32_t *block);       // NOT_FOUND / OOM
    int fork_sequence(uint32_t parent, uint32_t *child);   // NOT_FOUND
    void free_sequence(uint32_t seq);
    const BlockTable *table(uint32_t seq) const;
    int cow_last_block(uint32_t seq, uint32_t *old_block, uint32_t *new_block);
    int64_t num_sequences() const { return (int64_t)tables_.size(); }
    bool can_schedule() const { return allocator_.can_allocate(1); }
    int swap_out(uint32_t seq, std::vector<uint32_t> *blocks);
    int swap_in(uint32_t seq, int32_t n_blocks, std::vector<uint32_t> *blocks);

    // Extensions the reference has no counterpart for (its dense cache rolls
    // back with Tensor::narrow, src/kv_cache.rs:364-383):
    //  * truncate: keep the first n_tokens tokens, release the blocks past
    //    them (FIFO push_back, like free_sequence) and, when the new last
    //    block is owned by this sequence alone, set its fill to what remains.
    //  * cow_block: copy-on-write of the block at table index `index` (the
    //    reference's cow_last_block generalised to any index).
    int truncate(uint32_t seq, int64_t n_tokens);
    int cow_block(uint32_t seq, int64_t index, uint32_t *old_block, uint32_t *new_block);
    //  * undo_cow: puts old_block back at table index idx in place of the
    //    private copy new_block that cow_block made (the copy returns to the
    //    free list), for a caller whose device copy could not be issued.
    void undo_cow(uint32_t seq, size_t idx, uint32_t old_block, uint32_t new_block);

private:
    void set_own_fill(const BlockTable &t, size_t idx);

    BlockAllocator allocator_;
    std::unordered_map<uint32_t, BlockTable> tables_;
    uint32_t next_seq_id_ = 0;
};

}  // namespace airkv
