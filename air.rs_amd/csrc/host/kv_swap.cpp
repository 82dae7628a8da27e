// Host-side swap manager (src/kv_swap.rs:22-121).
#include "kv_swap.hpp"

#include "status.hpp"

namespace airkv {

int KvSwapManager::evict(uint32_t seq, const ReadFn &read, std::vector<uint32_t> *released) {
    const BlockTable *t = seq_mgr_.table(seq);
    if (!t) return fail(AIR_KV_E_NOT_FOUND, "sequence not found (%u)", seq);
    // copy device -> host before the blocks are released (:63-68)
    std::vector<uint32_t> blocks = t->physical_blocks;
    std::vector<uint8_t> buf(blocks.size() * block_bytes_);
    for (size_t i = 0; i < blocks.size(); ++i)
        if (int rc = read(blocks[i], buf.data() + i * block_bytes_, block_bytes_))
            return rc < 0 ? rc : fail(AIR_KV_E_HIP, "evict: read of block %u failed (%d)", blocks[i], rc);
    int rc = seq_mgr_.swap_out(seq, released);
    if (rc) return rc;
    cpu_bytes_used_ += buf.size();
    cpu_store_[seq] = std::move(buf);
    return AIR_KV_OK;
}

int KvSwapManager::restore(uint32_t seq, const WriteFn &write, std::vector<uint32_t> *blocks) {
    auto it = cpu_store_.find(seq);
    if (it == cpu_store_.end()) return fail(AIR_KV_E_NOT_FOUND, "no evicted data for sequence %u", seq);
    // the buffer leaves the store before swap_in, so a failed swap_in drops
    // it, as in the reference (:87-89)
    std::vector<uint8_t> buf = std::move(it->second);
    cpu_store_.erase(it);
    size_t n = block_bytes_ ? buf.size() / block_bytes_ : 0;
    int rc = seq_mgr_.swap_in(seq, (int32_t)n, blocks);
    if (rc) return rc;
    for (size_t i = 0; i < blocks->size(); ++i) {
        if (int wrc = write((*blocks)[i], buf.data() + i * block_bytes_, block_bytes_)) {
            // back to the evicted state: the new blocks return to the free
            // list and the saved bytes to the store
            std::vector<uint32_t> undo;
            (void)seq_mgr_.swap_out(seq, &undo);
            cpu_store_[seq] = std::move(buf);
            blocks->clear();
            return wrc < 0 ? wrc : fail(AIR_KV_E_HIP, "restore: write of a block failed (%d)", wrc);
        }
    }
    cpu_bytes_used_ = cpu_bytes_used_ > buf.size() ? cpu_bytes_used_ - buf.size() : 0;
    return AIR_KV_OK;
}

int KvSwapManager::maybe_evict(uint32_t seq, int64_t free_threshold, const ReadFn &read, bool *evicted) {
    // :112-121
    *evicted = false;
    if (seq_mgr_.allocator().num_free_blocks() < free_threshold && !is_evicted(seq)) {
        std::vector<uint32_t> released;
        const int rc = evict(seq, read, &released);
        *evicted = rc == AIR_KV_OK;
        // an unknown sequence is "not evicted", as in the reference; a
        // failed device read is reported
        if (rc != AIR_KV_OK && rc != AIR_KV_E_NOT_FOUND) return rc;
    }
    return AIR_KV_OK;
}

}  // namespace airkv
