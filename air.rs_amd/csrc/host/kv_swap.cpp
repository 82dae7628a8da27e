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
    for (size_t i = 0; i < blocks.size(); ++i) read(blocks[i], buf.data() + i * block_bytes_, block_bytes_);
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
    for (size_t i = 0; i < blocks->size(); ++i)
        write((*blocks)[i], buf.data() + i * block_bytes_, block_bytes_);
    cpu_bytes_used_ = cpu_bytes_used_ > buf.size() ? cpu_bytes_used_ - buf.size() : 0;
    return AIR_KV_OK;
}

int KvSwapManager::maybe_evict(uint32_t seq, int64_t free_threshold, const ReadFn &read, bool *evicted) {
    // :112-121
    *evicted = false;
    if (seq_mgr_.allocator().num_free_blocks() < free_threshold && !is_evicted(seq)) {
        std::vector<uint32_t> released;
        *evicted = evict(seq, read, &released) == AIR_KV_OK;
    }
    return AIR_KV_OK;
}

}  // namespace airkv
