// Host-side swap manager: the C++ counterpart of KvSwapManager
// (src/kv_swap.rs:22-121).  The device copy stays the caller's business, as in
// the reference: evict / restore take read / write callbacks (the reference's
// gpu_read / gpu_write closures, :55-57 and :83-86).
#pragma once

#include <cstddef>
#include <cstdint>
#include <functional>
#include <unordered_map>
#include <vector>

#include "paged_attention.hpp"

namespace airkv {

class KvSwapManager {
public:
    // The copies return AIR_KV_OK or a negative status.  A failed read
    // leaves the sequence resident and unchanged; a failed write puts the
    // restored sequence back into the evicted state with its saved bytes.
    // (The reference's closures return nothing, so a failed device copy
    // there would be released or dropped unnoticed.)
    using ReadFn = std::function<int(uint32_t block, uint8_t *dst, size_t bytes)>;
    using WriteFn = std::function<int(uint32_t block, const uint8_t *src, size_t bytes)>;

    KvSwapManager(int64_t capacity, int32_t block_size, size_t block_bytes)
        : seq_mgr_(capacity, block_size, nullptr), block_bytes_(block_bytes) {}

    SequenceManager &seq_mgr() { return seq_mgr_; }
    int evict(uint32_t seq, const ReadFn &read, std::vector<uint32_t> *released);   // :55-74
    int restore(uint32_t seq, const WriteFn &write, std::vector<uint32_t> *blocks); // :83-98
    bool is_evicted(uint32_t seq) const { return cpu_store_.count(seq) != 0; }
    // blocks a restore of `seq` will allocate (0 when nothing is stored)
    int64_t evicted_blocks(uint32_t seq) const {
        auto it = cpu_store_.find(seq);
        return it == cpu_store_.end() || !block_bytes_ ? 0 : (int64_t)(it->second.size() / block_bytes_);
    }
    int64_t evicted_count() const { return (int64_t)cpu_store_.size(); }
    int64_t cpu_bytes_used() const { return (int64_t)cpu_bytes_used_; }
    int maybe_evict(uint32_t seq, int64_t free_threshold, const ReadFn &read, bool *evicted);

private:
    SequenceManager seq_mgr_;
    std::unordered_map<uint32_t, std::vector<uint8_t>> cpu_store_;
    size_t block_bytes_;
    size_t cpu_bytes_used_ = 0;
};

}  // namespace airkv
