// extern "C" entry points for the host-side objects declared in air_kv.h.
#include <cstring>
#include <new>
#include <string>
#include <vector>

#include "air_kv.h"
#include "handles.hpp"
#include "status.hpp"

using airkv::fail;

namespace airkv {
std::string &last_error_slot() {
    static thread_local std::string msg;
    return msg;
}
}  // namespace airkv


namespace {

int check_geometry(int64_t capacity, int32_t block_size, const uint32_t *free_order) {
    if (capacity <= 0 || capacity > (int64_t)INT32_MAX)
        return fail(AIR_KV_E_INVALID_ARG, "capacity %lld out of range", (long long)capacity);
    if (block_size <= 0 || block_size > 4096)
        return fail(AIR_KV_E_INVALID_ARG, "block_size %d out of range", block_size);
    if (free_order) {
        std::vector<char> seen((size_t)capacity, 0);
        for (int64_t i = 0; i < capacity; ++i) {
            if ((int64_t)free_order[i] >= capacity || seen[free_order[i]])
                return fail(AIR_KV_E_INVALID_ARG, "free_order is not a permutation of 0..capacity-1");
            seen[free_order[i]] = 1;
        }
    }
    return AIR_KV_OK;
}

}  // namespace

extern "C" {

int air_kv_last_error(char *buf, size_t cap) {
    const std::string &m = airkv::last_error_slot();
    if (buf && cap) {
        size_t n = m.size() < cap - 1 ? m.size() : cap - 1;
        std::memcpy(buf, m.data(), n);
        buf[n] = '\0';
    }
    return (int)m.size();
}

// ---- BlockAllocator -------------------------------------------------------

int air_block_allocator_create(int64_t capacity, int32_t block_size, const uint32_t *free_order,
                               air_block_allocator **out) {
    if (!out) return fail(AIR_KV_E_INVALID_ARG, "out is NULL");
    if (int rc = check_geometry(capacity, block_size, free_order)) return rc;
    auto *a = new (std::nothrow) air_block_allocator{nullptr, true};
    if (!a) return fail(AIR_KV_E_OOM, "host allocation failed");
    a->impl = new (std::nothrow) airkv::BlockAllocator(capacity, block_size, free_order);
    if (!a->impl) { delete a; return fail(AIR_KV_E_OOM, "host allocation failed"); }
    *out = a;
    return AIR_KV_OK;
}

int air_block_allocator_destroy(air_block_allocator *a) {
    if (!a) return AIR_KV_OK;
    if (!a->owned) return fail(AIR_KV_E_STATE, "allocator is owned by a sequence manager");
    delete a->impl;
    delete a;
    return AIR_KV_OK;
}

#define CHECK_ALLOC(a) if (!(a)) return fail(AIR_KV_E_INVALID_ARG, "allocator is NULL")
#define CHECK_BLOCK(a, b) \
    if (!(a)->impl->valid(b)) return fail(AIR_KV_E_INVALID_ARG, "block %u outside the pool", (b))

int air_block_allocator_allocate(air_block_allocator *a, uint32_t *block) {
    CHECK_ALLOC(a);
    if (!block) return fail(AIR_KV_E_INVALID_ARG, "block is NULL");
    if (!a->impl->allocate(block)) return fail(AIR_KV_E_OOM, "pool exhausted");
    return AIR_KV_OK;
}

int air_block_allocator_share(air_block_allocator *a, uint32_t block) {
    CHECK_ALLOC(a);
    return a->impl->share(block);
}

int air_block_allocator_release(air_block_allocator *a, uint32_t block) {
    CHECK_ALLOC(a);
    return a->impl->release(block);
}

int air_block_allocator_ref_count(const air_block_allocator *a, uint32_t block, uint32_t *rc) {
    CHECK_ALLOC(a);
    CHECK_BLOCK(a, block);
    if (!rc) return fail(AIR_KV_E_INVALID_ARG, "rc is NULL");
    *rc = a->impl->ref_count(block);
    return AIR_KV_OK;
}

int64_t air_block_allocator_num_free(const air_block_allocator *a) {
    return a ? a->impl->num_free_blocks() : AIR_KV_E_INVALID_ARG;
}

int64_t air_block_allocator_num_used(const air_block_allocator *a) {
    return a ? a->impl->num_used_blocks() : AIR_KV_E_INVALID_ARG;
}

int air_block_allocator_cow_write(air_block_allocator *a, uint32_t block, uint32_t *out) {
    CHECK_ALLOC(a);
    CHECK_BLOCK(a, block);
    if (!out) return fail(AIR_KV_E_INVALID_ARG, "out is NULL");
    if (!a->impl->cow_write(block, out)) return fail(AIR_KV_E_OOM, "pool exhausted (cow_write)");
    return AIR_KV_OK;
}

int air_block_allocator_append_token(air_block_allocator *a, uint32_t block, int32_t *is_full) {
    CHECK_ALLOC(a);
    bool full = false;
    int rc = a->impl->append_token(block, &full);
    if (rc == AIR_KV_OK && is_full) *is_full = full ? 1 : 0;
    return rc;
}

int air_block_allocator_block_info(const air_block_allocator *a, uint32_t block,
                                   int32_t *num_tokens, int32_t *is_full) {
    CHECK_ALLOC(a);
    CHECK_BLOCK(a, block);
    const airkv::PhysicalBlock &b = a->impl->block(block);
    if (num_tokens) *num_tokens = b.num_tokens;
    if (is_full) *is_full = b.is_full ? 1 : 0;
    return AIR_KV_OK;
}

int air_block_allocator_can_allocate(const air_block_allocator *a, int64_t n) {
    CHECK_ALLOC(a);
    return a->impl->can_allocate(n) ? 1 : 0;
}

float air_block_allocator_utilization(const air_block_allocator *a) {
    return a ? a->impl->utilization() : -1.0f;
}

int64_t air_num_blocks_for_tokens(int64_t n_tokens, int32_t block_size) {
    if (block_size <= 0 || n_tokens < 0) return AIR_KV_E_INVALID_ARG;
    return airkv::BlockAllocator::num_blocks_for_tokens(n_tokens, block_size);
}

// ---- SequenceManager ------------------------------------------------------

int air_seq_manager_create(int64_t capacity, int32_t block_size, const uint32_t *free_order,
                           air_seq_manager **out) {
    if (!out) return fail(AIR_KV_E_INVALID_ARG, "out is NULL");
    if (int rc = check_geometry(capacity, block_size, free_order)) return rc;
    auto *m = new (std::nothrow) air_seq_manager{};
    if (!m) return fail(AIR_KV_E_OOM, "host allocation failed");
    m->impl = new (std::nothrow) airkv::SequenceManager(capacity, block_size, free_order);
    if (!m->impl) { delete m; return fail(AIR_KV_E_OOM, "host allocation failed"); }
    m->alloc_view = air_block_allocator{&m->impl->allocator(), false};
    m->owned = true;
    *out = m;
    return AIR_KV_OK;
}

int air_seq_manager_destroy(air_seq_manager *m) {
    if (!m) return AIR_KV_OK;
    if (!m->owned) return fail(AIR_KV_E_STATE, "sequence manager is owned by a swap manager");
    delete m->impl;
    delete m;
    return AIR_KV_OK;
}

air_block_allocator *air_seq_manager_allocator(air_seq_manager *m) {
    return m ? &m->alloc_view : nullptr;
}

#define CHECK_MGR(m) if (!(m)) return fail(AIR_KV_E_INVALID_ARG, "sequence manager is NULL")

int air_seq_create(air_seq_manager *m, uint32_t *seq) {
    CHECK_MGR(m);
    if (!seq) return fail(AIR_KV_E_INVALID_ARG, "seq is NULL");
    *seq = m->impl->create_sequence();
    return AIR_KV_OK;
}

int air_seq_append_token(air_seq_manager *m, uint32_t seq, uint32_t *block) {
    CHECK_MGR(m);
    uint32_t b;
    int rc = m->impl->append_token(seq, &b);
    if (rc == AIR_KV_OK && block) *block = b;
    return rc;
}

int air_seq_append_slots(air_seq_manager *m, uint32_t seq, int32_t n, int64_t *slots,
                         int32_t *n_done) {
    CHECK_MGR(m);
    if (n < 0 || (n > 0 && !slots)) return fail(AIR_KV_E_INVALID_ARG, "bad slot buffer");
    const int32_t bs = m->impl->block_size();
    int32_t i = 0;
    int rc = AIR_KV_OK;
    for (; i < n; ++i) {
        const airkv::BlockTable *t = m->impl->table(seq);
        if (!t) { rc = fail(AIR_KV_E_NOT_FOUND, "sequence not found (%u)", seq); break; }
        int64_t pos = t->num_tokens;
        uint32_t b;
        rc = m->impl->append_token(seq, &b);
        if (rc) break;
        slots[i] = (int64_t)b * bs + pos % bs;
    }
    if (n_done) *n_done = i;
    return rc;
}

int air_seq_fork(air_seq_manager *m, uint32_t parent, uint32_t *child) {
    CHECK_MGR(m);
    uint32_t c;
    int rc = m->impl->fork_sequence(parent, &c);
    if (rc == AIR_KV_OK && child) *child = c;
    return rc;
}

int air_seq_free(air_seq_manager *m, uint32_t seq) {
    CHECK_MGR(m);
    m->impl->free_sequence(seq);
    return AIR_KV_OK;
}

int air_seq_cow_last_block(air_seq_manager *m, uint32_t seq, uint32_t *old_block,
                           uint32_t *new_block) {
    CHECK_MGR(m);
    uint32_t o, nb;
    int rc = m->impl->cow_last_block(seq, &o, &nb);
    if (rc == AIR_KV_OK) {
        if (old_block) *old_block = o;
        if (new_block) *new_block = nb;
    }
    return rc;
}

int air_seq_truncate(air_seq_manager *m, uint32_t seq, int64_t n_tokens) {
    CHECK_MGR(m);
    return m->impl->truncate(seq, n_tokens);
}

int air_seq_cow_block(air_seq_manager *m, uint32_t seq, int64_t index, uint32_t *old_block,
                      uint32_t *new_block) {
    CHECK_MGR(m);
    uint32_t o, nb;
    int rc = m->impl->cow_block(seq, index, &o, &nb);
    if (rc == AIR_KV_OK) {
        if (old_block) *old_block = o;
        if (new_block) *new_block = nb;
    }
    return rc;
}

int air_seq_table(const air_seq_manager *m, uint32_t seq, uint32_t *blocks, int32_t cap,
                  int32_t *n_blocks, int64_t *n_tokens) {
    CHECK_MGR(m);
    const airkv::BlockTable *t = m->impl->table(seq);
    if (!t) return fail(AIR_KV_E_NOT_FOUND, "sequence not found (%u)", seq);
    int32_t n = (int32_t)t->physical_blocks.size();
    if (n_blocks) *n_blocks = n;
    if (n_tokens) *n_tokens = t->num_tokens;
    if (blocks) {
        if (cap < n) return fail(AIR_KV_E_INVALID_ARG, "table has %d blocks, cap %d", n, cap);
        for (int32_t i = 0; i < n; ++i) blocks[i] = t->physical_blocks[(size_t)i];
    }
    return AIR_KV_OK;
}

int air_seq_export_tables(const air_seq_manager *m, const uint32_t *seqs, int32_t n,
                          int32_t max_blocks, int32_t *tables, int32_t *seq_lens) {
    CHECK_MGR(m);
    if (n < 0 || max_blocks <= 0 || (n > 0 && (!seqs || !tables || !seq_lens)))
        return fail(AIR_KV_E_INVALID_ARG, "bad export buffers");
    const int32_t bs = m->impl->block_size();
    for (int32_t i = 0; i < n; ++i) {
        const airkv::BlockTable *t = m->impl->table(seqs[i]);
        if (!t) return fail(AIR_KV_E_NOT_FOUND, "sequence not found (%u)", seqs[i]);
        int64_t need = airkv::BlockAllocator::num_blocks_for_tokens(t->num_tokens, bs);
        if ((int64_t)t->physical_blocks.size() < need)
            return fail(AIR_KV_E_STATE, "sequence %u holds %zu blocks for %lld tokens (swapped out?)",
                        seqs[i], t->physical_blocks.size(), (long long)t->num_tokens);
        if ((int64_t)t->physical_blocks.size() > max_blocks)
            return fail(AIR_KV_E_INVALID_ARG, "sequence %u needs %zu table entries, max_blocks %d",
                        seqs[i], t->physical_blocks.size(), max_blocks);
        if (t->num_tokens > (int64_t)INT32_MAX) return fail(AIR_KV_E_INVALID_ARG, "sequence too long");
        int32_t *row = tables + (size_t)i * max_blocks;
        for (int32_t j = 0; j < max_blocks; ++j)
            row[j] = j < (int32_t)t->physical_blocks.size() ? (int32_t)t->physical_blocks[(size_t)j] : -1;
        seq_lens[i] = (int32_t)t->num_tokens;
    }
    return AIR_KV_OK;
}

int64_t air_seq_num_sequences(const air_seq_manager *m) {
    return m ? m->impl->num_sequences() : AIR_KV_E_INVALID_ARG;
}

int air_seq_can_schedule(const air_seq_manager *m) {
    CHECK_MGR(m);
    return m->impl->can_schedule() ? 1 : 0;
}

int air_seq_swap_out(air_seq_manager *m, uint32_t seq, uint32_t *blocks, int32_t cap,
                     int32_t *n_blocks) {
    CHECK_MGR(m);
    const airkv::BlockTable *t = m->impl->table(seq);
    if (t && blocks && (int64_t)t->physical_blocks.size() > cap)
        return fail(AIR_KV_E_INVALID_ARG, "swap_out: cap %d below %zu blocks", cap, t->physical_blocks.size());
    std::vector<uint32_t> out;
    int rc = m->impl->swap_out(seq, &out);
    if (rc) return rc;
    if (n_blocks) *n_blocks = (int32_t)out.size();
    if (blocks && !out.empty()) std::memcpy(blocks, out.data(), out.size() * sizeof(uint32_t));
    return AIR_KV_OK;
}

int air_seq_swap_in(air_seq_manager *m, uint32_t seq, int32_t n_blocks, uint32_t *blocks) {
    CHECK_MGR(m);
    std::vector<uint32_t> out;
    int rc = m->impl->swap_in(seq, n_blocks, &out);
    if (rc) return rc;
    if (blocks && !out.empty()) std::memcpy(blocks, out.data(), out.size() * sizeof(uint32_t));
    return AIR_KV_OK;
}

// ---- KvSwapManager ----------------------------------------------------------

int air_kv_swap_create(int64_t capacity, int32_t block_size, size_t block_bytes, air_kv_swap **out) {
    if (!out) return fail(AIR_KV_E_INVALID_ARG, "out is NULL");
    if (int rc = check_geometry(capacity, block_size, nullptr)) return rc;
    if (block_bytes == 0) return fail(AIR_KV_E_INVALID_ARG, "block_bytes is 0");
    auto *s = new (std::nothrow) air_kv_swap(capacity, block_size, block_bytes);
    if (!s) return fail(AIR_KV_E_OOM, "host allocation failed");
    s->mgr_view.impl = &s->impl.seq_mgr();
    s->mgr_view.alloc_view = air_block_allocator{&s->impl.seq_mgr().allocator(), false};
    s->mgr_view.owned = false;
    *out = s;
    return AIR_KV_OK;
}

int air_kv_swap_destroy(air_kv_swap *s) {
    delete s;
    return AIR_KV_OK;
}

air_seq_manager *air_kv_swap_seq_manager(air_kv_swap *s) { return s ? &s->mgr_view : nullptr; }

int air_kv_swap_evict(air_kv_swap *s, uint32_t seq, air_kv_block_read_fn read, void *ctx,
                      uint32_t *released, int32_t cap, int32_t *n_released) {
    if (!s || !read) return fail(AIR_KV_E_INVALID_ARG, "swap manager or read callback is NULL");
    const airkv::BlockTable *t = s->impl.seq_mgr().table(seq);
    if (t && released && (int64_t)t->physical_blocks.size() > cap)
        return fail(AIR_KV_E_INVALID_ARG, "evict: cap %d below %zu blocks", cap, t->physical_blocks.size());
    std::vector<uint32_t> out;
    int rc = s->impl.evict(seq, [&](uint32_t b, uint8_t *dst, size_t n) { return read(ctx, b, dst, n); }, &out);
    if (rc) return rc;
    if (n_released) *n_released = (int32_t)out.size();
    if (released && !out.empty()) std::memcpy(released, out.data(), out.size() * sizeof(uint32_t));
    return AIR_KV_OK;
}

int air_kv_swap_restore(air_kv_swap *s, uint32_t seq, air_kv_block_write_fn write, void *ctx,
                        uint32_t *blocks, int32_t cap, int32_t *n_blocks) {
    if (!s || !write) return fail(AIR_KV_E_INVALID_ARG, "swap manager or write callback is NULL");
    // the id buffer is checked before anything changes
    const int64_t need = s->impl.evicted_blocks(seq);
    if (blocks && need > cap)
        return fail(AIR_KV_E_INVALID_ARG, "restore: cap %d below %lld blocks", cap, (long long)need);
    std::vector<uint32_t> out;
    int rc = s->impl.restore(
        seq, [&](uint32_t b, const uint8_t *src, size_t n) { return write(ctx, b, src, n); }, &out);
    if (rc) return rc;
    if (n_blocks) *n_blocks = (int32_t)out.size();
    if (blocks && !out.empty()) std::memcpy(blocks, out.data(), out.size() * sizeof(uint32_t));
    return AIR_KV_OK;
}

int air_kv_swap_is_evicted(const air_kv_swap *s, uint32_t seq) {
    if (!s) return fail(AIR_KV_E_INVALID_ARG, "swap manager is NULL");
    return s->impl.is_evicted(seq) ? 1 : 0;
}

int64_t air_kv_swap_evicted_count(const air_kv_swap *s) {
    return s ? s->impl.evicted_count() : AIR_KV_E_INVALID_ARG;
}

int64_t air_kv_swap_cpu_bytes_used(const air_kv_swap *s) {
    return s ? s->impl.cpu_bytes_used() : AIR_KV_E_INVALID_ARG;
}

int air_kv_swap_maybe_evict(air_kv_swap *s, uint32_t seq, int64_t free_threshold,
                            air_kv_block_read_fn read, void *ctx, int32_t *evicted) {
    if (!s || !read) return fail(AIR_KV_E_INVALID_ARG, "swap manager or read callback is NULL");
    bool e = false;
    int rc = s->impl.maybe_evict(
        seq, free_threshold, [&](uint32_t b, uint8_t *dst, size_t n) { return read(ctx, b, dst, n); }, &e);
    if (evicted) *evicted = e ? 1 : 0;
    return rc;
}

}  // extern "C"
