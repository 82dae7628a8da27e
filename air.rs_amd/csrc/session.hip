// The paged SessionKvCache (src/kv_cache.rs:431-446): one sequence of a
// SequenceManager whose block table is shared by the per-layer pools.
//
// The reference's KvCacheManager keeps each layer as a dense tensor in host
// memory and copies it to the GPU every step (save_layer / load_layer,
// src/kv_cache.rs:244-339); here a layer's tokens stay in its device pool and
// a step only writes the new rows.  Host bookkeeping (block allocation,
// copy-on-write, truncation) happens in the sequence manager; device work is
// the append / gather / block-copy kernels, ordered on the caller's stream.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <new>
#include <vector>

#include "air_kv.h"
#include "host/handles.hpp"
#include "host/status.hpp"
#include "pool.hpp"

using airkv::fail;

struct air_kv_session {
    air_seq_manager *mgr = nullptr;
    std::vector<air_kv_pool *> pools;
    uint32_t seq = 0;
    std::vector<int64_t> len;          // tokens stored per layer
    // Staging for the small index arrays the kernels read (slots, block
    // lists, a table row): a pinned host buffer copied into a device buffer
    // on the caller's stream.  `done` is recorded after the last launch that
    // read the device buffer; both buffers are reused only once it completed.
    char *h_stage = nullptr;
    char *d_stage = nullptr;
    size_t stage_cap = 0;
    hipEvent_t done = nullptr;
    bool pending = false;
};

namespace {

int hip_fail(hipError_t e, const char *what) {
    return fail(AIR_KV_E_HIP, "%s: %s", what, hipGetErrorString(e));
}

airkv::SequenceManager &manager(air_kv_session *s) { return *s->mgr->impl; }

int wait_stage(air_kv_session *s) {
    if (!s->pending) return AIR_KV_OK;
    hipError_t e = hipEventSynchronize(s->done);
    if (e != hipSuccess) return hip_fail(e, "session staging wait");
    s->pending = false;
    return AIR_KV_OK;
}

// Makes the staging buffers hold at least `bytes` (waiting for the last
// launch that read them first).  After it succeeds, stage() of up to `bytes`
// can fail only in the copy itself.
int reserve_stage(air_kv_session *s, size_t bytes) {
    if (int rc = wait_stage(s)) return rc;
    if (bytes > s->stage_cap) {
        size_t cap = std::max<size_t>(bytes, 2 * s->stage_cap);
        cap = std::max<size_t>(cap, 4096);
        (void)hipHostFree(s->h_stage);
        (void)hipFree(s->d_stage);
        s->h_stage = nullptr;
        s->d_stage = nullptr;
        s->stage_cap = 0;
        hipError_t e = hipHostMalloc((void **)&s->h_stage, cap, hipHostMallocDefault);
        if (e != hipSuccess) return hip_fail(e, "session staging hipHostMalloc");
        e = hipMalloc((void **)&s->d_stage, cap);
        if (e != hipSuccess) return hip_fail(e, "session staging hipMalloc");
        s->stage_cap = cap;
    }
    return AIR_KV_OK;
}

// Copies `bytes` of host data to the device staging buffer on `st`.
int stage(air_kv_session *s, hipStream_t st, const void *src, size_t bytes, void **dev) {
    if (int rc = reserve_stage(s, bytes)) return rc;
    std::memcpy(s->h_stage, src, bytes);
    hipError_t e = hipMemcpyAsync(s->d_stage, s->h_stage, bytes, hipMemcpyHostToDevice, st);
    if (e != hipSuccess) return hip_fail(e, "session staging copy");
    *dev = s->d_stage;
    return AIR_KV_OK;
}

int mark_staged(air_kv_session *s, hipStream_t st) {
    hipError_t e = hipEventRecord(s->done, st);
    if (e != hipSuccess) return hip_fail(e, "session staging event");
    s->pending = true;
    return AIR_KV_OK;
}

int check_layer(const air_kv_session *s, int32_t layer) {
    if (!s) return fail(AIR_KV_E_INVALID_ARG, "session is NULL");
    if (layer < 0 || layer >= (int32_t)s->pools.size())
        return fail(AIR_KV_E_INVALID_ARG, "layer %d outside 0..%d", layer, (int)s->pools.size() - 1);
    return AIR_KV_OK;
}

// The table holds max(len) tokens: release what no layer uses any more.
int shrink_table(air_kv_session *s) {
    int64_t keep = 0;
    for (int64_t l : s->len) keep = std::max(keep, l);
    return manager(s).truncate(s->seq, keep);
}

int64_t row_elems(const air_kv_pool *p) { return (int64_t)p->desc.n_kv_heads * p->desc.head_dim; }

}  // namespace

extern "C" {

int air_kv_session_create(air_seq_manager *mgr, air_kv_pool *const *layer_pools, int32_t n_layers,
                          air_kv_session **out) {
    if (!mgr || !out || n_layers <= 0 || !layer_pools)
        return fail(AIR_KV_E_INVALID_ARG, "session needs a manager, >= 1 layer pools and an out pointer");
    const airkv::SequenceManager &m = *mgr->impl;
    for (int32_t l = 0; l < n_layers; ++l) {
        const air_kv_pool *p = layer_pools[l];
        if (!p) return fail(AIR_KV_E_INVALID_ARG, "layer %d pool is NULL", l);
        if (p->desc.block_size != m.block_size())
            return fail(AIR_KV_E_INVALID_ARG, "layer %d pool block_size %d != manager's %d", l,
                        p->desc.block_size, m.block_size());
        if (p->desc.num_blocks < m.allocator().total_blocks())
            return fail(AIR_KV_E_INVALID_ARG, "layer %d pool holds %lld blocks < manager capacity %lld", l,
                        (long long)p->desc.num_blocks, (long long)m.allocator().total_blocks());
    }
    auto *s = new (std::nothrow) air_kv_session();
    if (!s) return fail(AIR_KV_E_OOM, "host allocation failed");
    hipError_t e = hipEventCreateWithFlags(&s->done, hipEventDisableTiming);
    if (e != hipSuccess) {
        delete s;
        return hip_fail(e, "hipEventCreate");
    }
    s->mgr = mgr;
    s->pools.assign(layer_pools, layer_pools + n_layers);
    s->len.assign((size_t)n_layers, 0);
    s->seq = mgr->impl->create_sequence();
    *out = s;
    return AIR_KV_OK;
}

int air_kv_session_destroy(air_kv_session *s) {
    if (!s) return AIR_KV_OK;
    (void)wait_stage(s);
    s->mgr->impl->free_sequence(s->seq);
    (void)hipHostFree(s->h_stage);
    (void)hipFree(s->d_stage);
    (void)hipEventDestroy(s->done);
    delete s;
    return AIR_KV_OK;
}

int air_kv_session_fork(air_kv_session *parent, air_kv_session **out) {
    if (!parent || !out) return fail(AIR_KV_E_INVALID_ARG, "session or out is NULL");
    auto *s = new (std::nothrow) air_kv_session();
    if (!s) return fail(AIR_KV_E_OOM, "host allocation failed");
    hipError_t e = hipEventCreateWithFlags(&s->done, hipEventDisableTiming);
    if (e != hipSuccess) {
        delete s;
        return hip_fail(e, "hipEventCreate");
    }
    uint32_t child;
    if (int rc = manager(parent).fork_sequence(parent->seq, &child)) {
        (void)hipEventDestroy(s->done);
        delete s;
        return rc;
    }
    s->mgr = parent->mgr;
    s->pools = parent->pools;
    s->len = parent->len;
    s->seq = child;
    *out = s;
    return AIR_KV_OK;
}

int air_kv_session_seq_id(const air_kv_session *s, uint32_t *seq) {
    if (!s || !seq) return fail(AIR_KV_E_INVALID_ARG, "session or seq is NULL");
    *seq = s->seq;
    return AIR_KV_OK;
}

int air_kv_session_seq_len(const air_kv_session *s, int32_t layer, int64_t *len) {
    if (int rc = check_layer(s, layer)) return rc;
    if (!len) return fail(AIR_KV_E_INVALID_ARG, "len is NULL");
    *len = s->len[(size_t)layer];
    return AIR_KV_OK;
}

int air_kv_session_append(air_kv_session *s, void *stream, int32_t layer, const float *k,
                          const float *v, int64_t n_new) {
    if (int rc = check_layer(s, layer)) return rc;
    if (n_new < 0 || n_new > INT32_MAX) return fail(AIR_KV_E_INVALID_ARG, "n_new %lld out of range", (long long)n_new);
    if (n_new == 0) return AIR_KV_OK;
    if (!k || !v) return fail(AIR_KV_E_INVALID_ARG, "k or v is NULL");
    hipStream_t st = (hipStream_t)stream;
    airkv::SequenceManager &m = manager(s);
    const int32_t bs = m.block_size();
    const airkv::BlockTable *t = m.table(s->seq);
    if (!t) return fail(AIR_KV_E_NOT_FOUND, "sequence not found (%u)", s->seq);
    const int64_t p0 = s->len[(size_t)layer], p1 = p0 + n_new;
    const int64_t had = t->num_tokens;
    const int64_t nb = (int64_t)t->physical_blocks.size();
    if (nb < (had + bs - 1) / bs)
        return fail(AIR_KV_E_STATE, "sequence %u holds %lld blocks for %lld tokens (swapped out?)", s->seq,
                    (long long)nb, (long long)had);

    // Everything that can fail without a HIP error is checked before the
    // table changes: blocks that already exist and will be written are
    // copied first if another sequence shares them, blocks past the table
    // are allocated, and both draw on the free list; the staging buffers
    // are sized for the slots and the copy lists.
    const int64_t last_written = std::min<int64_t>((p1 - 1) / bs, nb - 1);
    int64_t n_shared = 0;
    for (int64_t i = p0 / bs; i <= last_written; ++i)
        if (m.allocator().ref_count(t->physical_blocks[(size_t)i]) > 1) ++n_shared;
    const int64_t need = n_shared + std::max<int64_t>(0, (p1 + bs - 1) / bs - nb);
    if (!m.allocator().can_allocate(need)) return fail(AIR_KV_E_OOM, "out of memory — no free blocks");
    const size_t stage_bytes = (size_t)n_new * 8 + (size_t)n_shared * 8;
    if (int rc = reserve_stage(s, stage_bytes)) return rc;

    // Table changes: copy-on-write of shared blocks, then the new tokens
    // (allocating on block boundaries).  Neither can fail after the checks
    // above; `undo` puts the table back if a later step does.
    std::vector<int32_t> cow_src, cow_dst;
    std::vector<int64_t> cow_idx;
    auto undo = [&]() {
        m.truncate(s->seq, had);
        for (size_t j = cow_idx.size(); j-- > 0;)
            m.undo_cow(s->seq, (size_t)cow_idx[j], (uint32_t)cow_src[j], (uint32_t)cow_dst[j]);
    };
    for (int64_t i = p0 / bs; i <= last_written; ++i) {
        const uint32_t b = m.table(s->seq)->physical_blocks[(size_t)i];
        if (m.allocator().ref_count(b) <= 1) continue;
        uint32_t o, nbk;
        if (int rc = m.cow_block(s->seq, i, &o, &nbk)) {
            undo();
            return rc;
        }
        cow_idx.push_back(i);
        cow_src.push_back((int32_t)o);
        cow_dst.push_back((int32_t)nbk);
    }
    for (int64_t p = had; p < p1; ++p) {
        uint32_t b;
        if (int rc = m.append_token(s->seq, &b)) {
            undo();
            return rc;
        }
    }
    t = m.table(s->seq);
    // Stage slots (int64) then the copy lists (int32) in one transfer.
    const size_t n_cow = cow_src.size();
    std::vector<char> host(stage_bytes);
    int64_t *slots = reinterpret_cast<int64_t *>(host.data());
    for (int64_t p = p0; p < p1; ++p)
        slots[p - p0] = (int64_t)t->physical_blocks[(size_t)(p / bs)] * bs + p % bs;
    int32_t *lists = reinterpret_cast<int32_t *>(host.data() + (size_t)n_new * 8);
    std::copy(cow_src.begin(), cow_src.end(), lists);
    std::copy(cow_dst.begin(), cow_dst.end(), lists + n_cow);
    void *dev;
    if (int rc = stage(s, st, host.data(), host.size(), &dev)) {
        undo();
        return rc;
    }
    const int64_t *d_slots = reinterpret_cast<const int64_t *>(dev);
    const int32_t *d_lists = reinterpret_cast<const int32_t *>((char *)dev + (size_t)n_new * 8);
    int rc = AIR_KV_OK;
    if (n_cow) {
        for (air_kv_pool *p : s->pools)
            if ((rc = air_kv_copy_blocks(p, stream, d_lists, d_lists + n_cow, (int32_t)n_cow))) break;
    }
    if (!rc) rc = air_kv_append(s->pools[(size_t)layer], stream, k, v, d_slots, (int32_t)n_new);
    const int rc2 = mark_staged(s, st);
    if (rc || rc2) {
        // The old blocks still hold their pages (copies only read them), so
        // the table goes back to them and the new blocks to the free list.
        undo();
        return rc ? rc : rc2;
    }
    s->len[(size_t)layer] = p1;
    return AIR_KV_OK;
}

int air_kv_session_save(air_kv_session *s, void *stream, int32_t layer, const float *k,
                        const float *v, int64_t n_tokens) {
    if (int rc = check_layer(s, layer)) return rc;
    if (n_tokens < 0) return fail(AIR_KV_E_INVALID_ARG, "n_tokens < 0");
    const int64_t have = s->len[(size_t)layer];
    if (n_tokens <= have) {
        s->len[(size_t)layer] = n_tokens;
        return shrink_table(s);
    }
    if (!k || !v) return fail(AIR_KV_E_INVALID_ARG, "k or v is NULL");
    const int64_t row = row_elems(s->pools[(size_t)layer]);
    return air_kv_session_append(s, stream, layer, k + have * row, v + have * row, n_tokens - have);
}

int air_kv_session_load(air_kv_session *s, void *stream, int32_t layer, void *out_k, void *out_v,
                        int32_t out_dtype) {
    if (int rc = check_layer(s, layer)) return rc;
    const int64_t n = s->len[(size_t)layer];
    if (n == 0) return AIR_KV_OK;
    if (n > INT32_MAX) return fail(AIR_KV_E_INVALID_ARG, "layer too long for one gather");
    const airkv::BlockTable *t = manager(s).table(s->seq);
    if (!t) return fail(AIR_KV_E_NOT_FOUND, "sequence not found (%u)", s->seq);
    const int32_t bs = manager(s).block_size();
    const int32_t nblk = (int32_t)((n + bs - 1) / bs);
    // [offset int64][len int32][pad][table int32 x nblk]
    std::vector<char> host(16 + (size_t)nblk * 4);
    const int64_t off = 0;
    const int32_t len32 = (int32_t)n;
    std::memcpy(host.data(), &off, 8);
    std::memcpy(host.data() + 8, &len32, 4);
    for (int32_t i = 0; i < nblk; ++i) {
        const int32_t b = (int32_t)t->physical_blocks[(size_t)i];
        std::memcpy(host.data() + 16 + (size_t)i * 4, &b, 4);
    }
    void *dev;
    hipStream_t st = (hipStream_t)stream;
    if (int rc = stage(s, st, host.data(), host.size(), &dev)) return rc;
    const char *d = (const char *)dev;
    int rc = air_kv_gather(s->pools[(size_t)layer], stream, reinterpret_cast<const int32_t *>(d + 16),
                           reinterpret_cast<const int32_t *>(d + 8), reinterpret_cast<const int64_t *>(d), 1,
                           nblk, out_k, out_v, out_dtype, AIR_KV_LAYOUT_TOKEN_MAJOR);
    if (int rc2 = mark_staged(s, st)) return rc ? rc : rc2;
    return rc;
}

int air_kv_session_clear(air_kv_session *s) {
    if (!s) return fail(AIR_KV_E_INVALID_ARG, "session is NULL");
    std::fill(s->len.begin(), s->len.end(), 0);
    return shrink_table(s);
}

int air_kv_session_truncate_to(air_kv_session *s, int64_t pos) {
    if (!s) return fail(AIR_KV_E_INVALID_ARG, "session is NULL");
    if (pos < 0) return fail(AIR_KV_E_INVALID_ARG, "pos < 0");
    for (int64_t &l : s->len) l = std::min(l, pos);
    return shrink_table(s);
}

int air_kv_session_memory_usage(const air_kv_session *s, size_t *bytes) {
    if (!s || !bytes) return fail(AIR_KV_E_INVALID_ARG, "session or bytes is NULL");
    const airkv::BlockTable *t = s->mgr->impl->table(s->seq);
    const size_t nblk = t ? t->physical_blocks.size() : 0;
    size_t per_block = 0;
    for (const air_kv_pool *p : s->pools) per_block += p->block_bytes;
    *bytes = nblk * per_block;
    return AIR_KV_OK;
}

}  // extern "C"
