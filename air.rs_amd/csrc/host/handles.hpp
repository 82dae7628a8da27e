// Definitions of the opaque C handles of air_kv.h that wrap host objects,
// shared by the translation units that implement their entry points.
#pragma once

#include "air_kv.h"
#include "kv_swap.hpp"
#include "paged_attention.hpp"

struct air_block_allocator {
    airkv::BlockAllocator *impl;
    bool owned;
};
struct air_seq_manager {
    airkv::SequenceManager *impl;
    air_block_allocator alloc_view;
    bool owned;
};
struct air_kv_swap {
    airkv::KvSwapManager impl;
    air_seq_manager mgr_view;
    air_kv_swap(int64_t c, int32_t bs, size_t bb) : impl(c, bs, bb) {}
};
