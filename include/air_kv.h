/*
 * air_kv.h -- C ABI of the MI355X-native paged KV-cache path.
 *
 * The reference (SunayHegde2006/Air.rs) has no FFI for this path; its seams
 * are Rust types and traits.  Each entry point below names the reference
 * interface it replaces.  A Rust caller binds these with `extern "C"` (see
 * the binding in the integration notes); this build's tests bind them with
 * ctypes.
 *
 * Conventions
 *  - Every function returns an int status: AIR_KV_OK (0) or a negative
 *    AIR_KV_E_* code.  The message of the last failure on the calling thread
 *    is available from air_kv_last_error().  The library never aborts.
 *  - Device-side entry points take raw device pointers, plain sizes and a
 *    `void *stream` (a hipStream_t; NULL = the default stream).  They only
 *    enqueue work and return; nothing synchronises unless documented.
 *  - A pool owns all of its device memory (pages and scales).  The caller
 *    owns every buffer it passes in.
 *  - Host-side objects (allocator, sequence manager, swap manager) are not
 *    thread-safe, as in the reference (src/paged_attention.rs:86-87); callers
 *    serialise access, as the reference's generator does with a Mutex
 *    (src/generator.rs:109-112).
 *
 * Device layout of a pool (one transformer layer):
 *   k_pages, v_pages   : [num_blocks][n_kv_heads][block_size][head_dim]
 *   k_scales, v_scales : [num_blocks][n_kv_heads][block_size][head_dim/scale_group]
 *                        f32, only for AIR_KV_INT8 / AIR_KV_FP8 pools
 *   slot = block * block_size + offset          (src/paged_attention.rs:216-234)
 * One block's bytes (K + V + scales) equal the reference's page size formula
 * n_heads * head_dim * 2 * dtype_bytes * BLOCK_SIZE (src/kv_swap.rs:37-38)
 * plus the scales of quantized pools.
 */
#ifndef AIR_KV_H
#define AIR_KV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
#define AIR_KV_OK 0
#define AIR_KV_E_INVALID_ARG (-1) /* bad pointer, size, dtype or shape */
#define AIR_KV_E_OOM (-2)         /* no free blocks / device allocation failed */
#define AIR_KV_E_NOT_FOUND (-3)   /* unknown sequence id / nothing evicted */
#define AIR_KV_E_HIP (-4)         /* a HIP runtime call failed */
#define AIR_KV_E_STATE (-5)       /* operation invalid in the object's state */

/* ---- element types ----------------------------------------------------- */
#define AIR_KV_F32 0
#define AIR_KV_BF16 1  /* stored with round-to-nearest-even (half 2.7.1 bf16::from_f32) */
#define AIR_KV_INT8 2  /* Q8_0 codes, src/kv_cache.rs:54-75, + f32 scale per group */
#define AIR_KV_FP8 3   /* reference E4M3 encoding, src/fp8.rs:54-112, + f32 scale per group */

/* gather output layouts */
#define AIR_KV_LAYOUT_HEAD_MAJOR 0  /* out[h][t][d]: flash_decode's k_cache (src/flash_decode.rs:153-163) */
#define AIR_KV_LAYOUT_TOKEN_MAJOR 1 /* out[t][h][d]: the dense [seq, n_kv, d] view (src/kv_cache.rs:121-122) */

/* Copies the last error message of this thread (NUL-terminated, truncated to
 * `cap`).  Returns the full message length. */
int air_kv_last_error(char *buf, size_t cap);

/* ======================================================================== */
/* Host side: block allocator, block tables, sequences                      */
/* ======================================================================== */

/* Replaces BlockAllocator (src/paged_attention.rs:89-196).  Block ids are
 * PhysicalBlockId(u32) (:50-51).  `free_order` (may be NULL) sets the initial
 * FIFO order of the free list (a permutation of 0..capacity-1); NULL gives
 * the reference's 0..capacity order (:103-105).  `block_size` replaces the
 * BLOCK_SIZE const (:40). */
typedef struct air_block_allocator air_block_allocator;
int air_block_allocator_create(int64_t capacity, int32_t block_size, const uint32_t *free_order,
                               air_block_allocator **out);
int air_block_allocator_destroy(air_block_allocator *a);
/* allocate (:115-121): AIR_KV_E_OOM where the reference returns None. */
int air_block_allocator_allocate(air_block_allocator *a, uint32_t *block);
/* share (:124-126) */
int air_block_allocator_share(air_block_allocator *a, uint32_t block);
/* release (:129-135).  Releasing a block whose refcount is already 0 returns
 * AIR_KV_E_STATE; the reference would push it onto the free list twice. */
int air_block_allocator_release(air_block_allocator *a, uint32_t block);
/* ref_count (:138-140) */
int air_block_allocator_ref_count(const air_block_allocator *a, uint32_t block, uint32_t *rc);
/* num_free_blocks / num_used_blocks (:143-150) */
int64_t air_block_allocator_num_free(const air_block_allocator *a);
int64_t air_block_allocator_num_used(const air_block_allocator *a);
/* cow_write (:155-167): *out = block when it has a single owner, else a new
 * block (metadata copied, old refcount decremented); AIR_KV_E_OOM = None.
 * Page contents are copied on the device by air_kv_copy_blocks. */
int air_block_allocator_cow_write(air_block_allocator *a, uint32_t block, uint32_t *out);
/* append_token (:170-178): AIR_KV_E_STATE where the reference asserts. */
int air_block_allocator_append_token(air_block_allocator *a, uint32_t block, int32_t *is_full);
/* block fill metadata PhysicalBlock{num_tokens, is_full} (:63-80) */
int air_block_allocator_block_info(const air_block_allocator *a, uint32_t block,
                                   int32_t *num_tokens, int32_t *is_full);
/* can_allocate (:182-184): 1 or 0 */
int air_block_allocator_can_allocate(const air_block_allocator *a, int64_t n);
/* utilization (:193-195) */
float air_block_allocator_utilization(const air_block_allocator *a);
/* num_blocks_for_tokens (:188-190) */
int64_t air_num_blocks_for_tokens(int64_t n_tokens, int32_t block_size);

/* Replaces SequenceManager (src/paged_attention.rs:243-382). */
typedef struct air_seq_manager air_seq_manager;
int air_seq_manager_create(int64_t capacity, int32_t block_size, const uint32_t *free_order,
                           air_seq_manager **out);
int air_seq_manager_destroy(air_seq_manager *m);
/* The manager's allocator (borrowed; lives as long as the manager). */
air_block_allocator *air_seq_manager_allocator(air_seq_manager *m);
/* create_sequence (:260-265): monotonic ids */
int air_seq_create(air_seq_manager *m, uint32_t *seq);
/* append_token (:269-286): *block = the physical block of the new token.
 * AIR_KV_E_NOT_FOUND = "sequence not found", AIR_KV_E_OOM = "out of memory". */
int air_seq_append_token(air_seq_manager *m, uint32_t seq, uint32_t *block);
/* n successive append_token calls; slots[i] = block * block_size + pos % block_size
 * of the i-th new token (the slot_mapping air_kv_append consumes).  On failure
 * *n_done tokens were appended (as n separate reference calls would leave). */
int air_seq_append_slots(air_seq_manager *m, uint32_t seq, int32_t n, int64_t *slots,
                         int32_t *n_done);
/* fork_sequence (:290-310) */
int air_seq_fork(air_seq_manager *m, uint32_t parent, uint32_t *child);
/* free_sequence (:313-319): unknown ids are ignored, as in the reference. */
int air_seq_free(air_seq_manager *m, uint32_t seq);
/* cow_last_block (:327-335): AIR_KV_E_NOT_FOUND where the reference returns
 * None for a missing sequence or an empty table, AIR_KV_E_OOM for a failed
 * allocation.  *old_block / *new_block tell the caller which page to copy.
 * A new private block gets this sequence's own fill of that block (the
 * reference copies the shared block's fill, :159-164; the two differ only
 * after a truncation into the shared block or a co-owner's append into it). */
int air_seq_cow_last_block(air_seq_manager *m, uint32_t seq, uint32_t *old_block,
                           uint32_t *new_block);
/* No counterpart in the reference (its dense cache rolls back with
 * Tensor::narrow, src/kv_cache.rs:364-383): keeps the first n_tokens tokens
 * of `seq`, releases the blocks past them to the free list (in table order)
 * and, when the new last block belongs to `seq` alone, sets its fill to what
 * remains.  A no-op when n_tokens >= the sequence's length. */
int air_seq_truncate(air_seq_manager *m, uint32_t seq, int64_t n_tokens);
/* cow_last_block generalised to the block at table index `index` (no
 * counterpart in the reference): a private copy replaces a shared block and
 * gets this sequence's own fill of it. */
int air_seq_cow_block(air_seq_manager *m, uint32_t seq, int64_t index, uint32_t *old_block,
                      uint32_t *new_block);
/* table (:322-324): copies the block ids (at most `cap`; `blocks` may be
 * NULL to ask only for the counts). */
int air_seq_table(const air_seq_manager *m, uint32_t seq, uint32_t *blocks, int32_t cap,
                  int32_t *n_blocks, int64_t *n_tokens);
/* Flattened int32 block tables [n][max_blocks] (unused entries = -1) and
 * int32 seq_lens[n] for the device kernels (BlockTable, :202-235). */
int air_seq_export_tables(const air_seq_manager *m, const uint32_t *seqs, int32_t n,
                          int32_t max_blocks, int32_t *tables, int32_t *seq_lens);
/* num_sequences (:338-340), can_schedule (:344-346) */
int64_t air_seq_num_sequences(const air_seq_manager *m);
int air_seq_can_schedule(const air_seq_manager *m);
/* swap_out (:353-362): releases the blocks and returns their ids. */
int air_seq_swap_out(air_seq_manager *m, uint32_t seq, uint32_t *blocks, int32_t cap,
                     int32_t *n_blocks);
/* swap_in (:369-381): allocates n fresh blocks for the sequence. */
int air_seq_swap_in(air_seq_manager *m, uint32_t seq, int32_t n_blocks, uint32_t *blocks);

/* Replaces KvSwapManager (src/kv_swap.rs:22-121).  The reference's
 * gpu_read / gpu_write closures (:55-57, :83-86) become callbacks; the pair
 * air_kv_pool_read_cb / air_kv_pool_write_cb binds them to a device pool.
 * Unlike the closures, a callback returns a status (AIR_KV_OK, or a negative
 * AIR_KV_E_* code; a positive value is reported as AIR_KV_E_HIP): evict stops
 * at a failed read before anything is released, and restore undoes its
 * swap_in after a failed write, keeping the saved bytes for another try. */
typedef int (*air_kv_block_read_fn)(void *ctx, uint32_t block, uint8_t *dst, size_t bytes);
typedef int (*air_kv_block_write_fn)(void *ctx, uint32_t block, const uint8_t *src, size_t bytes);
typedef struct air_kv_swap air_kv_swap;
int air_kv_swap_create(int64_t capacity, int32_t block_size, size_t block_bytes, air_kv_swap **out);
int air_kv_swap_destroy(air_kv_swap *s);
air_seq_manager *air_kv_swap_seq_manager(air_kv_swap *s);
/* evict (:55-74): copies every block of the sequence to host memory, then swap_out. */
int air_kv_swap_evict(air_kv_swap *s, uint32_t seq, air_kv_block_read_fn read, void *ctx,
                      uint32_t *released, int32_t cap, int32_t *n_released);
/* restore (:83-98): swap_in, then writes the saved bytes to the new blocks.
 * As in the reference, the saved bytes are dropped if swap_in fails. */
int air_kv_swap_restore(air_kv_swap *s, uint32_t seq, air_kv_block_write_fn write, void *ctx,
                        uint32_t *blocks, int32_t cap, int32_t *n_blocks);
int air_kv_swap_is_evicted(const air_kv_swap *s, uint32_t seq);
int64_t air_kv_swap_evicted_count(const air_kv_swap *s);
int64_t air_kv_swap_cpu_bytes_used(const air_kv_swap *s);
/* maybe_evict (:112-121): *evicted = 1 when an eviction happened.  An
 * unknown sequence gives *evicted = 0 and AIR_KV_OK, as the reference's
 * false; a failed read callback returns its status. */
int air_kv_swap_maybe_evict(air_kv_swap *s, uint32_t seq, int64_t free_threshold,
                            air_kv_block_read_fn read, void *ctx, int32_t *evicted);

/* ======================================================================== */
/* Device side: the paged pool and its kernels                              */
/* ======================================================================== */

typedef struct air_kv_pool_desc {
    int64_t num_blocks;  /* pool capacity in blocks (MAX_BLOCKS, src/paged_attention.rs:45, as a runtime value) */
    int32_t block_size;  /* tokens per block; 16 or 32 (reference default 16) */
    int32_t n_kv_heads;
    int32_t head_dim;    /* multiple of 32, at most 256 */
    int32_t dtype;       /* AIR_KV_F32 / BF16 / INT8 / FP8 */
    int32_t scale_group; /* elements per scale along head_dim (INT8/FP8); 32 = Q8_0 (src/kv_cache.rs:26) */
} air_kv_pool_desc;

typedef struct air_kv_pool air_kv_pool;

/* Allocates the pool on the current HIP device.  Pages are zero-filled. */
int air_kv_pool_create(const air_kv_pool_desc *desc, air_kv_pool **out);
int air_kv_pool_destroy(air_kv_pool *pool);
/* Pool geometry, device base pointers and the bytes of one block
 * (K + V + scales), the unit of air_kv_read_blocks / write_blocks. */
int air_kv_pool_info(const air_kv_pool *pool, air_kv_pool_desc *desc, void **k_pages,
                     void **v_pages, void **k_scales, void **v_scales, size_t *block_bytes);

/* Reshape-and-cache: writes k[t][h][:], v[t][h][:] (f32, [n_tokens][n_kv_heads]
 * [head_dim], device) into slot slot_mapping[t] (int64, device), converting to
 * the pool dtype (bf16 RNE; INT8/FP8 quantize each group of scale_group
 * elements with its own scale).  Replaces the Tensor::cat append of
 * src/model.rs:569 and the Q8 quantize of save_layer (src/kv_cache.rs:307-315).
 * Negative slots are skipped; slots beyond the pool are skipped and counted
 * (air_kv_pool_error_count). */
int air_kv_append(air_kv_pool *pool, void *stream, const float *k, const float *v,
                  const int64_t *slot_mapping, int32_t n_tokens);

/* Gather: copies sequence b's first seq_lens[b] tokens from its pages into
 * out_k / out_v + out_offsets[b] elements (all device pointers), in
 * AIR_KV_LAYOUT_HEAD_MAJOR or TOKEN_MAJOR order, as out_dtype (AIR_KV_F32, or
 * AIR_KV_BF16; INT8/FP8 pools are dequantized q*scale as in
 * src/kv_cache.rs:78-92 and src/fp8.rs:263-264).  block_tables is int32
 * [batch][max_blocks], seq_lens int32 [batch].  Replaces load_layer's dense
 * view (src/kv_cache.rs:244-283).  Out-of-range table entries are skipped and
 * counted. */
int air_kv_gather(air_kv_pool *pool, void *stream, const int32_t *block_tables,
                  const int32_t *seq_lens, const int64_t *out_offsets, int32_t batch,
                  int32_t max_blocks, void *out_k, void *out_v, int32_t out_dtype,
                  int32_t out_layout);

/* Workspace bytes air_paged_decode needs for this launch shape (it depends on
 * the pool's device: the slice count follows its compute-unit count). */
int air_paged_decode_workspace_size(const air_kv_pool *pool, int32_t n_q_heads, int32_t batch,
                                    int32_t max_blocks, int32_t max_splits, size_t *bytes);


/* Split-K paged decode attention for one new token per sequence:
 *   out[b][h] = softmax(q[b][h] . K_b[h / group]^T * scale) . V_b[h / group]
 * over all seq_lens[b] cached tokens, group = n_q_heads / n_kv_heads (the GQA
 * map of src/chunked_attn.rs:240-243).  Replaces ops::attention for seq_q = 1
 * (src/ops.rs:333-357, :514-568) and generalises flash_decode
 * (src/flash_decode.rs:153-173: split-K partials merged by log-sum-exp,
 * :114-142) to paged storage.  q: [batch][n_q_heads][head_dim] as q_dtype
 * (AIR_KV_F32 or AIR_KV_BF16); out likewise as out_dtype.  On the
 * matrix-core kernel F32 queries enter the products as two bf16 halves on
 * BF16 pools and rounded to bf16 on INT8 / FP8 pools (an error an order below
 * their quantization's).  The reference's
 * scale is 1/sqrt(head_dim).  max_splits (1..256) bounds the split-K work
 * division: no sequence is cut into more than max_splits partitions.  Pools
 * with head_dim 128, block_size 16 or 32 and group 1..16 -- bf16, and int8 /
 * fp8 with scale_group >= 32 -- take the matrix-core kernel, which cuts the
 * batch's cached tokens into equal slices per kv head (one wave each, at most
 * batch * max_splits), where a slice may end inside a sequence and hold
 * several, widened when the longest sequence would otherwise meet more than
 * max_splits of them (max_splits 1: one slice per kv head); other pools
 * (F32 pages, head_dim 64 or 256, groups above 16) cut each sequence into at
 * most max_splits fixed partitions, each workgroup serving up to 8 query
 * heads of a kv head (any group: the reference's head map takes any
 * n_q_heads / n_kv_heads, src/chunked_attn.rs:65-72).  Out-of-pool table
 * entries are skipped and counted (air_kv_pool_error_count); seq_lens outside
 * [0, max_blocks * block_size] are clamped and counted.  A sequence of length
 * 0 produces zeros.  The workspace is device
 * memory of at least air_paged_decode_workspace_size bytes (no initialisation
 * needed); calls that share a workspace must be ordered (same stream). */
int air_paged_decode(air_kv_pool *pool, void *stream, const void *q, int32_t q_dtype,
                     int32_t n_q_heads, const int32_t *block_tables, const int32_t *seq_lens,
                     int32_t batch, int32_t max_blocks, float scale, int32_t max_splits,
                     void *workspace, size_t ws_bytes, void *out, int32_t out_dtype);

/* One decode step's append and attention in one launch: the same pages and
 * outputs as air_kv_append of k_new / v_new (f32, [batch][n_kv_heads]
 * [head_dim]) at each sequence's token seq_lens[b] - 1 -- the slot its block
 * table gives that token, the slot SequenceManager::append_token hands out
 * (src/paged_attention.rs:225-248) -- followed by air_paged_decode with the
 * same arguments (the reference's decode step appends the token's K/V, then
 * attends, src/model.rs:577, src/ops.rs:333-357).  Each new row is written by
 * the wave that attends over it, so no launch orders the two.  Sequences of
 * length 0 append nothing; a sequence longer than its table, or whose last
 * block is outside the pool, appends nothing and is counted as by
 * air_paged_decode.  On the matrix-core decode (head_dim 128, block_size 16
 * or 32, group 1..16; BF16, or INT8 / FP8 with scale_group >= 32, whose new
 * rows are quantized exactly as air_kv_append quantizes them: the same codes
 * and group scales) this is one launch; every other pool takes the same
 * call as three launches on the stream (each sequence's slot from its
 * table, air_kv_append's kernel, then the decode), with the same pages and
 * outputs.  k_new and v_new are 16-byte aligned device pointers.  The
 * workspace is air_paged_decode's. */
int air_paged_decode_append(air_kv_pool *pool, void *stream, const void *q, int32_t q_dtype,
                            int32_t n_q_heads, const float *k_new, const float *v_new,
                            const int32_t *block_tables, const int32_t *seq_lens, int32_t batch,
                            int32_t max_blocks, float scale, int32_t max_splits, void *workspace,
                            size_t ws_bytes, void *out, int32_t out_dtype);

/* Bytes of the file-scope device array air_paged_decode_noalloc uses as its
 * workspace (one copy per GPU, held until the process ends). */
#define AIR_KV_NOALLOC_SCRATCH_BYTES (32u << 20)

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): air_paged_decode with its workspace taken from a
 * library-owned device array of AIR_KV_NOALLOC_SCRATCH_BYTES instead of a
 * caller buffer.  Same arguments, kernels and results as air_paged_decode;
 * it calls no hipMalloc / hipFree.  A launch whose
 * air_paged_decode_workspace_size exceeds the array returns
 * AIR_KV_E_INVALID_ARG (32 MiB holds configs c2-c5: c4 needs 17.3 MB).
 * Every call on one GPU shares that GPU's array, so the library orders them:
 * each call records an event on its stream after its launch, and a call on
 * another stream first makes its stream wait for the previous call's event
 * (an event created once per GPU, with the array's address lookup).  Calls
 * from several threads are serialised by a lock.  A caller capturing a HIP
 * graph should keep its no-alloc calls on the capturing stream: a switch of
 * stream adds a wait on an event recorded outside the capture. */
int air_paged_decode_noalloc(air_kv_pool *pool, void *stream, const void *q, int32_t q_dtype,
                             int32_t n_q_heads, const int32_t *block_tables, const int32_t *seq_lens,
                             int32_t batch, int32_t max_blocks, float scale, int32_t max_splits,
                             void *out, int32_t out_dtype);

/* Paged prefill attention (chunked, causal): sequence b's q_len = cu_q[b + 1]
 * - cu_q[b] newest tokens, whose K/V are already appended, attend over its
 * seq_lens[b] cached tokens; query row r (0-based within the sequence) sits at
 * position seq_lens[b] - q_len + r and sees keys 0 ..= that position:
 *   out[cu_q[b] + r][h] = softmax over those keys of q . K[h / group]^T * scale, . V
 * This is blockwise_attention_head with q_offset = seq_len - q_len
 * (src/chunked_attn.rs:114-213) for every query head, GQA kv head h / group
 * (:240-243) -- the causal prefill branch of ops::attention (src/ops.rs:333-357,
 * mask :762-790) over paged storage, for the 512-token prefill chunks of
 * src/generator.rs:46.  q / out: [total_q][n_q_heads][head_dim] as q_dtype /
 * out_dtype (AIR_KV_F32 or AIR_KV_BF16); cu_q: int32 [batch + 1] (device).
 * max_q_len sizes the launch (an upper bound of the q_len values; a larger
 * q_len is still computed in full).  scale must be finite and > 0 (the
 * reference's is 1/sqrt(head_dim)).  BF16, INT8 and FP8 pools with head_dim
 * 128 take the matrix-core kernel (quantized pages are dequantized q * scale
 * in registers); every other pool (F32 pages, other head dims) runs each
 * query row on air_paged_decode's split kernel over its causal keys, with f32
 * products, no workspace and the same error handling.  BF16 pools run the probability x value
 * products with f16 operands (11 significant bits each), INT8 / FP8 pools the
 * key x query products as well (keys, values and F32 queries rounded to f16
 * once); a work group whose result that way is not finite, or whose outputs
 * of a query row are all below 2^-14 in magnitude, is recomputed with bf16
 * operands: probabilities as two bf16 halves on BF16 pools, keys as two bf16
 * halves on INT8 / FP8 pools.  The f16 pass bounds each output's error
 * relative to the largest output of its query row, not to its own value
 * channel: a channel whose values lie far below the others' (under 2^-17
 * while others are near 1) keeps f16's absolute resolution, errors up to
 * 2^-24, not 1e-3 of its own magnitude.  A sequence whose rows do not lie in
 * [0, total_q], whose seq_len is outside [0, max_blocks * block_size] or
 * whose q_len exceeds its seq_len is counted (air_kv_pool_error_count) and its
 * rows (when they lie in [0, total_q]) are zero-filled; out-of-pool table
 * entries within a sequence's length are counted and read as zero keys and
 * values.  Rows of different sequences must not overlap.  workspace may be
 * NULL (every work group then walks all of its keys).  When the launch has
 * fewer work groups (32 query rows x one GQA group of heads) than its GPU
 * keeps resident, a 16-byte aligned device buffer of at least
 * air_paged_prefill_workspace_size bytes (no initialisation needed) lets
 * work groups longer than the batch's balanced load be cut into key ranges
 * on several workgroups and merged by log-sum-exp (kernels before and after
 * on the same stream), the combination flash_decode's split-K uses
 * (src/flash_decode.rs:114-142); for other launches the size is 0 and any
 * workspace is ignored.  Calls that share a workspace must be ordered (same
 * stream). */
int air_paged_prefill(air_kv_pool *pool, void *stream, const void *q, int32_t q_dtype,
                      int32_t n_q_heads, const int32_t *cu_q, int32_t total_q, int32_t max_q_len,
                      const int32_t *block_tables, const int32_t *seq_lens, int32_t batch,
                      int32_t max_blocks, float scale, void *workspace, size_t ws_bytes, void *out,
                      int32_t out_dtype);

/* Workspace bytes air_paged_prefill's key split needs for this launch shape
 * (0: the launch does not split).  It depends on the pool's device: the
 * resident-slot count follows its compute units. */
int air_paged_prefill_workspace_size(const air_kv_pool *pool, int32_t n_q_heads, int32_t batch,
                                     int32_t max_q_len, size_t *bytes);

/* ------------------------------------------------------------------------ */
/* SessionKvCache over pages                                                 */
/* ------------------------------------------------------------------------ */

/* The paged counterpart of SessionKvCache (src/kv_cache.rs:431-446) for one
 * sequence of `mgr`: layer l keeps its K/V in layer_pools[l] (every pool has
 * the manager's block_size and at least its capacity in blocks), and all
 * layers share the sequence's block table.  Creating a session creates the
 * sequence; destroying it frees the sequence's blocks.  The session is not
 * thread-safe (like the manager).  Device work is ordered on `stream`; the
 * session keeps small device and pinned host staging buffers of its own. */
typedef struct air_kv_session air_kv_session;
int air_kv_session_create(air_seq_manager *mgr, air_kv_pool *const *layer_pools, int32_t n_layers,
                          air_kv_session **out);
int air_kv_session_destroy(air_kv_session *s);
/* A new session whose sequence is fork_sequence(parent) (src/paged_attention.rs:290-310):
 * the child shares the parent's blocks and per-layer lengths; a shared block
 * is copied (in every layer's pool) before either session writes into it. */
int air_kv_session_fork(air_kv_session *parent, air_kv_session **out);
int air_kv_session_seq_id(const air_kv_session *s, uint32_t *seq);
/* seq_len(layer) (:433): tokens stored for the layer, 0 if empty. */
int air_kv_session_seq_len(const air_kv_session *s, int32_t layer, int64_t *len);
/* Appends n_new rows k/v (f32 [n_new][n_kv_heads][head_dim], device) after the
 * layer's stored tokens: the reshape-and-cache that replaces the
 * Tensor::cat of src/model.rs:569.  Allocates blocks on block boundaries. */
int air_kv_session_append(air_kv_session *s, void *stream, int32_t layer, const float *k,
                          const float *v, int64_t n_new);
/* save(layer, cache) (:436): the layer's cache becomes the n_tokens rows of
 * k/v (f32 [n_tokens][n_kv_heads][head_dim], device).  The decode loop only
 * grows a cache by concatenation, so rows already stored are taken as equal to
 * the first rows of k/v and are not rewritten: rows past the stored length are
 * appended, and a shorter n_tokens shortens the layer as truncate_to does. */
int air_kv_session_save(air_kv_session *s, void *stream, int32_t layer, const float *k,
                        const float *v, int64_t n_tokens);
/* load(layer) (:439): the layer's tokens as the dense [seq][n_kv_heads][head_dim]
 * view of LayerCache::Attention (src/kv_cache.rs:121-122) in out_k / out_v
 * (device, out_dtype AIR_KV_F32 or AIR_KV_BF16; 1-byte pools dequantize). */
int air_kv_session_load(air_kv_session *s, void *stream, int32_t layer, void *out_k, void *out_v,
                        int32_t out_dtype);
/* clear() (:442): every layer empty, all blocks released. */
int air_kv_session_clear(air_kv_session *s);
/* truncate_to(pos) (:445, src/kv_cache.rs:364-383): every layer keeps at most
 * pos tokens; blocks past them are released.  No device work. */
int air_kv_session_truncate_to(air_kv_session *s, int64_t pos);
/* Bytes of device memory the session's blocks occupy over all its layers
 * (the paged form of memory_usage, src/kv_cache.rs:388-414). */
int air_kv_session_memory_usage(const air_kv_session *s, size_t *bytes);

/* ------------------------------------------------------------------------ */
/* KvBlock wire format (prefill/decode disaggregation)                        */
/* ------------------------------------------------------------------------ */

/* Bytes of one KvBlock's data (src/pd_disagg.rs:39-49): bf16
 * [block_size][n_kv_heads][head_dim][2], K at index 0 and V at 1 of the last
 * axis: 4 * block_size * n_kv_heads * head_dim. */
int air_kv_block_wire_bytes(const air_kv_pool *pool, size_t *bytes);
/* Writes the wire data of blocks ids[i] (int32, device) to out + i * wire
 * bytes (device).  bf16 pools copy their bits, f32 pools round to nearest
 * even, int8 / fp8 pools dequantize (q * scale) then round.  Ids outside the
 * pool leave their slot untouched and are counted (air_kv_pool_error_count). */
int air_kv_pack_blocks(air_kv_pool *pool, void *stream, const int32_t *ids, int32_t n, void *out);
/* The inverse: wire data (device) into blocks ids[i].  bf16 pools take the
 * bits, f32 pools widen exactly, int8 / fp8 pools quantize each scale group
 * of every row exactly as air_kv_append does. */
int air_kv_unpack_blocks(air_kv_pool *pool, void *stream, const int32_t *ids, int32_t n,
                         const void *in);
/* KvBlock::int8_quantize (src/pd_disagg.rs:65-83) of n_blocks wire blocks of
 * elems_per_block bf16 elements each (device): one f32 scale per block
 * (absmax / 127, NaN ignored, 1.0 for an all-zero block) and int8 codes
 * round(x * (1 / scale)) in wire order.  Bit-exact with the reference. */
int air_kv_wire_int8_quantize(void *stream, const void *wire, int32_t n_blocks,
                              size_t elems_per_block, int8_t *codes, float *scales);
/* air_kv_pack_blocks followed by air_kv_wire_int8_quantize in one pass over
 * the pages (the TcpKvConnector send path, src/pd_disagg.rs:267-275):
 * codes + i * wire_bytes / 2 and scales[i] for block ids[i]. */
int air_kv_pack_blocks_int8(air_kv_pool *pool, void *stream, const int32_t *ids, int32_t n,
                            int8_t *codes, float *scales);

/* Host-side framing around the wire data (plain host memory, no device
 * work; every integer little-endian, as the reference's to_le_bytes).       */

/* KvBlock::serialise (src/pd_disagg.rs:52-62): [block_id:4][layer_idx:2]
 * [data_len:4][data], 10 + data_len bytes; out must hold them (cap). */
size_t air_kv_block_frame_bytes(size_t data_len);
int air_kv_block_serialise(uint32_t block_id, uint16_t layer_idx, const void *data, size_t data_len,
                           void *out, size_t cap, size_t *written);
/* KvBlock::deserialise (src/pd_disagg.rs:85-104): AIR_KV_E_INVALID_ARG where
 * the reference returns None (fewer than 10 bytes, or fewer than 10 +
 * data_len); *data points into buf. */
int air_kv_block_deserialise(const void *buf, size_t len, uint32_t *block_id, uint16_t *layer_idx,
                             const void **data, size_t *data_len);
/* n frames back to back, frame i for block_ids[i] with the block_bytes of
 * wire data at data + i * block_bytes (air_kv_pack_blocks' output copied to
 * the host): n * (10 + block_bytes) bytes. */
int air_kv_block_serialise_n(const uint32_t *block_ids, uint16_t layer_idx, const void *data,
                             size_t block_bytes, int32_t n, void *out);
/* The int8 transfer payload of TcpKvConnector::send_blocks
 * (src/pd_disagg.rs:267-276): [block_id:4][layer_idx:2][scale:4, f32]
 * [len:4][codes], 14 + n_codes bytes.  (The reference's receiver parses every
 * payload with KvBlock::deserialise, which reads the scale's bits as data_len;
 * air_kv_int8_payload_deserialise reads the layout the sender writes.) */
size_t air_kv_int8_payload_bytes(size_t n_codes);
int air_kv_int8_payload_serialise(uint32_t block_id, uint16_t layer_idx, float scale, const int8_t *codes,
                                  size_t n_codes, void *out, size_t cap, size_t *written);
int air_kv_int8_payload_deserialise(const void *buf, size_t len, uint32_t *block_id, uint16_t *layer_idx,
                                    float *scale, const int8_t **codes, size_t *n_codes);
/* n payloads back to back from air_kv_pack_blocks_int8's codes and scales
 * (copied to the host): n * (14 + codes_per_block) bytes. */
int air_kv_int8_payload_serialise_n(const uint32_t *block_ids, uint16_t layer_idx, const float *scales,
                                    const int8_t *codes, size_t codes_per_block, int32_t n, void *out);

/* ------------------------------------------------------------------------ */
/* kv_compress warm-tier codecs (src/kv_compress.rs)                          */
/* ------------------------------------------------------------------------ */

/* Batched codecs over rows of `dim` elements (dim 32, 64 or 128; rows are
 * device [n_rows][dim] arrays of rows_dtype AIR_KV_F32 or AIR_KV_BF16, 16-byte
 * aligned).  Every output is bit-exact with the reference's scalar code: one
 * row per lane folds its elements left to right, as the reference's
 * iterators do, and products and sums round separately.  All device
 * pointers; asynchronous on `stream`. */

/* CompressedKey::compress (src/kv_compress.rs:79-109) of each row:
 * bits[r][w] (ceil(dim / 64) words, bit i = row[i] >= mean, LSB first),
 * magnitude[r] = |row| (sqrt of the left fold of squares), mean[r]. */
int air_kv_key_compress(void *stream, const void *rows, int32_t rows_dtype, int64_t n_rows,
                        int32_t dim, uint64_t *bits, float *magnitude, float *mean);
/* CompressedKey::decompress (:112-127): out[r][i] = (+-1) * (magnitude /
 * sqrt(dim)) + mean, f32 (any dim >= 1). */
int air_kv_key_decompress(void *stream, const uint64_t *bits, const float *magnitude,
                          const float *mean, int64_t n_rows, int32_t dim, float *out);
/* CompressedValue::compress (:187-218): codes[r][i] = round((v - min) /
 * scale) clamped to [0, 255] (NaN -> 0), scale = (max - min) / 255 or 1.0,
 * NaN-ignoring min / max folds.  codes must be 16-byte aligned. */
int air_kv_value_compress(void *stream, const void *rows, int32_t rows_dtype, int64_t n_rows,
                          int32_t dim, uint8_t *codes, float *scale, float *min_val);
/* CompressedValue::decompress (:221-226): out = q * scale + min, f32. */
int air_kv_value_decompress(void *stream, const uint8_t *codes, const float *scale,
                            const float *min_val, int64_t n_rows, int32_t dim, float *out);
/* QjlKey::compress (:930-951) with the row-major [proj_dim][dim] f32 matrix
 * `proj` (qjl_projection_matrix, :989-1017, is built by the caller):
 * bit i of row r = (proj[i] . row > 0), magnitude[r] = |row|.  proj_dim
 * 1..512; bits[r] holds ceil(proj_dim / 64) words. */
int air_kv_qjl_compress(void *stream, const void *rows, int32_t rows_dtype, int64_t n_rows,
                        int32_t dim, const float *proj, int32_t proj_dim, uint64_t *bits,
                        float *magnitude);
/* QjlKey::approx_cos_sim / approx_dot (:959-975) of one query (query_bits,
 * device, ceil(proj_dim / 64) words) against n_keys keys: cos_sim[k] =
 * cos(pi * hamming / proj_dim) (the cosine evaluated by the host's libm, as
 * the reference's f32::cos), dot[k] = cos_sim[k] * key_magnitude[k] *
 * query_magnitude.  Either output may be NULL. */
int air_kv_qjl_scores(void *stream, const uint64_t *key_bits, const float *key_magnitude,
                      int64_t n_keys, int32_t proj_dim, const uint64_t *query_bits,
                      float query_magnitude, float *cos_sim, float *dot);
/* Warm-tier compression of whole pool blocks, CompressedKvEntry::compress
 * (:283-292) of every (head, token) row: the K rows of blocks ids[0..n) with
 * CompressedKey::compress and the V rows with CompressedValue::compress.
 * Rows are ordered [i][head][token] (n * n_kv_heads * block_size rows);
 * quantized pools are dequantized (q * scale) first.  Ids outside the pool
 * give zero outputs and are counted (air_kv_pool_error_count).  Pools with
 * head_dim 32, 64 or 128. */
int air_kv_compress_blocks(air_kv_pool *pool, void *stream, const int32_t *ids, int32_t n,
                           uint64_t *key_bits, float *key_magnitude, float *key_mean,
                           uint8_t *value_codes, float *value_scale, float *value_min);
/* QjlKey::compress of the K rows of pool blocks (same row order). */
int air_kv_qjl_compress_blocks(air_kv_pool *pool, void *stream, const int32_t *ids, int32_t n,
                               const float *proj, int32_t proj_dim, uint64_t *bits,
                               float *magnitude);

/* Copies whole blocks src[i] -> dst[i] (int32, device): the page copy that
 * BlockAllocator::cow_write leaves to "a real impl" (src/paged_attention.rs:160). */
int air_kv_copy_blocks(air_kv_pool *pool, void *stream, const int32_t *src_blocks,
                       const int32_t *dst_blocks, int32_t n);

/* Page-granular device<->host copies for swap (the gpu_read / gpu_write
 * closures of src/kv_swap.rs:55-98).  ids are host int32; host buffers hold
 * n * block_bytes bytes, block i at offset i * block_bytes laid out as
 * K slab, V slab, K scales, V scales.  Both calls synchronise the stream.
 * Blocks travel through a pool-owned 64 MB device staging buffer (allocated
 * on the first call, freed with the pool), one PCIe transfer per 64 MB; two
 * of these calls on one pool must not run concurrently. */
int air_kv_read_blocks(air_kv_pool *pool, void *stream, const int32_t *ids, int32_t n, void *host_dst);
int air_kv_write_blocks(air_kv_pool *pool, void *stream, const int32_t *ids, int32_t n,
                        const void *host_src);
/* air_kv_block_read_fn / write_fn adapters over a pool (ctx = air_kv_pool*),
 * on the default stream.  `bytes` must equal the pool's block_bytes (a swap
 * manager created with another block size gets AIR_KV_E_INVALID_ARG, and its
 * evict stops before releasing anything). */
int air_kv_pool_read_cb(void *ctx, uint32_t block, uint8_t *dst, size_t bytes);
int air_kv_pool_write_cb(void *ctx, uint32_t block, const uint8_t *src, size_t bytes);

/* Number of out-of-range slots / table entries the kernels have skipped since
 * the pool was created or last reset.  Synchronises the stream. */
int air_kv_pool_error_count(air_kv_pool *pool, void *stream, int64_t *count, int32_t reset);

#ifdef __cplusplus
}
#endif
#endif /* AIR_KV_H */
