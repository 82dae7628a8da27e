//! Safe Rust wrapper over `airkv-sys` (the C ABI in include/air_kv.h) with the
//! API surface of the reference's `src/paged_attention.rs`, `src/kv_swap.rs`,
//! `src/kv_cache.rs` (`SessionKvCache`) and `src/flash_decode.rs`:
//! the same type names, method names, argument meanings and `Option` /
//! `Result<_, &'static str>` conventions, so `InferenceGenerator` can switch
//! to it by changing its `use` lines.  Device work goes through [`KvPool`].
//!
//! This crate is source for Air.rs maintainers; it is not compiled in this
//! repository (there is no Rust toolchain in the build image).
//!
//! Differences from the reference, all on paths where the reference panics
//! or corrupts state: releasing a free block is refused (the reference
//! pushes it onto the free list twice), appending to a full block is an
//! error (the reference asserts), copy-on-write gives the private block the
//! sequence's own fill, and `try_evict` / `try_restore` take closures that
//! return a status (a failed read aborts the evict before any block is
//! released).  `SessionKvCache` and `flash_decode` take device pointers where
//! the reference takes candle tensors and host slices.

use std::ffi::c_void;
use std::marker::PhantomData;
use std::ptr;

use airkv_sys as sys;

/// `BLOCK_SIZE` of src/paged_attention.rs:40; the pool here takes 16 or 32.
pub const BLOCK_SIZE: usize = 16;
/// `MAX_BLOCKS` of src/paged_attention.rs:45 (a default: capacities are runtime values).
pub const MAX_BLOCKS: usize = 4096;

#[derive(Debug, Clone, Copy, PartialEq, Eq, Hash, PartialOrd, Ord)]
pub struct PhysicalBlockId(pub u32);
#[derive(Debug, Clone, Copy, PartialEq, Eq, Hash, PartialOrd, Ord)]
pub struct LogicalBlockId(pub u32);
#[derive(Debug, Clone, Copy, PartialEq, Eq, Hash, PartialOrd, Ord)]
pub struct SeqId(pub u32);

/// Block fill metadata (src/paged_attention.rs:63-80).
#[derive(Debug, Clone, Copy, PartialEq, Eq)]
pub struct PhysicalBlock {
    pub id: PhysicalBlockId,
    pub num_tokens: usize,
    pub is_full: bool,
}

/// The message of the last failure on this thread (air_kv_last_error).
pub fn last_error() -> String {
    let mut buf = vec![0u8; 1024];
    // SAFETY: the buffer is valid for its length; the library NUL-terminates.
    unsafe { sys::air_kv_last_error(buf.as_mut_ptr() as *mut _, buf.len()) };
    let end = buf.iter().position(|&b| b == 0).unwrap_or(buf.len());
    String::from_utf8_lossy(&buf[..end]).into_owned()
}

/// A failed library call: its status code and message.
#[derive(Debug, Clone)]
pub struct AirKvError {
    pub code: i32,
    pub message: String,
}

impl std::fmt::Display for AirKvError {
    fn fmt(&self, f: &mut std::fmt::Formatter<'_>) -> std::fmt::Result {
        write!(f, "airkv error {}: {}", self.code, self.message)
    }
}

impl std::error::Error for AirKvError {}

fn check(rc: i32) -> Result<i32, AirKvError> {
    if rc < 0 {
        Err(AirKvError { code: rc, message: last_error() })
    } else {
        Ok(rc)
    }
}

// ---------------------------------------------------------------------------
// BlockAllocator (src/paged_attention.rs:89-196)
// ---------------------------------------------------------------------------

/// FIFO block allocator with refcounts.  Owned, or borrowed from a
/// [`SequenceManager`] (then it must not outlive it).
pub struct BlockAllocator {
    raw: *mut sys::air_block_allocator,
    owned: bool,
}

impl BlockAllocator {
    /// `new(capacity)` (:99-112): free list 0..capacity.
    pub fn new(capacity: usize) -> Self {
        Self::with_free_order(capacity, BLOCK_SIZE, None)
    }

    /// A runtime block size and an initial FIFO order (a permutation of 0..capacity).
    pub fn with_free_order(capacity: usize, block_size: usize, free_order: Option<&[u32]>) -> Self {
        let mut raw = ptr::null_mut();
        let order = free_order.map_or(ptr::null(), |o| o.as_ptr());
        // SAFETY: out-pointer valid; `order` is null or `capacity` u32s.
        check(unsafe { sys::air_block_allocator_create(capacity as i64, block_size as i32, order, &mut raw) })
            .expect("air_block_allocator_create");
        Self { raw, owned: true }
    }

    pub fn allocate(&mut self) -> Option<PhysicalBlockId> {
        let mut id = 0u32;
        // SAFETY: handle valid for self's lifetime.
        (unsafe { sys::air_block_allocator_allocate(self.raw, &mut id) } == sys::AIR_KV_OK).then_some(PhysicalBlockId(id))
    }

    pub fn share(&mut self, block_id: PhysicalBlockId) {
        unsafe { sys::air_block_allocator_share(self.raw, block_id.0) };
    }

    /// Releasing a block whose refcount is already 0 is refused (the
    /// reference would push it onto the free list twice).
    pub fn release(&mut self, block_id: PhysicalBlockId) {
        unsafe { sys::air_block_allocator_release(self.raw, block_id.0) };
    }

    pub fn ref_count(&self, block_id: PhysicalBlockId) -> u32 {
        let mut rc = 0u32;
        unsafe { sys::air_block_allocator_ref_count(self.raw, block_id.0, &mut rc) };
        rc
    }

    pub fn num_free_blocks(&self) -> usize {
        unsafe { sys::air_block_allocator_num_free(self.raw) as usize }
    }

    pub fn num_used_blocks(&self) -> usize {
        unsafe { sys::air_block_allocator_num_used(self.raw) as usize }
    }

    /// Metadata copy; the page bytes are copied by [`KvPool::copy_blocks`].
    pub fn cow_write(&mut self, block_id: PhysicalBlockId) -> Option<PhysicalBlockId> {
        let mut out = 0u32;
        (unsafe { sys::air_block_allocator_cow_write(self.raw, block_id.0, &mut out) } == sys::AIR_KV_OK)
            .then_some(PhysicalBlockId(out))
    }

    /// Returns `true` if the block is now full; appending to a full block
    /// panics, as the reference's assert does.
    pub fn append_token(&mut self, block_id: PhysicalBlockId) -> bool {
        let mut full = 0i32;
        check(unsafe { sys::air_block_allocator_append_token(self.raw, block_id.0, &mut full) })
            .expect("cannot append to a full block");
        full != 0
    }

    pub fn block(&self, block_id: PhysicalBlockId) -> PhysicalBlock {
        let (mut n, mut full) = (0i32, 0i32);
        unsafe { sys::air_block_allocator_block_info(self.raw, block_id.0, &mut n, &mut full) };
        PhysicalBlock { id: block_id, num_tokens: n as usize, is_full: full != 0 }
    }

    pub fn can_allocate(&self, n: usize) -> bool {
        unsafe { sys::air_block_allocator_can_allocate(self.raw, n as i64) == 1 }
    }

    pub fn num_blocks_for_tokens(n_tokens: usize) -> usize {
        unsafe { sys::air_num_blocks_for_tokens(n_tokens as i64, BLOCK_SIZE as i32) as usize }
    }

    pub fn utilization(&self) -> f32 {
        unsafe { sys::air_block_allocator_utilization(self.raw) }
    }
}

impl Drop for BlockAllocator {
    fn drop(&mut self) {
        if self.owned {
            unsafe { sys::air_block_allocator_destroy(self.raw) };
        }
    }
}

// The C++ object is not thread-safe but may move between threads; callers
// serialise access (the reference's generator holds it in a Mutex).
unsafe impl Send for BlockAllocator {}

// ---------------------------------------------------------------------------
// BlockTable (src/paged_attention.rs:202-235)
// ---------------------------------------------------------------------------

/// A sequence's logical -> physical map, copied out of the manager.
#[derive(Debug, Clone, PartialEq, Eq)]
pub struct BlockTable {
    pub seq_id: SeqId,
    pub physical_blocks: Vec<PhysicalBlockId>,
    pub num_tokens: usize,
}

impl BlockTable {
    pub fn logical_block_for_token(token_pos: usize) -> LogicalBlockId {
        LogicalBlockId((token_pos / BLOCK_SIZE) as u32)
    }

    pub fn physical_block_for_token(&self, token_pos: usize) -> PhysicalBlockId {
        self.physical_blocks[token_pos / BLOCK_SIZE]
    }

    pub fn num_logical_blocks(&self) -> usize {
        self.physical_blocks.len()
    }

    pub fn last_block_offset(&self) -> usize {
        self.num_tokens % BLOCK_SIZE
    }
}

// ---------------------------------------------------------------------------
// SequenceManager (src/paged_attention.rs:243-382)
// ---------------------------------------------------------------------------

pub struct SequenceManager {
    raw: *mut sys::air_seq_manager,
    owned: bool,
    block_size: usize,
}

impl SequenceManager {
    pub fn new(block_capacity: usize) -> Self {
        Self::with_block_size(block_capacity, BLOCK_SIZE, None)
    }

    pub fn with_block_size(block_capacity: usize, block_size: usize, free_order: Option<&[u32]>) -> Self {
        let mut raw = ptr::null_mut();
        let order = free_order.map_or(ptr::null(), |o| o.as_ptr());
        check(unsafe { sys::air_seq_manager_create(block_capacity as i64, block_size as i32, order, &mut raw) })
            .expect("air_seq_manager_create");
        Self { raw, owned: true, block_size }
    }

    /// The manager's allocator (borrowed).
    pub fn allocator(&mut self) -> BlockAllocator {
        BlockAllocator { raw: unsafe { sys::air_seq_manager_allocator(self.raw) }, owned: false }
    }

    pub fn create_sequence(&mut self) -> SeqId {
        let mut s = 0u32;
        check(unsafe { sys::air_seq_create(self.raw, &mut s) }).expect("air_seq_create");
        SeqId(s)
    }

    pub fn append_token(&mut self, seq_id: SeqId) -> Result<PhysicalBlockId, &'static str> {
        let mut b = 0u32;
        match unsafe { sys::air_seq_append_token(self.raw, seq_id.0, &mut b) } {
            sys::AIR_KV_OK => Ok(PhysicalBlockId(b)),
            sys::AIR_KV_E_NOT_FOUND => Err("sequence not found"),
            sys::AIR_KV_E_OOM => Err("out of memory — no free blocks"),
            _ => Err("append_token failed"),
        }
    }

    /// `n` appends at once; returns the slot of every new token
    /// (`block * block_size + pos % block_size`), the slot mapping the device
    /// append consumes.
    pub fn append_slots(&mut self, seq_id: SeqId, n: usize) -> Result<Vec<i64>, &'static str> {
        let mut slots = vec![0i64; n];
        let mut done = 0i32;
        match unsafe { sys::air_seq_append_slots(self.raw, seq_id.0, n as i32, slots.as_mut_ptr(), &mut done) } {
            sys::AIR_KV_OK => Ok(slots),
            sys::AIR_KV_E_NOT_FOUND => Err("sequence not found"),
            sys::AIR_KV_E_OOM => Err("out of memory — no free blocks"),
            _ => Err("append failed"),
        }
    }

    pub fn fork_sequence(&mut self, parent_id: SeqId) -> Result<SeqId, &'static str> {
        let mut c = 0u32;
        match unsafe { sys::air_seq_fork(self.raw, parent_id.0, &mut c) } {
            sys::AIR_KV_OK => Ok(SeqId(c)),
            _ => Err("parent sequence not found"),
        }
    }

    pub fn free_sequence(&mut self, seq_id: SeqId) {
        unsafe { sys::air_seq_free(self.raw, seq_id.0) };
    }

    pub fn table(&self, seq_id: SeqId) -> Option<BlockTable> {
        let (mut nb, mut nt) = (0i32, 0i64);
        if unsafe { sys::air_seq_table(self.raw, seq_id.0, ptr::null_mut(), 0, &mut nb, &mut nt) } < 0 {
            return None;
        }
        let mut ids = vec![0u32; nb as usize];
        unsafe { sys::air_seq_table(self.raw, seq_id.0, ids.as_mut_ptr(), nb, &mut nb, &mut nt) };
        Some(BlockTable {
            seq_id,
            physical_blocks: ids.into_iter().map(PhysicalBlockId).collect(),
            num_tokens: nt as usize,
        })
    }

    /// Returns the block to write into (new when the last block was
    /// shared); the caller copies the page with [`KvPool::copy_blocks`].
    pub fn cow_last_block(&mut self, seq_id: SeqId) -> Option<PhysicalBlockId> {
        let (mut old, mut new) = (0u32, 0u32);
        (unsafe { sys::air_seq_cow_last_block(self.raw, seq_id.0, &mut old, &mut new) } == sys::AIR_KV_OK)
            .then_some(PhysicalBlockId(new))
    }

    pub fn num_sequences(&self) -> usize {
        unsafe { sys::air_seq_num_sequences(self.raw) as usize }
    }

    pub fn can_schedule(&self) -> bool {
        unsafe { sys::air_seq_can_schedule(self.raw) == 1 }
    }

    pub fn swap_out(&mut self, seq_id: SeqId) -> Result<Vec<PhysicalBlockId>, &'static str> {
        let n = self.table(seq_id).ok_or("sequence not found")?.physical_blocks.len();
        let mut ids = vec![0u32; n.max(1)];
        let mut got = 0i32;
        match unsafe { sys::air_seq_swap_out(self.raw, seq_id.0, ids.as_mut_ptr(), ids.len() as i32, &mut got) } {
            sys::AIR_KV_OK => Ok(ids[..got as usize].iter().map(|&b| PhysicalBlockId(b)).collect()),
            _ => Err("sequence not found"),
        }
    }

    pub fn swap_in(&mut self, seq_id: SeqId, n_blocks: usize) -> Result<Vec<PhysicalBlockId>, &'static str> {
        let mut ids = vec![0u32; n_blocks.max(1)];
        match unsafe { sys::air_seq_swap_in(self.raw, seq_id.0, n_blocks as i32, ids.as_mut_ptr()) } {
            sys::AIR_KV_OK => Ok(ids[..n_blocks].iter().map(|&b| PhysicalBlockId(b)).collect()),
            sys::AIR_KV_E_OOM => Err("out of memory — cannot swap in"),
            _ => Err("sequence not found"),
        }
    }

    /// Block tables of `seqs` as the device kernels read them: int32
    /// `[n][max_blocks]` (unused entries -1) and int32 lengths.
    pub fn export_tables(&self, seqs: &[SeqId], max_blocks: usize) -> Result<(Vec<i32>, Vec<i32>), AirKvError> {
        let ids: Vec<u32> = seqs.iter().map(|s| s.0).collect();
        let mut tables = vec![0i32; seqs.len() * max_blocks];
        let mut lens = vec![0i32; seqs.len()];
        check(unsafe {
            sys::air_seq_export_tables(self.raw, ids.as_ptr(), ids.len() as i32, max_blocks as i32,
                                       tables.as_mut_ptr(), lens.as_mut_ptr())
        })?;
        Ok((tables, lens))
    }

    pub fn block_size(&self) -> usize {
        self.block_size
    }

    pub(crate) fn raw(&self) -> *mut sys::air_seq_manager {
        self.raw
    }
}

impl Drop for SequenceManager {
    fn drop(&mut self) {
        if self.owned {
            unsafe { sys::air_seq_manager_destroy(self.raw) };
        }
    }
}

unsafe impl Send for SequenceManager {}

// ---------------------------------------------------------------------------
// KvSwapManager (src/kv_swap.rs:22-121)
// ---------------------------------------------------------------------------

pub struct KvSwapManager {
    raw: *mut sys::air_kv_swap,
    /// The manager's sequences (borrowed from the swap manager).
    pub seq_mgr: SequenceManager,
}

struct ReadCtx<'a, F: Fn(PhysicalBlockId, &mut [u8]) -> Result<(), AirKvError>>(&'a F);
struct WriteCtx<'a, F: Fn(PhysicalBlockId, &[u8]) -> Result<(), AirKvError>>(&'a F);

/// The status a failed closure hands back to the library: its own code when
/// it carries an AIR_KV_E_* value, AIR_KV_E_HIP (a device copy failed) otherwise.
fn closure_status(e: &AirKvError) -> i32 {
    if e.code < 0 { e.code } else { sys::AIR_KV_E_HIP }
}

unsafe extern "C" fn read_tramp<F>(ctx: *mut c_void, b: u32, dst: *mut u8, n: usize) -> i32
where
    F: Fn(PhysicalBlockId, &mut [u8]) -> Result<(), AirKvError>,
{
    let f = &*(ctx as *const ReadCtx<F>);
    match (f.0)(PhysicalBlockId(b), std::slice::from_raw_parts_mut(dst, n)) {
        Ok(()) => sys::AIR_KV_OK,
        Err(e) => closure_status(&e),
    }
}

unsafe extern "C" fn write_tramp<F>(ctx: *mut c_void, b: u32, src: *const u8, n: usize) -> i32
where
    F: Fn(PhysicalBlockId, &[u8]) -> Result<(), AirKvError>,
{
    let f = &*(ctx as *const WriteCtx<F>);
    match (f.0)(PhysicalBlockId(b), std::slice::from_raw_parts(src, n)) {
        Ok(()) => sys::AIR_KV_OK,
        Err(e) => closure_status(&e),
    }
}

/// `read_tramp` instantiated for the type of `_f` (a closure's type has no name).
fn read_tramp_for<F>(_f: &F) -> unsafe extern "C" fn(*mut c_void, u32, *mut u8, usize) -> i32
where
    F: Fn(PhysicalBlockId, &mut [u8]) -> Result<(), AirKvError>,
{
    read_tramp::<F>
}

/// The reference's `&'static str` errors for the swap statuses
/// (src/kv_swap.rs:55-98, src/paged_attention.rs:313-343), one per cause.
fn swap_status_str(rc: i32, not_found: &'static str) -> &'static str {
    match rc {
        sys::AIR_KV_E_NOT_FOUND => not_found,
        sys::AIR_KV_E_OOM => "out of memory — cannot swap in",
        sys::AIR_KV_E_HIP => "device block copy failed",
        sys::AIR_KV_E_INVALID_ARG => "invalid argument",
        _ => "swap failed",
    }
}

fn swap_error(rc: i32) -> AirKvError {
    AirKvError { code: rc, message: last_error() }
}

impl KvSwapManager {
    pub fn new(block_capacity: usize, block_bytes: usize) -> Self {
        let mut raw = ptr::null_mut();
        check(unsafe { sys::air_kv_swap_create(block_capacity as i64, BLOCK_SIZE as i32, block_bytes, &mut raw) })
            .expect("air_kv_swap_create");
        let seq_mgr = SequenceManager { raw: unsafe { sys::air_kv_swap_seq_manager(raw) }, owned: false, block_size: BLOCK_SIZE };
        Self { raw, seq_mgr }
    }

    /// evict (src/kv_swap.rs:50-74) with the reference's infallible closure.
    pub fn evict<F>(&mut self, seq_id: SeqId, gpu_read: F) -> Result<Vec<PhysicalBlockId>, &'static str>
    where
        F: Fn(PhysicalBlockId, &mut [u8]),
    {
        self.try_evict(seq_id, |b, dst| {
            gpu_read(b, dst);
            Ok(())
        })
        .map_err(|e| swap_status_str(e.code, "sequence not found"))
    }

    /// evict with a fallible device read: the first `Err` aborts the evict
    /// before any block is released and comes back as the error (its code
    /// when it is an AIR_KV_E_* value, AIR_KV_E_HIP otherwise).
    pub fn try_evict<F>(&mut self, seq_id: SeqId, gpu_read: F) -> Result<Vec<PhysicalBlockId>, AirKvError>
    where
        F: Fn(PhysicalBlockId, &mut [u8]) -> Result<(), AirKvError>,
    {
        let n = self.seq_mgr.table(seq_id).map_or(0, |t| t.physical_blocks.len());
        let ctx = ReadCtx(&gpu_read);
        let mut ids = vec![0u32; n.max(1)];
        let mut got = 0i32;
        let rc = unsafe {
            sys::air_kv_swap_evict(self.raw, seq_id.0, Some(read_tramp::<F>), &ctx as *const _ as *mut c_void,
                                   ids.as_mut_ptr(), ids.len() as i32, &mut got)
        };
        if rc != sys::AIR_KV_OK {
            return Err(swap_error(rc));
        }
        Ok(ids[..got as usize].iter().map(|&b| PhysicalBlockId(b)).collect())
    }

    /// Evicts with the device pool's own read callback (no host closure).
    pub fn evict_pool(&mut self, seq_id: SeqId, pool: &KvPool) -> Result<Vec<PhysicalBlockId>, AirKvError> {
        let n = self.seq_mgr.table(seq_id).map_or(0, |t| t.physical_blocks.len());
        let mut ids = vec![0u32; n.max(1)];
        let mut got = 0i32;
        check(unsafe {
            sys::air_kv_swap_evict(self.raw, seq_id.0, Some(sys::air_kv_pool_read_cb), pool.raw as *mut c_void,
                                   ids.as_mut_ptr(), ids.len() as i32, &mut got)
        })?;
        Ok(ids[..got as usize].iter().map(|&b| PhysicalBlockId(b)).collect())
    }

    /// restore (src/kv_swap.rs:83-98) with the reference's infallible closure.
    pub fn restore<F>(&mut self, seq_id: SeqId, gpu_write: F) -> Result<Vec<PhysicalBlockId>, &'static str>
    where
        F: Fn(PhysicalBlockId, &[u8]),
    {
        self.try_restore(seq_id, |b, src| {
            gpu_write(b, src);
            Ok(())
        })
        .map_err(|e| swap_status_str(e.code, "no evicted data for sequence"))
    }

    /// restore with a fallible device write; a failed write returns its
    /// error and leaves the sequence evicted (its new blocks freed, its bytes
    /// back in the host store).
    pub fn try_restore<F>(&mut self, seq_id: SeqId, gpu_write: F) -> Result<Vec<PhysicalBlockId>, AirKvError>
    where
        F: Fn(PhysicalBlockId, &[u8]) -> Result<(), AirKvError>,
    {
        let ctx = WriteCtx(&gpu_write);
        let mut ids = vec![0u32; 1 << 16];
        let mut got = 0i32;
        let rc = unsafe {
            sys::air_kv_swap_restore(self.raw, seq_id.0, Some(write_tramp::<F>), &ctx as *const _ as *mut c_void,
                                     ids.as_mut_ptr(), ids.len() as i32, &mut got)
        };
        if rc != sys::AIR_KV_OK {
            return Err(swap_error(rc));
        }
        Ok(ids[..got as usize].iter().map(|&b| PhysicalBlockId(b)).collect())
    }

    /// Restores with the device pool's own write callback (no host closure).
    pub fn restore_pool(&mut self, seq_id: SeqId, pool: &KvPool) -> Result<Vec<PhysicalBlockId>, AirKvError> {
        let mut ids = vec![0u32; 1 << 16];
        let mut got = 0i32;
        check(unsafe {
            sys::air_kv_swap_restore(self.raw, seq_id.0, Some(sys::air_kv_pool_write_cb), pool.raw as *mut c_void,
                                     ids.as_mut_ptr(), ids.len() as i32, &mut got)
        })?;
        Ok(ids[..got as usize].iter().map(|&b| PhysicalBlockId(b)).collect())
    }

    pub fn is_evicted(&self, seq_id: SeqId) -> bool {
        unsafe { sys::air_kv_swap_is_evicted(self.raw, seq_id.0) == 1 }
    }

    pub fn evicted_count(&self) -> usize {
        unsafe { sys::air_kv_swap_evicted_count(self.raw) as usize }
    }

    pub fn cpu_bytes_used(&self) -> usize {
        unsafe { sys::air_kv_swap_cpu_bytes_used(self.raw) as usize }
    }

    /// maybe_evict (src/kv_swap.rs:112-121): true when an eviction happened.
    pub fn maybe_evict<F>(&mut self, seq_id: SeqId, free_threshold: usize, gpu_read: F) -> bool
    where
        F: Fn(PhysicalBlockId, &mut [u8]),
    {
        let f = |b: PhysicalBlockId, dst: &mut [u8]| -> Result<(), AirKvError> {
            gpu_read(b, dst);
            Ok(())
        };
        let ctx = ReadCtx(&f);
        let mut ev = 0i32;
        let rc = unsafe {
            sys::air_kv_swap_maybe_evict(self.raw, seq_id.0, free_threshold as i64, Some(read_tramp_for(&f)),
                                         &ctx as *const _ as *mut c_void, &mut ev)
        };
        rc == sys::AIR_KV_OK && ev != 0
    }
}

impl Drop for KvSwapManager {
    fn drop(&mut self) {
        unsafe { sys::air_kv_swap_destroy(self.raw) };
    }
}

unsafe impl Send for KvSwapManager {}

// ---------------------------------------------------------------------------
// The device pool (one layer's K / V pages on the current HIP device)
// ---------------------------------------------------------------------------

/// Element type of a pool's pages.
#[derive(Debug, Clone, Copy, PartialEq, Eq)]
pub enum KvDtype {
    F32 = 0,
    Bf16 = 1,
    /// Q8_0 codes + one f32 scale per `scale_group` elements (src/kv_cache.rs:54-75)
    Int8 = 2,
    /// the reference E4M3 encoding + f32 scales (src/fp8.rs:54-112)
    Fp8 = 3,
}

/// A device stream (`hipStream_t`); null is the default stream.
pub type Stream = *mut c_void;

pub struct KvPool {
    raw: *mut sys::air_kv_pool,
    pub desc: sys::air_kv_pool_desc,
    pub block_bytes: usize,
}

impl KvPool {
    pub fn new(num_blocks: usize, block_size: usize, n_kv_heads: usize, head_dim: usize, dtype: KvDtype)
               -> Result<Self, AirKvError> {
        let desc = sys::air_kv_pool_desc {
            num_blocks: num_blocks as i64,
            block_size: block_size as i32,
            n_kv_heads: n_kv_heads as i32,
            head_dim: head_dim as i32,
            dtype: dtype as i32,
            scale_group: 32,
        };
        let mut raw = ptr::null_mut();
        check(unsafe { sys::air_kv_pool_create(&desc, &mut raw) })?;
        let mut d = desc;
        let (mut k, mut v, mut ks, mut vs) = (ptr::null_mut(), ptr::null_mut(), ptr::null_mut(), ptr::null_mut());
        let mut bb = 0usize;
        check(unsafe { sys::air_kv_pool_info(raw, &mut d, &mut k, &mut v, &mut ks, &mut vs, &mut bb) })?;
        Ok(Self { raw, desc: d, block_bytes: bb })
    }

    /// Reshape-and-cache of `n_tokens` f32 K/V rows (device pointers) into
    /// `slot_mapping` (device int64).
    ///
    /// # Safety
    /// The pointers are device memory of the sizes the C ABI documents.
    pub unsafe fn append(&self, stream: Stream, k: *const f32, v: *const f32, slot_mapping: *const i64,
                         n_tokens: usize) -> Result<(), AirKvError> {
        check(sys::air_kv_append(self.raw, stream, k, v, slot_mapping, n_tokens as i32)).map(|_| ())
    }

    /// Workspace bytes of one paged decode launch shape.
    pub fn decode_workspace_size(&self, n_q_heads: usize, batch: usize, max_blocks: usize, max_splits: usize)
                                 -> Result<usize, AirKvError> {
        let mut n = 0usize;
        check(unsafe {
            sys::air_paged_decode_workspace_size(self.raw, n_q_heads as i32, batch as i32, max_blocks as i32,
                                                 max_splits as i32, &mut n)
        })?;
        Ok(n)
    }

    /// Split-K paged decode: `out = softmax(q . K^T * scale) . V` per query
    /// head over each sequence's pages.
    ///
    /// # Safety
    /// Every pointer is device memory of the documented shape.
    #[allow(clippy::too_many_arguments)]
    pub unsafe fn paged_decode(&self, stream: Stream, q: *const c_void, q_dtype: KvDtype, n_q_heads: usize,
                               tables: *const i32, lens: *const i32, batch: usize, max_blocks: usize,
                               scale: f32, max_splits: usize, workspace: *mut c_void, ws_bytes: usize,
                               out: *mut c_void, out_dtype: KvDtype) -> Result<(), AirKvError> {
        check(sys::air_paged_decode(self.raw, stream, q, q_dtype as i32, n_q_heads as i32, tables, lens,
                                    batch as i32, max_blocks as i32, scale, max_splits as i32, workspace,
                                    ws_bytes, out, out_dtype as i32))
            .map(|_| ())
    }

    /// One decode step: appends `k_new` / `v_new` (f32
    /// `[batch][n_kv_heads][head_dim]`, 16-byte aligned) as each sequence's
    /// token `lens[b] - 1`, then attends as [`KvPool::paged_decode`]
    /// (src/model.rs:569-577).  One launch on bf16, int8 and fp8 pools with
    /// head_dim 128 and group 1..16; append, then decode, on every other pool.
    ///
    /// # Safety
    /// As [`KvPool::paged_decode`]; `k_new` / `v_new` are device arrays of
    /// `batch * n_kv_heads * head_dim` floats.
    #[allow(clippy::too_many_arguments)]
    pub unsafe fn paged_decode_append(&self, stream: Stream, q: *const c_void, q_dtype: KvDtype,
                                      n_q_heads: usize, k_new: *const f32, v_new: *const f32,
                                      tables: *const i32, lens: *const i32, batch: usize, max_blocks: usize,
                                      scale: f32, max_splits: usize, workspace: *mut c_void, ws_bytes: usize,
                                      out: *mut c_void, out_dtype: KvDtype) -> Result<(), AirKvError> {
        check(sys::air_paged_decode_append(self.raw, stream, q, q_dtype as i32, n_q_heads as i32, k_new, v_new,
                                           tables, lens, batch as i32, max_blocks as i32, scale,
                                           max_splits as i32, workspace, ws_bytes, out, out_dtype as i32))
            .map(|_| ())
    }

    /// The same decode with the library's own workspace array (for callers
    /// that cannot allocate device memory).
    ///
    /// # Safety
    /// As [`KvPool::paged_decode`].
    #[allow(clippy::too_many_arguments)]
    pub unsafe fn paged_decode_noalloc(&self, stream: Stream, q: *const c_void, q_dtype: KvDtype, n_q_heads: usize,
                                       tables: *const i32, lens: *const i32, batch: usize, max_blocks: usize,
                                       scale: f32, max_splits: usize, out: *mut c_void, out_dtype: KvDtype)
                                       -> Result<(), AirKvError> {
        check(sys::air_paged_decode_noalloc(self.raw, stream, q, q_dtype as i32, n_q_heads as i32, tables, lens,
                                            batch as i32, max_blocks as i32, scale, max_splits as i32, out,
                                            out_dtype as i32))
            .map(|_| ())
    }

    /// Copies whole blocks src[i] -> dst[i] (device int32 lists): the page
    /// copy that `cow_write` leaves undone.
    ///
    /// # Safety
    /// `src` / `dst` are device arrays of `n` ids.
    pub unsafe fn copy_blocks(&self, stream: Stream, src: *const i32, dst: *const i32, n: usize)
                              -> Result<(), AirKvError> {
        check(sys::air_kv_copy_blocks(self.raw, stream, src, dst, n as i32)).map(|_| ())
    }

    /// Whole blocks to host memory (`out.len() == ids.len() * block_bytes`).
    pub fn read_blocks(&self, stream: Stream, ids: &[i32], out: &mut [u8]) -> Result<(), AirKvError> {
        assert_eq!(out.len(), ids.len() * self.block_bytes);
        check(unsafe { sys::air_kv_read_blocks(self.raw, stream, ids.as_ptr(), ids.len() as i32, out.as_mut_ptr() as _) })
            .map(|_| ())
    }

    /// Host bytes back into whole blocks.
    pub fn write_blocks(&self, stream: Stream, ids: &[i32], src: &[u8]) -> Result<(), AirKvError> {
        assert_eq!(src.len(), ids.len() * self.block_bytes);
        check(unsafe { sys::air_kv_write_blocks(self.raw, stream, ids.as_ptr(), ids.len() as i32, src.as_ptr() as _) })
            .map(|_| ())
    }

    /// Skipped out-of-range slots / table entries since creation or the last reset.
    pub fn error_count(&self, stream: Stream, reset: bool) -> Result<i64, AirKvError> {
        let mut n = 0i64;
        check(unsafe { sys::air_kv_pool_error_count(self.raw, stream, &mut n, reset as i32) })?;
        Ok(n)
    }

    /// `flash_decode` (src/flash_decode.rs:153-173) over paged storage for
    /// one sequence: `out[h] = softmax(q[h] . K^T / sqrt(head_dim)) . V` for
    /// each of the `n_q_heads` query heads over the sequence's `kv_len`
    /// cached tokens, kv head `h / (n_q_heads / n_kv_heads)`.  The reference
    /// cuts the sequence into `chunk_size`-token chunks and merges their
    /// partials by log-sum-exp; here `chunk_size` sets the split-K bound
    /// (`ceil(kv_len / chunk_size)` pieces at most, 1..256) and the kernel
    /// does the same merge.  `q` / `out` are f32 `[n_q_heads][head_dim]`,
    /// `block_table` int32 `[max_blocks]` and `kv_len_dev` one int32 equal to
    /// `kv_len`, all device memory; the workspace is
    /// [`KvPool::decode_workspace_size`]`(n_q_heads, 1, max_blocks, splits)`
    /// bytes, splits as returned by [`KvPool::flash_decode_splits`].
    ///
    /// # Safety
    /// Every pointer is device memory of the stated shape.
    #[allow(clippy::too_many_arguments)]
    pub unsafe fn flash_decode(&self, stream: Stream, q: *const f32, n_q_heads: usize, block_table: *const i32,
                               max_blocks: usize, kv_len: usize, kv_len_dev: *const i32, chunk_size: usize,
                               workspace: *mut c_void, ws_bytes: usize, out: *mut f32) -> Result<(), AirKvError> {
        let scale = 1.0 / (self.desc.head_dim as f32).sqrt();
        self.paged_decode(stream, q as *const c_void, KvDtype::F32, n_q_heads, block_table, kv_len_dev, 1, max_blocks,
                          scale, Self::flash_decode_splits(kv_len, chunk_size), workspace, ws_bytes,
                          out as *mut c_void, KvDtype::F32)
    }

    /// The split-K bound [`KvPool::flash_decode`] uses: one piece per
    /// `chunk_size` tokens, 1..256.
    pub fn flash_decode_splits(kv_len: usize, chunk_size: usize) -> usize {
        assert!(chunk_size > 0);
        kv_len.div_ceil(chunk_size).clamp(1, 256)
    }

    pub fn as_raw(&self) -> *mut sys::air_kv_pool {
        self.raw
    }
}

impl Drop for KvPool {
    fn drop(&mut self) {
        unsafe { sys::air_kv_pool_destroy(self.raw) };
    }
}

unsafe impl Send for KvPool {}

// ---------------------------------------------------------------------------
// SessionKvCache (src/kv_cache.rs:431-446) over paged pools
// ---------------------------------------------------------------------------

/// One layer's dense K / V in device memory, `[n_tokens][n_kv_heads][head_dim]`
/// each as `dtype`: the paged cache's form of `LayerCache::Attention`
/// (src/kv_cache.rs:121-122) without candle tensors.
#[derive(Debug, Clone, Copy)]
pub struct LayerCache {
    pub k: *mut c_void,
    pub v: *mut c_void,
    pub n_tokens: usize,
    pub dtype: KvDtype,
}

/// The reference's per-session cache trait (src/kv_cache.rs:431-446), with
/// device buffers in place of candle tensors and [`AirKvError`] in place of
/// `candle_core::Error`.
pub trait SessionKvCache {
    /// Tokens stored for `layer` (0 if empty).
    fn seq_len(&self, layer: usize) -> usize;
    /// The layer's cache becomes `cache`'s rows (f32): rows past the stored
    /// length are appended; fewer rows shorten the layer.
    ///
    /// # Safety
    /// `cache.k` / `cache.v` are device arrays of `cache.n_tokens` f32 rows.
    unsafe fn save(&mut self, layer: usize, cache: LayerCache) -> Result<(), AirKvError>;
    /// Writes the layer's tokens into `into` (F32 or Bf16; 1-byte pools are
    /// dequantized) and returns it with `n_tokens = seq_len(layer)`.
    ///
    /// # Safety
    /// `into.k` / `into.v` are device arrays of at least `seq_len(layer)` rows.
    unsafe fn load(&self, layer: usize, into: LayerCache) -> Result<LayerCache, AirKvError>;
    /// Every layer empty, all blocks released.
    fn clear(&mut self);
    /// Every layer keeps at most `pos` tokens.
    fn truncate_to(&mut self, pos: usize);
}

/// A session's KV cache on paged device pools (one per layer), for one
/// sequence of a [`SequenceManager`]: the `KvCacheManager` of
/// src/kv_cache.rs:205-414 with paged storage.  It borrows the manager and
/// the pools; it is neither `Send` nor `Sync` (sessions of one manager
/// mutate it through the C ABI and must stay on one thread).
pub struct PagedSessionCache<'a> {
    raw: *mut sys::air_kv_session,
    /// Stream for the device work of `save` / `load` / `append`.
    pub stream: Stream,
    _borrow: PhantomData<(&'a SequenceManager, &'a KvPool)>,
}

impl<'a> PagedSessionCache<'a> {
    /// A new sequence in `mgr` with one pool per layer.
    pub fn new(mgr: &'a SequenceManager, layer_pools: &[&'a KvPool], stream: Stream) -> Result<Self, AirKvError> {
        let raws: Vec<*mut sys::air_kv_pool> = layer_pools.iter().map(|p| p.raw).collect();
        let mut raw = ptr::null_mut();
        check(unsafe { sys::air_kv_session_create(mgr.raw, raws.as_ptr(), raws.len() as i32, &mut raw) })?;
        Ok(Self { raw, stream, _borrow: PhantomData })
    }

    /// A session on `fork_sequence` of this one (src/paged_attention.rs:290-310):
    /// blocks are shared until either session writes into one.
    pub fn fork(&self) -> Result<PagedSessionCache<'a>, AirKvError> {
        let mut raw = ptr::null_mut();
        check(unsafe { sys::air_kv_session_fork(self.raw, &mut raw) })?;
        Ok(Self { raw, stream: self.stream, _borrow: PhantomData })
    }

    pub fn seq_id(&self) -> SeqId {
        let mut s = 0u32;
        check(unsafe { sys::air_kv_session_seq_id(self.raw, &mut s) }).expect("air_kv_session_seq_id");
        SeqId(s)
    }

    /// Appends `n_new` f32 rows after the layer's stored tokens (the decode
    /// step's reshape-and-cache).
    ///
    /// # Safety
    /// `k` / `v` are device arrays of `n_new` f32 rows.
    pub unsafe fn append(&mut self, layer: usize, k: *const f32, v: *const f32, n_new: usize)
                         -> Result<(), AirKvError> {
        check(sys::air_kv_session_append(self.raw, self.stream, layer as i32, k, v, n_new as i64)).map(|_| ())
    }

    /// Device bytes of the session's blocks over all layers (src/kv_cache.rs:388-414).
    pub fn memory_usage(&self) -> usize {
        let mut n = 0usize;
        check(unsafe { sys::air_kv_session_memory_usage(self.raw, &mut n) }).expect("air_kv_session_memory_usage");
        n
    }
}

impl SessionKvCache for PagedSessionCache<'_> {
    fn seq_len(&self, layer: usize) -> usize {
        let mut n = 0i64;
        match check(unsafe { sys::air_kv_session_seq_len(self.raw, layer as i32, &mut n) }) {
            Ok(_) => n as usize,
            Err(_) => 0,
        }
    }

    unsafe fn save(&mut self, layer: usize, cache: LayerCache) -> Result<(), AirKvError> {
        if cache.dtype != KvDtype::F32 {
            return Err(AirKvError { code: sys::AIR_KV_E_INVALID_ARG, message: "save takes f32 rows".into() });
        }
        check(sys::air_kv_session_save(self.raw, self.stream, layer as i32, cache.k as *const f32,
                                       cache.v as *const f32, cache.n_tokens as i64))
            .map(|_| ())
    }

    unsafe fn load(&self, layer: usize, into: LayerCache) -> Result<LayerCache, AirKvError> {
        check(sys::air_kv_session_load(self.raw, self.stream, layer as i32, into.k, into.v, into.dtype as i32))?;
        Ok(LayerCache { n_tokens: self.seq_len(layer), ..into })
    }

    fn clear(&mut self) {
        check(unsafe { sys::air_kv_session_clear(self.raw) }).expect("air_kv_session_clear");
    }

    fn truncate_to(&mut self, pos: usize) {
        check(unsafe { sys::air_kv_session_truncate_to(self.raw, pos.min(i64::MAX as usize) as i64) })
            .expect("air_kv_session_truncate_to");
    }
}

impl Drop for PagedSessionCache<'_> {
    fn drop(&mut self) {
        unsafe { sys::air_kv_session_destroy(self.raw) };
    }
}

// ---------------------------------------------------------------------------
// KvBlock wire format (src/pd_disagg.rs:39-104)
// ---------------------------------------------------------------------------

/// A KV block on the wire: bf16 `[block_size][n_kv_heads][head_dim][K|V]`.
#[derive(Debug, Clone, PartialEq, Eq)]
pub struct KvBlock {
    pub block_id: u32,
    pub layer_idx: u16,
    pub data: Vec<u8>,
}

impl KvBlock {
    /// `[block_id:4][layer_idx:2][data_len:4][data]`.
    pub fn serialise(&self) -> Vec<u8> {
        let mut out = vec![0u8; unsafe { sys::air_kv_block_frame_bytes(self.data.len()) }];
        let mut w = 0usize;
        check(unsafe {
            sys::air_kv_block_serialise(self.block_id, self.layer_idx, self.data.as_ptr() as _, self.data.len(),
                                        out.as_mut_ptr() as _, out.len(), &mut w)
        })
        .expect("KvBlock::serialise");
        out.truncate(w);
        out
    }

    pub fn deserialise(buf: &[u8]) -> Option<Self> {
        let (mut id, mut layer, mut data, mut n) = (0u32, 0u16, ptr::null(), 0usize);
        let rc = unsafe {
            sys::air_kv_block_deserialise(buf.as_ptr() as _, buf.len(), &mut id, &mut layer, &mut data, &mut n)
        };
        (rc == sys::AIR_KV_OK).then(|| KvBlock { block_id: id, layer_idx: layer, data: buf[10..10 + n].to_vec() })
    }
}
