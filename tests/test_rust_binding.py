"""The Rust binding source (air.rs_amd/rust: the airkv-sys raw crate and the
airkv safe wrapper) stays in step with include/air_kv.h.  No Rust toolchain
exists in this image, so the crates are checked as text: the generated
extern block equals what its generator writes from the header, it declares
every function the header declares, and the safe wrapper calls only declared
functions.  CPU only."""
import os
import re
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
RUST = os.path.join(ROOT, "air.rs_amd", "rust")
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
from test_abi import declared_functions  # noqa: E402


def _sys_src():
    return open(os.path.join(RUST, "airkv-sys", "src", "lib.rs")).read()


def test_generated_bindings_are_up_to_date():
    out = subprocess.run([sys.executable, os.path.join(RUST, "gen_sys.py"), "--print"], capture_output=True,
                         text=True, check=True).stdout
    assert out == _sys_src(), "air.rs_amd/rust/airkv-sys/src/lib.rs is stale: run air.rs_amd/rust/gen_sys.py"


def test_sys_crate_declares_every_header_function():
    declared = set(re.findall(r"pub fn (air_[a-z0-9_]+)\(", _sys_src()))
    assert declared == declared_functions(), declared ^ declared_functions()


def test_safe_wrapper_calls_only_declared_functions():
    wrapper = open(os.path.join(RUST, "airkv", "src", "lib.rs")).read()
    # calls, and functions passed as callbacks (Some(sys::air_...))
    used = set(re.findall(r"sys::(air_[a-z0-9_]+)\(", wrapper)) | set(re.findall(r"Some\(sys::(air_[a-z0-9_]+)\)", wrapper))
    declared = set(re.findall(r"pub fn (air_[a-z0-9_]+)\(", _sys_src()))
    assert used and used <= declared, used - declared
    # the reference's SequenceManager / BlockAllocator / KvSwapManager methods are all there
    for name in ("create_sequence", "append_token", "fork_sequence", "free_sequence", "table", "cow_last_block",
                 "num_sequences", "can_schedule", "swap_out", "swap_in", "allocate", "share", "release",
                 "ref_count", "num_free_blocks", "num_used_blocks", "cow_write", "can_allocate",
                 "num_blocks_for_tokens", "utilization", "evict", "restore", "is_evicted", "evicted_count",
                 "maybe_evict", "serialise", "deserialise", "try_evict", "try_restore", "restore_pool",
                 "flash_decode"):
        assert re.search(rf"pub (unsafe )?fn {name}\b", wrapper), name


def test_safe_wrapper_has_session_cache_and_flash_decode():
    """SessionKvCache (src/kv_cache.rs:431-446) as a trait with its five
    methods, implemented by PagedSessionCache over the air_kv_session_*
    calls; flash_decode (src/flash_decode.rs:153-173) as a one-sequence paged
    decode through air_paged_decode."""
    wrapper = open(os.path.join(RUST, "airkv", "src", "lib.rs")).read()
    trait = wrapper[wrapper.index("pub trait SessionKvCache"):]
    trait = trait[:trait.index("\n}\n")]
    for name in ("seq_len", "save", "load", "clear", "truncate_to"):
        assert re.search(rf"fn {name}\(", trait), name
    impl = wrapper[wrapper.index("impl SessionKvCache for PagedSessionCache"):]
    impl = impl[:impl.index("\n}\n")]
    for call in ("air_kv_session_seq_len", "air_kv_session_save", "air_kv_session_load", "air_kv_session_clear",
                 "air_kv_session_truncate_to"):
        assert f"sys::{call}(" in impl, call
    for call in ("air_kv_session_create", "air_kv_session_fork", "air_kv_session_append",
                 "air_kv_session_destroy", "air_kv_session_memory_usage"):
        assert f"sys::{call}(" in wrapper, call
    fd = wrapper[wrapper.index("pub unsafe fn flash_decode("):]
    fd = fd[:fd.index("\n    }\n")]
    assert "self.paged_decode(" in fd and "sqrt()" in fd


def test_swap_closures_report_failures():
    """The fallible swap closures map Err to an AIR_KV_E_* status in the
    trampolines, and evict / restore map each status to its own message
    instead of one catch-all."""
    wrapper = open(os.path.join(RUST, "airkv", "src", "lib.rs")).read()
    for tramp in ("read_tramp", "write_tramp"):
        body = wrapper[wrapper.index(f"unsafe extern \"C\" fn {tramp}"):]
        body = body[:body.index("\n}\n")]
        assert "Err(e) => closure_status(&e)" in body, tramp
    assert "sys::AIR_KV_E_HIP => \"device block copy failed\"" in wrapper
