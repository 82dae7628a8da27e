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
                 "maybe_evict", "serialise", "deserialise"):
        assert re.search(rf"pub fn {name}\b", wrapper), name
