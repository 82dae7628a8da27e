"""The C-ABI library loads without a GPU and exports every symbol that
include/*.h declares (no device calls are made here)."""
import ctypes
import glob
import os
import re
import subprocess

import airkv
from airkv import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        src = open(h).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        src = re.sub(r"//[^\n]*", "", src)
        for m in re.finditer(r"^\s*(?:[A-Za-z_][\w\s\*]*?)\b(air_[a-z0-9_]+)\s*\(", src, re.M):
            if "typedef" in src[max(0, m.start() - 0):m.end()].splitlines()[-1]:
                continue
            names.add(m.group(1))
    return names


def test_header_declares_the_expected_surface():
    names = declared_functions()
    for must in ("air_kv_pool_create", "air_kv_append", "air_kv_gather", "air_paged_decode",
                 "air_paged_decode_workspace_size", "air_kv_copy_blocks", "air_kv_read_blocks",
                 "air_kv_write_blocks", "air_seq_append_slots", "air_kv_swap_evict",
                 "air_block_allocator_cow_write", "air_kv_last_error"):
        assert must in names


def test_library_exports_every_declared_symbol():
    L = airkv.load()
    names = declared_functions()
    missing = [n for n in sorted(names) if not hasattr(L, n)]
    assert not missing, missing
    # the Python binding declares a signature for every one of them
    assert names == set(_lib.SIGNATURES), names ^ set(_lib.SIGNATURES)


def test_exported_symbols_are_c_linkage():
    out = subprocess.run(["nm", "-D", "--defined-only", airkv.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    for n in declared_functions():
        assert n in exported, n


def test_errors_are_reported_not_aborted():
    L = airkv.load()
    desc = _lib.PoolDesc(0, 16, 8, 128, airkv.BF16, 32)
    h = ctypes.c_void_p()
    rc = L.air_kv_pool_create(ctypes.byref(desc), ctypes.byref(h))
    assert rc == airkv.AIR_KV_E_INVALID_ARG
    assert "num_blocks" in airkv.last_error()
    desc = _lib.PoolDesc(4, 24, 8, 128, airkv.BF16, 32)
    assert L.air_kv_pool_create(ctypes.byref(desc), ctypes.byref(h)) == airkv.AIR_KV_E_INVALID_ARG
    assert "block_size" in airkv.last_error()
    assert L.air_kv_append(None, None, None, None, None, 1) == airkv.AIR_KV_E_INVALID_ARG


def test_last_error_truncates_safely():
    L = airkv.load()
    L.air_seq_create(None, None)
    buf = ctypes.create_string_buffer(4)
    n = L.air_kv_last_error(buf, 4)
    assert n > 3 and len(buf.value) == 3
