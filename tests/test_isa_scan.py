"""CPU scan of the built gfx950 code objects: no kernel writes through the
scalar data cache (scalar stores, scalar atomics, scalar cache write-back),
whatever the compiler chose for uniform addresses (e.g. the completion
tickets and counters).  Uses llvm-objdump on code built here."""
import glob
import os
import re
import subprocess

import pytest

import catena_amd as ca

FORBIDDEN = re.compile(r"\bs_(store_dword\w*|buffer_store\w*|scratch_store\w*|atomic_\w+|"
                       r"buffer_atomic_\w+|dcache_wb\w*|dcache_discard\w*)\b")


def test_no_scalar_cache_writes():
    tool = "/opt/rocm/llvm/bin/llvm-objdump"
    if not os.path.exists(tool):
        pytest.skip("llvm-objdump not available")
    objs = sorted(glob.glob(os.path.join(ca.LIB_DIR, "*.co")))
    assert objs
    for path in objs:
        text = subprocess.run([tool, "-d", "--mcpu=gfx950", path], capture_output=True, text=True,
                              check=True).stdout
        hits = sorted(set(FORBIDDEN.findall(text)))
        assert not hits, (os.path.basename(path), hits)
