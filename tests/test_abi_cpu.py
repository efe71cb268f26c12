"""CPU-side checks of the C ABI: the HIP library builds for gfx950, loads
without a GPU and exports every entry point include/srq.h declares."""
import os
import re
import subprocess

import pytest

import sr_go_tranformer_amd as srq

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    text = open(os.path.join(ROOT, "include", "srq.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(srq_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = srq.lib()
    names = header_functions()
    assert len(names) >= 35
    out = subprocess.run(["nm", "-D", "--defined-only", srq.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r" T (srq_\w+)", out))
    missing = [n for n in names if n not in exported]
    assert not missing, missing
    for n in names:
        getattr(L, n)
    assert sorted(srq.EXPORTS) == names


def test_abi_version_and_errors_without_device():
    L = srq.lib()
    assert L.srq_abi_version() == 1
    import ctypes as C
    # Null arguments are rejected before any device work, with a message.
    assert L.srq_exec_create(0, None) == srq.EINVAL
    assert b"null" in L.srq_last_error()
    assert L.srq_packed_bytes(srq.Q4, 3, 65, None, None) == srq.OK
    vb, sb = srq.packed_bytes(srq.Q4, 3, 65)
    assert (vb, sb) == (3 * 33, 3 * 2 * 4)
    assert srq.packed_bytes(srq.Q8, 7, 129) == (7 * 129, 7 * 3 * 4)
    assert srq.packed_bytes(srq.F32, 2, 5) == (40, 0)
    assert L.srq_packed_bytes(7, 1, 1, None, None) == srq.EINVAL


def test_built_for_gfx950():
    out = subprocess.run(["/opt/rocm/bin/roc-obj-ls", srq.LIB_PATH], capture_output=True, text=True)
    if out.returncode != 0:
        pytest.skip("roc-obj-ls unavailable")
    assert "gfx950" in out.stdout
