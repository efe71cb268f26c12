"""The gfx950 code of every HIP source writes memory through vector
instructions only: no scalar-cache stores, scalar atomics or scalar-cache
write-back/discard instructions appear in the compiler's assembly.

CPU-only: compiles each source with the library's own flags to assembly
(in parallel)."""
import concurrent.futures
import os
import re
import subprocess
import tempfile

import pytest

from sr_go_tranformer_amd import build as B

FORBIDDEN = re.compile(r"^\s*(s_store_|s_buffer_store|s_scratch_store|s_atomic_|s_buffer_atomic_|s_dcache_wb|"
                       r"s_dcache_discard)", re.M)
SOURCES = [s for s in B.SOURCES if s.endswith(".hip")]


def _assembly(src, tmp):
    out = os.path.join(tmp, src + ".s")
    cmd = [B.HIPCC, "-x", "hip", "--cuda-device-only", "-S"] + B.FLAGS + [
        "-I", os.path.join(B.HERE, "..", "include"), os.path.join(B.CSRC, src), "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, (src, r.stderr[-2000:])
    return src, open(out).read()


@pytest.mark.skipif(not os.path.exists(B.HIPCC), reason="hipcc not available")
def test_no_scalar_memory_writes():
    with tempfile.TemporaryDirectory() as tmp:
        with concurrent.futures.ThreadPoolExecutor(len(SOURCES)) as pool:
            results = list(pool.map(lambda s: _assembly(s, tmp), SOURCES))
    for src, asm in results:
        assert "gfx950" in asm, src
        hits = FORBIDDEN.findall(asm)
        assert not hits, (src, hits[:10])
