"""srq_linear_noalloc through the C ABI: the entry point that allocates
nothing (split-K scratch in the library's fixed device array) gives the
same bits as srq_linear on the same inputs, over two calls in a row whose
second is smaller (the array keeps the first call's contents), on the GEMM
path with split-K slices, on the GEMV path, and for Q4; a call whose plan
needs more scratch than the array holds runs in GEMM sub-batches, with the
same bits."""
import numpy as np
import pytest

import oracle
import sr_go_tranformer_amd as srq

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ex():
    e = srq.Executor(0)
    yield e
    e.close()


def run(ex, entry, w, x):
    n = x.shape[0]
    xb = ex.upload(np.ascontiguousarray(x, np.float32))
    yb = ex.empty(n * w.rows * 4)
    srq.check(getattr(srq.lib(), entry)(ex.h, yb.ptr, xb.ptr, w.h, n))
    ex.synchronize()
    return yb.to_numpy(np.float32, (n, w.rows))


@pytest.mark.parametrize("fmt,rows,cols,ns", [(srq.Q8, 4096, 4096, (200, 40)), (srq.Q4, 6144, 4096, (64, 17)),
                                              (srq.Q8, 2048, 1024, (7, 3))])
def test_noalloc_matches_linear(ex, fmt, rows, cols, ns):
    print("noalloc", fmt, rows, cols, ns, flush=True)
    rng = oracle.RNG(rows + cols)
    dense = rng.fill_normal(rows * cols, 0.02).reshape(rows, cols)
    w = srq.Weight.create(ex, dense, fmt)
    ow = oracle.Weight.from_dense(dense, oracle.Q8 if fmt == srq.Q8 else oracle.Q4)
    for n in ns:
        x = rng.fill_normal(n * cols, 1.0).reshape(n, cols)
        got = run(ex, "srq_linear_noalloc", w, x)
        want = run(ex, "srq_linear", w, x)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (n, float(np.abs(got - want).max()))
        ref = oracle.linear(ow, x, workers=8)
        err = np.abs(got.astype(np.float64) - ref) / np.maximum(1.0, np.abs(ref))
        assert err.max() <= 1e-4, (n, float(err.max()))


def test_noalloc_large_calls_run_in_sub_batches(ex):
    """1024 rows of an 8192 x 4096 Q8 matrix need 4 x 1024 x 8193 x 4 bytes
    of split-K scratch, above the 64 MiB array: the call runs as three GEMM
    sub-batches of 342 / 341 / 341 rows, bit-identical to srq_linear, and a
    smaller call afterwards still matches."""
    rows, cols = 8192, 4096
    rng = oracle.RNG(9)
    w = srq.Weight.create(ex, rng.fill_normal(rows * cols, 0.02).reshape(rows, cols), srq.Q8)
    for n in (1024, 600, 24):
        x = rng.fill_normal(n * cols, 1.0).reshape(n, cols)
        got = run(ex, "srq_linear_noalloc", w, x)
        want = run(ex, "srq_linear", w, x)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), n
