"""Pin the oracle's dequant-fused linear kernels against the FP64 closed
form the reference's tests use, plus batch/worker invariance and the wide
(FP64) fallback (q8_test.go:55-131, q4_test.go:145-191)."""
import numpy as np
import pytest

import oracle

FMAX = np.float32(np.finfo(np.float32).max)


def near(got, want, tol=2e-5):
    got = np.asarray(got, np.float64)
    assert np.all(np.isfinite(got))
    bound = tol * np.maximum(1.0, np.abs(want))
    bad = np.abs(got - want) > bound
    assert not bad.any(), (np.argwhere(bad)[:5], got[bad][:5], want[bad][:5])


@pytest.mark.parametrize("cols", [1, 2, 63, 64, 65, 129, 513])
def test_q8_linear_closed_form_and_invariance(cols):
    x, dense = oracle.linear_fixture(7, cols, 259)
    w = oracle.Weight.from_dense(dense, oracle.Q8)
    recon = w.dequant().astype(np.float64)
    want = x.astype(np.float64) @ recon.T
    base = None
    for workers in (1, 2, 4):
        got = oracle.linear(w, x, workers)
        near(got, want.astype(np.float32).astype(np.float64))
        if base is None:
            base = got
        assert np.array_equal(got.view(np.uint32), base.view(np.uint32))
        for r in range(7):
            one = oracle.linear(w, x[r:r + 1], workers)
            assert np.array_equal(one.view(np.uint32), got[r:r + 1].view(np.uint32))


def test_q8_extreme_activations_finite_and_invariant():
    x, dense = oracle.linear_fixture(7, 65, 259)
    dense = ((np.arange(dense.size) % 13 - 6).astype(np.float32) * np.float32(0.0001)).reshape(dense.shape)
    x = x.copy()
    x[2, 0] = FMAX / np.float32(4)
    x[5, 64] = np.float32(-1e37)
    w = oracle.Weight.from_dense(dense, oracle.Q8)
    want = oracle.linear_closed_f64(w, x)
    base = None
    for workers in (1, 2, 4):
        got = oracle.linear(w, x, workers)
        for r in range(7):
            one = oracle.linear(w, x[r:r + 1], workers)
            assert np.array_equal(one.view(np.uint32), got[r:r + 1].view(np.uint32))
            near(one[0], want[r])
        if base is None:
            base = got
        assert np.array_equal(got.view(np.uint32), base.view(np.uint32))


@pytest.mark.parametrize("cols", [1, 2, 3, 4, 63, 64, 65, 129, 513])
@pytest.mark.parametrize("extreme", [False, True])
def test_q4_linear_closed_form_and_invariance(cols, extreme):
    x, dense = oracle.linear_fixture(7, cols, 259)
    x = x.copy()
    if extreme:
        dense = dense * np.float32(0.001)
        x[2, 0] = FMAX / np.float32(4)
        x[5, cols - 1] = np.float32(-1e37)
    w = oracle.Weight.from_dense(dense, oracle.Q4)
    want = oracle.linear_closed_f64(w, x)
    base = None
    for workers in (1, 2, 4):
        got = oracle.linear(w, x, workers)
        for r in range(7):
            one = oracle.linear(w, x[r:r + 1], workers)
            assert np.array_equal(one.view(np.uint32), got[r:r + 1].view(np.uint32))
            near(one[0], want[r])
        if base is None:
            base = got
        assert np.array_equal(got.view(np.uint32), base.view(np.uint32))


@pytest.mark.parametrize("n", [1, 2, 3, 4, 5, 8])
def test_f32_linear_closed_form(n):
    x, dense = oracle.linear_fixture(n, 97, 70)
    w = oracle.Weight.from_dense(dense, oracle.F32)
    got = oracle.linear(w, x, 2)
    near(got, x.astype(np.float64) @ dense.astype(np.float64).T)


def test_wide_threshold_is_per_row():
    """q8NeedsWideSum (M:4346-4354) chooses per row: a neighbour's extreme
    value must not change an ordinary row's bits."""
    x, dense = oracle.linear_fixture(3, 130, 40)
    w = oracle.Weight.from_dense(dense, oracle.Q8)
    plain = oracle.linear(w, x)
    x2 = x.copy()
    x2[1, 7] = np.float32(3e34)
    mixed = oracle.linear(w, x2)
    assert np.array_equal(mixed[0].view(np.uint32), plain[0].view(np.uint32))
    assert np.array_equal(mixed[2].view(np.uint32), plain[2].view(np.uint32))
    # limit = f32(MaxFloat32 / (2*64*127)); exactly representable check
    limit = np.float32(float(FMAX) / (2 * 64 * 127))
    x3 = x.copy()
    x3[0, 0] = limit  # not above the limit -> ordinary path, may overflow nothing
    assert np.all(np.isfinite(oracle.linear(w, x3[:1]) * 0 + 1))


def test_sizes_zero_scale_and_negative_zero():
    """Zero blocks give zero scales and zero codes; -0 inputs stay harmless
    (q8_block_test.go:127-167)."""
    dense = np.zeros((33, 129), np.float32)
    dense[3, 5] = 1.0
    w = oracle.Weight.from_dense(dense, oracle.Q8)
    assert w.scales[0, 0] == 0 and w.scales[3, 0] == np.float32(1.0 / 127)
    x = np.full((2, 129), -0.0, np.float32)
    y = oracle.linear(w, x)
    assert np.all(y == 0)
