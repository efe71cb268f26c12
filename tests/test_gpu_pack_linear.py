"""GPU parity of packing and the dequant-fused linear kernels against the
oracle (srq_oracle.c), called through the C ABI.

Bars: packing bit-exact (values and scales); linear outputs within
|got - want| <= 1e-4 * max(1, |want|) of the oracle's reference-order f32
result (the reference tests' form, q8_test.go:63-82, at the 1e-4 bound);
batch invariance bit-exact for n <= 16 (one row alone == that row in a
batch, q8_test.go:88-92)."""
import numpy as np
import pytest

import oracle
import sr_go_tranformer_amd as srq

pytestmark = pytest.mark.gpu
TOL = 1e-4
FMAX = np.float32(np.finfo(np.float32).max)
TINY = np.float32(np.finfo(np.float32).smallest_subnormal)


@pytest.fixture(scope="module")
def ex():
    e = srq.Executor(0)
    yield e
    e.close()


def near(got, want, tol=TOL):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert np.all(np.isfinite(got))
    bound = tol * np.maximum(1.0, np.abs(want))
    err = np.abs(got - want)
    bad = err > bound
    assert not bad.any(), (int(bad.sum()), float((err / np.maximum(1, np.abs(want))).max()))


def edge_matrix(rows, cols, seed):
    rng = np.random.default_rng(seed)
    m = rng.normal(0, 0.02, size=(rows, cols)).astype(np.float32)
    specials = np.array([0.0, -0.0, TINY, -TINY, 1e-43, 1e-38, 1e-37, FMAX, -FMAX, 0.5, 1.5, -2.5, 127.0, 63.5, 3.5],
                        np.float32)
    mask = rng.random((rows, cols)) < 0.15
    m[mask] = rng.choice(specials, size=mask.sum())
    return m


@pytest.mark.parametrize("cols", [1, 2, 3, 31, 63, 64, 65, 127, 129, 193, 513, 1000])
@pytest.mark.parametrize("fmt", [srq.Q8, srq.Q4])
def test_pack_bit_exact_edges(ex, cols, fmt):
    print("pack edges", fmt, cols, flush=True)
    m = edge_matrix(9, cols, cols + fmt)
    v, s = srq.pack(ex, m, fmt)
    ov, os_ = oracle.pack(m, oracle.Q8 if fmt == srq.Q8 else oracle.Q4)
    assert np.array_equal(s.view(np.uint32), os_.view(np.uint32))
    assert np.array_equal(v.view(np.uint8), ov.view(np.uint8))


@pytest.mark.parametrize("fmt", [srq.Q8, srq.Q4])
def test_pack_bit_exact_7b_shape(ex, fmt):
    print("pack 14336x4096", fmt, flush=True)
    rng = oracle.RNG(11)
    m = rng.fill_normal(14336 * 4096, 0.02).reshape(14336, 4096)
    v, s = srq.pack(ex, m, fmt)
    ov, os_ = oracle.pack(m, oracle.Q8 if fmt == srq.Q8 else oracle.Q4)
    assert np.array_equal(s.view(np.uint32), os_.view(np.uint32))
    assert np.array_equal(v.view(np.uint8), ov.view(np.uint8))


@pytest.mark.parametrize("dtype", [srq.SRC_BF16, srq.SRC_F16])
def test_pack_half_sources(ex, dtype):
    """F16/BF16 words decode exactly (M:884-920, halfFloat M:838-850)."""
    rng = np.random.default_rng(5)
    words = rng.integers(0, 65536, size=(33, 130), dtype=np.uint32).astype(np.uint16)
    if dtype == srq.SRC_BF16:
        f = (words.astype(np.uint32) << 16).view(np.float32)
    else:
        f = words.view(np.float16).astype(np.float32)
    finite = np.isfinite(f)
    words = np.where(finite, words, np.uint16(0))
    f = np.where(finite, f, np.float32(0))
    for fmt, ofmt in ((srq.Q8, oracle.Q8), (srq.Q4, oracle.Q4)):
        v, s = srq.pack(ex, words, fmt, dtype=dtype)
        ov, os_ = oracle.pack(f, ofmt)
        assert np.array_equal(s.view(np.uint32), os_.view(np.uint32))
        assert np.array_equal(v.view(np.uint8), ov.view(np.uint8))


def test_pack_rejects_nonfinite(ex):
    m = np.zeros((2, 70), np.float32)
    m[1, 66] = np.inf
    with pytest.raises(srq.SrqError) as e:
        srq.pack(ex, m, srq.Q8)
    assert e.value.code == srq.ENONFINITE
    # the executor stays usable and the flag is cleared
    v, s = srq.pack(ex, np.ones((2, 70), np.float32), srq.Q8)
    assert np.all(v == 127)


def test_dequant_rows_match_copy_row(ex):
    rng = oracle.RNG(3)
    dense = rng.fill_normal(40 * 129, 0.02).reshape(40, 129)
    for fmt, ofmt in ((srq.Q8, oracle.Q8), (srq.Q4, oracle.Q4), (srq.F32, oracle.F32)):
        w = srq.Weight.create(ex, dense, fmt)
        ow = oracle.Weight.from_dense(dense, ofmt)
        rows = [0, 39, 7, 7, 20]
        got = w.dequant_rows(ex, rows)
        want = np.stack([ow.copy_row(r) for r in rows])
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def _q4_pairs_closed_form():
    """q4Pairs (M:3811-3817): [b][0] = sext(b & 15), [b][1] = sext(b >> 4)."""
    b = np.arange(256)
    lo, hi = b & 15, b >> 4
    return np.stack([np.where(lo > 7, lo - 16, lo), np.where(hi > 7, hi - 16, hi)], 1).astype(np.float64)


@pytest.mark.parametrize("n", [1, 3, 8, 40])
def test_q4_every_byte_decodes_to_pair_table(ex, n):
    """Every packed Q4 byte, in the GEMV (n <= 16) and MFMA GEMM (n > 16)
    kernels and in dequant_rows, decodes to the shared pair table."""
    print("q4 bytes", n, flush=True)
    rows, cols = 24, 1024  # 512 bytes per row: each byte value twice per row
    rng = np.random.default_rng(n)
    values = np.stack([rng.permutation(np.tile(np.arange(256, dtype=np.uint8), 2)) for _ in range(rows)])
    scales = np.ones((rows, cols // 64), np.float32)
    scales[::3] = np.float32(0.5)  # powers of two keep every product exact
    w = srq.Weight.wrap(ex, srq.Q4, values, scales, cols)
    table = _q4_pairs_closed_form()
    dense = table[values].reshape(rows, cols) * np.repeat(scales.astype(np.float64), 64, axis=1)
    got = w.dequant_rows(ex, list(range(rows)))
    assert np.array_equal(got.astype(np.float64), dense)
    # x of small integers: every partial sum is an exact f32 integer
    x = rng.integers(-3, 4, size=(n, cols)).astype(np.float32)
    y = srq.linear(ex, w, x)
    assert np.array_equal(y.astype(np.float64), x.astype(np.float64) @ dense.T)


def _weights(ex, dense, fmt):
    ofmt = {srq.Q8: oracle.Q8, srq.Q4: oracle.Q4, srq.F32: oracle.F32}[fmt]
    return srq.Weight.create(ex, dense, fmt), oracle.Weight.from_dense(dense, ofmt)


@pytest.mark.parametrize("cols", [1, 2, 3, 4, 63, 64, 65, 129, 513])
@pytest.mark.parametrize("fmt", [srq.Q8, srq.Q4, srq.F32])
def test_linear_reference_fixture_widths(ex, cols, fmt):
    """linearFixture(7, in, 259) widths of q8_test.go:55 / q4_test.go:146."""
    print("linear fixture", fmt, cols, flush=True)
    x, dense = oracle.linear_fixture(7, cols, 259)
    w, ow = _weights(ex, dense, fmt)
    got = srq.linear(ex, w, x)
    near(got, oracle.linear(ow, x))
    near(got, oracle.linear_closed_f64(ow, x), 2e-5 * 5)
    for r in range(7):
        one = srq.linear(ex, w, x[r:r + 1])
        assert np.array_equal(one.view(np.uint32), got[r:r + 1].view(np.uint32))


@pytest.mark.parametrize("fmt", [srq.Q8, srq.Q4])
@pytest.mark.parametrize("cols", [65, 4096])
def test_linear_extreme_activations_wide_path(ex, fmt, cols):
    """q8_test.go:98-131: MaxFloat32/4 and -1e37 inputs stay finite and the
    other rows keep their bits (the FP64 path is chosen per row)."""
    print("linear wide", fmt, cols, flush=True)
    x, dense = oracle.linear_fixture(7, cols, 259)
    x = x.copy()
    dense = dense * np.float32(0.001)
    x[2, 0] = FMAX / np.float32(4)
    x[5, cols - 1] = np.float32(-1e37)
    w, ow = _weights(ex, dense, fmt)
    got = srq.linear(ex, w, x)
    want = oracle.linear_closed_f64(ow, x)
    near(got, want, 2e-5)
    plain = srq.linear(ex, w, x[[0, 1, 3, 4, 6]])
    assert np.array_equal(plain.view(np.uint32), got[[0, 1, 3, 4, 6]].view(np.uint32))


@pytest.mark.parametrize("fmt", [srq.Q8, srq.Q4, srq.F32])
@pytest.mark.parametrize("shape", [(1024, 4096), (4096, 1024), (512, 2048), (300, 14336)])
@pytest.mark.parametrize("n", [1, 2, 3, 4, 5, 8, 9, 16])
def test_linear_gemv_shapes(ex, fmt, shape, n):
    print("gemv", fmt, shape, n, flush=True)
    rows, cols = shape
    rng = oracle.RNG(1000 + rows + n)
    dense = rng.fill_normal(rows * cols, 0.02).reshape(rows, cols)
    x = rng.fill_normal(n * cols, 1.0).reshape(n, cols)
    w, ow = _weights(ex, dense, fmt)
    got = srq.linear(ex, w, x)
    near(got, oracle.linear(ow, x, workers=8))
    one = srq.linear(ex, w, x[n - 1:n])
    assert np.array_equal(one.view(np.uint32), got[n - 1:n].view(np.uint32))


@pytest.mark.parametrize("shape", [(8197, 128), (16390, 1024)])
@pytest.mark.parametrize("n", [4, 5, 8])
def test_linear_gemv_row_groups(ex, shape, n):
    """Q8 GEMV with 4-8 batch rows over 8192+ output rows streams 4 rows
    per step against one read of the activations (row groups), the last
    group ragged (rows not a multiple of 4), rows of one chunk and of
    eight.  Against the oracle, and each batch row's bits equal those of
    its own 1-row launch (one row per step)."""
    print("gemv row groups", shape, n, flush=True)
    rows, cols = shape
    rng = oracle.RNG(77 + rows + n)
    dense = rng.fill_normal(rows * cols, 0.02).reshape(rows, cols)
    x = rng.fill_normal(n * cols, 1.0).reshape(n, cols)
    w, ow = _weights(ex, dense, srq.Q8)
    got = srq.linear(ex, w, x)
    near(got, oracle.linear(ow, x, workers=8))
    for k in range(n):
        one = srq.linear(ex, w, x[k:k + 1])
        assert np.array_equal(one.view(np.uint32), got[k:k + 1].view(np.uint32)), k


@pytest.mark.parametrize("fmt", [srq.Q8, srq.Q4, srq.F32])
@pytest.mark.parametrize("n", [17, 32, 33, 64, 100, 256])
@pytest.mark.parametrize("shape", [(640, 2048), (1000, 256), (300, 8192), (301, 2048)])
def test_linear_gemm_mfma(ex, fmt, n, shape):
    """32-row tiles (n <= 32) and 64-row tiles; K split into slices (narrow
    outputs, long K) and whole-K tiles (K = 256); slice sums four outputs at a
    time (rows % 4 == 0) or one (301 rows)."""
    print("gemm", fmt, n, shape, flush=True)
    rows, cols = shape
    rng = oracle.RNG(77 + n + cols)
    dense = rng.fill_normal(rows * cols, 0.02).reshape(rows, cols)
    x = rng.fill_normal(n * cols, 1.0).reshape(n, cols)
    w, ow = _weights(ex, dense, fmt)
    got = srq.linear(ex, w, x)
    near(got, oracle.linear(ow, x, workers=8))
    # rows keep their bits at any position of a large batch
    perm = np.roll(np.arange(n), 5)
    got2 = srq.linear(ex, w, x[perm])
    assert np.array_equal(got2.view(np.uint32), got[perm].view(np.uint32))


# (rows, cols) -> K slices of 5..16 64-input blocks (the Q8 kernel's
# unrolled instantiations: 5120 x 5120 takes 14, 7168 x 4096 16), last
# slices ragged, 1000 rows a partial tile; 16384 rows take 256-feature tiles.
UNROLLED_SHAPES = [(3072, 3072), (4096, 3072), (5120, 3072), (4096, 4096), (8192, 2304), (5120, 4096),
                   (6144, 4096), (3072, 8192), (16384, 3072), (1000, 704), (5120, 5120), (7168, 4096)]


@pytest.mark.parametrize("shape", UNROLLED_SHAPES)
def test_linear_gemm_unrolled_slices(ex, shape):
    """Q8 GEMM whose K slices hold 5..16 blocks, at 20 rows (32-row tiles)
    and 48 rows (64-row tiles): against the oracle, and the 20 rows keep
    their bits in the 48-row launch."""
    print("gemm unrolled", shape, flush=True)
    rows, cols = shape
    rng = oracle.RNG(5000 + rows + cols)
    dense = rng.fill_normal(rows * cols, 0.02).reshape(rows, cols)
    x = rng.fill_normal(48 * cols, 1.0).reshape(48, cols)
    w, ow = _weights(ex, dense, srq.Q8)
    got20 = srq.linear(ex, w, x[:20])
    near(got20, oracle.linear(ow, x[:20], workers=16))
    got48 = srq.linear(ex, w, x)
    assert np.array_equal(got48[:20].view(np.uint32), got20.view(np.uint32))


@pytest.mark.parametrize("fmt", [srq.Q8, srq.Q4])
@pytest.mark.parametrize("shape", [(200, 1024, 40), (200, 1024, 20), (1000, 256, 40), (1000, 256, 20)])
def test_linear_gemm_wide_rows(ex, shape, fmt):
    """Wide rows found by split-K slices (K = 1024) and by whole-K tiles
    (K = 256), with 32- and 64-row tiles (Q4 64-row tiles: 8 waves)."""
    rows, cols, n = shape
    print("gemm wide rows", fmt, shape, flush=True)
    x, dense = oracle.linear_fixture(n, cols, rows)
    x = x.copy()
    x[3, 5] = FMAX / np.float32(4)
    x[n - 3, 100] = np.float32(-1e37)
    w, ow = _weights(ex, dense * np.float32(0.001), fmt)
    got = srq.linear(ex, w, x)
    near(got, oracle.linear_closed_f64(ow, x), 2e-5)


@pytest.mark.parametrize("fmt", [srq.Q8, srq.Q4])
@pytest.mark.parametrize("n", [20, 64, 256])
@pytest.mark.parametrize("biased", [False, True])
def test_gemm_error_is_fp32_class(ex, fmt, n, biased):
    """The Q8/Q4 GEMM runs on bf16 MFMA with every activation split into
    three bf16 terms, which is exact; its error against the FP64 dot product
    of the same codes stays at FP32-accumulation level (2e-6 of sum |x||w|).
    biased: activations with their 8 low mantissa bits set and weights >= 0,
    so a dropped lowest term would err the same way on every product
    (~3e-5 of sum |x||w|) instead of averaging out."""
    print("gemm fp32 class", fmt, n, biased, flush=True)
    rows, cols = 384, 4096
    rng = np.random.default_rng(n + 7 * biased)
    dense = rng.normal(0, 0.02, size=(rows, cols)).astype(np.float32)
    x = rng.normal(0, 1.0, size=(n, cols)).astype(np.float32)
    if biased:
        dense = np.abs(dense)
        x = rng.uniform(1.0, 2.0, size=(n, cols)).astype(np.float32)
        x = (x.view(np.uint32) | np.uint32(0xFF)).view(np.float32)
    w, ow = _weights(ex, dense, fmt)
    got = srq.linear(ex, w, x).astype(np.float64)
    exact = oracle.linear_closed_f64(ow, x)
    mag = np.abs(x).astype(np.float64) @ np.abs(ow.dequant()).astype(np.float64).T
    err = (np.abs(got - exact) / mag).max()
    assert err < 2e-6, err


def test_linear_mistral_mlp_full_shape(ex):
    """The 7B decode shape 14336 x 4096, batch 1, against the oracle."""
    rng = oracle.RNG(2024)
    dense = rng.fill_normal(14336 * 4096, 0.02).reshape(14336, 4096)
    x = rng.fill_normal(4096, 1.0).reshape(1, 4096)
    w, ow = _weights(ex, dense, srq.Q8)
    got = srq.linear(ex, w, x)
    near(got, oracle.linear(ow, x, workers=8))


def test_linear_rejects_bad_arguments(ex):
    w = srq.Weight.create(ex, np.ones((4, 8), np.float32), srq.Q8)
    with pytest.raises(srq.SrqError):
        srq.linear(ex, w, np.zeros((0, 8), np.float32))
    b = ex.empty(64 * 1100)
    import ctypes as C
    assert srq.lib().srq_linear(ex.h, b.ptr, b.ptr, w.h, 1) == srq.EINVAL
    assert srq.lib().srq_linear(ex.h, b.ptr, C.c_void_p(b.value + 64), w.h, 1025) == srq.EINVAL


def _device_argmax(ex, logits):
    import ctypes as C
    rows, vocab = logits.shape
    buf = srq.DeviceBuffer.from_numpy(ex, np.ascontiguousarray(logits, np.float32))
    ids = np.zeros(rows, np.int32)
    srq.check(srq.lib().srq_argmax(ex.h, buf.ptr, rows, vocab, ids.ctypes.data_as(C.c_void_p)))
    return ids


@pytest.mark.parametrize("vocab", [1, 3, 4, 5, 1000, 4097, 32768, 50257, 128256])
def test_argmax_lowest_id_wins_ties(ex, vocab):
    """sampleWithBlocked at T=0 (M:7331-7358): strict '>' scan, so the first
    (lowest) id of the maximum wins; np.argmax has the same rule."""
    rng = np.random.default_rng(vocab)
    rows = 3
    logits = rng.integers(-50, 50, size=(rows, vocab)).astype(np.float32)  # many exact ties
    logits[1, :] = 7.0  # all equal: id 0
    if vocab > 10:
        logits[2, vocab - 1] = 1000.0
        logits[2, vocab // 2] = 1000.0  # tie between two far-apart ids
    assert np.array_equal(_device_argmax(ex, logits), np.argmax(logits, axis=1))


def test_argmax_rejects_nonfinite(ex):
    logits = np.zeros((2, 777), np.float32)
    for bad in (np.inf, -np.inf, np.nan):
        logits[1, 500] = bad
        with pytest.raises(srq.SrqError) as e:
            _device_argmax(ex, logits)
        assert e.value.code == srq.ENONFINITE
        logits[1, 500] = 0.0
    assert list(_device_argmax(ex, logits)) == [0, 0]
