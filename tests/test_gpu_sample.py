"""GPU sampling (srq_sample) against the oracle's restatement of
sampleWithBlocked (M:7320-7426), through the C ABI.

Bar: identical token ids and identical SplitMix64 state after the draw.  The
oracle sums f64 probabilities in candidate order; the device sums exact
fixed-point masses, so the two could part only for a draw within ~1e-12 of
a candidate boundary, which none of these seeded cases hits."""
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


def run(ex, logits, params, seeds, histories=None, blocked=None):
    rows, vocab = logits.shape
    buf = srq.DeviceBuffer.from_numpy(ex, np.ascontiguousarray(logits, np.float32))
    states = np.asarray(seeds, np.uint64).copy()
    ids = srq.sample(ex, buf.ptr, rows, vocab, params, states, histories, blocked)
    return ids, states


def oracle_rows(logits, t, k, p, rp, seeds, histories=None, blocked=None):
    ids, states = [], []
    for r in range(logits.shape[0]):
        rng = oracle.RNG(int(seeds[r]))
        hist = histories[r] if histories is not None else []
        b = int(blocked[r]) if blocked is not None else -1
        ids.append(oracle.sample(logits[r], hist, t, k, p, rp, rng, blocked=b))
        states.append(rng.state.value)
    return np.array(ids), np.array(states, np.uint64)


CASES = [  # temperature, top_k, top_p, repeat_penalty
    (0.0, 0, 1.0, 1.0), (0.0, 0, 1.0, 1.3), (0.8, 0, 1.0, 1.0), (0.8, 0, 0.9, 1.0), (1.0, 40, 1.0, 1.1),
    (0.7, 40, 0.95, 1.1), (1.3, 5, 0.5, 1.0), (0.5, 1, 1.0, 1.0), (2.0, 0, 0.2, 1.5),
]


@pytest.mark.parametrize("vocab", [1, 2, 7, 300, 4099, 32768])
@pytest.mark.parametrize("case", CASES)
def test_sample_matches_oracle(ex, vocab, case):
    t, k, p, rp = case
    print("sample", vocab, case, flush=True)
    rng = np.random.default_rng(vocab * 131 + int(t * 10) + k)
    rows = 6
    logits = rng.normal(0, 2.0, size=(rows, vocab)).astype(np.float32)
    seeds = rng.integers(0, 2**63, size=rows, dtype=np.uint64)
    hist = [list(rng.integers(0, vocab, size=rng.integers(0, 12))) for _ in range(rows)]
    blocked = np.full(rows, -1, np.int32)
    if vocab > 1:
        blocked[::2] = rng.integers(0, vocab, size=(rows + 1) // 2)
    params = srq.Sampling(t, k, p, rp)
    got, gst = run(ex, logits, params, seeds, hist, blocked)
    want, wst = oracle_rows(logits, t, k, p, rp, seeds, hist, blocked)
    assert np.array_equal(got, want), (got, want)
    assert np.array_equal(gst, wst)


@pytest.mark.parametrize("levels", [3, 40])
def test_sample_ties_rank_by_id(ex, levels):
    """Logits on a few levels: long runs of equal values, ranked by id
    (candidateBefore), across histogram refinement and LDS sorting."""
    rng = np.random.default_rng(levels)
    vocab, rows = 5000, 8
    logits = (rng.integers(0, levels, size=(rows, vocab)) * 0.25).astype(np.float32)
    seeds = rng.integers(0, 2**63, size=rows, dtype=np.uint64)
    for t, k, p, rp in [(1.0, 0, 1.0, 1.0), (0.9, 100, 1.0, 1.0), (1.1, 0, 0.6, 1.0), (0.0, 0, 1.0, 1.0)]:
        got, gst = run(ex, logits, srq.Sampling(t, k, p, rp), seeds)
        want, wst = oracle_rows(logits, t, k, p, rp, seeds)
        assert np.array_equal(got, want), (t, k, p, got, want)
        assert np.array_equal(gst, wst)


def test_sample_continuous_batching_parameters(ex):
    """The continuous-batching configuration's sampler (T 0.8, top-p 0.9,
    top-k off, no penalty) at a 128256-id vocabulary: a nearly flat row
    (nucleus of ~10^5 ids) and a peaked one, 32 rows."""
    rng = np.random.default_rng(7)
    rows, vocab = 32, 128256
    logits = rng.normal(0, 0.05, size=(rows, vocab)).astype(np.float32)
    logits[1::2] = rng.normal(0, 4.0, size=(rows // 2, vocab)).astype(np.float32)
    seeds = rng.integers(0, 2**63, size=rows, dtype=np.uint64)
    got, gst = run(ex, logits, srq.Sampling(0.8, 0, 0.9, 1.0), seeds)
    want, wst = oracle_rows(logits, 0.8, 0, 0.9, 1.0, seeds)
    assert np.array_equal(got, want)
    assert np.array_equal(gst, wst)


def test_sample_many_rows_run_in_groups(ex):
    """A call with more rows than one launch group's scratch holds (64 rows
    at a 128256-id vocabulary) samples them in groups: every id and state
    equals the oracle's, with histories, blocked ids and row_ids, whose
    per-row pointers move with each group."""
    rng = np.random.default_rng(33)
    rows, vocab = 90, 128256
    logits = rng.normal(0, 1.0, size=(rows, vocab)).astype(np.float32)
    logits[::3] = rng.normal(0, 4.0, size=((rows + 2) // 3, vocab)).astype(np.float32)
    hist = [list(rng.integers(0, vocab, size=rng.integers(0, 20))) for _ in range(rows)]
    blocked = np.where(np.arange(rows) % 2 == 0, rng.integers(0, vocab, size=rows), -1).astype(np.int32)
    seeds = rng.integers(0, 2**63, size=rows, dtype=np.uint64)
    for t, k, p, rp in [(0.8, 0, 0.9, 1.0), (0.7, 40, 0.95, 1.2)]:
        got, gst = run(ex, logits, srq.Sampling(t, k, p, rp), seeds, hist, blocked)
        want, wst = oracle_rows(logits, t, k, p, rp, seeds, hist, blocked)
        assert np.array_equal(got, want), (t, k, p, rp)
        assert np.array_equal(gst, wst)
    buf = srq.DeviceBuffer.from_numpy(ex, logits)
    sel = list(range(rows - 1, -1, -1))[:77]
    st = seeds[:77].copy()
    got = srq.sample(ex, buf.ptr, len(sel), vocab, srq.Sampling(0.8, 0, 0.9, 1.0), st, row_ids=sel)
    want, wst = oracle_rows(logits[sel], 0.8, 0, 0.9, 1.0, seeds[:77])
    assert np.array_equal(got, want)
    assert np.array_equal(st, wst)


def test_sample_draws_follow_the_distribution(ex):
    """Frequencies over many draws follow softmax(logits / T)."""
    logits = np.array([[2.0, 1.0, 0.0, -1.0, 1.0]], np.float32)
    t = 0.9
    counts = np.zeros(5)
    state = np.array([12345], np.uint64)
    buf = srq.DeviceBuffer.from_numpy(ex, logits)
    for _ in range(3000):
        counts[srq.sample(ex, buf.ptr, 1, 5, srq.Sampling(t, 0, 1.0, 1.0), state)[0]] += 1
    p = np.exp(logits[0] / t - logits[0].max() / t)
    p /= p.sum()
    assert np.abs(counts / counts.sum() - p).max() < 0.03


def test_sample_row_ids_select_rows(ex):
    """row_ids: a subset of the logits rows, in any order, samples exactly as
    those rows would compacted (the sessions of a step that want a token)."""
    rng = np.random.default_rng(21)
    rows, vocab = 9, 4099
    logits = rng.normal(0, 2.0, size=(rows, vocab)).astype(np.float32)
    logits[3] = 0.0  # a zeroed row that is not sampled
    buf = srq.DeviceBuffer.from_numpy(ex, logits)
    sel = [7, 2, 5, 0]
    seeds = rng.integers(0, 2**63, size=len(sel), dtype=np.uint64)
    for t, k, p in [(0.9, 40, 0.95), (0.8, 0, 0.9), (0.0, 0, 1.0)]:
        st = seeds.copy()
        got = srq.sample(ex, buf.ptr, len(sel), vocab, srq.Sampling(t, k, p, 1.0), st, row_ids=sel)
        want, wst = oracle_rows(logits[sel], t, k, p, 1.0, seeds)
        assert np.array_equal(got, want), (t, got, want)
        assert np.array_equal(st, wst)
    with pytest.raises(srq.SrqError) as e:
        srq.sample(ex, buf.ptr, 2, vocab, srq.Sampling(0.8, 0, 1.0, 1.0), seeds[:2].copy(), row_ids=[1, -1])
    assert e.value.code == srq.EINVAL


def test_sample_errors(ex):
    logits = np.zeros((2, 33), np.float32)
    logits[1, 7] = np.nan
    with pytest.raises(srq.SrqError) as e:
        run(ex, logits, srq.Sampling(0.8, 0, 1.0, 1.0), [1, 2])
    assert e.value.code == srq.ENONFINITE
    one = np.zeros((1, 1), np.float32)
    with pytest.raises(srq.SrqError) as e:
        run(ex, one, srq.Sampling(0.8, 0, 1.0, 1.0), [1], blocked=[0])
    assert e.value.code == srq.EINVAL
    with pytest.raises(srq.SrqError) as e:
        run(ex, one, srq.Sampling(-1.0, 0, 1.0, 1.0), [1])
    assert e.value.code == srq.EINVAL
    # the executor stays usable: greedy over a clean row
    ids, _ = run(ex, np.array([[0.0, 3.0, 3.0]], np.float32), srq.Sampling(0.0, 0, 1.0, 1.0), [5])
    assert list(ids) == [1]


def test_sample_flat_rows_rank_by_id(ex):
    """Rows holding one value (e.g. the zeroed rows of unselected sessions)
    and a run of 10^4 equal values at the nucleus edge: the candidates past
    one bucket's sort are ranked by id."""
    rng = np.random.default_rng(11)
    vocab = 128256
    logits = np.zeros((4, vocab), np.float32)
    logits[2, :] = -3.0
    logits[3, :] = rng.normal(0, 1.0, size=vocab).astype(np.float32)
    logits[3, 1000:11000] = 0.5
    seeds = rng.integers(0, 2**63, size=4, dtype=np.uint64)
    for t, k, p in [(0.8, 0, 0.9), (0.8, 0, 1.0), (1.0, 50000, 1.0), (0.5, 3000, 0.7)]:
        got, gst = run(ex, logits, srq.Sampling(t, k, p, 1.0), seeds)
        want, wst = oracle_rows(logits, t, k, p, 1.0, seeds)
        assert np.array_equal(got, want), (t, k, p, got, want)
        assert np.array_equal(gst, wst)
