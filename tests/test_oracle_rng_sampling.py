"""Pin the oracle's SplitMix64 RNG and sampler (M:1411-1439, M:7320-7426)."""
import math

import numpy as np
import pytest

import oracle

MASK = (1 << 64) - 1


def splitmix_py(state):
    """Independent Python-integer model of SplitMix64."""
    state = (state + 0x9E3779B97F4A7C15) & MASK
    z = state
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK
    return state, z ^ (z >> 31)


def test_splitmix64_published_vector_and_python_model():
    r = oracle.RNG(0)
    # Published first outputs of SplitMix64 from state 0.
    assert r.uint64() == 0xE220A8397B1DCDAF
    assert r.uint64() == 0x6E789E6AA1B965F4
    for seed in (1, 51, 2 ** 63 + 5, MASK):
        r = oracle.RNG(seed)
        s = seed
        for _ in range(50):
            s, want = splitmix_py(s)
            assert r.uint64() == want


def test_float64_and_normal_closed_form():
    seed = 12345
    r = oracle.RNG(seed)
    s = seed
    for _ in range(20):
        s, a = splitmix_py(s)
        s, b = splitmix_py(s)
        u1, u2 = (a >> 11) * 2.0 ** -53, (b >> 11) * 2.0 ** -53
        want = math.sqrt(-2 * math.log(1 - u1)) * math.cos(2 * math.pi * u2)
        assert abs(r.normal() - want) <= 1e-15 * max(1, abs(want))
    r = oracle.RNG(9)
    xs = r.fill_normal(200000, 1.0).astype(np.float64)
    assert abs(xs.mean()) < 0.01 and abs(xs.std() - 1) < 0.01


def test_intn_rejection_threshold():
    for bound in (1, 3, 7, 49152, 2 ** 40 + 3):
        r = oracle.RNG(77)
        s = 77
        threshold = ((1 << 64) - bound) % bound
        for _ in range(30):
            while True:
                s, x = splitmix_py(s)
                if x >= threshold:
                    want = x % bound
                    break
            assert r.intn(bound) == want


def test_greedy_with_penalty_and_block():
    logits = np.array([1.0, 3.0, 3.0, -2.0, 2.5], np.float32)
    rng = oracle.RNG(1)
    assert oracle.sample(logits, [], 0.0, 0, 1.0, 1.0, rng) == 1
    assert oracle.sample(logits, [], 0.0, 0, 1.0, 1.0, rng, blocked=1) == 2
    # penalty 2 halves positive seen logits: 3 -> 1.5 for id 1 and 2
    assert oracle.sample(logits, [1, 2], 0.0, 0, 1.0, 2.0, rng) == 4
    # greedy never consumes RNG state
    before = rng.state.value
    oracle.sample(logits, [], 0.0, 0, 1.0, 1.0, rng)
    assert rng.state.value == before
    assert oracle.sample(np.array([1.0, np.inf], np.float32), [], 0.0, 0, 1.0, 1.0, rng) < 0


def test_sampling_distribution_topk_topp():
    logits = np.array([2.0, 1.0, 0.5, 0.0, -1.0], np.float32)
    T = 0.8
    p = np.exp((logits.astype(np.float64) - 2.0) / T)
    rng = oracle.RNG(5)
    counts = np.zeros(5)
    n = 20000
    for _ in range(n):
        counts[oracle.sample(logits, [], T, 0, 1.0, 1.0, rng)] += 1
    want = p / p.sum()
    assert np.all(np.abs(counts / n - want) < 0.015)
    # top_k = 2 keeps ids 0, 1 only
    counts = np.zeros(5)
    for _ in range(4000):
        counts[oracle.sample(logits, [], T, 2, 1.0, 1.0, rng)] += 1
    assert counts[2:].sum() == 0 and abs(counts[0] / 4000 - p[0] / p[:2].sum()) < 0.03
    # top_p: cumulative mass reaching top_p*total cuts the tail
    cum = np.cumsum(p)
    keep = int(np.argmax(cum >= 0.9 * p.sum())) + 1
    counts = np.zeros(5)
    for _ in range(4000):
        counts[oracle.sample(logits, [], T, 0, 0.9, 1.0, rng)] += 1
    assert counts[keep:].sum() == 0


def test_sampling_draw_closed_form():
    """The draw walks candidates in candidateBefore order (logit desc, id
    asc) subtracting probabilities until negative (M:7416-7425)."""
    logits = np.array([0.0, 1.0, 1.0, 0.5], np.float32)
    T = 1.0
    seed = 99
    r = oracle.RNG(seed)
    got = oracle.sample(logits, [], T, 0, 1.0, 1.0, r)
    s, x = splitmix_py(seed)
    u = (x >> 11) * 2.0 ** -53
    order = [1, 2, 3, 0]
    probs = [math.exp((float(logits[i]) - 1.0) / T) for i in order]
    draw = u * sum(probs)
    want = order[-1]
    for i, pr in zip(order, probs):
        draw -= pr
        if draw < 0:
            want = i
            break
    assert got == want
