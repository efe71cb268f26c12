"""Pin the oracle's packer (srq_oracle.c) before trusting it.

Checks: the independent numpy float64 restatement (oracle/pack_np.py) agrees
bit-for-bit; hand-computed known answers that a round-half-even, a missing
nextafter or a swapped nibble would fail; the reference's own property tests
(q8_test.go:39-53, q4_test.go:95-143, q4_test.go:17-67)."""
import struct

import numpy as np
import pytest

import oracle
from oracle import pack_np

TINY = np.float32(np.finfo(np.float32).smallest_subnormal)
FMAX = np.float32(np.finfo(np.float32).max)


def f32(x):
    return np.float32(x)


def edge_matrix(rows, cols, seed):
    rng = np.random.default_rng(seed)
    m = rng.normal(0, 0.02, size=(rows, cols)).astype(np.float32)
    specials = np.array([0.0, -0.0, TINY, -TINY, 1e-43, 1e-38, 1e-37, FMAX, -FMAX, 0.5, 1.5, -2.5, 127.0,
                         -127.0, 63.5, 3.5, -3.5, 0.03], np.float32)
    mask = rng.random((rows, cols)) < 0.15
    m[mask] = rng.choice(specials, size=mask.sum())
    # an all-zero block, a block of one tie-heavy grid, an all-subnormal block
    if cols >= 64 and rows >= 3:
        m[0, :64] = 0
        m[1, :64] = (np.arange(64) - 32).astype(np.float32) * f32(0.5)
        m[2, :64] = TINY * (np.arange(64) % 5)
    return m


@pytest.mark.parametrize("cols", list(range(1, 194, 7)) + [64, 65, 127, 128, 129, 193, 513])
def test_c_packer_matches_numpy_restatement(cols):
    m = edge_matrix(5, cols, cols)
    v8, s8 = oracle.pack(m, oracle.Q8)
    n8, ns8 = pack_np.pack_q8(m)
    assert np.array_equal(s8.view(np.uint32), ns8.view(np.uint32))
    assert np.array_equal(v8, n8)
    v4, s4 = oracle.pack(m, oracle.Q4)
    n4, ns4 = pack_np.pack_q4(m)
    assert np.array_equal(s4.view(np.uint32), ns4.view(np.uint32))
    assert np.array_equal(v4, n4)


def test_random_normal_weights_match_numpy():
    r = oracle.RNG(7)
    m = r.fill_normal(300 * 577, 0.02).reshape(300, 577)
    for fmt, fn in ((oracle.Q8, pack_np.pack_q8), (oracle.Q4, pack_np.pack_q4)):
        v, s = oracle.pack(m, fmt)
        nv, ns = fn(m)
        assert np.array_equal(v, nv) and np.array_equal(s.view(np.uint32), ns.view(np.uint32))


def test_known_answers_round_half_away_and_scale():
    # amax 127 -> scale exactly 1; codes round half AWAY from zero.
    src = np.array([[127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 0.49999997, -126.5]], np.float32)
    v, s = oracle.pack(src, oracle.Q8)
    assert s[0, 0] == 1.0
    assert v[0].tolist() == [127, 1, 2, 3, -1, -2, -3, 0, -127]
    # Q4: amax 7 -> scale 1, clamp to +-7, two's-complement nibbles, low first.
    src = np.array([[7.0, -7.0, 0.5, -0.5, 3.0]], np.float32)
    v, s = oracle.pack(src, oracle.Q4)
    assert s[0, 0] == 1.0
    # codes 7,-7,1,-1,3 -> nibbles 7,9,1,15,3 -> bytes (9<<4|7),(15<<4|1),(0<<4|3)
    assert v[0].tolist() == [0x97, 0xF1, 0x03]


def test_scale_nextafter_branch():
    """lowBitScale rounds the scale down when f64(s)*L > amax (M:3887-3889).
    Find amax values hitting both branches and check the invariant exactly."""
    rng = np.random.default_rng(3)
    hits = 0
    for amax in np.concatenate([rng.random(20000).astype(np.float32) * 10, np.array([FMAX, 1e-30], np.float32)]):
        for levels in (127.0, 7.0):
            s = oracle.low_bit_scale(float(amax), levels)
            naive = np.float32(np.float64(amax) / levels)
            if float(naive) * levels > float(amax):
                hits += 1
                assert s == np.nextafter(naive, np.float32(0))
            else:
                assert s == naive
            assert float(np.float32(s)) * levels <= float(amax) * (1 + 1e-15) or s == TINY
    assert hits > 100  # both branches exercised
    assert oracle.low_bit_scale(0.0, 127) == 0.0
    assert oracle.low_bit_scale(float(TINY), 127) == TINY  # f32(tiny/127) == 0 -> tiny
    assert np.isfinite(oracle.low_bit_scale(float(FMAX), 127))


@pytest.mark.parametrize("levels,fmt", [(127, oracle.Q8), (7, oracle.Q4)])
def test_reference_scale_extremes_property(levels, fmt):
    """q8_test.go:39-53 and q4_test.go:128-142: finite scales and <= 0.501
    step reconstruction error at the extremes."""
    for maximum in [0.0, float(TINY), 1e-43, 1e-37, 0.03, 1.0, float(FMAX)]:
        m = np.float32(maximum)
        src = np.array([[-m, -m / np.float32(3), 0, m / np.float32(3), m]], np.float32)
        w = oracle.Weight.from_dense(src, fmt)
        scale = w.scales[0, 0]
        assert np.isfinite(scale) and scale >= 0 and not (maximum > 0 and scale == 0)
        got = w.copy_row(0)
        for j in range(5):
            assert np.isfinite(got[j])
            err = abs(float(got[j]) - float(src[0, j]))
            assert err <= float(scale) * 0.501 + float(m) * 2e-7


def test_q4_pairs_all_256_codes():
    """q4_test.go:95-126: every byte decodes low nibble first, sign-extended."""
    t = oracle.q4_pairs()
    for b in range(256):
        lo, hi = b & 15, b >> 4
        assert t[b, 0] == (lo - 16 if lo >= 8 else lo)
        assert t[b, 1] == (hi - 16 if hi >= 8 else hi)
    assert np.array_equal(t, pack_np.q4_pairs())


def test_q4_every_byte_roundtrip_odd_width():
    """Each byte code written into a 2x3 matrix reads back through copyRow;
    the odd width leaves a zero padding nibble and rows never overlap."""
    for b in range(256):
        codes = []
        for j in range(3):
            v = (b >> (4 * (j % 2))) & 15
            codes.append(v - 16 if v >= 8 else v)
        # amax 7 gives scale 1 when a 7 is present; build src = codes with a
        # guaranteed 7 in a 4th... keep width 3 by using scale from amax.
        src = np.array([codes, codes], np.float32)
        w = oracle.Weight.from_dense(src, oracle.Q4)
        for r in range(2):
            got = w.copy_row(r)
            amax = max(abs(c) for c in codes)
            if amax == 0:
                assert np.all(got == 0)
                continue
            scale = w.scales[r, 0]
            # Packed codes come from round(x/scale); decode must reproduce them.
            dec = oracle.q4_pairs()[w.values[r]].reshape(-1)[:3]
            assert np.all(np.abs(dec * scale - src[r]) <= scale * 0.501)
            assert w.values[r, 1] >> 4 == 0
            assert np.array_equal(got, (dec * scale).astype(np.float32))


def test_streamed_65_col_rows_equal_block_packer():
    """q4_test.go:17-67: 65-column rows cross block boundaries; streamed
    packing equals the per-block test packer (pack_np packs per block)."""
    x, w = oracle.linear_fixture(1, 65, 3)
    v, s = oracle.pack(w, oracle.Q4)
    nv, ns = pack_np.pack_q4(w)
    assert np.array_equal(v, nv) and np.array_equal(s, ns)
    assert v.shape == (3, 33) and s.shape == (3, 2)


def test_layout_byte_accounting_known_answers():
    """hfWeightLayoutFor (M:591-619) against the resident sizes the
    reference's receipts publish (Mistral-7B, Llama-3.2-3B)."""
    def layout(vocab, dim, layers, heads, kv, hidden, tied, fmt):
        kd = dim // heads * kv
        mats = [("embed", vocab, dim)]
        norms = 0
        for _ in range(layers):
            mats += [("q", dim, dim), ("k", kd, dim), ("v", kd, dim), ("o", dim, dim), ("gate", hidden, dim),
                     ("up", hidden, dim), ("down", dim, hidden)]
            norms += 2 * dim
        norms += dim
        if not tied:
            mats.append(("head", vocab, dim))
        total = norms * 4
        for name, r, c in mats:
            f = fmt if fmt != "q4-mixed" else ("q8" if name in ("embed", "head") else "q4")
            total += r * ((c + 63) // 64) * 4
            total += r * c if f == "q8" else r * ((c + 1) // 2)
        return total
    assert layout(32768, 4096, 32, 32, 8, 14336, False, "q8") == 7701807104
    assert layout(32768, 4096, 32, 32, 8, 14336, False, "q4-mixed") == 4212146176
    assert layout(128256, 3072, 28, 24, 8, 8192, True, "q8") == 3414061056
    assert layout(128256, 3072, 28, 24, 8, 8192, True, "q4") == 1807773696
    assert layout(128256, 3072, 28, 24, 8, 8192, True, "q4-mixed") == 2004774912
