"""Independent numpy float64 restatement of the reference's packer.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  Written separately from
srq_oracle.c so the two restatements can be checked bit-for-bit against each
other: a slip in one (a dropped nextafter, round-half-even instead of
half-away, a swapped nibble) fails the comparison.

Follows cmd/monolith/monolith.go:
  lowBitScale   M:3877-3891    q8Value / putQuantized  M:3840-3850, M:3893-3898
  q4 put        M:3819-3822    readParam block walk     M:857-880
  q4Pairs       M:3811-3817    copyRow                  M:3900-3921
"""
import numpy as np

TINY = np.float32(np.finfo(np.float32).smallest_subnormal)


def low_bit_scale(amax, levels):
    amax = np.asarray(amax, np.float32)
    s = (amax.astype(np.float64) / levels).astype(np.float32)
    s = np.where(s == 0, TINY, s)
    down = (s > TINY) & (s.astype(np.float64) * levels > amax.astype(np.float64))
    s = np.where(down, np.nextafter(s, np.float32(0)), s)
    return np.where(amax == 0, np.float32(0), s).astype(np.float32)


def round_half_away(q):
    """Go's math.Round on float64, without the floor(x+0.5) pitfall."""
    t = np.trunc(q)
    frac = np.abs(q - t)
    return np.where(frac >= 0.5, t + np.sign(q), t)


def _codes(src, scales, levels):
    rows, cols = src.shape
    s_cols = np.repeat(scales, 64, axis=1)[:, :cols].astype(np.float64)
    with np.errstate(divide="ignore", invalid="ignore"):
        q = round_half_away(src.astype(np.float64) / s_cols)
    q = np.clip(q, -levels, levels)
    q = np.where(s_cols == 0, 0, q)
    return q.astype(np.int64)


def _scales(src, levels):
    rows, cols = src.shape
    groups = (cols + 63) // 64
    padded = np.zeros((rows, groups * 64), np.float32)
    padded[:, :cols] = np.abs(src)
    amax = padded.reshape(rows, groups, 64).max(axis=2)
    return low_bit_scale(amax, levels)


def pack_q8(src):
    src = np.asarray(src, np.float32)
    scales = _scales(src, 127)
    return _codes(src, scales, 127).astype(np.int8), scales


def pack_q4(src):
    src = np.asarray(src, np.float32)
    rows, cols = src.shape
    scales = _scales(src, 7)
    q = _codes(src, scales, 7) & 15
    if cols % 2:
        q = np.concatenate([q, np.zeros((rows, 1), np.int64)], axis=1)
    packed = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8)
    return packed, scales


def q4_pairs():
    b = np.arange(256)
    lo = b & 15
    hi = b >> 4
    lo = np.where(lo >= 8, lo - 16, lo)
    hi = np.where(hi >= 8, hi - 16, hi)
    return np.stack([lo, hi], axis=1).astype(np.float32)


def dequant_q8(values, scales):
    rows, cols = values.shape
    s = np.repeat(scales, 64, axis=1)[:, :cols]
    return (values.astype(np.float32) * s).astype(np.float32)


def dequant_q4(values, scales, cols):
    t = q4_pairs()
    codes = t[values]  # [rows, stride, 2]
    codes = codes.reshape(values.shape[0], -1)[:, :cols]
    s = np.repeat(scales, 64, axis=1)[:, :cols]
    return (codes * s).astype(np.float32)
