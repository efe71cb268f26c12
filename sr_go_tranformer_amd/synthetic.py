"""Seeded synthetic models and prompts for benchmarks and tests.

Weights are drawn on the device with the reference's RNG semantics
(RNG{seed}.Normal()*0.02 per element, M:1411-1439, as NewModel initialises
matrices, M:5218): tensor t of the HF spec order (hfTensorSpecs,
M:406-421: embedding, then per layer input norm, q, k, v, o, post-attention
norm, gate, up, down, then the final norm and an untied head) uses
RNG{seed*1000003 + t}.  Norm weights are 1.  Matrices are packed on the
device by the model's format policy.
"""
import numpy as np

from . import (SRC_F32, T_ATTN_NORM, T_DOWN, T_EMBED, T_FFN_NORM, T_FINAL_NORM, T_GATE, T_K, T_O, T_OUTPUT, T_Q,
               T_UP, T_V, Model, fill_normal, make_config)

MASK = (1 << 64) - 1


class SplitMix64:
    """The reference's RNG (M:1411-1434) for host-side draws (prompts)."""

    def __init__(self, seed):
        self.state = seed & MASK

    def uint64(self):
        self.state = (self.state + 0x9E3779B97F4A7C15) & MASK
        z = self.state
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK
        return z ^ (z >> 31)

    def intn(self, n):
        bound = n
        threshold = ((1 << 64) - bound) % bound
        while True:
            x = self.uint64()
            if x >= threshold:
                return x % bound


def random_prompt(n, vocab, seed):
    r = SplitMix64(seed)
    return [r.intn(vocab) for _ in range(n)]


# Shapes of the benchmark configurations (HF Llama/Mistral profile).
SHAPES = {
    "smollm2-135m": dict(vocab=49152, dim=576, layers=30, heads=9, kv_heads=3, hidden=1536, tied=True,
                         rope_theta=10000.0),
    "llama3.2-1b": dict(vocab=128256, dim=2048, layers=16, heads=32, kv_heads=8, hidden=8192, tied=True,
                        rope_theta=500000.0),
    "mistral-7b": dict(vocab=32768, dim=4096, layers=32, heads=32, kv_heads=8, hidden=14336, tied=False,
                       rope_theta=10000.0),
    "llama3.2-3b": dict(vocab=128256, dim=3072, layers=28, heads=24, kv_heads=8, hidden=8192, tied=True,
                        rope_theta=500000.0),
}


def shape_config(name, context):
    s = SHAPES[name]
    return make_config(s["vocab"], s["dim"], s["layers"], s["heads"], s["kv_heads"], s["hidden"], context,
                       s["rope_theta"], 1e-5, s["tied"])


def build(ex, cfg, fmt, seed):
    """A device Model with seeded N(0, 0.02) matrices and unit norms."""
    d, kd, H, V = cfg.dim, cfg.dim // cfg.heads * cfg.kv_heads, cfg.hidden, cfg.vocab
    m = Model(ex, cfg, fmt)
    buf = ex.empty(max(V * d, H * d, d * d) * 4)
    t = 0

    def gen(kind, layer, rows, cols):
        nonlocal t
        fill_normal(ex, buf, rows * cols, seed * 1000003 + t, 0.02)
        m.load_device(kind, layer, buf.value, SRC_F32)
        t += 1

    ones = np.ones(d, np.float32)
    gen(T_EMBED, 0, V, d)
    for layer in range(cfg.layers):
        m.load(T_ATTN_NORM, layer, ones)
        t += 1
        for kind, rows, cols in ((T_Q, d, d), (T_K, kd, d), (T_V, kd, d), (T_O, d, d)):
            gen(kind, layer, rows, cols)
        m.load(T_FFN_NORM, layer, ones)
        t += 1
        for kind, rows, cols in ((T_GATE, H, d), (T_UP, H, d), (T_DOWN, d, H)):
            gen(kind, layer, rows, cols)
    m.load(T_FINAL_NORM, 0, ones)
    t += 1
    if not cfg.tied:
        gen(T_OUTPUT, 0, V, d)
    buf.close()
    return m


def decode_weight_bytes(cfg, fmt):
    """Weight bytes one decode token streams: every layer matrix, the final
    norm and the head (embedding lookups read one row: counted as one row)."""
    from . import packed_bytes, FORMATS
    d, kd, H, V = cfg.dim, cfg.dim // cfg.heads * cfg.kv_heads, cfg.hidden, cfg.vocab

    def mat(rows, cols, f):
        vb, sb = packed_bytes(FORMATS[f], rows, cols)
        return vb + sb

    layer_fmt = fmt if fmt != "q4-mixed" else "q4"
    head_fmt = fmt if fmt != "q4-mixed" else "q8"
    per_layer = (mat(d + 2 * kd, d, layer_fmt) + mat(d, d, layer_fmt) + mat(2 * H, d, layer_fmt) +
                 mat(d, H, layer_fmt) + 2 * d * 4)
    return per_layer * cfg.layers + mat(V, d, head_fmt) + d * 4 + mat(1, d, head_fmt)
