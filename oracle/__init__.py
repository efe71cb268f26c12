"""CPU oracle for sr_go_tranformer's quantized-weight inference path.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py may import this package, and only as the
checker (or the timed CPU baseline) -- never as the thing measured or
shipped.  The product (sr_go_tranformer_amd) never imports it.

The arithmetic lives in srq_oracle.c (a C restatement of
cmd/monolith/monolith.go, built by oracle/build.py); this module is a thin
ctypes/numpy wrapper around it.  pack_np.py holds an independent numpy
float64 restatement of the packer used to cross-check the C one.
"""
import ctypes as C
import os

import numpy as np

from . import build as _build

F32, Q8, Q4 = 0, 1, 2
N1, Q, K, V, O, N2, GATE, UP, DOWN, QB, KB, VB = range(12)

_lib = None


def lib():
    global _lib
    if _lib is None:
        path = _build.LIB
        if not os.path.exists(path) or os.path.getmtime(path) < os.path.getmtime(_build.SRC):
            _build.build(force=True)
        _lib = C.CDLL(path)
        _declare(_lib)
    return _lib


class Param(C.Structure):
    _fields_ = [("fmt", C.c_int), ("rows", C.c_int64), ("cols", C.c_int64),
                ("values", C.c_void_p), ("scales", C.c_void_p)]


class Config(C.Structure):
    _fields_ = [("vocab", C.c_int), ("dim", C.c_int), ("layers", C.c_int), ("heads", C.c_int),
                ("kv_heads", C.c_int), ("hidden", C.c_int), ("context", C.c_int),
                ("rope_theta", C.c_double), ("norm_eps", C.c_double), ("tied", C.c_int),
                ("rope_llama3", C.c_int), ("rope_factor", C.c_double), ("rope_low", C.c_double),
                ("rope_high", C.c_double), ("rope_original", C.c_int)]


def _declare(L):
    P = C.c_void_p
    L.or_rng_uint64.restype = C.c_uint64
    L.or_rng_uint64.argtypes = [C.POINTER(C.c_uint64)]
    L.or_rng_float64.restype = C.c_double
    L.or_rng_float64.argtypes = [C.POINTER(C.c_uint64)]
    L.or_rng_normal.restype = C.c_double
    L.or_rng_normal.argtypes = [C.POINTER(C.c_uint64)]
    L.or_rng_intn.restype = C.c_int64
    L.or_rng_intn.argtypes = [C.POINTER(C.c_uint64), C.c_int64]
    L.or_fill_normal.argtypes = [C.POINTER(C.c_uint64), C.c_double, P, C.c_int64]
    L.or_fill_uniform.argtypes = [C.POINTER(C.c_uint64), P, C.c_int64]
    L.or_low_bit_scale.restype = C.c_float
    L.or_low_bit_scale.argtypes = [C.c_float, C.c_double]
    L.or_q8_value.restype = C.c_int8
    L.or_q8_value.argtypes = [C.c_float, C.c_float]
    L.or_q4_value.restype = C.c_int8
    L.or_q4_value.argtypes = [C.c_float, C.c_float]
    L.or_pack_q8.argtypes = [P, C.c_int64, C.c_int64, P, P]
    L.or_pack_q4.argtypes = [P, C.c_int64, C.c_int64, P, P]
    L.or_q4_pairs.argtypes = [P]
    L.or_copy_row.argtypes = [C.c_int, C.c_int64, C.c_int64, P, P, C.c_int64, P]
    L.or_linear.argtypes = [C.POINTER(Param), P, P, C.c_int, C.c_int]
    L.or_linear_closed_f64.argtypes = [C.POINTER(Param), P, P, C.c_int]
    L.or_model_create.restype = P
    L.or_model_create.argtypes = [C.POINTER(Config)]
    L.or_model_destroy.argtypes = [P]
    L.or_model_set.restype = C.c_int
    L.or_model_set.argtypes = [P, C.c_int, C.c_int, C.POINTER(Param)]
    L.or_inverse_frequency.restype = C.c_float
    L.or_inverse_frequency.argtypes = [C.c_double, C.c_int, C.c_int, C.POINTER(Config)]
    L.or_model_cos.restype = P
    L.or_model_cos.argtypes = [P]
    L.or_model_sin.restype = P
    L.or_model_sin.argtypes = [P]
    L.or_cache_create.restype = P
    L.or_cache_create.argtypes = [P]
    L.or_cache_destroy.argtypes = [P]
    L.or_cache_pos.restype = C.c_int
    L.or_cache_pos.argtypes = [P]
    L.or_cache_row.restype = P
    L.or_cache_row.argtypes = [P, C.c_int, C.c_int, C.c_int]
    L.or_cache_set_rows.restype = C.c_int
    L.or_cache_set_rows.argtypes = [P, C.c_int, C.c_int, C.c_int, P, P]
    L.or_cache_set_pos.restype = C.c_int
    L.or_cache_set_pos.argtypes = [P, C.c_int]
    L.or_step.restype = C.c_int
    L.or_step.argtypes = [P, C.c_int, P, P, P, P, P, C.c_int]
    L.or_argmax.restype = C.c_int
    L.or_argmax.argtypes = [P, C.c_int]
    L.or_sample.restype = C.c_int
    L.or_sample.argtypes = [P, C.c_int, P, C.c_int, C.c_double, C.c_int, C.c_double, C.c_double,
                            C.POINTER(C.c_uint64), C.c_int]
    L.or_rms.argtypes = [P, P, P, C.c_int, C.c_int, C.c_double]
    L.or_rope.argtypes = [P, P, C.c_int, C.c_int]


def _ptr(a):
    return a.ctypes.data_as(C.c_void_p) if a is not None else None


# ---------------------------------------------------------------- RNG
class RNG:
    """SplitMix64 with the reference's Float64/Normal/Intn (M:1411-1439)."""

    def __init__(self, seed):
        self.state = C.c_uint64(seed)

    def uint64(self):
        return lib().or_rng_uint64(C.byref(self.state))

    def float64(self):
        return lib().or_rng_float64(C.byref(self.state))

    def normal(self):
        return lib().or_rng_normal(C.byref(self.state))

    def intn(self, n):
        return lib().or_rng_intn(C.byref(self.state), n)

    def fill_normal(self, count, scale):
        out = np.empty(count, np.float32)
        lib().or_fill_normal(C.byref(self.state), scale, _ptr(out), count)
        return out

    def fill_uniform(self, count):
        out = np.empty(count, np.float32)
        lib().or_fill_uniform(C.byref(self.state), _ptr(out), count)
        return out


def linear_fixture(n, cols, rows):
    """linearFixture (linear_backward_test.go:35-45): x[n*cols], W[rows*cols]."""
    r = RNG(51)
    x = r.fill_uniform(n * cols).reshape(n, cols)
    w = r.fill_uniform(cols * rows).reshape(rows, cols)
    return x, w


# ------------------------------------------------------------ packing
def low_bit_scale(amax, levels):
    return lib().or_low_bit_scale(amax, levels)


def pack(src, fmt):
    """Pack an f32 [rows, cols] matrix; returns (values, scales)."""
    src = np.ascontiguousarray(src, np.float32)
    rows, cols = src.shape
    groups = (cols + 63) // 64
    scales = np.zeros((rows, groups), np.float32)
    if fmt == Q8:
        values = np.zeros((rows, cols), np.int8)
        lib().or_pack_q8(_ptr(src), rows, cols, _ptr(values), _ptr(scales))
    elif fmt == Q4:
        values = np.zeros((rows, (cols + 1) // 2), np.uint8)
        lib().or_pack_q4(_ptr(src), rows, cols, _ptr(values), _ptr(scales))
    else:
        raise ValueError("pack format must be Q8 or Q4")
    return values, scales


def q4_pairs():
    t = np.zeros((256, 2), np.float32)
    lib().or_q4_pairs(_ptr(t))
    return t


class Weight:
    """An oracle-side weight (keeps its numpy storage alive)."""

    def __init__(self, fmt, rows, cols, values, scales=None):
        self.fmt, self.rows, self.cols = fmt, rows, cols
        self.values = np.ascontiguousarray(values)
        self.scales = None if scales is None else np.ascontiguousarray(scales, np.float32)
        self.param = Param(fmt, rows, cols, _ptr(self.values), _ptr(self.scales))

    @classmethod
    def from_dense(cls, dense, fmt):
        dense = np.ascontiguousarray(dense, np.float32)
        if fmt == F32:
            return cls(F32, dense.shape[0], dense.shape[1], dense)
        v, s = pack(dense, fmt)
        return cls(fmt, dense.shape[0], dense.shape[1], v, s)

    def copy_row(self, row):
        out = np.empty(self.cols, np.float32)
        lib().or_copy_row(self.fmt, self.rows, self.cols, _ptr(self.values), _ptr(self.scales), row, _ptr(out))
        return out

    def dequant(self):
        return np.stack([self.copy_row(r) for r in range(self.rows)]) if self.rows else \
            np.zeros((0, self.cols), np.float32)


def linear(w, x, workers=1):
    x = np.ascontiguousarray(x, np.float32).reshape(-1, w.cols)
    y = np.empty((x.shape[0], w.rows), np.float32)
    lib().or_linear(C.byref(w.param), _ptr(y), _ptr(x), x.shape[0], workers)
    return y


def linear_closed_f64(w, x):
    x = np.ascontiguousarray(x, np.float32).reshape(-1, w.cols)
    y = np.empty((x.shape[0], w.rows), np.float64)
    lib().or_linear_closed_f64(C.byref(w.param), _ptr(y), _ptr(x), x.shape[0])
    return y


# -------------------------------------------------------------- model
def make_config(vocab, dim, layers, heads, kv_heads, hidden, context, rope_theta=10000.0, norm_eps=1e-5,
                tied=True, llama3=None):
    c = Config(vocab, dim, layers, heads, kv_heads, hidden, context, rope_theta, norm_eps, int(tied), 0,
               0.0, 0.0, 0.0, 0)
    if llama3:
        c.rope_llama3 = 1
        c.rope_factor = llama3["factor"]
        c.rope_low = llama3["low_freq_factor"]
        c.rope_high = llama3["high_freq_factor"]
        c.rope_original = llama3["original_max_position_embeddings"]
    return c


def inverse_frequency(theta, head_dim, index, config=None):
    return lib().or_inverse_frequency(theta, head_dim, index, C.byref(config) if config is not None else None)


class Model:
    """Oracle model: weights is a dict {name: Weight} using the names of
    hfTensorSpecs (M:406-421) with 'model.' prefixes dropped."""

    def __init__(self, config, weights):
        self.config = config
        self.weights = weights
        self.h = lib().or_model_create(C.byref(config))
        if not self.h:
            raise ValueError("invalid oracle config")
        self._set(-1, 0, weights["embed_tokens"])
        self._set(-1, 1, weights["norm"])
        if "lm_head" in weights:
            self._set(-1, 2, weights["lm_head"])
        names = {N1: "input_layernorm", Q: "q_proj", K: "k_proj", V: "v_proj", O: "o_proj",
                 N2: "post_attention_layernorm", GATE: "gate_proj", UP: "up_proj", DOWN: "down_proj",
                 QB: "q_bias", KB: "k_bias", VB: "v_bias"}
        for layer in range(config.layers):
            for kind, nm in names.items():
                key = "layers.%d.%s" % (layer, nm)
                if key in weights:
                    self._set(layer, kind, weights[key])

    def _set(self, layer, kind, w):
        rc = lib().or_model_set(self.h, layer, kind, C.byref(w.param))
        if rc:
            raise ValueError("or_model_set failed %d" % rc)

    def close(self):
        if self.h:
            lib().or_model_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def rope_tables(self):
        hd = self.config.dim // self.config.heads
        n = self.config.context * (hd // 2)
        cos = np.ctypeslib.as_array(C.cast(lib().or_model_cos(self.h), C.POINTER(C.c_float)), (n,)).copy()
        sin = np.ctypeslib.as_array(C.cast(lib().or_model_sin(self.h), C.POINTER(C.c_float)), (n,)).copy()
        return cos.reshape(self.config.context, hd // 2), sin.reshape(self.config.context, hd // 2)

    def new_cache(self):
        return Cache(self)

    def step(self, caches, chunks, want=None, workers=1):
        sessions = len(caches)
        lens = np.array([len(c) for c in chunks], np.int32)
        tokens = np.concatenate([np.asarray(c, np.int32) for c in chunks]).astype(np.int32)
        handles = (C.c_void_p * sessions)(*[c.h for c in caches])
        w = None if want is None else np.array(want, np.uint8)
        logits = np.zeros((sessions, self.config.vocab), np.float32)
        rc = lib().or_step(self.h, sessions, C.cast(handles, C.c_void_p), _ptr(lens), _ptr(tokens), _ptr(w),
                           _ptr(logits), workers)
        if rc:
            raise RuntimeError("oracle step failed: %d" % rc)
        return logits


class Cache:
    def __init__(self, model):
        self.model = model
        self.h = lib().or_cache_create(model.h)

    @property
    def pos(self):
        return lib().or_cache_pos(self.h)

    def row(self, layer, pos, which):
        c = self.model.config
        kd = (c.dim // c.heads) * c.kv_heads
        p = lib().or_cache_row(self.h, layer, pos, which)
        if not p:
            raise IndexError("no such KV row")
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_float)), (kd,)).copy()

    def set_rows(self, layer, pos0, k, v):
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        rc = lib().or_cache_set_rows(self.h, layer, pos0, k.shape[0], _ptr(k), _ptr(v))
        if rc:
            raise ValueError("set_rows failed")

    def set_pos(self, pos):
        if lib().or_cache_set_pos(self.h, pos):
            raise ValueError("set_pos failed")

    def close(self):
        if self.h:
            lib().or_cache_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()


def argmax(logits):
    logits = np.ascontiguousarray(logits, np.float32)
    return lib().or_argmax(_ptr(logits), logits.shape[-1])


def sample(logits, history, temperature, top_k, top_p, repeat_penalty, rng, blocked=-1):
    logits = np.ascontiguousarray(logits, np.float32)
    hist = np.asarray(history, np.int32)
    return lib().or_sample(_ptr(logits), logits.shape[-1], _ptr(hist), len(hist), temperature, top_k, top_p,
                           repeat_penalty, C.byref(rng.state), blocked)


def rms(x, w, eps):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    y = np.empty_like(x)
    lib().or_rms(_ptr(y), _ptr(x), _ptr(w), x.shape[0], x.shape[1], eps)
    return y


def greedy(model, ids, count, chunk, workers=8):
    """inferHFIDs (M:1185-1240) without EOS stop: prefill in chunks, then
    count greedy tokens (fixed-step).  Returns (tokens, last-step logits list)."""
    cache = model.new_cache()
    nxt = None
    for lo in range(0, len(ids), chunk):
        nxt = model.step([cache], [ids[lo:lo + chunk]], workers=workers)[0]
    out, logits = [], []
    for i in range(count):
        best = argmax(nxt)
        if best < 0:
            raise RuntimeError("non-finite logits")
        logits.append(nxt)
        out.append(best)
        if i + 1 < count:
            nxt = model.step([cache], [[best]], workers=workers)[0]
    cache.close()
    return out, logits
