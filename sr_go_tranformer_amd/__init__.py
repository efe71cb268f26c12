"""sr_go_tranformer_amd -- MI355X (gfx950) quantized-weight inference path.

Python view of the C ABI in include/srq.h, implemented by the HIP library
libsrq.so built in place by sr_go_tranformer_amd/build.py.  Every call goes
to the native library; importing this package without the built library
raises immediately (there is no CPU fallback).

Names follow the reference's Go seam (cmd/monolith/monolith.go):
Executor ~ kernelExecutor, Weight ~ Param, Model/Pool/Cache ~ Model,
pagePool, KVCache, Model.step ~ prefillSelected, generate_greedy ~
inferHFIDs.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# SRQ_LIB names another build of the library (the host-sanitized one the CPU
# tests load under the sanitizer runtime).
LIB_PATH = os.environ.get("SRQ_LIB") or os.path.join(HERE, "libsrq.so")

F32, Q8, Q4 = 0, 1, 2
SRC_F32, SRC_BF16, SRC_F16 = 0, 1, 2
OK, EDEVICE, ENOMEM, EINVAL, ENOSPC, ENONFINITE, ERANGE, ECANCELED = 0, -5, -12, -22, -28, -33, -34, -125
EFILE, EFORMAT = -2, -74
T_EMBED, T_FINAL_NORM, T_OUTPUT = 0, 1, 2
T_ATTN_NORM, T_Q, T_K, T_V, T_O, T_FFN_NORM, T_GATE, T_UP, T_DOWN, T_Q_BIAS, T_K_BIAS, T_V_BIAS = range(10, 22)
T_QKV, T_GATE_UP = 22, 23  # fused storage views (srq_model_weight only)

FORMATS = {"f32": F32, "q8": Q8, "q4": Q4}


class SrqError(RuntimeError):
    def __init__(self, code, message):
        super().__init__("srq error %d: %s" % (code, message))
        self.code = code


class ModelConfig(C.Structure):
    _fields_ = [("vocab", C.c_int32), ("dim", C.c_int32), ("layers", C.c_int32), ("heads", C.c_int32),
                ("kv_heads", C.c_int32), ("hidden", C.c_int32), ("context", C.c_int32),
                ("rope_theta", C.c_double), ("norm_eps", C.c_double), ("tied", C.c_int32),
                ("qkv_bias", C.c_int32), ("rope_llama3", C.c_int32), ("rope_factor", C.c_double),
                ("rope_low", C.c_double), ("rope_high", C.c_double), ("rope_original", C.c_int32)]


_lib = None


def lib():
    """The loaded native library (raises if it was not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError("libsrq.so is not built: run sr_go_tranformer_amd/build.py (hipcc, gfx950)")
        _lib = C.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


EXPORTS = [
    "srq_abi_version", "srq_last_error", "srq_device_count", "srq_alloc", "srq_free", "srq_copy_h2d",
    "srq_copy_d2h", "srq_copy_d2d", "srq_exec_create", "srq_exec_destroy", "srq_exec_synchronize",
    "srq_exec_stream", "srq_fill_normal", "srq_packed_bytes", "srq_pack", "srq_pack_host", "srq_weight_create",
    "srq_weight_create_host", "srq_weight_wrap",
    "srq_weight_destroy", "srq_weight_info", "srq_dequant_rows", "srq_linear", "srq_linear_enqueue",
    "srq_linear_noalloc", "srq_model_create",
    "srq_model_load", "srq_model_load_host", "srq_model_destroy", "srq_model_resident_bytes", "srq_model_weight",
    "srq_model_rope_tables", "srq_model_load_safetensors", "srq_archive_check",
    "srq_pool_create", "srq_pool_destroy", "srq_cache_create", "srq_cache_destroy",
    "srq_cache_pos", "srq_cache_read", "srq_step", "srq_argmax", "srq_sample", "srq_decoder_create", "srq_decoder_run",
    "srq_decoder_tokens", "srq_decoder_destroy", "srq_generate_greedy",
]


def _declare(L):
    P, I32, I64 = C.c_void_p, C.c_int32, C.c_int64
    PP = C.POINTER(C.c_void_p)
    sig = {
        "srq_abi_version": (C.c_int, []),
        "srq_last_error": (C.c_char_p, []),
        "srq_device_count": (C.c_int, [C.POINTER(C.c_int)]),
        "srq_alloc": (C.c_int, [C.c_int, C.c_size_t, PP]),
        "srq_free": (C.c_int, [P]),
        "srq_copy_h2d": (C.c_int, [P, P, P, C.c_size_t]),
        "srq_copy_d2h": (C.c_int, [P, P, P, C.c_size_t]),
        "srq_copy_d2d": (C.c_int, [P, P, P, C.c_size_t]),
        "srq_exec_create": (C.c_int, [C.c_int, PP]),
        "srq_exec_destroy": (C.c_int, [P]),
        "srq_exec_synchronize": (C.c_int, [P]),
        "srq_exec_stream": (P, [P]),
        "srq_fill_normal": (C.c_int, [P, P, I64, C.c_uint64, C.c_double]),
        "srq_packed_bytes": (C.c_int, [C.c_int, I64, I64, C.POINTER(I64), C.POINTER(I64)]),
        "srq_pack": (C.c_int, [P, C.c_int, I64, I64, P, C.c_int, P, P]),
        "srq_pack_host": (C.c_int, [P, C.c_int, I64, I64, P, C.c_int, P, P, P]),
        "srq_weight_create": (C.c_int, [P, C.c_int, I64, I64, P, C.c_int, PP]),
        "srq_weight_create_host": (C.c_int, [P, C.c_int, I64, I64, P, C.c_int, P, PP]),
        "srq_weight_wrap": (C.c_int, [C.c_int, I64, I64, P, P, PP]),
        "srq_weight_destroy": (C.c_int, [P]),
        "srq_weight_info": (C.c_int, [P, C.POINTER(C.c_int), C.POINTER(I64), C.POINTER(I64), PP, PP]),
        "srq_dequant_rows": (C.c_int, [P, P, P, I32, P]),
        "srq_linear": (C.c_int, [P, P, P, P, I32]),
        "srq_linear_enqueue": (C.c_int, [P, P, P, P, I32]),
        "srq_linear_noalloc": (C.c_int, [P, P, P, P, I32]),
        "srq_model_create": (C.c_int, [P, C.POINTER(ModelConfig), C.c_char_p, PP]),
        "srq_model_load": (C.c_int, [P, C.c_int, C.c_int, P, C.c_int]),
        "srq_model_load_host": (C.c_int, [P, C.c_int, C.c_int, P, C.c_int, P]),
        "srq_model_destroy": (C.c_int, [P]),
        "srq_model_resident_bytes": (C.c_int, [P, C.POINTER(I64)]),
        "srq_model_weight": (C.c_int, [P, C.c_int, C.c_int, PP]),
        "srq_model_rope_tables": (C.c_int, [P, P, P]),
        "srq_model_load_safetensors": (C.c_int, [P, C.c_char_p, P, C.POINTER(I64)]),
        "srq_archive_check": (C.c_int, [C.POINTER(ModelConfig), C.c_char_p, C.POINTER(I64)]),
        "srq_pool_create": (C.c_int, [P, I32, PP]),
        "srq_pool_destroy": (C.c_int, [P]),
        "srq_cache_create": (C.c_int, [P, I32, PP]),
        "srq_cache_destroy": (C.c_int, [P]),
        "srq_cache_pos": (C.c_int, [P, C.POINTER(I32)]),
        "srq_cache_read": (C.c_int, [P, P, I32, I32, I32, P, P]),
        "srq_step": (C.c_int, [P, P, I32, P, P, P, P, PP, P, P]),
        "srq_argmax": (C.c_int, [P, P, I32, I32, P]),
        "srq_sample": (C.c_int, [P, P, I32, P, I32, P, P, P, I32, P, P, P]),
        "srq_decoder_create": (C.c_int, [P, P, P, I32, I32, I32, PP]),
        "srq_decoder_run": (C.c_int, [P, I32]),
        "srq_decoder_tokens": (C.c_int, [P, P, C.POINTER(I32)]),
        "srq_decoder_destroy": (C.c_int, [P]),
        "srq_generate_greedy": (C.c_int, [P, P, P, P, I32, I32, I32, I32, P, C.POINTER(I32)]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args


def check(rc):
    if rc != OK:
        msg = lib().srq_last_error()
        raise SrqError(rc, msg.decode() if msg else "")
    return rc


def _np_ptr(a):
    return a.ctypes.data_as(C.c_void_p)


class Executor:
    """kernelExecutor: one HIP stream plus scratch on one device."""

    def __init__(self, device=0):
        h = C.c_void_p()
        check(lib().srq_exec_create(device, C.byref(h)))
        self.h = h
        self.device = device

    @property
    def stream(self):
        return lib().srq_exec_stream(self.h)

    def synchronize(self):
        check(lib().srq_exec_synchronize(self.h))

    def close(self):
        if self.h:
            lib().srq_exec_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- device buffers
    def upload(self, array):
        return DeviceBuffer.from_numpy(self, array)

    def empty(self, nbytes):
        return DeviceBuffer(self, nbytes)


class DeviceBuffer:
    """Device memory from srq_alloc, freed on close/garbage collection."""

    def __init__(self, ex, nbytes):
        self.ex = ex
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        check(lib().srq_alloc(ex.device, max(self.nbytes, 1), C.byref(p)))
        self.ptr = p

    @classmethod
    def from_numpy(cls, ex, array):
        a = np.ascontiguousarray(array)
        b = cls(ex, a.nbytes)
        if a.nbytes:
            check(lib().srq_copy_h2d(ex.h, b.ptr, _np_ptr(a), a.nbytes))
        return b

    def to_numpy(self, dtype, shape):
        out = np.empty(shape, dtype)
        if out.nbytes > self.nbytes:
            raise ValueError("read past the buffer")
        if out.nbytes:
            check(lib().srq_copy_d2h(self.ex.h, _np_ptr(out), self.ptr, out.nbytes))
        return out

    def write(self, array):
        a = np.ascontiguousarray(array)
        if a.nbytes > self.nbytes:
            raise ValueError("write past the buffer")
        check(lib().srq_copy_h2d(self.ex.h, self.ptr, _np_ptr(a), a.nbytes))

    @property
    def value(self):
        return self.ptr.value

    def close(self):
        if self.ptr:
            lib().srq_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def fill_normal(ex, buf, count, seed, scale):
    """Device fill with f32(Normal()*scale) of RNG{seed} (see srq.h)."""
    check(lib().srq_fill_normal(ex.h, buf.ptr, count, seed, scale))


def packed_bytes(fmt, rows, cols):
    vb, sb = C.c_int64(), C.c_int64()
    check(lib().srq_packed_bytes(fmt, rows, cols, C.byref(vb), C.byref(sb)))
    return vb.value, sb.value


def pack(ex, src, fmt, dtype=SRC_F32, cols=None):
    """Pack a host [rows, cols] source (f32 array, or uint16 words with
    dtype SRC_BF16/SRC_F16) on the device; returns (values, scales) on host."""
    src = np.ascontiguousarray(src)
    rows, cols = src.shape[0], (cols if cols is not None else src.shape[1])
    vb, sb = packed_bytes(fmt, rows, cols)
    s = ex.upload(src)
    v, sc = ex.empty(vb), ex.empty(sb)
    check(lib().srq_pack(ex.h, fmt, rows, cols, s.ptr, dtype, v.ptr, sc.ptr))
    groups = (cols + 63) // 64
    if fmt == Q8:
        values = v.to_numpy(np.int8, (rows, cols))
    else:
        values = v.to_numpy(np.uint8, (rows, (cols + 1) // 2))
    return values, sc.to_numpy(np.float32, (rows, groups))


def pack_host(ex, src, fmt, dtype=SRC_F32, cols=None, cancel=None):
    """pack() through srq_pack_host: the host source is streamed by the
    library (pinned chunks), not uploaded first.  cancel: an optional
    ctypes.c_int32 polled between chunks."""
    src = np.ascontiguousarray(src)
    rows, cols = src.shape[0], (cols if cols is not None else src.shape[1])
    vb, sb = packed_bytes(fmt, rows, cols)
    v, sc = ex.empty(vb), ex.empty(sb)
    flag = C.byref(cancel) if cancel is not None else None
    check(lib().srq_pack_host(ex.h, fmt, rows, cols, _np_ptr(src), dtype, v.ptr, sc.ptr, flag))
    groups = (cols + 63) // 64
    if fmt == Q8:
        values = v.to_numpy(np.int8, (rows, cols))
    else:
        values = v.to_numpy(np.uint8, (rows, (cols + 1) // 2))
    return values, sc.to_numpy(np.float32, (rows, groups))


class Weight:
    """Param: a device-resident Q8/Q4/F32 matrix [rows, cols]."""

    def __init__(self, h, owner=None, keep=()):
        self.h = h
        self.owner = owner  # a Model whose storage this view borrows
        self.keep = keep
        fmt, rows, cols = C.c_int(), C.c_int64(), C.c_int64()
        vals, scl = C.c_void_p(), C.c_void_p()
        check(lib().srq_weight_info(h, C.byref(fmt), C.byref(rows), C.byref(cols), C.byref(vals), C.byref(scl)))
        self.fmt, self.rows, self.cols = fmt.value, rows.value, cols.value
        self.values_ptr, self.scales_ptr = vals.value, scl.value

    @classmethod
    def create(cls, ex, src, fmt, dtype=SRC_F32, cols=None):
        src = np.ascontiguousarray(src)
        rows, cols = src.shape[0], (cols if cols is not None else src.shape[1])
        s = ex.upload(src)
        h = C.c_void_p()
        check(lib().srq_weight_create(ex.h, fmt, rows, cols, s.ptr, dtype, C.byref(h)))
        return cls(h)

    @classmethod
    def create_host(cls, ex, src, fmt, dtype=SRC_F32, cols=None, cancel=None):
        """create() through srq_weight_create_host (host source streamed by
        the library)."""
        src = np.ascontiguousarray(src)
        rows, cols = src.shape[0], (cols if cols is not None else src.shape[1])
        h = C.c_void_p()
        flag = C.byref(cancel) if cancel is not None else None
        check(lib().srq_weight_create_host(ex.h, fmt, rows, cols, _np_ptr(src), dtype, flag, C.byref(h)))
        return cls(h)

    @classmethod
    def wrap(cls, ex, fmt, values, scales, cols):
        """Wrap host-packed storage (uploaded and kept alive by the weight)."""
        v = ex.upload(values)
        s = ex.upload(scales) if scales is not None else None
        h = C.c_void_p()
        check(lib().srq_weight_wrap(fmt, values.shape[0], cols, v.ptr, s.ptr if s else None, C.byref(h)))
        return cls(h, keep=(v, s))

    def packed(self, ex):
        vb, sb = packed_bytes(self.fmt, self.rows, self.cols)
        out_v = np.empty(vb, np.uint8)
        check(lib().srq_copy_d2h(ex.h, _np_ptr(out_v), C.c_void_p(self.values_ptr), vb))
        out_s = np.empty(sb // 4, np.float32)
        if sb:
            check(lib().srq_copy_d2h(ex.h, _np_ptr(out_s), C.c_void_p(self.scales_ptr), sb))
        return out_v, out_s

    def dequant_rows(self, ex, rows):
        rows = np.asarray(rows, np.int32)
        r = ex.upload(rows)
        out = ex.empty(len(rows) * self.cols * 4)
        check(lib().srq_dequant_rows(ex.h, self.h, r.ptr, len(rows), out.ptr))
        return out.to_numpy(np.float32, (len(rows), self.cols))

    def close(self):
        if self.h and self.owner is None:
            lib().srq_weight_destroy(self.h)
        self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def linear(ex, w, x):
    """y = x . W^T for host x [n, cols] through srq_linear; returns host y."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1, w.cols)
    n = x.shape[0]
    xb = ex.upload(x)
    yb = ex.empty(n * w.rows * 4)
    check(lib().srq_linear(ex.h, yb.ptr, xb.ptr, w.h, n))
    return yb.to_numpy(np.float32, (n, w.rows))


class Model:
    """HF Llama/Mistral/Qwen2 profile model resident on one device."""

    def __init__(self, ex, config, weight_format):
        self.ex = ex
        self.config = config
        h = C.c_void_p()
        check(lib().srq_model_create(ex.h, C.byref(config), weight_format.encode(), C.byref(h)))
        self.h = h
        self.format = weight_format

    def load(self, kind, layer, array, dtype=SRC_F32, cancel=None):
        """readParam: one tensor from a host array (f32, or uint16 words for
        SRC_BF16 / SRC_F16) through srq_model_load_host.  cancel: an
        optional ctypes.c_int32 polled between 16 MiB chunks."""
        array = np.ascontiguousarray(array)
        flag = C.byref(cancel) if cancel is not None else None
        check(lib().srq_model_load_host(self.h, kind, layer, _np_ptr(array), dtype, flag))

    def load_uploaded(self, kind, layer, array, dtype=SRC_F32):
        """The same tensor uploaded first, then srq_model_load (device source)."""
        buf = self.ex.upload(np.ascontiguousarray(array))
        check(lib().srq_model_load(self.h, kind, layer, buf.ptr, dtype))

    def load_device(self, kind, layer, ptr, dtype=SRC_F32):
        check(lib().srq_model_load(self.h, kind, layer, C.c_void_p(ptr), dtype))

    def load_safetensors(self, directory, cancel=None):
        """Every tensor of the profile from a Transformers archive directory
        (model.safetensors or an indexed set of shards); returns the
        archive's size in bytes.  cancel: an optional ctypes.c_int32 polled
        between chunks."""
        size = C.c_int64()
        flag = C.byref(cancel) if cancel is not None else None
        check(lib().srq_model_load_safetensors(self.h, os.fsencode(directory), flag, C.byref(size)))
        return size.value

    def resident_bytes(self):
        b = C.c_int64()
        check(lib().srq_model_resident_bytes(self.h, C.byref(b)))
        return b.value

    def weight(self, kind, layer=0):
        h = C.c_void_p()
        check(lib().srq_model_weight(self.h, kind, layer, C.byref(h)))
        return Weight(h, owner=self)

    def rope_tables(self):
        hd = self.config.dim // self.config.heads
        cos = np.empty((self.config.context, hd // 2), np.float32)
        sin = np.empty_like(cos)
        check(lib().srq_model_rope_tables(self.h, _np_ptr(cos), _np_ptr(sin)))
        return cos, sin

    def pool(self, max_pages):
        return Pool(self, max_pages)

    def step(self, caches, chunks, want=None, cancel=None, host=True):
        """prefillSelected: returns host logits [sessions, vocab], or with
        host=False the device pointer of the step's logits (borrowed until
        the executor's next step)."""
        sessions = len(caches)
        lens = np.array([len(c) for c in chunks], np.int32)
        tokens = np.concatenate([np.asarray(c, np.int32) for c in chunks]).astype(np.int32)
        handles = (C.c_void_p * sessions)(*[c.h for c in caches])
        w = None if want is None else np.array(want, np.uint8)
        out = np.zeros((sessions, self.config.vocab), np.float32) if host else None
        dev = C.c_void_p()
        cflag = None if cancel is None else C.cast(C.pointer(cancel), C.c_void_p)
        check(lib().srq_step(self.ex.h, self.h, sessions, C.cast(handles, C.c_void_p), _np_ptr(lens), _np_ptr(tokens),
                             _np_ptr(w) if w is not None else None, C.byref(dev),
                             _np_ptr(out) if host else None, cflag))
        self.last_logits_ptr = dev.value
        return out if host else dev

    def argmax_last(self, rows=1):
        ids = np.zeros(rows, np.int32)
        check(lib().srq_argmax(self.ex.h, C.c_void_p(self.last_logits_ptr), rows, self.config.vocab, _np_ptr(ids)))
        return ids

    def generate_greedy(self, cache, ids, count, chunk=16, eos=-1):
        ids = np.asarray(ids, np.int32)
        out = np.zeros(count, np.int32)
        produced = C.c_int32()
        rc = lib().srq_generate_greedy(self.ex.h, self.h, cache.h, _np_ptr(ids), len(ids), chunk, count, eos,
                                       _np_ptr(out), C.byref(produced))
        if rc != OK:
            try:
                check(rc)
            except SrqError as e:
                e.tokens = out[:produced.value].tolist()
                raise
        return out[:produced.value].tolist()

    def close(self):
        if self.h:
            lib().srq_model_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Pool:
    def __init__(self, model, max_pages):
        self.model = model
        h = C.c_void_p()
        check(lib().srq_pool_create(model.h, max_pages, C.byref(h)))
        self.h = h

    def cache(self, reserve_pages):
        return Cache(self, reserve_pages)

    def close(self):
        if self.h:
            lib().srq_pool_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Cache:
    def __init__(self, pool, reserve_pages):
        self.pool = pool
        h = C.c_void_p()
        check(lib().srq_cache_create(pool.h, reserve_pages, C.byref(h)))
        self.h = h

    @property
    def pos(self):
        p = C.c_int32()
        check(lib().srq_cache_pos(self.h, C.byref(p)))
        return p.value

    def read(self, layer, pos0, count):
        cfg = self.pool.model.config
        kd = cfg.dim // cfg.heads * cfg.kv_heads
        k = np.zeros((count, kd), np.float32)
        v = np.zeros((count, kd), np.float32)
        check(lib().srq_cache_read(self.pool.model.ex.h, self.h, layer, pos0, count, _np_ptr(k), _np_ptr(v)))
        return k, v

    def close(self):
        if self.h:
            lib().srq_cache_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Sampling(C.Structure):
    """srq_sampling: temperature (0: greedy), top_k (0: off), top_p (>= 1:
    off), repeat_penalty (1: off)."""
    _fields_ = [("temperature", C.c_double), ("top_k", C.c_int32), ("top_p", C.c_double),
                ("repeat_penalty", C.c_double)]


def sample(ex, logits_ptr, rows, vocab, params, rng_states, histories=None, blocked=None, row_ids=None):
    """srq_sample over device logits; rng_states (np.uint64 [rows]) is
    advanced in place; histories: list of per-row id lists or None; row_ids:
    the logits row each of the rows samples (None: row k)."""
    rng = np.ascontiguousarray(rng_states, np.uint64)
    assert rng.shape == (rows,) and rng is rng_states, "rng_states must be a contiguous uint64 array"
    ids = np.zeros(rows, np.int32)
    hist = hl = None
    stride = 0
    if histories is not None:
        stride = max(1, max(len(h) for h in histories))
        hist = np.zeros((rows, stride), np.int32)
        hl = np.zeros(rows, np.int32)
        for r, h in enumerate(histories):
            hist[r, :len(h)] = h
            hl[r] = len(h)
    blk = None if blocked is None else np.ascontiguousarray(blocked, np.int32)
    sel = None if row_ids is None else np.ascontiguousarray(row_ids, np.int32)
    ptr = lambda a: None if a is None else _np_ptr(a)
    check(lib().srq_sample(ex.h, logits_ptr, rows, ptr(sel), vocab, C.byref(params), ptr(hist), ptr(hl), stride,
                           ptr(blk), _np_ptr(rng), _np_ptr(ids)))
    return ids


class Decoder:
    """Graph-replayed greedy decode loop on one cache."""

    def __init__(self, model, cache, first_token, max_steps, eager=False):
        self.model = model
        h = C.c_void_p()
        check(lib().srq_decoder_create(model.ex.h, model.h, cache.h, int(first_token), max_steps, 1 if eager else 0,
                                       C.byref(h)))
        self.h = h
        self.max_steps = max_steps

    def run(self, steps):
        check(lib().srq_decoder_run(self.h, steps))

    def tokens(self):
        """Tokens produced so far.  On SRQ_ENONFINITE the SrqError carries
        the tokens before the failing step as .tokens."""
        out = np.zeros(self.max_steps, np.int32)
        n = C.c_int32()
        rc = lib().srq_decoder_tokens(self.h, _np_ptr(out), C.byref(n))
        if rc != OK:
            try:
                check(rc)
            except SrqError as e:
                e.tokens = out[:n.value].tolist()
                raise
        return out[:n.value].tolist()

    def close(self):
        if self.h:
            lib().srq_decoder_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def make_config(vocab, dim, layers, heads, kv_heads, hidden, context, rope_theta=10000.0, norm_eps=1e-5, tied=True,
                qkv_bias=False, llama3=None):
    c = ModelConfig(vocab, dim, layers, heads, kv_heads, hidden, context, rope_theta, norm_eps, int(tied),
                    int(qkv_bias), 0, 0.0, 0.0, 0.0, 0)
    if llama3:
        c.rope_llama3 = 1
        c.rope_factor = llama3["factor"]
        c.rope_low = llama3["low_freq_factor"]
        c.rope_high = llama3["high_freq_factor"]
        c.rope_original = llama3["original_max_position_embeddings"]
    return c
