"""GPU parity of the batched step (prefillSelected), KV pages, selective
heads, greedy generation and the graph-replayed decoder, through the C ABI.

Bars: FP32 models match Transformers' logits and every K/V row of the
reference's fixtures at the reference's own 2e-5 (hf_inference_test.go:74);
quantized models match the oracle's quantized step within
|got - want| <= 1e-4 * max(1, |want|); greedy token sequences are identical
to the oracle's."""
import ctypes as C

import numpy as np
import pytest

import oracle
import sr_go_tranformer_amd as srq
from tests import gpu_models, hf_fixtures

pytestmark = pytest.mark.gpu
TOL = 1e-4


@pytest.fixture(scope="module")
def ex():
    e = srq.Executor(0)
    yield e
    e.close()


def near(got, want, tol=TOL, floor=1.0):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert np.all(np.isfinite(got))
    err = np.abs(got - want) / np.maximum(floor, np.abs(want))
    assert err.max() <= tol, (float(err.max()), int(err.argmax()))


def absnear(got, want, tol):
    got = np.asarray(got, np.float64)
    assert np.all(np.isfinite(got))
    err = np.abs(got - np.asarray(want, np.float64))
    assert err.max() <= tol, (float(err.max()), int(err.argmax()))


@pytest.mark.parametrize("name", hf_fixtures.NAMES)
@pytest.mark.parametrize("chunk", [1, 4, 16, 35])
def test_fp32_step_matches_transformers(ex, name, chunk):
    print("fixture", name, "chunk", chunk, flush=True)
    fx = hf_fixtures.load(name)
    m = gpu_models.load_fixture(ex, fx, "f32", use_raw=True)
    pool = m.pool(8)
    cache = pool.cache(4)
    for lo in range(0, 35, chunk):
        hi = min(lo + chunk, 35)
        absnear(m.step([cache], [fx.ids[lo:hi]])[0], fx.logits[hi - 1], 2e-5)
    for pos in range(35, len(fx.ids)):
        absnear(m.step([cache], [[fx.ids[pos]]])[0], fx.logits[pos], 2e-5)
    assert cache.pos == len(fx.ids)
    for layer in range(fx.layers):
        k, v = cache.read(layer, 0, len(fx.ids))
        absnear(k, fx.k[layer], 2e-5)
        absnear(v, fx.v[layer], 2e-5)


@pytest.mark.parametrize("name", ["llama_f32", "llama_untied-f32", "llama3_f32", "llama3_f16", "mistral_f32",
                                  "mistral_f16", "mistral_bf16", "qwen2_f32", "qwen2_f16", "qwen2_untied-bf16"])
@pytest.mark.parametrize("fmt", ["q8", "q4", "q4-mixed"])
def test_quantized_step_matches_oracle(ex, name, fmt):
    print("quantized", name, fmt, flush=True)
    fx = hf_fixtures.load(name)
    m = gpu_models.load_fixture(ex, fx, fmt, use_raw=True)
    om = fx.oracle_model(fmt)
    pool = m.pool(8)
    cache, ocache = pool.cache(4), om.new_cache()
    lo = 0
    for c in (33, 1, 2, 1):
        near(m.step([cache], [fx.ids[lo:lo + c]])[0], om.step([ocache], [fx.ids[lo:lo + c]])[0])
        lo += c
    for layer in range(fx.layers):
        k, v = cache.read(layer, 0, 37)
        near(k, np.stack([ocache.row(layer, p, 0) for p in range(37)]))
        near(v, np.stack([ocache.row(layer, p, 1) for p in range(37)]))


@pytest.mark.parametrize("name", ["llama_f32", "mistral_f32", "qwen2_f32"])
def test_ragged_sessions_and_selective_heads(ex, name):
    fx = hf_fixtures.load(name)
    m = gpu_models.load_fixture(ex, fx, "f32")
    pool = m.pool(16)
    ca, cb = pool.cache(4), pool.cache(4)
    got = m.step([ca, cb], [fx.ids[:35], fx.ids[:4]])
    absnear(got[0], fx.logits[34], 2e-5)
    absnear(got[1], fx.logits[3], 2e-5)
    got = m.step([ca, cb], [[fx.ids[35]], [fx.ids[4]]])
    absnear(got[0], fx.logits[35], 2e-5)
    absnear(got[1], fx.logits[4], 2e-5)
    cc, cd = pool.cache(4), pool.cache(4)
    sel = m.step([cc, cd], [fx.ids[:35], fx.ids[:4]], want=[False, True])
    assert np.all(sel[0] == 0)
    absnear(sel[1], fx.logits[3], 2e-5)
    assert (cc.pos, cd.pos) == (35, 4)


def test_step_validation_never_mutates(ex):
    fx = hf_fixtures.load("llama_f32")
    m = gpu_models.load_fixture(ex, fx, "q8")
    pool = m.pool(6)
    c = pool.cache(4)
    m.step([c], [fx.ids[:3]])

    def code(fn):
        with pytest.raises(srq.SrqError) as e:
            fn()
        return e.value.code

    assert code(lambda: m.step([c], [[fx.vocab]])) == srq.EINVAL
    assert code(lambda: m.step([c, c], [[1], [2]])) == srq.EINVAL
    assert code(lambda: m.step([c], [[]])) == srq.EINVAL
    assert code(lambda: m.step([c], [list(range(1, 127))])) == srq.ERANGE
    small = pool.cache(1)
    assert code(lambda: m.step([small], [list(range(1, 40))])) == srq.ENOSPC
    flag = C.c_int32(1)
    assert code(lambda: m.step([c], [[5]], cancel=flag)) == srq.ECANCELED
    assert code(lambda: pool.cache(2)) == srq.ENOSPC  # 4 + 1 + 2 > 6 pages
    assert c.pos == 3 and small.pos == 0
    out = m.step([c], [[5]])
    assert np.all(np.isfinite(out)) and c.pos == 4


def test_queued_step_equals_waited_step(ex):
    """srq_step with neither a host copy nor a cancel flag returns once the
    step is queued: positions are committed at once, and the device logits
    and K/V rows that later calls read are, bit for bit, those of the same
    steps made with a host copy (which wait for the device)."""
    fx = hf_fixtures.load("llama_f32")
    m = gpu_models.load_fixture(ex, fx, "q8")
    pool = m.pool(8)
    a, b = pool.cache(3), pool.cache(3)
    ids = [int(t) for t in fx.ids[:10]]
    for lo in range(0, len(ids), 4):
        want = m.step([a], [ids[lo:lo + 4]])
    for lo in range(0, len(ids), 4):
        dev = m.step([b], [ids[lo:lo + 4]], host=False)
        assert b.pos == min(lo + 4, len(ids))
    got = np.empty_like(want)
    srq.check(srq.lib().srq_copy_d2h(ex.h, got.ctypes.data_as(C.c_void_p), dev, got.nbytes))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    for layer in range(fx.layers):
        ka, va = a.read(layer, 0, len(ids))
        kb, vb = b.read(layer, 0, len(ids))
        assert np.array_equal(ka.view(np.uint32), kb.view(np.uint32)), layer
        assert np.array_equal(va.view(np.uint32), vb.view(np.uint32)), layer
    a.close()
    b.close()
    pool.close()
    m.close()


def test_greedy_generate_and_decoder(ex):
    fx = hf_fixtures.load("mistral_f32")
    for fmt in ("q8", "q4-mixed"):
        m = gpu_models.load_fixture(ex, fx, fmt)
        om = fx.oracle_model(fmt)
        pool = m.pool(16)
        ids = fx.ids[:20]
        want, _ = oracle.greedy(om, ids, 40, 7)
        c = pool.cache(4)
        got = m.generate_greedy(c, ids, 40, chunk=7)
        assert got == want, (got, want)
        assert c.pos == 20 + 40 - 1
        # EOS stops generation: the first produced token is the stop id.
        c2 = pool.cache(4)
        stop = want[5]
        got = m.generate_greedy(c2, ids, 40, chunk=7, eos=stop)
        k = want.index(stop) + 1
        assert got == want[:k] and c2.pos == 20 + k - 1
        # Decoder API: first token from the prefill argmax, then replays.
        c3 = pool.cache(4)
        m.step([c3], [ids])
        first = int(m.argmax_last()[0])
        assert first == want[0]
        d = srq.Decoder(m, c3, first, 30)
        d.run(10)
        d.run(20)
        assert d.tokens() == want[1:31] and c3.pos == 50
        d.close()
        c4 = pool.cache(4)
        m.step([c4], [ids])
        d = srq.Decoder(m, c4, first, 12, eager=True)
        d.run(12)
        assert d.tokens() == want[1:13] and c4.pos == 32
        d.close()


def test_long_context_decode(ex):
    """Decode past 1024 positions at head_dim 128: more than 16 attention
    splits, so the split + combine path replaces the fused one.  Greedy
    tokens (graph-replayed and eager decoders, batched steps) against the
    oracle's."""
    cfg = srq.make_config(512, 256, 2, 2, 1, 512, 1400, 10000.0, 1e-5, True)
    m, norms = gpu_models.synthetic(ex, cfg, "q8", 5)
    om = gpu_models.oracle_from_device(ex, m, cfg, norms)
    ids = [int(t) for t in np.random.default_rng(3).integers(0, cfg.vocab, size=1100)]
    want, _ = oracle.greedy(om, ids, 12, 256)
    pool = m.pool(3 * 36)
    for eager in (False, True):
        c = pool.cache(36)
        for lo in range(0, len(ids), 256):
            m.step([c], [ids[lo:lo + 256]])
        first = int(m.argmax_last()[0])
        assert first == want[0]
        d = srq.Decoder(m, c, first, 11, eager=eager)
        d.run(11)
        assert d.tokens() == want[1:12], (eager, d.tokens(), want[1:12])
        d.close()
    c = pool.cache(36)
    got = m.generate_greedy(c, ids, 12, chunk=256)
    assert got == want


@pytest.mark.parametrize("dim,heads,kv_heads", [(512, 4, 1), (512, 8, 1), (512, 8, 8), (384, 6, 2), (1024, 8, 1)])
def test_prefill_attention_tiles_match_oracle(ex, dim, heads, kv_heads):
    """Prefill-sized steps (at least 32 rows, at least 8 rows per query tile)
    take the MFMA flash kernel: head_dim 128 or 64, GQA groups of 1..8
    query heads (two passes past 4), key splits, partial tiles at chunk and
    session ends, two sessions in one step.  Logits against the oracle's
    step at 1e-4, then greedy continuation identical."""
    print("flash", dim, heads, kv_heads, flush=True)
    cfg = srq.make_config(300, dim, 2, heads, kv_heads, 256, 1400, 10000.0, 1e-5, True)
    m, norms = gpu_models.synthetic(ex, cfg, "q8", 11)
    om = gpu_models.oracle_from_device(ex, m, cfg, norms)
    rng = np.random.default_rng(dim + heads + kv_heads)
    a_ids = [int(t) for t in rng.integers(0, cfg.vocab, size=700)]
    b_ids = [int(t) for t in rng.integers(0, cfg.vocab, size=300)]
    pool = m.pool(64)
    ca, cb = pool.cache(24), pool.cache(24)
    oa, ob = om.new_cache(), om.new_cache()
    # one session: 37 (tile remainder), then 256 at offset 37, then 200
    lo = 0
    for c in (37, 256, 200):
        near(m.step([ca], [a_ids[lo:lo + c]])[0], om.step([oa], [a_ids[lo:lo + c]])[0])
        lo += c
    # two sessions in one step: 40 rows of B (fresh) and 167 rows of A (past 493)
    got = m.step([cb, ca], [b_ids[:40], a_ids[lo:lo + 167]])
    want = om.step([ob, oa], [b_ids[:40], a_ids[lo:lo + 167]])
    near(got[0], want[0])
    near(got[1], want[1])
    # K/V rows written by the tiled steps drive a later decode
    for layer in range(cfg.layers):
        k, v = ca.read(layer, 0, 660)
        near(k, np.stack([oa.row(layer, p, 0) for p in range(660)]))
        near(v, np.stack([oa.row(layer, p, 1) for p in range(660)]))


@pytest.mark.parametrize("dim,heads,kv_heads,fmt", [(512, 4, 1, "q8"), (1024, 8, 2, "q8"), (1024, 8, 2, "q4")])
def test_qkv_bias_through_fused_rope_reduction(ex, dim, heads, kv_heads, fmt):
    """q/k/v biases (the Qwen2 profile) on split-K q/k/v GEMMs: the split
    reduction adds the bias, applies RoPE and writes K/V (rope_kv_kernel's
    arithmetic, M:3933-3940, M:5264-5289).  Logits and every K/V row of
    40- and 33-row steps, then a 3-row GEMV step, against the oracle."""
    print("qkv bias", dim, heads, kv_heads, fmt, flush=True)
    cfg = srq.make_config(300, dim, 2, heads, kv_heads, 512, 1400, 10000.0, 1e-5, True, qkv_bias=True)
    m, norms = gpu_models.synthetic(ex, cfg, fmt, 31)
    kvdim = dim // heads * kv_heads
    rng = np.random.default_rng(dim + heads)
    for layer in range(cfg.layers):
        for kind, name, width in ((srq.T_Q_BIAS, "q_bias", dim), (srq.T_K_BIAS, "k_bias", kvdim),
                                  (srq.T_V_BIAS, "v_bias", kvdim)):
            b = rng.normal(0.0, 0.5, size=width).astype(np.float32)
            m.load(kind, layer, b)
            norms["layers.%d.%s" % (layer, name)] = b
    om = gpu_models.oracle_from_device(ex, m, cfg, norms)
    ids = [int(t) for t in rng.integers(0, cfg.vocab, size=76)]
    pool = m.pool(8)
    c, oc = pool.cache(4), om.new_cache()
    lo = 0
    for n in (40, 33, 3):
        near(m.step([c], [ids[lo:lo + n]])[0], om.step([oc], [ids[lo:lo + n]])[0])
        lo += n
    for layer in range(cfg.layers):
        k, v = c.read(layer, 0, lo)
        near(k, np.stack([oc.row(layer, p, 0) for p in range(lo)]))
        near(v, np.stack([oc.row(layer, p, 1) for p in range(lo)]))


def test_wide_rows_through_fused_reductions(ex):
    """A value projection scaled to ~1e34 makes the attention output exceed
    f32(MaxFloat32/(2*64*127)) (M:4346-4354), so the o projection of a
    40-row step (split-K MFMA GEMM, residual and RMSNorm in its reduction),
    of a 4-row step and of a 1-row step (the streaming GEMV) computes those
    rows in FP64 (linearQ8WideInto, M:4356-4382).  Logits and K/V rows
    against the oracle's step."""
    cfg = srq.make_config(300, 512, 2, 4, 1, 512, 1400, 10000.0, 1e-5, True)
    m, norms = gpu_models.synthetic(ex, cfg, "q8", 21)
    kvdim = cfg.dim // cfg.heads * cfg.kv_heads
    v = (np.random.default_rng(5).normal(0.0, 0.02, size=(kvdim, cfg.dim)) * 1e36).astype(np.float32)
    m.load(srq.T_V, 0, v)
    om = gpu_models.oracle_from_device(ex, m, cfg, norms)
    ids = [int(t) for t in np.random.default_rng(6).integers(0, cfg.vocab, size=45)]
    pool = m.pool(8)
    c, oc = pool.cache(4), om.new_cache()
    got = m.step([c], [ids[:40]])[0]
    want = om.step([oc], [ids[:40]])[0]
    assert np.all(np.isfinite(got))
    near(got, want)
    # the next rows (a 4-row step, then one row: the streaming GEMV's FP64
    # pass)
    near(m.step([c], [ids[40:44]])[0], om.step([oc], [ids[40:44]])[0])
    near(m.step([c], [ids[44:]])[0], om.step([oc], [ids[44:]])[0])
    # V rows of ~1e35: an entry near cancellation carries the f32 rounding of
    # its ~1e35 terms, so the bound is relative to the row's largest entry.
    for layer in range(cfg.layers):
        k, vv = c.read(layer, 0, 45)
        want_v = np.stack([oc.row(layer, p, 1) for p in range(45)]).astype(np.float64)
        bound = 1e-4 * np.abs(want_v).max(axis=1, keepdims=True)
        assert np.all(np.abs(vv.astype(np.float64) - want_v) <= bound), layer


def test_smollm2_shape_greedy_identity(ex):
    """SmolLM2-135M architecture (576 / 30 layers / 9:3 heads / 1536 /
    49152 tied), seeded N(0, 0.02) weights, Q8; 32-token prompt (one MFMA
    chunk) and 64 greedy tokens, identical to the oracle."""
    cfg = srq.make_config(49152, 576, 30, 9, 3, 1536, 2048, 10000.0, 1e-5, True)
    m, norms = gpu_models.synthetic(ex, cfg, "q8", seed=1)
    om = gpu_models.oracle_from_device(ex, m, cfg, norms)
    r = oracle.RNG(99)
    ids = [r.intn(cfg.vocab) for _ in range(32)]
    want, wlog = oracle.greedy(om, ids, 64, 32)
    margins = [float(np.sort(l)[-1] - np.sort(l)[-2]) for l in wlog]
    print("min top-2 margin %.3g" % min(margins), flush=True)
    pool = m.pool(8)
    c = pool.cache(4)
    got = m.generate_greedy(c, ids, 64, chunk=32)
    assert got == want
    # the first logits (MFMA prefill of 32 rows) within the bound
    c2 = pool.cache(4)
    first = m.step([c2], [ids])[0]
    near(first, wlog[0])


def test_fill_normal_matches_serial_rng(ex):
    buf = ex.empty(100000 * 4)
    srq.fill_normal(ex, buf, 100000, 12345, 0.02)
    got = buf.to_numpy(np.float32, (100000,))
    want = oracle.RNG(12345).fill_normal(100000, 0.02)
    diff = got.view(np.int32).astype(np.int64) - want.view(np.int32).astype(np.int64)
    assert np.abs(diff).max() <= 1 and (diff != 0).mean() < 1e-3


def test_fused_storage_views(ex):
    """SRQ_T_QKV / SRQ_T_GATE_UP borrow the fused matrices the step streams:
    their rows are the q, k, v (gate, up) rows, so a GEMV over the fused view
    equals the per-matrix GEMVs bit for bit."""
    fx = hf_fixtures.load("mistral_f32")
    m = gpu_models.load_fixture(ex, fx, "q8")
    x = np.random.default_rng(3).normal(size=(2, fx.dim)).astype(np.float32)
    for layer in (0, fx.layers - 1):
        gu = m.weight(srq.T_GATE_UP, layer)
        assert (gu.rows, gu.cols) == (2 * fx.hidden, fx.dim)
        got = srq.linear(ex, gu, x)
        want = np.concatenate([srq.linear(ex, m.weight(srq.T_GATE, layer), x),
                               srq.linear(ex, m.weight(srq.T_UP, layer), x)], axis=1)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        qkv = m.weight(srq.T_QKV, layer)
        got = srq.linear(ex, qkv, x)
        want = np.concatenate([srq.linear(ex, m.weight(k, layer), x) for k in (srq.T_Q, srq.T_K, srq.T_V)], axis=1)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    with pytest.raises(srq.SrqError):
        m.weight(srq.T_GATE_UP, fx.layers)
