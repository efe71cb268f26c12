"""Batch and chunk invariance, multi-session long-context steps and the
decoder's error and ownership rules, on the GPU through the C ABI.

The reference's kernels give a row the same bits whatever else shares the
call (q8_test.go:83-92, quant_pair_test.go:12-41) and chunked prefill equals
tokenwise prefill (prompt_prefill_test.go:71-120).  Here a row's bits
depend only on which path computes it: the GEMV (srq_linear n <= 16, steps
of at most 4 rows) or the MFMA GEMM (above), and for attention the split
kernels or, for prefill-sized steps, the flash kernel.  Within a path they
do not depend on n, on the row's position or on the other sessions."""
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


def near(got, want, tol=TOL):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert np.all(np.isfinite(got))
    err = np.abs(got - want) / np.maximum(1.0, np.abs(want))
    assert err.max() <= tol, (float(err.max()), int(err.argmax()))


def same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


@pytest.mark.parametrize("fmt,rows,cols", [(srq.Q8, 4096, 4096), (srq.Q4, 6144, 4096), (srq.Q8, 28672, 4096),
                                           (srq.Q8, 1000, 1056), (srq.F32, 512, 2048)])
def test_linear_rows_independent_of_n(ex, fmt, rows, cols):
    """srq_linear: the GEMV rows (n <= 16) and the MFMA GEMM rows (n > 16,
    bf16 three-term kernel, or the FP32 kernel for widths off 64 and F32
    weights) each give every row the same bits for any n."""
    print("linear invariance", fmt, rows, cols, flush=True)
    rng = oracle.RNG(rows * 3 + cols)
    dense = rng.fill_normal(rows * cols, 0.02).reshape(rows, cols)
    w = srq.Weight.create(ex, dense, fmt)
    x = rng.fill_normal(256 * cols, 1.0).reshape(256, cols)
    gemv = {n: srq.linear(ex, w, x[:n]) for n in (1, 3, 8, 16)}
    for n in (3, 8, 16):
        assert same_bits(gemv[n][:1], gemv[1]), n
        assert same_bits(gemv[n][:3], gemv[3][:3]), n
    gemm = {n: srq.linear(ex, w, x[:n]) for n in (17, 33, 64, 256)}
    for n in (33, 64, 256):
        assert same_bits(gemm[n][:17], gemm[17]), n
    assert same_bits(gemm[256][:64], gemm[64])
    # a row's bits do not depend on its position in the batch either
    perm = x[:64][::-1].copy()
    assert same_bits(srq.linear(ex, w, perm)[::-1], gemm[64])
    ofmt = {srq.Q8: oracle.Q8, srq.Q4: oracle.Q4, srq.F32: oracle.F32}[fmt]
    ow = oracle.Weight.from_dense(dense, ofmt)
    near(gemm[64], oracle.linear(ow, x[:64], workers=16))


def _step_alone_and_in_batches(ex, cfg, seed, prompt_n, ns, heads=1, fmt="q8"):
    """Session A's decode logits at position prompt_n in steps of n rows:
    A's row plus companion sessions of at most 3 rows each (so no step is
    prefill-sized), of which the first heads - 1 want logits too.  A's
    prefix is prefilled the same way each time."""
    m, norms = gpu_models.synthetic(ex, cfg, fmt, seed)
    om = gpu_models.oracle_from_device(ex, m, cfg, norms)
    rng = np.random.default_rng(seed)
    a_ids = [int(t) for t in rng.integers(0, cfg.vocab, size=prompt_n + 1)]
    pool = m.pool(2 * ((prompt_n + 32) // 32 + 1) + 100)
    oc = om.new_cache()
    for lo in range(0, prompt_n, 256):
        om.step([oc], [a_ids[lo:min(lo + 256, prompt_n)]], workers=16)
    want = om.step([oc], [[a_ids[prompt_n]]], workers=16)[0]
    out = {}
    for n in ns:
        ca = pool.cache((prompt_n + 32) // 32 + 1)
        for lo in range(0, prompt_n, 256):
            m.step([ca], [a_ids[lo:min(lo + 256, prompt_n)]])
        comp, rows = [], n - 1
        while rows > 0:
            k = min(3, rows)
            comp.append([int(t) for t in rng.integers(0, cfg.vocab, size=k)])
            rows -= k
        caches = [pool.cache(1) for _ in comp]
        want_rows = [True] + [k < heads - 1 for k in range(len(comp))]
        got = m.step([ca] + caches, [[a_ids[prompt_n]]] + comp, want=want_rows)
        near(got[0], want)
        out[n] = got[0]
        for c in caches:
            c.close()
        ca.close()
    return out


@pytest.mark.parametrize("prompt_n", [40, 1100])
def test_step_rows_independent_of_batch(ex, prompt_n):
    """A decode row's logits are bit-identical in steps of 1, 3 and 4 rows
    (GEMV layers) and in steps of 5, 8, 9, 12, 16, 17, 33, 64 and 256 rows
    (MFMA GEMM layers: 16-, 32- and 64-row tiles over the same K slices), at
    40 and 1100 positions (attention: fused split + merge up to 64 rows,
    split + combine for 256, past 16 splits in the combine's grouped
    summation order).  The head takes the GEMV for up to 4 sessions wanting
    logits and the GEMM above: within each, the logits do not depend on how
    many sessions want them."""
    print("step invariance", prompt_n, flush=True)
    cfg = srq.make_config(512, 256, 2, 2, 1, 512, 1400, 10000.0, 1e-5, True)
    seed = 5 + prompt_n
    out = _step_alone_and_in_batches(ex, cfg, seed, prompt_n, (1, 3, 4, 5, 8, 9, 12, 16, 17, 33, 64, 256))
    for n in (3, 4):
        assert same_bits(out[n], out[1]), n
    for n in (8, 9, 12, 16, 17, 33, 64, 256):
        assert same_bits(out[n], out[5]), n
    for heads in (2, 4):
        got = _step_alone_and_in_batches(ex, cfg, seed, prompt_n, (64,), heads=heads)
        assert same_bits(got[64], out[64]), heads
    many = {h: _step_alone_and_in_batches(ex, cfg, seed, prompt_n, (64, 256), heads=h) for h in (5, 17, 40)}
    assert same_bits(many[40][64], many[17][64]) and same_bits(many[40][256], many[17][64])
    assert same_bits(many[5][64], many[17][64])


def test_step_rows_independent_of_batch_q4_tiles(ex):
    """Q4 layers: steps of 9 and 16 rows (16-row GEMM tiles), 17 and 32
    (32-row tiles) and 64 (64-row tiles) give a decode row the same bits."""
    print("q4 tile-height step invariance", flush=True)
    cfg = srq.make_config(512, 256, 2, 2, 1, 512, 1400, 10000.0, 1e-5, True)
    out = _step_alone_and_in_batches(ex, cfg, 41, 40, (9, 16, 17, 32, 64), fmt="q4")
    for n in (16, 17, 32, 64):
        assert same_bits(out[n], out[9]), n


def test_step_rows_independent_of_batch_wide_slices(ex):
    """Llama-3.2-3B widths (dim 3072, 8 KV heads of 128, FFN 8192), one
    layer: the down projection's K slices hold 13 blocks, so steps of 5, 8
    and 16 rows (16-row pair-streamed tiles), 17 and 32 (32-row pair-streamed
    tiles) and 33 and 64 (64-row unrolled tiles) run three kernels over the
    same slices; a decode row keeps the 5-row step's bits (and the oracle's
    logits within 1e-4)."""
    print("wide-slice step invariance", flush=True)
    cfg = srq.make_config(512, 3072, 1, 24, 8, 8192, 200, 10000.0, 1e-5, True)
    out = _step_alone_and_in_batches(ex, cfg, 61, 40, (5, 8, 16, 17, 32, 33, 64))
    for n in (8, 16, 17, 32, 33, 64):
        assert same_bits(out[n], out[5]), n


def test_step_rows_independent_of_batch_row_groups(ex):
    """Steps of 3 and 4 rows stream the 4100-unit gate/up GEMV two units
    per step and the 8200-id head four rows per step (row groups, the last
    group ragged); a decode row's logits keep the bits of a 1-row step."""
    print("row-group step invariance", flush=True)
    cfg = srq.make_config(8200, 256, 1, 2, 1, 4100, 300, 10000.0, 1e-5, True)
    out = _step_alone_and_in_batches(ex, cfg, 23, 40, (1, 3, 4), heads=4)
    for n in (3, 4):
        assert same_bits(out[n], out[1]), n


@pytest.mark.parametrize("fmt", ["q8", "q4"])
def test_step_rows_independent_of_batch_long_context(ex, fmt):
    """Width 1024 (8 heads x 128), Q8 and Q4, at 4200 positions: more than
    64 attention splits per row (split + combine attention).  Steps of 1,
    2, 3 and 4 rows (GEMV layers) give A's row the same bits, and so do steps
    of 5 and 8 rows (GEMM layers)."""
    print("long-context step invariance", fmt, flush=True)
    cfg = srq.make_config(512, 1024, 2, 8, 2, 1024, 4300, 10000.0, 1e-5, True)
    out = _step_alone_and_in_batches(ex, cfg, 31, 4200, (1, 2, 3, 4, 5, 8), fmt=fmt)
    for n in (2, 3, 4):
        assert same_bits(out[n], out[1]), n
    assert same_bits(out[8], out[5])


def test_long_row_fused_and_sliced_merge_same_bits(ex):
    """A decode row at 1100 positions (18 splits) alone takes the fused
    split + merge kernel; beside a row at 3200 positions the step has more
    than 48 splits and takes split + combine, where the row's one-head merge
    runs on 8 workgroups per head (slices of the head's dims).  The row's
    logits are bit-identical, and match the oracle's."""
    print("fused vs sliced merge", flush=True)
    cfg = srq.make_config(512, 256, 2, 2, 1, 512, 3400, 10000.0, 1e-5, True)
    m, norms = gpu_models.synthetic(ex, cfg, "q8", 53)
    om = gpu_models.oracle_from_device(ex, m, cfg, norms)
    rng = np.random.default_rng(53)
    a_ids = [int(t) for t in rng.integers(0, cfg.vocab, size=1101)]
    b_ids = [int(t) for t in rng.integers(0, cfg.vocab, size=3201)]
    pool = m.pool(2 * (36 + 102) + 8)

    def prefill(ids):
        c = pool.cache((len(ids) + 32) // 32 + 1)
        for lo in range(0, len(ids), 256):
            m.step([c], [ids[lo:min(lo + 256, len(ids))]])
        return c

    ca = prefill(a_ids[:1100])
    alone = m.step([ca], [[a_ids[1100]]])[0]
    ca.close()
    ca, cb = prefill(a_ids[:1100]), prefill(b_ids[:3200])
    beside = m.step([ca, cb], [[a_ids[1100]], [b_ids[3200]]], want=[True, False])[0]
    ca.close()
    cb.close()
    assert same_bits(alone, beside)
    oc = om.new_cache()
    for lo in range(0, 1100, 256):
        om.step([oc], [a_ids[lo:min(lo + 256, 1100)]], workers=16)
    near(alone, om.step([oc], [[a_ids[1100]]], workers=16)[0])


def test_multi_session_long_context_steps(ex):
    """Six sessions past 1024 positions decode one token per step together
    (a 6-row step: fused attention over more than 16 splits); logits
    against the oracle's step, then greedy continuations identical."""
    cfg = srq.make_config(512, 256, 2, 2, 1, 512, 1400, 10000.0, 1e-5, True)
    m, norms = gpu_models.synthetic(ex, cfg, "q8", 17)
    om = gpu_models.oracle_from_device(ex, m, cfg, norms)
    rng = np.random.default_rng(17)
    lens = [1030, 1060, 1100, 1125, 1150, 1201]
    prompts = [[int(t) for t in rng.integers(0, cfg.vocab, size=n)] for n in lens]
    pool = m.pool(6 * 40)
    caches = [pool.cache(40) for _ in lens]
    ocs = [om.new_cache() for _ in lens]
    for i, p in enumerate(prompts):
        for lo in range(0, len(p), 256):
            m.step([caches[i]], [p[lo:lo + 256]])
            last = om.step([ocs[i]], [p[lo:lo + 256]], workers=16)[0]
        prompts[i] = p + [oracle.argmax(last)]
    toks = [[p[-1]] for p in prompts]
    for step in range(6):
        got = m.step(caches, [[t[-1]] for t in toks])
        want = om.step(ocs, [[t[-1]] for t in toks], workers=16)
        for i in range(len(lens)):
            near(got[i], want[i])
            best = oracle.argmax(want[i])
            assert int(np.argmax(got[i])) == best, (step, i)
            toks[i].append(best)


@pytest.mark.parametrize("name", ["llama_f32", "mistral_f32", "qwen2_f32", "llama3_bf16"])
@pytest.mark.parametrize("fmt", ["q8", "q4-mixed"])
def test_chunked_prefill_greedy_identical(ex, name, fmt):
    """prompt_prefill_test.go:71-120: prefill in chunks of 1, 16 and 256
    tokens (the whole prompt) gives the same greedy continuation, equal to
    the oracle's."""
    fx = hf_fixtures.load(name)
    m = gpu_models.load_fixture(ex, fx, fmt, use_raw=True)
    om = fx.oracle_model(fmt)
    ids = fx.ids[:24]
    want, _ = oracle.greedy(om, ids, 24, 7)
    pool = m.pool(16)
    for chunk in (1, 16, 256):
        c = pool.cache(2)
        assert m.generate_greedy(c, ids, 24, chunk=chunk) == want, chunk
        c.close()


def test_decoder_nonfinite_logits_and_cache_ownership(ex):
    """A step whose logits are not finite ends the decode (inferHFIDs,
    M:1212-1238): the tokens before it are returned with SRQ_ENONFINITE and
    the position is committed through that step.  A NaN scale poked into one
    head row after five good replays makes step six non-finite.  While the
    decoder lives, its cache refuses srq_step and a second decoder."""
    fx = hf_fixtures.load("llama_untied-f32")
    m = gpu_models.load_fixture(ex, fx, "q8")
    pool = m.pool(16)
    ids = fx.ids[:20]
    c = pool.cache(2)
    m.step([c], [ids])
    first = int(m.argmax_last()[0])
    d = srq.Decoder(m, c, first, 20)
    with pytest.raises(srq.SrqError) as e:
        m.step([c], [[1]])
    assert e.value.code == srq.EINVAL
    with pytest.raises(srq.SrqError) as e:
        srq.Decoder(m, c, first, 4)
    assert e.value.code == srq.EINVAL
    d.run(5)
    good = d.tokens()
    assert len(good) == 5 and c.pos == 25
    head = m.weight(srq.T_OUTPUT)
    groups = (head.cols + 63) // 64
    row = 7
    addr = head.scales_ptr + row * groups * 4
    saved = np.zeros(1, np.float32)
    srq.check(srq.lib().srq_copy_d2h(ex.h, saved.ctypes.data_as(C.c_void_p), C.c_void_p(addr), 4))
    nan = np.array([np.nan], np.float32)
    srq.check(srq.lib().srq_copy_h2d(ex.h, C.c_void_p(addr), nan.ctypes.data_as(C.c_void_p), 4))
    d.run(5)
    with pytest.raises(srq.SrqError) as e:
        d.tokens()
    assert e.value.code == srq.ENONFINITE
    assert e.value.tokens == good
    assert c.pos == 26
    d.close()
    # the cache is free again; generation with the NaN row fails at once
    c2 = pool.cache(2)
    with pytest.raises(srq.SrqError) as e:
        m.generate_greedy(c2, ids, 8, chunk=20)
    assert e.value.code == srq.ENONFINITE and e.value.tokens == []
    srq.check(srq.lib().srq_copy_h2d(ex.h, C.c_void_p(addr), saved.ctypes.data_as(C.c_void_p), 4))
    out = m.step([c], [[good[-1]]])
    assert np.all(np.isfinite(out)) and c.pos == 27
