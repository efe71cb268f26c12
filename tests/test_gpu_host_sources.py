"""Host-source packing (readParam streams host values, M:857-880) and
in-flight step cancellation (the context check as each layer starts,
M:6376-6378), on the GPU through the C ABI.

Host-source entry points must give the same bits as their device-source
counterparts, reject non-finite values, and stop between 16 MiB chunks
when the cancel flag is set; a step whose flag is raised while it runs must
stop early, commit nothing, and leave the cache usable."""
import ctypes as C
import threading
import time

import numpy as np
import pytest

import oracle
import sr_go_tranformer_amd as srq
from sr_go_tranformer_amd import synthetic as syn
from tests import gpu_models, hf_fixtures

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ex():
    e = srq.Executor(0)
    yield e
    e.close()


def bf16_words(a):
    """Round-to-nearest-even f32 -> bf16 words (uint16)."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


@pytest.mark.parametrize("fmt", [srq.Q8, srq.Q4])
@pytest.mark.parametrize("rows,cols", [(4200, 1100), (37, 257), (1, 64)])
def test_pack_host_equals_device(ex, fmt, rows, cols):
    """4200 x 1100 f32 is 18.5 MB: two staging chunks."""
    print("pack host", fmt, rows, cols, flush=True)
    src = oracle.RNG(rows + cols).fill_normal(rows * cols, 0.05).reshape(rows, cols)
    for dt, data in ((srq.SRC_F32, src), (srq.SRC_BF16, bf16_words(src)), (srq.SRC_F16, src.astype(np.float16).view(np.uint16))):
        v_dev, s_dev = srq.pack(ex, data, fmt, dt, cols=cols)
        v_host, s_host = srq.pack_host(ex, data, fmt, dt, cols=cols)
        assert np.array_equal(v_dev, v_host) and np.array_equal(s_dev.view(np.uint32), s_host.view(np.uint32)), dt


@pytest.mark.parametrize("fmt", [srq.F32, srq.Q8, srq.Q4])
def test_weight_create_host_equals_device(ex, fmt):
    rows, cols = 3000, 2000  # 24 MB of f32: two chunks
    src = oracle.RNG(99).fill_normal(rows * cols, 0.02).reshape(rows, cols)
    a = srq.Weight.create(ex, src, fmt)
    b = srq.Weight.create_host(ex, src, fmt)
    va, sa = a.packed(ex)
    vb, sb = b.packed(ex)
    assert np.array_equal(va, vb) and np.array_equal(sa.view(np.uint32), sb.view(np.uint32))
    x = oracle.RNG(5).fill_normal(3 * cols, 1.0).reshape(3, cols)
    assert np.array_equal(srq.linear(ex, a, x).view(np.uint32), srq.linear(ex, b, x).view(np.uint32))
    a.close()
    b.close()


@pytest.mark.parametrize("name,fmt", [("llama_f32", "q8"), ("qwen2_f32", "q4-mixed"), ("llama3_bf16", "q8")])
def test_model_load_host_equals_device(ex, name, fmt):
    """Every tensor of a fixture loaded from host memory (srq_model_load_host)
    and from an uploaded copy (srq_model_load): identical storage, identical
    logits."""
    fx = hf_fixtures.load(name)
    cfg = gpu_models.fixture_config(fx)
    dt = {"BF16": srq.SRC_BF16, "F16": srq.SRC_F16}.get(fx.dtype, srq.SRC_F32)
    a, b = srq.Model(ex, cfg, fmt), srq.Model(ex, cfg, fmt)
    for nm, arr in fx.w.items():
        kind, layer = gpu_models.kind_of(nm)
        src, d = (fx.raw[nm], dt) if nm in fx.raw else (arr, srq.SRC_F32)
        a.load(kind, layer, src, d)
        b.load_uploaded(kind, layer, src, d)
    kinds = [srq.T_EMBED] + ([] if cfg.tied else [srq.T_OUTPUT])
    for k in kinds:
        assert [x.tobytes() for x in a.weight(k).packed(ex)] == [x.tobytes() for x in b.weight(k).packed(ex)], k
    for layer in range(cfg.layers):
        for k in (srq.T_QKV, srq.T_O, srq.T_GATE_UP, srq.T_DOWN):
            pa, pb = a.weight(k, layer).packed(ex), b.weight(k, layer).packed(ex)
            assert pa[0].tobytes() == pb[0].tobytes() and pa[1].tobytes() == pb[1].tobytes(), (layer, k)
    ids = fx.ids[:12]
    pa, pb = a.pool(4), b.pool(4)
    ca, cb = pa.cache(1), pb.cache(1)
    la, lb = a.step([ca], [ids]), b.step([cb], [ids])
    assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
    for c in (ca, cb):
        c.close()
    a.close()
    b.close()


def test_host_sources_reject_nonfinite_and_cancel(ex):
    rows, cols = 4200, 1100
    src = oracle.RNG(3).fill_normal(rows * cols, 0.05).reshape(rows, cols)
    bad = src.copy()
    bad[4100, 7] = np.inf  # in the second chunk
    with pytest.raises(srq.SrqError) as e:
        srq.pack_host(ex, bad, srq.Q8)
    assert e.value.code == srq.ENONFINITE
    with pytest.raises(srq.SrqError) as e:
        srq.Weight.create_host(ex, bad, srq.Q4)
    assert e.value.code == srq.ENONFINITE
    flag = C.c_int32(1)
    with pytest.raises(srq.SrqError) as e:
        srq.pack_host(ex, src, srq.Q8, cancel=flag)
    assert e.value.code == srq.ECANCELED
    # a canceled model load leaves the tensor unwritten
    fx = hf_fixtures.load("llama_f32")
    m = gpu_models.load_fixture(ex, fx, "q8")
    before = m.weight(srq.T_EMBED).packed(ex)
    with pytest.raises(srq.SrqError) as e:
        m.load(srq.T_EMBED, 0, np.zeros_like(fx.w["embed_tokens"]), cancel=flag)
    assert e.value.code == srq.ECANCELED
    after = m.weight(srq.T_EMBED).packed(ex)
    assert before[0].tobytes() == after[0].tobytes() and before[1].tobytes() == after[1].tobytes()
    nan_norm = np.full(fx.w["norm"].shape, np.nan, np.float32)
    with pytest.raises(srq.SrqError) as e:
        m.load(srq.T_FINAL_NORM, 0, nan_norm)
    assert e.value.code == srq.ENONFINITE
    m.close()


def test_step_cancel_in_flight(ex):
    """A 32-layer model prefills 1024 tokens.  A flag raised from another
    thread shortly after the step starts stops it within about 8-12 layers: the
    call fails with SRQ_ECANCELED well before a full step's time, the cache
    position is unchanged, and the next step on the same cache gives the
    same logits as an uncanceled step."""
    cfg = srq.make_config(2048, 2048, 32, 16, 4, 8192, 1100, 10000.0, 1e-5, True)
    m = syn.build(ex, cfg, "q8", 21)
    pool = m.pool(80)
    prompt = syn.random_prompt(1024, cfg.vocab, 21)
    c0 = pool.cache(33)
    m.step([c0], [prompt])  # warm the workspace and code paths
    c0.close()
    # a full step's time: the median of three, so one slow call on a busy
    # host does not set the bar
    fulls = []
    for _ in range(3):
        c1 = pool.cache(33)
        t0 = time.perf_counter()
        want = m.step([c1], [prompt])
        fulls.append(time.perf_counter() - t0)
        c1.close()
    full = sorted(fulls)[1]
    flag = C.c_int32(0)
    c2 = pool.cache(33)
    delay = full * 0.1

    def raise_flag():
        time.sleep(delay)
        flag.value = 1

    th = threading.Thread(target=raise_flag)
    th.start()
    t0 = time.perf_counter()
    with pytest.raises(srq.SrqError) as e:
        m.step([c2], [prompt], cancel=flag)
    took = time.perf_counter() - t0
    th.join()
    print("full step %.2f ms, canceled after %.2f ms (flag at %.2f ms)" % (full * 1e3, took * 1e3, delay * 1e3),
          flush=True)
    assert e.value.code == srq.ECANCELED
    assert c2.pos == 0
    # layers are enqueued at most eight ahead of the GPU, so the step stops
    # within about 12 layers (of 32) after the flag rises at 10%; 75% leaves room
    # for a loaded host
    assert took < 0.75 * full
    flag.value = 0
    got = m.step([c2], [prompt], cancel=flag)
    assert c2.pos == 1024
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    c2.close()
    m.close()
