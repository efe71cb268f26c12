"""Pin the oracle's step (RMSNorm, half-split RoPE with the reference's FP32
tables, paged KV, attention, SwiGLU, selective head) against the
reference's own Transformers fixtures (hf_inference_test.go:32-124, tol
2e-5) and its quantized forward against the FP32 forward on
copyRow-reconstructed weights (q8_test.go:241-274, tol 3e-5)."""
import json
import os

import numpy as np
import pytest

import oracle
from tests import hf_fixtures

FIXTURES = hf_fixtures.NAMES


def near(got, want, tol):
    got = np.asarray(got)
    assert np.all(np.isfinite(got))
    err = np.abs(got.astype(np.float64) - np.asarray(want, np.float64))
    assert err.max() <= tol, (err.max(), int(err.argmax()))


@pytest.mark.parametrize("name", FIXTURES)
@pytest.mark.parametrize("chunk", [1, 4, 16, 35])
def test_fp32_forward_matches_transformers(name, chunk):
    fx = hf_fixtures.load(name)
    m = fx.oracle_model("f32")
    cache = m.new_cache()
    for lo in range(0, 35, chunk):
        hi = min(lo + chunk, 35)
        got = m.step([cache], [fx.ids[lo:hi]], workers=2)[0]
        near(got, fx.logits[hi - 1], 2e-5)
    for pos in range(35, len(fx.ids)):
        got = m.step([cache], [[fx.ids[pos]]])[0]
        near(got, fx.logits[pos], 2e-5)
    for layer in range(fx.layers):
        for pos in range(len(fx.ids)):
            near(cache.row(layer, pos, 0), fx.k[layer, pos], 2e-5)
            near(cache.row(layer, pos, 1), fx.v[layer, pos], 2e-5)


@pytest.mark.parametrize("name", ["llama_f32", "mistral_f32", "qwen2_f32"])
def test_ragged_sessions(name):
    fx = hf_fixtures.load(name)
    m = fx.oracle_model("f32")
    ca, cb = m.new_cache(), m.new_cache()
    got = m.step([ca, cb], [fx.ids[:35], fx.ids[:4]])
    near(got[0], fx.logits[34], 2e-5)
    near(got[1], fx.logits[3], 2e-5)
    got = m.step([ca, cb], [[fx.ids[35]], [fx.ids[4]]])
    near(got[0], fx.logits[35], 2e-5)
    near(got[1], fx.logits[4], 2e-5)
    # selective head: unselected rows are zeroed, selected rows unchanged
    cc, cd = m.new_cache(), m.new_cache()
    sel = m.step([cc, cd], [fx.ids[:35], fx.ids[:4]], want=[False, True])
    assert np.all(sel[0] == 0)
    near(sel[1], fx.logits[3], 2e-5)


@pytest.mark.parametrize("name", ["llama_f32", "llama_untied-f32", "llama3_f32", "llama3_f16", "mistral_f32",
                                  "mistral_f16", "qwen2_f32", "qwen2_f16", "qwen2_untied-bf16"])
@pytest.mark.parametrize("fmt", ["q8", "q4", "q4-mixed"])
def test_quantized_forward_equals_reconstructed_dense(name, fmt):
    fx = hf_fixtures.load(name)
    qm = fx.oracle_model(fmt)
    recon = {}
    for key, w in qm.weights.items():
        recon[key] = w.dequant() if w.fmt != oracle.F32 else w.values.reshape(-1) if w.rows == 1 else w.values
    dm = fx.oracle_model("f32", dense_override=recon)
    for chunks in ([33, 1, 2, 1],):
        cq, cd = qm.new_cache(), dm.new_cache()
        lo = 0
        for c in chunks:
            a = qm.step([cq], [fx.ids[lo:lo + c]])[0]
            b = dm.step([cd], [fx.ids[lo:lo + c]])[0]
            near(a, b, 3e-5)
            lo += c


def test_llama3_frequency_oracle():
    """testdata/hf-llama3/frequencies.json: Transformers' FP32 inverse
    frequencies, including the narrow-band rounding regression, at the
    reference's own bound of 2e-7 relative (hf_llama3_test.go:159-163)."""
    path = os.path.join(hf_fixtures.GOLDEN, "llama3_frequencies.json")
    cases = json.load(open(path))
    assert len(cases) >= 2
    for case in cases:
        s = case.get("scaling")
        cfg = oracle.make_config(8, case["head_dim"], 1, 1, 1, 8, 8, case["theta"], 1e-5, True, s)
        for j, want in enumerate(case["inverse_frequencies"]):
            got = oracle.inverse_frequency(case["theta"], case["head_dim"], j, cfg)
            assert np.isfinite(got)
            assert abs(float(np.float32(got)) - float(np.float32(want))) <= 2e-7 * max(1e-12, abs(want)), \
                (case["theta"], j, got, want)


def test_greedy_tie_rule_and_nonfinite():
    logits = np.array([0.5, 2.0, 2.0, -1.0], np.float32)
    assert oracle.argmax(logits) == 1
    assert oracle.argmax(np.array([-0.0, 0.0], np.float32)) == 0
    assert oracle.argmax(np.array([1.0, np.nan], np.float32)) == -1
    assert oracle.argmax(np.array([np.inf, 1.0], np.float32)) == -1


def test_step_validation_errors():
    fx = hf_fixtures.load("llama_f32")
    m = fx.oracle_model("f32")
    c = m.new_cache()
    with pytest.raises(RuntimeError):
        m.step([c], [[fx.vocab]])  # token outside vocabulary
    with pytest.raises(RuntimeError):
        m.step([c, c], [[1], [2]])  # duplicate cache
    with pytest.raises(RuntimeError):
        m.step([c], [list(range(1, 130))])  # context exhausted (128)
    assert c.pos == 0  # failed calls never commit positions
