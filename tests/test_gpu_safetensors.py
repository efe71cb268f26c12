"""GPU loading of Transformers archives (srq_model_load_safetensors:
openHFArchiveFormat + readParam, monolith.go:648-920) through the C ABI.

Bars: a model loaded from an archive holds bit-identical packed weights and
gives bit-identical step logits to the same model loaded tensor by tensor
from the fixture's source words (itself pinned to Transformers and the
oracle by test_gpu_model.py); FP32 models also match Transformers' logits at
the reference's 2e-5 (hf_inference_test.go:74).  Failure cases follow
TestHFRejectTensorCorruption's NaN case and TestHFArchiveAndConversion's
cancellation (hf_loader_test.go:80-213)."""
import ctypes as C
import os
import struct

import numpy as np
import pytest

import sr_go_tranformer_amd as srq
from sr_go_tranformer_amd import hf
from tests import archives, gpu_models, hf_fixtures

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ex():
    e = srq.Executor(0)
    yield e
    e.close()


def matrices(cfg):
    out = [(srq.T_EMBED, 0)] + ([] if cfg.tied else [(srq.T_OUTPUT, 0)])
    for layer in range(cfg.layers):
        out += [(k, layer) for k in (srq.T_QKV, srq.T_O, srq.T_GATE_UP, srq.T_DOWN)]
    return out


def logits_of(m, ids):
    cache = m.pool(8).cache(4)
    out = [m.step([cache], [ids[:33]])[0]]
    for t in ids[33:]:
        out.append(m.step([cache], [[t]])[0])
    return np.stack(out)


@pytest.mark.parametrize("name", hf_fixtures.NAMES)
@pytest.mark.parametrize("fmt,shards", [("f32", 1), ("q8", 3), ("q4-mixed", 2)])
def test_archive_matches_tensor_loads(ex, tmp_path, name, fmt, shards):
    print("archive", name, fmt, shards, flush=True)
    fx = hf_fixtures.load(name)
    d = str(tmp_path)
    archives.fixture_archive(d, fx, shards)
    m, prof = hf.open_model(ex, d, fmt)
    ref = gpu_models.load_fixture(ex, fx, fmt, use_raw=True)
    for kind, layer in matrices(m.config):
        a, b = m.weight(kind, layer).packed(ex), ref.weight(kind, layer).packed(ex)
        assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1]), (kind, layer)
    got, want = logits_of(m, fx.ids), logits_of(ref, fx.ids)
    assert np.array_equal(got, want)
    if fmt == "f32":
        assert np.abs(got - fx.logits[32:]).max() <= 2e-5
    assert prof.bos == fx.cfg["bos_token_id"]
    m.close()
    ref.close()


def test_reference_archive_values(ex, tmp_path):
    """TestHFArchiveAndConversion: mixed F32 / F16 / BF16 tensors of 1.5
    load as 1.5 (F32 storage) and as Q8 code 127 with scale 1.5/127."""
    d = str(tmp_path)
    archives.reference_archive(d, sharded=True)
    cfg, _ = hf.read_config(d)
    for fmt in ("f32", "q8"):
        m = srq.Model(ex, cfg, fmt)
        size = m.load_safetensors(d)
        assert size == os.path.getsize(os.path.join(d, "part.safetensors"))
        for kind, layer in matrices(cfg):
            vals, scl = m.weight(kind, layer).packed(ex)
            if fmt == "f32":
                assert np.all(vals.view(np.float32) == np.float32(1.5))
            else:
                assert np.all(vals.view(np.int8) == 127)
                assert np.all(scl == np.float32(1.5 / 127))  # q8Scale: f32 of the f64 quotient
        m.close()


@pytest.mark.parametrize("dtype_index", [0, 1, 2])
def test_nonfinite_names_tensor_and_executor_recovers(ex, tmp_path, dtype_index):
    """The NaN case of TestHFRejectTensorCorruption, per source dtype: the
    load fails with SRQ_ENONFINITE naming the tensor; the executor's error
    word is left clear, so a clean load afterwards succeeds."""
    d = str(tmp_path)
    header, payload = archives.reference_archive(d)
    specs = archives.profile_specs(archives.TEST_CONFIG)
    name = specs[dtype_index][0]  # F32, F16, BF16 by spec index
    meta = header[name]
    bad = bytearray(payload)
    o = meta["data_offsets"][0]
    word = {"F32": struct.pack("<f", float("nan")), "F16": struct.pack("<H", 0x7C00),
            "BF16": struct.pack("<H", 0xFF80)}[meta["dtype"]]
    bad[o + len(word) * 3:o + len(word) * 4] = word
    archives.write_shard(os.path.join(d, "model.safetensors"), header, bytes(bad))
    cfg, _ = hf.read_config(d)
    m = srq.Model(ex, cfg, "q8")
    with pytest.raises(srq.SrqError) as e:
        m.load_safetensors(d)
    assert e.value.code == srq.ENONFINITE
    assert "non-finite HF weight in " + name in str(e.value)
    archives.write_shard(os.path.join(d, "model.safetensors"), header, payload)
    m.load_safetensors(d)
    m.close()


def test_cancel_and_validation_before_writes(ex, tmp_path):
    d = str(tmp_path)
    header, payload = archives.reference_archive(d)
    cfg, _ = hf.read_config(d)
    m = srq.Model(ex, cfg, "f32")
    flag = C.c_int32(1)
    with pytest.raises(srq.SrqError) as e:
        m.load_safetensors(d, cancel=flag)
    assert e.value.code == srq.ECANCELED
    m.load_safetensors(d)
    before = m.weight(srq.T_EMBED).packed(ex)[0].copy()
    # A corrupt archive is rejected before any weight is written.
    header2 = dict(header)
    header2["model.norm.weight"] = dict(header["model.norm.weight"], dtype="I8")
    archives.write_shard(os.path.join(d, "model.safetensors"), header2, payload)
    with pytest.raises(srq.SrqError) as e:
        m.load_safetensors(d)
    assert e.value.code == srq.EFORMAT
    assert np.array_equal(m.weight(srq.T_EMBED).packed(ex)[0], before)
    m.close()
