"""Host-side archive and config checks (no GPU): srq_archive_check restates
openHFArchiveFormat (monolith.go:648-850) and hf.read_config restates
readHFConfig (monolith.go:253-386).  Cases follow the reference's own
hf_loader_test.go (TestHFRejectTensorCorruption :149-213, TestUniqueJSON
:230-237, TestHFRejectMetadata :112-148, TestHFArchiveAndConversion :80-110)
plus the checks those leave open."""
import ctypes as C
import json
import os
import struct

import numpy as np
import pytest

import sr_go_tranformer_amd as srq
from tests.archives import (TEST_CONFIG, fixture_archive, profile_specs, reference_archive, shard_bytes,
                            write_json, write_shard)
from tests.hf_fixtures import NAMES, load as load_fixture
from sr_go_tranformer_amd import hf

EMBED = "model.embed_tokens.weight"


def check(directory, cfg=None):
    c, _ = hf.read_config(directory) if cfg is None else (cfg, None)
    return hf.check_archive(c, directory)


def expect(directory, code, text):
    with pytest.raises(srq.SrqError) as e:
        check(directory)
    assert e.value.code == code, e.value
    assert text in str(e.value), e.value


@pytest.mark.parametrize("sharded", [False, True])
def test_reference_archive_accepted(tmp_path, sharded):
    header, payload = reference_archive(str(tmp_path), sharded)
    name = "part.safetensors" if sharded else "model.safetensors"
    assert check(str(tmp_path)) == os.path.getsize(tmp_path / name)
    assert len(header) == len(profile_specs(TEST_CONFIG))


@pytest.mark.parametrize("name", NAMES)
@pytest.mark.parametrize("shards", [1, 3])
def test_golden_archives_accepted(tmp_path, name, shards):
    fx = load_fixture(name)
    fixture_archive(str(tmp_path), fx, shards)
    total = sum(os.path.getsize(tmp_path / f) for f in os.listdir(tmp_path) if f.endswith(".safetensors"))
    assert check(str(tmp_path)) == total


CORRUPTIONS = [  # kind, error code, message fragment
    ("missing", srq.EFORMAT, "Safetensors overlapping or unindexed bytes"),  # its bytes stay behind
    ("extra", srq.EFORMAT, 'unexpected or duplicate HF tensor "lm_head.weight"'),
    ("shape", srq.EFORMAT, "HF tensor shape mismatch: model.embed_tokens.weight"),
    ("dtype", srq.EFORMAT, "invalid HF tensor dtype/extent: model.embed_tokens.weight"),
    ("overflow", srq.EFORMAT, "invalid HF tensor dtype/extent"),
    ("overlap", srq.EFORMAT, "Safetensors overlapping or unindexed bytes"),
    ("truncated", srq.EFORMAT, "invalid HF tensor dtype/extent"),
    ("trailing", srq.EFORMAT, "Safetensors trailing/unindexed bytes"),
    ("duplicate", srq.EFORMAT, "duplicate JSON key"),
    ("header bound", srq.EFORMAT, "Safetensors file size/type limit"),  # 8 bytes: below the 10-byte floor
    ("bad shard path", srq.EFORMAT, "unsupported HF shard index name/path"),
    ("wrong shard", srq.EFORMAT, "unexpected or duplicate HF tensor"),
]


@pytest.mark.parametrize("kind,code,text", CORRUPTIONS, ids=[c[0] for c in CORRUPTIONS])
def test_reject_tensor_corruption(tmp_path, kind, code, text):
    """TestHFRejectTensorCorruption (hf_loader_test.go:149-213), the archive
    cases (the NaN case needs the device and is a GPU test)."""
    d = str(tmp_path)
    header, payload = reference_archive(d)
    meta = header[EMBED]
    if kind == "missing":
        del header[EMBED]
    elif kind == "extra":
        header["lm_head.weight"] = meta
    elif kind == "shape":
        meta["shape"] = [(1 << 63) - 1, 8]
    elif kind == "dtype":
        meta["dtype"] = "I32"
    elif kind == "overflow":
        meta["data_offsets"] = [0, (1 << 63) - 1]
    elif kind == "overlap":
        meta["data_offsets"] = [1, 258 * 8 * 4 + 1]
    elif kind == "truncated":
        payload = payload[:-1]
    elif kind == "trailing":
        payload = payload + b"\0"
    elif kind in ("bad shard path", "wrong shard"):
        index = {k: "model.safetensors" for k in header}
        if kind == "bad shard path":
            index[EMBED] = "../model.safetensors"
        else:
            index[EMBED] = "other.safetensors"
            write_shard(os.path.join(d, "other.safetensors"), {})
        write_json(os.path.join(d, "model.safetensors.index.json"), {"weight_map": index})
    path = os.path.join(d, "model.safetensors")
    write_shard(path, header, payload)
    if kind == "header bound":
        with open(path, "wb") as f:
            f.write(struct.pack("<Q", (1 << 64) - 1))
    if kind == "duplicate":
        with open(path, "wb") as f:
            f.write(shard_bytes(b'{"x":{},"x":{}}'))
    if kind == "truncated":
        # the embed tensor's extent still fits; the last tensor's does not
        text = "invalid HF tensor dtype/extent: model.norm.weight"
    expect(d, code, text)


@pytest.mark.parametrize("doc,text", [
    (b'{"a":1,"a":2}', "duplicate JSON key"),
    (b'{"a":{"b":1,"b":2}}', "duplicate JSON key"),
    (b'{} {}', "trailing JSON data"),
    (b'{"x":', "unexpected end of JSON"),
    (b'{"x":' + b"[" * 33 + b"]" * 33 + b"}", "JSON complexity limit"),
    (b'{"\xff":1}', "invalid JSON UTF-8"),
    (b'{"\xed\xa0\x80":1}', "invalid JSON UTF-8"),          # encoded surrogate
    (b'{"\xc0\xaf":1}', "invalid JSON UTF-8"),              # overlong '/'
    (b'{"\\u0061":1,"a":2}', "duplicate JSON key"),         # keys compare unescaped
    (b'{"x":NaN}', "invalid JSON"),
    (b'{"x":01}', "invalid JSON"),
    (b'{"x":"\x01"}', "control character"),
    (b'{"x":[1,]}', "invalid JSON"),
    (b'[]', "header must start with object"),
])
def test_header_json_rules(tmp_path, doc, text):
    """TestUniqueJSON (hf_loader_test.go:230-237) and the RFC 8259 grammar,
    through a shard header."""
    d = str(tmp_path)
    reference_archive(d)
    with open(os.path.join(d, "model.safetensors"), "wb") as f:
        f.write(shard_bytes(doc))
    expect(d, srq.EFORMAT, text)


def test_header_depth_32_accepted_as_json(tmp_path):
    """Nesting of exactly 32 levels under the root passes the JSON rules (the
    archive is then rejected for its content, not its depth)."""
    d = str(tmp_path)
    reference_archive(d)
    doc = b'{"x":' + b"[" * 31 + b"]" * 31 + b"}"
    with open(os.path.join(d, "model.safetensors"), "wb") as f:
        f.write(shard_bytes(doc))
    expect(d, srq.EFORMAT, 'unexpected or duplicate HF tensor "x"')


@pytest.mark.parametrize("edit,text", [
    (lambda h: h.__setitem__("__metadata__", {"format": 1}), "__metadata__ must map strings to strings"),
    (lambda h: h[EMBED].__setitem__("extra", 1), 'unknown field "extra"'),
    (lambda h: h[EMBED].__setitem__("shape", [258.0, 8]), "shape is not a list of integers"),
    (lambda h: h[EMBED].__setitem__("data_offsets", [0, 8256.0]), "data_offsets is not a list of integers"),
    (lambda h: h[EMBED].__setitem__("dtype", 4), "dtype is not a string"),
    (lambda h: h[EMBED].__setitem__("data_offsets", [0]), "invalid HF tensor dtype/extent"),
    (lambda h: h[EMBED].__setitem__("shape", [258, 8, 1]), "HF tensor shape mismatch"),
])
def test_header_entry_decoding(tmp_path, edit, text):
    """json.Decoder with DisallowUnknownFields into {dtype, shape,
    data_offsets} (monolith.go:790-794), and the metadata map."""
    d = str(tmp_path)
    header, payload = reference_archive(d)
    edit(header)
    write_shard(os.path.join(d, "model.safetensors"), header, payload)
    expect(d, srq.EFORMAT, text)


def test_header_field_names_fold_case(tmp_path):
    """encoding/json matches field names case-insensitively (and through the
    long-s fold): such a header is accepted, as the reference accepts it."""
    d = str(tmp_path)
    header, payload = reference_archive(d)
    m = header.pop(EMBED)
    header[EMBED] = {"DType": m["dtype"], "ſhape": m["shape"], "DATA_OFFSETS": m["data_offsets"]}
    header["__metadata__"] = {"format": "pt", "note": None}
    write_shard(os.path.join(d, "model.safetensors"), header, payload)
    assert check(d) > 0


def test_index_rules(tmp_path):
    d = str(tmp_path)
    header, payload = reference_archive(d, sharded=True)
    idx = os.path.join(d, "model.safetensors.index.json")
    index = {k: "part.safetensors" for k in header}
    # one entry short
    short = dict(index)
    short.pop(EMBED)
    write_json(idx, {"weight_map": short})
    expect(d, srq.EFORMAT, "HF shard index tensor count mismatch")
    # no weight_map at all
    write_json(idx, {"metadata": {}})
    expect(d, srq.EFORMAT, "HF shard index tensor count mismatch")
    # a file name without the suffix, with a backslash, empty
    for bad in ("part.bin", "a\\part.safetensors", ""):
        write_json(idx, {"weight_map": dict(index, **{EMBED: bad})})
        expect(d, srq.EFORMAT, "unsupported HF shard index name/path")
    # a name outside the profile
    other = dict(index)
    other.pop(EMBED)
    other["model.embed.weight"] = "part.safetensors"
    write_json(idx, {"weight_map": other})
    expect(d, srq.EFORMAT, "unsupported HF shard index name/path")
    # an index naming a shard that does not exist
    write_json(idx, {"weight_map": dict(index, **{EMBED: "gone.safetensors"})})
    expect(d, srq.EFILE, "gone.safetensors")
    # duplicate keys in the index
    with open(idx, "w") as f:
        f.write('{"weight_map": {"a": "x.safetensors", "a": "y.safetensors"}}')
    expect(d, srq.EFORMAT, "duplicate JSON key")
    # weight_map under another capitalisation decodes into the same field
    write_json(idx, {"Weight_Map": index})
    assert check(d) == os.path.getsize(os.path.join(d, "part.safetensors"))
    # more than 128 shards
    cfg = dict(TEST_CONFIG, num_hidden_layers=16)
    write_json(os.path.join(d, "config.json"), cfg)
    names = [n for n, _ in profile_specs(cfg)]
    assert len(names) > 128
    write_json(idx, {"weight_map": {n: "s%03d.safetensors" % i for i, n in enumerate(names)}})
    expect(d, srq.EFORMAT, "HF shard count limit")


def test_file_limits(tmp_path):
    d = str(tmp_path)
    header, payload = reference_archive(d)
    path = os.path.join(d, "model.safetensors")
    with open(path, "wb") as f:
        f.write(b"\x02\0\0\0\0\0\0\0{}")  # 10 bytes: smallest accepted size, empty header
    expect(d, srq.EFORMAT, "missing HF tensor")
    with open(path, "wb") as f:
        f.write(b"\x01\0\0\0\0\0\0\0{")
    expect(d, srq.EFORMAT, "Safetensors file size/type limit")
    for n in ((1 << 64) - 1, 1, (4 << 20) + 1, 3):  # beyond the limits, below 2, beyond the file
        with open(path, "wb") as f:
            f.write(struct.pack("<Q", n) + b"{}")
        expect(d, srq.EFORMAT, "Safetensors header length limit")
    # larger than every parameter at 4 bytes plus the header limit
    params = sum(int(np.prod(s)) for _, s in profile_specs(TEST_CONFIG))
    write_shard(path, header, payload + b"\0" * (params * 4 + (4 << 20) + 8 - len(payload)))
    expect(d, srq.EFORMAT, "Safetensors file size/type limit")
    os.remove(path)
    expect(d, srq.EFILE, "model.safetensors")
    os.mkdir(path)
    expect(d, srq.EFORMAT, "Safetensors file size/type limit")


def test_profile_tensors_follow_config(tmp_path):
    """Qwen2 requires the q/k/v biases, an untied config requires lm_head
    (hfProfileSpecs monolith.go:426-440)."""
    d = str(tmp_path)
    qwen = dict(TEST_CONFIG, architectures=["Qwen2ForCausalLM"], model_type="qwen2")
    reference_archive(d, cfg=qwen)
    assert check(d) > 0
    reference_archive(d)  # a Llama archive (no biases) under the Qwen2 config
    write_json(os.path.join(d, "config.json"), qwen)
    expect(d, srq.EFORMAT, 'missing HF tensor "model.layers.0.self_attn.q_proj.bias"')
    untied = dict(TEST_CONFIG, tie_word_embeddings=False)
    write_json(os.path.join(d, "config.json"), untied)
    expect(d, srq.EFORMAT, 'missing HF tensor "lm_head.weight"')
    reference_archive(d, cfg=untied)
    assert check(d) > 0


# ------------------------------------------------------------ config.json
@pytest.mark.parametrize("name", NAMES)
def test_golden_configs_read(tmp_path, name):
    """Every committed Transformers fixture's config reads to the model
    configuration the GPU tests build for it."""
    fx = load_fixture(name)
    write_json(os.path.join(str(tmp_path), "config.json"), fx.cfg)
    cfg, prof = hf.read_config(str(tmp_path))
    assert (cfg.vocab, cfg.dim, cfg.layers, cfg.heads, cfg.kv_heads, cfg.hidden) == \
        (fx.vocab, fx.dim, fx.layers, fx.heads, fx.kv_heads, fx.hidden)
    assert cfg.context == min(fx.context, 2048)
    assert (cfg.rope_theta, cfg.norm_eps, bool(cfg.tied)) == (fx.theta, fx.eps, fx.tied)
    assert bool(cfg.qkv_bias) == any(k.endswith("_bias") for k in fx.w)
    assert bool(cfg.rope_llama3) == bool(fx.llama3)
    assert prof.bos == fx.cfg["bos_token_id"]


REJECT = [  # TestHFRejectMetadata (hf_loader_test.go:112-148)
    ("architecture", lambda c: c.__setitem__("model_type", "qwen2")),
    ("bias", lambda c: c.__setitem__("attention_bias", True)),
    ("scaled rope", lambda c: c.__setitem__("rope_scaling", {"type": "linear", "factor": 2})),
    ("head dimension mismatch", lambda c: c.__setitem__("head_dim", 8)),
    ("bad dim", lambda c: c.__setitem__("hidden_size", (1 << 63) - 1)),
    ("bad special", lambda c: c.__setitem__("eos_token_id", None)),
    ("missing special", lambda c: c.pop("bos_token_id")),
    # and the rules those leave open
    ("unknown field", lambda c: c.__setitem__("rope_type", "default")),
    ("float int", lambda c: c.__setitem__("hidden_size", 8.0)),
    ("duplicate eos", lambda c: c.__setitem__("eos_token_id", [2, 2])),
    ("eos list off llama", lambda c: c.update(model_type="qwen2", architectures=["Qwen2ForCausalLM"],
                                               eos_token_id=[2, 3])),
    ("mistral sliding", lambda c: c.update(model_type="mistral", architectures=["MistralForCausalLM"])),
    ("gelu", lambda c: c.__setitem__("hidden_act", "gelu")),
    ("odd head dim", lambda c: c.update(hidden_size=6, num_attention_heads=2)),
    ("kv heads", lambda c: c.__setitem__("num_key_value_heads", 3)),
    ("theta", lambda c: c.__setitem__("rope_theta", 1)),
    ("layer types", lambda c: c.update(model_type="qwen2", architectures=["Qwen2ForCausalLM"],
                                       layer_types=["full_attention", "sliding_attention"])),
    ("llama3 rope fields", lambda c: c.__setitem__("rope_scaling", {"rope_type": "llama3", "factor": 8.0})),
    ("llama3 rope original", lambda c: c.__setitem__("rope_scaling", {
        "rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
        "original_max_position_embeddings": 65})),
]


@pytest.mark.parametrize("case,change", REJECT, ids=[r[0] for r in REJECT])
def test_reject_config(tmp_path, case, change):
    c = json.loads(json.dumps(TEST_CONFIG))
    change(c)
    write_json(os.path.join(str(tmp_path), "config.json"), c)
    with pytest.raises(hf.HFError):
        hf.read_config(str(tmp_path))


def test_config_context_and_eos_list(tmp_path):
    d = str(tmp_path)
    c = dict(TEST_CONFIG, eos_token_id=[2, 7, 9])
    write_json(os.path.join(d, "config.json"), c)
    cfg, prof = hf.read_config(d, 32)
    assert cfg.context == 32 and prof.eos == 2 and prof.extra_eos == [7, 9]
    assert prof.is_eos(9) and not prof.is_eos(3)
    with pytest.raises(hf.HFError):
        hf.read_config(d, 65)  # beyond max_position_embeddings (the reference's context bound case)
    ok = dict(TEST_CONFIG, rope_scaling={"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0,
                                         "high_freq_factor": 4.0, "original_max_position_embeddings": 32})
    write_json(os.path.join(d, "config.json"), ok)
    cfg, _ = hf.read_config(d)
    assert cfg.rope_llama3 == 1 and cfg.rope_original == 32 and cfg.rope_factor == 8.0


@pytest.mark.parametrize("seed", range(4))
def test_random_header_corruption_fails_cleanly(tmp_path, seed):
    """Archive headers come from untrusted files: random byte edits,
    truncations and insertions of the reference archive's header (and of its
    8-byte length field and the index) each return SRQ_OK or one of the
    archive error codes, never anything else.  Run under the
    host-sanitized library (tests/test_sanitized_cpu.py), this also checks
    the parser never reads or writes out of bounds."""
    d = str(tmp_path)
    header, payload = reference_archive(d, sharded=True)
    path = os.path.join(d, "part.safetensors")
    index = os.path.join(d, "model.safetensors.index.json")
    raw = shard_bytes(header, payload)
    raw_index = open(index, "rb").read()
    hlen = struct.unpack("<Q", raw[:8])[0]
    rng = np.random.default_rng(seed)
    codes = {srq.OK, srq.EFORMAT, srq.EFILE, srq.EINVAL}
    for trial in range(60):
        buf = bytearray(raw)
        idx = bytearray(raw_index)
        kind = trial % 5
        if kind == 0:  # flip bytes of the JSON header
            for p in rng.integers(8, 8 + hlen, size=int(rng.integers(1, 6))):
                buf[p] = int(rng.integers(0, 256))
        elif kind == 1:  # cut the file short
            del buf[int(rng.integers(0, 8 + hlen + 64)):]
        elif kind == 2:  # insert bytes into the header
            p = int(rng.integers(8, 8 + hlen))
            buf[p:p] = bytes(rng.integers(0, 256, size=int(rng.integers(1, 40)), dtype=np.uint8))
        elif kind == 3:  # a wrong header length
            lengths = [0, 1, hlen - 1, hlen + 1, 1 << 40, (1 << 64) - 1]
            buf[:8] = struct.pack("<Q", lengths[int(rng.integers(0, len(lengths)))])
        else:  # corrupt the shard index instead
            for p in rng.integers(0, len(idx), size=int(rng.integers(1, 6))):
                idx[p] = int(rng.integers(0, 256))
        with open(path, "wb") as f:
            f.write(bytes(buf))
        with open(index, "wb") as f:
            f.write(bytes(idx))
        size = C.c_int64()
        cfg, _ = hf.read_config(d)
        rc = srq.lib().srq_archive_check(C.byref(cfg), os.fsencode(d), C.byref(size))
        assert rc in codes, (seed, trial, kind, rc)
