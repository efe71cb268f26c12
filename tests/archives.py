"""Writers of Transformers safetensors archives for the loader tests: the
reference's own synthetic archive recipe (hfFixture, hf_loader_test.go:44-79)
and the committed golden fixtures re-serialised (single file or sharded)."""
import json
import os
import struct

import numpy as np

ATTN = ("q_proj", "k_proj", "v_proj", "o_proj")
MLP = ("gate_proj", "up_proj", "down_proj")

# hfTestConfig (hf_loader_test.go:14-16).
TEST_CONFIG = {"architectures": ["LlamaForCausalLM"], "model_type": "llama", "vocab_size": 258, "hidden_size": 8,
               "intermediate_size": 12, "num_hidden_layers": 2, "num_attention_heads": 2, "num_key_value_heads": 1,
               "max_position_embeddings": 64, "rope_theta": 10000, "rms_norm_eps": 1e-5, "hidden_act": "silu",
               "tie_word_embeddings": True, "bos_token_id": 1, "eos_token_id": 2}


def profile_specs(cfg):
    """hfProfileSpecs (monolith.go:407-440): names and shapes in order."""
    d, h, layers = cfg["hidden_size"], cfg["intermediate_size"], cfg["num_hidden_layers"]
    kd = d // cfg["num_attention_heads"] * cfg.get("num_key_value_heads", cfg["num_attention_heads"])
    out = [("model.embed_tokens.weight", [cfg["vocab_size"], d])]
    for i in range(layers):
        p = "model.layers.%d." % i
        out += [(p + "input_layernorm.weight", [d]), (p + "self_attn.q_proj.weight", [d, d]),
                (p + "self_attn.k_proj.weight", [kd, d]), (p + "self_attn.v_proj.weight", [kd, d]),
                (p + "self_attn.o_proj.weight", [d, d]), (p + "post_attention_layernorm.weight", [d]),
                (p + "mlp.gate_proj.weight", [h, d]), (p + "mlp.up_proj.weight", [h, d]),
                (p + "mlp.down_proj.weight", [d, h])]
    out.append(("model.norm.weight", [d]))
    if cfg.get("model_type") == "qwen2":
        for i in range(layers):
            p = "model.layers.%d.self_attn." % i
            out += [(p + "q_proj.bias", [d]), (p + "k_proj.bias", [kd]), (p + "v_proj.bias", [kd])]
    if not cfg.get("tie_word_embeddings", False):
        out.append(("lm_head.weight", [cfg["vocab_size"], d]))
    return out


def shard_bytes(header, payload=b""):
    """8-byte little-endian header length, the header JSON, the payload."""
    hb = header if isinstance(header, bytes) else json.dumps(header).encode()
    return struct.pack("<Q", len(hb)) + hb + payload


def write_shard(path, header, payload=b""):
    with open(path, "wb") as f:
        f.write(shard_bytes(header, payload))


def write_json(path, value):
    with open(path, "w") as f:
        json.dump(value, f)


def reference_archive(directory, sharded=False, cfg=None):
    """The reference's hfFixture: every tensor of the profile filled with
    1.5, dtypes cycling F32, F16, BF16 by spec index.  Returns (header,
    payload) of the single shard."""
    cfg = dict(cfg or TEST_CONFIG)
    write_json(os.path.join(directory, "config.json"), cfg)
    header, payload, index = {}, bytearray(), {}
    words = {"F32": struct.pack("<f", 1.5), "F16": struct.pack("<H", 0x3E00), "BF16": struct.pack("<H", 0x3FC0)}
    for i, (name, shape) in enumerate(profile_specs(cfg)):
        dtype = ("F32", "F16", "BF16")[i % 3]
        start = len(payload)
        payload += words[dtype] * int(np.prod(shape))
        header[name] = {"dtype": dtype, "shape": shape, "data_offsets": [start, len(payload)]}
        index[name] = "part.safetensors"
    name = "model.safetensors"
    if sharded:
        name = "part.safetensors"
        write_json(os.path.join(directory, "model.safetensors.index.json"), {"weight_map": index})
    write_shard(os.path.join(directory, name), header, bytes(payload))
    return header, bytes(payload)


def hf_name(key):
    """Fixture key (tests/golden/make_golden.py) -> Transformers name."""
    if key == "embed_tokens":
        return "model.embed_tokens.weight"
    if key == "norm":
        return "model.norm.weight"
    if key == "lm_head":
        return "lm_head.weight"
    _, layer, nm = key.split(".")
    p = "model.layers.%s." % layer
    if nm in ("q_bias", "k_bias", "v_bias"):
        return p + "self_attn.%s_proj.bias" % nm[0]
    if nm in ATTN:
        return p + "self_attn.%s.weight" % nm
    if nm in MLP:
        return p + "mlp.%s.weight" % nm
    return p + nm + ".weight"


def fixture_archive(directory, fx, shards=1, metadata=True):
    """Write config.json and the fixture's tensors as safetensors: the
    source dtype's own bytes (F16/BF16 words, F32 values), split into
    `shards` files with an index when shards > 1."""
    write_json(os.path.join(directory, "config.json"), fx.cfg)
    tensors = []
    for key in sorted(fx.w):
        if key in fx.raw:
            data = np.ascontiguousarray(fx.raw[key], "<u2").tobytes()
            dtype = fx.dtype
        else:
            data = np.ascontiguousarray(fx.w[key], "<f4").tobytes()
            dtype = "F32"
        tensors.append((hf_name(key), dtype, list(fx.w[key].shape), data))
    groups = [tensors[i::shards] for i in range(shards)]
    files = ["model.safetensors"] if shards == 1 else \
        ["model-%05d-of-%05d.safetensors" % (i + 1, shards) for i in range(shards)]
    index = {}
    for fname, group in zip(files, groups):
        header, payload = {}, bytearray()
        if metadata:
            header["__metadata__"] = {"format": "pt"}
        for name, dtype, shape, data in group:
            header[name] = {"dtype": dtype, "shape": shape, "data_offsets": [len(payload), len(payload) + len(data)]}
            payload += data
            index[name] = fname
        write_shard(os.path.join(directory, fname), header, bytes(payload))
    if shards > 1:
        write_json(os.path.join(directory, "model.safetensors.index.json"),
                   {"metadata": {"total_size": sum(len(t[3]) for t in tensors)}, "weight_map": index})
