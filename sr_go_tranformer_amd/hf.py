"""Transformers model directories: config.json and the safetensors archive.

read_config restates readHFConfig (cmd/monolith/monolith.go:253-386) for the
Llama / Qwen2 / full-attention Mistral profiles: the same allowed fields,
typed decoding, profile checks, EOS lists, Llama 3 RoPE scaling, context cap
and shape limits (Config.validateShapeLimits M:100-114).  The archive itself
is checked and loaded by the native library (srq_archive_check,
srq_model_load_safetensors: openHFArchiveFormat M:648-850).
"""
import ctypes as C
import json
import math
import os
from dataclasses import dataclass, field

import numpy as np

from . import Model, check, lib, make_config

MAX_CONFIG_BYTES = 1 << 20       # readHFConfig's readBoundedJSON limit (M:255)
BASE_VOCAB = 258                 # baseVocab (M:46)
MAX_HF_VOCAB = 262144            # maxHFVocab (M:49)
MAX_HF_PARAMETERS = 8_000_000_000  # maxHFParameters (M:48)
INT64 = (-(1 << 63), (1 << 63) - 1)

ALLOWED = ("architectures model_type vocab_size hidden_size intermediate_size num_hidden_layers "
           "num_attention_heads num_key_value_heads max_position_embeddings rope_theta rms_norm_eps hidden_act "
           "tie_word_embeddings attention_bias mlp_bias rope_interleaved attention_dropout pretraining_tp "
           "bos_token_id eos_token_id pad_token_id initializer_range is_llama_config torch_dtype dtype "
           "transformers_version transformers.js_config use_cache _name_or_path _attn_implementation").split()
EXTRA = {"qwen2": "use_sliding_window sliding_window max_window_layers layer_types".split(),
         "llama": ["head_dim", "rope_scaling"], "mistral": ["head_dim", "sliding_window"]}
ARCH = {"llama": "LlamaForCausalLM", "qwen2": "Qwen2ForCausalLM", "mistral": "MistralForCausalLM"}
ROPE_FIELDS = ("rope_type", "factor", "low_freq_factor", "high_freq_factor", "original_max_position_embeddings")


class HFError(ValueError):
    """A config.json the profile does not accept."""


@dataclass
class HFProfile:
    model_type: str
    bos: int
    eos: int
    extra_eos: list = field(default_factory=list)
    context: int = 0          # the model's max_position_embeddings

    def is_eos(self, token):
        """hfConfig.isEOS (M:162-172)."""
        return token == self.eos or token in self.extra_eos


def unique_json(data):
    """uniqueJSON (M:176-228): strict UTF-8, no duplicate keys at any level,
    nesting at most 32 deep, at most 2e6 values, one document."""
    try:
        text = data.decode("utf-8")
    except UnicodeDecodeError:
        raise HFError("invalid JSON UTF-8")

    def pairs(items):
        seen = set()
        for k, _ in items:
            if k in seen:
                raise HFError("duplicate/invalid JSON key %r" % k)
            seen.add(k)
        return dict(items)

    def constant(name):
        raise HFError("invalid JSON literal %s" % name)

    try:
        value = json.loads(text, object_pairs_hook=pairs, parse_constant=constant)
    except json.JSONDecodeError as e:
        raise HFError("invalid JSON: %s" % e)
    nodes = 0
    stack = [(value, 0)]
    while stack:
        v, depth = stack.pop()
        nodes += 1
        if depth > 32 or nodes > 2_000_000:
            raise HFError("JSON complexity limit")
        if isinstance(v, dict):
            stack.extend((x, depth + 1) for x in v.values())
        elif isinstance(v, list):
            stack.extend((x, depth + 1) for x in v)
    return value


def _go_int(v, name):
    """encoding/json into a Go int: an integral JSON number in int64 range
    (null leaves zero)."""
    if v is None:
        return 0
    if isinstance(v, bool) or not isinstance(v, int) or not INT64[0] <= v <= INT64[1]:
        raise HFError("HF config field %s: want an integer" % name)
    return v


def _go_float(v, name):
    if v is None:
        return 0.0
    if isinstance(v, bool) or not isinstance(v, (int, float)):
        raise HFError("HF config field %s: want a number" % name)
    return float(v)


def _go_str(v, name):
    if v is None:
        return ""
    if not isinstance(v, str):
        raise HFError("HF config field %s: want a string" % name)
    return v


def _go_bool(v, name):
    if v is None:
        return False
    if not isinstance(v, bool):
        raise HFError("HF config field %s: want a boolean" % name)
    return v


def _go_strs(v, name):
    if v is None:
        return []
    if not isinstance(v, list):
        raise HFError("HF config field %s: want a list of strings" % name)
    return [_go_str(x, name) for x in v]


def _finite(x):
    return not (math.isinf(x) or math.isnan(x))


def read_config(directory, context_limit=0):
    """(ModelConfig, HFProfile) of a Transformers directory's config.json,
    accepted only for the profiles the engine runs (M:253-386).  The
    context is context_limit when positive, else min(model maximum, 2048)."""
    path = os.path.join(directory, "config.json")
    if not os.path.isfile(path) or os.path.getsize(path) > MAX_CONFIG_BYTES:
        raise HFError("config.json: metadata size/type limit")
    with open(path, "rb") as f:
        raw = unique_json(f.read(MAX_CONFIG_BYTES + 1))
    if not isinstance(raw, dict):
        raise HFError("config.json is not a JSON object")
    if "model_type" not in raw:
        raise HFError("invalid HF model_type")
    model_type = _go_str(raw["model_type"], "model_type")
    if model_type == "gpt2":
        raise HFError("GPT-2 profiles are not part of this engine")
    keys = set(ALLOWED) | set(EXTRA.get(model_type, []))
    if model_type == "mistral" and ("sliding_window" not in raw or raw["sliding_window"] is not None):
        raise HFError("Mistral requires explicit sliding_window:null; sliding attention is not supported")
    for k, v in raw.items():
        if k == "rope_scaling" and v is None:
            continue
        if k not in keys:
            raise HFError("unsupported HF config field %r" % k)
    eos_raw = raw.get("eos_token_id")
    extra_eos = []
    if isinstance(eos_raw, list):
        if model_type != "llama" or not 1 <= len(eos_raw) <= 8:
            raise HFError("Llama eos_token_id requires 1..8 integer IDs")
        seen = set()
        for i, value in enumerate(eos_raw):
            if value is None or isinstance(value, bool) or not isinstance(value, int) or value < 0 \
                    or value > INT64[1] or value in seen:
                raise HFError("Llama eos_token_id contains an invalid or duplicate ID")
            seen.add(value)
            if i > 0:
                extra_eos.append(value)
        eos_raw = eos_raw[0]
    g = raw.get
    architectures = _go_strs(g("architectures"), "architectures")
    head_dim = _go_int(g("head_dim"), "head_dim")
    vocab = _go_int(g("vocab_size"), "vocab_size")
    dim = _go_int(g("hidden_size"), "hidden_size")
    hidden = _go_int(g("intermediate_size"), "intermediate_size")
    layers = _go_int(g("num_hidden_layers"), "num_hidden_layers")
    heads = _go_int(g("num_attention_heads"), "num_attention_heads")
    kv_heads = _go_int(g("num_key_value_heads"), "num_key_value_heads")
    context = _go_int(g("max_position_embeddings"), "max_position_embeddings")
    theta = _go_float(g("rope_theta"), "rope_theta")
    eps = _go_float(g("rms_norm_eps"), "rms_norm_eps")
    act = _go_str(g("hidden_act"), "hidden_act")
    tied = _go_bool(g("tie_word_embeddings"), "tie_word_embeddings")
    attention_bias = _go_bool(g("attention_bias"), "attention_bias")
    mlp_bias = _go_bool(g("mlp_bias"), "mlp_bias")
    interleaved = _go_bool(g("rope_interleaved"), "rope_interleaved")
    dropout = _go_float(g("attention_dropout"), "attention_dropout")
    tp = _go_int(g("pretraining_tp"), "pretraining_tp")
    bos = _go_int(g("bos_token_id"), "bos_token_id")
    eos = _go_int(eos_raw, "eos_token_id")
    sliding = _go_bool(g("use_sliding_window"), "use_sliding_window")
    layer_types = _go_strs(g("layer_types"), "layer_types")
    rope = g("rope_scaling")
    if rope is not None and not isinstance(rope, dict):
        raise HFError("HF config field rope_scaling: want an object")
    for id_ in extra_eos:
        if id_ >= vocab:
            raise HFError("Llama EOS ID outside vocabulary")
    if "head_dim" in raw and (raw["head_dim"] is None or heads < 1 or dim % heads != 0 or head_dim != dim // heads):
        raise HFError("HF head_dim must equal hidden_size / num_attention_heads")
    llama3 = None
    if rope is not None:
        if len(rope) != len(ROPE_FIELDS):
            raise HFError("Llama 3 RoPE requires exactly five canonical fields")
        for key in ROPE_FIELDS:
            if rope.get(key) is None:
                raise HFError("missing or null Llama 3 RoPE field %r" % key)
        r_type = _go_str(rope["rope_type"], "rope_type")
        factor = _go_float(rope["factor"], "factor")
        low = _go_float(rope["low_freq_factor"], "low_freq_factor")
        high = _go_float(rope["high_freq_factor"], "high_freq_factor")
        original = _go_int(rope["original_max_position_embeddings"], "original_max_position_embeddings")
        if (model_type != "llama" or r_type != "llama3" or not _finite(factor) or not _finite(low)
                or not _finite(high) or factor < 1 or factor > 1e6 or low < 1e-6 or high <= low
                or np.float32(high) <= np.float32(low) or high > 1e6 or original < 1 or original > 131072
                or original > context):
            raise HFError("unsupported or invalid Llama 3 RoPE scaling")
        llama3 = {"factor": factor, "low_freq_factor": low, "high_freq_factor": high,
                  "original_max_position_embeddings": original}
    arch = ARCH.get(model_type, "")
    if (arch == "" or architectures != [arch] or act != "silu" or attention_bias or mlp_bias or interleaved
            or dropout != 0 or tp not in (0, 1) or sliding):
        raise HFError("unsupported HF profile: require Llama, Qwen2 or full-attention Mistral, SiLU, supported "
                      "half-split RoPE and full causal attention")
    if layer_types and len(layer_types) != layers:
        raise HFError("HF layer_types count mismatch")
    if any(kind != "full_attention" for kind in layer_types):
        raise HFError("unsupported HF attention layer type")
    if (raw.get("bos_token_id") is None or raw.get("eos_token_id") is None or not 0 <= bos < vocab
            or not 0 <= eos < vocab):
        raise HFError("HF profile requires scalar BOS/EOS IDs within vocabulary")
    if context_limit < 0 or context_limit > context:
        raise HFError("HF context limit must be within model context")
    ctx = context_limit if context_limit > 0 else min(context, 2048)
    # Config.validateShapeLimits (M:100-114) with the HF limits.
    if (vocab < BASE_VOCAB or vocab > MAX_HF_VOCAB or dim < 2 or dim > 8192 or hidden < 1 or hidden > 32768
            or layers < 1 or layers > 128 or heads < 1 or heads > dim or kv_heads < 1 or kv_heads > heads
            or ctx < 1 or ctx > 32768):
        raise HFError("invalid model dimensions")
    if dim % heads != 0 or heads % kv_heads != 0 or (dim // heads) % 2 != 0:
        raise HFError("dim must be divisible by heads with an even head dimension; heads must be divisible by "
                      "kv_heads")
    if not _finite(theta) or theta <= 1 or not _finite(eps) or eps < 1e-12 or eps > 1:
        raise HFError("invalid RoPE theta or RMS epsilon")
    kvdim = dim // heads * kv_heads
    params = vocab * dim + layers * (2 * dim + 2 * dim * dim + 2 * dim * kvdim + 3 * dim * hidden) + dim
    if params > MAX_HF_PARAMETERS:
        raise HFError("model exceeds %d parameter allocation limit" % MAX_HF_PARAMETERS)
    # hfParameterCount (M:387-400): Qwen2 biases and the untied head.
    if model_type == "qwen2":
        params += layers * (dim + 2 * kvdim)
    if not tied:
        params += vocab * dim
    if params > MAX_HF_PARAMETERS:
        raise HFError("HF model exceeds %d parameters including biases and output head" % MAX_HF_PARAMETERS)
    cfg = make_config(vocab, dim, layers, heads, kv_heads, hidden, ctx, theta, eps, tied,
                      qkv_bias=model_type == "qwen2", llama3=llama3)
    return cfg, HFProfile(model_type, bos, eos, extra_eos, context)


def check_archive(config, directory):
    """srq_archive_check: the archive's metadata against config, on the host
    only; returns the archive's size in bytes."""
    size = C.c_int64()
    check(lib().srq_archive_check(C.byref(config), os.fsencode(directory), C.byref(size)))
    return size.value


def open_model(ex, directory, weight_format="f32", context_limit=0, cancel=None):
    """loadHFModelFormat (M:4979-5050): (Model, HFProfile) of a
    Transformers directory, weights packed to weight_format ("f32", "q8",
    "q4", "q4-mixed") on ex's device."""
    cfg, profile = read_config(directory, context_limit)
    check_archive(cfg, directory)
    m = Model(ex, cfg, weight_format)
    try:
        m.load_safetensors(directory, cancel)
    except Exception:
        m.close()
        raise
    return m, profile
