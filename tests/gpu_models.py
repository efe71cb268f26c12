"""Helpers that build device models (through the C ABI) and their oracle
twins from the committed fixtures or from seeded synthetic weights."""
import numpy as np

import oracle
import sr_go_tranformer_amd as srq

KIND = {"q_proj": srq.T_Q, "k_proj": srq.T_K, "v_proj": srq.T_V, "o_proj": srq.T_O, "gate_proj": srq.T_GATE,
        "up_proj": srq.T_UP, "down_proj": srq.T_DOWN, "input_layernorm": srq.T_ATTN_NORM,
        "post_attention_layernorm": srq.T_FFN_NORM, "q_bias": srq.T_Q_BIAS, "k_bias": srq.T_K_BIAS,
        "v_bias": srq.T_V_BIAS}
MATRICES = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")
OFMT = {srq.F32: oracle.F32, srq.Q8: oracle.Q8, srq.Q4: oracle.Q4}


def kind_of(name):
    if name == "embed_tokens":
        return srq.T_EMBED, 0
    if name == "norm":
        return srq.T_FINAL_NORM, 0
    if name == "lm_head":
        return srq.T_OUTPUT, 0
    _, layer, nm = name.split(".")
    return KIND[nm], int(layer)


def fixture_config(fx):
    return srq.make_config(fx.vocab, fx.dim, fx.layers, fx.heads, fx.kv_heads, fx.hidden, fx.context, fx.theta,
                           fx.eps, fx.tied, qkv_bias=any(k.endswith("_bias") for k in fx.w), llama3=fx.llama3)


def load_fixture(ex, fx, fmt, use_raw=False):
    """Device model of a tests/golden fixture.  use_raw loads F16/BF16
    fixtures from their 16-bit words (device decode + pack)."""
    m = srq.Model(ex, fixture_config(fx), fmt)
    dt = {"BF16": srq.SRC_BF16, "F16": srq.SRC_F16}.get(fx.dtype, srq.SRC_F32)
    for name, arr in fx.w.items():
        kind, layer = kind_of(name)
        if use_raw and name in fx.raw:
            m.load(kind, layer, fx.raw[name], dt)
        else:
            m.load(kind, layer, arr)
    return m


def oracle_from_device(ex, m, cfg, norms):
    """Oracle model reading the device model's packed weights back, plus
    the given FP32 vectors (norms/biases) by name."""
    weights = {}

    def take(name, w):
        vals, scl = w.packed(ex)
        if w.fmt == srq.F32:
            weights[name] = oracle.Weight(oracle.F32, w.rows, w.cols, vals.view(np.float32).reshape(w.rows, w.cols))
        elif w.fmt == srq.Q8:
            weights[name] = oracle.Weight(oracle.Q8, w.rows, w.cols, vals.view(np.int8).reshape(w.rows, w.cols),
                                          scl.reshape(w.rows, -1))
        else:
            weights[name] = oracle.Weight(oracle.Q4, w.rows, w.cols, vals.reshape(w.rows, -1), scl.reshape(w.rows, -1))

    take("embed_tokens", m.weight(srq.T_EMBED))
    if not cfg.tied:
        take("lm_head", m.weight(srq.T_OUTPUT))
    for layer in range(cfg.layers):
        for nm in MATRICES:
            take("layers.%d.%s" % (layer, nm), m.weight(KIND[nm], layer))
    for name, vec in norms.items():
        vec = np.asarray(vec, np.float32).reshape(-1)
        weights[name] = oracle.Weight(oracle.F32, 1, vec.shape[0], vec)
    ocfg = oracle.make_config(cfg.vocab, cfg.dim, cfg.layers, cfg.heads, cfg.kv_heads, cfg.hidden, cfg.context,
                              cfg.rope_theta, cfg.norm_eps, bool(cfg.tied))
    return oracle.Model(ocfg, weights)


def synthetic(ex, cfg, fmt, seed):
    """Seeded device model (sr_go_tranformer_amd.synthetic) plus its unit
    norms by oracle name."""
    from sr_go_tranformer_amd import synthetic as syn
    m = syn.build(ex, cfg, fmt, seed)
    ones = np.ones(cfg.dim, np.float32)
    norms = {"norm": ones}
    for layer in range(cfg.layers):
        norms["layers.%d.input_layernorm" % layer] = ones
        norms["layers.%d.post_attention_layernorm" % layer] = ones
    return m, norms
