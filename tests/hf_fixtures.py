"""Load the committed Transformers fixtures (tests/golden/hf_*.npz, made by
tests/golden/make_golden.py from the reference's testdata/hf-* directories)
into oracle models and into the shapes the GPU tests need."""
import json
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
NAMES = ["llama_f32", "llama_f16", "llama_bf16", "llama_untied-f32", "llama3_f32", "llama3_f16", "llama3_bf16",
         "mistral_f32", "mistral_f16", "mistral_bf16", "qwen2_f32", "qwen2_f16", "qwen2_untied-bf16"]
MATRICES = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")


class Fixture:
    def __init__(self, name):
        self.name = name
        z = np.load(os.path.join(GOLDEN, "hf_%s.npz" % name))
        self.cfg = json.loads(str(z["config"]))
        self.ids = [int(i) for i in z["ids"]]
        self.logits = z["logits"]
        self.k = z["k"]
        self.v = z["v"]
        self.dtype = str(z["dtype"])
        self.w = {k[2:]: z[k] for k in z.files if k.startswith("w/")}
        self.raw = {k[4:]: z[k] for k in z.files if k.startswith("raw/")}
        c = self.cfg
        self.vocab = c["vocab_size"]
        self.dim = c["hidden_size"]
        self.layers = c["num_hidden_layers"]
        self.heads = c["num_attention_heads"]
        self.kv_heads = c.get("num_key_value_heads", self.heads)
        self.hidden = c["intermediate_size"]
        self.context = c["max_position_embeddings"]
        self.theta = float(c.get("rope_theta", 10000.0))
        self.eps = float(c.get("rms_norm_eps", 1e-5))
        self.tied = bool(c.get("tie_word_embeddings", True))
        self.llama3 = c.get("rope_scaling")

    def matrix_format(self, name, fmt):
        """hfMatrixFormat (M:572-582): q4-mixed keeps embeddings/head Q8."""
        if fmt != "q4-mixed":
            return fmt
        return "q8" if name in ("embed_tokens", "lm_head") else "q4"

    def is_matrix(self, name):
        return name in ("embed_tokens", "lm_head") or name.split(".")[-1] in MATRICES

    def oracle_config(self):
        import oracle
        return oracle.make_config(self.vocab, self.dim, self.layers, self.heads, self.kv_heads, self.hidden,
                                  self.context, self.theta, self.eps, self.tied, self.llama3)

    def oracle_model(self, fmt="f32", dense_override=None):
        import oracle
        codes = {"f32": oracle.F32, "q8": oracle.Q8, "q4": oracle.Q4}
        weights = {}
        src = dense_override if dense_override is not None else self.w
        for name, arr in src.items():
            arr = np.asarray(arr, np.float32)
            if arr.ndim == 1:
                weights[name] = oracle.Weight(oracle.F32, 1, arr.shape[0], arr)
            elif self.is_matrix(name):
                weights[name] = oracle.Weight.from_dense(arr, codes[self.matrix_format(name, fmt)])
            else:
                weights[name] = oracle.Weight(oracle.F32, arr.shape[0], arr.shape[1], arr)
        return oracle.Model(self.oracle_config(), weights)


def load(name):
    return Fixture(name)
