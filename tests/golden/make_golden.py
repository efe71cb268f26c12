"""Regenerate the committed golden fixtures under tests/golden/.

Run in the build container (it reads the reference checkout, which the GPU
machine does not have):  python tests/golden/make_golden.py

1. hf_*.npz -- the reference's own Transformers fixtures
   (testdata/hf-{llama,llama3,mistral,qwen2}/*/: config.json,
   model.safetensors, reference.json; used by hf_inference_test.go:32-124)
   re-encoded as numpy arrays: the source tensors (decoded to f32, plus the
   raw 16-bit words for F16/BF16 sources), the 37 input IDs, Transformers'
   FP32 logits for every position and every K/V row.  Pure data: inputs and
   expected outputs.  The weight file's SHA-256 is checked against the one
   reference.json binds before anything is written.
2. llama3_frequencies.json -- testdata/hf-llama3/frequencies.json, the
   Transformers RoPE inverse-frequency vectors (hf_llama3_test.go:132).
"""
import hashlib
import json
import os
import shutil
import struct
import sys

import numpy as np

REF = "/root/reference/testdata"
HERE = os.path.dirname(os.path.abspath(__file__))

FIXTURES = ["hf-llama/f32", "hf-llama/f16", "hf-llama/bf16", "hf-llama/untied-f32", "hf-llama3/f32",
            "hf-llama3/f16", "hf-llama3/bf16", "hf-mistral/f32", "hf-mistral/f16", "hf-mistral/bf16",
            "hf-qwen2/f32", "hf-qwen2/f16", "hf-qwen2/untied-bf16"]


def read_safetensors(path):
    b = open(path, "rb").read()
    n = struct.unpack("<Q", b[:8])[0]
    header = json.loads(b[8:8 + n])
    data = b[8 + n:]
    out = {}
    for name, meta in header.items():
        if name == "__metadata__":
            continue
        lo, hi = meta["data_offsets"]
        raw = data[lo:hi]
        dt = meta["dtype"]
        shape = meta["shape"]
        if dt == "F32":
            out[name] = (dt, np.frombuffer(raw, "<f4").reshape(shape).copy(), None)
        elif dt == "BF16":
            words = np.frombuffer(raw, "<u2").reshape(shape).copy()
            out[name] = (dt, (words.astype(np.uint32) << 16).view(np.float32), words)
        elif dt == "F16":
            words = np.frombuffer(raw, "<u2").reshape(shape).copy()
            out[name] = (dt, words.view(np.float16).astype(np.float32), words)
        else:
            raise ValueError(dt)
    return out, b


def main():
    for fx in FIXTURES:
        d = os.path.join(REF, fx)
        cfg = json.load(open(os.path.join(d, "config.json")))
        ref = json.load(open(os.path.join(d, "reference.json")))
        tensors, blob = read_safetensors(os.path.join(d, "model.safetensors"))
        if hashlib.sha256(blob).hexdigest() != ref["weight_sha256"]:
            raise SystemExit("weight identity mismatch for " + fx)
        arrays = {
            "config": np.array(json.dumps(cfg)),
            "ids": np.array(ref["ids"], np.int32),
            "logits": np.array(ref["logits"], np.float64).astype(np.float32),
            "k": np.array([layer["k"] for layer in ref["cache"]], np.float64).astype(np.float32),
            "v": np.array([layer["v"] for layer in ref["cache"]], np.float64).astype(np.float32),
            "weight_sha256": np.array(ref["weight_sha256"]),
        }
        for name, (dt, f32, words) in tensors.items():
            key = name.replace("model.", "", 1) if name.startswith("model.") else name
            key = key.replace(".weight", "").replace(".bias", "_bias")
            key = key.replace("self_attn.", "").replace("mlp.", "")
            key = key.replace("q_proj_bias", "q_bias").replace("k_proj_bias", "k_bias").replace("v_proj_bias", "v_bias")
            arrays["w/" + key] = f32
            arrays["dtype"] = np.array(dt)
            if words is not None:
                arrays["raw/" + key] = words
        out = os.path.join(HERE, "hf_" + fx.replace("hf-", "").replace("/", "_") + ".npz")
        np.savez_compressed(out, **arrays)
        print(out, os.path.getsize(out))
    shutil.copyfile(os.path.join(REF, "hf-llama3", "frequencies.json"), os.path.join(HERE, "llama3_frequencies.json"))
    return 0


if __name__ == "__main__":
    sys.exit(main())
