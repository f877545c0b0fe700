"""Copies the data that the reference's own tests hold for this path into small fixtures.

Sources (read as data from the reference checkout at /root/reference; run here only):
  tests/HFLabs.ML.LLM.LevelZero.Tests/golden/rope.golden.json         -> rope.golden.json (verbatim data)
  tests/HFLabs.ML.LLM.LevelZero.Tests/RopeLlama3Tests.cs:9-17         -> llama3_table.json (the Expected array)
  tests/HFLabs.ML.LLM.LevelZero.Tests/golden/qwen2.5-0.5b-instruct.layers.golden.json
                                                                     -> qwen25_layers_slice.npz
    (layers 0 and 11, first 6 tokens, the tensors whose relations involve no weight matrix:
     input, input_norm, attn_out, post_norm, mlp_out, output)

Usage: python tests/golden/extract_reference_fixtures.py
"""
from __future__ import annotations

import base64
import json
import re
from pathlib import Path

import numpy as np

REF = Path("/root/reference/tests/HFLabs.ML.LLM.LevelZero.Tests")
HERE = Path(__file__).resolve().parent
TOKENS = 6
LAYERS = ("0", "11")
TENSORS = ("input", "input_norm", "attn_out", "post_norm", "mlp_out", "output")


def main() -> None:
    rope = json.loads((REF / "golden" / "rope.golden.json").read_text())
    (HERE / "rope.golden.json").write_text(json.dumps(rope, indent=1))

    src = (REF / "RopeLlama3Tests.cs").read_text()
    block = re.search(r"Expected\s*=\s*\[(.*?)\];", src, re.S).group(1)
    values = [float(v.rstrip("f")) for v in re.findall(r"[-+0-9.eE]+f", block)]
    params = dict(head_dim=64, theta=500000.0, max_position_embeddings=131072, type="llama3", factor=32.0,
                  low_freq_factor=1.0, high_freq_factor=4.0, original_max_position_embeddings=8192)
    (HERE / "llama3_table.json").write_text(json.dumps(dict(params=params, expected=values), indent=1))

    layers = json.loads((REF / "golden" / "qwen2.5-0.5b-instruct.layers.golden.json").read_text())
    arrays = {}
    for li in LAYERS:
        entry = layers["layers"][li]
        for name in TENSORS:
            t = entry[name]
            a = np.frombuffer(base64.b64decode(t["data"]), dtype="<f4").reshape(t["shape"])
            arrays[f"l{li}/{name}"] = a[:TOKENS].astype(np.float32)
    np.savez_compressed(HERE / "qwen25_layers_slice.npz", eps=np.float32(1e-6), **arrays)
    print("wrote rope.golden.json, llama3_table.json, qwen25_layers_slice.npz")


if __name__ == "__main__":
    main()
