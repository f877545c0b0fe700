"""Writes the tiny end-to-end decoder fixtures (tests/golden/hf_tiny_*.npz).

The reference's own end-to-end goldens (tests/HFLabs.ML.LLM.LevelZero.Tests/golden/
gen_generation_golden.py, gen_layer_golden.py) come from Hugging Face transformers run in fp32
with eager attention. The checkpoints they need are not available here, so this script builds
the same transformers model classes from a config object with seeded random weights (no
download) and records, for a fixed prompt: every weight, the logits after each prompt
position, the greedy continuation and its per-step top-2 margins.

Usage: python tests/golden/gen_hf_tiny.py   (CPU, a few seconds)
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import torch
from transformers import LlamaConfig, LlamaForCausalLM, Qwen2Config, Qwen2ForCausalLM

HERE = Path(__file__).resolve().parent
PROMPT = [3, 17, 42, 5, 88, 23, 9, 61, 12, 70]
NEW_TOKENS = 12

CASES = {
    # Llama-3.x-shaped: GQA, no bias, untied head, llama3 RoPE scaling.
    "llama": dict(
        cls=(LlamaConfig, LlamaForCausalLM),
        config=dict(vocab_size=97, hidden_size=64, intermediate_size=160, num_hidden_layers=2,
                    num_attention_heads=4, num_key_value_heads=2, head_dim=16, max_position_embeddings=256,
                    rms_norm_eps=1e-5, tie_word_embeddings=False, attention_bias=False,
                    rope_parameters=dict(rope_type="llama3", rope_theta=500000.0, factor=8.0,
                                         low_freq_factor=1.0, high_freq_factor=4.0,
                                         original_max_position_embeddings=64)),
        seed=11),
    # Qwen2.5-shaped: GQA, q/k/v bias, tied embeddings, plain RoPE.
    "qwen2": dict(
        cls=(Qwen2Config, Qwen2ForCausalLM),
        config=dict(vocab_size=101, hidden_size=64, intermediate_size=128, num_hidden_layers=2,
                    num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=256,
                    rms_norm_eps=1e-6, tie_word_embeddings=True,
                    rope_parameters=dict(rope_type="default", rope_theta=1000000.0)),
        seed=12),
}


def make(name: str) -> None:
    case = CASES[name]
    cfg_cls, model_cls = case["cls"]
    torch.manual_seed(case["seed"])
    config = cfg_cls(**case["config"], attn_implementation="eager")
    model = model_cls(config).to(torch.float32).eval()
    with torch.no_grad():
        # Norm weights away from 1 and non-zero biases, so a dropped term shows.
        for n, p in model.named_parameters():
            if n.endswith("norm.weight"):
                p.copy_(1.0 + 0.1 * torch.randn_like(p))
            elif n.endswith(".bias"):
                p.copy_(0.05 * torch.randn_like(p))
            elif p.dim() == 2:
                p.copy_(0.08 * torch.randn_like(p))
        ids = torch.tensor([PROMPT])
        out = model(ids, use_cache=False)
        prompt_logits = out.logits[0].numpy().astype(np.float32)
        seq = list(PROMPT)
        margins = []
        for _ in range(NEW_TOKENS):
            lg = model(torch.tensor([seq]), use_cache=False).logits[0, -1]
            top = torch.topk(lg, 2).values
            margins.append(float(top[0] - top[1]))
            seq.append(int(torch.argmax(lg)))
    weights = {n: p.detach().numpy().astype(np.float32) for n, p in model.named_parameters()}
    if config.tie_word_embeddings:
        weights["lm_head.weight"] = weights["model.embed_tokens.weight"]
    meta = dict(config={k: v for k, v in case["config"].items()}, prompt=PROMPT, generated=seq[len(PROMPT):],
                margins=margins, torch=torch.__version__)
    np.savez_compressed(HERE / f"hf_tiny_{name}.npz", prompt_logits=prompt_logits,
                        meta=np.array(json.dumps(meta)), **{"w/" + k: v for k, v in weights.items()})
    print(f"wrote hf_tiny_{name}.npz: generated {meta['generated']}, min margin {min(margins):.4f}")


if __name__ == "__main__":
    for n in CASES:
        make(n)
