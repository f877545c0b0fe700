"""The reference's own decode step, operator by operator, on this library's LlmKernelSuite entry
points: what an unchanged C# LlmModel.Step (LlmModel.cs:402-444) over LlmDecoderLayer.Forward and
MixFull (LlmDecoderLayer.cs:129-196, :291-334) issues once the LevelZero operators are bound to
libl0hip (the drop-in path), for Llama-shaped int8 models (no biases, no QK-norm, rotary dim =
head_dim).

Per layer: RMSNorm; GemvQ8.Quantize once and Execute for q, k and v (LlmMatrix.ProjectShared,
LlmMatrix.cs:177-218); RoPE.ExecuteWithFrequencies; KvCacheStore; Attention; Quantize + Execute for O
(LlmMatrix.Project, :122-144); RMSNorm with the residual add; Quantize once and Execute for gate and
up; SwiGLU; Quantize + Execute for down; Add. Before the layers Embedding, after them RMSNorm,
Quantize + Execute for lm_head and Sampling (AppendHead, LlmModel.cs:387-400): 18 operators per
layer and 5 per token. Activations stay fp32 between operators, as in the reference.
"""
from __future__ import annotations

import numpy as np

from . import api
from ._lib import F16

PROJECTIONS = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")


class ReferenceStep:
    """Device buffers of one model in the reference's per-matrix layout, and its decode step.

    weights: HuggingFace names -> int8 projections as (storage, int8 [N, K], fp16 scale bits [N])
    (the form LlmModel.export_matrix returns) and fp32 vectors. caches: per layer the device
    addresses of fp16 K and V caches of max_seq_len rows, copied into buffers of this object."""

    def __init__(self, device: api.Device, config: api.HfConfig, weights: dict, max_seq_len: int,
                 caches: list[tuple[int, int]] | None = None):
        c = config
        self.device, self.config, self.max_seq_len = device, c, max_seq_len
        self.suite = api.LlmKernelSuite(device)
        self.h, self.inter, self.vocab = c.hidden_size, c.intermediate_size, c.vocab_size
        self.nh, self.nkv, self.hd = c.num_attention_heads, c.num_key_value_heads, c.head_dim
        self.qd, self.kvd = self.nh * self.hd, self.nkv * self.hd
        self._bufs: list[api.Buffer] = []
        try:
            self._upload(weights, caches)
        except Exception:
            self.close()
            raise

    def _up(self, a) -> api.Buffer:
        b = self.device.alloc_shared(np.ascontiguousarray(a))
        self._bufs.append(b)
        return b

    def _alloc(self, nbytes: int) -> api.Buffer:
        b = self.device.alloc(nbytes)
        self._bufs.append(b)
        return b

    def _upload(self, w: dict, caches) -> None:
        c, s = self.config, self.suite
        cache_bytes = self.max_seq_len * self.kvd * 2
        self.layers = []
        for i in range(c.num_layers):
            p = f"model.layers.{i}."
            mats = {}
            for n in PROJECTIONS:
                key = p + ("self_attn." if n[0] in "qkvo" else "mlp.") + n + ".weight"
                _, q8, sc = w[key]
                mats[n] = (self._up(q8), self._up(np.asarray(sc).view(np.uint16)), q8.shape[0], q8.shape[1])
            kc, vc = self._alloc(cache_bytes), self._alloc(cache_bytes)
            if caches is not None:  # the cache rows as 32-bit words
                s.copy_execute(caches[i][0], kc, 0, cache_bytes // 4)
                s.copy_execute(caches[i][1], vc, 0, cache_bytes // 4)
            else:
                kc.zero()
                vc.zero()
            self.layers.append(dict(mats=mats, in_norm=self._up(np.float32(w[p + "input_layernorm.weight"])),
                                    post_norm=self._up(np.float32(w[p + "post_attention_layernorm.weight"])),
                                    kc=kc, vc=vc))
        self.emb = self._up(np.float32(w["model.embed_tokens.weight"]))
        self.final_norm = self._up(np.float32(w["model.norm.weight"]))
        _, lm8, lms = w["lm_head.weight"]
        self.lm = (self._up(lm8), self._up(np.asarray(lms).view(np.uint16)))
        h, qd, kvd, inter = self.h, self.qd, self.kvd, self.inter
        self.hidden, self.normed = self._alloc(4 * h), self._alloc(4 * h)
        self.q, self.k, self.v = self._alloc(4 * qd), self._alloc(4 * kvd), self._alloc(4 * kvd)
        self.attn, self.proj = self._alloc(4 * qd), self._alloc(4 * h)
        self.gate, self.up, self.down = self._alloc(4 * inter), self._alloc(4 * inter), self._alloc(4 * h)
        self.logits, self.sampled = self._alloc(4 * self.vocab), self._alloc(4)
        self.token, self.position = self._alloc(4), self._alloc(4)
        inv, self.attn_scale = api.rope_frequencies(self.hd, c.rope_theta, c.max_position_embeddings)
        self.inv_freq = self._up(np.float32(inv))
        # EnsureQ8Scratch and the attention workspace are sized before any recording (LlmModel.cs:139-144)
        s.ensure_q8_scratch(1, max(h, inter, qd))
        self.scratch = s.q8_scratch
        s.attention_reserve(1, self.nh, self.nkv, self.hd, self.max_seq_len)

    def set_token(self, token: int, position: int) -> None:
        """Token id and position for the next step (LlmModel.Step writes both, :413; MixFull writes the
        position, LlmDecoderLayer.cs:320)."""
        self.token.write(np.array([token], dtype=np.int32))
        self.position.write(np.array([position], dtype=np.int32))

    def _project(self, mat, n_out: int, n_in: int, x, y) -> None:  # LlmMatrix.Project, int8 storage
        self.suite.gemv_q8_quantize(1, n_in, x, self.scratch)
        self.suite.gemv_q8_execute(n_out, n_in, self.scratch, mat[0], mat[1], y)

    def step(self, position: int) -> None:
        """Issues one token's operators (the caller records them, or not)."""
        s, h, inter, qd, kvd = self.suite, self.h, self.inter, self.qd, self.kvd
        eps = self.config.rms_norm_eps
        s.embedding_execute(self.token, self.emb, self.hidden, h, h)
        for L in self.layers:
            m = L["mats"]
            s.rmsnorm_execute(self.hidden, None, L["in_norm"], self.normed, eps, h, 1, False)
            s.gemv_q8_quantize(1, h, self.normed, self.scratch)  # ProjectShared: one Quantize for q, k, v
            for name, y in (("q_proj", self.q), ("k_proj", self.k), ("v_proj", self.v)):
                s.gemv_q8_execute(m[name][2], h, self.scratch, m[name][0], m[name][1], y)
            s.rope_execute_with_frequencies(self.q, self.k, self.position, self.inv_freq, self.hd, self.nh, self.nkv,
                                            self.attn_scale, 1, self.hd)
            s.kv_cache_store_execute(self.k, self.v, L["kc"], L["vc"], position, kvd, cache_dtype=F16)
            s.attention_execute(self.q, L["kc"], L["vc"], self.attn, self.hd, self.nh, self.nkv, position + 1,
                                self.max_seq_len, cache_dtype=F16)
            self._project(m["o_proj"], h, qd, self.attn, self.proj)
            s.rmsnorm_execute(self.hidden, self.proj, L["post_norm"], self.normed, eps, h, 1, True)
            s.gemv_q8_quantize(1, h, self.normed, self.scratch)  # ProjectShared: gate and up
            s.gemv_q8_execute(inter, h, self.scratch, m["gate_proj"][0], m["gate_proj"][1], self.gate)
            s.gemv_q8_execute(inter, h, self.scratch, m["up_proj"][0], m["up_proj"][1], self.up)
            s.swiglu_execute(self.gate, self.up, inter)
            self._project(m["down_proj"], h, inter, self.gate, self.down)
            s.add_execute(self.hidden, self.down, h)
        s.rmsnorm_execute(self.hidden, None, self.final_norm, self.normed, eps, h, 1, False)
        self._project(self.lm, self.vocab, h, self.normed, self.logits)
        s.sampling_execute(self.logits, self.sampled, 0.0, 0.0, self.vocab)

    def record_step(self, position: int) -> None:
        """The step as one recording (LlmModel.Step, :416-443); end_recording runs it once."""
        self.device.begin_recording()
        try:
            self.step(position)
        except Exception:
            self.device.abort_recording()
            raise
        self.device.end_recording()

    def read_sampled(self) -> int:
        return int(self.sampled.read(np.int32, 1)[0])

    def read_logits(self) -> np.ndarray:
        return self.logits.read(np.float32, self.vocab)

    def close(self) -> None:
        for b in self._bufs:
            b.free()
        self._bufs = []
