"""Qwen3 forward oracle (test infrastructure only): numpy fp32, the reference CPU eager path.

Restates src/models/qwen3/model.rs:155-534 with the `pt` attention backend
(src/models/attention/backend.rs:1183-1498) and the ops of src/layers/ops.rs:8-127:

    h = embed[ids]
    per layer: x = rms(h) | add_rms(h, r);  qkv = x Wqkv^T;  q,k = rope(qk_norm(q, k));
               cache <- (k, v);  a = causal GQA softmax(q k^T / sqrt(D)) v;
               x, r = add_rms(a Wo^T, r);  h = (silu(x Wg^T) * x Wu^T) Wd^T
    logits = add_rms(h, r) Wlm^T

Weights are a dict of float32 arrays with the Hugging Face names used by
``llm_infer_rust_amd.model.Qwen3Model.named_parameters`` (qkv and gate/up packed).
Pinned by Hugging Face `transformers`' own Qwen3ForCausalLM (an independent implementation of
the same architecture) on seeded random weights with non-unit norm weights: prompt + cached
decode logits within 1e-4 at two tiny shapes (tied / untied head, rope_theta 1e4 / 1e6, GQA
group 2 / 4) and at 2 layers of the Qwen3-0.6B widths (tests/test_oracle_qwen3_hf.py, whose
mutation tests show that QK-norm after RoPE, a post-attention norm without the residual, a
wrong rope_theta or a tied/untied mix-up each fail it); by the reference's self-consistency
fixture (model.rs:730-900): prefill + cached decode gives the same logits as a full forward
over the whole sequence, and chunked prefill the same as one-shot prefill; and by the
attention / norm / RoPE oracles it is built from.
"""
from __future__ import annotations

import numpy as np

from . import attention, layer_ops, norms


def _rms(x, w, eps):
    return norms.rms_norm_f32(x, w, eps)


class Qwen3Oracle:
    def __init__(self, cfg, weights: dict[str, np.ndarray]):
        self.cfg = cfg
        self.w = {k: np.asarray(v, np.float32) for k, v in weights.items()}
        self.cos, self.sin = layer_ops.rope_tables(cfg.max_position_embeddings, cfg.head_dim,
                                                   cfg.rope_theta)
        self.reset()

    def reset(self) -> None:
        """Drop the per-layer K/V cache (lists of [T, Hkv, D] float32)."""
        self.k_cache = [np.zeros((0, self.cfg.num_kv_heads, self.cfg.head_dim), np.float32)
                        for _ in range(self.cfg.num_layers)]
        self.v_cache = [c.copy() for c in self.k_cache]

    def _attention(self, q, k_all, v_all, start):
        """Causal GQA attention of queries at positions start.. over cached keys (the pinned
        attention oracle, backend.rs:1463-1498), returned in float32."""
        cfg = self.cfg
        return attention.attention_against_cache(q, k_all, v_all, start, cfg.num_attention_heads,
                                                 cfg.num_kv_heads).astype(np.float32)

    def forward(self, ids: np.ndarray, start: int, last_only: bool = False) -> np.ndarray:
        """Append ``ids`` at positions start.. to the cache; return logits for every row (or
        only the last, as the reference computes them only at ``logits_indices``)."""
        cfg, w = self.cfg, self.w
        ids = np.asarray(ids, np.int64)
        t = ids.size
        hq, hkv, d = cfg.num_attention_heads, cfg.num_kv_heads, cfg.head_dim
        eps = cfg.rms_norm_eps
        pos = start + np.arange(t)
        h = w["model.embed_tokens.weight"][ids]
        r = None
        for i in range(cfg.num_layers):
            p = f"model.layers.{i}."
            if r is None:
                r = h
                x = _rms(h, w[p + "input_layernorm.weight"], eps)
            else:
                x, r = norms.add_rms_norm_f32(h, r, w[p + "input_layernorm.weight"], eps)
            qkv = x @ w[p + "self_attn.qkv_proj.weight"].T
            q = qkv[:, : hq * d].reshape(t, hq, d)
            k = qkv[:, hq * d:(hq + hkv) * d].reshape(t, hkv, d)
            v = qkv[:, (hq + hkv) * d:].reshape(t, hkv, d)
            q = _rms(q, w[p + "self_attn.q_norm.weight"], eps)
            k = _rms(k, w[p + "self_attn.k_norm.weight"], eps)
            q = layer_ops.rope(q, pos, self.cos, self.sin)
            k = layer_ops.rope(k, pos, self.cos, self.sin)
            if self.k_cache[i].shape[0] != start:
                raise ValueError("oracle cache length does not match the start position")
            self.k_cache[i] = np.concatenate([self.k_cache[i], k])
            self.v_cache[i] = np.concatenate([self.v_cache[i], v.astype(np.float32)])
            a = self._attention(q, self.k_cache[i], self.v_cache[i], start).reshape(t, hq * d)
            o = a @ w[p + "self_attn.o_proj.weight"].T
            x, r = norms.add_rms_norm_f32(o, r, w[p + "post_attention_layernorm.weight"], eps)
            gu = x @ w[p + "mlp.gate_up_proj.weight"].T
            h = layer_ops.silu_mul(gu) @ w[p + "mlp.down_proj.weight"].T
        if last_only:
            h, r = h[-1:], r[-1:]
        h, _ = norms.add_rms_norm_f32(h, r, w["model.norm.weight"], eps)
        lm = w["model.embed_tokens.weight"] if cfg.tie_word_embeddings else w["lm_head.weight"]
        return (h @ lm.T).astype(np.float32)

    def greedy(self, prompt: np.ndarray, steps: int) -> tuple[list[int], float]:
        """Prefill + cached greedy decode; returns tokens and the smallest top-1/top-2 margin."""
        self.reset()
        logits = self.forward(prompt, 0)[-1]
        tokens, margins = [], []
        pos = len(prompt)
        for _ in range(steps):
            top2 = np.partition(logits, -2)[-2:]
            margins.append(float(abs(top2[1] - top2[0])))
            tok = int(np.argmax(logits))
            tokens.append(tok)
            logits = self.forward(np.array([tok]), pos)[-1]
            pos += 1
        return tokens, min(margins) if margins else float("inf")


def random_weights(cfg, seed: int, std: float = 0.02,
                   norm_range: tuple[float, float] | None = None) -> dict[str, np.ndarray]:
    """Seeded N(0, std) float32 matrices, Hugging Face names. Norm weights are 1, or, with
    ``norm_range``, U(lo, hi) from a second generator (seed + 1) so the matrices are the same
    either way; non-unit norm weights make a swapped or misplaced norm visible."""
    rng = np.random.default_rng(seed)
    nrng = np.random.default_rng(seed + 1)

    def normw(n):
        if norm_range is None:
            return np.ones(n, np.float32)
        return nrng.uniform(norm_range[0], norm_range[1], n).astype(np.float32)
    h, d, f = cfg.hidden_size, cfg.head_dim, cfg.intermediate_size
    qkv = (cfg.num_attention_heads + 2 * cfg.num_kv_heads) * d

    def mat(*shape):
        return (rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float32)

    w = {"model.embed_tokens.weight": mat(cfg.vocab_size, h),
         "model.norm.weight": normw(h)}
    if not cfg.tie_word_embeddings:
        w["lm_head.weight"] = mat(cfg.vocab_size, h)
    for i in range(cfg.num_layers):
        p = f"model.layers.{i}."
        w[p + "input_layernorm.weight"] = normw(h)
        w[p + "self_attn.qkv_proj.weight"] = mat(qkv, h)
        w[p + "self_attn.q_norm.weight"] = normw(d)
        w[p + "self_attn.k_norm.weight"] = normw(d)
        w[p + "self_attn.o_proj.weight"] = mat(h, cfg.num_attention_heads * d)
        w[p + "post_attention_layernorm.weight"] = normw(h)
        w[p + "mlp.gate_up_proj.weight"] = mat(2 * f, h)
        w[p + "mlp.down_proj.weight"] = mat(h, f)
    return w
