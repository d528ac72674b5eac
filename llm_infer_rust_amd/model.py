"""Dense Qwen3 decoder on the gfx950 kernels (the model the attention path serves).

Follows the reference layer sequence (``src/models/qwen3/model.rs:155-534``):

    hidden = embed(ids)
    per layer:  (x, residual) = input_norm(hidden, residual)        rms_norm / add_rms_norm
                qkv = x W_qkv^T                                       packed [T, (Hq+2Hkv) D]
                q, k <- rope(qk_norm(q, k)); cache[write_loc] <- (k, v)   one fused pass here
                a = attention(q, k, v)                                 decode / prefill plan
                (x, residual) = add_rms_norm(a W_o^T, residual)
                hidden = (silu(x W_gate^T) * x W_up^T) W_down^T
    logits = add_rms_norm(hidden, residual)[logits_indices] W_lm^T

For decode batches (at most 256 rows) the QKV, o_proj and down projections run on this
library's projection kernel (QKV with its split-K partials summed inside the QK-norm/RoPE/
store pass, o_proj and down fused with the residual RMSNorm that follows them) and gate_up runs
fused with SiLU x mul; prefill-sized products and the lm_head are
library GEMMs (torch -> hipBLASLt). Everything around them is this library's HIP code. Configuration fields and defaults follow ``src/models/qwen3/config.rs:9-42``.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F

from . import ops
from .backend import Attention, AttentionBatch, AttentionSpec
from .kv_cache import BaseAttention, ModelError


@dataclass(frozen=True)
class Qwen3Config:
    hidden_size: int
    num_layers: int
    num_attention_heads: int
    num_kv_heads: int
    intermediate_size: int
    vocab_size: int
    head_dim: int = 128
    max_position_embeddings: int = 8192
    rope_theta: float = 10_000.0
    rms_norm_eps: float = 1e-6
    tie_word_embeddings: bool = False

    @staticmethod
    def qwen3_8b() -> "Qwen3Config":
        """Qwen3-8B dimensions (36 layers, hidden 4096, 32/8 heads, FFN 12288)."""
        return Qwen3Config(4096, 36, 32, 8, 12288, 151936, 128, 40960, 1_000_000.0, 1e-6, False)

    @staticmethod
    def qwen3_0_6b() -> "Qwen3Config":
        """Qwen3-0.6B dimensions (28 layers, hidden 1024, 16/8 heads, FFN 3072)."""
        return Qwen3Config(1024, 28, 16, 8, 3072, 151936, 128, 40960, 1_000_000.0, 1e-6, True)

    def validate(self) -> None:
        if min(self.hidden_size, self.num_layers, self.num_attention_heads, self.num_kv_heads,
               self.intermediate_size, self.vocab_size, self.head_dim) <= 0:
            raise ModelError("Qwen3 dimensions must be positive")
        if self.num_attention_heads % self.num_kv_heads:
            raise ModelError("num_attention_heads must be a multiple of num_kv_heads")

    @property
    def qkv_width(self) -> int:
        return (self.num_attention_heads + 2 * self.num_kv_heads) * self.head_dim


class Qwen3Layer:
    def __init__(self, cfg: Qwen3Config, dtype: torch.dtype, device: torch.device):
        h, d = cfg.hidden_size, cfg.head_dim
        self.input_layernorm = torch.ones(h, dtype=dtype, device=device)
        self.qkv_proj = torch.empty(cfg.qkv_width, h, dtype=dtype, device=device)
        self.q_norm = torch.ones(d, dtype=dtype, device=device)
        self.k_norm = torch.ones(d, dtype=dtype, device=device)
        self.o_proj = torch.empty(h, cfg.num_attention_heads * d, dtype=dtype, device=device)
        self.post_attention_layernorm = torch.ones(h, dtype=dtype, device=device)
        self.gate_up_proj = torch.empty(2 * cfg.intermediate_size, h, dtype=dtype, device=device)
        self.down_proj = torch.empty(h, cfg.intermediate_size, dtype=dtype, device=device)
        self.base_attention = BaseAttention()

    def matrices(self) -> list[torch.Tensor]:
        return [self.qkv_proj, self.o_proj, self.gate_up_proj, self.down_proj]


class Qwen3Model:
    """Weights plus forward; one ``Attention`` shared by all layers."""

    def __init__(self, cfg: Qwen3Config, dtype: torch.dtype = torch.bfloat16,
                 device: torch.device | str = "cuda", attention_backend: str = "mi355x"):
        cfg.validate()
        device = torch.device(device)
        self.cfg = cfg
        self.dtype = dtype
        self.device = device
        self.embed_tokens = torch.empty(cfg.vocab_size, cfg.hidden_size, dtype=dtype,
                                        device=device)
        self.layers = [Qwen3Layer(cfg, dtype, device) for _ in range(cfg.num_layers)]
        self.norm = torch.ones(cfg.hidden_size, dtype=dtype, device=device)
        self.lm_head = (self.embed_tokens if cfg.tie_word_embeddings else
                        torch.empty(cfg.vocab_size, cfg.hidden_size, dtype=dtype, device=device))
        self.rope = ops.HalfSplitRope(cfg.max_position_embeddings, cfg.head_dim, cfg.rope_theta,
                                      device)
        self.attention = Attention.new(attention_backend, AttentionSpec(
            cfg.num_attention_heads, cfg.num_kv_heads, cfg.head_dim, dtype, device))

    # ------------------------------------------------------------------ weights
    def init_random(self, seed: int, std: float = 0.02) -> "Qwen3Model":
        """Seeded N(0, std) matrices and embeddings; norm weights stay 1 (synthetic weights)."""
        g = torch.Generator(device=self.device)
        g.manual_seed(seed)
        mats = [self.embed_tokens] + [m for layer in self.layers for m in layer.matrices()]
        if not self.cfg.tie_word_embeddings:
            mats.append(self.lm_head)
        for m in mats:
            m.normal_(0.0, std, generator=g)
        return self

    def named_parameters(self) -> dict[str, torch.Tensor]:
        """Hugging Face parameter names (qkv and gate/up stay packed)."""
        out = {"model.embed_tokens.weight": self.embed_tokens, "model.norm.weight": self.norm}
        if not self.cfg.tie_word_embeddings:
            out["lm_head.weight"] = self.lm_head
        for i, layer in enumerate(self.layers):
            p = f"model.layers.{i}."
            out[p + "input_layernorm.weight"] = layer.input_layernorm
            out[p + "self_attn.qkv_proj.weight"] = layer.qkv_proj
            out[p + "self_attn.q_norm.weight"] = layer.q_norm
            out[p + "self_attn.k_norm.weight"] = layer.k_norm
            out[p + "self_attn.o_proj.weight"] = layer.o_proj
            out[p + "post_attention_layernorm.weight"] = layer.post_attention_layernorm
            out[p + "mlp.gate_up_proj.weight"] = layer.gate_up_proj
            out[p + "mlp.down_proj.weight"] = layer.down_proj
        return out

    def load_weights(self, weights) -> int:
        """Copy tensors by Hugging Face name (``named_parameters`` names); every parameter must
        be supplied with its exact shape (src/models/qwen3/model.rs:231-300). Returns the count."""
        params = self.named_parameters()
        loaded = 0
        for name, value in weights.items():
            if name not in params:
                raise ModelError(f"unexpected weight {name}")
            t = torch.as_tensor(value)
            if tuple(t.shape) != tuple(params[name].shape):
                raise ModelError(f"weight {name} has shape {tuple(t.shape)}, "
                                 f"expected {tuple(params[name].shape)}")
            params[name].copy_(t.to(params[name].dtype))
            loaded += 1
        if loaded != len(params):
            missing = sorted(set(params) - set(weights))
            raise ModelError(f"missing weights: {missing[:4]}")
        return loaded

    def bind_kv_cache(self, pool, reserved_slot: int = 0) -> None:
        """Bind every layer to its views of a ``KVCachePool`` (page 0 reserved)."""
        if pool.layout.num_layers != self.cfg.num_layers:
            raise ModelError("KV pool layer count does not match the model")
        for i, layer in enumerate(self.layers):
            kc, vc = pool.layer(i)
            layer.base_attention.bind_kv_cache(kc, vc)
            layer.base_attention.set_reserved_write_slot(reserved_slot)
        self.attention.bind_cache_layout(pool.layout.page_size)

    def check_write_errors(self) -> None:
        for layer in self.layers:
            layer.base_attention.check_write_errors()

    # ------------------------------------------------------------------ forward
    def forward(self, input_ids: torch.Tensor, positions: torch.Tensor,
                attention_batch: AttentionBatch, write_loc: torch.Tensor | None,
                logits_indices: torch.Tensor | None = None,
                logits_out: torch.Tensor | None = None) -> torch.Tensor:
        """Logits ``[N, vocab]`` for the selected rows (all rows when ``logits_indices`` is
        None). Safe to capture in a HIP graph: no host synchronisation happens inside."""
        cfg = self.cfg
        if input_ids.dim() != 1 or positions.shape != input_ids.shape:
            raise ModelError("input_ids and positions must have identical lengths")
        t = input_ids.size(0)
        hq, hkv, d = cfg.num_attention_heads, cfg.num_kv_heads, cfg.head_dim
        eps = cfg.rms_norm_eps
        hidden = F.embedding(input_ids, self.embed_tokens)
        residual = hidden
        x = ops.rms_norm(hidden, self.layers[0].input_layernorm, eps)
        n_layers = len(self.layers)
        for i, layer in enumerate(self.layers):
            qkv = ops.linear_qk_norm_rope_store(x, layer.qkv_proj, hq, hkv, layer.q_norm,
                                                layer.k_norm, eps, positions, self.rope,
                                                layer.base_attention, write_loc)
            q = qkv[:, : hq * d].view(t, hq, d)
            k = qkv[:, hq * d:(hq + hkv) * d].view(t, hkv, d)
            v = qkv[:, (hq + hkv) * d:].view(t, hkv, d)
            attn = attention_batch.forward(q, k, v, layer.base_attention)
            # o_proj + post-attention norm, down + the next layer's input norm (the final
            # norm after the last layer): each a projection fused with its residual RMSNorm.
            x, residual = ops.linear_add_rms_norm(attn, layer.o_proj, residual,
                                                  layer.post_attention_layernorm, eps)
            # gate_up with SiLU x mul (one launch for decode batches)
            act = ops.linear_silu_mul(x, layer.gate_up_proj)
            next_norm = self.layers[i + 1].input_layernorm if i + 1 < n_layers else self.norm
            x, residual = ops.linear_add_rms_norm(act, layer.down_proj, residual, next_norm, eps)
        hidden = x
        if logits_indices is not None:
            hidden = hidden.index_select(0, logits_indices)
        if logits_out is not None:
            torch.matmul(hidden, self.lm_head.t(), out=logits_out)
            return logits_out
        return F.linear(hidden, self.lm_head)


__all__ = ["Qwen3Config", "Qwen3Model", "Qwen3Layer"]
