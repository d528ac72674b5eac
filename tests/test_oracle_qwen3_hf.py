"""The Qwen3 oracle's layer composition against Hugging Face `transformers` (CPU only).

`tests/golden/qwen3_hf_fixtures.npz` holds logits that `transformers.Qwen3ForCausalLM`
(float32, eager attention) computed on seeded random weights; the script beside it wrote them.
Here `oracle.qwen3.Qwen3Oracle` rebuilds the same weights from the seed and runs the same prompt
and cached decode steps (the reference composition, src/models/qwen3/model.rs:424-534). This
pins what the reference's own cached == full invariant (model.rs:730-900) cannot: the order of
QK-norm and RoPE, which residual feeds each norm, the rope_theta in use, tied and untied heads.

The mutation tests check that plausible composition mistakes fail the same comparison.
"""
from pathlib import Path

import numpy as np
import pytest

from llm_infer_rust_amd.model import Qwen3Config
from oracle import layer_ops, norms
from oracle import qwen3 as oq

FIXTURES = Path(__file__).parent / "golden" / "qwen3_hf_fixtures.npz"
# fp32 logits: at most this far from transformers' (two fp32 evaluations of the same sums).
ATOL = 1e-4

CASES = {
    "tiny_untied": (Qwen3Config(hidden_size=256, num_layers=2, num_attention_heads=4,
                                num_kv_heads=2, intermediate_size=512, vocab_size=300,
                                head_dim=128, max_position_embeddings=256,
                                rope_theta=1_000_000.0, tie_word_embeddings=False), 11, 0.05),
    "tiny_tied_theta1e4": (Qwen3Config(hidden_size=384, num_layers=3, num_attention_heads=8,
                                       num_kv_heads=2, intermediate_size=640, vocab_size=320,
                                       head_dim=128, max_position_embeddings=256,
                                       rope_theta=10_000.0, tie_word_embeddings=True), 12, 0.05),
    "qwen3_0_6b_widths_2_layers": (
        Qwen3Config(**{**Qwen3Config.qwen3_0_6b().__dict__, "num_layers": 2}), 13, 0.02),
}
NORM_RANGE = (0.5, 1.5)


@pytest.fixture(scope="module")
def fixtures():
    with np.load(FIXTURES) as z:
        return {k: z[k] for k in z.files}


def oracle_logits(model: oq.Qwen3Oracle, prompt, decode):
    rows = [model.forward(prompt, 0)]
    pos = len(prompt)
    for tok in decode:
        rows.append(model.forward(np.array([tok]), pos))
        pos += 1
    return np.concatenate(rows)


def case_inputs(fixtures, name):
    return {k.split(".", 1)[1]: v for k, v in fixtures.items() if k.startswith(name + ".")}


def compare(name, fixtures, model_cls=oq.Qwen3Oracle, cfg=None, weights=None):
    base_cfg, seed, std = CASES[name]
    cfg = cfg or base_cfg
    w = weights if weights is not None else oq.random_weights(base_cfg, seed, std=std,
                                                             norm_range=NORM_RANGE)
    g = case_inputs(fixtures, name)
    got = oracle_logits(model_cls(cfg, w), g["prompt"], g["decode"])
    argmax = got.argmax(1)
    if "columns" in g:
        got = got[:, g["columns"]]
    return got, argmax, g


@pytest.mark.parametrize("name", list(CASES))
def test_oracle_matches_transformers_qwen3(name, fixtures):
    got, argmax, g = compare(name, fixtures)
    want = g["logits"]
    assert got.shape == want.shape
    err = float(np.abs(got - want).max())
    scale = float(np.abs(want).max())
    print(f"{name}: max_abs {err:.2e} (logit scale {scale:.2f})")
    assert err <= ATOL
    # The full-vocabulary argmax of every row too (sampled columns hold only part of it).
    np.testing.assert_array_equal(argmax, g["argmax"])


class RopeBeforeNorm(oq.Qwen3Oracle):
    """Mutation: RoPE applied before QK-norm."""

    def forward(self, ids, start, last_only=False):
        real_rope, real_rms = layer_ops.rope, oq._rms

        # RoPE moves into the norm of the q/k head rows (the 3-D inputs), ahead of it.
        def rms_rope_first(x, w, eps):
            if x.ndim == 3:
                pos = start + np.arange(x.shape[0])
                x = real_rope(x, pos, self.cos, self.sin)
            return real_rms(x, w, eps)

        def no_rope(x, pos, cos, sin):
            return x

        oq._rms, layer_ops.rope = rms_rope_first, no_rope
        try:
            return super().forward(ids, start, last_only)
        finally:
            oq._rms, layer_ops.rope = real_rms, real_rope


class PostNormOnAttentionOutput(oq.Qwen3Oracle):
    """Mutation: post_attention_layernorm fed the attention output alone (residual dropped
    from the sum that is normalised)."""

    def forward(self, ids, start, last_only=False):
        real = norms.add_rms_norm_f32
        state = {"n": 0}

        def add_rms(x, r, w, eps):
            state["n"] += 1
            y, s = real(x, r, w, eps)
            if state["n"] % 2 == 0:  # the second add_rms of each layer is the post-attn one
                y = norms.rms_norm_f32(x, w, eps)
            return y, s

        norms.add_rms_norm_f32 = add_rms
        try:
            return super().forward(ids, start, last_only)
        finally:
            norms.add_rms_norm_f32 = real


def test_mutation_wrong_rope_theta_fails(fixtures):
    cfg, seed, std = CASES["tiny_tied_theta1e4"]
    wrong = Qwen3Config(**{**cfg.__dict__, "rope_theta": 1_000_000.0})
    got, _, g = compare("tiny_tied_theta1e4", fixtures, cfg=wrong)
    assert np.abs(got - g["logits"]).max() > 100 * ATOL


def test_mutation_rope_before_qk_norm_fails(fixtures):
    got, _, g = compare("tiny_untied", fixtures, model_cls=RopeBeforeNorm)
    assert np.abs(got - g["logits"]).max() > 100 * ATOL


def test_mutation_post_attention_norm_without_residual_fails(fixtures):
    got, _, g = compare("tiny_untied", fixtures, model_cls=PostNormOnAttentionOutput)
    assert np.abs(got - g["logits"]).max() > 100 * ATOL


def test_mutation_untied_head_read_as_tied_fails(fixtures):
    cfg, seed, std = CASES["tiny_untied"]
    tied = Qwen3Config(**{**cfg.__dict__, "tie_word_embeddings": True})
    got, _, g = compare("tiny_untied", fixtures, cfg=tied)
    assert np.abs(got - g["logits"]).max() > 100 * ATOL
