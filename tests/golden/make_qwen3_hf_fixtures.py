"""Writes qwen3_hf_fixtures.npz: Qwen3 logits from Hugging Face `transformers`' own Qwen3
architecture (an implementation independent of this repository's reading of
src/models/qwen3/model.rs:424-534), on seeded random weights.

Each case builds the weights with `oracle.qwen3.random_weights` (seeded numpy, norm weights
drawn from U(0.5, 1.5) so a misplaced or swapped norm changes the output), loads them into
`transformers.Qwen3ForCausalLM` in float32 with eager attention, and records the logits of a
prompt forward plus a few cached decode steps (`past_key_values`). The test that reads the
file rebuilds the same weights from the seed, so only ids and logits are stored.

Cases: two tiny shapes (untied embeddings / rope_theta 1e6 / GQA group 2; tied / rope_theta
1e4 / group 4 / 3 layers) with every logit stored, and 2 layers at the Qwen3-0.6B widths
(hidden 1024, 16 / 8 heads, FFN 3072, vocab 151,936, tied, rope_theta 1e6) with 512 sampled
vocabulary columns of every row plus each row's argmax and maximum.

Run: python tests/golden/make_qwen3_hf_fixtures.py   (CPU, about a minute)
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from llm_infer_rust_amd.model import Qwen3Config  # noqa: E402
from oracle import qwen3 as oq  # noqa: E402

OUT = Path(__file__).with_name("qwen3_hf_fixtures.npz")

CASES = {
    "tiny_untied": dict(
        cfg=Qwen3Config(hidden_size=256, num_layers=2, num_attention_heads=4, num_kv_heads=2,
                        intermediate_size=512, vocab_size=300, head_dim=128,
                        max_position_embeddings=256, rope_theta=1_000_000.0,
                        tie_word_embeddings=False),
        seed=11, std=0.05, prompt=13, steps=4, columns=None),
    "tiny_tied_theta1e4": dict(
        cfg=Qwen3Config(hidden_size=384, num_layers=3, num_attention_heads=8, num_kv_heads=2,
                        intermediate_size=640, vocab_size=320, head_dim=128,
                        max_position_embeddings=256, rope_theta=10_000.0,
                        tie_word_embeddings=True),
        seed=12, std=0.05, prompt=21, steps=3, columns=None),
    "qwen3_0_6b_widths_2_layers": dict(
        cfg=Qwen3Config(**{**Qwen3Config.qwen3_0_6b().__dict__, "num_layers": 2}),
        seed=13, std=0.02, prompt=16, steps=3, columns=512),
}
NORM_RANGE = (0.5, 1.5)


def hf_model(cfg: Qwen3Config, w: dict[str, np.ndarray]):
    from transformers import Qwen3Config as HFConfig
    from transformers import Qwen3ForCausalLM

    hc = HFConfig(vocab_size=cfg.vocab_size, hidden_size=cfg.hidden_size,
                  intermediate_size=cfg.intermediate_size, num_hidden_layers=cfg.num_layers,
                  num_attention_heads=cfg.num_attention_heads,
                  num_key_value_heads=cfg.num_kv_heads, head_dim=cfg.head_dim,
                  max_position_embeddings=cfg.max_position_embeddings,
                  rope_theta=cfg.rope_theta, rms_norm_eps=cfg.rms_norm_eps,
                  tie_word_embeddings=cfg.tie_word_embeddings, attention_bias=False,
                  use_sliding_window=False, attn_implementation="eager",
                  torch_dtype=torch.float32)
    m = Qwen3ForCausalLM(hc).float().eval()
    hq, hkv, d, f = cfg.num_attention_heads, cfg.num_kv_heads, cfg.head_dim, cfg.intermediate_size
    sd = {"model.embed_tokens.weight": w["model.embed_tokens.weight"],
          "model.norm.weight": w["model.norm.weight"]}
    sd["lm_head.weight"] = w.get("lm_head.weight", w["model.embed_tokens.weight"])
    for i in range(cfg.num_layers):
        p = f"model.layers.{i}."
        qkv = w[p + "self_attn.qkv_proj.weight"]
        sd[p + "self_attn.q_proj.weight"] = qkv[: hq * d]
        sd[p + "self_attn.k_proj.weight"] = qkv[hq * d:(hq + hkv) * d]
        sd[p + "self_attn.v_proj.weight"] = qkv[(hq + hkv) * d:]
        gu = w[p + "mlp.gate_up_proj.weight"]
        sd[p + "mlp.gate_proj.weight"] = gu[:f]
        sd[p + "mlp.up_proj.weight"] = gu[f:]
        for name in ("self_attn.o_proj", "self_attn.q_norm", "self_attn.k_norm",
                     "input_layernorm", "post_attention_layernorm", "mlp.down_proj"):
            sd[p + name + ".weight"] = w[p + name + ".weight"]
    sd = {k: torch.from_numpy(np.ascontiguousarray(v)) for k, v in sd.items()}
    missing, unexpected = m.load_state_dict(sd, strict=False)
    assert not unexpected, unexpected
    assert set(missing) <= {"lm_head.weight"}, missing
    return m


def run_case(spec) -> dict[str, np.ndarray]:
    cfg = spec["cfg"]
    w = oq.random_weights(cfg, spec["seed"], std=spec["std"], norm_range=NORM_RANGE)
    rng = np.random.default_rng(spec["seed"] + 100)
    prompt = rng.integers(0, cfg.vocab_size, spec["prompt"])
    decode = rng.integers(0, cfg.vocab_size, spec["steps"])
    m = hf_model(cfg, w)
    rows = []
    with torch.no_grad():
        out = m(input_ids=torch.from_numpy(prompt)[None], use_cache=True)
        rows.append(out.logits[0].numpy())
        past = out.past_key_values
        for tok in decode:
            out = m(input_ids=torch.tensor([[int(tok)]]), past_key_values=past, use_cache=True)
            past = out.past_key_values
            rows.append(out.logits[0].numpy())
    logits = np.concatenate(rows).astype(np.float32)
    rec = {"prompt": prompt.astype(np.int64), "decode": decode.astype(np.int64),
           "argmax": logits.argmax(1).astype(np.int64), "max": logits.max(1)}
    if spec["columns"] is None:
        rec["logits"] = logits
    else:
        cols = np.sort(rng.choice(cfg.vocab_size, spec["columns"], replace=False))
        rec["columns"] = cols.astype(np.int64)
        rec["logits"] = np.ascontiguousarray(logits[:, cols])
    return rec


def main() -> None:
    torch.manual_seed(0)
    arrays = {}
    for name, spec in CASES.items():
        for key, val in run_case(spec).items():
            arrays[f"{name}.{key}"] = val
        print(name, "done", flush=True)
    np.savez_compressed(OUT, **arrays)
    print("wrote", OUT)


if __name__ == "__main__":
    main()
