"""The config-5 architecture (Qwen3-8B widths: hidden 4096, 32 q / 8 kv heads, FFN 12288,
vocab 151,936) through ``Qwen3Model`` and the serving ``Engine`` on hipGraph decode, at two
layers so the fp32 oracle stays fast.

* Teacher-forced logits of one request (prefill, then graph-replayed decode steps) against
  the fp32 Qwen3 oracle on the same bf16 weights: cos-sim and max-abs per step.
* A continuous batch of 64 requests with the benchmark's joint sampling (T 0.7, top-k 50,
  top-p 0.9): every drawn token lies in the reference's surviving set for its row
  (``sampling.rs:411-428`` restated by ``oracle.sampling.joint_keep``), every request emits
  exactly its token budget, and every KV page returns to the allocator.
"""
import dataclasses

import numpy as np
import pytest
import torch

from engine_helpers import RecordingEngine
from llm_infer_rust_amd.engine import EngineConfig
from llm_infer_rust_amd.model import Qwen3Config, Qwen3Model
from llm_infer_rust_amd.sampling import SamplingParams
from oracle import bf16 as obf
from oracle import qwen3 as oq
from oracle import sampling as osamp

pytestmark = pytest.mark.gpu

CFG = dataclasses.replace(Qwen3Config.qwen3_8b(), num_layers=2, max_position_embeddings=4096)


def weights_8b(seed: int, std: float = 0.02) -> dict[str, torch.Tensor]:
    """Seeded N(0, std) bf16 matrices (norm weights 1) with the Hugging Face names."""
    g = torch.Generator().manual_seed(seed)
    h, d, f, v = CFG.hidden_size, CFG.head_dim, CFG.intermediate_size, CFG.vocab_size
    qkv = CFG.qkv_width

    def mat(*shape):
        return (torch.randn(*shape, generator=g) * std).to(torch.bfloat16)

    w = {"model.embed_tokens.weight": mat(v, h), "lm_head.weight": mat(v, h),
         "model.norm.weight": torch.ones(h, dtype=torch.bfloat16)}
    for i in range(CFG.num_layers):
        p = f"model.layers.{i}."
        w[p + "input_layernorm.weight"] = torch.ones(h, dtype=torch.bfloat16)
        w[p + "self_attn.qkv_proj.weight"] = mat(qkv, h)
        w[p + "self_attn.q_norm.weight"] = torch.ones(d, dtype=torch.bfloat16)
        w[p + "self_attn.k_norm.weight"] = torch.ones(d, dtype=torch.bfloat16)
        w[p + "self_attn.o_proj.weight"] = mat(h, CFG.num_attention_heads * d)
        w[p + "post_attention_layernorm.weight"] = torch.ones(h, dtype=torch.bfloat16)
        w[p + "mlp.gate_up_proj.weight"] = mat(2 * f, h)
        w[p + "mlp.down_proj.weight"] = mat(h, f)
    return w


@pytest.fixture(scope="module")
def model8b(gpu):
    w = weights_8b(11)
    model = Qwen3Model(CFG, torch.bfloat16, gpu)
    assert model.load_weights(w) == len(w)
    yield model, w
    del model
    torch.cuda.empty_cache()


def test_8b_shape_teacher_forced_logits_match_oracle(model8b):
    model, w = model8b
    eng = RecordingEngine(model, EngineConfig(page_size=16, max_running_req=4, max_seq_len=256,
                                              graph_batch_sizes=(1, 2, 4)))
    prompt = np.random.default_rng(12).integers(0, CFG.vocab_size, 48)
    req = eng.add_request(prompt, SamplingParams(max_tokens=6))
    eng.run_until_complete()
    assert len(req.output) == 6 and eng.stats["graph_steps"] == eng.stats["decode_steps"] == 5
    oracle = oq.Qwen3Oracle(CFG, {k: v.float().numpy() for k, v in w.items()})
    want = [oracle.forward(prompt, 0)[-1]]
    pos = prompt.size
    for t in req.output[:-1]:
        want.append(oracle.forward(np.array([t]), pos)[-1])
        pos += 1
    exact = 0
    for step, ((uids, got, picked), ref) in enumerate(zip(eng.records, want)):
        assert uids == [req.uid]
        g = got[0].double().numpy()
        cos = float(g @ ref / (np.linalg.norm(g) * np.linalg.norm(ref)))
        err = float(np.abs(g - ref).max())
        print(f"step {step}: cos {cos:.6f} max-abs {err:.4f} (max |logit| "
              f"{float(np.abs(ref).max()):.3f})")
        assert cos > 0.999
        assert err < 0.05 * float(np.abs(ref).max()) + 0.02
        # Greedy: the engine's token is the oracle's argmax unless the oracle's own
        # top-1/top-2 gap is inside the measured logit error.
        deficit = float(ref.max() - ref[picked[0]])
        exact += int(deficit == 0.0)
        assert deficit <= 2 * err
    print(f"8B shape: {exact}/6 tokens are the oracle's exact argmax")


def test_8b_shape_continuous_batch_sampling_properties(model8b):
    model, _ = model8b
    n_req, n_in, n_out = 64, 96, 8
    eng = RecordingEngine(model, EngineConfig(page_size=16, max_running_req=64, max_seq_len=128,
                                              max_prefill_tokens_per_batch=2048, seed=2),
                          keep_rows=64)
    rng = np.random.default_rng(13)
    params = SamplingParams(temperature=0.7, top_k=50, top_p=0.9, max_tokens=n_out,
                            ignore_eos=True)
    reqs = [eng.add_request(rng.integers(0, CFG.vocab_size, n_in), params)
            for _ in range(n_req)]
    eng.run_until_complete()
    assert eng.stats["prefill_batches"] >= 3  # 6144 prompt tokens over a 2048-token budget
    assert eng.stats["graph_steps"] == eng.stats["decode_steps"] > 0
    assert all(len(r.output) == n_out for r in reqs)
    assert len(eng.pages.free) == eng.pool.layout.num_pages
    checked = 0
    for uids, logits, picked in eng.records:
        for i in range(0, len(uids), 4):  # every 4th row of every draw
            t = int(picked[i])
            assert 0 <= t < CFG.vocab_size
            s = osamp.scaled_logits(logits[i].numpy(), 0.7, obf.round_bf16)
            keep = osamp.joint_keep(s, 50, 0.9)
            assert keep[t], (uids[i], t)
            checked += 1
    print(f"checked {checked} draws against the joint top-k/top-p survivors")
    assert checked >= n_req * n_out // 4
