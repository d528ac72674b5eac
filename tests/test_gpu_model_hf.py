"""The bf16 GPU Qwen3 model against Hugging Face `transformers`' logits (the fixtures of
`tests/golden/qwen3_hf_fixtures.npz`, float32 weights and arithmetic): a prompt prefill and
cached decode steps through the engine's own batch metadata, attention backend and KV pool.

The GPU model runs on the same weights rounded to bf16 with bf16 activations, so its logits
follow transformers' in direction (cos-sim > 0.999 per row) and within a few percent of the
largest logit; rows whose fp32 top-1/top-2 gap is wide must pick the same token.
"""
from pathlib import Path

import numpy as np
import pytest
import torch

from llm_infer_rust_amd.batch import BatchRequest, DecodeRequest
from llm_infer_rust_amd.engine import Engine, EngineConfig
from llm_infer_rust_amd.model import Qwen3Model
from oracle import bf16 as obf
from oracle import qwen3 as oq
from test_gpu_model_cached_routes import _decode, _prefill
from test_oracle_qwen3_hf import CASES, NORM_RANGE

pytestmark = pytest.mark.gpu

FIXTURES = Path(__file__).parent / "golden" / "qwen3_hf_fixtures.npz"


@pytest.mark.parametrize("name", ["tiny_untied", "tiny_tied_theta1e4"])
def test_gpu_model_matches_transformers(gpu, name):
    cfg, seed, std = CASES[name]
    with np.load(FIXTURES) as z:
        g = {k.split(".", 1)[1]: z[k] for k in z.files if k.startswith(name + ".")}
    w = {k: obf.round_bf16(v)
         for k, v in oq.random_weights(cfg, seed, std=std, norm_range=NORM_RANGE).items()}
    model = Qwen3Model(cfg, torch.bfloat16, gpu)
    assert model.load_weights({k: torch.from_numpy(v) for k, v in w.items()}) == len(w)
    page = 4
    eng = Engine(model, EngineConfig(page_size=page, max_running_req=2, max_seq_len=64,
                                     use_graphs=False))
    prompt, decode = g["prompt"], g["decode"]
    total = len(prompt) + len(decode)
    pages = list(range(1, -(-total // page) + 1))
    rows, _ = _prefill(eng, [BatchRequest(prompt, 0, len(prompt), pages)])
    got = [rows]
    length = len(prompt)
    for tok in decode:
        length += 1
        got.append(_decode(eng, [DecodeRequest(1, length, int(tok), pages)]))
    got = np.concatenate(got)
    want = g["logits"]
    assert got.shape == want.shape
    cos = (got * want).sum(1) / (np.linalg.norm(got, axis=1) * np.linalg.norm(want, axis=1))
    err = float(np.abs(got - want).max())
    scale = float(np.abs(want).max())
    print(f"{name}: cos min {cos.min():.6f} max|diff| {err:.4f} (|logit| max {scale:.3f})")
    assert cos.min() > 0.999
    assert err <= 0.03 * scale
    top2 = np.sort(want, axis=1)[:, -2:]
    wide = (top2[:, 1] - top2[:, 0]) > 4 * err
    np.testing.assert_array_equal(got.argmax(1)[wide], want.argmax(1)[wide])
