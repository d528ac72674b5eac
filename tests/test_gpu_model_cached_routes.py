"""Cached, chunked and mixed batches against one full forward, at the model level.

Mirrors the reference's `paged_decode_and_cached_prefix_prefill_match_full_forward`
(`src/models/qwen3/model.rs:730-900`): one sequence is run as a cold prefill of every token
(the "full" forward), then through the KV cache along the routes that test takes -- a prefill
of the first part, one decode step, a cached-prefix prefill of the rest; the same sequence as
three chunks; a second request prefilled on other pages and then a mixed batch of the first
request's middle chunk with the second request's decode row (the reference's
`prepare_mixed_prefill` layout: a decode row is a one-token prefill row over its cache) --
and each route's logits must equal the full forward's rows. The reference compares fp32 CPU
paths within 1e-5; here both sides are the bf16 GPU path, so the rows agree to bf16
rounding of differently ordered sums, and the full forward itself is held against the fp32
oracle.
"""
import numpy as np
import pytest
import torch

from llm_infer_rust_amd.backend import AttentionMetadata, BatchPhase, DecodeHostMetadata
from llm_infer_rust_amd.batch import BatchRequest, DecodeRequest
from llm_infer_rust_amd.engine import Engine, EngineConfig
from test_gpu_model import TINY, build

pytestmark = pytest.mark.gpu


def _prefill(eng, rows):
    model = eng.model
    b = eng.batches.prepare_prefill(rows)
    ids_d, pos_d, loc_d, cu_d, pre_d, tab_d = eng._upload(
        b.input_ids, b.positions, b.write_loc, b.cu_seqlens_q, b.prefix_lens, b.block_table)
    meta = AttentionMetadata(BatchPhase.PREFILL, write_loc=loc_d, cu_seqlens_q=cu_d,
                             prefix_lens=pre_d, block_table=tab_d,
                             host_cu_seqlens_q=b.cu_seqlens_q.tolist(),
                             host_prefix_lens=b.prefix_lens.tolist())
    batch = model.attention.prepare(meta, len(b.input_ids))
    out = model.forward(ids_d, pos_d, batch, loc_d).float().cpu().numpy()
    model.check_write_errors()
    return out, out[b.logits_indices]


def _decode(eng, reqs):
    model = eng.model
    b = eng.tables.prepare(reqs)
    ids_d, pos_d, loc_d, lens_d, table_d = eng._upload(
        b.input_ids, b.positions, b.write_loc, b.cache_seqlens, b.block_table)
    meta = AttentionMetadata(BatchPhase.DECODE,
                             decode_host=DecodeHostMetadata(b.cache_seqlens.tolist()),
                             write_loc=loc_d, block_table=table_d, cache_seqlens=lens_d)
    batch = model.attention.prepare(meta, len(reqs))
    out = model.forward(ids_d, pos_d, batch, loc_d).float().cpu().numpy()
    model.check_write_errors()
    return out


def _close(got, want, what):
    got, want = np.atleast_2d(got), np.atleast_2d(want)
    cos = (got * want).sum(1) / (np.linalg.norm(got, axis=1) * np.linalg.norm(want, axis=1))
    err = float(np.abs(got - want).max())
    scale = float(np.abs(want).max())
    print(f"{what}: cos {cos.min():.7f} max|diff| {err:.4g} (|logit| max {scale:.3g})")
    # Routes through different kernels (decode vs prefill attention, the decode-batch GEMM
    # vs hipBLASLt) round bf16 intermediates differently over the layers: the north star's
    # attention tolerance (cos-sim > 0.9999) and 1% of the largest logit.
    assert cos.min() > 0.9999, what
    assert err <= 1e-2 * scale + 4e-3, what


@pytest.mark.parametrize("length,page", [(4, 2), (100, 16), (150, 3)])
def test_cached_chunked_and_mixed_routes_match_full_forward(gpu, length, page):
    model, oracle = build(TINY, 11, gpu)
    eng = Engine(model, EngineConfig(page_size=page, max_running_req=2, max_seq_len=256,
                                     use_graphs=False))
    seq = np.random.default_rng(length).integers(0, TINY.vocab_size, length)
    need = -(-length // page)
    pages1 = list(range(1, need + 1))                 # page 0 is the pool's reserved page
    pages2 = list(range(need + 1, 2 * need + 1))

    full, _ = _prefill(eng, [BatchRequest(seq, 0, length, pages1)])
    want = oracle.forward(seq, 0)
    cos = (full * want).sum(1) / (np.linalg.norm(full, axis=1) * np.linalg.norm(want, axis=1))
    assert cos.min() > 0.999 and np.abs(full - want).max() < 0.05 * np.abs(want).max() + 0.02

    # Prefill of the first half, one decode step, cached-prefix prefill of the rest.
    a = length // 2
    _, last = _prefill(eng, [BatchRequest(seq, 0, a, pages1)])
    _close(last, full[a - 1], "prefill(0, a)")
    got = _decode(eng, [DecodeRequest(1, a + 1, int(seq[a]), pages1)])
    _close(got, full[a], "decode at a")
    _, last = _prefill(eng, [BatchRequest(seq, a + 1, length, pages1)])
    _close(last, full[length - 1], "prefill(a + 1, L) over the cache")

    # The same sequence as three chunks, then as one cold prefill.
    c1, c2 = max(1, length // 4), (3 * length) // 4
    for lo, hi in ((0, c1), (c1, c2), (c2, length)):
        _, last = _prefill(eng, [BatchRequest(seq, lo, hi, pages1)])
        _close(last, full[hi - 1], f"chunk ({lo}, {hi})")
    _, last = _prefill(eng, [BatchRequest(seq, 0, length, pages1)])
    _close(last, full[length - 1], "cold prefill")

    # A second request on other pages, then its decode row mixed with a middle chunk of
    # the first request in one prefill batch.
    _, last = _prefill(eng, [BatchRequest(seq[:length - 1], 0, length - 1, pages2)])
    _close(last, full[length - 2], "second request prefill")
    _, last = _prefill(eng, [BatchRequest(seq, c1, c2, pages1),
                             BatchRequest(seq, length - 1, length, pages2)])
    _close(last, full[[c2 - 1, length - 1]], "mixed chunk + decode row")
