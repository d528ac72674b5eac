"""Attention over a KV pool whose unowned slots hold NaN, with -1 past each block-table row.

A pool allocated with torch.empty, or pages freed by other requests, can hold any bit pattern,
NaN included. The reference reads only the slots a request owns (its length, page by page),
so a NaN in the unused tail of a request's last page, in a page no request owns, or a -1
block-table entry past its last page never reaches the result. Here every slot that no request
owns is NaN and every table entry past a request's pages is -1; decode (both kernels, split
requests included) and paged prefill must match the float64 oracle, which reads only the
owned slots, within the usual max-abs 2e-2 / cos 0.9999.
"""
import numpy as np
import pytest
import torch

from llm_infer_rust_amd.backend import Attention, AttentionMetadata, AttentionSpec, BatchPhase
from llm_infer_rust_amd.kv_cache import BaseAttention
from oracle import attention as oatt

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
MIN_COS = 0.9999
D = 128


def f32(t):
    return t.float().cpu().numpy()


def assert_close(got, want, what=""):
    got = np.asarray(got, np.float64).ravel()
    want = np.asarray(want, np.float64).ravel()
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    err = float(np.abs(got - want).max())
    cs = float(got @ want / (np.linalg.norm(got) * np.linalg.norm(want) + 1e-30))
    assert err <= MAX_ABS and cs > MIN_COS, f"{what} max_abs={err} cos={cs}"


def poisoned_pool(lens, page, hkv, g, rng, spare_pages=7):
    """NaN-filled K and V pools with each request's first `len` slots holding N(0,1) data on
    randomly permuted pages, page 0 and `spare_pages` unowned pages left NaN; block table
    padded with -1 past each request's pages."""
    pages_per = [(int(L) + page - 1) // page for L in lens]
    pool_pages = sum(pages_per) + 1 + spare_pages
    perm = rng.permutation(pool_pages - 1) + 1
    cols = max(pages_per) + 3
    table = np.full((len(lens), cols), -1, dtype=np.int32)
    kc = torch.full((pool_pages, page, hkv, D), float("nan"))
    vc = torch.full((pool_pages, page, hkv, D), float("nan"))
    off = 0
    for b, (L, npg) in enumerate(zip(lens, pages_per)):
        table[b, :npg] = perm[off: off + npg]
        off += npg
        for t in range(int(L)):
            p, s = table[b, t // page], t % page
            kc[p, s] = torch.randn(hkv, D, generator=g)
            vc[p, s] = torch.randn(hkv, D, generator=g)
    return kc, vc, table


@pytest.mark.parametrize("hq,page", [(16, 1), (16, 5), (32, 16), (32, 3)])
def test_decode_ignores_unowned_slots(gpu, hq, page):
    hkv = 8
    g = torch.Generator().manual_seed(hq * 10 + page)
    rng = np.random.default_rng(hq + page)
    lens = np.array([1, 17, 2900, 16, 333, 5000, 2], dtype=np.int32)
    kc, vc, table = poisoned_pool(lens, page, hkv, g, rng)
    q = torch.randn(len(lens), hq, D, generator=g)
    q, kc, vc = (t.to(torch.bfloat16).to(gpu) for t in (q, kc, vc))
    attn = Attention.new("mi355x", AttentionSpec(hq, hkv, D, torch.bfloat16, gpu))
    attn.bind_cache_layout(page)
    cache = BaseAttention()
    cache.bind_kv_cache(kc, vc)
    meta = AttentionMetadata(BatchPhase.DECODE, block_table=torch.from_numpy(table).to(gpu),
                             cache_seqlens=torch.from_numpy(lens).to(gpu))
    batch = attn.prepare(meta, len(lens))
    out = batch.forward(q, q, q, cache)
    want = oatt.decode_with_cache(f32(q), f32(kc), f32(vc), np.maximum(table, 0), lens, page)
    assert_close(f32(out).reshape(want.shape), want, f"decode hq={hq} page={page}")


@pytest.mark.parametrize("page", [16, 7])
def test_paged_prefill_ignores_unowned_slots(gpu, page):
    """Prefix and new tokens in the pool (the new tokens' K/V stored, as the model does before
    attention); the tail of each request's last page and every unowned page hold NaN."""
    hq, hkv = 32, 8
    g = torch.Generator().manual_seed(page)
    rng = np.random.default_rng(page)
    prefixes, extends = [100, 1, 1500], [20, 64, 3]
    lens = [p + e for p, e in zip(prefixes, extends)]
    kc, vc, table = poisoned_pool(lens, page, hkv, g, rng)
    bounds = [0] + np.cumsum(extends).tolist()
    n = bounds[-1]
    q = torch.randn(n, hq, D, generator=g)
    slots = [int(table[b, t // page]) * page + t % page
             for b, (p, e) in enumerate(zip(prefixes, extends)) for t in range(p, p + e)]
    k_new = kc.view(-1, hkv, D)[slots]
    v_new = vc.view(-1, hkv, D)[slots]
    q, k_new, v_new, kc, vc = (t.to(torch.bfloat16).to(gpu) for t in (q, k_new, v_new, kc, vc))
    attn = Attention.new("mi355x", AttentionSpec(hq, hkv, D, torch.bfloat16, gpu))
    attn.bind_cache_layout(page)
    cache = BaseAttention()
    cache.bind_kv_cache(kc, vc)
    meta = AttentionMetadata(BatchPhase.PREFILL,
                             cu_seqlens_q=torch.tensor(bounds, dtype=torch.int32, device=gpu),
                             prefix_lens=torch.tensor(prefixes, dtype=torch.int32, device=gpu),
                             block_table=torch.from_numpy(table).to(gpu))
    batch = attn.prepare(meta, n)
    out = batch.forward(q, k_new, v_new, cache)
    want = oatt.prefill_with_cache(f32(q), f32(kc), f32(vc), np.maximum(table, 0), bounds,
                                   prefixes, page)
    assert_close(f32(out).reshape(want.shape), want, f"paged prefill page={page}")
