"""Seeded random sweeps of decode and prefill shapes against the float64 oracle.

Each case draws its head counts (GQA groups 1..8, kv-head counts that do and do not fill an
8-head or 4-head slice), page size, batch, lengths (including single-token rows and
requests that end mid-tile or mid-page), prefixes and dtype from a fixed seed, so the
kernels' dispatch paths (vector and matrix-core decode, ragged and paged prefill with
every head-group shape) are all exercised across edge positions. Tolerance as in the
per-kernel tests: max-abs <= 2e-2 and cosine similarity > 0.9999.
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
HEADS = [(8, 8), (16, 8), (32, 8), (64, 8), (16, 4), (32, 4), (4, 4), (24, 6), (4, 2), (8, 1)]
PAGES = [1, 2, 3, 8, 16, 32]


def f32(t):
    return t.float().cpu().numpy()


def assert_close(got, want, what):
    got = np.asarray(got, np.float64).ravel()
    want = np.asarray(want, np.float64).ravel()
    err = float(np.abs(got - want).max())
    cs = float(got @ want / (np.linalg.norm(got) * np.linalg.norm(want) + 1e-30))
    assert err <= MAX_ABS and cs > MIN_COS, f"{what} max_abs={err} cos={cs}"


def backend(gpu, hq, hkv, page, dtype):
    attn = Attention.new("mi355x", AttentionSpec(hq, hkv, 128, dtype, gpu))
    attn.bind_cache_layout(page)
    return attn


def page_table(rng, lengths, page):
    """Disjoint random pages per request (page 0 stays reserved)."""
    pages_per = [(int(n) + page - 1) // page for n in lengths]
    pool = sum(pages_per) + 1
    perm = rng.permutation(pool - 1) + 1
    table = np.zeros((len(lengths), max(pages_per)), np.int32)
    off = 0
    for r, n in enumerate(pages_per):
        table[r, :n] = perm[off: off + n]
        off += n
    return table, pool


@pytest.mark.parametrize("case", range(20))
def test_decode_sweep(gpu, case):
    rng = np.random.default_rng(1000 + case)
    g = torch.Generator().manual_seed(1000 + case)
    hq, hkv = HEADS[rng.integers(len(HEADS))]
    page = int(rng.choice(PAGES))
    dtype = torch.float16 if rng.random() < 0.3 else torch.bfloat16
    b = int(rng.choice([1, 3, 17, 64]))
    hi = int(rng.choice([1, 40, 700, 3000]))
    lengths = rng.integers(1, hi + 1, size=b).astype(np.int32)
    lengths[rng.integers(b)] = hi  # the longest request sets the table width
    table, pool = page_table(rng, lengths, page)
    kc = torch.randn(pool, page, hkv, 128, generator=g).to(dtype).to(gpu)
    vc = torch.randn(pool, page, hkv, 128, generator=g).to(dtype).to(gpu)
    q = torch.randn(b, hq, 128, generator=g).to(dtype).to(gpu)
    attn = backend(gpu, hq, hkv, page, dtype)
    cache = BaseAttention()
    cache.bind_kv_cache(kc, vc)
    meta = AttentionMetadata(BatchPhase.DECODE, block_table=torch.from_numpy(table).to(gpu),
                             cache_seqlens=torch.from_numpy(lengths).to(gpu))
    out = attn.prepare(meta, b).forward(q, q, q, cache)
    want = oatt.decode_with_cache(f32(q), f32(kc), f32(vc), table, lengths, page)
    assert_close(f32(out).reshape(want.shape), want,
                 f"case {case}: hq={hq} hkv={hkv} page={page} b={b} hi={hi} {dtype}")


@pytest.mark.parametrize("case", range(16))
def test_prefill_sweep(gpu, case):
    rng = np.random.default_rng(2000 + case)
    g = torch.Generator().manual_seed(2000 + case)
    hq, hkv = HEADS[rng.integers(len(HEADS))]
    if hq // hkv not in (1, 2, 4, 8):
        hq = hkv * 4
    dtype = torch.float16 if rng.random() < 0.3 else torch.bfloat16
    b = int(rng.integers(1, 7))
    ext = rng.integers(1, int(rng.choice([2, 70, 300])) + 1, size=b)
    paged = bool(rng.random() < 0.6)
    prefixes = (rng.integers(0, 600, size=b) * (rng.random(b) < 0.8)) if paged else np.zeros(b, int)
    if paged and not prefixes.any():
        prefixes[0] = 1
    bounds = [0] + np.cumsum(ext).tolist()
    n = bounds[-1]
    q = torch.randn(n, hq, 128, generator=g).to(dtype).to(gpu)
    meta_kw = dict(cu_seqlens_q=torch.tensor(bounds, dtype=torch.int32, device=gpu),
                   prefix_lens=torch.tensor(prefixes.tolist(), dtype=torch.int32, device=gpu))
    cache = BaseAttention()
    if paged:
        page = int(rng.choice(PAGES))
        table, pool = page_table(rng, prefixes + ext, page)
        kc = torch.randn(pool, page, hkv, 128, generator=g).to(dtype).to(gpu)
        vc = torch.randn(pool, page, hkv, 128, generator=g).to(dtype).to(gpu)
        cache.bind_kv_cache(kc, vc)
        k = v = q  # paged mode reads every key from the cache
    else:
        page = 16
        table = np.zeros((b, int(ext.max()) // page + 1), np.int32)
        k = torch.randn(n, hkv, 128, generator=g).to(dtype).to(gpu)
        v = torch.randn(n, hkv, 128, generator=g).to(dtype).to(gpu)
    attn = backend(gpu, hq, hkv, page, dtype)
    meta = AttentionMetadata(BatchPhase.PREFILL, block_table=torch.from_numpy(table).to(gpu),
                             **meta_kw)
    batch = attn.prepare(meta, n)
    assert batch.plan.plan.paged == paged
    out = batch.forward(q, k, v, cache)
    if paged:
        want = oatt.prefill_with_cache(f32(q), f32(kc), f32(vc), table, bounds,
                                       prefixes.tolist(), page)
    else:
        want = oatt.prefill_ragged(f32(q), f32(k), f32(v), bounds)
    assert_close(f32(out).reshape(want.shape), want,
                 f"case {case}: hq={hq} hkv={hkv} paged={paged} page={page} ext={ext.tolist()} "
                 f"prefixes={prefixes.tolist()} {dtype}")


@pytest.mark.parametrize("page", [64, 128])
def test_large_pages_decode_and_paged_prefill(gpu, page):
    """Pages of a whole prefill key tile (64) and larger (128, the general copy path), for
    decode and for paged prefill over cached prefixes (ending mid-page and on page borders)."""
    rng = np.random.default_rng(page)
    g = torch.Generator().manual_seed(page)
    hq, hkv, dtype = 32, 8, torch.bfloat16
    lengths = np.array([1, 63, 64, 65, 129, 700, 2 * page, 2000], np.int32)
    table, pool = page_table(rng, lengths, page)
    kc = torch.randn(pool, page, hkv, 128, generator=g).to(dtype).to(gpu)
    vc = torch.randn(pool, page, hkv, 128, generator=g).to(dtype).to(gpu)
    cache = BaseAttention()
    cache.bind_kv_cache(kc, vc)
    attn = backend(gpu, hq, hkv, page, dtype)
    b = lengths.size
    q = torch.randn(b, hq, 128, generator=g).to(dtype).to(gpu)
    meta = AttentionMetadata(BatchPhase.DECODE, block_table=torch.from_numpy(table).to(gpu),
                             cache_seqlens=torch.from_numpy(lengths).to(gpu))
    out = attn.prepare(meta, b).forward(q, q, q, cache)
    want = oatt.decode_with_cache(f32(q), f32(kc), f32(vc), table, lengths, page)
    assert_close(f32(out).reshape(want.shape), want, f"decode page={page}")
    # Paged prefill: the last `ext` tokens of each request are the new queries.
    ext = np.minimum(lengths, np.array([1, 5, 64, 1, 70, 33, 3, 130]))
    pref = lengths - ext
    bounds = [0] + np.cumsum(ext).tolist()
    n = bounds[-1]
    qp = torch.randn(n, hq, 128, generator=g).to(dtype).to(gpu)
    meta = AttentionMetadata(BatchPhase.PREFILL,
                             cu_seqlens_q=torch.tensor(bounds, dtype=torch.int32, device=gpu),
                             prefix_lens=torch.tensor(pref.tolist(), dtype=torch.int32, device=gpu),
                             block_table=torch.from_numpy(table).to(gpu))
    batch = attn.prepare(meta, n)
    assert batch.plan.plan.paged
    got = f32(batch.forward(qp, qp, qp, cache)).reshape(n, hq, 128)
    want = oatt.prefill_with_cache(f32(qp), f32(kc), f32(vc), table, bounds, pref, page)
    assert_close(got, want, f"prefill page={page}")
