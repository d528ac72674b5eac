"""Ragged and paged causal prefill through the C ABI against the oracle.

Tolerance (every case): max-abs <= 2e-2 and cosine similarity > 0.9999 against
the float64 oracle on the same rounded inputs (the reference itself allows
0.03125, backend.rs:1846). Paged page metadata is compared bit-exactly.
"""
import numpy as np
import pytest
import torch

from llm_infer_rust_amd.backend import (Attention, AttentionMetadata, AttentionSpec, BatchPhase,
                                        ModelError)
from llm_infer_rust_amd.kv_cache import BaseAttention
from oracle import attention as oatt
from oracle import plan as oplan

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
MIN_COS = 0.9999


def f32(t):
    return t.float().cpu().numpy()


def assert_close(got, want, what=""):
    got = np.asarray(got, np.float64).ravel()
    want = np.asarray(want, np.float64).ravel()
    err = float(np.abs(got - want).max())
    cs = float(got @ want / (np.linalg.norm(got) * np.linalg.norm(want) + 1e-30))
    assert err <= MAX_ABS and cs > MIN_COS, f"{what} max_abs={err} cos={cs}"


def randn(shape, g, dtype, gpu):
    return torch.randn(*shape, generator=g).to(dtype).to(gpu)


def make(gpu, hq, hkv, page, dtype):
    attn = Attention.new("mi355x", AttentionSpec(hq, hkv, 128, dtype, gpu))
    attn.bind_cache_layout(page)
    return attn


def meta_for(gpu, bounds, prefixes, table):
    return AttentionMetadata(BatchPhase.PREFILL,
                             cu_seqlens_q=torch.tensor(bounds, dtype=torch.int32, device=gpu),
                             prefix_lens=torch.tensor(prefixes, dtype=torch.int32, device=gpu),
                             block_table=table)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_reference_ragged_and_cached_cases(gpu, fixtures, dtype):
    fx = fixtures["prefill_cases"]
    g = torch.Generator().manual_seed(5)
    attn = make(gpu, 16, 8, fx["page_size"], dtype)
    kc = randn(fx["cache_shape"], g, dtype, gpu)
    vc = randn(fx["cache_shape"], g, dtype, gpu)
    cache = BaseAttention()
    cache.bind_kv_cache(kc, vc)
    table = torch.arange(64, dtype=torch.int32, device=gpu).view(2, 32)
    for lengths, prefixes in fx["cases"]:
        bounds = [0, lengths[0], lengths[0] + lengths[1]]
        n = bounds[-1]
        packed = randn((n, fx["packed_width"]), g, dtype, gpu)
        q = packed[:, :2048].view(-1, 16, 128)
        k = packed[:, 2048:3072].view(-1, 8, 128)
        v = packed[:, 3072:].view(-1, 8, 128)
        batch = attn.prepare(meta_for(gpu, bounds, prefixes, table), n)
        plan = batch.plan.plan
        paged = any(p > 0 for p in prefixes)
        assert plan.paged == paged
        actual = batch.forward(q, k, v, cache)
        storage = torch.full((n + 3, 2048), 99.0, dtype=dtype, device=gpu)
        target = storage[:n]
        ptr = target.data_ptr()
        batch.forward_into(q, k, v, cache, target)
        assert target.data_ptr() == ptr and torch.equal(actual, target)
        assert bool((storage[n:] == 99.0).all())
        if paged:
            want = oatt.prefill_with_cache(f32(q), f32(kc), f32(vc), table.cpu().numpy(), bounds,
                                           prefixes, fx["page_size"])
            md = plan.read_metadata()
            _, indptr, indices, last = oplan.prefill_page_metadata(
                table.cpu().numpy(), bounds, prefixes, fx["page_size"])
            assert md["kv_indptr"] == indptr.tolist()
            assert md["indices"] == indices.tolist()
            assert md["last_page_len"] == last.tolist()
        else:
            want = oatt.prefill_ragged(f32(q), f32(k), f32(v), bounds)
        assert_close(f32(actual).reshape(want.shape), want, f"{lengths} {prefixes} {dtype}")
        del batch


@pytest.mark.parametrize("hq,hkv", [(16, 16), (32, 8), (64, 8), (4, 2)])
def test_ragged_gqa_groups(gpu, hq, hkv):
    g = torch.Generator().manual_seed(hq + hkv)
    bounds = [0, 1, 70, 200, 333, 334]
    n = bounds[-1]
    q = randn((n, hq, 128), g, torch.bfloat16, gpu)
    k = randn((n, hkv, 128), g, torch.bfloat16, gpu)
    v = randn((n, hkv, 128), g, torch.bfloat16, gpu)
    attn = make(gpu, hq, hkv, 16, torch.bfloat16)
    table = torch.zeros(len(bounds) - 1, 32, dtype=torch.int32, device=gpu)
    batch = attn.prepare(meta_for(gpu, bounds, [0] * (len(bounds) - 1), table), n)
    out = batch.forward(q, k, v, BaseAttention())
    want = oatt.prefill_ragged(f32(q), f32(k), f32(v), bounds)
    assert_close(f32(out).reshape(want.shape), want, f"hq={hq} hkv={hkv}")


def test_config3_ragged_shape(gpu):
    """8 sequences, lengths U[256,2048], Hq16/Hkv8, packed QKV stride 4096."""
    rng = np.random.default_rng(3)
    g = torch.Generator().manual_seed(3)
    lens = rng.integers(256, 2049, size=8)
    bounds = [0] + np.cumsum(lens).tolist()
    n = bounds[-1]
    packed = randn((n, 4096), g, torch.bfloat16, gpu)
    q = packed[:, :2048].view(-1, 16, 128)
    k = packed[:, 2048:3072].view(-1, 8, 128)
    v = packed[:, 3072:].view(-1, 8, 128)
    attn = make(gpu, 16, 8, 16, torch.bfloat16)
    table = torch.zeros(8, 2048 // 16, dtype=torch.int32, device=gpu)
    batch = attn.prepare(meta_for(gpu, bounds, [0] * 8, table), n)
    assert batch.plan.plan.info()["split_items"] == 0  # enough items to fill the device
    out = batch.forward(q, k, v, BaseAttention())
    want = oatt.prefill_ragged(f32(q), f32(k), f32(v), bounds)
    assert_close(f32(out).reshape(want.shape), want, "config3")


def test_config4_paged_shape_sampled_rows(gpu):
    """16 requests, prefix U[1024,8192] over a random page permutation, extend U[64,512],
    Hq32/Hkv8, page 16. The oracle checks 12 query rows per request (first, last, random)."""
    rng = np.random.default_rng(4)
    g = torch.Generator().manual_seed(4)
    page = 16
    pref = rng.integers(1024, 8193, size=16)
    ext = rng.integers(64, 513, size=16)
    bounds = [0] + np.cumsum(ext).tolist()
    pages_per = (pref + ext + page - 1) // page
    cols = int(pages_per.max())
    total_pages = int(pages_per.sum())
    pool = total_pages + 1
    perm = rng.permutation(pool - 1) + 1
    table = np.zeros((16, cols), np.int32)
    off = 0
    for r in range(16):
        table[r, : pages_per[r]] = perm[off: off + pages_per[r]]
        off += pages_per[r]
    kc = randn((pool, page, 8, 128), g, torch.bfloat16, gpu)
    vc = randn((pool, page, 8, 128), g, torch.bfloat16, gpu)
    n = bounds[-1]
    q = randn((n, 32, 128), g, torch.bfloat16, gpu)
    attn = make(gpu, 32, 8, page, torch.bfloat16)
    cache = BaseAttention()
    cache.bind_kv_cache(kc, vc)
    tdev = torch.from_numpy(table).to(gpu)
    batch = attn.prepare(meta_for(gpu, bounds, pref.tolist(), tdev), n)
    assert batch.plan.plan.paged and batch.plan.plan.info()["split_items"] == 0
    out = f32(batch.forward(q, q, q, cache)).reshape(n, 32, 128)
    kcf, vcf, qf = f32(kc), f32(vc), f32(q)
    flat_k = kcf.reshape(-1, 8, 128)
    flat_v = vcf.reshape(-1, 8, 128)
    for r in range(16):
        e = int(ext[r])
        rows = sorted(set([0, e - 1] + rng.integers(0, e, size=10).tolist()))
        for i in rows:
            horizon = int(pref[r]) + i + 1
            slots = oatt.slots_of(table[r], horizon, page)
            want = oatt.attention_against_cache(qf[bounds[r] + i: bounds[r] + i + 1],
                                                flat_k[slots], flat_v[slots], horizon - 1, 32, 8)
            assert_close(out[bounds[r] + i], want[0], f"req={r} row={i}")


def test_prefill_plan_reuse_and_errors(gpu):
    attn = make(gpu, 16, 8, 16, torch.bfloat16)
    table = torch.arange(64, dtype=torch.int32, device=gpu).view(2, 32)
    batch = attn.prepare(meta_for(gpu, [0, 17, 18], [0, 0], table), 18)
    handle = batch.plan.plan.handle
    with pytest.raises(ModelError, match="still in use"):
        attn.prepare(meta_for(gpu, [0, 17, 18], [0, 0], table), 18)
    del batch
    batch = attn.prepare(meta_for(gpu, [0, 1, 18], [255, 16], table), 18)
    assert batch.plan.plan.handle == handle and batch.plan.plan.paged
    del batch
    with pytest.raises(ModelError, match="too small"):
        attn.prepare(meta_for(gpu, [0, 1, 2], [600, 0], table), 2)


@pytest.mark.parametrize("hq,hkv", [(16, 8), (32, 8), (8, 8)])
def test_ragged_mixed_tiny_and_long_sequences(gpu, hq, hkv):
    """One- and two-token sequences, sequences ending exactly on and just past a 64-key
    tile or a query block, and longer ones in one batch (every row checked)."""
    g = torch.Generator().manual_seed(100 + hq)
    lens = [1, 64, 65, 2, 127, 128, 129, 300, 5, 33, 640, 1, 96, 200]
    bounds = [0] + np.cumsum(lens).tolist()
    n = bounds[-1]
    q = randn((n, hq, 128), g, torch.bfloat16, gpu)
    k = randn((n, hkv, 128), g, torch.bfloat16, gpu)
    v = randn((n, hkv, 128), g, torch.bfloat16, gpu)
    attn = make(gpu, hq, hkv, 16, torch.bfloat16)
    table = torch.zeros(len(lens), 64, dtype=torch.int32, device=gpu)
    batch = attn.prepare(meta_for(gpu, bounds, [0] * len(lens), table), n)
    out = batch.forward(q, k, v, BaseAttention())
    want = oatt.prefill_ragged(f32(q), f32(k), f32(v), bounds)
    assert_close(f32(out).reshape(want.shape), want, f"hq={hq} hkv={hkv}")


@pytest.mark.parametrize("seed", [1, 5])
def test_paged_small_prefixes_and_tiny_extends(gpu, seed):
    """Paged prefill with prefixes of 0 to a few pages (ending on and off page borders)
    and extends of 1 to 130 tokens (page 16, Hq32/Hkv8, random page permutation); every
    row checked."""
    rng = np.random.default_rng(seed)
    g = torch.Generator().manual_seed(seed)
    page = 16
    pref = np.array([0, 1, 15, 16, 63, 64, 200, 0, 31, 500])
    ext = np.array([1, 1, 2, 70, 1, 64, 33, 130, 3, 1])
    bounds = [0] + np.cumsum(ext).tolist()
    pages_per = (pref + ext + page - 1) // page
    cols = int(pages_per.max())
    pool = int(pages_per.sum()) + 1
    perm = rng.permutation(pool - 1) + 1
    table = np.zeros((len(ext), cols), np.int32)
    off = 0
    for r in range(len(ext)):
        table[r, : pages_per[r]] = perm[off: off + pages_per[r]]
        off += pages_per[r]
    kc = randn((pool, page, 8, 128), g, torch.bfloat16, gpu)
    vc = randn((pool, page, 8, 128), g, torch.bfloat16, gpu)
    n = bounds[-1]
    q = randn((n, 32, 128), g, torch.bfloat16, gpu)
    attn = make(gpu, 32, 8, page, torch.bfloat16)
    cache = BaseAttention()
    cache.bind_kv_cache(kc, vc)
    batch = attn.prepare(meta_for(gpu, bounds, pref.tolist(), torch.from_numpy(table).to(gpu)), n)
    assert batch.plan.plan.paged
    out = f32(batch.forward(q, q, q, cache)).reshape(n, 32, 128)
    flat_k = f32(kc).reshape(-1, 8, 128)
    flat_v = f32(vc).reshape(-1, 8, 128)
    qf = f32(q)
    for r in range(len(ext)):
        for i in range(int(ext[r])):
            horizon = int(pref[r]) + i + 1
            slots = oatt.slots_of(table[r], horizon, page)
            want = oatt.attention_against_cache(qf[bounds[r] + i: bounds[r] + i + 1],
                                                flat_k[slots], flat_v[slots], horizon - 1, 32, 8)
            assert_close(out[bounds[r] + i], want[0], f"seed={seed} req={r} row={i}")


@pytest.mark.parametrize("dtype,page", [(torch.bfloat16, 16), (torch.float16, 16),
                                        (torch.bfloat16, 3), (torch.bfloat16, 1)])
def test_long_prefix_few_queries_is_split_along_keys(gpu, dtype, page):
    """A chunked-prefill continuation: one request with an 8,192-token cached prefix (random
    page permutation) and 64 new tokens, beside a 3-token request, Hq32/Hkv8, pages of 16, 3
    (the general copy path: pages that do not divide a 64-key tile) and 1. That
    is 16 work items for 256 CUs, so the plan cuts the long items along their keys and a
    merge launch combines the chunks (the reference's split-KV prefill plan,
    flashinfer_plan_run.cu:312-316); every row checked against the oracle."""
    rng = np.random.default_rng(21)
    g = torch.Generator().manual_seed(21)
    pref = np.array([8192, 5])
    ext = np.array([64, 3])
    bounds = [0] + np.cumsum(ext).tolist()
    pages_per = (pref + ext + page - 1) // page
    pool = int(pages_per.sum()) + 1
    perm = rng.permutation(pool - 1) + 1
    table = np.zeros((2, int(pages_per.max())), np.int32)
    table[0, : pages_per[0]] = perm[: pages_per[0]]
    table[1, : pages_per[1]] = perm[pages_per[0]: pages_per[0] + pages_per[1]]
    kc = randn((pool, page, 8, 128), g, dtype, gpu)
    vc = randn((pool, page, 8, 128), g, dtype, gpu)
    n = bounds[-1]
    q = randn((n, 32, 128), g, dtype, gpu)
    attn = make(gpu, 32, 8, page, dtype)
    cache = BaseAttention()
    cache.bind_kv_cache(kc, vc)
    batch = attn.prepare(meta_for(gpu, bounds, pref.tolist(), torch.from_numpy(table).to(gpu)), n)
    info = batch.plan.plan.info()
    assert info["split_items"] == 8 and info["num_items"] > 64, info
    out = f32(batch.forward(q, q, q, cache)).reshape(n, 32, 128)
    want = oatt.prefill_with_cache(f32(q), f32(kc), f32(vc), table, bounds, pref, page)
    for r in range(2):
        assert_close(out[bounds[r]:bounds[r + 1]], want[bounds[r]:bounds[r + 1]], f"req={r}")


@pytest.mark.parametrize("hq,hkv,dtype", [(2, 2, torch.bfloat16), (4, 2, torch.bfloat16),
                                          (8, 1, torch.bfloat16), (4, 2, torch.float16)])
def test_single_long_sequence_is_split_along_keys(gpu, hq, hkv, dtype):
    """One 2,000-token ragged sequence with few heads (4-wave items of 128, 64 and 32
    queries): too few items for the device, so long items are split along their keys and
    merged; every row checked."""
    g = torch.Generator().manual_seed(hq * 10 + hkv)
    bounds = [0, 2000]
    q = randn((2000, hq, 128), g, dtype, gpu)
    k = randn((2000, hkv, 128), g, dtype, gpu)
    v = randn((2000, hkv, 128), g, dtype, gpu)
    attn = make(gpu, hq, hkv, 16, dtype)
    table = torch.zeros(1, 128, dtype=torch.int32, device=gpu)
    batch = attn.prepare(meta_for(gpu, bounds, [0], table), 2000)
    assert batch.plan.plan.info()["split_items"] > 0
    out = batch.forward(q, k, v, BaseAttention())
    want = oatt.prefill_ragged(f32(q), f32(k), f32(v), bounds)
    assert_close(f32(out).reshape(want.shape), want, f"hq={hq} hkv={hkv}")
