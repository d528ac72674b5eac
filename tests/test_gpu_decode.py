"""Paged decode attention through the C ABI against the oracle.

Tolerance (written here, applied to every case): max-abs <= 2e-2 (tighter than
the reference's 0.03125, backend.rs:1748) and cosine similarity > 0.9999
against the float64 oracle on the same bf16/fp16-rounded inputs. Page metadata
(indptr / indices / last_page_len) is compared bit-exactly.
"""
import numpy as np
import pytest
import torch

from llm_infer_rust_amd.backend import (Attention, AttentionMetadata, AttentionSpec, BatchPhase,
                                        DecodeHostMetadata, ModelError)
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


def make_backend(gpu, hq, hkv, page_size, dtype=torch.bfloat16):
    spec = AttentionSpec(hq, hkv, 128, dtype, gpu)
    attn = Attention.new("mi355x", spec)
    attn.bind_cache_layout(page_size)
    return attn


def randn(shape, g, dtype, gpu):
    return torch.randn(*shape, generator=g).to(dtype).to(gpu)


def test_reference_plan_reuse_cases(gpu, fixtures):
    fx = fixtures["decode_plans"]
    g = torch.Generator().manual_seed(11)
    attn = make_backend(gpu, 16, 8, fx["page_size"])
    cache = BaseAttention()
    kc = randn(fx["cache_shape"], g, torch.bfloat16, gpu)
    vc = randn(fx["cache_shape"], g, torch.bfloat16, gpu)
    cache.bind_kv_cache(kc, vc)
    table = torch.arange(32, dtype=torch.int32, device=gpu).view(2, 16)
    packed = randn((2, 4096), g, torch.bfloat16, gpu)
    q = packed[:, :2048].view(2, 16, 128)
    assert not q.is_contiguous()
    handle, warm = None, None
    for rows, length in fx["cases"]:
        lens = [length, length - length // 2][:rows]
        meta = AttentionMetadata(BatchPhase.DECODE, block_table=table[:rows],
                                 cache_seqlens=torch.tensor(lens, dtype=torch.int32, device=gpu),
                                 max_seqlen=length)
        batch = attn.prepare(meta, rows)
        with pytest.raises(ModelError, match="still in use"):
            attn.prepare(meta, rows)
        plan = batch.plan.plan
        if handle is None:
            handle, warm = plan.handle, plan.allocations()
        else:
            assert plan.handle == handle
            assert plan.allocations() == warm
        query = q[:rows]
        out = batch.forward(query, query, query, cache)
        want = oatt.decode_with_cache(f32(query), f32(kc), f32(vc), table[:rows].cpu().numpy(),
                                      lens, fx["page_size"])
        assert_close(f32(out), want, f"rows={rows} len={length}")
        del batch


@pytest.mark.parametrize("page_size", [1, 16])
def test_page_metadata_bit_exact_and_work_list(gpu, page_size):
    g = torch.Generator().manual_seed(page_size)
    rng = np.random.default_rng(page_size)
    b, cols = 37, 300
    table = rng.integers(0, 1 << 22, size=(b, cols)).astype(np.int32)
    lens = rng.integers(1, cols * page_size + 1, size=b).astype(np.int32)
    attn = make_backend(gpu, 16, 8, page_size)
    meta = AttentionMetadata(BatchPhase.DECODE,
                             block_table=torch.from_numpy(table).to(gpu),
                             cache_seqlens=torch.from_numpy(lens).to(gpu))
    batch = attn.prepare(meta, b)
    md = batch.plan.plan.read_metadata()
    indptr, indices, last = oplan.decode_page_metadata(table, lens, page_size)
    assert md["indptr"] == indptr.tolist()
    assert md["indices"] == indices.tolist()
    assert md["last_page_len"] == last.tolist()
    oplan.check_work_list(md["work"], md["merge"], lens.tolist())
    del g


def test_host_lengths_path_matches_device_readback(gpu):
    rng = np.random.default_rng(4)
    b, cols = 9, 64
    table = rng.integers(0, 5000, size=(b, cols)).astype(np.int32)
    lens = rng.integers(1, cols + 1, size=b).astype(np.int32)
    attn = make_backend(gpu, 16, 8, 1)
    meta = AttentionMetadata(BatchPhase.DECODE, block_table=torch.from_numpy(table).to(gpu),
                             cache_seqlens=torch.from_numpy(lens).to(gpu),
                             decode_host=DecodeHostMetadata(lens.tolist()))
    batch = attn.prepare(meta, b)
    md = batch.plan.plan.read_metadata()
    indptr, indices, last = oplan.decode_page_metadata(table, lens, 1)
    assert md["indptr"] == indptr.tolist() and md["indices"] == indices.tolist()
    del batch
    bad = AttentionMetadata(BatchPhase.DECODE, block_table=torch.from_numpy(table).to(gpu),
                            cache_seqlens=torch.from_numpy(lens).to(gpu),
                            decode_host=DecodeHostMetadata([cols + 1] * b))
    with pytest.raises(ModelError, match="exceeds block table capacity"):
        attn.prepare(bad, b)


def _random_decode_case(gpu, g, rng, b, hq, hkv, page_size, lo, hi, pool_pages, dtype):
    lens = rng.integers(lo, hi + 1, size=b).astype(np.int32)
    cols = int((hi + page_size - 1) // page_size)
    if pool_pages - 1 >= b * cols:
        table = (rng.permutation(pool_pages - 1)[: b * cols] + 1).reshape(b, cols)
    else:  # small pools: pages may repeat across requests
        table = rng.integers(1, pool_pages, size=(b, cols))
    table = table.astype(np.int32)
    kc = randn((pool_pages, page_size, hkv, 128), g, dtype, gpu)
    vc = randn((pool_pages, page_size, hkv, 128), g, dtype, gpu)
    q = randn((b, hq, 128), g, dtype, gpu)
    return lens, table, kc, vc, q


@pytest.mark.parametrize("hq,hkv,page_size,dtype", [
    (16, 8, 1, torch.bfloat16), (32, 8, 16, torch.bfloat16), (8, 8, 4, torch.bfloat16),
    (64, 8, 1, torch.bfloat16), (16, 8, 1, torch.float16), (4, 2, 3, torch.float16),
    # slices of 4 kv heads, two slices of 8, page sizes that do not divide the 16-token tile
    (16, 4, 3, torch.bfloat16), (32, 16, 7, torch.bfloat16), (8, 4, 16, torch.float16),
    # groups of 4 and 8 q heads run the matrix-core kernel: fp16, odd pages, 4-head slices
    (32, 8, 5, torch.float16), (64, 8, 16, torch.bfloat16), (32, 4, 1, torch.bfloat16)])
def test_decode_matches_oracle(gpu, hq, hkv, page_size, dtype):
    g = torch.Generator().manual_seed(hq * 7 + page_size)
    rng = np.random.default_rng(hq + page_size)
    lens, table, kc, vc, q = _random_decode_case(gpu, g, rng, 24, hq, hkv, page_size, 1, 3000,
                                                 4000 // page_size + 800, dtype)
    attn = make_backend(gpu, hq, hkv, page_size, dtype)
    cache = BaseAttention()
    cache.bind_kv_cache(kc, vc)
    meta = AttentionMetadata(BatchPhase.DECODE, block_table=torch.from_numpy(table).to(gpu),
                             cache_seqlens=torch.from_numpy(lens).to(gpu))
    batch = attn.prepare(meta, len(lens))
    out = batch.forward(q, q, q, cache)
    want = oatt.decode_with_cache(f32(q), f32(kc), f32(vc), table, lens, page_size)
    assert_close(f32(out).reshape(want.shape), want, f"hq={hq} hkv={hkv} P={page_size}")
    # static output: same address, padding rows untouched
    storage = torch.full((len(lens) + 2, hq * 128), 99.0, dtype=dtype, device=gpu)
    target = storage[: len(lens)]
    ptr = target.data_ptr()
    batch.forward_into(q, q, q, cache, target)
    assert target.data_ptr() == ptr
    assert torch.equal(target, out)
    assert bool((storage[len(lens):] == 99.0).all())


@pytest.mark.parametrize("hq", [16, 32])
def test_long_and_tiny_requests_split_across_workgroups(gpu, hq):
    """Requests far longer than one workgroup's share (and than one work item) next to
    requests of a few tokens: every share boundary and item cut is merged exactly (group 2
    on the vector kernel, group 4 on the matrix-core kernel)."""
    g = torch.Generator().manual_seed(99)
    page = 2
    lens = np.array([20011, 5, 9000, 1, 2048, 4097], dtype=np.int32)
    pages_per = (lens + page - 1) // page
    cols = int(pages_per.max())
    pool_pages = int(pages_per.sum()) + 1
    perm = np.random.default_rng(99).permutation(pool_pages - 1) + 1
    table = np.zeros((len(lens), cols), dtype=np.int32)
    off = 0
    for b, n in enumerate(pages_per):
        table[b, :n] = perm[off: off + n]
        off += n
    kc = randn((pool_pages, page, 8, 128), g, torch.bfloat16, gpu)
    vc = randn((pool_pages, page, 8, 128), g, torch.bfloat16, gpu)
    q = randn((len(lens), hq, 128), g, torch.bfloat16, gpu)
    attn = make_backend(gpu, hq, 8, page)
    cache = BaseAttention()
    cache.bind_kv_cache(kc, vc)
    meta = AttentionMetadata(BatchPhase.DECODE, block_table=torch.from_numpy(table).to(gpu),
                             cache_seqlens=torch.from_numpy(lens).to(gpu))
    batch = attn.prepare(meta, len(lens))
    md = batch.plan.plan.read_metadata()
    oplan.check_work_list(md["work"], md["merge"], lens.tolist())
    out = batch.forward(q, q, q, cache)
    want = oatt.decode_with_cache(f32(q), f32(kc), f32(vc), table, lens, page)
    assert_close(f32(out).reshape(want.shape), want, f"long/tiny hq={hq}")


def test_config2_shape_parity(gpu):
    """Config 2 at full shape: B=64, Hq16/Hkv8, page 1, L~U[512,4096], random slots."""
    g = torch.Generator().manual_seed(2024)
    rng = np.random.default_rng(2024)
    pool = 1 << 20
    lens, table, kc, vc, q = _random_decode_case(gpu, g, rng, 64, 16, 8, 1, 512, 4096, pool,
                                                 torch.bfloat16)
    attn = make_backend(gpu, 16, 8, 1)
    cache = BaseAttention()
    cache.set_reserved_write_slot(0)
    cache.bind_kv_cache(kc, vc)
    # write the new token of each request before attention (int64 positions)
    knew = randn((64, 8, 128), g, torch.bfloat16, gpu)
    vnew = randn((64, 8, 128), g, torch.bfloat16, gpu)
    loc = torch.tensor([table[b, lens[b] - 1] for b in range(64)], dtype=torch.int64, device=gpu)
    cache.write_kv(knew, vnew, loc)
    meta = AttentionMetadata(BatchPhase.DECODE, block_table=torch.from_numpy(table).to(gpu),
                             cache_seqlens=torch.from_numpy(lens).to(gpu))
    batch = attn.prepare(meta, 64)
    info = batch.plan.plan.info()
    assert info["num_items"] > 64  # split-KV engaged
    out = batch.forward(q, q, q, cache)
    want = oatt.decode_with_cache(f32(q), f32(kc), f32(vc), table, lens, 1)
    assert_close(f32(out).reshape(want.shape), want, "config2")
    cache.check_write_errors()


def test_graph_plan_replays_dynamic_lengths_and_padded_rows(gpu, fixtures):
    fx = fixtures["graph_replay_lengths"]
    g = torch.Generator().manual_seed(17)
    page = 16
    max_len = 1024
    rows_cap = max(fx["rows"])
    cols = max_len // page
    kc = randn((rows_cap * cols + 1, page, 8, 128), g, torch.bfloat16, gpu)
    vc = randn((rows_cap * cols + 1, page, 8, 128), g, torch.bfloat16, gpu)
    kc[0].zero_()
    vc[0].zero_()
    cache = BaseAttention()
    cache.set_reserved_write_slot(0)
    cache.bind_kv_cache(kc, vc)
    attn = make_backend(gpu, 16, 8, page)
    # fixed graph buffers: pad rows point at page 0 with length 1
    table = torch.zeros(rows_cap, cols, dtype=torch.int32, device=gpu)
    lengths = torch.ones(rows_cap, dtype=torch.int32, device=gpu)
    state = attn.prepare_decode_graph(AttentionMetadata(BatchPhase.DECODE, block_table=table,
                                                        cache_seqlens=lengths))
    with pytest.raises(ModelError, match="already registered"):
        attn.prepare_decode_graph(AttentionMetadata(BatchPhase.DECODE, block_table=table,
                                                    cache_seqlens=lengths))
    handle = state.plan.handle
    allocs = state.plan.allocations()
    rng = np.random.default_rng(17)
    q = randn((rows_cap, 16, 128), g, torch.bfloat16, gpu)
    for rows in fx["rows"]:
        for length in fx["lengths"]:
            lens = [max(1, length - 3 * r) for r in range(rows)]
            src = rng.permutation(rows_cap * cols)[: rows * cols].reshape(rows, cols) + 1
            table.zero_()
            table[:rows] = torch.from_numpy(src.astype(np.int32)).to(gpu)
            lengths.fill_(1)
            lengths[:rows] = torch.tensor(lens, dtype=torch.int32, device=gpu)
            state.prepare_replay(DecodeHostMetadata(lens))
            assert state.plan.handle == handle and state.plan.allocations() == allocs
            meta = AttentionMetadata(BatchPhase.DECODE, block_table=table,
                                     cache_seqlens=lengths)
            batch = attn.prepare(meta, rows_cap)
            assert batch.plan.plan is state.plan
            out = batch.forward(q, q, q, cache)
            want = oatt.decode_with_cache(f32(q[:rows]), f32(kc), f32(vc),
                                          table[:rows].cpu().numpy(), lens, page)
            assert_close(f32(out)[:rows].reshape(want.shape), want, f"rows={rows} len={length}")
            del batch
