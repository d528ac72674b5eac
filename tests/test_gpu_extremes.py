"""Decode and prefill at the extremes of the serving range, against the float64 oracle.

* a 131,072-token decode context next to 1-17 token requests (page sizes 1 and 16; the long
  request is cut into many work items because one item's page entries must fit in LDS);
* the full 256-request decode batch at the Qwen3-8B serving shape (page 16, GQA group 4,
  KV lengths 1024-1536, the largest captured decode-graph bucket), and the same batch at nearly
  equal lengths, which the planner places as whole requests;
* paged prefill over a 65,536-token cached prefix next to a 1-token prefix and a 1-token
  extend (query rows sampled: first, last and random);
* two decode plans and a prefill plan on three concurrent streams, equal to serial runs.
Tolerance as in the per-kernel tests: max-abs <= 2e-2 and cosine similarity > 0.9999.
"""
import numpy as np
import pytest
import torch

from llm_infer_rust_amd.backend import Attention, AttentionMetadata, AttentionSpec, BatchPhase
from llm_infer_rust_amd.kv_cache import BaseAttention
from oracle import attention as oatt
from oracle import plan as oplan

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
MIN_COS = 0.9999


def f32(t):
    return t.float().cpu().numpy()


def assert_close(got, want, what):
    got = np.asarray(got, np.float64).ravel()
    want = np.asarray(want, np.float64).ravel()
    err = float(np.abs(got - want).max())
    cs = float(got @ want / (np.linalg.norm(got) * np.linalg.norm(want) + 1e-30))
    assert err <= MAX_ABS and cs > MIN_COS, f"{what} max_abs={err} cos={cs}"


def backend(gpu, hq, hkv, page):
    attn = Attention.new("mi355x", AttentionSpec(hq, hkv, 128, torch.bfloat16, gpu))
    attn.bind_cache_layout(page)
    return attn


def paged_pool(rng, g, gpu, lengths, page, hkv):
    """Disjoint random pages per request (page 0 reserved) and bf16 N(0,1) K/V pools."""
    pages_per = [(int(n) + page - 1) // page for n in lengths]
    pool = sum(pages_per) + 1
    perm = rng.permutation(pool - 1) + 1
    table = np.zeros((len(lengths), max(pages_per)), np.int32)
    off = 0
    for r, n in enumerate(pages_per):
        table[r, :n] = perm[off: off + n]
        off += n
    kc = torch.randn(pool, page, hkv, 128, generator=g).to(torch.bfloat16).to(gpu)
    vc = torch.randn(pool, page, hkv, 128, generator=g).to(torch.bfloat16).to(gpu)
    return table, kc, vc


def run_decode(gpu, hq, hkv, page, lengths, seed):
    rng = np.random.default_rng(seed)
    g = torch.Generator().manual_seed(seed)
    lengths = np.asarray(lengths, np.int32)
    table, kc, vc = paged_pool(rng, g, gpu, lengths, page, hkv)
    q = torch.randn(len(lengths), hq, 128, generator=g).to(torch.bfloat16).to(gpu)
    cache = BaseAttention()
    cache.bind_kv_cache(kc, vc)
    meta = AttentionMetadata(BatchPhase.DECODE, block_table=torch.from_numpy(table).to(gpu),
                             cache_seqlens=torch.from_numpy(lengths).to(gpu))
    batch = backend(gpu, hq, hkv, page).prepare(meta, len(lengths))
    md = batch.plan.plan.read_metadata()
    oplan.check_work_list(md["work"], md["merge"], lengths.tolist())
    out = batch.forward(q, q, q, cache)
    want = oatt.decode_with_cache(f32(q), f32(kc), f32(vc), table, lengths, page)
    return f32(out).reshape(want.shape), want, md


@pytest.mark.parametrize("hq,page", [(16, 1), (32, 16)])
def test_decode_128k_context_next_to_tiny_requests(gpu, hq, page):
    got, want, md = run_decode(gpu, hq, 8, page, [131072, 3, 17, 1], 131)
    items_of_long = sum(1 for i in range(len(md["work"]) // 4) if md["work"][4 * i] == 0)
    assert items_of_long > 16  # the long context is split over many items and merged
    assert_close(got, want, f"128k hq={hq} page={page}")


def test_decode_full_batch_at_serving_shape(gpu):
    rng = np.random.default_rng(256)
    lengths = rng.integers(1024, 1537, size=256)
    got, want, _ = run_decode(gpu, 32, 8, 16, lengths, 256)
    assert_close(got, want, "batch 256 page 16 group 4")


def test_decode_whole_requests_at_near_equal_lengths(gpu):
    """256 requests of 1,248-1,312 tokens (the config-5 decode steps): the planner places whole
    requests (no split, so no partials and no merge launch) instead of cutting requests to even
    out a tile or two; the result must still match the oracle."""
    rng = np.random.default_rng(1280)
    lengths = 1280 + rng.integers(-32, 33, size=256)
    got, want, md = run_decode(gpu, 32, 8, 16, lengths, 1280)
    assert len(md["work"]) // 4 == 256 and all(c == 1 for c in md["merge"][1::2])
    assert_close(got, want, "batch 256 whole requests")


def test_paged_prefill_64k_prefix_sampled_rows(gpu):
    rng = np.random.default_rng(64)
    g = torch.Generator().manual_seed(64)
    page, hq, hkv = 16, 32, 8
    pref = np.array([65536, 1, 3000], np.int64)
    ext = np.array([700, 130, 1], np.int64)
    bounds = [0] + np.cumsum(ext).tolist()
    table, kc, vc = paged_pool(rng, g, gpu, (pref + ext).tolist(), page, hkv)
    n = bounds[-1]
    q = torch.randn(n, hq, 128, generator=g).to(torch.bfloat16).to(gpu)
    cache = BaseAttention()
    cache.bind_kv_cache(kc, vc)
    meta = AttentionMetadata(
        BatchPhase.PREFILL, block_table=torch.from_numpy(table).to(gpu),
        cu_seqlens_q=torch.tensor(bounds, dtype=torch.int32, device=gpu),
        prefix_lens=torch.tensor(pref.tolist(), dtype=torch.int32, device=gpu))
    batch = backend(gpu, hq, hkv, page).prepare(meta, n)
    assert batch.plan.plan.paged
    out = f32(batch.forward(q, q, q, cache)).reshape(n, hq, 128)
    qf = f32(q)
    flat_k = f32(kc).reshape(-1, hkv, 128)
    flat_v = f32(vc).reshape(-1, hkv, 128)
    for r in range(len(ext)):
        e = int(ext[r])
        rows = sorted(set([0, e - 1] + rng.integers(0, e, size=12).tolist()))
        for i in rows:
            horizon = int(pref[r]) + i + 1
            slots = oatt.slots_of(table[r], horizon, page)
            want = oatt.attention_against_cache(qf[bounds[r] + i: bounds[r] + i + 1],
                                                flat_k[slots], flat_v[slots], horizon - 1, hq,
                                                hkv)
            assert_close(out[bounds[r] + i], want[0], f"req={r} row={i}")


def test_plans_on_concurrent_streams_match_serial_runs(gpu):
    """Two decode plans and a prefill plan launched on three streams at once (each plan owns
    its workspace; the library keeps no shared device state) give the bytes of serial runs."""
    rng = np.random.default_rng(77)
    g = torch.Generator().manual_seed(77)
    cases = []
    for hq, page, lens in ((32, 16, rng.integers(200, 3000, size=48)),
                           (16, 1, rng.integers(1, 2000, size=33))):
        table, kc, vc = paged_pool(rng, g, gpu, lens, page, 8)
        q = torch.randn(len(lens), hq, 128, generator=g).to(torch.bfloat16).to(gpu)
        cache = BaseAttention()
        cache.bind_kv_cache(kc, vc)
        meta = AttentionMetadata(BatchPhase.DECODE,
                                 block_table=torch.from_numpy(table).to(gpu),
                                 cache_seqlens=torch.from_numpy(lens.astype(np.int32)).to(gpu))
        batch = backend(gpu, hq, 8, page).prepare(meta, len(lens))
        cases.append((batch, q, cache))
    bounds = [0, 700, 1500]
    n = bounds[-1]
    pq = torch.randn(n, 16, 128, generator=g).to(torch.bfloat16).to(gpu)
    pk = torch.randn(n, 8, 128, generator=g).to(torch.bfloat16).to(gpu)
    pv = torch.randn(n, 8, 128, generator=g).to(torch.bfloat16).to(gpu)
    pmeta = AttentionMetadata(BatchPhase.PREFILL,
                              cu_seqlens_q=torch.tensor(bounds, dtype=torch.int32, device=gpu),
                              prefix_lens=torch.zeros(2, dtype=torch.int32, device=gpu),
                              block_table=torch.zeros(2, 128, dtype=torch.int32, device=gpu))
    pbatch = backend(gpu, 16, 8, 16).prepare(pmeta, n)
    pcache = BaseAttention()
    serial = [b.forward(q, q, q, c).clone() for b, q, c in cases]
    serial.append(pbatch.forward(pq, pk, pv, pcache).clone())
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream() for _ in range(3)]
    outs = []
    for _ in range(3):  # a few rounds so launches overlap
        for s in streams:
            s.wait_stream(torch.cuda.current_stream())
        round_outs = []
        for s, (b, q, c) in zip(streams, cases):
            with torch.cuda.stream(s):
                round_outs.append(b.forward(q, q, q, c))
        with torch.cuda.stream(streams[2]):
            round_outs.append(pbatch.forward(pq, pk, pv, pcache))
        for s in streams:
            torch.cuda.current_stream().wait_stream(s)
        outs.append(round_outs)
    torch.cuda.synchronize()
    for round_outs in outs:
        for got, want in zip(round_outs, serial):
            assert torch.equal(got, want)
