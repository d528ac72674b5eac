"""Pin the CPU oracle against the reference's fixtures, library routines,
closed forms and brute force (CPU only)."""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as att
from oracle import bf16, kv_store, norms, plan


# ---------------------------------------------------------------- rounding
def test_bf16_rounding_matches_torch_casts():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(10000).astype(np.float32) * 10,
        np.array([0.0, -0.0, np.inf, -np.inf, 1e-40, -1e-40, 3.4e38, 1.00390625, 1.01171875,
                  65504.0, 1.0 + 2**-8, 1.0 + 3 * 2**-8], np.float32),
    ])
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(bf16.bf16_bits(x), want)
    nan_bits = bf16.bf16_bits(np.array([np.nan], np.float32))
    assert np.isnan(bf16.bf16_to_f32(nan_bits))[0]
    np.testing.assert_array_equal(
        bf16.round_f16(x[:10000]),
        torch.from_numpy(x[:10000]).half().float().numpy())


# ---------------------------------------------------------------- K/V store
def test_kv_store_reference_device_fixture(fixtures):
    fx = fixtures["kv_store_device"]
    rng = np.random.default_rng(1)
    for width in fx["widths"]:
        packed = rng.standard_normal((5, 6, width)).astype(np.float32)
        k = packed[:, 2:4]
        v = packed[:, 4:6]
        kc = np.full((3, 4, 2, width), fx["k_fill"], np.float32)
        vc = np.full((3, 4, 2, width), fx["v_fill"], np.float32)
        ok, ov = kv_store.write_kv(kc, vc, k, v, np.array(fx["locations"]), fx["reserved"])
        ek, ev = kc.reshape(12, 2, width).copy(), vc.reshape(12, 2, width).copy()
        for row, slot in fx["expected_rows"]:
            ek[slot] = k[row]
            ev[slot] = v[row]
        np.testing.assert_array_equal(ok.reshape(12, 2, width), ek)
        np.testing.assert_array_equal(ov.reshape(12, 2, width), ev)
        # slot 0 is reserved: untouched
        assert (ok.reshape(12, 2, width)[0] == fx["k_fill"]).all()


def test_kv_store_reference_cpu_fixture(fixtures):
    fx = fixtures["kv_store_cpu"]
    kc = np.zeros(fx["cache_shape"], np.float32)
    kv = np.ones((2, 1, 2), np.float32)
    ok, _ = kv_store.write_kv(kc, kc, kv, kv, np.array(fx["locations"]), fx["reserved"])
    rows = ok.reshape(4, 2)
    for slot, total in fx["expected_row_sums"].items():
        assert rows[int(slot)].sum() == total
    for bad in fx["invalid_locations"]:
        with pytest.raises(kv_store.KVStoreError):
            kv_store.write_kv(kc, kc, kv[:1], kv[:1], np.array([bad]), fx["reserved"])


def test_kv_store_roundtrip_fixture(fixtures):
    fx = fixtures["kv_store_roundtrip"]
    kc = np.zeros(fx["cache_shape"], np.float32)
    k = np.array(fx["k"], np.float32).reshape(fx["kv_shape"])
    v = np.array(fx["v"], np.float32).reshape(fx["kv_shape"])
    ok, ov = kv_store.write_kv(kc, kc, k, v, np.array(fx["locations"]), -1)
    table = np.array([fx["locations"]])
    slots = att.slots_of(table[0], 2, 1)
    assert ok.reshape(-1, 1, 2)[slots].ravel().tolist() == fx["expected_k"]
    assert ov.reshape(-1, 1, 2)[slots].ravel().tolist() == fx["expected_v"]


# ---------------------------------------------------------------- page metadata
def test_decode_page_metadata_hand_case():
    table = np.array([[7, 8, 9, 0], [5, 0, 0, 0], [1, 2, 3, 4]], np.int32)
    indptr, indices, last = plan.decode_page_metadata(table, np.array([3, 1, 7]), 2)
    assert indptr.tolist() == [0, 2, 3, 7]
    assert indices.tolist() == [7, 8, 5, 1, 2, 3, 4]
    assert last.tolist() == [1, 1, 1]
    indptr, indices, last = plan.decode_page_metadata(table, np.array([4, 2, 8]), 2)
    assert last.tolist() == [2, 2, 2]
    assert indptr.tolist() == [0, 2, 3, 7]


@pytest.mark.parametrize("page_size", [1, 2, 16])
def test_decode_page_metadata_two_routes_agree(page_size):
    rng = np.random.default_rng(page_size)
    for _ in range(20):
        b = int(rng.integers(1, 9))
        cols = int(rng.integers(1, 40))
        table = rng.integers(0, 1 << 20, size=(b, cols)).astype(np.int32)
        lens = rng.integers(1, cols * page_size + 1, size=b)
        a = plan.decode_page_metadata(table, lens, page_size)
        m = plan.decode_page_metadata_masked(table, lens, page_size)
        for x, y in zip(a, m):
            np.testing.assert_array_equal(x, y)


def test_decode_page_metadata_rejects_bad_lengths():
    table = np.zeros((2, 4), np.int32)
    with pytest.raises(plan.PlanError):
        plan.decode_page_metadata(table, np.array([0, 1]), 1)
    with pytest.raises(plan.PlanError):
        plan.decode_page_metadata(table, np.array([9, 1]), 2)


def test_prefill_page_metadata_modes():
    table = np.arange(64, dtype=np.int32).reshape(2, 32)
    paged, indptr, _, _ = plan.prefill_page_metadata(table, [0, 17, 18], [0, 0], 16)
    assert not paged and indptr.tolist() == [0, 17, 18]
    paged, indptr, indices, last = plan.prefill_page_metadata(table, [0, 1, 18], [255, 16], 16)
    assert paged
    assert indptr.tolist() == [0, 16, 19]  # 256 tokens -> 16 pages; 33 tokens -> 3 pages
    assert indices.tolist() == list(range(16)) + [32, 33, 34]
    assert last.tolist() == [16, 1]
    with pytest.raises(plan.PlanError):
        plan.prefill_page_metadata(table, [0, 1, 1], [0, 0], 16)


def test_work_list_checker_rejects_gaps():
    lengths = [10]
    plan.check_work_list([0, 0, 10, -1], [-1, 1], lengths)
    with pytest.raises(AssertionError):
        plan.check_work_list([0, 0, 5, -1], [-1, 1], lengths)
    with pytest.raises(AssertionError):
        plan.check_work_list([0, 0, 5, 0, 0, 6, 10, 1], [0, 2], lengths)


# ---------------------------------------------------------------- norms
def test_add_rms_norm_residual_fixture(fixtures):
    fx = fixtures["add_rms_norm_residual"]
    w = fx["width"]
    x = np.full((1, w), fx["x"], np.float32)
    r = np.tile(np.array(fx["residual_pattern"], np.float32), w // 2)[None]
    weight = np.full(w, fx["weight"], np.float32)
    out, s = norms.add_rms_norm_f32(x, r, weight, fx["eps"])
    assert (bf16.round_bf16(out) == fx["expected_out"]).all()
    assert bf16.round_bf16(s)[0, :2].tolist() == fx["expected_residual_head"]
    # the fixture distinguishes normalising the rounded sum (old semantics)
    rounded = norms.rms_norm_f32(bf16.round_bf16(s), weight, fx["eps"])
    assert not (bf16.round_bf16(rounded) == fx["expected_out"]).all()


def test_rms_norm_matches_library_routine():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((33, 1024)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 1024).astype(np.float32)
    want = F.rms_norm(torch.from_numpy(x), (1024,), torch.from_numpy(w), eps=1e-6).numpy()
    np.testing.assert_allclose(norms.rms_norm_f32(x, w, 1e-6), want, rtol=2e-6, atol=2e-6)


def test_rms_norm_closed_forms():
    c = np.float32(0.75)
    x = np.full((2, 64), c, np.float32)
    w = np.full(64, 2.0, np.float32)
    got = norms.rms_norm_f32(x, w, 1e-6)
    np.testing.assert_allclose(got, 2.0 * c / math.sqrt(c * c + 1e-6), rtol=1e-6)
    # scale invariance (eps -> 0): rms(a x) == rms(x)
    rng = np.random.default_rng(4)
    y = rng.standard_normal((4, 128)).astype(np.float32)
    np.testing.assert_allclose(norms.rms_norm_f32(3 * y, np.ones(128), 0.0),
                               norms.rms_norm_f32(y, np.ones(128), 0.0), rtol=1e-5)
    q, k = norms.qk_norm_f32(y[:, None], y[:2, None], np.ones(128), 2 * np.ones(128), 1e-6)
    np.testing.assert_allclose(k, 2 * q[:2], rtol=1e-6)


# ---------------------------------------------------------------- attention
def _sdpa_reference(q, k, v, prefix, hq, hkv):
    """torch SDPA (float64) as an independent library route."""
    qt = torch.from_numpy(q).double().transpose(0, 1)
    kt = torch.from_numpy(k).double().transpose(0, 1).repeat_interleave(hq // hkv, 0)
    vt = torch.from_numpy(v).double().transpose(0, 1).repeat_interleave(hq // hkv, 0)
    lq, lk = q.shape[0], k.shape[0]
    visible = torch.arange(lk)[None, :] <= (torch.arange(lq)[:, None] + prefix)
    out = F.scaled_dot_product_attention(qt, kt, vt, attn_mask=visible)
    return out.transpose(0, 1).numpy()


@pytest.mark.parametrize("lq,lk,prefix,hq,hkv", [
    (1, 37, 36, 16, 8), (5, 5, 0, 4, 4), (7, 20, 13, 8, 2), (3, 9, 6, 32, 8), (16, 16, 0, 2, 1)])
def test_attention_matches_sdpa(lq, lk, prefix, hq, hkv):
    rng = np.random.default_rng(lq * 100 + lk)
    d = 128
    q = rng.standard_normal((lq, hq, d))
    k = rng.standard_normal((lk, hkv, d))
    v = rng.standard_normal((lk, hkv, d))
    got = att.attention_against_cache(q, k, v, prefix, hq, hkv)
    np.testing.assert_allclose(got, _sdpa_reference(q, k, v, prefix, hq, hkv), atol=1e-12)


def test_attention_matches_brute_force_tiny():
    rng = np.random.default_rng(9)
    q = rng.standard_normal((3, 1, 4))
    k = rng.standard_normal((5, 1, 4))
    v = rng.standard_normal((5, 1, 4))
    prefix = 2
    vis = [[j <= prefix + i for j in range(5)] for i in range(3)]
    want = att.brute_force_attention(q[:, 0].tolist(), k[:, 0].tolist(), v[:, 0].tolist(), vis,
                                     1 / math.sqrt(4))
    got = att.attention_against_cache(q, k, v, prefix, 1, 1)[:, 0]
    np.testing.assert_allclose(got, np.array(want), atol=1e-12)


def test_attention_closed_forms():
    rng = np.random.default_rng(11)
    q = rng.standard_normal((4, 2, 8))
    v = rng.standard_normal((6, 1, 8))
    # identical keys -> uniform weights -> running mean of visible values
    k = np.tile(rng.standard_normal((1, 1, 8)), (6, 1, 1))
    got = att.attention_against_cache(q, k, v, 2, 2, 1)
    for i in range(4):
        np.testing.assert_allclose(got[i, 0], v[: 3 + i, 0].mean(0), atol=1e-12)
        np.testing.assert_allclose(got[i, 1], v[: 3 + i, 0].mean(0), atol=1e-12)
    # the first causal query sees only key 0 -> output equals v[0]
    got = att.attention_against_cache(q, rng.standard_normal((6, 1, 8)), v, 0, 2, 1)
    np.testing.assert_allclose(got[0, 0], v[0, 0], atol=1e-12)


def test_reference_tiny_decode_fixture(fixtures):
    fx = fixtures["tiny_decode"]
    k = np.array(fx["k"], np.float64)[:, None]
    v = np.array(fx["v"], np.float64)[:, None]
    kc = np.zeros((1, 4, 1, 2))
    vc = np.zeros((1, 4, 1, 2))
    kc, vc = kv_store.write_kv(kc, vc, k, v, np.array(fx["locations"]), -1)
    q = np.array(fx["q"], np.float64)[:, None]
    table = np.array(fx["req_to_token"])
    lens = fx["cache_seqlens"]
    eager = att.decode_with_cache(q, kc, vc, np.clip(table, 0, None), lens, 1)
    # padded / masked formulation (decode_with_cache_padded, backend.rs:1375-1420)
    flat_k, flat_v = kc.reshape(-1, 1, 2), vc.reshape(-1, 1, 2)
    idx = np.clip(table, 0, None)
    valid = (table >= 0) & (np.arange(4)[None] < np.array(lens)[:, None])
    scores = np.einsum("bd,bjd->bj", q[:, 0], flat_k[idx][:, :, 0]) / math.sqrt(2)
    scores = np.where(valid, scores, -np.inf)
    p = np.exp(scores - scores.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    padded = np.einsum("bj,bjd->bd", p, flat_v[idx][:, :, 0])
    assert np.abs(eager[:, 0] - padded).max() < fx["tolerance"]
    # request 1 sees a single key -> its value
    np.testing.assert_allclose(eager[1, 0], [6, 6], atol=1e-12)


def test_reference_tiny_prefill_fixtures(fixtures):
    fx = fixtures["tiny_ragged_prefill"]
    q = np.array(fx["q"], np.float64)[:, None]
    v = np.array(fx["v"], np.float64)[:, None]
    got = att.prefill_ragged(q, q, v, fx["boundaries"])
    for s, e in zip(fx["boundaries"][:-1], fx["boundaries"][1:]):
        np.testing.assert_allclose(got[s:e], _sdpa_reference(q[s:e], q[s:e], v[s:e], 0, 1, 1),
                                   atol=fx["tolerance"])
    fx = fixtures["tiny_cached_prefill"]
    kc = np.zeros((1, 8, 1, 2))
    kc, vc = kv_store.write_kv(kc, kc.copy(), np.array(fx["all_k"], np.float64)[:, None],
                               np.array(fx["all_v"], np.float64)[:, None], np.arange(8), -1)
    q = np.array(fx["q"], np.float64)[:, None]
    table = np.clip(np.array(fx["req_to_token"]), 0, None)
    got = att.prefill_with_cache(q, kc, vc, table, fx["boundaries"], fx["prefixes"], 1)
    flat_k, flat_v = kc.reshape(-1, 1, 2), vc.reshape(-1, 1, 2)
    for r, (s, e) in enumerate(zip(fx["boundaries"][:-1], fx["boundaries"][1:])):
        n = fx["prefixes"][r] + e - s
        slots = table[r, :n]
        want = _sdpa_reference(q[s:e], flat_k[slots], flat_v[slots], fx["prefixes"][r], 1, 1)
        np.testing.assert_allclose(got[s:e], want, atol=fx["tolerance"])


def test_torch_cpu_baseline_agrees_with_oracle():
    rng = np.random.default_rng(5)
    b, hq, hkv, d, ps = 3, 4, 2, 128, 2
    pages = 40
    kc = rng.standard_normal((pages, ps, hkv, d)).astype(np.float32)
    vc = rng.standard_normal((pages, ps, hkv, d)).astype(np.float32)
    q = rng.standard_normal((b, hq, d)).astype(np.float32)
    table = rng.permutation(pages)[: b * 10].reshape(b, 10).astype(np.int32)
    lens = [7, 20, 1]
    want = att.decode_with_cache(q, kc, vc, table, lens, ps)
    got = att.decode_with_cache_torch(torch.from_numpy(q), torch.from_numpy(kc),
                                      torch.from_numpy(vc), torch.from_numpy(table), lens, ps)
    np.testing.assert_allclose(got.numpy().reshape(b, hq, d), want, atol=1e-5)


def test_torch_cpu_prefill_and_norm_baselines_agree_with_oracle():
    """The timed torch-CPU restatements of prefill (ragged and over a cached prefix) and the
    norms give the numpy oracle's results."""
    rng = np.random.default_rng(6)
    hq, hkv, d = 4, 2, 128
    bounds = [0, 5, 17, 18]
    n = bounds[-1]
    q = rng.standard_normal((n, hq, d)).astype(np.float32)
    k = rng.standard_normal((n, hkv, d)).astype(np.float32)
    v = rng.standard_normal((n, hkv, d)).astype(np.float32)
    want = att.prefill_ragged(q, k, v, bounds)
    got = att.prefill_ragged_torch(torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v),
                                   bounds)
    np.testing.assert_allclose(got.numpy().reshape(want.shape), want, atol=1e-5)
    ps, pages = 4, 30
    kc = rng.standard_normal((pages, ps, hkv, d)).astype(np.float32)
    vc = rng.standard_normal((pages, ps, hkv, d)).astype(np.float32)
    table = rng.permutation(pages)[:24].reshape(3, 8).astype(np.int32)
    prefixes = [3, 0, 9]
    want = att.prefill_with_cache(q, kc, vc, table, bounds, prefixes, ps)
    got = att.prefill_with_cache_torch(torch.from_numpy(q), torch.from_numpy(kc),
                                       torch.from_numpy(vc), torch.from_numpy(table), bounds,
                                       prefixes, ps)
    np.testing.assert_allclose(got.numpy().reshape(want.shape), want, atol=1e-5)
    x = rng.standard_normal((6, 256)).astype(np.float32)
    r = rng.standard_normal((6, 256)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 256).astype(np.float32)
    np.testing.assert_allclose(norms.rms_norm_torch(torch.from_numpy(x), torch.from_numpy(w),
                                                    1e-6).numpy(),
                               norms.rms_norm_f32(x, w, 1e-6), rtol=1e-5, atol=1e-6)
    out, res = norms.add_rms_norm_torch(torch.from_numpy(x), torch.from_numpy(r),
                                        torch.from_numpy(w), 1e-6)
    want_out, want_sum = norms.add_rms_norm_f32(x, r, w, 1e-6)
    np.testing.assert_allclose(out.numpy(), want_out, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(res.numpy(), want_sum, rtol=1e-6, atol=1e-6)
