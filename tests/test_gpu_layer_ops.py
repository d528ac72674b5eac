"""RoPE, fused QK-norm/RoPE/K-V store and SiLU*up on the GPU against the oracle.

Tolerances: the reference bounds rope at max-abs 0.0625 and silu at 0.03125 for bf16
(src/layers/ops.rs:299-330); here every element must additionally be within one unit in the
last place of the activation dtype of the oracle's fp32 value, and cos-sim > 0.9999. The fused
pass must equal the three separate launches bit for bit.
"""
import numpy as np
import pytest
import torch

from llm_infer_rust_amd import ops
from llm_infer_rust_amd.kv_cache import BaseAttention, ModelError
from oracle import bf16 as obf
from oracle import layer_ops as olay
from oracle import norms as onorm

pytestmark = pytest.mark.gpu

NAME = {torch.bfloat16: "bf16", torch.float16: "f16"}
ULP_BITS = {torch.bfloat16: 8, torch.float16: 11}


def f32(t):
    return t.float().cpu().numpy()


def within_one_ulp(got, want_f32, dtype):
    want = obf.round_to(want_f32, NAME[dtype])
    ulp = np.maximum(np.abs(want), 2.0 ** -14) * 2.0 ** (1 - ULP_BITS[dtype])
    bad = np.abs(got - want) > ulp + 1e-5  # slack for fma-contracted differences near zero
    assert not bad.any(), (np.abs(got - want).max(), int(bad.sum()))
    a, b = got.ravel().astype(np.float64), want_f32.ravel().astype(np.float64)
    assert a @ b / (np.linalg.norm(a) * np.linalg.norm(b) + 1e-30) > 0.9999


def packed_qkv(tokens, hq, hkv, dtype, gpu, seed, extra=0):
    g = torch.Generator().manual_seed(seed)
    width = (hq + 2 * hkv) * 128 + extra
    packed = torch.randn(tokens, width, generator=g).to(dtype).to(gpu)
    q = packed[:, : hq * 128].view(tokens, hq, 128)
    k = packed[:, hq * 128:(hq + hkv) * 128].view(tokens, hkv, 128)
    v = packed[:, (hq + hkv) * 128:(hq + 2 * hkv) * 128].view(tokens, hkv, 128)
    return packed, q, k, v


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("tokens,hq,hkv", [(3, 16, 8), (64, 32, 8), (257, 16, 8)])
def test_rope_matches_oracle(gpu, dtype, tokens, hq, hkv):
    packed, q, k, v = packed_qkv(tokens, hq, hkv, dtype, gpu, tokens + hq)
    rope = ops.HalfSplitRope(4096, 128, 1_000_000.0, gpu)
    g = torch.Generator().manual_seed(tokens)
    pos = torch.randint(0, 4096, (tokens,), generator=g)
    pos[0] = 0
    if tokens > 2:
        pos[1] = -1     # outside the table: untouched
        pos[2] = 4096
    q0, k0, v0 = f32(q), f32(k), v.clone()
    rope.apply(q, k, pos.to(gpu))
    cos, sin = f32(rope.cos), f32(rope.sin)
    within_one_ulp(f32(q), olay.rope(q0, pos.numpy(), cos, sin), dtype)
    within_one_ulp(f32(k), olay.rope(k0, pos.numpy(), cos, sin), dtype)
    assert torch.equal(v, v0)  # V bytes untouched
    assert np.array_equal(f32(q)[0], q0[0])  # position 0 is exactly the identity


def test_rope_generic_width(gpu):
    # width 64 and an odd head stride take the any-width kernel.
    g = torch.Generator().manual_seed(3)
    buf = torch.randn(5, 3 * 66, generator=g).to(torch.bfloat16).to(gpu)
    q = buf[:, :132].as_strided((5, 2, 64), (198, 66, 1))
    k = buf[:, 132:].as_strided((5, 1, 64), (198, 66, 1), buf[:, 132:].storage_offset())
    cos, sin = olay.rope_tables(64, 64, 10_000.0)
    pos = torch.tensor([0, 5, 63, 64, 7])
    q0, k0 = f32(q), f32(k)
    ops.rope(q, k, pos.to(gpu), torch.from_numpy(cos).to(gpu), torch.from_numpy(sin).to(gpu))
    within_one_ulp(f32(q), olay.rope(q0, pos.numpy(), cos, sin), torch.bfloat16)
    within_one_ulp(f32(k), olay.rope(k0, pos.numpy(), cos, sin), torch.bfloat16)


def bound_attention(pages, page_size, hkv, dtype, gpu, reserved):
    kc = torch.full((pages, page_size, hkv, 128), -3.0, dtype=dtype, device=gpu)
    vc = torch.full((pages, page_size, hkv, 128), 5.0, dtype=dtype, device=gpu)
    att = BaseAttention()
    att.bind_kv_cache(kc, vc)
    att.set_reserved_write_slot(reserved)
    return att


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("index_dtype", [torch.int32, torch.int64])
@pytest.mark.parametrize("stages", ["all", "norm+rope", "rope+store", "norm+store"])
def test_fused_pass_equals_separate_launches(gpu, dtype, index_dtype, stages):
    tokens, hq, hkv = 37, 16, 8
    _, q, k, v = packed_qkv(tokens, hq, hkv, dtype, gpu, 11)
    g = torch.Generator().manual_seed(12)
    qw = torch.empty(128).uniform_(0.5, 1.5, generator=g).to(dtype).to(gpu)
    kw = torch.empty(128).uniform_(0.5, 1.5, generator=g).to(dtype).to(gpu)
    pos = torch.randint(0, 2048, (tokens,), generator=g).to(gpu)
    rope = ops.HalfSplitRope(2048, 128, 1_000_000.0, gpu)
    loc = torch.randperm(64 * 4, generator=g)[:tokens].to(index_dtype)
    loc[3] = 0  # the reserved slot is skipped
    loc = loc.to(gpu)
    norm = "norm" in stages or stages == "all"
    rot = "rope" in stages or stages == "all"
    store = "store" in stages or stages == "all"

    q1, k1 = q.clone(), k.clone()
    a1 = bound_attention(64, 4, hkv, dtype, gpu, 0)
    if norm:
        ops.qk_norm(q1, k1, qw, kw, 1e-6)
    if rot:
        rope.apply(q1, k1, pos)
    if store:
        a1.write_kv(k1, v, loc)

    a2 = bound_attention(64, 4, hkv, dtype, gpu, 0)
    ops.qk_norm_rope_store(q, k, v, qw if norm else None, kw if norm else None, 1e-6,
                           pos if rot else None, rope if rot else None,
                           a2 if store else None, loc if store else None)
    assert torch.equal(q, q1) and torch.equal(k, k1)
    assert torch.equal(a2.k_cache, a1.k_cache) and torch.equal(a2.v_cache, a1.v_cache)
    a2.check_write_errors()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("tokens,hq,hkv,hidden", [(1, 32, 8, 4096), (64, 32, 8, 4096),
                                                  (256, 32, 8, 4096), (37, 16, 8, 1024),
                                                  (200, 16, 2, 2048)])
def test_fused_qkv_projection_pass_equals_the_two_steps(gpu, dtype, tokens, hq, hkv, hidden):
    """The QKV projection + QK-norm/RoPE/store entry (split-K partials summed inside the pass)
    against the library's projection followed by the fused pass: packed qkv (q and k rotated,
    v as projected) and both caches bit for bit, with and without a K split."""
    from llm_infer_rust_amd import _native
    from llm_infer_rust_amd._native import lib

    n = (hq + 2 * hkv) * 128
    g = torch.Generator().manual_seed(tokens + hidden)
    x = torch.randn(tokens, hidden, generator=g).to(dtype).to(gpu)
    w = (torch.randn(n, hidden, generator=g) * 0.02).to(dtype).to(gpu)
    qw = torch.empty(128).uniform_(0.5, 1.5, generator=g).to(dtype).to(gpu)
    kw = torch.empty(128).uniform_(0.5, 1.5, generator=g).to(dtype).to(gpu)
    pos = torch.randint(0, 4096, (tokens,), generator=g).to(gpu)
    rope = ops.HalfSplitRope(4096, 128, 1_000_000.0, gpu)
    loc = torch.randperm(512 * 16, generator=g)[:tokens]
    loc[tokens // 2] = 0  # the reserved slot is skipped
    loc = loc.to(gpu)
    splits_bytes = lib().mi355x_linear_workspace_bytes(tokens, n, hidden,
                                                       _native.device_cus(x.device), -1, -1)
    print(f"tokens {tokens} N {n} K {hidden}: split-K workspace {splits_bytes} bytes")

    a1 = bound_attention(512, 16, hkv, dtype, gpu, 0)
    qkv1 = ops.decode_linear(x, w)
    ops.qk_norm_rope_store(qkv1[:, :hq * 128].view(tokens, hq, 128),
                           qkv1[:, hq * 128:(hq + hkv) * 128].view(tokens, hkv, 128),
                           qkv1[:, (hq + hkv) * 128:].view(tokens, hkv, 128), qw, kw, 1e-6,
                           pos, rope, a1, loc)
    a2 = bound_attention(512, 16, hkv, dtype, gpu, 0)
    qkv2 = ops.linear_qk_norm_rope_store(x, w, hq, hkv, qw, kw, 1e-6, pos, rope, a2, loc)
    assert torch.equal(qkv2, qkv1)
    assert torch.equal(a2.k_cache, a1.k_cache) and torch.equal(a2.v_cache, a1.v_cache)
    a2.check_write_errors()
    if (tokens, hidden) == (256, 4096):
        assert splits_bytes > 0  # the partials route is the one exercised here


def test_fused_qkv_route_refuses_before_launching(gpu):
    """An argument the pass would refuse (here: no v_cache) is reported before the projection
    is queued: qkv keeps its contents and the cache is untouched."""
    from llm_infer_rust_amd import _native
    from llm_infer_rust_amd._native import lib

    tokens, hq, hkv, hidden = 256, 32, 8, 4096
    n = (hq + 2 * hkv) * 128
    x = torch.randn(tokens, hidden, device=gpu).to(torch.bfloat16)
    w = (torch.randn(n, hidden, device=gpu) * 0.02).to(torch.bfloat16)
    qw = torch.ones(128, dtype=torch.bfloat16, device=gpu)
    pos = torch.arange(tokens, device=gpu)
    rope = ops.HalfSplitRope(4096, 128, 1_000_000.0, gpu)
    att = bound_attention(512, 16, hkv, torch.bfloat16, gpu, 0)
    loc = torch.arange(1, tokens + 1, dtype=torch.int64, device=gpu)
    cus = _native.device_cus(x.device)
    need = lib().mi355x_linear_workspace_bytes(tokens, n, hidden, cus, -1, -1)
    assert need > 0  # the split-K route, whose partials a refused pass would strand
    ws = torch.empty(need, dtype=torch.uint8, device=gpu)
    qkv = torch.full((tokens, n), 7.0, dtype=torch.bfloat16, device=gpu)
    before = att.k_cache.clone()
    kc, _ = att.cache_tensors()
    err = lib().mi355x_linear_qk_norm_rope_store(
        x.data_ptr(), hidden, w.data_ptr(), hidden, qkv.data_ptr(), n, tokens, hidden, hq, hkv,
        ws.data_ptr(), need, cus, qw.data_ptr(), qw.data_ptr(), pos.data_ptr(),
        rope.cos.data_ptr(), rope.sin.data_ptr(), rope.max_positions, kc.data_ptr(), None,
        loc.data_ptr(), True, kc.size(0) * kc.size(1), 0, None, 1e-6, 0,
        torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert err is not None and b"v_cache" in err
    assert bool((qkv == 7.0).all())
    assert torch.equal(att.k_cache, before)


def test_fused_pass_reports_out_of_range_slot(gpu):
    _, q, k, v = packed_qkv(4, 16, 8, torch.bfloat16, gpu, 5)
    att = bound_attention(8, 1, 8, torch.bfloat16, gpu, -1)
    before = att.k_cache.clone()
    loc = torch.tensor([1, 2, 8, 3], dtype=torch.int64, device=gpu)  # 8 is outside
    ops.qk_norm_rope_store(q, k, v, None, None, 1e-6, None, None, att, loc)
    with pytest.raises(ModelError, match="outside the bound KV cache"):
        att.check_write_errors()
    assert torch.equal(att.k_cache[0], before[0]) and torch.equal(att.k_cache[4:], before[4:])
    assert torch.equal(att.k_cache[1, 0], k[0]) and torch.equal(att.v_cache[3, 0], v[3])


def test_fused_pass_matches_oracle_composition(gpu):
    tokens, hq, hkv = 19, 32, 8
    _, q, k, v = packed_qkv(tokens, hq, hkv, torch.bfloat16, gpu, 21)
    g = torch.Generator().manual_seed(22)
    qw = torch.empty(128).uniform_(0.5, 1.5, generator=g).to(torch.bfloat16).to(gpu)
    kw = torch.empty(128).uniform_(0.5, 1.5, generator=g).to(torch.bfloat16).to(gpu)
    pos = torch.randint(0, 40960, (tokens,), generator=g)
    rope = ops.HalfSplitRope(40960, 128, 1_000_000.0, gpu)
    q0, k0 = f32(q), f32(k)
    ops.qk_norm_rope_store(q, k, v, qw, kw, 1e-6, pos.to(gpu), rope)
    cos, sin = f32(rope.cos), f32(rope.sin)
    qn = obf.round_to(onorm.rms_norm_f32(q0, f32(qw), 1e-6), "bf16")
    kn = obf.round_to(onorm.rms_norm_f32(k0, f32(kw), 1e-6), "bf16")
    # A normalised element may sit one ulp from the oracle's before rotation and the rotation
    # rounds once more: allow two bf16 ulps of the result, plus the cos-sim gate.
    for got, base in ((f32(q), qn), (f32(k), kn)):
        want = olay.rope(base, pos.numpy(), cos, sin)
        ulp = np.maximum(np.abs(want), 2.0 ** -14) * 2.0 ** -7
        assert (np.abs(got - want) <= 2 * ulp + 1e-5).all()
        a, b = got.ravel().astype(np.float64), want.ravel().astype(np.float64)
        assert a @ b / (np.linalg.norm(a) * np.linalg.norm(b)) > 0.9999


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("tokens,width", [(1, 8), (1, 3072), (3, 13), (65, 3072), (2, 8200),
                                          (256, 12288)])
def test_silu_mul_matches_oracle(gpu, dtype, tokens, width):
    # Shapes of the reference test silu_matches_fp32_reference_for_decode_prefill_and_tail_widths
    # (ops.rs:321-345) plus the Qwen3-8B decode shape.
    g = torch.Generator().manual_seed(tokens * width)
    gate_up = torch.randn(tokens, 2 * width, generator=g).to(dtype).to(gpu)
    out = ops.silu_and_mul(gate_up)
    want = olay.silu_mul(f32(gate_up))
    got = f32(out)
    assert np.abs(got - obf.round_to(want, NAME[dtype])).max() <= 0.03125
    within_one_ulp(got, want, dtype)
