"""RMSNorm / add-RMSNorm / QK-norm on the GPU against the fp32 oracle.

Tolerances: the reference's own bounds (src/layers/ops.rs:276-432) — max-abs
0.03125 (bf16 rms / qk), 0.0625 (bf16 add-rms), 0.0078125 (fp16) — and the
residual write-back bit-exact. We additionally require cos-sim > 0.9999.
"""
import numpy as np
import pytest
import torch

from llm_infer_rust_amd import ops
from oracle import bf16 as obf
from oracle import norms as onorm

pytestmark = pytest.mark.gpu

TOL = {torch.bfloat16: (0.03125, 0.0625), torch.float16: (0.0078125, 0.0078125)}
NAME = {torch.bfloat16: "bf16", torch.float16: "f16"}


def f32(t):
    return t.float().cpu().numpy()


def cos(a, b):
    a, b = a.ravel().astype(np.float64), b.ravel().astype(np.float64)
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b) + 1e-30))


def check(actual, expected_f32, dtype, tol):
    want = obf.round_to(expected_f32, NAME[dtype])
    got = f32(actual)
    err = np.abs(got - want).max()
    assert err <= tol, err
    assert cos(got, expected_f32) > 0.9999


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,width", [(3, 1024), (1, 8), (65, 4096), (7, 13), (2, 16384),
                                        (256, 4096), (300, 2056), (4100, 4096)])
def test_rms_norm(gpu, dtype, rows, width):
    g = torch.Generator().manual_seed(rows * width)
    x = torch.randn(rows, width, generator=g).to(dtype).to(gpu)
    w = torch.empty(width).uniform_(0.5, 1.5, generator=g).to(dtype).to(gpu)
    out = ops.rms_norm(x, w, 1e-6)
    check(out, onorm.rms_norm_f32(f32(x), f32(w), 1e-6), dtype, TOL[dtype][0])


def test_rms_norm_row_stride(gpu):
    g = torch.Generator().manual_seed(5)
    storage = torch.randn(9, 1040, generator=g).to(torch.bfloat16).to(gpu)
    x = storage[:, :1024]
    w = torch.randn(1024, generator=g).to(torch.bfloat16).to(gpu)
    out = ops.rms_norm(x, w, 1e-6)
    assert out.is_contiguous()
    check(out, onorm.rms_norm_f32(f32(x), f32(w), 1e-6), torch.bfloat16, 0.03125)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("tokens", [1, 3, 65])
@pytest.mark.parametrize("width", [13, 1024, 4096])
def test_add_rms_norm_matches_fp32_sum(gpu, dtype, tokens, width):
    g = torch.Generator().manual_seed(19 + tokens + width)
    x = torch.randn(tokens, width, generator=g).to(dtype).to(gpu)
    r = torch.randn(tokens, width, generator=g).to(dtype).to(gpu)
    w = torch.randn(width, generator=g).to(dtype).to(gpu)
    want_out, want_sum = onorm.add_rms_norm_f32(f32(x), f32(r), f32(w), 1e-6)
    xp, rp = x.data_ptr(), r.data_ptr()
    out, summed = ops.add_rms_norm(x, r, w, 1e-6)
    assert out.data_ptr() == xp and summed.data_ptr() == rp
    np.testing.assert_array_equal(f32(summed), obf.round_to(want_sum, NAME[dtype]))
    check(out, want_out, dtype, TOL[dtype][1])


def test_add_rms_norm_residual_fixture(gpu, fixtures):
    fx = fixtures["add_rms_norm_residual"]
    w = fx["width"]
    x = torch.full((1, w), fx["x"], dtype=torch.bfloat16, device=gpu)
    r = torch.tensor(fx["residual_pattern"]).repeat(w // 2)[None].to(torch.bfloat16).to(gpu)
    weight = torch.full((w,), fx["weight"], dtype=torch.bfloat16, device=gpu)
    out, s = ops.add_rms_norm(x, r, weight, fx["eps"])
    assert bool((out == fx["expected_out"]).all())
    assert f32(s)[0, :2].tolist() == fx["expected_residual_head"]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("padding", [1, 16])
def test_add_rms_norm_padded_rows_untouched(gpu, dtype, padding):
    g = torch.Generator().manual_seed(41 + padding)
    storage = torch.randn(5, 1024 + padding, generator=g).to(dtype).to(gpu)
    rstore = torch.randn(5, 1024 + padding, generator=g).to(dtype).to(gpu)
    x, r = storage[:, :1024], rstore[:, :1024]
    w = torch.randn(1024, generator=g).to(dtype).to(gpu)
    pad_x, pad_r = storage[:, 1024:].clone(), rstore[:, 1024:].clone()
    want_out, want_sum = onorm.add_rms_norm_f32(f32(x), f32(r), f32(w), 1e-6)
    out, s = ops.add_rms_norm(x, r, w, 1e-6)
    np.testing.assert_array_equal(f32(s), obf.round_to(want_sum, NAME[dtype]))
    check(out, want_out, dtype, TOL[dtype][1])
    assert torch.equal(storage[:, 1024:], pad_x) and torch.equal(rstore[:, 1024:], pad_r)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_qk_norm_packed_qkv_leaves_v(gpu, dtype):
    g = torch.Generator().manual_seed(7)
    packed = torch.randn(3, 4096, generator=g).to(dtype).to(gpu)
    q = packed[:, :2048].view(3, 16, 128)
    k = packed[:, 2048:3072].view(3, 8, 128)
    qw = torch.randn(128, generator=g).to(dtype).to(gpu)
    kw = torch.randn(128, generator=g).to(dtype).to(gpu)
    want_q, want_k = onorm.qk_norm_f32(f32(q), f32(k), f32(qw), f32(kw), 1e-6)
    v_before = packed[:, 3072:].clone()
    qp, kp = q.data_ptr(), k.data_ptr()
    qn, kn = ops.qk_norm(q, k, qw, kw, 1e-6)
    assert qn.data_ptr() == qp and kn.data_ptr() == kp
    check(qn, want_q, dtype, TOL[dtype][0])
    check(kn, want_k, dtype, TOL[dtype][0])
    assert torch.equal(packed[:, 3072:], v_before)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_qk_norm_partial_heads(gpu, dtype):
    g = torch.Generator().manual_seed(43)
    packed = torch.randn(3, 7, 128, generator=g).to(dtype).to(gpu)
    q, k = packed[:, 0:3], packed[:, 3:5]
    v_before = packed[:, 5:7].clone()
    qw = torch.randn(128, generator=g).to(dtype).to(gpu)
    kw = torch.randn(128, generator=g).to(dtype).to(gpu)
    want_q, want_k = onorm.qk_norm_f32(f32(q), f32(k), f32(qw), f32(kw), 1e-6)
    ops.qk_norm(q, k, qw, kw, 1e-6)
    check(q, want_q, dtype, TOL[dtype][0])
    check(k, want_k, dtype, TOL[dtype][0])
    assert torch.equal(packed[:, 5:7], v_before)


def test_config3_norm_shapes(gpu):
    """8192 x 1024 hidden rows and the 8k-token packed QKV of the prefill config."""
    g = torch.Generator().manual_seed(33)
    x = torch.randn(8192, 1024, generator=g).to(torch.bfloat16).to(gpu)
    r = torch.randn(8192, 1024, generator=g).to(torch.bfloat16).to(gpu)
    w = torch.empty(1024).uniform_(0.5, 1.5, generator=g).to(torch.bfloat16).to(gpu)
    check(ops.rms_norm(x, w, 1e-6), onorm.rms_norm_f32(f32(x), f32(w), 1e-6), torch.bfloat16,
          0.03125)
    want_out, want_sum = onorm.add_rms_norm_f32(f32(x), f32(r), f32(w), 1e-6)
    ops.add_rms_norm(x, r, w, 1e-6)
    np.testing.assert_array_equal(f32(r), obf.round_bf16(want_sum))
    check(x, want_out, torch.bfloat16, 0.0625)
    packed = torch.randn(8192, 4096, generator=g).to(torch.bfloat16).to(gpu)
    q = packed[:, :2048].view(-1, 16, 128)
    k = packed[:, 2048:3072].view(-1, 8, 128)
    qw = torch.empty(128).uniform_(0.5, 1.5, generator=g).to(torch.bfloat16).to(gpu)
    kw = torch.empty(128).uniform_(0.5, 1.5, generator=g).to(torch.bfloat16).to(gpu)
    want_q, want_k = onorm.qk_norm_f32(f32(q), f32(k), f32(qw), f32(kw), 1e-6)
    vb = packed[:, 3072:].clone()
    ops.qk_norm(q, k, qw, kw, 1e-6)
    check(q, want_q, torch.bfloat16, 0.03125)
    check(k, want_k, torch.bfloat16, 0.03125)
    assert torch.equal(packed[:, 3072:], vb)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_qk_norm_many_rows_with_a_ragged_tail(gpu, dtype):
    """1,367 tokens x (16 + 8) heads = 32,808 head rows: the multi-row narrow kernel, with a
    last workgroup that is only partly filled (32,808 is not a multiple of its 32 rows)."""
    g = torch.Generator().manual_seed(47)
    packed = torch.randn(1367, 4096, generator=g).to(dtype).to(gpu)
    q = packed[:, :2048].view(-1, 16, 128)
    k = packed[:, 2048:3072].view(-1, 8, 128)
    qw = torch.empty(128).uniform_(0.5, 1.5, generator=g).to(dtype).to(gpu)
    kw = torch.empty(128).uniform_(0.5, 1.5, generator=g).to(dtype).to(gpu)
    want_q, want_k = onorm.qk_norm_f32(f32(q), f32(k), f32(qw), f32(kw), 1e-6)
    vb = packed[:, 3072:].clone()
    ops.qk_norm(q, k, qw, kw, 1e-6)
    check(q, want_q, dtype, TOL[dtype][0])
    check(k, want_k, dtype, TOL[dtype][0])
    assert torch.equal(packed[:, 3072:], vb)


def check_rel(actual, expected_f32, dtype, tol):
    """`check` with the absolute bound widened to one unit in the last place of large outputs
    (the spike row normalises to ~64, where a bf16 ulp is 0.5)."""
    want = obf.round_to(expected_f32, NAME[dtype])
    got = f32(actual)
    ulp = 2.0 ** (-7 if dtype == torch.bfloat16 else -10)
    bound = np.maximum(tol, ulp * np.abs(want))
    assert (np.abs(got - want) <= bound).all(), float((np.abs(got - want) - bound).max())
    assert cos(got, expected_f32) > 0.9999


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_norms_on_pathological_rows(gpu, dtype):
    """All-zero rows (rsqrt(eps) times 0 = 0), one large element among small ones (the sum of
    squares must not lose the small ones' share of the output), large magnitudes (bf16 / fp16
    values near 200, squares summed in fp32) and tiny magnitudes (values ~1e-3, where eps
    dominates): RMSNorm, add-RMSNorm and QK-norm against the fp32 oracle."""
    g = torch.Generator().manual_seed(77)
    width = 4096
    rows = [torch.zeros(width), torch.randn(width, generator=g) * 1e-3,
            torch.randn(width, generator=g) * 200]
    spike = torch.randn(width, generator=g) * 0.01
    spike[1234] = 150.0
    rows.append(spike)
    x = torch.stack(rows).to(dtype).to(gpu)
    w = torch.empty(width).uniform_(0.5, 1.5, generator=g).to(dtype).to(gpu)
    out = ops.rms_norm(x, w, 1e-6)
    assert bool(torch.isfinite(out).all()) and bool((out[0] == 0).all())
    check_rel(out, onorm.rms_norm_f32(f32(x), f32(w), 1e-6), dtype, TOL[dtype][0])
    r = torch.flip(x, [0]).contiguous()
    want_out, want_sum = onorm.add_rms_norm_f32(f32(x), f32(r), f32(w), 1e-6)
    out, summed = ops.add_rms_norm(x.clone(), r, w, 1e-6)
    np.testing.assert_array_equal(f32(summed), obf.round_to(want_sum, NAME[dtype]))
    check_rel(out, want_out, dtype, TOL[dtype][1])
    # QK-norm: the same rows as heads of width 128 (zero heads, spike heads, tiny heads)
    q = x.view(4, 32, 128).clone()
    k = x.view(4, 32, 128)[:, :8].clone()
    qw = w[:128].contiguous()
    kw = w[128:256].contiguous()
    want_q = onorm.rms_norm_f32(f32(q).reshape(-1, 128), f32(qw), 1e-6)
    want_k = onorm.rms_norm_f32(f32(k).reshape(-1, 128), f32(kw), 1e-6)
    ops.qk_norm(q, k, qw, kw, 1e-6)
    check_rel(q.reshape(-1, 128), want_q, dtype, TOL[dtype][0])
    check_rel(k.reshape(-1, 128), want_k, dtype, TOL[dtype][0])
