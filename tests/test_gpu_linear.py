"""Decode-batch projection kernel (mi355x_linear) against a float64 product.

The kernel accumulates in fp32 and rounds once, like hipBLASLt and the reference's
cuBLAS matmul (src/layers/linear.rs:5-7). Tolerance: every element within one unit in
the last place of the output dtype of the float64 value plus the fp32 accumulation
bound (K * 2^-24 * sum |x||w|), and cosine similarity > 0.99999.
"""
import pytest
import torch
import torch.nn.functional as F

from llm_infer_rust_amd import ops
from llm_infer_rust_amd._native import NativeError, lib

pytestmark = pytest.mark.gpu

MANTISSA = {torch.bfloat16: 8, torch.float16: 11}
N_CONFIGS = 8  # tile shapes compiled into the library


def operands(m, n, k, dtype, gpu, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=g).to(dtype).to(gpu)
    w = (torch.randn(n, k, generator=g) * 0.05).to(dtype).to(gpu)
    return x, w


def check_product(out, x, w):
    ref = x.double() @ w.double().T
    bound = (x.double().abs() @ w.double().abs().T) * (x.size(1) * 2.0 ** -24)
    ulp = ref.abs().clamp_min(2.0 ** -14) * 2.0 ** (1 - MANTISSA[out.dtype])
    err = (out.double() - ref).abs()
    bad = err > ulp + bound
    assert not bool(bad.any()), (float(err.max()), int(bad.sum()))
    a, b = out.double().flatten(), ref.flatten()
    assert float(a @ b / (a.norm() * b.norm() + 1e-30)) > 0.99999


@pytest.mark.parametrize("m", [1, 5, 64, 200, 256])
@pytest.mark.parametrize("n,k", [(6144, 4096), (4096, 4096), (4096, 12288)])
def test_qwen3_8b_decode_projections(gpu, m, n, k):
    x, w = operands(m, n, k, torch.bfloat16, gpu, m + n + k)
    check_product(ops.decode_linear(x, w), x, w)


@pytest.mark.parametrize("config", range(N_CONFIGS))
@pytest.mark.parametrize("splits", [1, 2, 4])
def test_every_tiling_with_ragged_edges(gpu, config, splits):
    """M and N not multiples of any tile (rows and columns past the edge are clamped on
    load and skipped on store); K split into 1, 2 or 4 ranges."""
    x, w = operands(97, 388, 1024, torch.bfloat16, gpu, 10 * config + splits)
    check_product(ops.decode_linear(x, w, config=config, splits=splits), x, w)


def test_float16_and_strided_operands(gpu):
    base_x, w = operands(40, 260, 640, torch.float16, gpu, 7)
    wide = torch.zeros(40, 640 + 64, dtype=torch.float16, device=gpu)
    wide[:, 32:32 + 640] = base_x
    x = wide[:, 32:32 + 640]  # row stride 704, 64-byte offset
    out_wide = torch.full((40, 300), 7.0, dtype=torch.float16, device=gpu)
    out = out_wide[:, 20:280]
    ops.decode_linear(x, w, out=out)
    check_product(out, base_x, w)
    assert bool((out_wide[:, :20] == 7).all()) and bool((out_wide[:, 280:] == 7).all())


def test_split_partials_reduce_to_the_unsplit_result(gpu):
    x, w = operands(128, 512, 2048, torch.bfloat16, gpu, 3)
    one = ops.decode_linear(x, w, config=6, splits=1)
    for s in (2, 4, 8):
        many = ops.decode_linear(x, w, config=6, splits=s)
        check_product(many, x, w)
        # fp32 partial sums differ from one pass only by fp32 rounding: within one ulp
        diff = (many.float() - one.float()).abs()
        assert float(diff.max()) <= float(one.float().abs().max()) * 2.0 ** -7


def test_rejected_shapes_and_workspace(gpu):
    x, w = operands(8, 64, 96, torch.bfloat16, gpu, 1)  # K % 64 != 0
    with pytest.raises(NativeError, match="unsupported shape"):
        ops.decode_linear(x, w)
    x, w = operands(8, 66, 128, torch.bfloat16, gpu, 1)  # N % 4 != 0
    with pytest.raises(NativeError, match="unsupported shape"):
        ops.decode_linear(x, w)
    x, w = operands(64, 256, 1024, torch.bfloat16, gpu, 1)
    out = torch.empty(64, 256, dtype=torch.bfloat16, device=gpu)
    small = torch.empty(1024, dtype=torch.uint8, device=gpu)
    err = lib().mi355x_linear(x.data_ptr(), 1024, w.data_ptr(), 1024, out.data_ptr(), 256, 64,
                              256, 1024, small.data_ptr(), small.numel(), 256, 6, 4, 0,
                              torch.cuda.current_stream().cuda_stream)
    assert err is not None and b"workspace" in err


def test_routing_policy(gpu):
    """QKV / o_proj / down at decode sizes take the kernel; gate_up, lm_head and
    prefill-sized products stay on hipBLASLt (identical to F.linear)."""
    assert ops.uses_decode_kernel(256, 6144, 4096)
    assert ops.uses_decode_kernel(1, 4096, 4096)
    assert ops.uses_decode_kernel(256, 4096, 12288)
    assert not ops.uses_decode_kernel(8, 4096, 12288)
    assert not ops.uses_decode_kernel(256, 24576, 4096)
    assert not ops.uses_decode_kernel(257, 6144, 4096)
    x, w = operands(300, 256, 512, torch.bfloat16, gpu, 5)
    assert torch.equal(ops.linear(x, w), F.linear(x, w))
    x, w = operands(100, 256, 512, torch.bfloat16, gpu, 6)
    assert torch.equal(ops.linear(x, w), ops.decode_linear(x, w))


def test_graph_replays_match_eager(gpu):
    """Captured split-K launches (workspace from the graph's pool) replayed several times
    with eager work in between; every replay equals the eager result."""
    x, w = operands(256, 4096, 4096, torch.bfloat16, gpu, 11)
    eager = ops.decode_linear(x, w).clone()
    static_out = torch.empty_like(eager)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        ops.decode_linear(x, w, out=static_out)  # warm the allocator off the capture
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ops.decode_linear(x, w, out=static_out)
    for i in range(4):
        static_out.fill_(float(i))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(static_out, eager), f"replay {i}"
        _ = ops.decode_linear(x, w * 0.5)  # eager work reusing the allocator between replays
        torch.cuda.synchronize()



@pytest.mark.parametrize("m,n,k,dtype", [(256, 4096, 4096, torch.bfloat16),
                                         (256, 4096, 12288, torch.bfloat16),
                                         (100, 2048, 1024, torch.bfloat16),
                                         (1, 4096, 4096, torch.bfloat16),
                                         (64, 2048, 64, torch.bfloat16),
                                         (256, 4096, 4096, torch.float16),
                                         (64, 2048, 64, torch.float16)])
def test_fused_residual_norm_equals_separate_passes(gpu, m, n, k, dtype):
    """mi355x_linear_add_rms_norm == decode_linear then add_rms_norm, bit for bit, for split
    (fp32 partials reduced in the norm pass) and unsplit (K = 64) projections, in bf16 and
    fp16."""
    x, w = operands(m, n, k, dtype, gpu, m * 7 + n + k)
    g = torch.Generator().manual_seed(n + k)
    residual = torch.randn(m, n, generator=g).to(dtype).to(gpu)
    gamma = (torch.rand(n, generator=g) + 0.5).to(dtype).to(gpu)
    res_sep = residual.clone()
    y = ops.decode_linear(x, w)
    want, _ = ops.add_rms_norm(y, res_sep, gamma, 1e-6)
    res_fused = residual.clone()
    got, res_out = ops.linear_add_rms_norm(x, w, res_fused, gamma, 1e-6)
    assert res_out.data_ptr() == res_fused.data_ptr()
    assert torch.equal(res_fused, res_sep)
    assert torch.equal(got, want)


def test_fused_residual_norm_falls_back_outside_decode_sizes(gpu):
    """Prefill-sized rows (or widths the fused pass does not take) run the two steps."""
    x, w = operands(300, 1024, 512, torch.bfloat16, gpu, 9)
    g = torch.Generator().manual_seed(9)
    residual = torch.randn(300, 1024, generator=g).to(torch.bfloat16).to(gpu)
    gamma = (torch.rand(1024, generator=g) + 0.5).to(torch.bfloat16).to(gpu)
    res_a, res_b = residual.clone(), residual.clone()
    got, _ = ops.linear_add_rms_norm(x, w, res_a, gamma, 1e-6)
    want, _ = ops.add_rms_norm(F.linear(x, w), res_b, gamma, 1e-6)
    assert torch.equal(got, want) and torch.equal(res_a, res_b)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("config", [0, 6, 7])
@pytest.mark.parametrize("m,width,k", [(256, 12288, 4096), (1, 12288, 4096), (97, 1000, 512),
                                       (64, 196, 128)])
def test_fused_gate_up_silu_equals_two_steps(gpu, config, m, width, k, dtype):
    """mi355x_linear_silu_mul == decode_linear (same tiling, K unsplit) then silu_and_mul,
    bit for bit, including widths that end inside a tile and ragged rows, in bf16 and fp16;
    and within the tolerance of silu(g) * u on the float64 product."""
    x, w = operands(m, 2 * width, k, dtype, gpu, m + width + k + config)
    fused = ops.decode_linear_silu_mul(x, w, config=config)
    two_step = ops.silu_and_mul(ops.decode_linear(x, w, config=config, splits=1))
    assert torch.equal(fused, two_step)
    y = x.double() @ w.double().T
    g, u = y[:, :width], y[:, width:]
    want = g * torch.sigmoid(g) * u
    a, b = fused.double().flatten(), want.flatten()
    assert float(a @ b / (a.norm() * b.norm() + 1e-30)) > 0.9999
    assert float((fused.double() - want).abs().max()) <= 2e-2 * float(want.abs().max()) + 1e-3


def test_fused_gate_up_silu_routing_and_fallback(gpu):
    """Decode-sized products take the fused launch; prefill-sized ones run hipBLASLt then
    the SiLU pass, identical to the two calls."""
    assert ops.uses_silu_kernel(256, 12288, 4096)
    assert not ops.uses_silu_kernel(257, 12288, 4096)
    x, w = operands(300, 512, 256, torch.bfloat16, gpu, 21)
    assert torch.equal(ops.linear_silu_mul(x, w), ops.silu_and_mul(F.linear(x, w)))
    x, w = operands(40, 512, 256, torch.bfloat16, gpu, 22)
    assert torch.equal(ops.linear_silu_mul(x, w), ops.decode_linear_silu_mul(x, w))
    with pytest.raises(NativeError, match="unsupported shape"):
        ops.decode_linear_silu_mul(*operands(8, 2 * 66, 128, torch.bfloat16, gpu, 23))
    # An empty batch routes to the two-step path like F.linear.
    x0, w0 = operands(1, 512, 256, torch.bfloat16, gpu, 24)
    assert not ops.uses_silu_kernel(0, 256, 256) and not ops.uses_decode_kernel(0, 512, 256)
    assert ops.linear_silu_mul(x0[:0], w0).shape == (0, 256)
    assert ops.linear(x0[:0], w0).shape == (0, 512)
