"""mi355x_linear_noalloc (split-K partials in the library's per-GPU scratch array) against
mi355x_linear (partials in a caller workspace), called through the C ABI: bit-identical
outputs on two calls in a row, the second smaller, plus the size limit."""
import ctypes

import pytest
import torch

from llm_infer_rust_amd import _native

pytestmark = pytest.mark.gpu


def _call_linear(lib, x, w, out, ws, cus, stream):
    m, k = x.shape
    n = w.shape[0]
    err = lib.mi355x_linear(x.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0),
                            out.data_ptr(), out.stride(0), m, n, k,
                            None if ws is None else ws.data_ptr(),
                            0 if ws is None else ws.numel(), cus, -1, -1, 0, stream)
    assert err is None, err


def _call_noalloc(lib, x, w, out, cus, stream):
    m, k = x.shape
    n = w.shape[0]
    return lib.mi355x_linear_noalloc(x.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0),
                                     out.data_ptr(), out.stride(0), m, n, k, cus, -1, -1, 0,
                                     stream)


def test_noalloc_linear_matches_workspace_linear(gpu):
    lib = _native.lib()
    cus = _native.device_cus(gpu)
    stream = torch.cuda.current_stream().cuda_stream
    g = torch.Generator().manual_seed(5)
    # QKV of a Qwen3-8B decode step at 256 rows (split K), then a smaller o_proj-like call.
    needs = {}
    for m, n, k in ((256, 6144, 4096), (64, 4096, 4096), (37, 1024, 4096)):
        need = lib.mi355x_linear_workspace_bytes(m, n, k, cus, -1, -1)
        needs[m] = need
        print(f"[noalloc] m={m} n={n} k={k} split-K bytes={need}", flush=True)
        x = torch.randn(m, k, generator=g).to(torch.bfloat16).to(gpu)
        w = (torch.randn(n, k, generator=g) * 0.05).to(torch.bfloat16).to(gpu)
        ws = torch.empty(max(need, 16), dtype=torch.uint8, device=gpu) if need else None
        want = torch.empty(m, n, dtype=torch.bfloat16, device=gpu)
        got = torch.full((m, n), 7.0, dtype=torch.bfloat16, device=gpu)
        _call_linear(lib, x, w, want, ws, cus, stream)
        err = _call_noalloc(lib, x, w, got, cus, stream)
        assert err is None, err
        torch.cuda.synchronize()
        assert torch.equal(got, want), (m, n, k)
    # The 256-row QKV call splits K, so its partials went through the scratch array.
    assert needs[256] > 0, needs


def test_noalloc_linear_refuses_oversized_partials(gpu):
    lib = _native.lib()
    stream = torch.cuda.current_stream().cuda_stream
    # Forced 4-way split of a 4096 x 4096 product: 256 MiB of partials > 32 MiB.
    m, n, k = 4096, 4096, 4096
    assert lib.mi355x_linear_workspace_bytes(m, n, k, 256, 0, 4) > 32 << 20
    x = torch.zeros(m, k, dtype=torch.bfloat16, device=gpu)
    w = torch.zeros(n, k, dtype=torch.bfloat16, device=gpu)
    out = torch.zeros(m, n, dtype=torch.bfloat16, device=gpu)
    err = lib.mi355x_linear_noalloc(x.data_ptr(), k, w.data_ptr(), k, out.data_ptr(), n, m, n,
                                    k, 256, 0, 4, 0, stream)
    assert err is not None and b"32 MiB" in err
