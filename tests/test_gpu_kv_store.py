"""K/V store on the GPU through the C ABI: bit-exact against the oracle."""
import numpy as np
import pytest
import torch

from llm_infer_rust_amd.kv_cache import BaseAttention, ModelError
from oracle import kv_store as okv

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.view(torch.int16).cpu().numpy()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("width", [7, 128])
@pytest.mark.parametrize("index_dtype", [torch.int32, torch.int64])
def test_reference_fixture_packed_strides_padding_unwritten(gpu, fixtures, dtype, width,
                                                            index_dtype):
    fx = fixtures["kv_store_device"]
    torch.manual_seed(0)
    packed = torch.randn(5, 6, width, dtype=dtype, device=gpu)
    k, v = packed[:, 2:4], packed[:, 4:6]
    kc = torch.full((3, 4, 2, width), fx["k_fill"], dtype=dtype, device=gpu)
    vc = torch.full_like(kc, fx["v_fill"])
    packed_before = packed.clone()
    exp_k, exp_v = okv.write_kv(_bits(kc), _bits(vc), _bits(k), _bits(v),
                                np.array(fx["locations"]), fx["reserved"])
    att = BaseAttention()
    att.set_reserved_write_slot(fx["reserved"])
    att.bind_kv_cache(kc, vc)
    loc = torch.tensor(fx["locations"], dtype=index_dtype, device=gpu)
    att.write_kv(k, v, loc)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_bits(kc), exp_k)
    np.testing.assert_array_equal(_bits(vc), exp_v)
    assert torch.equal(packed, packed_before)
    att.check_write_errors()
    # decode: a one-token view overwrites only the selected slot
    nxt = torch.tensor([fx["decode_location"]], dtype=torch.int32, device=gpu)
    att.write_kv(k[:1], v[:1], nxt)
    exp_k, exp_v = okv.write_kv(exp_k, exp_v, _bits(k[:1]), _bits(v[:1]),
                                np.array([fx["decode_location"]]), fx["reserved"])
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_bits(kc), exp_k)
    np.testing.assert_array_equal(_bits(vc), exp_v)


def test_invalid_locations_are_reported_not_written(gpu, fixtures):
    fx = fixtures["kv_store_invalid"]
    for bad in fx["invalid_locations"]:
        kc = torch.zeros(fx["cache_shape"], dtype=torch.bfloat16, device=gpu)
        vc = torch.zeros_like(kc)
        att = BaseAttention()
        att.set_reserved_write_slot(fx["reserved"])
        att.bind_kv_cache(kc, vc)
        kv = torch.ones(1, 2, 128, dtype=torch.bfloat16, device=gpu)
        att.write_kv(kv, kv, torch.tensor([bad], dtype=torch.int32, device=gpu))
        with pytest.raises(ModelError, match="outside the bound KV cache"):
            att.check_write_errors()
        assert int(kc.abs().sum().item()) == 0 and int(vc.abs().sum().item()) == 0
        att.check_write_errors()  # the error word was cleared


def test_config2_scatter_into_large_pool(gpu):
    """64 new tokens at int64 positions of a 4M-slot pool (page size 1), bit-exact."""
    g = torch.Generator().manual_seed(2)
    slots = 1 << 22
    kc = torch.zeros(slots, 1, 8, 128, dtype=torch.bfloat16, device=gpu)
    vc = torch.zeros_like(kc)
    k = torch.randn(64, 8, 128, generator=g).to(torch.bfloat16).to(gpu)
    v = torch.randn(64, 8, 128, generator=g).to(torch.bfloat16).to(gpu)
    loc = (torch.randperm(slots - 1, generator=g)[:64] + 1).to(torch.int64).to(gpu)
    att = BaseAttention()
    att.set_reserved_write_slot(0)
    att.bind_kv_cache(kc, vc)
    att.write_kv(k, v, loc)
    torch.cuda.synchronize()
    assert torch.equal(kc[loc, 0], k) and torch.equal(vc[loc, 0], v)
    # nothing else was written: the pool sum equals the sum of the written rows
    assert int(kc.view(torch.int32).sum(dtype=torch.int64)) == \
        int(k.view(torch.int32).sum(dtype=torch.int64))
    assert int(vc.view(torch.int32).sum(dtype=torch.int64)) == \
        int(v.view(torch.int32).sum(dtype=torch.int64))
    att.check_write_errors()


def test_packed_qkv_views_and_empty(gpu):
    g = torch.Generator().manual_seed(3)
    packed = torch.randn(300, 4096, generator=g).to(torch.bfloat16).to(gpu)
    k = packed[:, 2048:3072].view(300, 8, 128)
    v = packed[:, 3072:4096].view(300, 8, 128)
    kc = torch.zeros(100, 16, 8, 128, dtype=torch.bfloat16, device=gpu)
    vc = torch.zeros_like(kc)
    loc = torch.randperm(1600, generator=g)[:300].to(torch.int32).to(gpu)
    att = BaseAttention()
    att.bind_kv_cache(kc, vc)
    att.write_kv(k, v, loc)
    att.write_kv(k[:0], v[:0], loc[:0])
    torch.cuda.synchronize()
    flat_k, flat_v = kc.view(-1, 8, 128), vc.view(-1, 8, 128)
    assert torch.equal(flat_k[loc.long()], k) and torch.equal(flat_v[loc.long()], v)
