"""Host-side seam logic that needs no GPU: backend parsing/validation and the
per-invocation prefill snapshot (CPU only)."""
import pytest
import torch

from llm_infer_rust_amd.backend import (Attention, AttentionBackendKind, AttentionMetadata,
                                        AttentionSpec, BatchPhase, PrefillMetadata)
from llm_infer_rust_amd.kv_cache import BaseAttention, KVCacheLayout, ModelError


def test_backend_kind_parse():
    assert AttentionBackendKind.parse("MI355X") == AttentionBackendKind.MI355X
    assert AttentionBackendKind.parse("hip") == AttentionBackendKind.MI355X
    assert AttentionBackendKind.parse("pytorch") == AttentionBackendKind.PT
    assert AttentionBackendKind.parse("flash-attention") == AttentionBackendKind.FLASH_ATTENTION
    assert AttentionBackendKind.parse("flashinfer") == AttentionBackendKind.FLASHINFER
    with pytest.raises(ModelError, match="unknown attention backend"):
        AttentionBackendKind.parse("triton")


def _spec(**kw):
    base = dict(num_heads=16, num_kv_heads=8, head_dim=128, dtype=torch.bfloat16,
                device=torch.device("cuda", 0))
    base.update(kw)
    return AttentionSpec(**base)


def test_validate_rejects_unsupported_geometry():
    with pytest.raises(ModelError, match="head_dim=128"):
        Attention.validate("mi355x", _spec(head_dim=64))
    with pytest.raises(ModelError, match="GPU"):
        Attention.validate("mi355x", _spec(device=torch.device("cpu")))
    with pytest.raises(ModelError, match="GPU"):
        Attention.validate("mi355x", _spec(dtype=torch.float32))
    with pytest.raises(ModelError, match="query heads per kv head"):
        Attention.validate("mi355x", _spec(num_heads=24, num_kv_heads=8))
    with pytest.raises(ModelError, match="not provided"):
        Attention.validate("flashinfer", _spec())


def test_prefill_snapshot_validation():
    meta = AttentionMetadata(BatchPhase.PREFILL, cu_seqlens_q=torch.tensor([0, 2, 3],
                                                                          dtype=torch.int32),
                             prefix_lens=torch.tensor([1, 0], dtype=torch.int32))
    snap = PrefillMetadata.prepare(meta, 3)
    assert snap.boundaries == [0, 2, 3] and snap.prefixes == [1, 0] and snap.has_prefix()
    with pytest.raises(ModelError, match="cu_seqlens_q"):
        PrefillMetadata.prepare(meta, 4)
    bad = AttentionMetadata(BatchPhase.PREFILL, cu_seqlens_q=torch.tensor([0, 2, 2],
                                                                         dtype=torch.int32),
                            prefix_lens=torch.tensor([0, 0], dtype=torch.int32))
    with pytest.raises(ModelError, match="cu_seqlens_q"):
        PrefillMetadata.prepare(bad, 2)
    neg = AttentionMetadata(BatchPhase.PREFILL, cu_seqlens_q=torch.tensor([0, 2],
                                                                         dtype=torch.int32),
                            prefix_lens=torch.tensor([-1], dtype=torch.int32))
    with pytest.raises(ModelError, match="prefix"):
        PrefillMetadata.prepare(neg, 2)
    dec = PrefillMetadata.prepare(AttentionMetadata(BatchPhase.DECODE), 5)
    assert dec.boundaries == [0, 5] and dec.prefixes == [0]


def test_base_attention_shape_checks_precede_device_work():
    att = BaseAttention()
    att.write_kv(torch.zeros(1, 1, 2), torch.zeros(1, 1, 2), None)  # unbound: no-op
    with pytest.raises(ModelError):
        att.bind_kv_cache(torch.zeros(2, 2, 1, 2), torch.zeros(2, 2, 1, 3))
    att.k_cache = torch.zeros(2, 2, 1, 2)
    att.v_cache = torch.zeros(2, 2, 1, 2)
    with pytest.raises(ModelError, match="matching"):
        att.write_kv(torch.zeros(1, 1, 2), torch.zeros(2, 1, 2), torch.zeros(1))
    with pytest.raises(ModelError, match="write_loc length"):
        att.write_kv(torch.zeros(1, 1, 2), torch.zeros(1, 1, 2), torch.zeros(2))
    with pytest.raises(ModelError, match="head shape"):
        att.write_kv(torch.zeros(1, 2, 2), torch.zeros(1, 2, 2), torch.zeros(1))


def test_kv_pool_layout():
    assert KVCacheLayout(28, 100, 16, 8, 128).tensor_shape() == (2, 28, 101, 16, 8, 128)
    with pytest.raises(ModelError):
        KVCacheLayout(28, 0, 16, 8, 128).tensor_shape()


def test_fused_qkv_route_checks_the_weight_shape():
    """``ops.linear_qk_norm_rope_store`` derives head_dim from the QKV weight: rows that are not
    a whole number of (Hq + 2 Hkv) heads are refused before anything runs."""
    import torch

    from llm_infer_rust_amd import ops
    from llm_infer_rust_amd._native import NativeError

    x = torch.zeros(4, 64)
    with pytest.raises(NativeError, match="q_heads \\+ 2 k_heads"):
        ops.linear_qk_norm_rope_store(x, torch.zeros(3 * 128 + 1, 64), 1, 1, None, None, 1e-6,
                                      None, None, None, None)
    with pytest.raises(NativeError, match="q_heads \\+ 2 k_heads"):
        ops.linear_qk_norm_rope_store(x, torch.zeros(512, 64), 0, 2, None, None, 1e-6, None,
                                      None, None, None)


def test_default_decode_graph_buckets():
    """Decode graphs are captured for 1, 2, 4, 8 and every multiple of 8 up to the running
    limit, so a partly filled step carries at most 7 pad rows; explicit sizes are kept."""
    from llm_infer_rust_amd.engine import Engine, EngineConfig

    eng = Engine.__new__(Engine)  # the bucket rule needs only the config
    eng.cfg = EngineConfig()
    sizes = eng._bucket_sizes()
    assert sizes[:5] == [1, 2, 4, 8, 16] and sizes[-1] == 256 and len(sizes) == 35
    assert all(b - a <= 8 for a, b in zip(sizes, sizes[1:]))
    eng.cfg = EngineConfig(max_running_req=20)
    assert eng._bucket_sizes() == [1, 2, 4, 8, 16, 20]
    eng.cfg = EngineConfig(max_running_req=3)
    assert eng._bucket_sizes() == [1, 2, 3]
    eng.cfg = EngineConfig(graph_batch_sizes=(4, 1, 4))
    assert eng._bucket_sizes() == [1, 4]
