"""Attention oracle (test infrastructure only).

numpy float64 restatements of the reference's libtorch eager attention:
  attention_against_cache  src/models/attention/backend.rs:1463-1498
  blocked_attention_mask   backend.rs:1455-1461 (key j blocked iff j > prefix + i)
  decode_with_cache        backend.rs:1331-1371 (per-request gather + attention,
                           query at position len-1 sees every cached key)
  prefill_ragged           backend.rs:898-911  (pt backend, no prefix)
  prefill_with_cache       backend.rs:1297-1329 (cached prefix, bottom-right causal)
Slots of a paged request follow the page table: token j of request r lives in
slot table[r, j // P] * P + j % P (flashinfer_bridge.cpp:108-118 pages; the
KV pool layout of src/engine/kvcache/pool.rs:81-104).

The torch-CPU fp32 functions (``*_torch``: decode, ragged prefill, prefill over a
cached prefix) restate the same reference CPU path op for op in libtorch
(index_select, repeat_interleave, bmm, masked_fill, softmax); they are the timed
CPU baseline, not a checker.
"""
from __future__ import annotations

import math

import numpy as np


def blocked_attention_mask(query_len: int, key_len: int, prefix: int) -> np.ndarray:
    qpos = np.arange(query_len)[:, None] + prefix
    kpos = np.arange(key_len)[None, :]
    return kpos > qpos


def attention_against_cache(q: np.ndarray, k: np.ndarray, v: np.ndarray, prefix_len: int,
                            num_heads: int, num_kv_heads: int,
                            blocked: np.ndarray | None = None) -> np.ndarray:
    """q [Lq, Hq, D], k/v [Lk, Hkv, D] -> [Lq, Hq, D] in float64."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    lq, _, d = q.shape
    group = num_heads // num_kv_heads
    kk = np.repeat(k, group, axis=1)  # repeat_interleave over the head axis
    vv = np.repeat(v, group, axis=1)
    if blocked is None:
        blocked = blocked_attention_mask(lq, k.shape[0], prefix_len)
    # [H, Lq, D] @ [H, D, Lk] through BLAS matmul
    scores = np.matmul(q.transpose(1, 0, 2), kk.transpose(1, 2, 0)) * (1.0 / math.sqrt(d))
    scores = np.where(blocked[None, :, :], -np.inf, scores)
    mx = scores.max(axis=-1, keepdims=True)
    p = np.exp(scores - mx)
    p /= p.sum(axis=-1, keepdims=True)
    return np.matmul(p, vv.transpose(1, 0, 2)).transpose(1, 0, 2)


def slots_of(table_row: np.ndarray, length: int, page_size: int) -> np.ndarray:
    j = np.arange(length)
    return np.asarray(table_row, np.int64)[j // page_size] * page_size + j % page_size


def decode_with_cache(q: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
                      block_table: np.ndarray, lengths, page_size: int) -> np.ndarray:
    """q [B, Hq, D]; caches [pages, P, Hkv, D]; one query per request at position len-1."""
    b, hq, d = q.shape
    hkv = k_cache.shape[2]
    flat_k = k_cache.reshape(-1, hkv, d)
    flat_v = v_cache.reshape(-1, hkv, d)
    out = np.empty((b, hq, d), np.float64)
    for r in range(b):
        length = int(lengths[r])
        if length <= 0:
            raise ValueError("cache_seqlens must be positive")
        s = slots_of(block_table[r], length, page_size)
        out[r] = attention_against_cache(q[r:r + 1], flat_k[s], flat_v[s], length - 1, hq,
                                         hkv)[0]
    return out


def prefill_ragged(q: np.ndarray, k: np.ndarray, v: np.ndarray, cu_seqlens) -> np.ndarray:
    """q [N, Hq, D], k/v [N, Hkv, D]; causal attention within each sequence."""
    out = np.empty(q.shape, np.float64)
    hq, hkv = q.shape[1], k.shape[1]
    for s, e in zip(list(cu_seqlens)[:-1], list(cu_seqlens)[1:]):
        out[s:e] = attention_against_cache(q[s:e], k[s:e], v[s:e], 0, hq, hkv)
    return out


def prefill_with_cache(q: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
                       block_table: np.ndarray, cu_seqlens, prefixes,
                       page_size: int) -> np.ndarray:
    """Extend queries over prefix + extend keys read from the paged cache."""
    hq, d = q.shape[1], q.shape[2]
    hkv = k_cache.shape[2]
    flat_k = k_cache.reshape(-1, hkv, d)
    flat_v = v_cache.reshape(-1, hkv, d)
    out = np.empty(q.shape, np.float64)
    bounds = list(cu_seqlens)
    for r, (s, e) in enumerate(zip(bounds[:-1], bounds[1:])):
        prefix = int(prefixes[r])
        slots = slots_of(block_table[r], prefix + e - s, page_size)
        out[s:e] = attention_against_cache(q[s:e], flat_k[slots], flat_v[slots], prefix, hq, hkv)
    return out


def brute_force_attention(q, k, v, visible, scale):
    """Pure-Python loops for tiny shapes: q [Lq][D], k/v [Lk][D], visible[i][j] bool."""
    out = []
    for i, qi in enumerate(q):
        scores = [sum(a * b for a, b in zip(qi, kj)) * scale if visible[i][j] else None
                  for j, kj in enumerate(k)]
        mx = max(s for s in scores if s is not None)
        w = [math.exp(s - mx) if s is not None else 0.0 for s in scores]
        tot = sum(w)
        out.append([sum(w[j] * v[j][c] for j in range(len(k))) / tot for c in range(len(v[0]))])
    return out


# ---------------------------------------------------------------------------
# torch-CPU fp32 restatement (timed CPU baseline)
# ---------------------------------------------------------------------------
def attention_against_cache_torch(q, k, v, prefix_len: int, num_heads: int, num_kv_heads: int):
    import torch

    lq = q.size(0)
    qt = q.transpose(0, 1)
    rep = num_heads // num_kv_heads
    kt = k.transpose(0, 1).repeat_interleave(rep, dim=0)
    vt = v.transpose(0, 1).repeat_interleave(rep, dim=0)
    qpos = torch.arange(lq) + prefix_len
    kpos = torch.arange(k.size(0))
    blocked = kpos.unsqueeze(0) > qpos.unsqueeze(1)
    scale = 1.0 / math.sqrt(q.size(-1))
    s = torch.bmm(qt, kt.transpose(1, 2)) * scale
    s = s.masked_fill(blocked.unsqueeze(0), float("-inf")).softmax(-1)
    return torch.bmm(s, vt).transpose(0, 1).reshape(lq, num_heads * q.size(-1))


def decode_with_cache_torch(q, k_cache, v_cache, block_table, lengths, page_size: int):
    """Per-request gather + attention, fp32 libtorch on CPU (backend.rs:1331-1371)."""
    import torch

    b, hq, d = q.shape
    hkv = k_cache.size(2)
    flat_k = k_cache.view(-1, hkv, d)
    flat_v = v_cache.view(-1, hkv, d)
    outs = []
    for r in range(b):
        length = int(lengths[r])
        j = torch.arange(length)
        slots = block_table[r].long()[j // page_size] * page_size + j % page_size
        ck = flat_k.index_select(0, slots)
        cv = flat_v.index_select(0, slots)
        outs.append(attention_against_cache_torch(q[r:r + 1], ck, cv, length - 1, hq, hkv))
    return torch.cat(outs, 0)


def prefill_ragged_torch(q, k, v, cu_seqlens):
    """Per-sequence causal attention, fp32 libtorch on CPU (the reference's SDPA prefill
    plan, backend.rs:981-1142, without a cached prefix)."""
    import torch

    hq, hkv = q.size(1), k.size(1)
    outs = []
    for s, e in zip(list(cu_seqlens)[:-1], list(cu_seqlens)[1:]):
        outs.append(attention_against_cache_torch(q[s:e], k[s:e], v[s:e], 0, hq, hkv))
    return torch.cat(outs, 0)


def prefill_with_cache_torch(q, k_cache, v_cache, block_table, cu_seqlens, prefixes,
                             page_size: int):
    """Extend queries over prefix + extend keys gathered from the paged cache, fp32 libtorch
    on CPU (backend.rs:1297-1329)."""
    import torch

    hq, hkv, d = q.size(1), k_cache.size(2), q.size(2)
    flat_k = k_cache.view(-1, hkv, d)
    flat_v = v_cache.view(-1, hkv, d)
    outs = []
    for r, (s, e) in enumerate(zip(list(cu_seqlens)[:-1], list(cu_seqlens)[1:])):
        length = int(prefixes[r]) + (e - s)
        j = torch.arange(length)
        slots = block_table[r].long()[j // page_size] * page_size + j % page_size
        outs.append(attention_against_cache_torch(q[s:e], flat_k.index_select(0, slots),
                                                  flat_v.index_select(0, slots),
                                                  int(prefixes[r]), hq, hkv))
    return torch.cat(outs, 0)
