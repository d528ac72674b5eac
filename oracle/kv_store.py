"""K/V store oracle (test infrastructure only).

Restates the reference's CPU write path ``BaseAttention::write_kv``
(src/models/attention/base.rs:123-151): every location must lie in
``[0, capacity)`` (else the whole call is an error and nothing is written on
the CPU path), locations equal to the reserved slot are skipped, the rest are
bitwise row copies ``cache[loc[t]] = x[t]``. The device kernel's rule
(third_party/sglang/kvcache.cuh:199-207) is the same per token.
"""
from __future__ import annotations

import numpy as np


class KVStoreError(ValueError):
    pass


def write_kv(k_cache: np.ndarray, v_cache: np.ndarray, k: np.ndarray, v: np.ndarray,
             loc: np.ndarray, reserved: int) -> tuple[np.ndarray, np.ndarray]:
    """Return updated copies of the caches. Caches: [pages, P, H, D] (any dtype)."""
    if k.shape != v.shape or k.ndim != 3:
        raise KVStoreError("K/V input must have matching (tokens, kv_heads, head_dim) shapes")
    if loc.size != k.shape[0]:
        raise KVStoreError("write_loc length must equal the number of K/V tokens")
    capacity = k_cache.shape[0] * k_cache.shape[1]
    kc = k_cache.copy().reshape(capacity, k_cache.shape[2], k_cache.shape[3])
    vc = v_cache.copy().reshape(capacity, v_cache.shape[2], v_cache.shape[3])
    for t, slot in enumerate(np.asarray(loc).tolist()):
        if slot < 0 or slot >= capacity:
            raise KVStoreError("write_loc points outside the bound KV cache")
    for t, slot in enumerate(np.asarray(loc).tolist()):
        if slot == reserved:
            continue
        kc[slot] = k[t]
        vc[slot] = v[t]
    return kc.reshape(k_cache.shape), vc.reshape(v_cache.shape)
