"""Paged KV-cache layout and per-layer K/V binding with the gfx950 K/V store.

Mirrors:
* ``KVCachePool`` buffer layout ``[2, layers, pages + 1, page_size, kv_heads,
  head_dim]`` with physical page 0 reserved and zeroed
  (``src/engine/kvcache/pool.rs:81-104,150-179``);
* ``BaseAttention`` (``src/models/attention/base.rs:10-152``): layer-local
  ``(pages, page_size, kv_heads, head_dim)`` K/V views, the reserved write
  slot, and ``write_kv`` with its shape checks and error messages.

Device writes go through ``mi355x_store_kv``. Out-of-range slots are never
written; they are counted in a per-binding device word and reported by
``check_write_errors()`` (the reference aborts with a device assert instead,
``third_party/sglang/kvcache.cuh:199-201``).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from ._native import NativeError, check, lib, stream_of


class ModelError(RuntimeError):
    """The reference's ``ModelRunnerError::Model``."""


@dataclass(frozen=True)
class KVCacheLayout:
    num_layers: int
    num_pages: int
    page_size: int
    num_kv_heads: int
    head_dim: int

    def tensor_shape(self) -> tuple[int, ...]:
        if 0 in (self.num_layers, self.num_pages, self.page_size, self.num_kv_heads,
                 self.head_dim):
            raise ModelError("all KV-cache dimensions must be greater than zero")
        return (2, self.num_layers, self.num_pages + 1, self.page_size, self.num_kv_heads,
                self.head_dim)


class KVCachePool:
    """One contiguous K/V buffer for every layer; page 0 is reserved and zeroed."""

    def __init__(self, layout: KVCacheLayout, dtype: torch.dtype, device: torch.device | str):
        self.layout = layout
        self.buffer = torch.empty(layout.tensor_shape(), dtype=dtype, device=device)
        self.buffer[:, :, 0].zero_()

    def layer(self, index: int) -> tuple[torch.Tensor, torch.Tensor]:
        return self.buffer[0, index], self.buffer[1, index]


class BaseAttention:
    """Owns one attention layer's stable K/V views into its cache group."""

    def __init__(self) -> None:
        self.k_cache: torch.Tensor | None = None
        self.v_cache: torch.Tensor | None = None
        self._reserved_write_slot = -1
        self._errors: torch.Tensor | None = None

    def reserved_write_slot(self) -> int:
        return self._reserved_write_slot

    def set_reserved_write_slot(self, slot: int) -> None:
        self._reserved_write_slot = int(slot)

    def bind_kv_cache(self, k_cache: torch.Tensor, v_cache: torch.Tensor) -> None:
        if k_cache.shape != v_cache.shape or k_cache.dim() != 4:
            raise ModelError(
                "K/V cache must have matching (pages, page_size, kv_heads, head_dim) shapes")
        self.k_cache = k_cache
        self.v_cache = v_cache
        self._errors = torch.zeros(1, dtype=torch.int32, device=k_cache.device)

    def is_bound(self) -> bool:
        return self.k_cache is not None

    def cache_tensors(self) -> tuple[torch.Tensor, torch.Tensor]:
        if self.k_cache is None or self.v_cache is None:
            raise ModelError("paged-KV attention requires a bound KV cache")
        return self.k_cache, self.v_cache

    def write_kv(self, k: torch.Tensor, v: torch.Tensor, write_loc: torch.Tensor | None,
                 _phase: object = None) -> None:
        """Writes ``(tokens, kv_heads, head_dim)`` K/V rows to flattened page slots."""
        if self.k_cache is None or self.v_cache is None or write_loc is None:
            return
        if k.shape != v.shape or k.dim() != 3:
            raise ModelError("K/V input must have matching (tokens, kv_heads, head_dim) shapes")
        if write_loc.numel() != k.size(0):
            raise ModelError("write_loc length must equal the number of K/V tokens")
        kc, vc = self.k_cache, self.v_cache
        if kc.size(2) != k.size(1) or kc.size(3) != k.size(2):
            raise ModelError("K/V input head shape does not match the bound cache")
        # Checks of the reference ATen bridge (kv_store_bridge.cpp:16-32).
        if not k.is_cuda:
            raise NativeError("KV store requires GPU tensors")
        for t in (v, kc, vc):
            if not t.is_cuda or t.device != k.device or t.dtype != k.dtype:
                raise NativeError("KV store device/dtype mismatch")
        if (k.dtype not in (torch.bfloat16, torch.float16) or k.stride(2) != 1
                or v.stride(2) != 1 or not kc.is_contiguous() or not vc.is_contiguous()
                or k.size(1) <= 0 or k.size(2) <= 0):
            raise NativeError("invalid KV store shape/stride")
        if (not write_loc.is_cuda or write_loc.device != k.device or write_loc.dim() != 1
                or not write_loc.is_contiguous()
                or write_loc.dtype not in (torch.int32, torch.int64)):
            raise NativeError("invalid KV store locations")
        check(lib().mi355x_store_kv(
            k.data_ptr(), v.data_ptr(), kc.data_ptr(), vc.data_ptr(), write_loc.data_ptr(),
            k.size(0), k.size(1), k.size(2), kc.size(0) * kc.size(1), k.stride(0), k.stride(1),
            v.stride(0), v.stride(1), self._reserved_write_slot,
            write_loc.dtype == torch.int64, self._errors.data_ptr(), stream_of(k)), "KV store")

    def error_word(self) -> torch.Tensor | None:
        """Device int32 counter of rejected (out-of-range) slots."""
        return self._errors

    def check_write_errors(self) -> None:
        """Raise if any earlier write_kv saw a slot outside the cache (synchronises)."""
        if self._errors is None:
            return
        count = int(self._errors.item())
        if count:
            self._errors.zero_()
            raise ModelError("write_loc points outside the bound KV cache")
