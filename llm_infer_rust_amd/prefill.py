"""Ragged and paged causal prefill plans on the gfx950 kernels.

Mirrors ``prepare_flashinfer_prefill`` / ``flashinfer_prefill``
(src/models/attention/backend.rs:684-804) and the ATen bridge checks of
``sglang_flashinfer_prepare_prefill`` / ``sglang_flashinfer_prefill``
(src/models/attention/flashinfer_bridge.cpp:250-346): the plan is built once
per forward from the host snapshot of ``cu_seqlens_q`` and ``prefix_lens``;
it is paged iff some prefix > 0; a supplied output tensor is written in place
and returned.
"""
from __future__ import annotations

import ctypes

import torch

from . import _native
from ._native import check, dtype_code, last_error, lib, stream_of
from .kv_cache import ModelError


class PrefillPlan:
    def __init__(self, handle: int):
        self.handle = handle
        self.paged = False
        self.total_q = 0
        self.page_size = 0

    def info(self) -> dict[str, int]:
        buf = (ctypes.c_int64 * 6)()
        check(lib().mi355x_prefill_plan_info(self.handle, buf), "prefill plan info")
        keys = ("batch", "total_q", "paged", "num_items", "total_pages", "split_items")
        return dict(zip(keys, list(buf)))

    def allocations(self) -> int:
        return int(lib().mi355x_prefill_workspace_allocations(self.handle))

    def read_metadata(self, stream: int = 0) -> dict[str, list[int]]:
        info = self.info()
        b, pages = info["batch"], info["total_pages"]
        indptr = (ctypes.c_int32 * (b + 1))()
        indices = (ctypes.c_int32 * max(pages, 1))()
        last = (ctypes.c_int32 * b)()
        check(lib().mi355x_prefill_plan_read(self.handle, indptr, indices, last, stream),
              "prefill plan read")
        md = {"kv_indptr": list(indptr)}
        if info["paged"]:
            md["indices"] = list(indices)[:pages]
            md["last_page_len"] = list(last)
        return md

    def __del__(self):
        if getattr(self, "handle", None):
            try:  # deferred when a graph capture is in progress (see _native.release_handle)
                _native.release_handle("mi355x_prefill_plan_drop", self.handle)
            except Exception:  # interpreter shutdown
                pass
            self.handle = None


def prepare_prefill_plan(existing: PrefillPlan | None, metadata, prefill, spec,
                         page_size: int) -> PrefillPlan:
    _native.release_deferred()  # plans parked during a capture (outside one now)
    cu = metadata.cu_seqlens_q
    prefixes = metadata.prefix_lens
    table = metadata.block_table
    if cu is None:
        raise ModelError("missing cu_seqlens_q")
    if prefixes is None:
        raise ModelError("missing prefix_lens")
    if table is None:
        raise ModelError("missing block_table")
    if (not cu.is_cuda or cu.dtype != torch.int32 or cu.dim() != 1 or not cu.is_contiguous()
            or not prefixes.is_cuda or prefixes.dtype != torch.int32 or prefixes.dim() != 1
            or prefixes.size(0) + 1 != cu.size(0) or prefixes.device != cu.device
            or table.device != cu.device or table.dim() != 2 or table.dtype != torch.int32
            or table.size(0) != prefixes.size(0) or table.stride(1) != 1):
        raise ModelError("invalid mi355x prefill metadata")
    dt = {torch.bfloat16: 0, torch.float16: 1}.get(spec.dtype)
    if dt is None:
        raise ModelError("mi355x attention requires bfloat16 or float16")
    b = len(prefill.prefixes)
    qh = (ctypes.c_int32 * (b + 1))(*prefill.boundaries)
    ph = (ctypes.c_int32 * b)(*prefill.prefixes)
    handle = lib().mi355x_prefill_prepare(
        existing.handle if existing else None, cu.data_ptr(), table.data_ptr(), b,
        table.size(1), table.stride(0), qh, ph, spec.num_heads, spec.num_kv_heads, page_size, dt,
        stream_of(cu))
    if not handle:
        raise ModelError(f"mi355x prefill plan failed: {last_error()}")
    plan = existing if existing is not None else PrefillPlan(handle)
    if handle != plan.handle:
        raise ModelError("prefill plan address changed")
    plan.paged = prefill.has_prefix()
    plan.total_q = prefill.boundaries[-1]
    plan.page_size = int(page_size)
    return plan


def run_prefill(plan: PrefillPlan, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                out: torch.Tensor | None = None) -> torch.Tensor:
    """q [N, Hq, 128]; ragged k/v [N, Hkv, 128] views or paged caches [pages, P, Hkv, 128]."""
    for t in (q, k, v):
        if not t.is_cuda or t.dtype != q.dtype or t.stride(-1) != 1 or t.size(-1) != 128 \
                or t.stride(-2) != 128:
            raise ModelError("invalid mi355x prefill tensors")
    if q.dim() != 3 or q.size(0) != plan.total_q or k.shape != v.shape:
        raise ModelError("mi355x prefill shape mismatch")
    if plan.paged:
        if k.dim() != 4 or not k.is_contiguous() or not v.is_contiguous():
            raise ModelError("mi355x prefill shape mismatch")
        hkv = k.size(2)
        if k.size(1) != plan.page_size:
            raise ModelError("mi355x prefill shape mismatch")
        k_sn = v_sn = hkv * 128
    else:
        if k.dim() != 3 or k.size(0) != q.size(0):
            raise ModelError("mi355x prefill shape mismatch")
        hkv = k.size(1)
        k_sn, v_sn = k.stride(0), v.stride(0)
    if out is None:
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    elif out.shape != q.shape or out.dtype != q.dtype or not out.is_contiguous():
        raise ModelError("invalid static prefill output")
    check(lib().mi355x_prefill_run(
        plan.handle, q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), k_sn, 128,
        v.data_ptr(), v_sn, 128, out.data_ptr(), out.stride(0), out.stride(1), q.size(0),
        q.size(1), hkv, plan.page_size, dtype_code(q), stream_of(q)), "mi355x prefill")
    return out

