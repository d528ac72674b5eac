"""Attention-backend seam with the gfx950 backend (``--attention-backend mi355x``).

Host mirror of the reference's ``src/models/attention/backend.rs``:

* ``AttentionBackendKind.parse`` (``backend.rs:31-41``) gains the ``mi355x``
  (alias ``hip``) value;
* ``Attention.new / validate / bind_cache_layout / prepare /
  prepare_decode_graph`` (``backend.rs:104-183``): ``prepare`` runs once per
  forward and the returned ``AttentionBatch`` is reused by every layer;
* ``AttentionBatch.forward / forward_into`` (``backend.rs:185-247``);
* ``PrefillMetadata`` host snapshot and ``cu_seqlens_q`` validation
  (``backend.rs:70-97,1500-1532``);
* plan reuse rules of the FlashInfer backend (``backend.rs:386-438``): a new
  batch may not be prepared while the previous one is still referenced.

Only the ``mi355x`` kind is implemented by this package; the reference's own
``pt``/``fa``/``flashinfer`` kinds parse but are rejected by ``validate``.
"""
from __future__ import annotations

import ctypes
import enum
import math
import weakref
from dataclasses import dataclass, field
from typing import Sequence

import numpy as np
import torch

from . import _native
from ._native import NativeError, check, dtype_code, last_error, lib, stream_of
from .kv_cache import BaseAttention, ModelError


class BatchPhase(enum.Enum):
    PREFILL = "prefill"
    DECODE = "decode"


class AttentionBackendKind(enum.Enum):
    PT = "pt"
    FLASH_ATTENTION = "fa"
    FLASHINFER = "flashinfer"
    MI355X = "mi355x"

    @staticmethod
    def parse(name: str) -> "AttentionBackendKind":
        key = name.lower()
        if key in ("pt", "pytorch"):
            return AttentionBackendKind.PT
        if key in ("fa", "flashattention", "flash-attention"):
            return AttentionBackendKind.FLASH_ATTENTION
        if key == "flashinfer":
            return AttentionBackendKind.FLASHINFER
        if key in ("mi355x", "hip"):
            return AttentionBackendKind.MI355X
        raise ModelError(
            f"unknown attention backend {name!r}; expected \"pt\", \"fa\", \"flashinfer\", "
            "or \"mi355x\"")


@dataclass(frozen=True)
class AttentionSpec:
    num_heads: int
    num_kv_heads: int
    head_dim: int
    dtype: torch.dtype
    device: torch.device


@dataclass
class DecodeHostMetadata:
    cache_seqlens: Sequence[int]    # a list, or an int32 array passed without a copy
    block_table_versions: list[int] | None = None


@dataclass
class AttentionMetadata:
    """Per-invocation metadata (``src/engine/model_runner.rs:47-59``). int32 tensors."""
    forward_mode: BatchPhase
    decode_host: DecodeHostMetadata | None = None
    write_loc: torch.Tensor | None = None
    cu_seqlens_q: torch.Tensor | None = None
    prefix_lens: torch.Tensor | None = None
    block_table: torch.Tensor | None = None
    req_to_token: torch.Tensor | None = None
    cache_seqlens: torch.Tensor | None = None
    max_seqlen: int | None = None
    # Scheduler-side host copies of cu_seqlens_q / prefix_lens. When present the backend
    # plans from them instead of reading the device tensors back (no sync per forward).
    host_cu_seqlens_q: list[int] | None = None
    host_prefix_lens: list[int] | None = None


@dataclass
class MetadataRequirements:
    block_table: bool
    req_to_token: bool


@dataclass
class PrefillMetadata:
    """Host snapshot read once per invocation, never in a layer forward."""
    boundaries: list[int] = field(default_factory=list)
    prefixes: list[int] = field(default_factory=list)

    @staticmethod
    def prepare(metadata: AttentionMetadata | None, total_tokens: int) -> "PrefillMetadata":
        boundaries = batch_boundaries(metadata, total_tokens)
        if metadata is not None and metadata.forward_mode == BatchPhase.PREFILL:
            if metadata.host_prefix_lens is not None:
                prefixes = [int(x) for x in metadata.host_prefix_lens]
            elif metadata.prefix_lens is None:
                raise ModelError("missing prefix_lens")
            else:
                prefixes = [int(x) for x in metadata.prefix_lens.cpu().tolist()]
        else:
            prefixes = [0] * (len(boundaries) - 1)
        if len(prefixes) + 1 != len(boundaries) or any(p < 0 for p in prefixes):
            raise ModelError("invalid prefill prefix lengths")
        return PrefillMetadata(boundaries, prefixes)

    def has_prefix(self) -> bool:
        return any(p > 0 for p in self.prefixes)


def batch_boundaries(metadata: AttentionMetadata | None, total_tokens: int) -> list[int]:
    if metadata is None or metadata.forward_mode == BatchPhase.DECODE \
            or (metadata.cu_seqlens_q is None and metadata.host_cu_seqlens_q is None):
        return [0, total_tokens]
    return prefill_boundaries(metadata, total_tokens)


def prefill_boundaries(metadata: AttentionMetadata, total_tokens: int) -> list[int]:
    if metadata.host_cu_seqlens_q is not None:
        b = [int(x) for x in metadata.host_cu_seqlens_q]
    elif metadata.cu_seqlens_q is None:
        raise ModelError("cached prefill requires cu_seqlens_q")
    else:
        b = [int(x) for x in metadata.cu_seqlens_q.cpu().tolist()]
    if (len(b) < 2 or b[0] != 0 or b[-1] != total_tokens
            or any(b[i] >= b[i + 1] for i in range(len(b) - 1))):
        raise ModelError("invalid prefill cu_seqlens_q")
    return b


# ---------------------------------------------------------------------------
# Native plans
# ---------------------------------------------------------------------------
class DecodePlan:
    """Owns one native decode plan handle (``mi355x_decode_prepare``)."""

    def __init__(self, handle: int, graph: bool):
        self.handle = handle
        self.graph = graph

    def info(self) -> dict[str, int]:
        buf = (ctypes.c_int64 * 6)()
        check(lib().mi355x_decode_plan_info(self.handle, buf), "decode plan info")
        keys = ("batch", "total_pages", "num_items", "chunk_tokens", "items_capacity", "cus")
        return dict(zip(keys, list(buf)))

    def allocations(self) -> int:
        return int(lib().mi355x_decode_workspace_allocations(self.handle))

    def read_metadata(self, stream: int = 0) -> dict[str, list[int]]:
        info = self.info()
        b, pages, items = info["batch"], info["total_pages"], info["num_items"]
        indptr = (ctypes.c_int32 * (b + 1))()
        indices = (ctypes.c_int32 * max(pages, 1))()
        last = (ctypes.c_int32 * b)()
        work = (ctypes.c_int32 * max(4 * items, 1))()
        merge = (ctypes.c_int32 * (2 * b))()
        check(lib().mi355x_decode_plan_read(self.handle, indptr, indices, last, work, merge,
                                            stream), "decode plan read")
        return {"indptr": list(indptr), "indices": list(indices)[:pages],
                "last_page_len": list(last), "work": list(work)[:4 * items],
                "merge": list(merge)}

    def __del__(self):
        if getattr(self, "handle", None):
            try:  # deferred when a graph capture is in progress (see _native.release_handle)
                _native.release_handle("mi355x_decode_plan_drop", self.handle)
            except Exception:  # interpreter shutdown
                pass
            self.handle = None


def prepare_decode_plan(existing: DecodePlan | None, metadata: AttentionMetadata,
                        spec: AttentionSpec, page_size: int, graph: bool) -> DecodePlan:
    """``prepare_flashinfer_decode`` (backend.rs:574-640) on the native planner."""
    _native.release_deferred()  # plans parked during a capture (outside one now)
    table = metadata.block_table
    lengths = metadata.cache_seqlens
    if table is None:
        raise ModelError("decode requires block_table")
    if lengths is None:
        raise ModelError("decode requires cache_seqlens")
    if not table.is_cuda or not lengths.is_cuda:
        raise ModelError("decode metadata must be GPU tensors")
    if (table.dim() != 2 or lengths.dim() != 1 or table.size(0) != lengths.size(0)
            or table.dtype != torch.int32 or lengths.dtype != torch.int32
            or table.stride(1) != 1 or not lengths.is_contiguous()):
        raise ModelError("invalid decode block table or lengths")
    dt = {torch.bfloat16: 0, torch.float16: 1}.get(spec.dtype)
    if dt is None:
        raise ModelError("mi355x attention requires bfloat16 or float16")
    host = None
    rows = 0
    if metadata.decode_host is not None:
        values = np.ascontiguousarray(metadata.decode_host.cache_seqlens, np.int32)
        rows = values.size
        if rows == 0:
            raise ModelError("invalid host decode metadata")
        host = values.ctypes.data  # ``values`` outlives the call
    handle = lib().mi355x_decode_prepare(
        existing.handle if existing else None, table.data_ptr(), table.size(0), table.size(1),
        table.stride(0), lengths.data_ptr(), spec.num_heads, spec.num_kv_heads, spec.head_dim,
        page_size, dt, graph, host, rows, stream_of(table))
    if not handle:
        raise ModelError(f"mi355x decode plan failed: {last_error()}")
    if existing is not None:
        if handle != existing.handle:
            raise ModelError("decode plan address changed")
        return existing
    return DecodePlan(handle, graph)


def run_decode(plan: DecodePlan, q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
               out: torch.Tensor | None = None) -> torch.Tensor:
    """Paged decode on a prepared plan. q: [B, Hq, 128] (any 16-byte aligned strides)."""
    if not (q.is_cuda and k_cache.is_cuda and v_cache.is_cuda):
        raise ModelError("mi355x decode requires GPU tensors")
    if q.dim() != 3 or q.stride(2) != 1 or not k_cache.is_contiguous() \
            or not v_cache.is_contiguous() or k_cache.dim() != 4:
        raise ModelError("mi355x decode requires [B,Hq,D] queries and contiguous caches")
    if out is None:
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    elif out.shape != q.shape or out.dtype != q.dtype or out.stride(2) != 1:
        raise ModelError("invalid decode output")
    check(lib().mi355x_decode_run(
        plan.handle, q.data_ptr(), q.stride(0), q.stride(1), k_cache.data_ptr(),
        v_cache.data_ptr(), out.data_ptr(), out.stride(0), out.stride(1), q.size(0), q.size(1),
        k_cache.size(2), k_cache.size(1), dtype_code(q), stream_of(q)), "mi355x decode")
    return out


# ---------------------------------------------------------------------------
# Backend seam
# ---------------------------------------------------------------------------
class _BackendPlan:
    """Which native plan a batch holds: ("decode", DecodePlan) | ("prefill", PrefillPlan)."""

    def __init__(self, kind: str, plan: object):
        self.kind = kind
        self.plan = plan


class MI355XAttentionBackend:
    """gfx950 paged decode / ragged + paged prefill (the ``mi355x`` kind)."""

    def __init__(self) -> None:
        self._decode_plan: DecodePlan | None = None
        self._prefill_plan = None
        self._decode_owner: weakref.ref | None = None
        self._prefill_owner: weakref.ref | None = None
        self._graph_plans: dict[int, weakref.ref] = {}

    def metadata_requirements(self, _phase: BatchPhase) -> MetadataRequirements:
        return MetadataRequirements(block_table=True, req_to_token=False)

    def supports_cuda_graph(self) -> bool:
        return True

    def prepare_decode_graph(self, metadata: AttentionMetadata, spec: AttentionSpec,
                             page_size: int) -> "DecodeGraphState":
        table = metadata.block_table
        if table is None:
            raise ModelError("missing graph block_table")
        if metadata.cache_seqlens is None:
            raise ModelError("missing graph cache_seqlens")
        plan = prepare_decode_plan(None, metadata, spec, page_size, graph=True)
        self._graph_plans = {k: v for k, v in self._graph_plans.items() if v() is not None}
        key = table.data_ptr()
        if key in self._graph_plans:
            raise ModelError("decode graph buffers are already registered")
        state = DecodeGraphState(plan, table, metadata.cache_seqlens, spec, page_size)
        self._graph_plans[key] = weakref.ref(plan)
        return state

    def prepare(self, batch: "AttentionBatch", metadata: AttentionMetadata | None,
                prefill: PrefillMetadata, spec: AttentionSpec,
                page_size: int | None) -> _BackendPlan | None:
        if metadata is not None and metadata.forward_mode == BatchPhase.DECODE:
            if metadata.block_table is not None:
                ref = self._graph_plans.get(metadata.block_table.data_ptr())
                plan = ref() if ref else None
                if plan is not None:  # planned outside capture/replay
                    return _BackendPlan("decode", plan)
            if page_size is None:
                raise ModelError("mi355x attention requires a bound KV cache")
            if self._decode_owner is not None and self._decode_owner() is not None:
                raise ModelError("previous mi355x batch is still in use")
            self._decode_plan = prepare_decode_plan(self._decode_plan, metadata, spec, page_size,
                                                    graph=False)
            self._decode_owner = weakref.ref(batch)
            return _BackendPlan("decode", self._decode_plan)
        if metadata is not None:
            if page_size is None:
                raise ModelError("mi355x attention requires a bound KV cache")
            if self._prefill_owner is not None and self._prefill_owner() is not None:
                raise ModelError("previous mi355x prefill batch is still in use")
            from .prefill import prepare_prefill_plan
            self._prefill_plan = prepare_prefill_plan(self._prefill_plan, metadata, prefill,
                                                      spec, page_size)
            self._prefill_owner = weakref.ref(batch)
            return _BackendPlan("prefill", self._prefill_plan)
        raise ModelError("mi355x attention requires attention metadata")

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cache: BaseAttention,
                plan: _BackendPlan, head_dim: int,
                output: torch.Tensor | None = None) -> torch.Tensor:
        if plan.kind == "decode":
            kc, vc = cache.cache_tensors()
            out = None if output is None else output.view(q.shape)
            res = run_decode(plan.plan, q, kc, vc, out)
            return res.reshape(q.size(0), q.size(1) * head_dim)
        from .prefill import run_prefill
        out = None if output is None else output.view(q.shape)
        if plan.plan.paged:
            kc, vc = cache.cache_tensors()
            res = run_prefill(plan.plan, q, kc, vc, out)
        else:
            res = run_prefill(plan.plan, q, k, v, out)
        return res.reshape(q.size(0), q.size(1) * head_dim)


class DecodeGraphState:
    """Re-plans outside the graph at a fixed plan address (``backend.rs:490-530``)."""

    def __init__(self, plan: DecodePlan, table: torch.Tensor, lengths: torch.Tensor,
                 spec: AttentionSpec, page_size: int):
        self.plan = plan
        self.table = table
        self.lengths = lengths
        self.spec = spec
        self.page_size = page_size

    def prepare_replay(self, host: DecodeHostMetadata | None) -> None:
        if host is not None and len(host.cache_seqlens) < self.table.size(0):
            seqlens = np.ones(self.table.size(0), np.int32)  # pad rows read page 0
            seqlens[:len(host.cache_seqlens)] = host.cache_seqlens
            host = DecodeHostMetadata(seqlens)
        meta = AttentionMetadata(forward_mode=BatchPhase.DECODE, decode_host=host,
                                 block_table=self.table, cache_seqlens=self.lengths)
        prepare_decode_plan(self.plan, meta, self.spec, self.page_size, graph=True)

    def needs_req_to_token(self) -> bool:
        return False


class Attention:
    """One selected implementation for all layers of a model."""

    def __init__(self, backend: MI355XAttentionBackend, spec: AttentionSpec):
        self.backend = backend
        self.spec = spec
        self.page_size: int | None = None

    @staticmethod
    def new(name: str, spec: AttentionSpec) -> "Attention":
        Attention.validate(name, spec)
        return Attention(MI355XAttentionBackend(), spec)

    @staticmethod
    def validate(name: str, spec: AttentionSpec) -> None:
        kind = AttentionBackendKind.parse(name)
        if kind != AttentionBackendKind.MI355X:
            raise ModelError(f"attention backend {name!r} is not provided by this library")
        if torch.device(spec.device).type != "cuda" or spec.dtype not in (torch.bfloat16,
                                                                           torch.float16):
            raise ModelError("mi355x attention requires a GPU and bfloat16 or float16")
        if spec.head_dim != 128:
            raise ModelError("mi355x attention currently requires head_dim=128")
        group = spec.num_heads // max(spec.num_kv_heads, 1)
        if spec.num_kv_heads <= 0 or spec.num_heads % spec.num_kv_heads or group not in (1, 2,
                                                                                         4, 8):
            raise ModelError("mi355x attention supports 1, 2, 4 or 8 query heads per kv head")
        lib()  # fail loudly now if the HIP library is missing

    def bind_cache_layout(self, page_size: int) -> None:
        self.page_size = int(page_size)

    def supports_cuda_graph(self) -> bool:
        return self.backend.supports_cuda_graph()

    def metadata_requirements(self, phase: BatchPhase) -> MetadataRequirements:
        return self.backend.metadata_requirements(phase)

    def prepare_decode_graph(self, metadata: AttentionMetadata) -> DecodeGraphState:
        if self.page_size is None:
            raise ModelError("graph requires a bound KV cache")
        return self.backend.prepare_decode_graph(metadata, self.spec, self.page_size)

    def prepare(self, metadata: AttentionMetadata | None, total_tokens: int) -> "AttentionBatch":
        prefill = PrefillMetadata.prepare(metadata, total_tokens)
        batch = AttentionBatch(self.backend, self.spec, metadata, prefill)
        batch.plan = self.backend.prepare(batch, metadata, prefill, self.spec, self.page_size)
        return batch


class AttentionBatch:
    """Prepared once per model forward and reused by every decoder layer."""

    def __init__(self, backend: MI355XAttentionBackend, spec: AttentionSpec,
                 metadata: AttentionMetadata | None, prefill: PrefillMetadata):
        self.backend = backend
        self.spec = spec
        self.metadata = metadata
        self.prefill = prefill
        self.plan: _BackendPlan | None = None

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                cache: BaseAttention) -> torch.Tensor:
        return self.backend.forward(q, k, v, cache, self.plan, self.spec.head_dim)

    def forward_into(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                     cache: BaseAttention, output: torch.Tensor) -> None:
        """Write into a caller-owned static output, preserving its address."""
        if (q.dim() != 3 or tuple(output.shape) != (q.size(0),
                                                    self.spec.num_heads * self.spec.head_dim)
                or output.dtype != self.spec.dtype or output.device != q.device
                or not output.is_contiguous()):
            raise ModelError("invalid static attention output")
        self.backend.forward(q, k, v, cache, self.plan, self.spec.head_dim, output)


def sm_scale(head_dim: int) -> float:
    return 1.0 / math.sqrt(head_dim)


__all__ = [
    "Attention", "AttentionBatch", "AttentionBackendKind", "AttentionMetadata", "AttentionSpec",
    "BatchPhase", "DecodeGraphState", "DecodeHostMetadata", "DecodePlan", "MetadataRequirements",
    "ModelError", "NativeError", "PrefillMetadata", "prepare_decode_plan", "run_decode",
]
