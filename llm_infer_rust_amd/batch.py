"""Scheduler-side batch metadata for the attention path, on the host.

Restates, in numpy, the two places where the reference turns scheduler state into the int32
metadata the attention backend consumes:

* ``BatchContext.prepare_prefill`` -- ``src/engine/batch_context.rs:216-300``: per request the
  uncached prompt slice ``[cached_len, end_len)``, its positions, its cache slots
  ``page * page_size + offset`` (``cache_location``, ``:349-356``), ``cu_seqlens_q``,
  ``prefix_lens``, the row of the last token of each request (``logits_indices``) and a block
  table of ``ceil(max_seq_len / page_size)`` columns padded with -1 (``:266-279``);
* ``DecodeTables.prepare`` -- ``src/scheduler/decode.rs:168-422``: one row per decoding request
  (its last token at position ``len - 1``, ``cache_seqlens = len``, the slot of that position)
  over a block table whose rows persist across steps. A row is rewritten in full when a
  different request lands on it or when its request's pages change other than by appending
  (the request's page version; the reference compares the page lists and rewrites from the
  first difference), only its new pages are written when it grows, and the columns past a
  row's pages hold -1. Every change gives the row a new table version
  (``block_table_versions`` of ``DecodeHostMetadata``).

Both are pure host code: the engine uploads their arrays in one pinned copy per step, and the
attention planners read the host lengths directly, never the device copies.
"""
from __future__ import annotations

import itertools
from dataclasses import dataclass, field
from typing import Sequence

import numpy as np


class BatchError(ValueError):
    """The reference's ``BatchContextError`` / ``SchedulerError::InvalidDecode``."""


def _i32(value: int, what: str) -> int:
    if not 0 <= value < 2 ** 31:
        raise BatchError(f"{what} exceeds i32")
    return value


@dataclass
class BatchRequest:
    """One prefill row (``batch_context.rs`` ``BatchRequest``): the whole prompt, the tokens
    already cached, the exclusive end of this chunk (``None``: the whole prompt) and the
    request's pages."""

    input_ids: Sequence[int]
    cached_len: int = 0
    end_len: int | None = None
    page_ids: Sequence[int] = ()


@dataclass
class PrefillBatch:
    input_ids: np.ndarray       # int64 [tokens]
    positions: np.ndarray       # int64 [tokens]
    write_loc: np.ndarray       # int64 [tokens] cache slots
    cu_seqlens_q: np.ndarray    # int32 [rows + 1]
    prefix_lens: np.ndarray     # int32 [rows]
    logits_indices: np.ndarray  # int64 [rows]: the row of each request's last token
    block_table: np.ndarray     # int32 [rows, max_blocks], -1 past each request's pages
    max_seqlen: int


class BatchContext:
    """Prefill metadata for a fixed ``(max_running_req, max_seq_len, page_size)``."""

    def __init__(self, max_running_req: int, max_seq_len: int, page_size: int):
        if max_running_req <= 0 or max_seq_len <= 0 or page_size <= 0:
            raise BatchError("batch context sizes must be greater than zero")
        self.max_running_req = max_running_req
        self.max_seq_len = max_seq_len
        self.page_size = page_size
        self.max_blocks = -(-max_seq_len // page_size)

    def prepare_prefill(self, requests: Sequence[BatchRequest]) -> PrefillBatch:
        if not requests:
            raise BatchError("prefill batch is empty")
        if len(requests) > self.max_running_req:
            raise BatchError("request count exceeds max_running_req")
        ids, pos, loc = [], [], []
        cu = [0]
        prefixes, last_rows = [], []
        table = np.full((len(requests), self.max_blocks), -1, np.int32)
        for row, req in enumerate(requests):
            total = len(req.input_ids)
            if total > self.max_seq_len:
                raise BatchError("request input exceeds max_seq_len")
            end = total if req.end_len is None else req.end_len
            if not req.cached_len <= end <= total:
                raise BatchError("prefill end_len must be within cached_len..=input length")
            if end == req.cached_len:
                raise BatchError("request has no uncached tokens")
            pages = np.asarray(req.page_ids, np.int64)
            need = -(-end // self.page_size)
            if pages.size < need:
                raise BatchError(
                    "request has no writable KV page for position "
                    f"{max(req.cached_len, pages.size * self.page_size)}")
            p = np.arange(req.cached_len, end, dtype=np.int64)
            slots = pages[p // self.page_size] * self.page_size + p % self.page_size
            if slots.size and int(slots.max()) >= 2 ** 31:
                raise BatchError("KV cache location exceeds i32")
            ids.append(np.asarray(req.input_ids[req.cached_len:end], np.int64))
            pos.append(p)
            loc.append(slots)
            prefixes.append(req.cached_len)
            cu.append(_i32(cu[-1] + (end - req.cached_len), "cumulative sequence length"))
            last_rows.append(cu[-1] - 1)
            cols = min(pages.size, self.max_blocks)
            if cols and int(pages[:cols].max()) >= 2 ** 31:
                raise BatchError("page id exceeds i32")
            table[row, :cols] = pages[:cols]
        return PrefillBatch(np.concatenate(ids), np.concatenate(pos), np.concatenate(loc),
                            np.asarray(cu, np.int32), np.asarray(prefixes, np.int32),
                            np.asarray(last_rows, np.int64), table,
                            max(c1 - c0 for c0, c1 in zip(cu, cu[1:])))


@dataclass
class DecodeRequest:
    """One decoding request: its id, its current length (prompt + fed outputs, the token at
    ``length - 1`` is the one fed this step), that token, its pages, and a page version the
    owner bumps whenever it changes pages it already had (not only appends)."""

    uid: int
    length: int
    input_id: int
    page_ids: Sequence[int]
    page_version: int = 0


@dataclass
class DecodeBatch:
    request_ids: list[int]
    input_ids: np.ndarray       # int64 [rows]
    positions: np.ndarray       # int64 [rows]
    write_loc: np.ndarray       # int64 [rows]
    cache_seqlens: np.ndarray   # int32 [rows]
    block_table: np.ndarray     # int32 [rows, max_blocks] (a view of the persistent rows)
    table_versions: list[int]
    max_seqlen: int


@dataclass
class _Row:
    uid: int | None = None
    pages: int = 0            # page columns currently written
    page_version: int = 0
    table_version: int = 0


_table_versions = itertools.count(1)


@dataclass
class DecodeTables:
    """Persistent decode block-table rows (``DecodeManager``, ``decode.rs:168-422``)."""

    max_running_req: int
    max_seq_len: int
    page_size: int
    mapped_pages: int = 0     # page entries written so far (what the tests count)
    table: np.ndarray = field(init=False)
    rows: list[_Row] = field(init=False)

    def __post_init__(self):
        if self.max_running_req <= 0 or self.max_seq_len <= 0 or self.page_size <= 0:
            raise BatchError("decode table sizes must be greater than zero")
        self.max_blocks = -(-self.max_seq_len // self.page_size)
        self.table = np.full((self.max_running_req, self.max_blocks), -1, np.int32)
        self.rows = [_Row() for _ in range(self.max_running_req)]

    def prepare(self, requests: Sequence[DecodeRequest]) -> DecodeBatch | None:
        n = len(requests)
        if n == 0:
            return None
        if n > self.max_running_req:
            raise BatchError("request count exceeds max_running_req")
        ps, max_len, max_blocks = self.page_size, self.max_seq_len, self.max_blocks
        rows = self.rows
        ids, lens, loc = [0] * n, [0] * n, [0] * n
        for r, req in enumerate(requests):
            length = req.length
            if not 0 < length <= max_len:
                raise BatchError(f"request {req.uid} length {length} is outside "
                                 f"1..={max_len}")
            pages = req.page_ids
            count = len(pages)
            page_index, offset = divmod(length - 1, ps)
            if page_index >= count:
                raise BatchError(f"request {req.uid} has no writable KV page for position "
                                 f"{length - 1}")
            slot = pages[page_index] * ps + offset
            if slot >= 2 ** 31:
                raise BatchError("KV slot exceeds i32")
            ids[r] = req.input_id
            lens[r] = length
            loc[r] = slot
            row = rows[r]
            if (row.uid != req.uid or row.page_version != req.page_version
                    or row.pages != (count if count < max_blocks else max_blocks)):
                self._map_row(r, req)  # new request, changed pages, or a page appended
        lens_a = np.array(lens, np.int32)
        return DecodeBatch([req.uid for req in requests], np.array(ids, np.int64),
                           lens_a.astype(np.int64) - 1, np.array(loc, np.int64), lens_a,
                           self.table[:n], [row.table_version for row in rows[:n]],
                           max(lens))

    def _map_row(self, r: int, req: DecodeRequest) -> None:
        row = self.rows[r]
        pages = req.page_ids
        count = min(len(pages), self.max_blocks)
        if row.uid == req.uid and row.page_version == req.page_version and row.pages == count:
            return  # unchanged (the common decode step: no new page)
        reset = row.uid != req.uid or row.page_version != req.page_version
        start = 0 if reset else row.pages
        if reset:
            self.table[r, :] = -1
        elif count < row.pages:
            self.table[r, count:row.pages] = -1
            start = count
        if count > start:
            values = np.asarray(pages[start:count], np.int64)
            if int(values.max()) >= 2 ** 31:
                raise BatchError("page ID exceeds i32")
            self.table[r, start:count] = values
            self.mapped_pages += count - start
        if reset or count != row.pages:
            row.table_version = next(_table_versions)
        row.uid = req.uid
        row.pages = count
        row.page_version = req.page_version


__all__ = ["BatchError", "BatchRequest", "PrefillBatch", "BatchContext", "DecodeRequest",
           "DecodeBatch", "DecodeTables"]
