"""Page-metadata and work-list oracle (test infrastructure only).

Decode page metadata (bit-exact contract), two routes:
  * host loop      src/models/attention/flashinfer_bridge.cpp:104-118 and the
                   pack kernel src/models/attention/flashinfer_plan_run.cu:24-34
  * masked select  src/models/attention/flashinfer_bridge.cpp:132-138
Prefill paged metadata: flashinfer_bridge.cpp:266-292 (kv length = prefix +
extend; paged iff some prefix > 0).
"""
from __future__ import annotations

import numpy as np


class PlanError(ValueError):
    pass


def decode_page_metadata(block_table: np.ndarray, lengths: np.ndarray, page_size: int):
    """(indptr, indices, last_page_len) by the host-loop route, with its checks."""
    table = np.asarray(block_table, dtype=np.int32)
    batch, columns = table.shape
    indptr = [0]
    total = 0
    for r in range(batch):
        length = int(lengths[r])
        if length <= 0 or length > columns * page_size:
            raise PlanError("host cache length exceeds block table capacity")
        total += (length + page_size - 1) // page_size
        if total > 2**31 - 1:
            raise PlanError("page indptr overflow")
        indptr.append(total)
    indices = []
    last = []
    for r in range(batch):
        pages = indptr[r + 1] - indptr[r]
        indices.extend(int(x) for x in table[r, :pages])
        last.append((int(lengths[r]) - 1) % page_size + 1)
    return (np.asarray(indptr, np.int32), np.asarray(indices, np.int32),
            np.asarray(last, np.int32))


def decode_page_metadata_masked(block_table: np.ndarray, lengths: np.ndarray, page_size: int):
    """Same metadata by the reference's tensor route (floor-divide, cumsum, masked select)."""
    table = np.asarray(block_table, dtype=np.int32)
    lens = np.asarray(lengths, dtype=np.int32)
    pages = (lens + page_size - 1) // page_size
    indptr = np.concatenate([np.zeros(1, np.int32), np.cumsum(pages, dtype=np.int32)])
    columns = np.arange(table.shape[1])
    mask = columns[None, :] < pages[:, None]
    indices = table[mask].astype(np.int32)  # row-major like masked_select
    last = ((lens - 1) % page_size + 1).astype(np.int32)
    return indptr, indices, last


def prefill_page_metadata(block_table: np.ndarray, q_indptr: np.ndarray, prefixes: np.ndarray,
                          page_size: int):
    """(paged, kv_indptr, indices, last_page_len) for a prefill batch."""
    qp = np.asarray(q_indptr, np.int64)
    pp = np.asarray(prefixes, np.int64)
    batch = pp.size
    table = np.asarray(block_table, np.int32)
    paged = False
    for i in range(batch):
        if pp[i] < 0 or qp[i + 1] <= qp[i] or qp[0] != 0:
            raise PlanError("invalid prefill lengths")
        if (pp[i] + qp[i + 1] - qp[i] + page_size - 1) // page_size > table.shape[1]:
            raise PlanError("prefill block table is too small")
        paged |= bool(pp[i] > 0)
    if not paged:
        return False, qp.astype(np.int32), None, None
    lengths = pp + qp[1:] - qp[:-1]
    indptr, indices, last = decode_page_metadata_masked(table, lengths, page_size)
    return True, indptr, indices, last


def check_work_list(work: np.ndarray, merge: np.ndarray, lengths: np.ndarray) -> None:
    """Invariants of a split-KV work list: every token of every request is in exactly
    one item; items of a request are contiguous, ordered and disjoint; partial slots
    are distinct and the merge table points at each split request's slots."""
    work = np.asarray(work, np.int64).reshape(-1, 4)
    merge = np.asarray(merge, np.int64).reshape(-1, 2)
    batch = len(lengths)
    assert merge.shape[0] == batch
    covered = [[] for _ in range(batch)]
    slots = []
    for req, beg, end, slot in work.tolist():
        assert 0 <= req < batch
        assert 0 <= beg < end <= lengths[req]
        covered[req].append((beg, end, slot))
        if slot >= 0:
            slots.append(slot)
    assert len(slots) == len(set(slots))
    for r in range(batch):
        spans = covered[r]
        assert spans, f"request {r} has no work"
        pos = 0
        for beg, end, _ in spans:
            assert beg == pos
            pos = end
        assert pos == lengths[r]
        first, count = merge[r]
        assert count == len(spans)
        if count == 1:
            assert spans[0][2] == -1 and first == -1
        else:
            assert [s for _, _, s in spans] == list(range(first, first + count))
