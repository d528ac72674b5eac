"""Scheduler-side batch metadata (``llm_infer_rust_amd.batch``) against the reference's own
fixtures for ``BatchContext::prepare_prefill`` (``src/engine/batch_context.rs`` tests) and
``DecodeManager`` (``src/scheduler/decode.rs`` tests), with the block table in place of the
reference's ``req_to_token`` where a test checks only that layout. Pure host code: CPU only."""
import numpy as np
import pytest

from llm_infer_rust_amd.batch import (BatchContext, BatchError, BatchRequest, DecodeRequest,
                                      DecodeTables)


def test_prepares_prefill_tensors_and_page_tables():
    # batch_context.rs:486-525 prepares_prefill_tensors_and_page_tables
    ctx = BatchContext(2, 8, 2)
    b = ctx.prepare_prefill([BatchRequest([10, 11, 12], 2, None, [5, 3]),
                             BatchRequest([20, 21], 0, None, [7])])
    assert b.input_ids.tolist() == [12, 20, 21]
    assert b.positions.tolist() == [2, 0, 1]
    assert b.write_loc.tolist() == [6, 14, 15]
    assert b.logits_indices.tolist() == [0, 2]
    assert b.cu_seqlens_q.tolist() == [0, 1, 3] and b.cu_seqlens_q.dtype == np.int32
    assert b.prefix_lens.tolist() == [2, 0] and b.prefix_lens.dtype == np.int32
    assert b.block_table.tolist() == [[5, 3, -1, -1], [7, -1, -1, -1]]
    assert b.block_table.dtype == np.int32 and b.max_seqlen == 2


def test_mixed_rows_layout():
    # batch_context.rs:528-575: a prefill row and a one-token row at position 2 share one
    # prefill batch (the decode row is a request with two cached tokens).
    ctx = BatchContext(4, 8, 2)
    b = ctx.prepare_prefill([BatchRequest([1, 2], 0, None, [0]),
                             BatchRequest([7, 7, 0], 2, None, [1, 2])])
    assert b.cu_seqlens_q.tolist() == [0, 2, 3]
    assert b.prefix_lens.tolist() == [0, 2]
    assert b.write_loc.tolist() == [0, 1, 4]
    assert b.logits_indices.tolist() == [1, 2]
    assert b.block_table.tolist() == [[0, -1, -1, -1], [1, 2, -1, -1]]


@pytest.mark.parametrize("cached,end", [(3, 2), (1, 4), (2, 2)])
def test_chunk_bounds_are_validated(cached, end):
    # batch_context.rs plain_and_mixed_prefill_share_chunk_validation
    with pytest.raises(BatchError):
        BatchContext(2, 8, 2).prepare_prefill([BatchRequest([10, 11, 12], cached, end, [1, 2])])


def test_prefill_rejections():
    # batch_context.rs rejects_oversized_mixed_prefill / rejects_requests_without_uncached_tokens
    # / rejects_prefill_without_a_writable_page (position 2 in both cases)
    with pytest.raises(BatchError, match="exceeds max_seq_len"):
        BatchContext(1, 2, 2).prepare_prefill([BatchRequest([1, 2, 3], 0, None, [0, 1])])
    with pytest.raises(BatchError, match="no uncached tokens"):
        BatchContext(1, 4, 2).prepare_prefill([BatchRequest([1], 1, None, [])])
    for cached in (0, 2):
        with pytest.raises(BatchError, match="position 2$"):
            BatchContext(1, 4, 2).prepare_prefill([BatchRequest([1, 2, 3], cached, None, [0])])
    with pytest.raises(BatchError, match="max_running_req"):
        BatchContext(1, 4, 2).prepare_prefill([BatchRequest([1], 0, None, [1])] * 2)


def _tables():
    return DecodeTables(max_running_req=2, max_seq_len=6, page_size=2)  # decode.rs manager()


def _running(uid, input_ids, pages, version=0):
    return DecodeRequest(uid, len(input_ids), input_ids[-1], pages, version)


def test_builds_decode_tensors_and_page_metadata():
    # decode.rs:483-522
    b = _tables().prepare([_running(4, [11, 12, 13], [5, 6]), _running(7, [21, 22], [9])])
    assert b.request_ids == [4, 7]
    assert b.input_ids.tolist() == [13, 22]
    assert b.positions.tolist() == [2, 1]
    assert b.write_loc.tolist() == [12, 19]
    assert b.cache_seqlens.tolist() == [3, 2] and b.cache_seqlens.dtype == np.int32
    assert b.max_seqlen == 3
    assert b.block_table.reshape(-1).tolist() == [5, 6, -1, 9, -1, -1]
    assert b.block_table.dtype == np.int32


def test_empty_batch_is_none():
    # decode.rs empty_and_finished_requests_produce_no_batch (finished requests are filtered
    # by the engine before the tables see them)
    assert _tables().prepare([]) is None


def test_reused_rows_clear_stale_page_entries():
    # decode.rs:669-691
    t = _tables()
    t.prepare([_running(1, [1, 2, 3, 4], [5, 6])])
    b = t.prepare([_running(2, [9], [1])])
    assert b.block_table.reshape(-1).tolist() == [1, -1, -1]


def test_out_of_range_sequence_is_rejected():
    # decode.rs:693-700
    with pytest.raises(BatchError, match="outside 1..=6"):
        _tables().prepare([_running(1, [1, 2, 3, 4, 5, 6, 7], [0, 1, 2, 3])])
    with pytest.raises(BatchError, match="no writable KV page for position 2"):
        _tables().prepare([_running(1, [1, 2, 3], [4])])


def test_growth_maps_only_new_pages_and_page_changes_rebuild():
    # decode.rs:702-754 growing_decode_only_maps_new_tokens_and_handles_page_changes, and the
    # version rule of exercise_table_requirements (:537-621)
    t = _tables()
    pages = [5, 6, 7]
    t.prepare([_running(1, [1, 2], pages)])
    assert t.mapped_pages == 3
    v0 = t.rows[0].table_version
    b = t.prepare([_running(1, [1, 2, 3], pages)])       # grows inside its pages
    assert t.mapped_pages == 3 and b.table_versions == [v0]
    b = t.prepare([_running(1, [1, 2, 3, 4], pages)])
    assert t.mapped_pages == 3 and b.table_versions == [v0]
    pages = [9, 6, 7]                                     # a page changes: full rewrite
    b = t.prepare([_running(1, [1, 2, 3, 4], pages, version=1)])
    assert t.mapped_pages == 6 and b.table_versions[0] != v0
    assert b.block_table[0].tolist() == [9, 6, 7]
    assert b.write_loc.tolist() == [13]
    b = t.prepare([_running(1, [1], [9], version=1)])   # shrinks: the tail is cleared
    assert b.block_table[0].tolist() == [9, -1, -1]
    v1 = b.table_versions[0]
    b = t.prepare([_running(1, [1, 2, 3], [9, 4], version=1)])   # appends a page
    assert b.block_table[0].tolist() == [9, 4, -1] and b.table_versions[0] != v1
    assert t.mapped_pages == 7


def test_compacting_rows_keeps_each_request_mapping():
    # decode.rs:756-780 compacting_rows_and_reusing_pages_preserves_request_mappings
    t = _tables()
    a, b = _running(1, [1, 2], [5]), _running(2, [3, 4], [6])
    t.prepare([a, b])
    b = _running(2, [3, 4, 5], [6, 7])
    out = t.prepare([b])
    assert out.block_table[0].tolist() == [6, 7, -1]
    c = _running(3, [9], [6])
    out = t.prepare([c, b])
    assert out.block_table.tolist() == [[6, -1, -1], [6, 7, -1]]
    assert out.write_loc.tolist() == [12, 14]


def test_request_count_is_bounded():
    with pytest.raises(BatchError, match="max_running_req"):
        _tables().prepare([_running(i, [1], [i + 1]) for i in range(3)])


def test_staged_decode_step_matches_only_its_rows_and_lengths():
    """A decode step staged one step early (``engine._Ahead``) is used only for the same graph,
    the same rows in the same order, each at the length it was staged for."""
    from types import SimpleNamespace

    import numpy as np

    from llm_infer_rust_amd.engine import _Ahead

    def row(uid, cursor, outputs):
        return SimpleNamespace(uid=uid, cursor=cursor, output=[7] * outputs)

    graph, other = object(), object()
    staged = _Ahead([3, 5], [12, 21], graph, np.zeros(4, np.int64), np.zeros(2, np.int32))
    rows = [row(3, 10, 2), row(5, 20, 1)]
    assert staged.matches(rows, graph)
    assert not staged.matches(rows, other)                        # another graph bucket
    assert not staged.matches(rows[::-1], graph)                  # order changed
    assert not staged.matches(rows[:1], graph)                    # a row ended
    assert not staged.matches(rows + [row(9, 4, 1)], graph)       # a row joined
    assert not staged.matches([row(3, 10, 3), rows[1]], graph)    # length moved on
    assert not staged.matches([row(4, 10, 2), rows[1]], graph)    # another request
