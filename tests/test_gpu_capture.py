"""Native plans released by Python's garbage collector while a HIP graph is being captured.

A decode or prefill plan frees its device buffers and waits on its upload event when it is
dropped (`mi355x_decode_plan_drop`, `mi355x_prefill_plan_drop`); in a global-mode stream capture
those calls invalidate the capture. Plans held in reference cycles are only dropped when the
collector runs, which can happen in the middle of a capture (an engine capturing its decode
graphs after an earlier engine became garbage). A plan finalized during a capture must park its
handle and be released after the capture instead.
"""
import gc

import pytest
import torch

from llm_infer_rust_amd.backend import (AttentionMetadata, AttentionSpec, BatchPhase,
                                        prepare_decode_plan)

pytestmark = pytest.mark.gpu


def _plan_in_a_cycle(gpu):
    table = torch.arange(1, 9, dtype=torch.int32, device=gpu).view(2, 4)
    lens = torch.tensor([5, 9], dtype=torch.int32, device=gpu)
    meta = AttentionMetadata(BatchPhase.DECODE, block_table=table, cache_seqlens=lens)
    plan = prepare_decode_plan(None, meta, AttentionSpec(16, 8, 128, torch.bfloat16, gpu), 4,
                               False)
    holder = {"plan": plan}
    holder["self"] = holder  # only the collector can free it
    return plan.handle


def test_plan_collected_during_capture_leaves_the_capture_valid(gpu):
    gc.collect()
    enabled = gc.isenabled()
    gc.disable()  # the test decides when the collector runs
    try:
        handle = _plan_in_a_cycle(gpu)
        assert handle
        torch.cuda.synchronize()
        x = torch.zeros(1024, device=gpu)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            y = x + 1.0
            gc.collect()  # finalizes the plan inside the capture
            z = y * 2.0
        for _ in range(3):
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(z, torch.full_like(z, 2.0))
    finally:
        if enabled:
            gc.enable()
    # The parked handle is released at the next safe point (any later plan release).
    from llm_infer_rust_amd import _native
    _native.release_deferred()
    assert _native.deferred_count() == 0
