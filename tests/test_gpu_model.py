"""Qwen3 model and serving engine on the GPU against the fp32 Qwen3 oracle.

Greedy checks: the GPU engine's free-running token list must equal the oracle's (fp32 on the
same bf16 weights) up to the first step whose oracle top-1/top-2 gap lies inside the measured
bf16 logit error (a genuine near tie, where bf16 arithmetic may pick either); and, teacher-
forced over every step, each emitted token is an argmax of the oracle's logits for the same
prefix within that error. Logits must also agree in direction (cos-sim) with the oracle's.
"""
import numpy as np
import pytest
import torch

from engine_helpers import RecordingEngine
from llm_infer_rust_amd.backend import BatchPhase
from llm_infer_rust_amd.batch import BatchRequest
from llm_infer_rust_amd.engine import Engine, EngineConfig
from llm_infer_rust_amd.model import Qwen3Config, Qwen3Model
from llm_infer_rust_amd.sampling import SamplingParams
from oracle import bf16 as obf
from oracle import qwen3 as oq

pytestmark = pytest.mark.gpu

TINY = Qwen3Config(hidden_size=512, num_layers=2, num_attention_heads=8, num_kv_heads=2,
                   intermediate_size=1024, vocab_size=512, head_dim=128,
                   max_position_embeddings=1024, rope_theta=1_000_000.0)


def build(cfg, seed, gpu, std=0.05):
    w = {k: obf.round_bf16(v) for k, v in oq.random_weights(cfg, seed, std).items()}
    model = Qwen3Model(cfg, torch.bfloat16, gpu)
    assert model.load_weights({k: torch.from_numpy(v) for k, v in w.items()}) == len(w)
    return model, oq.Qwen3Oracle(cfg, w)


def check_teacher_forced(oracle, prompt, tokens, tol):
    oracle.reset()
    logits = oracle.forward(prompt, 0)[-1]
    pos = len(prompt)
    worst, exact = 0.0, 0
    for t in tokens:
        deficit = float(logits.max() - logits[t])
        worst = max(worst, deficit)
        exact += int(deficit == 0.0)
        logits = oracle.forward(np.array([t]), pos)[-1]
        pos += 1
    print(f"teacher-forced: {exact}/{len(tokens)} exact argmax, worst deficit {worst:.4f}")
    assert worst <= tol


@pytest.mark.parametrize("use_graphs", [True, False])
def test_engine_greedy_matches_oracle(gpu, use_graphs):
    model, oracle = build(TINY, 1, gpu)
    cfg = EngineConfig(page_size=16, max_running_req=8, max_prefill_tokens_per_batch=96,
                       max_seq_len=256, use_graphs=use_graphs)
    eng = Engine(model, cfg)
    rng = np.random.default_rng(2)
    lens = [5, 40, 130, 17, 64]  # 130 > budget: chunked, continued as a paged prefill
    prompts = [rng.integers(0, TINY.vocab_size, n) for n in lens]
    reqs = [eng.add_request(p, SamplingParams(max_tokens=12)) for p in prompts]
    eng.run_until_complete()
    assert eng.stats["prefill_batches"] >= 3
    if use_graphs:
        assert eng.stats["graph_steps"] == eng.stats["decode_steps"] > 0
    for req, prompt in zip(reqs, prompts):
        assert len(req.output) == 12 and req.first_token_time is not None
        check_teacher_forced(oracle, prompt, req.output, tol=0.05)
    assert len(eng.pages.free) == eng.pool.layout.num_pages  # every page returned


def test_decode_graph_logits_match_eager(gpu):
    """Every decode step's logits from a graph replay (3 live rows in a 4-row bucket, one pad
    row at page 0 / slot 0) against the eager forward of the same rows: greedy sampling keeps
    both runs on the same tokens, so each step compares the same inputs. A pad row writing a
    live slot, or a position off by one, changes the logits of later steps far beyond the
    bf16 tolerance used here."""
    model, _ = build(TINY, 3, gpu)
    runs = []
    for graphs in (True, False):
        eng = RecordingEngine(model, EngineConfig(max_running_req=4, max_seq_len=128,
                                                  use_graphs=graphs, seed=9,
                                                  graph_batch_sizes=(4,)))
        rng = np.random.default_rng(4)
        for n in (7, 33, 20):
            eng.add_request(rng.integers(0, TINY.vocab_size, n), SamplingParams(max_tokens=8))
        eng.run_until_complete()
        if graphs:
            assert eng.stats["graph_steps"] == eng.stats["decode_steps"] > 0
        else:
            assert eng.stats["graph_steps"] == 0
        runs.append(eng.records)
        del eng
        torch.cuda.synchronize()
    graph, eager = runs
    assert len(graph) == len(eager)
    for step, ((ug, lg, pg), (ue, le, pe)) in enumerate(zip(graph, eager)):
        assert ug == ue and pg == pe, step  # same rows, same greedy tokens
        a, b = lg.double(), le.double()
        cos = torch.nn.functional.cosine_similarity(a, b, dim=1)
        err = float((a - b).abs().max())
        assert float(cos.min()) > 0.99999, (step, cos)
        assert err <= 1e-2 * float(b.abs().max()) + 4e-3, (step, err)


def test_prefill_logits_match_oracle(gpu):
    model, oracle = build(TINY, 5, gpu)
    eng = Engine(model, EngineConfig(max_running_req=2, max_seq_len=128, use_graphs=False))
    prompt = np.random.default_rng(6).integers(0, TINY.vocab_size, 50)
    req = eng.add_request(prompt, SamplingParams(max_tokens=1))
    picked = eng._select_prefill()
    # Run the prefill by hand to read the logits the sampler would see.
    from llm_infer_rust_amd.backend import AttentionMetadata, BatchPhase
    eng.waiting.remove(req)
    eng.running.append(req)
    req.admitted = True
    eng._ensure_pages(req, 50)
    b = eng.batches.prepare_prefill([BatchRequest(prompt, 0, 50, req.pages)])
    ids_d, pos_d, loc_d, cu_d, pre_d, tab_d = eng._upload(
        b.input_ids, b.positions, b.write_loc, b.cu_seqlens_q, b.prefix_lens, b.block_table)
    meta = AttentionMetadata(BatchPhase.PREFILL, write_loc=loc_d, cu_seqlens_q=cu_d,
                             prefix_lens=pre_d, block_table=tab_d,
                             host_cu_seqlens_q=[0, 50], host_prefix_lens=[0])
    batch = model.attention.prepare(meta, 50)
    got = model.forward(ids_d, pos_d, batch, loc_d).float().cpu().numpy()
    want = oracle.forward(prompt, 0)
    cos = (got * want).sum(1) / (np.linalg.norm(got, axis=1) * np.linalg.norm(want, axis=1))
    assert cos.min() > 0.999, cos.min()
    assert np.abs(got - want).max() < 0.05 * np.abs(want).max() + 0.02
    assert picked


def test_config1_shape_greedy_tokens_match_oracle(gpu):
    """Config 1 (Qwen3-0.6B dimensions, 128 random prompt ids, 64 greedy tokens) through the
    engine with graph decode, against the fp32 oracle's own free-running greedy run on the
    same bf16 weights."""
    cfg = Qwen3Config.qwen3_0_6b()
    model, oracle = build(cfg, 0, gpu, std=0.02)
    eng = RecordingEngine(model, EngineConfig(max_running_req=1, max_seq_len=256,
                                              graph_batch_sizes=(1,)))
    prompt = np.random.default_rng(0).integers(0, cfg.vocab_size, 128)
    req = eng.add_request(prompt, SamplingParams(max_tokens=64))
    eng.run_until_complete()
    assert len(req.output) == 64
    # Teacher-forced over all 64 steps: the oracle's logits for the GPU's own prefix. At a
    # step whose logits differ by at most e (max-abs), bf16 arithmetic can only pick a
    # token whose oracle logit is within 2 e of the maximum.
    oracle.reset()
    want = [oracle.forward(prompt, 0)[-1]]
    pos = prompt.size
    for t in req.output[:-1]:
        want.append(oracle.forward(np.array([t]), pos)[-1])
        pos += 1
    errs, exact = [], 0
    for (_, got, picked), ref in zip(eng.records, want):
        e = float(np.abs(got[0].double().numpy() - ref).max())
        assert e < 0.05 * float(np.abs(ref).max()) + 0.02
        deficit = float(ref.max() - ref[picked[0]])
        assert deficit <= 2 * e, (deficit, e)
        exact += int(deficit == 0.0)
        errs.append(e)
    # Free-running: the oracle's own greedy run from the same prompt. The token lists must
    # agree up to the first step where the oracle's top-1/top-2 gap is inside 2 e (a genuine
    # near tie; past it the two sequences legitimately differ).
    oracle.reset()
    logits, pos, ref, gaps = want[0], prompt.size, [], []
    oracle.forward(prompt, 0)
    for _ in range(64):
        top2 = np.sort(logits)[-2:]
        gaps.append(float(top2[1] - top2[0]))
        ref.append(int(np.argmax(logits)))
        logits = oracle.forward(np.array([ref[-1]]), pos)[-1]
        pos += 1
    same = next((i for i, (a, b) in enumerate(zip(req.output, ref)) if a != b), 64)
    print(f"config 1: {same}/64 leading greedy tokens identical to the oracle's, {exact}/64 "
          f"exact argmax teacher-forced; logit error max {max(errs):.4f}; smallest oracle "
          f"gap {min(gaps):.4f}")
    if same < 64:
        assert gaps[same] <= 2 * errs[same], (same, gaps[same], errs[same])


def test_chunked_long_prompt_uses_split_prefill(gpu):
    """A 2,100-token prompt through a 512-token prefill budget: the later chunks are paged
    prefills over long cached prefixes with few items for the device, which the plan splits
    along the keys (split-KV + merge). The first generated tokens must stay within the bf16
    error bound of the oracle's argmax, teacher-forced."""
    model, oracle = build(TINY, 7, gpu)
    eng = Engine(model, EngineConfig(page_size=16, max_running_req=2,
                                     max_prefill_tokens_per_batch=512, max_seq_len=2200,
                                     use_graphs=False))
    prompt = np.random.default_rng(8).integers(0, TINY.vocab_size, 2100)
    seen = []
    real_prepare = model.attention.prepare

    def spy(meta, n):
        batch = real_prepare(meta, n)
        if meta.forward_mode == BatchPhase.PREFILL:
            seen.append(batch.plan.plan.info()["split_items"])
        return batch

    model.attention.prepare = spy
    try:
        req = eng.add_request(prompt, SamplingParams(max_tokens=4))
        eng.run_until_complete()
    finally:
        model.attention.prepare = real_prepare
    assert eng.stats["prefill_batches"] == 5 and max(seen) > 0, seen
    assert len(req.output) == 4
    check_teacher_forced(oracle, prompt, req.output, tol=0.05)


def test_decode_staged_ahead_matches_unstaged(gpu):
    """The graph path stages each decode step while the previous one runs and uses it only
    when the rows, their order and lengths are the ones it was staged for. Greedy tokens with
    staging on must equal those with staging off (same graph bucket, so the same kernels), and
    a request that ends on its end-of-sequence token must discard the staged step: it stops
    right after that token and the other requests carry on unchanged."""
    model, _ = build(TINY, 12, gpu)
    rng = np.random.default_rng(13)
    prompts = [rng.integers(0, TINY.vocab_size, n) for n in (9, 30, 21)]

    def run(eos=None, staged=True):
        eng = Engine(model, EngineConfig(max_running_req=4, max_seq_len=128, seed=3,
                                         graph_batch_sizes=(4,)))
        if not staged:
            eng._prepare_ahead = lambda rows: None
        reqs = [eng.add_request(p, SamplingParams(max_tokens=10),
                                eos_token_id=eos if i == 0 else None)
                for i, p in enumerate(prompts)]
        eng.run_until_complete()
        out = [list(r.output) for r in reqs]
        stats = dict(eng.stats)
        del eng
        torch.cuda.synchronize()
        return out, stats

    plain, st_off = run(staged=False)
    staged, st_on = run()
    assert st_off["ahead_steps"] == 0 and st_on["ahead_steps"] > 0
    assert staged == plain
    # End request 0 on the token it emits at step 4 (its first occurrence there).
    stop = next(i for i in range(3, 9) if plain[0][i] not in plain[0][:i])
    cut, st_eos = run(eos=plain[0][stop])
    assert cut[0] == plain[0][:stop + 1]
    assert cut[1:] == plain[1:]
    assert st_eos["ahead_steps"] > 0


def test_staged_decode_step_is_discarded_when_a_request_arrives(gpu):
    """A request added between steps while every running request decodes: the next step runs
    its prefill first (which rewrites the pinned staging block) and must not use the decode step
    staged before. Greedy tokens must equal a run with staging off, step for step."""
    model, _ = build(TINY, 14, gpu)
    rng = np.random.default_rng(15)
    first = [rng.integers(0, TINY.vocab_size, n) for n in (12, 25)]
    late = rng.integers(0, TINY.vocab_size, 19)

    def run(staged):
        eng = Engine(model, EngineConfig(max_running_req=4, max_seq_len=128, seed=5,
                                         graph_batch_sizes=(4,)))
        if not staged:
            eng._prepare_ahead = lambda rows: None
        reqs = [eng.add_request(p, SamplingParams(max_tokens=9)) for p in first]
        for _ in range(4):  # one prefill step, then decode steps that stage their successors
            eng.step()
        if staged:  # a step is staged (or already launched) when the request arrives
            assert eng._ahead is not None or eng._inflight is not None
        reqs.append(eng.add_request(late, SamplingParams(max_tokens=9)))
        eng.run_until_complete()
        out = [list(r.output) for r in reqs]
        stats = dict(eng.stats)
        del eng
        torch.cuda.synchronize()
        return out, stats

    plain, _ = run(False)
    staged, stats = run(True)
    assert staged == plain and all(len(o) == 9 for o in staged)
    assert stats["ahead_steps"] > 0


def test_overlapped_decode_matches_serial(gpu):
    """The overlap of consecutive decode steps (``scheduler.rs:935-1000``): the next graph step
    is launched with its input tokens fed on the device before the host reads them. Tokens must
    equal the serial engine's under temperature/top-k/top-p sampling (same sampling calls, same
    rows, same seed offsets), with requests ending by length at different steps and one ending
    on its end-of-sequence token (the launched step is dropped and the live rows decode
    again)."""
    model, _ = build(TINY, 17, gpu)
    rng = np.random.default_rng(19)
    prompts = [rng.integers(0, TINY.vocab_size, n) for n in (11, 27, 18, 33)]
    budgets = (12, 9, 14, 12)

    def run(overlap, eos=None):
        eng = Engine(model, EngineConfig(max_running_req=8, max_seq_len=128, seed=7,
                                         graph_batch_sizes=(4, 8), overlap_decode=overlap))
        reqs = [eng.add_request(p, SamplingParams(temperature=0.7, top_k=20, top_p=0.9,
                                                  max_tokens=m),
                                eos_token_id=eos if i == 2 else None)
                for i, (p, m) in enumerate(zip(prompts, budgets))]
        eng.run_until_complete()
        out = [list(r.output) for r in reqs]
        stats = dict(eng.stats)
        del eng
        torch.cuda.synchronize()
        return out, stats

    serial, st_serial = run(False)
    overlapped, st = run(True)
    assert st_serial["overlap_steps"] == 0 and st["overlap_steps"] > 0
    assert st["graph_steps"] == st["decode_steps"] == st_serial["decode_steps"]
    assert overlapped == serial
    assert [len(o) for o in overlapped] == list(budgets)
    stop = next(i for i in range(3, 10) if serial[2][i] not in serial[2][:i])
    cut_serial, _ = run(False, eos=serial[2][stop])
    cut, st_cut = run(True, eos=serial[2][stop])
    assert cut == cut_serial and cut[2] == serial[2][:stop + 1]
    assert st_cut["overlap_steps"] > 0


def test_non_final_prefill_chunk_ends_the_step(gpu):
    """``scheduler.rs`` step_serial: a step whose prefill batch carries a chunk that is not its
    request's last returns before decode. A short request admitted with a long one therefore
    holds its first token until the long prompt's last chunk has run."""
    model, _ = build(TINY, 16, gpu)
    rng = np.random.default_rng(17)
    eng = Engine(model, EngineConfig(page_size=16, max_running_req=2,
                                     max_prefill_tokens_per_batch=48, max_seq_len=256,
                                     use_graphs=False))
    short = eng.add_request(rng.integers(0, TINY.vocab_size, 8), SamplingParams(max_tokens=4))
    long = eng.add_request(rng.integers(0, TINY.vocab_size, 120), SamplingParams(max_tokens=4))
    eng.step()  # short (8) + the long prompt's first chunk (32, page-aligned): no decode
    assert len(short.output) == 1 and long.cursor == 32 and eng.stats["decode_steps"] == 0
    while long.cursor < long.prompt.size:
        eng.step()
        if long.cursor < long.prompt.size:
            assert eng.stats["decode_steps"] == 0 and len(short.output) == 1
    assert eng.stats["decode_steps"] == 1 and len(short.output) == 2  # the last chunk's step
    eng.run_until_complete()
    assert len(short.output) == 4 and len(long.output) == 4
