"""Continuous-batching serving loop around the Qwen3 model on the gfx950 path.

Mirrors the parts of the reference engine that feed the attention hot path:

* ``EngineConfig`` defaults from ``ServerArgs`` (``src/engine/engine.rs:64-82``): page size 16,
  256 running requests, 8192 prefill tokens per batch; decode graphs for batch sizes 1, 2, 4, 8
  and every multiple of 8 up to 256 (finer than the reference's powers of two, see
  ``Engine._bucket_sizes``);
* the serial scheduler step (``src/scheduler/scheduler.rs:205-271``): one prefill batch (FIFO,
  token budget, the last request chunked when it does not fit), then one decode step over every
  running request;
* batch metadata from ``batch.BatchContext`` / ``batch.DecodeTables``
  (``src/engine/batch_context.rs:216-360``, ``src/scheduler/decode.rs:168-422``): int32
  ``block_table`` (-1 past a request's pages) / ``cache_seqlens`` / ``cu_seqlens_q`` /
  ``prefix_lens``, slots ``page * page_size + offset`` for ``write_loc``. Decode block-table
  rows persist across steps and change only when a row gets another request or a page; one
  pinned staging block is uploaded per step and the planner reads host lengths, never device
  ones;
* ``DecodeGraphRunner`` (``src/engine/graph.rs:26-329``): fixed input buffers per captured batch
  size, pad rows pointing at the reserved page 0 (length 1, slot 0 skipped by the K/V store),
  and the attention plan re-made outside the graph before each replay
  (``DecodeGraphState.prepare_replay``);
* sampling with a pinned asynchronous readback (``src/engine/sampling.rs:193-237``);
* the CPU/GPU overlap of consecutive decode steps (``scheduler.rs:935-1000`` step_overlap):
  the next graph step is launched with its input tokens copied on the device from this step's
  sampling output, before the host reads them (``Engine._launch_ahead``).
"""
from __future__ import annotations

import gc
import time
from dataclasses import dataclass, field

import numpy as np
import torch

from . import _native
from .backend import AttentionMetadata, BatchPhase, DecodeHostMetadata
from .batch import BatchContext, BatchRequest, DecodeBatch, DecodeRequest, DecodeTables
from .kv_cache import KVCacheLayout, KVCachePool, ModelError
from .model import Qwen3Model
from .sampling import Sampler, SamplingParams


@dataclass
class EngineConfig:
    page_size: int = 16
    max_running_req: int = 256
    max_prefill_tokens_per_batch: int = 8192
    max_seq_len: int = 4096
    num_pages: int | None = None           # default: every running request at max_seq_len
    graph_batch_sizes: tuple[int, ...] | None = None  # default 1, 2, 4, 8, 16, 24, ... <= max_running_req
    use_graphs: bool = True
    # Launch the next graph decode step before this step's tokens reach the host, feeding them
    # on the device (the reference's CPU/GPU overlap mode, ``scheduler.rs:935-1000``); only
    # when the next step decodes exactly this step's rows (no prefill waiting, no row ending by
    # length). False: the serial step of ``scheduler.rs:225-271`` every time.
    overlap_decode: bool = True
    seed: int = 0


@dataclass(eq=False)
class Request:
    uid: int
    prompt: np.ndarray
    params: SamplingParams
    eos_token_id: int | None = None
    output: list[int] = field(default_factory=list)
    pages: list[int] = field(default_factory=list)
    cursor: int = 0                 # prompt tokens already in the cache
    admitted: bool = False          # holds a running slot
    arrival: float = 0.0
    first_token_time: float | None = None
    finish_time: float | None = None

    @property
    def cached_len(self) -> int:
        """Tokens whose K/V are in the cache (the prompt cursor, then every fed output)."""
        return self.cursor + max(len(self.output) - 1, 0)

    def finished(self) -> bool:
        if not self.output:
            return False
        if len(self.output) >= self.params.max_tokens:
            return True
        return (not self.params.ignore_eos and self.eos_token_id is not None
                and self.output[-1] == self.eos_token_id)


class PageAllocator:
    """Physical pages 1..num_pages; page 0 is the reserved zero page."""

    def __init__(self, num_pages: int):
        self.free = list(range(num_pages, 0, -1))

    def alloc(self, n: int) -> list[int]:
        if n > len(self.free):
            raise ModelError("out of KV-cache pages")
        out = self.free[-n:][::-1] if n else []
        del self.free[len(self.free) - n:]
        return out

    def release(self, pages: list[int]) -> None:
        self.free.extend(reversed(pages))


def _words(a: np.ndarray) -> np.ndarray:
    """An int32/int64 array as a flat run of 8-byte words (int32 padded to an even count)."""
    flat = np.ascontiguousarray(a).reshape(-1)
    if flat.dtype == np.int32:
        if flat.size % 2:
            flat = np.concatenate([flat, np.zeros(1, np.int32)])
        return flat.view(np.int64)
    return flat.astype(np.int64, copy=False)


def _views(block: torch.Tensor, arrays) -> list[torch.Tensor]:
    """Typed views of a word block laid out as ``_words`` packs ``arrays``."""
    out, off = [], 0
    for a in arrays:
        if a.dtype == np.int32:
            words = (a.size + 1) // 2
            out.append(block[off:off + words].view(torch.int32)[:a.size].view(a.shape))
        else:
            words = a.size
            out.append(block[off:off + words].view(a.shape))
        off += words
    return out


class _DecodeGraph:
    """One captured decode step; its inputs are views of one device word block."""

    def __init__(self, bs: int, cols: int, vocab: int, device: torch.device,
                 dtype: torch.dtype):
        self.bs = bs
        shapes = (np.zeros(bs, np.int64), np.zeros(bs, np.int64), np.zeros(bs, np.int64),
                  np.zeros(bs, np.int32), np.zeros((bs, cols), np.int32))
        words = sum(_words(a).size for a in shapes)
        self.block = torch.zeros(words, dtype=torch.int64, device=device)
        (self.input_ids, self.positions, self.write_loc, self.cache_seqlens,
         self.block_table) = _views(self.block, shapes)
        self.cache_seqlens.fill_(1)
        self.logits = torch.empty(bs, vocab, dtype=dtype, device=device)
        self.graph: torch.cuda.CUDAGraph | None = None
        self.state = None
        self.batch = None


@dataclass
class _InFlight:
    """A graph decode step launched before the previous step's tokens reached the host: its
    rows (the previous step's, in order) and the graph whose logits it fills."""

    rows: list
    graph: _DecodeGraph


@dataclass
class _Ahead:
    """A decode step staged one step early: its rows, their lengths, the graph bucket and the
    staged words (the input-token run still to be written once the tokens are known)."""

    uids: list[int]
    lengths: list[int]
    graph: _DecodeGraph
    host: np.ndarray
    lens: np.ndarray

    def same_rows(self, rows: list) -> bool:
        """Staged for exactly these rows, in this order (none of them ends by length)."""
        return len(rows) == len(self.uids) and all(r.uid == u for r, u in zip(rows, self.uids))

    def matches(self, rows: list, graph: _DecodeGraph) -> bool:
        """The staged step is the one to run: same graph, same rows in the same order, each
        at the length it was staged for (pages only grow, and the staging ensured them)."""
        return (graph is self.graph and len(rows) == len(self.uids)
                and all(r.uid == u and r.cursor + len(r.output) == n
                        for r, u, n in zip(rows, self.uids, self.lengths)))


class Engine:
    def __init__(self, model: Qwen3Model, config: EngineConfig | None = None):
        self.model = model
        self.cfg = config or EngineConfig()
        cfg, mcfg = self.cfg, model.cfg
        self.device = model.device
        self.page_size = cfg.page_size
        self.cols = -(-cfg.max_seq_len // cfg.page_size)  # block-table columns
        num_pages = cfg.num_pages or cfg.max_running_req * self.cols
        self.pool = KVCachePool(KVCacheLayout(mcfg.num_layers, num_pages, cfg.page_size,
                                              mcfg.num_kv_heads, mcfg.head_dim),
                                model.dtype, self.device)
        model.bind_kv_cache(self.pool, reserved_slot=0)
        self.pages = PageAllocator(num_pages)
        self.batches = BatchContext(cfg.max_running_req, cfg.max_seq_len, cfg.page_size)
        self.tables = DecodeTables(cfg.max_running_req, cfg.max_seq_len, cfg.page_size)
        self.sampler = Sampler(cfg.seed)
        self.waiting: list[Request] = []
        self.running: list[Request] = []
        self.finished: list[Request] = []
        self._next_uid = 0
        self._staging = torch.empty(0, dtype=torch.int64, pin_memory=True)
        self._staging_copy: torch.cuda.Event | None = None
        self._ahead: _Ahead | None = None           # next decode step, staged while this one runs
        self._inflight: _InFlight | None = None     # next decode step, already launched
        self._pending_rows: list[Request] | None = None
        self.graphs: dict[int, _DecodeGraph] = {}
        self.stats = {"prefill_batches": 0, "decode_steps": 0, "graph_steps": 0,
                      "ahead_steps": 0, "overlap_steps": 0}
        if cfg.use_graphs:
            self.capture_graphs()

    # ------------------------------------------------------------------ requests
    def add_request(self, prompt, params: SamplingParams,
                    eos_token_id: int | None = None) -> Request:
        prompt = np.asarray(prompt, dtype=np.int64)
        params = params.normalized()
        if prompt.ndim != 1 or prompt.size == 0:
            raise ModelError("prompt must be a non-empty 1-D id list")
        if prompt.size + params.max_tokens > self.cfg.max_seq_len:
            raise ModelError("prompt + max_tokens exceeds max_seq_len")
        req = Request(self._next_uid, prompt, params, eos_token_id, arrival=time.perf_counter())
        self._next_uid += 1
        self.waiting.append(req)
        return req

    def _ensure_pages(self, req: Request, tokens: int) -> None:
        need = -(-tokens // self.page_size) - len(req.pages)
        if need > 0:
            req.pages.extend(self.pages.alloc(need))

    def _staging_words(self, total: int) -> np.ndarray:
        """The pinned staging block as ``total`` writable int64 words. The previous upload's
        copy out of it is asynchronous, so wait for that copy before the block is rewritten."""
        self._ahead = None  # a step staged ahead lives in this block: rewriting it voids that
        if self._staging_copy is not None:
            self._staging_copy.synchronize()
            self._staging_copy = None
        if self._staging.numel() < total:
            self._staging = torch.empty(max(total, 2 * self._staging.numel()), dtype=torch.int64,
                                        pin_memory=True)
        return self._staging.numpy()[:total]

    def _send(self, total: int, dst: torch.Tensor | None = None) -> torch.Tensor:
        """One asynchronous host-to-device copy of the first ``total`` staged words (into
        ``dst`` when given), remembered so the next writer waits for it."""
        src = self._staging[:total]
        if dst is None:
            dst = src.to(self.device, non_blocking=True)
        else:
            dst.copy_(src, non_blocking=True)
        self._staging_copy = torch.cuda.Event()
        self._staging_copy.record(torch.cuda.current_stream(self.device))
        return dst

    def _pack(self, arrays) -> int:
        """Copy int32/int64 arrays into the pinned staging buffer as 8-byte words."""
        words = [_words(a) for a in arrays]
        total = sum(w.size for w in words)
        host = self._staging_words(total)
        off = 0
        for w in words:
            host[off:off + w.size] = w
            off += w.size
        return total

    def _upload(self, *arrays: np.ndarray) -> list[torch.Tensor]:
        """One pinned staging block, one host-to-device copy; returns typed device views."""
        return _views(self._send(self._pack(arrays)), arrays)

    # ------------------------------------------------------------------ prefill
    def _select_prefill(self) -> list[tuple[Request, int]]:
        budget = self.cfg.max_prefill_tokens_per_batch
        picked: list[tuple[Request, int]] = []
        admitted = len(self.running)
        # A chunked request continues first (scheduler/prefill.rs select_continuation).
        queue = [r for r in self.running if r.cursor < r.prompt.size] + self.waiting
        for req in queue:
            if budget <= 0:
                break
            if not req.admitted:
                if admitted >= self.cfg.max_running_req:
                    break
                admitted += 1
            remaining = req.prompt.size - req.cursor
            take = min(remaining, budget)
            if take < remaining:  # chunks end on a page boundary
                take -= (req.cursor + take) % self.page_size
                if take <= 0:
                    break
            picked.append((req, take))
            budget -= take
        return picked

    def _run_prefill(self, picked: list[tuple[Request, int]]) -> None:
        rows = []
        for req, take in picked:
            if not req.admitted:
                req.admitted = True
                self.waiting.remove(req)
                self.running.append(req)
            self._ensure_pages(req, req.cursor + take)
            rows.append(BatchRequest(req.prompt, req.cursor, req.cursor + take, req.pages))
        b = self.batches.prepare_prefill(rows)
        # Logits only for requests whose prompt ends in this batch (possibly none).
        last = np.asarray([i for (req, take), i in zip(picked, b.logits_indices)
                           if req.cursor + take == req.prompt.size], np.int64)
        ids_d, pos_d, loc_d, idx_d, cu_d, prefix_d, table_d = self._upload(
            b.input_ids, b.positions, b.write_loc, last, b.cu_seqlens_q, b.prefix_lens,
            b.block_table)
        meta = AttentionMetadata(BatchPhase.PREFILL, write_loc=loc_d, cu_seqlens_q=cu_d,
                                 prefix_lens=prefix_d, block_table=table_d,
                                 host_cu_seqlens_q=b.cu_seqlens_q.tolist(),
                                 host_prefix_lens=b.prefix_lens.tolist())
        batch = self.model.attention.prepare(meta, int(b.cu_seqlens_q[-1]))
        logits = self.model.forward(ids_d, pos_d, batch, loc_d, idx_d)
        del batch
        for req, take in picked:
            req.cursor += take
        done = [req for req, _ in picked if req.cursor == req.prompt.size]
        self.stats["prefill_batches"] += 1
        if done:
            self._sample_and_commit(logits, done)

    # ------------------------------------------------------------------ decode
    def _decode_rows(self) -> list[Request]:
        return [r for r in self.running if r.cursor == r.prompt.size and r.output
                and not r.finished()]

    def _decode_batch(self, rows: list[Request]) -> DecodeBatch:
        ps = self.page_size
        reqs = []
        for req in rows:
            length = req.cursor + len(req.output)  # cached_len + 1: the fed token's position + 1
            if -(-length // ps) > len(req.pages):
                self._ensure_pages(req, length)
            reqs.append(DecodeRequest(req.uid, length, req.output[-1], req.pages))
        return self.tables.prepare(reqs)

    def _run_decode(self, rows: list[Request]) -> None:
        n = len(rows)
        graph = self._graph_for(n)
        ahead, self._ahead = self._ahead, None
        if graph is not None:
            if ahead is not None and ahead.matches(rows, graph):
                host, lens = ahead.host, ahead.lens
                host[:n] = [req.output[-1] for req in rows]  # the tokens sampled last step
                self.stats["ahead_steps"] += 1
            else:
                host, lens = self._stage_replay(graph, self._decode_batch(rows))
            self._launch_replay(graph, host, lens)
            logits = graph.logits[:n]
            self.stats["graph_steps"] += 1
        else:
            b = self._decode_batch(rows)
            ids_d, pos_d, loc_d, lens_d, table_d = self._upload(
                b.input_ids, b.positions, b.write_loc, b.cache_seqlens, b.block_table)
            meta = AttentionMetadata(BatchPhase.DECODE, decode_host=DecodeHostMetadata(
                b.cache_seqlens.tolist()), write_loc=loc_d, block_table=table_d,
                cache_seqlens=lens_d)
            batch = self.model.attention.prepare(meta, n)
            logits = self.model.forward(ids_d, pos_d, batch, loc_d)
            del batch
        self.stats["decode_steps"] += 1
        if graph is not None:
            self._pending_rows = rows  # the sampler's wait runs the next step's host work
        self._sample_and_commit(logits, rows)

    def _prepare_ahead(self, rows: list[Request]) -> None:
        """While this step runs on the GPU: stage the next decode step for the rows that will
        still decode (this step's sampling cannot end them by length; an end-of-sequence token
        or a prefill that changes the row set discards the staging, see ``_Ahead.matches``)."""
        if self.waiting or any(r.cursor < r.prompt.size for r in self.running):
            return  # the next step starts with a prefill and changes the decode rows
        nxt = [r for r in rows if len(r.output) + 1 < r.params.max_tokens]
        graph = self._graph_for(len(nxt)) if nxt else None
        if graph is None:
            return
        ps = self.page_size
        lengths = [req.cursor + len(req.output) + 1 for req in nxt]  # after this step's token
        need = sum(max(0, -(-n // ps) - len(req.pages)) for req, n in zip(nxt, lengths))
        if need > len(self.pages.free):
            return  # the next step raises "out of KV-cache pages" itself, after this commit
        reqs = []
        for req, length in zip(nxt, lengths):
            if -(-length // ps) > len(req.pages):
                self._ensure_pages(req, length)
            reqs.append(DecodeRequest(req.uid, length, 0, req.pages))
        host, lens = self._stage_replay(graph, self.tables.prepare(reqs))
        self._ahead = _Ahead([r.uid for r in nxt], lengths, graph, host, lens)

    def _launch_ahead(self, pending, rows: list[Request]) -> _InFlight | None:
        """Launch the staged step now when it decodes exactly this step's rows: its words go
        to the graph inputs with the input-token run overwritten on the device by this step's
        sampled ids (the -1 of an invalid row clamped to 0; that row raises at its commit and
        the launched step is dropped), then the re-plan and the replay. The host reads this
        step's tokens afterwards, while the next step runs."""
        ahead = self._ahead
        if ahead is None or not self.cfg.overlap_decode or not ahead.same_rows(rows):
            return None
        self._ahead = None
        g, n = ahead.graph, len(rows)
        self._send(ahead.host.size, g.block)
        torch.clamp(pending.ids, min=0, out=g.input_ids[:n])
        g.state.prepare_replay(DecodeHostMetadata(ahead.lens))
        g.graph.replay()
        return _InFlight(rows, g)

    def _sample_and_commit(self, logits: torch.Tensor, rows: list[Request]) -> None:
        pending = self.sampler.defer_batch(logits, [r.params for r in rows])
        ahead_rows, self._pending_rows = self._pending_rows, None
        inflight = None
        if ahead_rows is not None:
            self._prepare_ahead(ahead_rows)
            inflight = self._launch_ahead(pending, ahead_rows)
        ids = pending.finish()
        now = time.perf_counter()
        done = []
        for req, tok in zip(rows, ids):
            req.output.append(tok)
            if req.first_token_time is None:
                req.first_token_time = now
            if req.finished():
                req.finish_time = now
                done.append(req)
        for req in done:
            self.running.remove(req)
            self.finished.append(req)
            self.pages.release(req.pages)
            req.pages = []
        self._inflight = inflight

    # ------------------------------------------------------------------ graphs
    def _bucket_sizes(self) -> list[int]:
        """Captured decode batch sizes: 1, 2, 4, 8, then every multiple of 8 up to
        max_running_req (and max_running_req itself). The reference captures powers of two
        (``graph.rs:92-96``), which replays a partly filled step (the ramp-up while prompts are
        still being prefilled, the tail as requests finish) on up to twice its rows; with
        multiples of 8 a step carries at most 7 pad rows. Measured at config 5 (256 x 1024 ->
        512): 12,280-12,439 output tok/s against 11,989-12,152 with power-of-two buckets and
        12,287-12,291 with eager decode launches, alternating runs on one box."""
        if self.cfg.graph_batch_sizes is not None:
            return sorted(set(self.cfg.graph_batch_sizes))
        top = self.cfg.max_running_req
        out = [bs for bs in (1, 2, 4, 8) if bs < top] + list(range(16, top, 8)) + [top]
        return sorted(set(out))

    def _graph_for(self, n: int) -> _DecodeGraph | None:
        for bs in sorted(self.graphs):
            if bs >= n:
                return self.graphs[bs]
        return None

    def capture_graphs(self) -> None:
        """Capture one decode step per bucket, largest first, sharing one memory pool.

        Garbage is collected before the captures and the collector is paused during them: a
        finalizer that calls into HIP (a native plan's release, for one) would otherwise be
        able to run in the middle of a capture and invalidate it. Plans finalized anyway are
        parked and released after the last capture (``_native.release_handle``)."""
        gc.collect()
        collecting = gc.isenabled()
        gc.disable()
        try:
            self._capture_buckets()
        finally:
            if collecting:
                gc.enable()
            _native.release_deferred()

    def _capture_buckets(self) -> None:
        model = self.model
        pool = torch.cuda.graph_pool_handle()
        for bs in sorted(self._bucket_sizes(), reverse=True):
            g = _DecodeGraph(bs, self.cols, model.cfg.vocab_size, self.device, model.dtype)
            meta = AttentionMetadata(BatchPhase.DECODE, write_loc=g.write_loc,
                                     block_table=g.block_table, cache_seqlens=g.cache_seqlens)
            g.state = model.attention.prepare_decode_graph(meta)
            g.state.prepare_replay(DecodeHostMetadata([1] * bs))
            g.batch = model.attention.prepare(meta, bs)
            side = torch.cuda.Stream(self.device)
            side.wait_stream(torch.cuda.current_stream(self.device))
            with torch.cuda.stream(side):  # warm-up run: library workspaces, hipBLASLt choice
                model.forward(g.input_ids, g.positions, g.batch, g.write_loc,
                              logits_out=g.logits)
            torch.cuda.current_stream(self.device).wait_stream(side)
            torch.cuda.synchronize(self.device)
            g.graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g.graph, pool=pool):
                model.forward(g.input_ids, g.positions, g.batch, g.write_loc,
                              logits_out=g.logits)
            torch.cuda.synchronize(self.device)
            self.graphs[bs] = g

    def _stage_replay(self, g: _DecodeGraph, b: DecodeBatch) -> tuple[np.ndarray, np.ndarray]:
        """Write a decode batch into the pinned staging block in the graph's input layout
        (``_DecodeGraph``: three int64 runs, then the int32 lengths and block table). Pad rows
        (``graph.rs:285-320``): token 1 at position 0, the reserved slot 0, length 1, every
        block-table column page 0. Returns the staged words and the staged lengths."""
        n, bs, cols = b.input_ids.size, g.bs, self.cols
        len_words, tab_words = (bs + 1) // 2, (bs * cols + 1) // 2
        host = self._staging_words(3 * bs + len_words + tab_words)
        for k, (src, pad) in enumerate(((b.input_ids, 1), (b.positions, 0), (b.write_loc, 0))):
            run = host[k * bs:(k + 1) * bs]
            run[:n] = src
            run[n:] = pad
        lens = host[3 * bs:3 * bs + len_words].view(np.int32)[:bs]
        lens[:n] = b.cache_seqlens
        lens[n:] = 1
        table = host[3 * bs + len_words:].view(np.int32)[:bs * cols].reshape(bs, cols)
        table[:n] = b.block_table
        table[n:] = 0
        return host, lens

    def _launch_replay(self, g: _DecodeGraph, host: np.ndarray, lens: np.ndarray) -> None:
        """One copy into the graph's inputs, the host-length re-plan, the replay."""
        self._send(host.size, g.block)
        g.state.prepare_replay(DecodeHostMetadata(lens))
        g.graph.replay()

    # ------------------------------------------------------------------ loop
    def step(self) -> None:
        """Prefill, then decode every running request (``scheduler.rs:204-271`` step_serial);
        a step whose prefill ran a chunk that is not its request's last ends there. A decode
        step launched ahead by the previous step (``_launch_ahead``) is this step's decode: its
        tokens are sampled and committed, and it may launch its own successor. If one of its
        rows ended on an end-of-sequence token meanwhile, the launched step is dropped and the
        live rows decode again (its K/V writes are rewritten with the same values)."""
        if self._inflight is not None:
            fl, self._inflight = self._inflight, None
            if all(not r.finished() for r in fl.rows):
                self.stats["decode_steps"] += 1
                self.stats["graph_steps"] += 1
                self.stats["ahead_steps"] += 1
                self.stats["overlap_steps"] += 1
                self._pending_rows = fl.rows
                self._sample_and_commit(fl.graph.logits[:len(fl.rows)], fl.rows)
                return
        picked = self._select_prefill()
        if picked:
            self._run_prefill(picked)
            if any(req.cursor < req.prompt.size for req, _ in picked):
                return
        rows = self._decode_rows()
        if rows:
            self._run_decode(rows)

    def has_work(self) -> bool:
        return bool(self.waiting or self.running)

    def run_until_complete(self) -> list[Request]:
        while self.has_work():
            self.step()
        self.model.check_write_errors()
        return self.finished


__all__ = ["Engine", "EngineConfig", "Request", "PageAllocator"]
