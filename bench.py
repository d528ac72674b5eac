"""Benchmark of the gfx950 attention hot path (one GPU).

Workload: paged bf16 decode attention plus the K/V
store of the new token: batch 64, 16 q / 8 kv heads, head_dim 128, per-request
KV length uniform in [512, 4096], page size 1, page table a seeded random
permutation of a 4M-slot pool, Q/K/V ~ N(0,1), sm_scale 1/sqrt(128), one new
token's K/V written per request via int64 positions.

A step = write_kv(64 new tokens) + decode attention for one layer, on a plan
prepared once per forward (as the reference reuses one plan across layers).
`value` = algorithmic bytes of a step / measured step time. The roofline
object is for the decode kernels alone, timed with HIP events on the stream
they run on.

Prints ONE JSON line.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

import torch

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
COPY_CAL_BYTES = 256 << 20
# Prefill / norm sections time a fixed number of launches (after a fixed warm-up), so
# their figures do not depend on --steps; sustained prefill runs clock down under the
# MFMA load, and these counts measure that sustained rate.
PREFILL_WARMUP = 100
SECTION_REPS = 100
# The device's power management settles over tens of milliseconds of load (measured:
# cfg4 prefill launches fall from ~550 to ~410 us over the first ~100 launches, decode
# from ~113 to ~109 us), so every timed region is preceded by a fixed device warm-up of
# the same work, and the decode launches of the roofline figure are timed over their own
# fixed count. The headline value still times exactly --steps steps after --warmup.
DEVICE_WARMUP_STEPS = 300
ROOFLINE_REPS = 200
LAYERS = 4  # KV pools the decode steps rotate over (4 x 16 GiB)
TRAFFIC_SUMMARY = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                               "decode_cfg2_traffic.txt")


def host_threads() -> int:
    """Threads for the CPU baselines: the process's share of the host's cores. The GPU box
    gives one GPU's job a 16-CPU share (exported as OMP_NUM_THREADS) whatever os.cpu_count()
    reports for the whole host, so the share, not the host count, is what runs without
    oversubscription; both are recorded by ``host_cpu``."""
    share = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else None
    env = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    return max(1, min(x for x in (share, env or None, os.cpu_count() or 1) if x))


def host_cpu(threads: int) -> dict:
    """The host CPU a baseline ran on: lscpu's model name, os.cpu_count(), the CPUs this
    process may run on, and the threads torch and the numpy BLAS actually use."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    info = {"model": model, "os_cpu_count": os.cpu_count(),
            "affinity_cpus": (len(os.sched_getaffinity(0))
                              if hasattr(os, "sched_getaffinity") else None),
            "threads": threads, "torch_threads": torch.get_num_threads()}
    try:
        from threadpoolctl import threadpool_info
        info["blas_threads"] = sorted({p.get("num_threads") for p in threadpool_info()
                                       if p.get("user_api") == "blas"})
    except Exception:  # threadpoolctl absent: the env var is what the BLAS read at load
        info["blas_threads"] = os.environ.get("OPENBLAS_NUM_THREADS") or os.environ.get(
            "OMP_NUM_THREADS")
    return info


def set_host_threads() -> int:
    """Applies ``host_threads()`` to torch and to the numpy BLAS; returns the count."""
    threads = host_threads()
    torch.set_num_threads(threads)
    try:
        from threadpoolctl import threadpool_limits
        threadpool_limits(threads)
    except Exception:
        pass
    return threads


def measured_traffic():
    """HBM bytes per decode launch from the committed rocprofv3 --pmc summary, if any."""
    try:
        with open(TRAFFIC_SUMMARY) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(float(line.split(":", 1)[1]))
    except OSError:
        return None
    return None
def e2e_section(dev, args) -> dict:
    """Qwen3-8B shapes, random bf16 weights N(0, 0.02) (seeded), 256
    requests x 1024 random ids -> 512 output tokens each, continuous batching, hipGraph decode,
    joint sampling T 0.7 / top-k 50 / top-p 0.9 with a fixed seed. All requests arrive at t=0;
    TTFT is arrival -> first sampled token on the host."""
    from llm_infer_rust_amd.engine import Engine, EngineConfig
    from llm_infer_rust_amd.model import Qwen3Config, Qwen3Model
    from llm_infer_rust_amd.sampling import SamplingParams
    import dataclasses
    import numpy as np

    cfg = Qwen3Config.qwen3_8b()
    if args.e2e_layers:
        cfg = dataclasses.replace(cfg, num_layers=args.e2e_layers)
    t0 = time.perf_counter()
    model = Qwen3Model(cfg, torch.bfloat16, dev).init_random(seed=args.seed)
    n_req, n_in, n_out = args.e2e_requests, args.e2e_input, args.e2e_output
    rng = np.random.default_rng(args.seed)
    params = SamplingParams(temperature=0.7, top_k=50, top_p=0.9, ignore_eos=True,
                            max_tokens=n_out)
    prompts = [rng.integers(0, cfg.vocab_size, n_in) for _ in range(n_req)]

    def serve(use_graphs: bool) -> dict:
        eng = Engine(model, EngineConfig(page_size=16, max_running_req=256,
                                         max_prefill_tokens_per_batch=8192,
                                         max_seq_len=n_in + n_out, seed=args.seed,
                                         use_graphs=use_graphs))
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        reqs = [eng.add_request(p, params) for p in prompts]
        eng.run_until_complete()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        ttft = sorted((r.first_token_time - r.arrival) * 1e3 for r in reqs)
        out_tokens = sum(len(r.output) for r in reqs)
        # Properties of the full-size run (after the timed region): every request produced
        # its whole budget of in-vocabulary tokens, every KV page came back, and with graphs
        # every decode step was a graph replay. A plumbing bug fails the bench here rather
        # than passing silently.
        checks = {
            "all_outputs_full_length": all(len(r.output) == n_out for r in reqs),
            "all_tokens_in_vocab": all(0 <= t < cfg.vocab_size for r in reqs for t in r.output),
            "all_pages_returned": len(eng.pages.free) == eng.pool.layout.num_pages,
        }
        if use_graphs:
            checks["every_decode_step_a_graph_replay"] = (
                eng.stats["graph_steps"] == eng.stats["decode_steps"] > 0)
        failed = [k for k, ok in checks.items() if not ok]
        if failed:
            raise AssertionError(f"e2e run failed its output checks: {failed}")
        out = {"output_tok_s": round(out_tokens / wall, 1),
               "p50_ttft_ms": round(statistics.median(ttft), 1),
               "p90_ttft_ms": round(ttft[int(0.9 * (len(ttft) - 1))], 1),
               "wall_s": round(wall, 3), "output_tokens": out_tokens,
               "prefill_batches": eng.stats["prefill_batches"],
               "decode_steps": eng.stats["decode_steps"],
               "graph_steps": eng.stats["graph_steps"], "ahead_steps": eng.stats["ahead_steps"],
               "overlap_steps": eng.stats["overlap_steps"], "checks": checks}
        del eng
        torch.cuda.empty_cache()
        return out

    torch.cuda.synchronize()
    setup_s = time.perf_counter() - t0
    graph = serve(True)  # the config-5 run: hipGraph-captured decode
    result = {
        **graph,
        "input_tokens": n_req * n_in,
        "setup_s": round(setup_s, 1),
        "config": {"model": "Qwen3-8B shape (random bf16 N(0,0.02) weights)",
                   "layers": cfg.num_layers, "requests": n_req, "input": n_in,
                   "output": n_out, "page_size": 16, "max_prefill_tokens": 8192,
                   "sampling": "T0.7 k50 p0.9 seed %d" % args.seed},
    }
    if not getattr(args, "e2e_graph_only", False):
        # The same serving run with the decode step launched eagerly (no graph), reported
        # beside the graph figure on the same box. The pause before it (outside both timed
        # regions) separates the two runs in a kernel trace (--summarize-gaps).
        time.sleep(0.5)
        eager = serve(False)
        result["eager_decode"] = {k: eager[k] for k in ("output_tok_s", "p50_ttft_ms",
                                                          "p90_ttft_ms", "wall_s")}
    del model
    torch.cuda.empty_cache()
    if not getattr(args, "no_cpu_baseline", False):
        result["cpu_baseline"] = e2e_cpu_baseline(args.seed)
    return result


def e2e_cpu_baseline(seed: int) -> dict:
    """Host-CPU reference for config 5 (reported baseline): the oracle's numpy fp32
    restatement of the reference CPU eager forward (model.rs:155-534, `pt` backend) at the
    Qwen3-8B widths, one request: a 1024-token prefill (logits of the last row only, as the
    reference computes them at logits_indices) and 8 cached decode steps, timed with 1 and
    with 2 decoder layers. Each time is a fixed part (embedding, final norm, lm_head) plus a
    per-layer part; the two fits give the 36-layer model's TTFT and per-token decode time."""
    import dataclasses
    import numpy as np
    from llm_infer_rust_amd.model import Qwen3Config
    from oracle import qwen3 as oq  # the CPU baseline only

    cfg8 = Qwen3Config.qwen3_8b()
    cfg2 = dataclasses.replace(cfg8, num_layers=2, max_position_embeddings=2048)
    cfg1 = dataclasses.replace(cfg2, num_layers=1)
    w2 = oq.random_weights(cfg2, seed)
    w1 = {k: v for k, v in w2.items() if not k.startswith("model.layers.1.")}
    prompt = np.random.default_rng(seed).integers(0, cfg8.vocab_size, 1024)
    steps = 8
    times = {}
    threads = set_host_threads()
    for layers, cfg, w in ((1, cfg1, w1), (2, cfg2, w2)):
        m = oq.Qwen3Oracle(cfg, w)
        t0 = time.perf_counter()
        tok = int(np.argmax(m.forward(prompt, 0, last_only=True)[-1]))
        t_pre = time.perf_counter() - t0
        pos = prompt.size
        t0 = time.perf_counter()
        for _ in range(steps):
            tok = int(np.argmax(m.forward(np.array([tok]), pos)[-1]))
            pos += 1
        times[layers] = (t_pre, (time.perf_counter() - t0) / steps)
        del m
    del w1, w2

    def at_36(i):
        per_layer = times[2][i] - times[1][i]
        return times[1][i] - per_layer + cfg8.num_layers * per_layer

    ttft_s, token_s = at_36(0), at_36(1)
    return {"value": round(1.0 / token_s, 3), "unit": "output tok/s (one request)",
            "ttft_ms": round(ttft_s * 1e3, 1), "cores": threads, "kind": "port",
            "host": host_cpu(threads),
            "sample": ("numpy fp32 restatement of the reference CPU eager forward at the "
                       "Qwen3-8B widths, one request: 1024-token prefill + 8 decode steps "
                       "timed at 1 and 2 layers, fixed + per-layer parts extrapolated to 36 "
                       f"layers (measured: prefill {times[1][0]:.2f} / {times[2][0]:.2f} s, "
                       f"decode {times[1][1] * 1e3:.0f} / {times[2][1] * 1e3:.0f} ms per token)")}


def summarize_kernel_trace(path: str, top: int = 40) -> str:
    """Per-(kernel, grid) launch statistics from a rocprofv3 kernel_trace.csv: kernels that
    run at several shapes (one prefill template serves config 4 and the long-prefix
    continuation, for example) get a row per grid size, which the profiler's own stats merge.
    Host-side text processing only (no GPU)."""
    import csv
    import re

    rows: dict = {}
    total = 0.0
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            dur = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
            grid = int(r.get("Grid_Size_X", 0) or 0) * int(r.get("Grid_Size_Y", 1) or 1) * int(
                r.get("Grid_Size_Z", 1) or 1)
            name = r["Kernel_Name"].replace("void ", "", 1)
            name = name.replace("mi355x::(anonymous namespace)::", "")
            name = re.sub(r"\(anonymous namespace\)::", "", name)
            name = re.sub(r"\(.*", "", name)
            rows.setdefault((name[:70], grid), []).append(dur)
            total += dur
    lines = [f"{'kernel':70s} {'grid':>10s} {'calls':>7s} {'avg_us':>9s} {'median_us':>9s} "
             f"{'min_us':>8s} {'max_us':>8s} {'share%':>7s}"]
    ranked = sorted(rows.items(), key=lambda kv: -sum(kv[1]))[:top]
    for (name, grid), d in ranked:
        d = sorted(d)
        lines.append(f"{name:70s} {grid:10d} {len(d):7d} {sum(d) / len(d):9.2f} "
                     f"{d[len(d) // 2]:9.2f} {d[0]:8.2f} {d[-1]:8.2f} "
                     f"{100 * sum(d) / total:7.2f}")
    return "\n".join(lines)


def summarize_counters(paths: list, match: str = "") -> str:
    """Per-(kernel, grid) means of every counter in rocprofv3 --pmc counter_collection.csv
    files (one file per counter pass; kernels whose name contains `match`). Host-side text
    processing only (no GPU)."""
    import csv
    import re

    acc: dict = {}
    for path in paths:
        per: dict = {}
        with open(path, newline="") as f:
            for r in csv.DictReader(f):
                name = r["Kernel_Name"].replace("void ", "", 1)
                name = re.sub(r"\(anonymous namespace\)::", "", name.replace("mi355x::", ""))
                name = re.sub(r"\(.*", "", name)
                if match not in name:
                    continue
                key = (name[:70], int(r.get("Grid_Size", 0) or 0))
                per.setdefault((r["Dispatch_Id"], key), {})[r["Counter_Name"]] = float(
                    r["Counter_Value"])
        for (_, key), counters in per.items():
            for c, v in counters.items():
                acc.setdefault(key, {}).setdefault(c, []).append(v)
    lines = []
    for (name, grid), counters in sorted(acc.items()):
        n = max(len(v) for v in counters.values())
        lines.append(f"{name}  grid {grid}  dispatches {n}")
        for c in sorted(counters):
            v = counters[c]
            lines.append(f"    {c:36s} {sum(v) / len(v):18.1f}")
    return "\n".join(lines)


def summarize_gaps(path: str, idle_s: float = 0.2) -> str:
    """Idle time between consecutive kernels in a rocprofv3 kernel_trace.csv, per stretch of
    activity (stretches are split at host pauses longer than `idle_s`). Run on a trace of
    `--only e2e`, the two long stretches are the serving run with graph-replayed decode and
    the one with eager decode. Host-side text processing only (no GPU)."""
    import csv

    spans, names = [], {}
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            name = r["Kernel_Name"].replace("(anonymous namespace)::", "").split("(")[0]
            spans.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]),
                          "decode_mma_kernel" in r["Kernel_Name"],
                          names.setdefault(name[:48], len(names))))
    spans.sort()
    label = {v: k for k, v in names.items()}
    stretches, cur = [], []
    for sp in spans:
        if cur and sp[0] - max(x[1] for x in cur[-64:]) > idle_s * 1e9:
            stretches.append(cur)
            cur = []
        cur.append(sp)
    if cur:
        stretches.append(cur)
    lines = [f"{'stretch':>7s} {'kernels':>8s} {'decode_attn':>11s} {'span_s':>8s} {'busy_s':>8s} "
             f"{'idle_%':>7s} {'gap_median_us':>13s} {'gap_mean_us':>11s}"]
    by_prev = []
    for i, st in enumerate(stretches):
        if len(st) < 1000:
            continue
        gaps, end, last = [], st[0][1], st[0][3]
        busy = 0
        after = {}  # idle time by the kernel whose end it follows
        for b, e, _, k in st:
            busy += e - b
            gap = (b - end) / 1e3 if b > end else 0.0
            gaps.append(gap)
            if gap > 0:
                t = after.setdefault(last, [0.0, 0])
                t[0] += gap
                t[1] += 1
            if e >= end:
                end, last = e, k
        gaps = sorted(gaps[1:])
        span = (end - st[0][0]) / 1e9
        lines.append(f"{i:7d} {len(st):8d} {sum(1 for x in st if x[2]):11d} {span:8.3f} "
                     f"{busy / 1e9:8.3f} {100 * (1 - busy / 1e9 / span):7.2f} "
                     f"{gaps[len(gaps) // 2]:13.2f} {sum(gaps) / len(gaps):11.2f}")
        by_prev.append((i, span, after))
    for i, span, after in by_prev:
        lines.append(f"# stretch {i}: idle time by the kernel it follows (top 8)")
        lines.append(f"{'kernel':50s} {'idle_ms':>9s} {'% span':>7s} {'gaps':>7s} {'mean_us':>8s}")
        for k, (t, n) in sorted(after.items(), key=lambda kv: -kv[1][0])[:8]:
            lines.append(f"{label[k]:50s} {t / 1e3:9.2f} {100 * t / 1e6 / span:7.2f} {n:7d} "
                         f"{t / n:8.2f}")
    return "\n".join(lines)


METRIC = "decode-attn HBM GB/s (% peak); prefill MFMA util; output tok/s Qwen3-8B"


def parse_args():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=2000)
    p.add_argument("--warmup", type=int, default=500)
    p.add_argument("--seed", type=int, default=2)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-requests", type=int, default=16,
                   help="requests in the bounded CPU-baseline sample")
    p.add_argument("--decode-only", action="store_true",
                   help="skip the prefill and norm measurements")
    p.add_argument("--only", choices=["prefill", "norms", "e2e", "ceilings", "serving_ops"],
                   help="print only this section's measurements (tuning aid)")
    p.add_argument("--e2e-requests", type=int, default=256)
    p.add_argument("--e2e-input", type=int, default=1024)
    p.add_argument("--e2e-output", type=int, default=512)
    p.add_argument("--e2e-layers", type=int, default=None,
                   help="override the layer count (smoke runs only; the reported config is 36)")
    p.add_argument("--skip-e2e", action="store_true")
    p.add_argument("--summarize-kernel-trace", metavar="CSV",
                   help="print per-(kernel, grid) statistics of a rocprofv3 kernel_trace.csv "
                        "and exit (host only)")
    p.add_argument("--summarize-counters", metavar="CSV", nargs="+",
                   help="print per-(kernel, grid) means of rocprofv3 --pmc counter_collection "
                        "CSVs and exit (host only; --counter-match filters kernel names)")
    p.add_argument("--counter-match", default="", help="kernel-name filter for "
                   "--summarize-counters")
    p.add_argument("--summarize-gaps", metavar="CSV",
                   help="print the idle time between consecutive kernels of a rocprofv3 "
                        "kernel_trace.csv, per stretch of activity, and exit (host only)")
    p.add_argument("--e2e-graph-only", action="store_true",
                   help="skip the eager-decode comparison run of the e2e section")
    p.add_argument("--copy-calibration", action="store_true",
                   help="run one 256 MiB device-to-device copy first (PMC byte-count "
                        "calibration for FETCH_SIZE / WRITE_SIZE)")
    return p.parse_args()


def build_workload(seed: int, dev: torch.device):
    B, HQ, HKV, D, POOL = 64, 16, 8, 128, 1 << 22
    g = torch.Generator().manual_seed(seed)
    lengths = torch.randint(512, 4097, (B,), generator=g, dtype=torch.int32)
    perm = torch.randperm(POOL - 1, generator=g)[: int(lengths.sum())] + 1  # slot 0 reserved
    cols = 4096
    table = torch.zeros(B, cols, dtype=torch.int32)
    off = 0
    for b in range(B):
        n = int(lengths[b])
        table[b, :n] = perm[off: off + n].to(torch.int32)
        off += n
    gd = torch.Generator(device=dev).manual_seed(seed)
    # One KV pool per layer, as the model binds a separate [pages, P, Hkv, D] view per
    # layer; steps rotate over them so no launch re-reads the previous launch's rows
    # from the 256 MiB Infinity Cache.
    kcs, vcs = [], []
    for _ in range(LAYERS):
        kc = torch.randn(POOL, 1, HKV, D, generator=gd, device=dev, dtype=torch.bfloat16)
        vc = torch.randn(POOL, 1, HKV, D, generator=gd, device=dev, dtype=torch.bfloat16)
        kc[0].zero_()
        vc[0].zero_()
        kcs.append(kc)
        vcs.append(vc)
    kc, vc = kcs[0], vcs[0]
    q = torch.randn(B, HQ, D, generator=gd, device=dev, dtype=torch.bfloat16)
    knew = torch.randn(B, HKV, D, generator=gd, device=dev, dtype=torch.bfloat16)
    vnew = torch.randn(B, HKV, D, generator=gd, device=dev, dtype=torch.bfloat16)
    loc = torch.tensor([int(table[b, int(lengths[b]) - 1]) for b in range(B)],
                       dtype=torch.int64, device=dev)
    return dict(B=B, HQ=HQ, HKV=HKV, D=D, POOL=POOL, lengths=lengths, table=table, kc=kc, vc=vc,
                kcs=kcs, vcs=vcs, q=q, knew=knew, vnew=vnew, loc=loc)


def decode_bytes(lengths, hq, hkv, d) -> int:
    total = int(lengths.sum())
    b = lengths.numel()
    return total * hkv * d * 2 * 2 + total * 4 + b * hq * d * 2 * 2


def store_bytes(b, hkv, d) -> int:
    return b * (hkv * d * 2 * 2 + hkv * d * 2 * 2) + b * 8


def cpu_baseline(w, requests: int):
    """Oracle's torch-CPU fp32 restatement of the reference decode path on a sample."""
    from oracle import attention as oatt

    threads = set_host_threads()
    idx = list(range(requests))
    lens = [int(w["lengths"][i]) for i in idx]
    # Compact CPU pool holding only the sampled requests' slots (same gather pattern).
    slots = torch.cat([w["table"][i, :lens[i]].long() for i in idx])
    kc = w["kc"].view(w["POOL"], -1)[slots.to(w["kc"].device)].float().cpu()
    vc = w["vc"].view(w["POOL"], -1)[slots.to(w["vc"].device)].float().cpu()
    kc = kc.view(-1, 1, w["HKV"], w["D"])
    vc = vc.view(-1, 1, w["HKV"], w["D"])
    table = torch.zeros(len(idx), max(lens), dtype=torch.int32)
    off = 0
    for r, n in enumerate(lens):
        table[r, :n] = torch.arange(off, off + n, dtype=torch.int32)
        off += n
    q = w["q"][idx].float().cpu()
    oatt.decode_with_cache_torch(q, kc, vc, table, lens, 1)  # warm-up
    times = []
    for _ in range(5):
        t0 = time.perf_counter()
        oatt.decode_with_cache_torch(q, kc, vc, table, lens, 1)
        times.append(time.perf_counter() - t0)
    sec = statistics.median(times)
    nbytes = decode_bytes(torch.tensor(lens), w["HQ"], w["HKV"], w["D"])
    return {"value": nbytes / sec / 1e9, "unit": "GB/s", "cores": threads, "kind": "port",
            "host": host_cpu(threads),
            "sample": f"{len(idx)} of 64 requests ({sum(lens)} KV tokens), libtorch fp32 CPU "
                      "decode_with_cache restatement, median of 5"}


def _event_time_ms(fn, reps: int) -> float:
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    fn()
    torch.cuda.synchronize()
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def _graph_time_us(fn, launches: int = 100, replays: int = 20) -> float:
    """Per-launch device time of ``fn`` with the host out of the loop: ``launches`` calls
    are captured in one hipGraph and the graph is replayed ``replays`` times between HIP
    events, so the figure is kernel time plus the graph's inter-node gaps, not the rate
    at which Python issues launches."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # warm-up on the capture stream (allocator, lazy init)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(launches):
            fn()
    g.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(replays):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    del g
    return e0.elapsed_time(e1) * 1e3 / (replays * launches)


def replan_section(dev) -> dict:
    """Steady-state decode re-planning (the per-step host work of a served decode batch):
    an existing plan re-made from host lengths (no device read-back), median host time per
    call, at cfg2 (64 rows, page 1) and at the 256-row Qwen3-8B bucket (page 16,
    ~1,000-1,600-token contexts). The first, cold call is reported separately."""
    from llm_infer_rust_amd.backend import (AttentionMetadata, AttentionSpec, BatchPhase,
                                            DecodeHostMetadata, prepare_decode_plan)

    out = {}
    for name, rows, page, lo, hi, hq in (("cfg2_64x_page1", 64, 1, 512, 4096, 16),
                                         ("cfg5_256x_page16", 256, 16, 1024, 1536, 32)):
        g = torch.Generator().manual_seed(rows)
        lens = torch.randint(lo, hi + 1, (rows,), generator=g, dtype=torch.int32)
        cols = (hi + page - 1) // page
        table = torch.randint(1, 1 << 20, (rows, cols), generator=g, dtype=torch.int32)
        spec = AttentionSpec(hq, 8, 128, torch.bfloat16, dev)
        table_d, lens_d = table.to(dev), lens.to(dev)
        host = lens.tolist()

        def meta():
            return AttentionMetadata(BatchPhase.DECODE, block_table=table_d, cache_seqlens=lens_d,
                                     decode_host=DecodeHostMetadata(host))

        torch.cuda.synchronize()
        t0 = time.perf_counter()
        plan = prepare_decode_plan(None, meta(), spec, page, graph=False)
        torch.cuda.synchronize()
        cold = (time.perf_counter() - t0) * 1e3
        times = []
        for i in range(60):
            m = meta()
            t0 = time.perf_counter()
            prepare_decode_plan(plan, m, spec, page, graph=False)
            times.append((time.perf_counter() - t0) * 1e3)
        torch.cuda.synchronize()
        out[name] = {"warm_ms": round(statistics.median(times[10:]), 4),
                     "cold_ms": round(cold, 3), "rows": rows, "page_size": page}
        del plan
    return out


def _cpu_median_ms(fn, runs: int = 3) -> tuple[float, int]:
    """Median wall time of ``fn`` on the host cores (one warm-up run), and the threads used."""
    threads = set_host_threads()
    fn()
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        times.append((time.perf_counter() - t0) * 1e3)
    return sorted(times)[len(times) // 2], threads


def prefill_sections(dev, reps: int, cpu: bool = True) -> dict:
    """cfg3 ragged causal prefill and cfg4 paged prefill over a cached prefix (bf16 MFMA),
    each with the oracle's torch-CPU fp32 restatement timed on a sample (reported baseline)."""
    from llm_infer_rust_amd.backend import (AttentionMetadata, AttentionSpec, BatchPhase,
                                            PrefillMetadata)
    from llm_infer_rust_amd.prefill import prepare_prefill_plan, run_prefill

    out = {}
    # cfg3: 8 sequences, L ~ U[256, 2048], Hq16/Hkv8, packed QKV stride 4096.
    g = torch.Generator().manual_seed(3)
    lens = torch.randint(256, 2049, (8,), generator=g)
    bounds = [0] + torch.cumsum(lens, 0).tolist()
    n = bounds[-1]
    gd = torch.Generator(device=dev).manual_seed(3)
    packed = torch.randn(n, 4096, generator=gd, device=dev, dtype=torch.bfloat16)
    q = packed[:, :2048].view(-1, 16, 128)
    k = packed[:, 2048:3072].view(-1, 8, 128)
    v = packed[:, 3072:].view(-1, 8, 128)
    meta = AttentionMetadata(BatchPhase.PREFILL,
                             cu_seqlens_q=torch.tensor(bounds, dtype=torch.int32, device=dev),
                             prefix_lens=torch.zeros(8, dtype=torch.int32, device=dev),
                             block_table=torch.zeros(8, 128, dtype=torch.int32, device=dev))
    spec = AttentionSpec(16, 8, 128, torch.bfloat16, dev)
    plan = prepare_prefill_plan(None, meta, PrefillMetadata(bounds, [0] * 8), spec, 16)
    o = torch.empty_like(q)
    for _ in range(PREFILL_WARMUP):
        run_prefill(plan, q, k, v, o)
    ms = _event_time_ms(lambda: run_prefill(plan, q, k, v, o), reps)
    flops = 4 * 16 * 128 * sum(int(x) * (int(x) + 1) // 2 for x in lens)
    tf = flops / (ms * 1e-3) / 1e12
    out["prefill_ragged_cfg3"] = {"us": round(ms * 1e3, 2), "flops": flops,
                                  "TFLOP/s": round(tf, 2),
                                  "mfma_frac": round(tf / BF16_PEAK_TFLOPS, 4),
                                  "tokens": n}
    if cpu:
        from oracle import attention as oatt  # the CPU baseline only

        sb = bounds[:3]  # the first two sequences
        qs, ks, vs = (t[: sb[-1]].float().cpu() for t in (q, k, v))
        cms, threads = _cpu_median_ms(lambda: oatt.prefill_ragged_torch(qs, ks, vs, sb))
        sflops = 4 * 16 * 128 * sum(int(x) * (int(x) + 1) // 2 for x in lens[:2])
        out["prefill_ragged_cfg3"]["cpu_baseline"] = {
            "value": round(sflops / (cms * 1e-3) / 1e9, 2), "unit": "GFLOP/s", "cores": threads, "host": host_cpu(threads),
            "kind": "port", "sample": f"first 2 of 8 sequences ({sb[-1]} tokens), torch-CPU fp32 "
                                      "SDPA prefill restatement, median of 3"}
    del plan
    # cfg4: 16 requests, prefix ~ U[1024, 8192], extend ~ U[64, 512], Hq32/Hkv8, page 16.
    g = torch.Generator().manual_seed(4)
    page = 16
    pref = torch.randint(1024, 8193, (16,), generator=g)
    ext = torch.randint(64, 513, (16,), generator=g)
    pages_per = (pref + ext + page - 1) // page
    cols = int(pages_per.max())
    pool = int(pages_per.sum()) + 1
    perm = torch.randperm(pool - 1, generator=g) + 1
    table = torch.zeros(16, cols, dtype=torch.int32)
    off = 0
    for r in range(16):
        m = int(pages_per[r])
        table[r, :m] = perm[off: off + m].to(torch.int32)
        off += m
    kc = torch.randn(pool, page, 8, 128, generator=gd, device=dev, dtype=torch.bfloat16)
    vc = torch.randn(pool, page, 8, 128, generator=gd, device=dev, dtype=torch.bfloat16)
    bounds = [0] + torch.cumsum(ext, 0).tolist()
    n = bounds[-1]
    q = torch.randn(n, 32, 128, generator=gd, device=dev, dtype=torch.bfloat16)
    meta = AttentionMetadata(BatchPhase.PREFILL,
                             cu_seqlens_q=torch.tensor(bounds, dtype=torch.int32, device=dev),
                             prefix_lens=pref.to(torch.int32).to(dev),
                             block_table=table.to(dev))
    spec = AttentionSpec(32, 8, 128, torch.bfloat16, dev)
    plan = prepare_prefill_plan(None, meta, PrefillMetadata(bounds, pref.tolist()), spec, page)
    o = torch.empty_like(q)
    for _ in range(PREFILL_WARMUP):
        run_prefill(plan, q, kc, vc, o)
    ms = _event_time_ms(lambda: run_prefill(plan, q, kc, vc, o), reps)
    flops = 4 * 32 * 128 * sum(int(e) * int(p) + int(e) * (int(e) + 1) // 2
                               for e, p in zip(ext, pref))
    tf = flops / (ms * 1e-3) / 1e12
    out["prefill_paged_cfg4"] = {"us": round(ms * 1e3, 2), "flops": flops,
                                 "TFLOP/s": round(tf, 2),
                                 "mfma_frac": round(tf / BF16_PEAK_TFLOPS, 4),
                                 "extend_tokens": n, "prefix_tokens": int(pref.sum())}
    if cpu:
        from oracle import attention as oatt  # the CPU baseline only

        # Two requests: their pages gathered into a compact CPU cache (page ids renumbered).
        rows = [0, 1]
        used = torch.cat([table[r, : int(pages_per[r])].long() for r in rows])
        kcs = kc[used.to(dev)].float().cpu()
        vcs = vc[used.to(dev)].float().cpu()
        ctable = torch.zeros(len(rows), int(pages_per[rows].max()), dtype=torch.int64)
        off = 0
        for i, r in enumerate(rows):
            m = int(pages_per[r])
            ctable[i, :m] = torch.arange(off, off + m)
            off += m
        sb = [0] + torch.cumsum(ext[rows], 0).tolist()
        qs = q[: sb[-1]].float().cpu()
        cms, threads = _cpu_median_ms(lambda: oatt.prefill_with_cache_torch(
            qs, kcs, vcs, ctable, sb, pref[rows].tolist(), page))
        sflops = 4 * 32 * 128 * sum(int(ext[r]) * int(pref[r]) +
                                    int(ext[r]) * (int(ext[r]) + 1) // 2 for r in rows)
        out["prefill_paged_cfg4"]["cpu_baseline"] = {
            "value": round(sflops / (cms * 1e-3) / 1e9, 2), "unit": "GFLOP/s", "cores": threads, "host": host_cpu(threads),
            "kind": "port", "sample": f"2 of 16 requests ({sb[-1]} extend tokens over "
                                      f"{int(pref[rows].sum())} cached), torch-CPU fp32 "
                                      "restatement, median of 3"}
    del plan
    # A chunked-prefill continuation, which the configs above do not cover: one request with
    # an 8,192-token cached prefix and 64 new tokens (Hq32/Hkv8, page 16, random pages). Only
    # 8 items for 256 CUs, so the plan splits them along their keys and merges the chunks.
    page, prefix, extend = 16, 8192, 64
    n_pages = (prefix + extend + page - 1) // page
    perm = (torch.randperm(n_pages, generator=g) + 1).to(torch.int32)
    kc = torch.randn(n_pages + 1, page, 8, 128, generator=gd, device=dev, dtype=torch.bfloat16)
    vc = torch.randn(n_pages + 1, page, 8, 128, generator=gd, device=dev, dtype=torch.bfloat16)
    q = torch.randn(extend, 32, 128, generator=gd, device=dev, dtype=torch.bfloat16)
    meta = AttentionMetadata(BatchPhase.PREFILL,
                             cu_seqlens_q=torch.tensor([0, extend], dtype=torch.int32, device=dev),
                             prefix_lens=torch.tensor([prefix], dtype=torch.int32, device=dev),
                             block_table=perm.view(1, -1).to(dev))
    plan = prepare_prefill_plan(None, meta, PrefillMetadata([0, extend], [prefix]), spec, page)
    o = torch.empty_like(q)
    for _ in range(PREFILL_WARMUP):
        run_prefill(plan, q, kc, vc, o)
    ms = _event_time_ms(lambda: run_prefill(plan, q, kc, vc, o), reps)
    flops = 4 * 32 * 128 * (extend * prefix + extend * (extend + 1) // 2)
    info = plan.info()
    out["prefill_paged_long_prefix"] = {
        "us": round(ms * 1e3, 2), "flops": flops, "TFLOP/s": round(flops / (ms * 1e-3) / 1e12, 2),
        "work_items": info["num_items"], "split_items": info["split_items"],
        "shape": f"1 request, prefix {prefix}, extend {extend}, Hq32/Hkv8, page {page}"}
    return out


def ceilings_section(dev, w, reps: int) -> dict:
    """Measured ceilings of this GPU for the two bounds (ceilings/ceilings.hip):
    the cfg2 decode memory pattern without arithmetic (random 2 KiB K and V rows at the same
    slots, rotating over the same 4 pools), a contiguous read of the same byte count, bf16 MFMA
    on random operands, and the prefill kernel's per-tile work on LDS-resident random tiles."""
    import ctypes
    from llm_infer_rust_amd import _native  # noqa: F401  (HIP runtime loaded by torch first)
    lib = ctypes.CDLL(os.path.join(os.path.dirname(os.path.abspath(__file__)),
                                   "ceilings", "libmi355x_calib.so"))
    for name in ("mi355x_calib_gather", "mi355x_calib_stream", "mi355x_calib_mfma",
                 "mi355x_calib_attention_core"):
        getattr(lib, name).restype = ctypes.c_char_p
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    lens = w["lengths"].tolist()
    slots = torch.cat([w["table"][b, :n] for b, n in enumerate(lens)]).to(torch.int32).to(dev)
    rows = int(slots.numel())
    nbytes = rows * 2 * w["HKV"] * w["D"] * 2

    def check(err):
        if err:
            raise RuntimeError(err.decode())

    def gather(i):
        check(lib.mi355x_calib_gather(ctypes.c_void_p(w["kcs"][i % LAYERS].data_ptr()),
                                      ctypes.c_void_p(w["vcs"][i % LAYERS].data_ptr()),
                                      ctypes.c_void_p(slots.data_ptr()), rows,
                                      ctypes.c_void_p(sink.data_ptr()), stream))

    def stream_read(i):
        check(lib.mi355x_calib_stream(ctypes.c_void_p(w["kcs"][i % LAYERS].data_ptr()), nbytes,
                                      ctypes.c_void_p(sink.data_ptr()), stream))

    def timed(fn, n):
        fn(0)
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(n):
            fn(i)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n

    out = {}
    ms = timed(gather, reps)
    out["gather_2k_rows"] = {"us": round(ms * 1e3, 2), "bytes": nbytes,
                             "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1)}
    # In-flight sweep of the same gather (rows per wave x workgroups), at the decode's
    # random slots and at the same slots sorted (row-buffer locality, same bytes).
    lib.mi355x_calib_gather_depth.restype = ctypes.c_char_p
    sorted_slots = torch.sort(slots).values
    sweep = {}
    for label, sl in (("random", slots), ("sorted", sorted_slots)):
        for depth, blocks in ((1, 1024), (2, 1024), (4, 1024), (8, 1024), (8, 256), (2, 4096)):
            def g(i, sl=sl, depth=depth, blocks=blocks):
                check(lib.mi355x_calib_gather_depth(
                    ctypes.c_void_p(w["kcs"][i % LAYERS].data_ptr()),
                    ctypes.c_void_p(w["vcs"][i % LAYERS].data_ptr()),
                    ctypes.c_void_p(sl.data_ptr()), rows, depth, blocks,
                    ctypes.c_void_p(sink.data_ptr()), stream))
            ms = timed(g, reps)
            sweep[f"{label}_d{depth}_wg{blocks}"] = round(nbytes / (ms * 1e-3) / 1e9, 1)
    out["gather_sweep_GB/s"] = sweep
    # Per-CU rate of direct global -> LDS copies (8 waves x 8 KiB in flight per workgroup),
    # all from HBM and half from L2, at the QKV projection's 192 workgroups and at 256.
    lib.mi355x_calib_load_rate.restype = ctypes.c_char_p
    lib.mi355x_calib_load_rate.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32,
                                           ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p]
    span = 6 << 30  # inside one 8 GiB pool: a multiple of 192 and 256 x 8 MiB
    load = {}
    for blocks in (192, 256):
        iters = span // (blocks * 8 * 1024 * 8) // 2  # each wave walks half its region
        for mix in (0, 1):
            ms = timed(lambda i, b=blocks, m=mix, it=iters: check(lib.mi355x_calib_load_rate(
                ctypes.c_void_p(w["kcs"][i % LAYERS].data_ptr()), span, it, m, b, stream)), reps)
            moved = blocks * 8 * iters * 8 * 1024
            load[f"{'mixed_l2_hbm' if mix else 'hbm'}_wg{blocks}"] = round(
                moved / (ms * 1e-3) / 1e9 / blocks, 1)
    out["load_rate_GB/s_per_CU"] = load
    ms = timed(stream_read, reps)
    out["stream_read"] = {"us": round(ms * 1e3, 2), "bytes": nbytes,
                          "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1)}
    blocks, iters = 4096, 1024
    ms = timed(lambda i: check(lib.mi355x_calib_mfma(blocks, iters,
                                                     ctypes.c_void_p(sink.data_ptr()), stream)), 5)
    flops = blocks * 8 * iters * 4 * 32768
    out["mfma_bf16_random"] = {"TFLOP/s": round(flops / (ms * 1e-3) / 1e12, 1)}
    blocks, iters = 1024, 400
    ms = timed(lambda i: check(lib.mi355x_calib_attention_core(
        blocks, iters, ctypes.c_void_p(sink.data_ptr()), stream)), 5)
    flops = blocks * 8 * iters * 32 * 32768
    out["attention_core_random"] = {"TFLOP/s": round(flops / (ms * 1e-3) / 1e12, 1)}
    # The same work as 8 waves x 32 queries and as 4 waves x 64 queries (half the LDS
    # reads), each workgroup's shader cycles read back: cycles per tile, and the clock the
    # chip held (one workgroup per CU at a time, blocks / CUs of them per CU in sequence).
    lib.mi355x_calib_attention_core_cycles.restype = ctypes.c_char_p
    cycles = torch.zeros(blocks, dtype=torch.int64, device=dev)
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    per_cu = blocks / cus
    core = {}
    for variant, name in ((0, "waves8_q32"), (1, "waves4_q64")):
        ms = timed(lambda i, v=variant: check(lib.mi355x_calib_attention_core_cycles(
            blocks, iters, v, ctypes.c_void_p(cycles.data_ptr()), ctypes.c_void_p(sink.data_ptr()),
            stream)), 5)
        mean = float(cycles.double().mean())
        core[name] = {"TFLOP/s": round(blocks * iters * 2 ** 23 / (ms * 1e-3) / 1e12, 1),
                      "cycles_per_tile": round(mean / iters),
                      "GHz": round(mean * per_cu / (ms * 1e6), 3),
                      "ns_per_tile": round(ms * 1e6 / (per_cu * iters), 1)}
    out["attention_core_cycles"] = core
    return out


def _cpu_single_ms(fn, runs: int = 3) -> float:
    """Median wall time of a single-threaded (numpy) host routine after one warm-up run."""
    fn()
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        times.append((time.perf_counter() - t0) * 1e3)
    return sorted(times)[len(times) // 2]


def serving_ops_section(dev, reps: int, cpu: bool = True) -> dict:
    """The config-5 kernels around the attention path at its shapes, each timed over `reps`
    launches with HIP events, with the bytes (or FLOPs) it moves and a reported CPU baseline:
    joint top-k / top-p sampling of 256 rows x 151,936 (sampling.rs:239-321),
    the fused QK-norm -> RoPE -> K/V store pass of a 256-row decode step and of an 8192-token
    prompt batch, SiLU x mul of the prompt batch, and the four decode-batch projections at 256
    rows (row f3; fused_ops.cu:108-171,340-372, linear.rs), plus the decode layer's fused QKV
    projection + QK-norm/RoPE/store route. Kernel figures are device time from a replayed
    hipGraph of captured calls (``eager_us``: the eager per-call rate beside them); the
    projections rotate over three weight sets (~1.16 GB) so the weights stream from HBM, as in
    serving."""
    import numpy as np
    from llm_infer_rust_amd import ops
    from llm_infer_rust_amd.kv_cache import BaseAttention
    from llm_infer_rust_amd.sampling import Sampler, SamplingParams

    gd = torch.Generator(device=dev).manual_seed(9)

    def rnd(*shape, scale=1.0):
        return (torch.randn(*shape, generator=gd, device=dev) * scale).to(torch.bfloat16)

    out = {}
    # Sampling (T 0.7, top-k 50, top-p 0.9, as config 5).
    rows, vocab = 256, 151936
    logits = rnd(rows, vocab, scale=2.0)
    sampler = Sampler(2)
    params = [SamplingParams(temperature=0.7, top_k=50, top_p=0.9)] * rows
    ids = torch.empty(rows, dtype=torch.int64, device=dev)
    ms = _event_time_ms(lambda: sampler.sample_batch_device(logits, params, out=ids), reps)
    nbytes = rows * vocab * 2
    res = {"us": round(ms * 1e3, 2), "rows/s": round(rows / (ms * 1e-3), 1), "bytes": nbytes,
           "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1),
           "note": "eager calls through Sampler (host parameter handling included); bytes are "
                   "one pass over the logits; the kernel makes two for top-k rows, up to five "
                   "otherwise (the row stays in L2)"}
    if cpu:
        from oracle import sampling as osamp  # the CPU baseline only
        sample = logits[:8].float().cpu().numpy()
        t8, k8, p8 = np.full(8, 0.7, np.float32), np.full(8, 50), np.full(8, 0.9, np.float32)
        cms = _cpu_single_ms(lambda: osamp.sample_rows(sample, t8, k8, p8, 2, 0))
        res["cpu_baseline"] = {
            "value": round(8 / (cms * 1e-3), 2), "unit": "rows/s", "cores": 1, "kind": "port",
            "sample": "8 of the 256 rows, numpy restatement of the joint top-k/top-p rule with "
                      "the same Philox/Gumbel draw, median of 3"}
    out["sample_256x151936"] = res
    del logits

    # Fused QK-norm -> RoPE -> K/V store (Qwen3-8B heads: 32 q, 8 kv, head_dim 128).
    rope = ops.HalfSplitRope(40960, 128, 1_000_000.0, dev)
    pages = 8192
    kc = torch.zeros(pages, 16, 8, 128, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    att = BaseAttention()
    att.set_reserved_write_slot(0)
    att.bind_kv_cache(kc, vc)
    qw = (torch.rand(128, generator=gd, device=dev) + 0.5).to(torch.bfloat16)
    kw = (torch.rand(128, generator=gd, device=dev) + 0.5).to(torch.bfloat16)
    for name, t in (("head_rows_decode_256", 256), ("head_rows_prefill_8192", 8192)):
        qkv = rnd(t, 48 * 128)
        q = qkv[:, :4096].view(t, 32, 128)
        k = qkv[:, 4096:5120].view(t, 8, 128)
        v = qkv[:, 5120:].view(t, 8, 128)
        positions = torch.randint(0, 2048, (t,), generator=gd, device=dev)
        loc = torch.randperm(pages * 16 - 1, generator=gd, device=dev)[:t] + 1
        call = (lambda q=q, k=k, v=v, positions=positions, loc=loc: ops.qk_norm_rope_store(
            q, k, v, qw, kw, 1e-6, positions, rope, att, loc))
        eager_ms = _event_time_ms(call, reps)
        us = _graph_time_us(call)
        nbytes = t * 128 * 2 * (32 * 2 + 8 * 2 + 8 + 16) + 16 * t
        res = {"us": round(us, 2), "bytes": nbytes, "GB/s": round(nbytes / (us * 1e-6) / 1e9, 1),
               "hbm_frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
               "eager_us": round(eager_ms * 1e3, 2)}
        if cpu:
            from oracle import layer_ops as olo, norms as onorms  # the CPU baseline only
            n = min(t, 1024)
            qs, ks = q[:n].float().cpu(), k[:n].float().cpu()
            qwc, kwc = qw.float().cpu(), kw.float().cpu()
            cos, sin = olo.rope_tables(40960, 128, 1_000_000.0)
            pos = positions[:n].cpu().numpy()
            kcc = torch.zeros(n + 1, 8, 128)
            lc = torch.arange(1, n + 1)
            vs = v[:n].float().cpu()

            def cpu_pass():
                qn, kn = onorms.qk_norm_torch(qs, ks, qwc, kwc, 1e-6)
                olo.rope(qn.numpy(), pos, cos, sin)
                kr = torch.from_numpy(olo.rope(kn.numpy(), pos, cos, sin))
                kcc.index_copy_(0, lc, kr)
                kcc.index_copy_(0, lc, vs)
            cms, threads = _cpu_median_ms(cpu_pass)
            cbytes = n * 128 * 2 * (32 * 2 + 8 * 2 + 8 + 16) + 16 * n
            res["cpu_baseline"] = {
                "value": round(cbytes / (cms * 1e-3) / 1e9, 2), "unit": "GB/s", "cores": threads, "host": host_cpu(threads),
                "kind": "port", "sample": f"{n} of the {t} tokens, torch-CPU / numpy restatement "
                                          "(ops.rs:39-51, 84-97, base.rs:123-151), median of 3"}
        out[name] = res
    del kc, vc

    # SiLU x mul of the prompt batch: gate_up [8192, 2 x 12288].
    gu = rnd(8192, 2 * 12288)
    act = torch.empty(8192, 12288, dtype=torch.bfloat16, device=dev)
    eager_ms = _event_time_ms(lambda: ops.silu_and_mul(gu, out=act), reps)
    us = _graph_time_us(lambda: ops.silu_and_mul(gu, out=act))
    nbytes = 3 * 8192 * 12288 * 2
    res = {"us": round(us, 2), "bytes": nbytes, "GB/s": round(nbytes / (us * 1e-6) / 1e9, 1),
           "hbm_frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
           "eager_us": round(eager_ms * 1e3, 2)}
    if cpu:
        from oracle import layer_ops as olo  # the CPU baseline only
        sample = gu[:256].float().cpu().numpy()
        cms = _cpu_single_ms(lambda: olo.silu_mul(sample))
        res["cpu_baseline"] = {"value": round(3 * 256 * 12288 * 2 / (cms * 1e-3) / 1e9, 2),
                               "unit": "GB/s", "cores": 1, "kind": "port",
                               "sample": "256 of the 8192 rows, numpy restatement (ops.rs:53-61), "
                                         "median of 3"}
    out["silu_mul_8192x12288"] = res
    del gu, act

    # Decode-batch projections at 256 rows (Qwen3-8B): QKV, o_proj, gate_up + SiLU, down.
    x = rnd(256, 12288, scale=0.5)
    shapes = (("qkv", 6144, 4096), ("o_proj", 4096, 4096), ("gate_up_silu", 24576, 4096),
              ("down", 4096, 12288))
    n_sets = 3  # 3 x 386 MB of weights: more than the 256 MB MALL, so they stream from HBM
    sets = [{nm: rnd(n, kk, scale=0.02) for nm, n, kk in shapes} for _ in range(n_sets)]
    kc = torch.zeros(2048, 16, 8, 128, dtype=torch.bfloat16, device=dev)
    att = BaseAttention()
    att.set_reserved_write_slot(0)
    att.bind_kv_cache(kc, torch.zeros_like(kc))
    positions = torch.randint(0, 2048, (256,), generator=gd, device=dev)
    loc = torch.randperm(2048 * 16 - 1, generator=gd, device=dev)[:256] + 1
    for nm, n, kk in shapes + (("qkv_norm_rope_store", 6144, 4096),):
        xs = x[:, :kk]
        if nm == "gate_up_silu":
            o = torch.empty(256, n // 2, dtype=torch.bfloat16, device=dev)
            fn = lambda i, xs=xs, o=o, nm=nm: ops.decode_linear_silu_mul(
                xs, sets[i % n_sets][nm], out=o)
        elif nm == "qkv_norm_rope_store":  # the decode layer's fused QKV route
            fn = lambda i, xs=xs: ops.linear_qk_norm_rope_store(
                xs, sets[i % n_sets]["qkv"], 32, 8, qw, kw, 1e-6, positions, rope, att, loc)
        else:
            o = torch.empty(256, n, dtype=torch.bfloat16, device=dev)
            fn = lambda i, xs=xs, o=o, nm=nm: ops.decode_linear(xs, sets[i % n_sets][nm], out=o)
        state = {"i": 0}

        def step(fn=fn, state=state):
            fn(state["i"])
            state["i"] += 1
        eager_ms = _event_time_ms(step, reps)
        us = _graph_time_us(step, launches=3 * n_sets * 10)  # the captured calls rotate the sets
        wbytes = n * kk * 2
        flops = 2 * 256 * n * kk
        res = {"us": round(us, 2), "weight_bytes": wbytes,
               "TB/s": round(wbytes / (us * 1e-6) / 1e12, 3),
               "TFLOP/s": round(flops / (us * 1e-6) / 1e12, 1), "eager_us": round(eager_ms * 1e3, 2)}
        if cpu:
            xc = xs[:16].float().cpu()
            wc = sets[0]["qkv" if nm == "qkv_norm_rope_store" else nm].float().cpu()
            cms, threads = _cpu_median_ms(lambda: xc @ wc.T)
            res["cpu_baseline"] = {"value": round(2 * 16 * n * kk / (cms * 1e-3) / 1e9, 2),
                                   "unit": "GFLOP/s", "cores": threads, "host": host_cpu(threads), "kind": "port",
                                   "sample": "16 of the 256 rows, torch-CPU fp32 x @ w^T "
                                             "(linear.rs:5-7), median of 3"}
        out[f"linear_256_{nm}"] = res
    del sets, x, kc, att
    torch.cuda.empty_cache()
    return out


def norm_sections(dev, reps: int, cpu: bool = True) -> dict:
    """cfg3 norms on 8192 x 1024 hidden rows and the 8192-token packed QKV (HBM-bound), each
    with the oracle's torch-CPU restatement timed on the full rows (reported baseline)."""
    from llm_infer_rust_amd import ops

    gd = torch.Generator(device=dev).manual_seed(33)
    # Rotate over buffer sets (> 1 GiB in total) so reads come from HBM, not from the
    # 256 MiB Infinity Cache left warm by the previous call.
    sets = 24
    xs = [torch.randn(8192, 1024, generator=gd, device=dev, dtype=torch.bfloat16)
          for _ in range(sets)]
    rs = [torch.randn(8192, 1024, generator=gd, device=dev, dtype=torch.bfloat16)
          for _ in range(sets)]
    outs = [torch.empty(8192, 1024, device=dev, dtype=torch.bfloat16) for _ in range(sets)]
    w = torch.rand(1024, generator=gd, device=dev).add_(0.5).to(torch.bfloat16)
    packs = [torch.randn(8192, 4096, generator=gd, device=dev, dtype=torch.bfloat16)
             for _ in range(8)]
    qw = torch.rand(128, generator=gd, device=dev).add_(0.5).to(torch.bfloat16)
    kw = torch.rand(128, generator=gd, device=dev).add_(0.5).to(torch.bfloat16)
    lib, stream = ops._native.lib(), torch.cuda.current_stream().cuda_stream
    it = [0]

    def rms():
        i = it[0] = it[0] + 1
        x, o = xs[i % sets], outs[i % sets]
        ops._native.check(lib.mi355x_rms_norm(x.data_ptr(), w.data_ptr(), o.data_ptr(), 8192,
                                              1, 1024, 1024, 0, 1e-6, 0, stream), "rms")

    def add_rms():
        i = it[0] = it[0] + 1
        ops.add_rms_norm(xs[i % sets], rs[i % sets], w, 1e-6)

    def qk():
        i = it[0] = it[0] + 1
        p = packs[i % len(packs)]
        ops.qk_norm(p[:, :2048].view(-1, 16, 128), p[:, 2048:3072].view(-1, 8, 128), qw, kw,
                    1e-6)

    # Decode-size residual norm of the Qwen3-8B e2e step: 256 rows x 4096.
    dx = [torch.randn(256, 4096, generator=gd, device=dev, dtype=torch.bfloat16)
          for _ in range(sets)]
    dr = [torch.randn(256, 4096, generator=gd, device=dev, dtype=torch.bfloat16)
          for _ in range(sets)]
    w4 = torch.rand(4096, generator=gd, device=dev).add_(0.5).to(torch.bfloat16)

    def add_rms_decode():
        i = it[0] = it[0] + 1
        ops.add_rms_norm(dx[i % sets], dr[i % sets], w4, 1e-6)

    # Reference point for these sizes: torch's device copy of the rms_norm bytes
    # (16 MiB in, 16 MiB out), same buffer rotation.
    def copy_ref():
        i = it[0] = it[0] + 1
        outs[i % sets].copy_(xs[i % sets])

    res = {}
    gx, gr = dx[0], dr[0]
    g_us = _graph_time_us(lambda: ops.add_rms_norm(gx, gr, w4, 1e-6))
    res["add_rms_norm_256x4096_graph"] = {
        "us": round(g_us, 3), "bytes": 4 * 256 * 4096 * 2,
        "GB/s": round(4 * 256 * 4096 * 2 / (g_us * 1e-6) / 1e9, 1),
        "note": "one buffer set replayed from a hipGraph (L2/MALL-resident after the first)"}
    for name, fn, nbytes in (
            ("rms_norm", rms, 2 * 8192 * 1024 * 2),
            ("add_rms_norm", add_rms, 4 * 8192 * 1024 * 2),
            ("qk_norm", qk, 2 * 8192 * 24 * 128 * 2),
            ("add_rms_norm_256x4096", add_rms_decode, 4 * 256 * 4096 * 2),
            ("torch_copy_16MiB_ref", copy_ref, 2 * 8192 * 1024 * 2)):
        ms = _event_time_ms(fn, reps)
        gbs = nbytes / (ms * 1e-3) / 1e9
        res[name] = {"us": round(ms * 1e3, 2), "bytes": nbytes, "GB/s": round(gbs, 1),
                     "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}
    if cpu:
        from oracle import norms as onorms  # the CPU baseline only

        xc, rc, wc = xs[0].cpu(), rs[0].cpu(), w.cpu()
        pc = packs[0].cpu()
        qc, kc = pc[:, :2048].reshape(-1, 16, 128), pc[:, 2048:3072].reshape(-1, 8, 128)
        qwc, kwc = qw.cpu(), kw.cpu()
        for name, fn in (("rms_norm", lambda: onorms.rms_norm_torch(xc, wc, 1e-6)),
                         ("add_rms_norm", lambda: onorms.add_rms_norm_torch(xc, rc, wc, 1e-6)),
                         ("qk_norm", lambda: onorms.qk_norm_torch(qc, kc, qwc, kwc, 1e-6))):
            cms, threads = _cpu_median_ms(fn)
            res[name]["cpu_baseline"] = {
                "value": round(res[name]["bytes"] / (cms * 1e-3) / 1e9, 2), "unit": "GB/s",
                "cores": threads, "host": host_cpu(threads), "kind": "port",
                "sample": "full rows, torch-CPU restatement of ops.rs, median of 3"}
    return res


def main():
    args = parse_args()
    if args.summarize_kernel_trace:
        print(summarize_kernel_trace(args.summarize_kernel_trace))
        return
    if args.summarize_gaps:
        print(summarize_gaps(args.summarize_gaps))
        return
    if args.summarize_counters:
        print(summarize_counters(args.summarize_counters, args.counter_match))
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only; run with --gpus 1"}))
        sys.exit(2)
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from llm_infer_rust_amd.backend import (AttentionMetadata, AttentionSpec, BatchPhase,
                                            prepare_decode_plan, run_decode)
    from llm_infer_rust_amd.kv_cache import BaseAttention

    dev = torch.device("cuda", 0)
    if args.copy_calibration:
        src = torch.empty(COPY_CAL_BYTES // 2, dtype=torch.bfloat16, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    if args.only == "e2e":
        print(json.dumps({"e2e": e2e_section(dev, args)}))
        return
    if args.only in ("prefill", "norms", "serving_ops"):
        fn = {"prefill": prefill_sections, "norms": norm_sections,
              "serving_ops": serving_ops_section}[args.only]
        print(json.dumps({args.only: fn(dev, SECTION_REPS, cpu=not args.no_cpu_baseline)}))
        return
    w = build_workload(args.seed, dev)
    if args.only == "ceilings":
        print(json.dumps({"ceilings": ceilings_section(dev, w, max(min(args.steps, 50), 5))}))
        return
    B, HQ, HKV, D = w["B"], w["HQ"], w["HKV"], w["D"]
    caches = []
    for kc, vc in zip(w["kcs"], w["vcs"]):
        c = BaseAttention()
        c.set_reserved_write_slot(0)
        c.bind_kv_cache(kc, vc)
        caches.append(c)
    spec = AttentionSpec(HQ, HKV, D, torch.bfloat16, dev)
    table_d = w["table"].to(dev)
    lens_d = w["lengths"].to(dev)
    meta = AttentionMetadata(BatchPhase.DECODE, block_table=table_d, cache_seqlens=lens_d)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    plan = prepare_decode_plan(None, meta, spec, 1, graph=False)
    torch.cuda.synchronize()
    plan_ms = (time.perf_counter() - t0) * 1e3
    info = plan.info()
    out = torch.empty_like(w["q"])

    def step(i):
        c = caches[i % LAYERS]
        c.write_kv(w["knew"], w["vnew"], w["loc"])
        run_decode(plan, w["q"], c.k_cache, c.v_cache, out)

    for i in range(DEVICE_WARMUP_STEPS + args.warmup):
        step(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(i)
    torch.cuda.synchronize()
    step_ms = (time.perf_counter() - t0) * 1e3 / args.steps

    # Decode kernels alone, HIP events on the current (launch) stream.
    reps = ROOFLINE_REPS
    for i in range(reps // 2):
        run_decode(plan, w["q"], w["kcs"][i % LAYERS], w["vcs"][i % LAYERS], out)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(reps):
        run_decode(plan, w["q"], w["kcs"][i % LAYERS], w["vcs"][i % LAYERS], out)
    e1.record()
    torch.cuda.synchronize()
    decode_ms = e0.elapsed_time(e1) / reps
    e0.record()
    for i in range(reps):
        caches[i % LAYERS].write_kv(w["knew"], w["vnew"], w["loc"])
    e1.record()
    torch.cuda.synchronize()
    store_ms = e0.elapsed_time(e1) / reps
    for c in caches:
        c.check_write_errors()

    cpu = cpu_baseline(w, args.cpu_requests) if not args.no_cpu_baseline else None
    dbytes = decode_bytes(w["lengths"], HQ, HKV, D)
    sbytes = store_bytes(B, HKV, D)
    achieved = dbytes / (decode_ms * 1e-3) / 1e9
    result = {
        "metric": METRIC,
        "value": round((dbytes + sbytes) / (step_ms * 1e-3) / 1e9, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) Q/K/V, seeded randperm page table)",
        "config": {"workload": "cfg2 paged decode + KV store: B=64, Hq16/Hkv8, D128, "
                               "L~U[512,4096], page 1, 4M-slot pool",
                   "kv_tokens": int(w["lengths"].sum()), "page_size": 1,
                   "split_kv_items": info["num_items"], "chunk_tokens": info["chunk_tokens"]},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(),
                     "kernel": "decode_dma_kernel+merge_kernel (one mi355x_decode_run)",
                     "algorithmic_bytes": dbytes, "avg_launch_us": round(decode_ms * 1e3, 3)},
        "kv_store": {"us": round(store_ms * 1e3, 3), "bytes": sbytes,
                     "GB/s": round(sbytes / (store_ms * 1e-3) / 1e9, 2)},
        "plan_prepare_ms": round(plan_ms, 3),
    }
    if cpu is not None:
        result["cpu_baseline"] = cpu
        # The K/V store on the host (base.rs:123-151: index_copy_ of the new rows into the
        # cache), the same 64 rows into a 65,536-slot CPU pool.
        kpool = torch.zeros(65536, HKV, D, dtype=torch.bfloat16)
        vpool = torch.zeros_like(kpool)
        kn, vn = w["knew"].cpu(), w["vnew"].cpu()
        cloc = torch.randperm(65535, generator=torch.Generator().manual_seed(7))[:B] + 1
        cms, threads = _cpu_median_ms(lambda: (kpool.index_copy_(0, cloc, kn),
                                               vpool.index_copy_(0, cloc, vn)), runs=21)
        result["kv_store"]["cpu_baseline"] = {
            "value": round(sbytes / (cms * 1e-3) / 1e9, 3), "unit": "GB/s", "cores": threads, "host": host_cpu(threads),
            "kind": "port", "sample": "64 rows into a 65,536-slot CPU pool, median of 21"}
    # Small kernels by graph replay (device time per launch, no Python launch overhead).
    kv_graph_us = _graph_time_us(lambda: caches[0].write_kv(w["knew"], w["vnew"], w["loc"]))
    for c in caches:
        c.check_write_errors()
    result["kv_store"]["graph_us"] = round(kv_graph_us, 3)
    result["kv_store"]["graph_GB/s"] = round(sbytes / (kv_graph_us * 1e-6) / 1e9, 2)
    result["replan"] = replan_section(dev)
    if not args.decode_only:
        result["prefill"] = prefill_sections(dev, SECTION_REPS, cpu=not args.no_cpu_baseline)
        result["norms"] = norm_sections(dev, SECTION_REPS, cpu=not args.no_cpu_baseline)
        result["serving_ops"] = serving_ops_section(dev, SECTION_REPS,
                                                    cpu=not args.no_cpu_baseline)
        ceil = ceilings_section(dev, w, min(reps, 50))
        ceil["decode_vs_gather"] = round(achieved / ceil["gather_2k_rows"]["GB/s"], 4)
        core = ceil["attention_core_random"]["TFLOP/s"]
        ceil["prefill_vs_core"] = {k: round(v["TFLOP/s"] / core, 4)
                                   for k, v in result["prefill"].items()}
        result["ceilings"] = ceil
    # The decode workload's 64 GiB of KV pools are released before the e2e model is built.
    del w, caches, plan, out, table_d, lens_d, meta, step, c
    torch.cuda.empty_cache()
    if not args.skip_e2e and not args.decode_only:
        result["e2e"] = e2e_section(dev, args)
    print(json.dumps(result))


if __name__ == "__main__":
    main()
