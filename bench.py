"""Benchmark of the Qwen3 attention hot path on one MI355X.

Headline (the metric line): paged decode attention at the Qwen3-8B shape,
batch 64, 32 q / 8 kv heads, head_dim 128, page 16, contexts U[512, 4096]
(seed 2) -- microseconds per layer and achieved HBM bandwidth against the
8 TB/s MI355X peak. A step is one decode-attention call over the batch (the
stream-K kernel plus its cut-unit merge kernel, both on the caller's stream).
Three copies of the KV pool are rotated so repeated steps cannot be served
from the 256 MB MALL. The K timed steps are bracketed by one pair of HIP
events recorded on the stream the kernels run on (and by synchronisations
for the wall clock); a second pass times each call separately for the median
and p10/p90.

Also measured (in "secondary"): the whole decode block (fused QK
norm+RoPE+store, then attention), the varlen prefill at the Qwen3-8B
16-sequence shape (TFLOP/s against 2.5 PFLOP/s bf16 dense), the fused QK
norm+RoPE+store at that shape (GB/s), the Qwen3-32B bs32 32k-context decode,
the Qwen3-4B mixed batch (prefill+store then decode), the decode block as
one fused launch, and batched sampling over 64 rows of the Qwen3 vocabulary
(three filter settings). The CPU baseline
runs the reference's CPU decode path (per-token gather loop +
repeat_interleave + SDPA, restated in the oracle) on a bounded sample of the
same batch on this host's cores.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
       python bench.py --workload NAME  (one workload alone, e.g. for a
                                         profile of its kernels)
       python bench.py --copy-probe   (a plain device copy of known size, the
                                       calibration run for HBM byte counters)
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0    # MI355X dense bf16 MFMA
METRIC = "paged decode attn µs/layer + achieved HBM TB/s (% peak), Qwen3-8B shape bs64"
HEADLINE = "qwen3-8b-decode-bs64"
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "paged_decode_traffic.json")


def time_region(fn, steps, warmup):
    """warmup untimed calls, then `steps` calls bracketed by synchronisations
    and one pair of events on the current stream. Returns (event ms per call,
    wall ms per call)."""
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for i in range(steps):
        fn(warmup + i)
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return e0.elapsed_time(e1) / steps, wall * 1e3 / steps


def time_each(fn, n, offset=0):
    """Per-call event durations (ms) of n calls."""
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(n)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(n)]
    for i in range(n):
        starts[i].record()
        fn(offset + i)
        ends[i].record()
    torch.cuda.synchronize()
    return sorted(s.elapsed_time(e) for s, e in zip(starts, ends))


def _spread(ev):
    return {"median": statistics.median(ev) * 1e3, "p10": ev[len(ev) // 10] * 1e3,
            "p90": ev[(9 * len(ev)) // 10] * 1e3}


def bench_decode(name, steps, warmup, num_workgroups=0, copies=3, with_block=False):
    from tinyserver_amd import workloads as W
    from tinyserver_amd.kernels import paged_attention_forward, paged_decode_step, qk_norm_rope_store

    dev = torch.device("cuda:0")
    w = W.make(name, device=dev)
    B = len(w.ctx_lens)
    seq_lens = w.ctx_lens.to(torch.int32).to(dev)
    pools = [(w.k_cache, w.v_cache)] + [(w.k_cache.clone(), w.v_cache.clone()) for _ in range(copies - 1)]
    cu = torch.arange(B + 1, dtype=torch.int32, device=dev)
    pos = w.positions.to(dev)
    q_rot, _ = qk_norm_rope_store(w.q, w.k, w.v, w.q_weight, w.k_weight, w.cos, w.sin, w.eps, pools[0][0],
                                  pools[0][1], w.block_tables, cu, pos, return_k=False)
    out = torch.empty_like(q_rot)

    def attn(i):
        kc, vc = pools[i % copies]
        paged_attention_forward(q_rot, kc, vc, w.block_tables, W.PAGE, seq_lens, num_workgroups=num_workgroups,
                                out=out)

    ev_ms, wall_ms = time_region(attn, steps, warmup)
    spread = _spread(time_each(attn, max(20, min(steps, 200)), warmup + steps))
    nbytes = W.decode_bytes(w.ctx_lens, w.num_heads, w.num_kv_heads)
    res = {
        "workload": name,
        "batch": B,
        "num_heads": w.num_heads,
        "num_kv_heads": w.num_kv_heads,
        "sum_ctx": int(w.ctx_lens.sum()),
        "bytes_per_call": nbytes,
        "us_per_call": ev_ms * 1e3,
        "us_per_call_median": spread["median"],
        "us_per_call_p10": spread["p10"],
        "us_per_call_p90": spread["p90"],
        "wall_ms_per_step": wall_ms,
    }
    res["achieved_gbs"] = nbytes / (res["us_per_call"] * 1e-6) / 1e9
    res["pct_peak_hbm"] = 100.0 * res["achieved_gbs"] / HBM_PEAK_GBS
    res["tokens_per_s"] = B / (res["us_per_call"] * 1e-6)
    if with_block:
        qw, kw, cos, sin = w.q_weight, w.k_weight, w.cos, w.sin

        def block(i):
            kc, vc = pools[i % copies]
            qr, _ = qk_norm_rope_store(w.q, w.k, w.v, qw, kw, cos, sin, w.eps, kc, vc, w.block_tables, cu, pos,
                                       return_k=False)
            paged_attention_forward(qr, kc, vc, w.block_tables, W.PAGE, seq_lens, num_workgroups=num_workgroups,
                                    out=out)

        res["block_us_per_call"] = time_region(block, steps, warmup)[0] * 1e3

        def block_fused(i):  # the same step as one fused call (two launches)
            kc, vc = pools[i % copies]
            paged_decode_step(w.q, w.k, w.v, qw, kw, cos, sin, w.eps, kc, vc, w.block_tables, seq_lens,
                              num_workgroups=num_workgroups, out=out)

        res["block_fused_us_per_call"] = time_region(block_fused, steps, warmup)[0] * 1e3
    return res, w


def bench_prefill(name, steps, warmup):
    from tinyserver_amd import workloads as W
    from tinyserver_amd.kernels import flash_attn_varlen_func, qk_norm_rope_store

    dev = torch.device("cuda:0")
    w = W.make(name, device=dev)
    T, hq, hkv = w.q.shape[0], w.q.shape[1], w.k.shape[1]
    D = w.q.shape[2]
    q_rot, k_rot = qk_norm_rope_store(w.q, w.k, w.v, w.q_weight, w.k_weight, w.cos, w.sin, w.eps, w.k_cache,
                                      w.v_cache, w.block_tables, w.cu_seqlens)
    out = torch.empty_like(q_rot)

    def attn(i):
        flash_attn_varlen_func(q_rot, k_rot, w.v, w.cu_seqlens, w.cu_seqlens, w.max_seqlen, w.max_seqlen, True, out=out)

    ev_ms, _ = time_region(attn, steps, warmup)
    flops = W.prefill_flops(w.seq_lens, hq)
    us = ev_ms * 1e3

    def norm_store(i):
        qk_norm_rope_store(w.q, w.k, w.v, w.q_weight, w.k_weight, w.cos, w.sin, w.eps, w.k_cache, w.v_cache,
                           w.block_tables, w.cu_seqlens)

    ns_us = time_region(norm_store, steps, warmup)[0] * 1e3
    # read q, k, v, cos, sin, weights; write rotated q and k, and K/V into the cache
    ns_bytes = 2 * T * D * (hq + 2 * hkv) + 2 * 2 * T * D + 2 * 2 * D + 2 * T * D * (hq + hkv) + 2 * 2 * T * hkv * D

    def block(i):
        qr, kr = qk_norm_rope_store(w.q, w.k, w.v, w.q_weight, w.k_weight, w.cos, w.sin, w.eps, w.k_cache,
                                    w.v_cache, w.block_tables, w.cu_seqlens)
        flash_attn_varlen_func(qr, kr, w.v, w.cu_seqlens, w.cu_seqlens, w.max_seqlen, w.max_seqlen, True, out=out)

    block_us = time_region(block, steps, warmup)[0] * 1e3
    return {
        "workload": name,
        "tokens": T,
        "gflop": flops / 1e9,
        "us_per_call": us,
        "tflops": flops / (us * 1e-6) / 1e12,
        "pct_peak_mfma": 100.0 * flops / (us * 1e-6) / 1e12 / BF16_PEAK_TFLOPS,
        "tokens_per_s": T / (us * 1e-6),
        "norm_rope_store_us": ns_us,
        "norm_rope_store_gbs": ns_bytes / (ns_us * 1e-6) / 1e9,
        "block_us_per_call": block_us,
    }


def bench_sampling(steps, warmup, batch=64, vocab=151936):
    """sample_tokens over a Qwen3-vocab batch: bf16 logits (N(0, 2.5) plus a
    few boosted tokens per row), temperature 0.8, top_k 50, top_p 0.9 (the
    engine's usual settings), seeded uniforms. One launch per call."""
    from tinyserver_amd.kernels import sample_tokens

    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(21)
    logits = torch.randn(batch, vocab, generator=g) * 2.5
    logits.scatter_add_(1, torch.randint(0, vocab, (batch, 8), generator=g), torch.rand(batch, 8, generator=g) * 12)
    logits = logits.to(dev, torch.bfloat16)
    temperature = torch.full((batch,), 0.8, device=dev)
    top_k = torch.full((batch,), 50, dtype=torch.int64, device=dev)
    top_p = torch.full((batch,), 0.9, device=dev)
    uniforms = torch.rand(batch, generator=g).to(dev)
    out = torch.empty(batch, dtype=torch.int64, device=dev)
    cases = {}
    for label, k, p in (("topk50_topp0.9", 50, 0.9), ("topp0.9", 0, 0.9), ("full", 0, 1.0)):
        top_k.fill_(k)
        top_p.fill_(p)

        def call(i):
            sample_tokens(logits, temperature, top_k, top_p, uniforms, out=out)

        us = time_region(call, steps, warmup)[0] * 1e3
        cases[label] = {"us_per_call": us, "logits_gbs": batch * vocab * 2 / (us * 1e-6) / 1e9}
    return {"workload": f"sample_tokens bs{batch} vocab{vocab} bf16", "batch": batch, "vocab": vocab, **cases}


def cpu_baseline(w, target_seconds=10.0, max_reps=50):
    """The reference's CPU decode path (gather loop + repeat_interleave + SDPA) on
    the whole batch, timed on this host: repeated for about `target_seconds` of
    CPU work, the median run reported."""
    from oracle import paged as op
    from tinyserver_amd import workloads as W

    n = len(w.ctx_lens)
    pages = sorted({p for lst in w.block_lists[:n] for p in lst})
    remap = {p: i for i, p in enumerate(pages)}
    idx = torch.tensor(pages, device=w.k_cache.device)
    kc, vc = w.k_cache[idx].cpu(), w.v_cache[idx].cpu()
    tables = [[remap[p] for p in lst] for lst in w.block_lists[:n]]
    q = w.q[:n].cpu().transpose(0, 1).unsqueeze(0).contiguous()  # (1, Hq, n, D)
    positions = [int(x) - 1 for x in w.ctx_lens[:n]]
    times = []
    t_start = time.perf_counter()
    while not times or (time.perf_counter() - t_start < target_seconds and len(times) < max_reps):
        t0 = time.perf_counter()
        op.decode_cpu_path(q, kc, vc, tables, positions, literal_gather=True)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    nbytes = W.decode_bytes(w.ctx_lens[:n], w.num_heads, w.num_kv_heads)
    return {
        "value": nbytes / t / 1e12,
        "unit": "TB/s",
        "cores": torch.get_num_threads(),
        "host_cpus": os.cpu_count(),
        "kind": "port",
        "sample": f"reference CPU decode path (per-token gather loop + repeat_interleave + SDPA) on all {n} "
                  f"sequences ({int(w.ctx_lens[:n].sum())} context tokens), median of {len(times)} runs "
                  f"({sum(times):.1f} s of CPU work)",
        "sample_seconds": t,
        "us_per_layer": t * 1e6,
    }


def copy_probe(nbytes=1 << 30, reps=5):
    """A plain device-to-device copy of known size (the counter calibration)."""
    x = torch.empty(nbytes // 2, dtype=torch.bfloat16, device="cuda").fill_(1.0)
    y = torch.empty_like(x)
    for _ in range(reps):
        y.copy_(x)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe": {"bytes_read": nbytes, "bytes_written": nbytes, "launches": reps}}), flush=True)


def measured_traffic():
    """HBM bytes per decode call from the committed rocprofv3 --pmc summary."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
        return t["fetch_bytes_per_call"] + t["write_bytes_per_call"], t
    except (OSError, KeyError, ValueError):
        return None, None


def _round(d):
    return {k: (round(v, 3) if isinstance(v, float) else _round(v) if isinstance(v, dict) else v)
            for k, v in d.items()}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--num-workgroups", type=int, default=0)
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-probe", action="store_true")
    ap.add_argument("--workload", default=None, help="run one workload of tinyserver_amd.workloads alone")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: the attention path is benchmarked on a single MI355X "
              "(sharding is described, not run); use --gpus 1", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(2)
    if args.copy_probe:
        copy_probe()
        return
    from tinyserver_amd import _lib

    _lib.load()
    if args.workload:
        if args.workload == "sampling-qwen3-vocab-bs64":
            res = bench_sampling(args.steps, args.warmup)
        elif "prefill" in args.workload:
            res = bench_prefill(args.workload, args.steps, args.warmup)
        else:
            res, _ = bench_decode(args.workload, args.steps, args.warmup, args.num_workgroups)
        print(json.dumps({"workload": args.workload, "steps": args.steps, "warmup": args.warmup, **_round(res)}),
              flush=True)
        return
    head, w = bench_decode(HEADLINE, args.steps, args.warmup, args.num_workgroups, with_block=True)
    traffic, traffic_src = measured_traffic()
    line = {
        "metric": METRIC,
        "value": round(head["achieved_gbs"] / 1000.0, 4),
        "unit": "TB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["wall_ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) bf16 K/V pool, shuffled page-16 block tables)",
        "config": {
            "workload": HEADLINE,
            "batch": head["batch"],
            "num_heads": head["num_heads"],
            "num_kv_heads": head["num_kv_heads"],
            "head_dim": 128,
            "page": 16,
            "ctx": "U[512,4096], seed 2",
            "sum_ctx": head["sum_ctx"],
            "num_workgroups": args.num_workgroups,
        },
        "us_per_layer": round(head["us_per_call"], 2),
        "us_per_layer_median": round(head["us_per_call_median"], 2),
        "us_per_layer_p10_p90": [round(head["us_per_call_p10"], 2), round(head["us_per_call_p90"], 2)],
        "pct_peak_hbm": round(head["pct_peak_hbm"], 2),
        "tokens_per_s": round(head["tokens_per_s"], 1),
        "decode_block_us_per_layer": round(head["block_us_per_call"], 2),
        "decode_block_fused_us_per_layer": round(head["block_fused_us_per_call"], 2),
        "roofline": {
            "bound": "hbm",
            "achieved": round(head["achieved_gbs"], 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(head["achieved_gbs"] / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "kernel": "paged_decode_stream + paged_decode_stream_merge (one decode call)",
            "bytes_per_launch": head["bytes_per_call"],
            "traffic_source": os.path.relpath(TRAFFIC_FILE, ROOT) if traffic_src else None,
        },
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(w)
    del w
    torch.cuda.empty_cache()
    if not args.no_secondary:
        sec = {}
        n2 = max(10, args.steps // 5)
        s, w2 = bench_decode("qwen3-32b-decode-bs32", n2, 3, copies=1)
        del w2
        torch.cuda.empty_cache()
        sec["qwen3-32b-decode-bs32"] = _round(s)
        s, w2 = bench_decode("qwen3-4b-mixed-decode", n2, 3)
        del w2
        torch.cuda.empty_cache()
        sec["qwen3-4b-mixed-decode"] = _round(s)
        for name in ("qwen3-8b-prefill-16seq", "qwen3-4b-mixed-prefill"):
            sec[name] = _round(bench_prefill(name, n2, 3))
        sec["sampling-qwen3-vocab-bs64"] = _round(bench_sampling(n2, 3))
        line["secondary"] = sec
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
