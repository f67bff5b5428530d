"""Benchmark of the Qwen3 attention hot path on one MI355X.

Headline (the metric line): paged decode attention at the Qwen3-8B shape,
batch 64, 32 q / 8 kv heads, head_dim 128, page 16, contexts U[512, 4096]
(seed 2) -- microseconds per layer and achieved HBM bandwidth against the
8 TB/s MI355X peak. A step is one decode-attention call over the batch (the
stream kernel plus its merge kernel, both on the caller's stream). Three
copies of the KV pool are rotated so repeated steps cannot be served from
the 256 MB MALL. The K timed steps are bracketed by one pair of HIP events
recorded on the stream the kernels run on (and by synchronisations for the
wall clock); a second pass times each call separately for the median and
p10/p90.

Also measured (in "secondary"), each with its roofline and a CPU baseline:
  qwen3-0.6b-decode-bs4     the reference's CPU-runnable decode case
  qwen3-32b-decode-bs32     32k-context decode
  qwen3-8b-prefill-16seq    varlen prefill (TFLOP/s against 2.5 PFLOP/s bf16
                            dense), its fused norm/RoPE/store (GB/s) and
                            the standalone K/V store (GB/s), mapped and paged
  qwen3-4b-mixed            the continuous-batching step on one shared pool,
                            in scheduler order: the prefill batch's
                            norm/RoPE/store and varlen attention, then the
                            decode batch's norm/RoPE/store and paged
                            attention; per-launch times and rooflines; and
                            as one norm/RoPE/store of both batches plus
                            mixed_attention (both attentions in one call)
  qwen3-4b-mixed-chunk      the same decode batch beside two short prefill
                            chunks, where mixed_attention runs one kernel
  qwen3-8b-decode-bs64-page256  the headline batch on the server's default
                            256-token pages (decode and its fused store)
  sampling-qwen3-vocab-bs64 batched sampling over 64 Qwen3-vocab rows
The headline line also carries the decode block (norm/RoPE/store, then
attention) as two launches and as the single fused launch.

CPU baselines run on this host's cores, on the same seeded inputs, as two
variants (server/model/patches/qwen3.py): "literal", the reference's own CPU
branches (decode: per-token gather loop + repeat_interleave + SDPA, :359-385
and :423-466; prefill: one SDPA with a block-diagonal causal mask over the
packed tokens, :132-171), and "vectorized", the same math with index_select
gathers and per-sequence causal SDPA. Each is bounded to a few seconds of
CPU work: a batch that one pass does not fit is sampled sequence by
sequence and scaled by context length, as its "sample" says.

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


# ------------------------------------------------------------------ timing --
# Untimed calls before each timed region also run for at least this long
# (the secondary lines set it): the shader clock ramps under sustained load,
# and a few warmup calls of a short launch leave it mid-ramp.
_MIN_WARM_MS = 0.0


def time_region(fn, steps, warmup):
    """warmup untimed calls (and more, to _MIN_WARM_MS of wall time), then
    `steps` calls bracketed by synchronisations and one pair of events on the
    current stream. Returns (event ms per call, wall ms per call)."""
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    if _MIN_WARM_MS > 0:
        t_end = time.perf_counter() + _MIN_WARM_MS / 1e3
        i = warmup
        while time.perf_counter() < t_end:
            for _ in range(8):
                fn(i)
                i += 1
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


def norm_store_bytes(tokens, hq, hkv, d=128, elem=2):
    """Algorithmic bytes of the fused norm/RoPE/store: read q, k, v, cos, sin
    and the two weights; write the rotated q and k and the K/V cache rows."""
    return (elem * tokens * d * (hq + 2 * hkv) + 2 * elem * tokens * d + 2 * elem * d
            + elem * tokens * d * (hq + hkv) + 2 * elem * tokens * hkv * d)


def kv_store_bytes(tokens, hkv, d=128, elem=2):
    """Algorithmic bytes of the paged K/V store: read the new K and V rows,
    write them into the pool."""
    return 4 * elem * tokens * hkv * d


def _roof_hbm(nbytes, us):
    gbs = nbytes / (us * 1e-6) / 1e9
    return {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes_per_launch": int(nbytes)}


def _roof_mfma(flops, us):
    tf = flops / (us * 1e-6) / 1e12
    return {"bound": "mfma", "achieved": round(tf, 1), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(tf / BF16_PEAK_TFLOPS, 4), "flops_per_launch": int(flops)}


# ----------------------------------------------------------- CPU baselines --
def _threads():
    return {"cores": torch.get_num_threads(), "host_cpus": os.cpu_count()}


def _timed_passes(run_item, n_items, weights, target_s):
    """Time run_item(i) over items 0..n-1 in order, whole passes until about
    target_s seconds of work (at least one item). Returns (seconds for one
    whole pass, description of the sample)."""
    passes, done_w, done_t, t_start = [], 0.0, 0.0, time.perf_counter()
    total_w = float(sum(weights))
    while True:
        t_pass, i = 0.0, 0
        while i < n_items:
            t0 = time.perf_counter()
            run_item(i)
            dt = time.perf_counter() - t0
            t_pass += dt
            done_w += weights[i]
            done_t += dt
            i += 1
            if time.perf_counter() - t_start > target_s and not passes:
                break
        if i == n_items:
            passes.append(t_pass)
        if time.perf_counter() - t_start > target_s or len(passes) >= 20:
            break
    if passes:
        return statistics.median(passes), f"median of {len(passes)} whole passes ({done_t:.1f} s of CPU work)"
    return done_t * total_w / done_w, (f"first {i} of {n_items} sequences ({done_w / total_w:.1%} of the batch's "
                                       f"context), scaled to the whole batch by context length ({done_t:.1f} s)")


def cpu_decode_baseline(w, literal, target_s):
    """The reference's CPU decode attention (server/model/patches/qwen3.py:
    359-385, restated in oracle.paged.decode_cpu_path) on w's batch: the
    literal per-token gather loop (:444-466) or the index_select gather. The
    new tokens are already in the pool: attention only."""
    from oracle import paged as op
    from tinyserver_amd import workloads as W

    n = len(w.ctx_lens)
    pages = sorted({p for lst in w.block_lists for p in lst})
    remap = {p: i for i, p in enumerate(pages)}
    idx = torch.tensor(pages, device=w.k_cache.device)
    kc, vc = w.k_cache[idx].cpu(), w.v_cache[idx].cpu()
    tables = [[remap[p] for p in lst] for lst in w.block_lists]
    q = w.q.cpu().transpose(0, 1).unsqueeze(0).contiguous()  # (1, Hq, B, D)
    positions = [int(x) - 1 for x in w.ctx_lens]

    def one(i):
        op.decode_cpu_path(q[:, :, i:i + 1], kc, vc, tables[i:i + 1], positions[i:i + 1], literal_gather=literal)

    t, sample = _timed_passes(one, n, [int(x) for x in w.ctx_lens], target_s)
    nbytes = W.decode_bytes(w.ctx_lens, w.num_heads, w.num_kv_heads, page=w.k_cache.shape[2])
    return {"value": round(nbytes / t / 1e12, 6), "unit": "TB/s", **_threads(), "kind": "port",
            "variant": "literal" if literal else "vectorized",
            "path": ("per-token gather loop + repeat_interleave + SDPA (qwen3.py:359-385, 423-466)" if literal
                     else "index_select page gather + repeat_interleave + SDPA per sequence"),
            "sample": sample, "us_per_layer": round(t * 1e6, 1), "tokens_per_s": round(n / t, 2)}


def cpu_prefill_baseline(p, literal, target_s):
    """The reference's CPU prefill attention on p's packed batch: one SDPA
    with a block-diagonal causal mask (qwen3.py:132-171, literal) or one
    causal SDPA per sequence (vectorized). Attention only."""
    from oracle import varlen as ov
    from tinyserver_amd import workloads as W

    q, k, v, cu = p.q.cpu(), p.k.cpu(), p.v.cpu(), p.cu_seqlens.cpu()
    lens = [int(x) for x in p.seq_lens]
    flops = W.prefill_flops(lens, q.shape[1])
    if literal:
        qh, kh, vh = (t.transpose(0, 1)[None].contiguous() for t in (q, k, v))

        def one(_):
            ov.prefill_sdpa_block_mask(qh, kh, vh, lens, q.shape[2])

        t, sample = _timed_passes(one, 1, [1], target_s)
        sample = "the whole packed batch, " + sample
    else:
        def one(i):
            ov.prefill_sdpa_per_sequence(q[cu[i]:cu[i + 1]], k[cu[i]:cu[i + 1]], v[cu[i]:cu[i + 1]],
                                         torch.tensor([0, lens[i]]))

        t, sample = _timed_passes(one, len(lens), [n * n for n in lens], target_s)
    return {"value": round(flops / t / 1e12, 6), "unit": "TFLOP/s", **_threads(), "kind": "port",
            "variant": "literal" if literal else "vectorized",
            "path": ("one SDPA with a block-diagonal causal mask over the packed tokens (qwen3.py:132-171)"
                     if literal else "one causal SDPA per sequence"),
            "sample": sample, "us_per_layer": round(t * 1e6, 1), "tokens_per_s": round(sum(lens) / t, 1)}


def cpu_sampling_baseline(logits, temperature, top_k, top_p, uniforms, target_s):
    """The reference's batched sampler (server/model/sampling.py:119-194, its
    torch ops restated in oracle.sampling) on the CPU."""
    from oracle import sampling as osm

    args = [t.cpu() for t in (logits, temperature, top_k, top_p, uniforms)]
    t, sample = _timed_passes(lambda _: osm.sample_tokens(*args), 1, [1], target_s)
    nbytes = logits.numel() * logits.element_size()
    return {"value": round(nbytes / t / 1e9, 4), "unit": "GB/s of logits", **_threads(), "kind": "port",
            "variant": "literal", "path": "sort + softmax + cumsum + searchsorted, fp32", "sample": sample,
            "us_per_call": round(t * 1e6, 1)}


# ------------------------------------------------------------- GPU parts --
def _decode_pools(w, copies):
    return [(w.k_cache, w.v_cache)] + [(w.k_cache.clone(), w.v_cache.clone()) for _ in range(copies - 1)]


def _decode_kernels(w, page, num_workgroups):
    """The launches of one decode call: a workspace of the tile prefix alone
    (no partial slots) is the library's one-workgroup-per-unit form."""
    from tinyserver_amd.kernels.paged_attention import decode_workspace_bytes

    B = len(w.ctx_lens)
    ws = decode_workspace_bytes(B, w.num_heads, w.num_kv_heads, w.q.shape[-1], w.block_tables.shape[1], page,
                                num_workgroups)
    if ws <= (4 * (B + 1) + 255) // 256 * 256:
        return "paged_decode_stream (one workgroup per unit, no merge launch)"
    return "paged_decode_stream + paged_decode_stream_merge"


def bench_decode(name, steps, warmup, num_workgroups=0, copies=3, with_block=False, **make_kw):
    from tinyserver_amd import workloads as W
    from tinyserver_amd.kernels import paged_attention_forward, paged_decode_step, qk_norm_rope_store

    dev = torch.device("cuda:0")
    w = W.make(name, device=dev, **make_kw)
    B = len(w.ctx_lens)
    page = w.k_cache.shape[2]
    seq_lens = w.ctx_lens.to(torch.int32).to(dev)
    pools = _decode_pools(w, copies)
    cu = torch.arange(B + 1, dtype=torch.int32, device=dev)
    pos = w.positions.to(dev)
    q_rot, _ = qk_norm_rope_store(w.q, w.k, w.v, w.q_weight, w.k_weight, w.cos, w.sin, w.eps, pools[0][0],
                                  pools[0][1], w.block_tables, cu, pos, return_k=False)
    out = torch.empty_like(q_rot)

    def attn(i):
        kc, vc = pools[i % copies]
        paged_attention_forward(q_rot, kc, vc, w.block_tables, page, seq_lens, num_workgroups=num_workgroups,
                                out=out)

    ev_ms, wall_ms = time_region(attn, steps, warmup)
    spread = _spread(time_each(attn, max(20, min(steps, 200)), warmup + steps))
    nbytes = W.decode_bytes(w.ctx_lens, w.num_heads, w.num_kv_heads, page=page)
    us = ev_ms * 1e3
    res = {
        "workload": name if page == W.PAGE else f"{name}-page{page}",
        "batch": B, "num_heads": w.num_heads, "num_kv_heads": w.num_kv_heads, "page": page,
        "sum_ctx": int(w.ctx_lens.sum()), "bytes_per_call": nbytes,
        "us_per_call": us, "us_per_call_median": spread["median"], "us_per_call_p10": spread["p10"],
        "us_per_call_p90": spread["p90"], "wall_ms_per_step": wall_ms,
        "achieved_gbs": nbytes / (us * 1e-6) / 1e9, "tokens_per_s": B / (us * 1e-6),
        "roofline": {**_roof_hbm(nbytes, us), "kernel": _decode_kernels(w, page, num_workgroups)},
    }
    res["pct_peak_hbm"] = 100.0 * res["achieved_gbs"] / HBM_PEAK_GBS
    if with_block:
        qw, kw, cos, sin = w.q_weight, w.k_weight, w.cos, w.sin

        def store(i):
            kc, vc = pools[i % copies]
            qk_norm_rope_store(w.q, w.k, w.v, qw, kw, cos, sin, w.eps, kc, vc, w.block_tables, cu, pos,
                               return_k=False)

        s_us = time_region(store, steps, warmup)[0] * 1e3
        sb = norm_store_bytes(B, w.num_heads, w.num_kv_heads)
        res["norm_rope_store_us"] = s_us
        res["norm_rope_store_roofline"] = _roof_hbm(sb, s_us)
        # The same calls replayed from a captured graph (as a serving loop
        # runs a decode step): GPU time without the Python enqueue, which
        # bounds the eager figures of small batches.
        res["graph_us_per_call"] = _graph_us_per_call(attn, steps, warmup)
        res["norm_rope_store_graph_us"] = _graph_us_per_call(store, steps, warmup)

        def block(i):
            kc, vc = pools[i % copies]
            qr, _ = qk_norm_rope_store(w.q, w.k, w.v, qw, kw, cos, sin, w.eps, kc, vc, w.block_tables, cu, pos,
                                       return_k=False)
            paged_attention_forward(qr, kc, vc, w.block_tables, page, seq_lens, num_workgroups=num_workgroups,
                                    out=out)

        res["block_us_per_call"] = time_region(block, steps, warmup)[0] * 1e3
        res["block_graph_us_per_call"] = _graph_us_per_call(block, steps, warmup)

        def block_fused(i):  # the same step as one fused call (two launches)
            kc, vc = pools[i % copies]
            paged_decode_step(w.q, w.k, w.v, qw, kw, cos, sin, w.eps, kc, vc, w.block_tables, seq_lens,
                              num_workgroups=num_workgroups, out=out)

        try:
            res["block_fused_us_per_call"] = time_region(block_fused, steps, warmup)[0] * 1e3
            res["block_fused_graph_us_per_call"] = _graph_us_per_call(block_fused, steps, warmup)
        except NotImplementedError as e:  # outside the fused kernel's coverage
            res["block_fused_us_per_call"] = None
            res["block_fused_note"] = str(e)
    del pools
    return res, w


def bench_prefill(name, steps, warmup):
    from tinyserver_amd import workloads as W
    from tinyserver_amd.kernels import (flash_attn_varlen_func, qk_norm_rope_store, store_kv_cache_batched,
                                        store_kv_cache_paged)

    dev = torch.device("cuda:0")
    w = W.make(name, device=dev)
    T, hq, hkv = w.q.shape[0], w.q.shape[1], w.k.shape[1]
    q_rot, k_rot = qk_norm_rope_store(w.q, w.k, w.v, w.q_weight, w.k_weight, w.cos, w.sin, w.eps, w.k_cache,
                                      w.v_cache, w.block_tables, w.cu_seqlens)
    out = torch.empty_like(q_rot)

    def attn(i):
        flash_attn_varlen_func(q_rot, k_rot, w.v, w.cu_seqlens, w.cu_seqlens, w.max_seqlen, w.max_seqlen, True, out=out)

    us = time_region(attn, steps, warmup)[0] * 1e3
    spread = _spread(time_each(attn, max(20, min(steps, 200)), warmup + steps))
    flops = W.prefill_flops(w.seq_lens, hq)

    def norm_store(i):
        qk_norm_rope_store(w.q, w.k, w.v, w.q_weight, w.k_weight, w.cos, w.sin, w.eps, w.k_cache, w.v_cache,
                           w.block_tables, w.cu_seqlens)

    ns_us = time_region(norm_store, steps, warmup)[0] * 1e3
    ns_spread = _spread(time_each(norm_store, max(20, min(steps, 200)), warmup + steps))
    ns_bytes = norm_store_bytes(T, hq, hkv)

    # The standalone K/V store, as the reference's prefill calls it: the new
    # rows as a contiguous (Hkv, T, D) copy and int64 block/slot mappings
    # (server/model/patches/qwen3.py:296-313), and the one-launch form with
    # device-side addressing from the block tables and cu_seqlens.
    k_src, v_src = w.k.transpose(0, 1).contiguous(), w.v.transpose(0, 1).contiguous()
    page = w.k_cache.shape[2]
    seq_of = torch.repeat_interleave(torch.arange(len(w.seq_lens), device=dev), w.seq_lens.to(dev))
    pos = torch.arange(T, device=dev) - w.cu_seqlens.long()[seq_of]
    block_mapping = w.block_tables.long()[seq_of, pos // page]
    slot_mapping = pos % page

    def kv_store_mapped(i):
        store_kv_cache_batched(k_src, v_src, w.k_cache, w.v_cache, block_mapping, slot_mapping)

    def kv_store_paged(i):
        store_kv_cache_paged(w.k.transpose(0, 1), w.v.transpose(0, 1), w.k_cache, w.v_cache, w.block_tables,
                             w.cu_seqlens)

    kv_bytes = kv_store_bytes(T, hkv)
    kvm_us = time_region(kv_store_mapped, steps, warmup)[0] * 1e3
    kvp_us = time_region(kv_store_paged, steps, warmup)[0] * 1e3

    def block(i):
        qr, kr = qk_norm_rope_store(w.q, w.k, w.v, w.q_weight, w.k_weight, w.cos, w.sin, w.eps, w.k_cache,
                                    w.v_cache, w.block_tables, w.cu_seqlens)
        flash_attn_varlen_func(qr, kr, w.v, w.cu_seqlens, w.cu_seqlens, w.max_seqlen, w.max_seqlen, True, out=out)

    block_us = time_region(block, steps, warmup)[0] * 1e3
    return {
        "workload": name, "tokens": T, "gflop": flops / 1e9,
        "us_per_call": us, "us_per_call_median": spread["median"], "us_per_call_p10": spread["p10"],
        "us_per_call_p90": spread["p90"], "tflops": flops / (us * 1e-6) / 1e12,
        "pct_peak_mfma": 100.0 * flops / (us * 1e-6) / 1e12 / BF16_PEAK_TFLOPS,
        "tokens_per_s": T / (us * 1e-6),
        "roofline": {**_roof_mfma(flops, us), "kernel": _prefill_kernel(w.q.shape[1] // w.k.shape[1], w.q.shape[2])},
        "norm_rope_store_us": ns_us, "norm_rope_store_us_median": ns_spread["median"],
        "norm_rope_store_us_p10": ns_spread["p10"], "norm_rope_store_us_p90": ns_spread["p90"],
        "norm_rope_store_gbs": ns_bytes / (ns_us * 1e-6) / 1e9,
        "norm_rope_store_roofline": _roof_hbm(ns_bytes, ns_us),
        "kv_store_mapped_us": kvm_us, "kv_store_mapped_roofline": _roof_hbm(kv_bytes, kvm_us),
        "kv_store_paged_us": kvp_us, "kv_store_paged_roofline": _roof_hbm(kv_bytes, kvp_us),
        "block_us_per_call": block_us,
    }, w


def bench_mixed(name, steps, warmup, copies=3):
    """The continuous-batching step on one shared pool, in scheduler order:
    the prefill batch's fused norm/RoPE/store and varlen attention, then the
    decode batch's norm/RoPE/store and paged attention, on one stream. Timed
    as a whole step and launch by launch (each alone, on the same inputs);
    and as one norm/RoPE/store of both batches plus one attention launch
    (mixed_attention)."""
    from tinyserver_amd import workloads as W
    from tinyserver_amd.kernels import (flash_attn_varlen_func, mixed_attention, paged_attention_forward,
                                        qk_norm_rope_store)

    dev = torch.device("cuda:0")
    m = W.make(name, device=dev)
    p, d = m.prefill, m.decode
    pools = _decode_pools(d, copies)
    B = len(d.ctx_lens)
    cu_d = torch.arange(B + 1, dtype=torch.int32, device=dev)
    pos, seq_lens = d.positions.to(dev), d.ctx_lens.to(torch.int32).to(dev)
    T, hq, hkv = p.q.shape[0], p.q.shape[1], p.k.shape[1]

    def pre_store(i):
        kc, vc = pools[i % copies]
        return qk_norm_rope_store(p.q, p.k, p.v, p.q_weight, p.k_weight, p.cos, p.sin, p.eps, kc, vc,
                                  p.block_tables, p.cu_seqlens)

    def dec_store(i):
        kc, vc = pools[i % copies]
        return qk_norm_rope_store(d.q, d.k, d.v, d.q_weight, d.k_weight, d.cos, d.sin, d.eps, kc, vc,
                                  d.block_tables, cu_d, pos, return_k=False)[0]

    qp, kp = pre_store(0)
    qd = dec_store(0)
    out_p, out_d = torch.empty_like(qp), torch.empty_like(qd)

    def pre_attn(i):
        flash_attn_varlen_func(qp, kp, p.v, p.cu_seqlens, p.cu_seqlens, p.max_seqlen, p.max_seqlen, True, out=out_p)

    def dec_attn(i):
        kc, vc = pools[i % copies]
        paged_attention_forward(qd, kc, vc, d.block_tables, W.PAGE, seq_lens, out=out_d)

    def step(i):
        kc, vc = pools[i % copies]
        q1, k1 = pre_store(i)
        flash_attn_varlen_func(q1, k1, p.v, p.cu_seqlens, p.cu_seqlens, p.max_seqlen, p.max_seqlen, True, out=out_p)
        q2 = dec_store(i)
        paged_attention_forward(q2, kc, vc, d.block_tables, W.PAGE, seq_lens, out=out_d)

    # The same step as an engine batching both would issue it: one
    # norm/RoPE/store over the tokens of both batches (packed outside the
    # timed region, as the engine's metadata step would), then both attention
    # calls in one launch (mixed_attention, + the decode merge).
    width = max(p.block_tables.shape[1], d.block_tables.shape[1])

    def pad(t):
        return torch.nn.functional.pad(t, (0, width - t.shape[1]))

    ppos = torch.cat([torch.arange(int(n)) for n in p.seq_lens.cpu()]).to(dev)
    pk = dict(q=torch.cat([p.q, d.q]), k=torch.cat([p.k, d.k]), v=torch.cat([p.v, d.v]),
              cos=torch.cat([p.cos, d.cos]), sin=torch.cat([p.sin, d.sin]),
              bt=torch.cat([pad(p.block_tables), pad(d.block_tables)]),
              cu=torch.cat([p.cu_seqlens, T + torch.arange(1, B + 1, dtype=torch.int32, device=dev)]),
              pos=torch.cat([ppos, pos]).to(torch.int64))
    q_all = torch.empty_like(pk["q"])
    k_all = torch.empty_like(pk["k"])

    def packed_store(i):
        kc, vc = pools[i % copies]
        qk_norm_rope_store(pk["q"], pk["k"], pk["v"], p.q_weight, p.k_weight, pk["cos"], pk["sin"], p.eps, kc, vc,
                           pk["bt"], pk["cu"], pk["pos"], q_out=q_all, k_out=k_all)

    packed_store(0)

    cus = torch.cuda.get_device_properties(dev).multi_processor_count

    def one_attn(i, prefill_workgroups=0):
        kc, vc = pools[i % copies]
        mixed_attention(q_all[:T], k_all[:T], p.v, p.cu_seqlens, p.max_seqlen, q_all[T:], kc, vc, d.block_tables,
                        seq_lens, prefill_workgroups=prefill_workgroups, prefill_out=out_p, out=out_d)

    def step_one(i):
        packed_store(i)
        one_attn(i)

    step_us = time_region(step, steps, warmup)[0] * 1e3
    step_one_us = time_region(step_one, steps, warmup)[0] * 1e3
    # The GPU time of each form without the host's enqueue cost (its eager
    # launches of small batches are host-bound).
    step_graph_us = _graph_us_per_call(step, steps, warmup)
    step_one_graph_us = _graph_us_per_call(step_one, steps, warmup)
    graph_parts = {k: _graph_us_per_call(f, steps, warmup)
                   for k, f in (("prefill_norm_rope_store", pre_store), ("prefill_attention", pre_attn),
                                ("decode_norm_rope_store", dec_store), ("decode_attention", dec_attn),
                                ("packed_norm_rope_store", packed_store), ("mixed_attention", one_attn),
                                ("one_kernel", lambda i: one_attn(i, cus)))}
    t = {k: time_region(f, steps, warmup)[0] * 1e3
         for k, f in (("prefill_norm_rope_store", pre_store), ("prefill_attention", pre_attn),
                      ("decode_norm_rope_store", dec_store), ("decode_attention", dec_attn))}
    t_one = {k: time_region(f, steps, warmup)[0] * 1e3
             for k, f in (("norm_rope_store", packed_store), ("mixed_attention", one_attn),
                          ("one_kernel", lambda i: one_attn(i, cus)))}
    flops = W.prefill_flops(p.seq_lens, hq)
    dbytes = W.decode_bytes(d.ctx_lens, d.num_heads, d.num_kv_heads)
    launches = {
        "prefill_norm_rope_store": {"us": t["prefill_norm_rope_store"],
                                    "roofline": _roof_hbm(norm_store_bytes(T, hq, hkv), t["prefill_norm_rope_store"])},
        "prefill_attention": {"us": t["prefill_attention"], "roofline": _roof_mfma(flops, t["prefill_attention"])},
        "decode_norm_rope_store": {"us": t["decode_norm_rope_store"],
                                   "roofline": _roof_hbm(norm_store_bytes(B, hq, hkv), t["decode_norm_rope_store"])},
        "decode_attention": {"us": t["decode_attention"], "roofline": _roof_hbm(dbytes, t["decode_attention"])},
    }
    del pools
    return {
        "workload": name, "prefill_seqs": len(p.seq_lens), "prefill_tokens": T, "decode_batch": B,
        "sum_ctx": int(d.ctx_lens.sum()), "pool_pages": int(m.k_cache.shape[0]),
        "step_us": step_us, "step_graph_us": step_graph_us, "launch_graph_us": graph_parts,
        "sum_of_launches_us": sum(t.values()),
        "tokens_per_s": (T + B) / (step_us * 1e-6), "launches": launches,
        "order": "prefill norm/RoPE/store -> varlen attention -> decode norm/RoPE/store -> paged attention",
        "one_launch": {
            "step_us": step_one_us, "step_graph_us": step_one_graph_us,
            "tokens_per_s": (T + B) / (step_one_us * 1e-6),
            "order": "norm/RoPE/store of both batches' tokens -> mixed_attention (varlen attention + paged "
                     "attention in one kernel, + the decode merge)",
            "norm_rope_store_us": t_one["norm_rope_store"],
            "mixed_attention_us": t_one["mixed_attention"],
            "mixed_attention_path": ("one kernel" if T <= 512 and B * d.block_tables.shape[1] * W.PAGE <= 131072
                                     else "two launches (more than 512 prefill tokens or 131072 decode table tokens)"),
            "one_kernel_us": t_one["one_kernel"],
            "separate_attention_sum_us": t["prefill_attention"] + t["decode_attention"],
            "roofline": {"decode_hbm": _roof_hbm(dbytes, t_one["one_kernel"]),
                         "prefill_mfma": _roof_mfma(flops, t_one["one_kernel"]),
                         "note": "the one kernel: decode bytes and prefill FLOPs each over its whole time"},
        },
    }, m


def bench_sampling(steps, warmup, batch=64, vocab=151936, copies=16):
    """sample_tokens over a Qwen3-vocab batch: bf16 logits (N(0, 2.5) plus a
    few boosted tokens per row), seeded uniforms; four filter settings, the
    last the reference server's default request (temperature 1.0, top_p
    0.95, top_k 0: server/api/schema.py:11-15). The calls rotate over
    `copies` copies of the logits (16 x 19.4 MB, past the 256 MB MALL), so
    each call reads its row from HBM. One launch per call, timed eagerly and
    replayed from a captured graph."""
    from tinyserver_amd.kernels import sample_tokens

    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(21)
    logits = torch.randn(batch, vocab, generator=g) * 2.5
    logits.scatter_add_(1, torch.randint(0, vocab, (batch, 8), generator=g), torch.rand(batch, 8, generator=g) * 12)
    logits = logits.to(dev, torch.bfloat16)
    pool = [logits] + [logits.clone() for _ in range(copies - 1)]
    temperature = torch.full((batch,), 0.8, device=dev)
    top_k = torch.full((batch,), 50, dtype=torch.int64, device=dev)
    top_p = torch.full((batch,), 0.9, device=dev)
    uniforms = torch.rand(batch, generator=g).to(dev)
    out = torch.empty(batch, dtype=torch.int64, device=dev)
    cases = {}
    nbytes = batch * vocab * 2
    for label, temp, k, pp in (("topk50_topp0.9", 0.8, 50, 0.9), ("topp0.9", 0.8, 0, 0.9), ("full", 0.8, 0, 1.0),
                               ("server_default_t1_topp0.95", 1.0, 0, 0.95)):
        temperature.fill_(temp)
        top_k.fill_(k)
        top_p.fill_(pp)

        def call(i):
            sample_tokens(pool[i % copies], temperature, top_k, top_p, uniforms, out=out)

        us = time_region(call, steps, warmup)[0] * 1e3
        gus = _graph_us_per_call(call, steps, warmup)
        cases[label] = {"temperature": temp, "top_k": k, "top_p": pp, "us_per_call": us, "graph_us_per_call": gus,
                        "logits_gbs": nbytes / (gus * 1e-6) / 1e9,
                        "roofline": {**_roof_hbm(nbytes, gus), "kernel": "sample_tokens_kernel",
                                     "note": f"per call in a captured graph of 20 calls over {copies} logits "
                                             "copies (the eager us_per_call also holds the Python enqueue)"}}
    temperature.fill_(0.8)
    top_k.fill_(50)
    top_p.fill_(0.9)
    del pool
    return {"workload": f"sample_tokens bs{batch} vocab{vocab} bf16", "batch": batch, "vocab": vocab,
            "logits_copies": copies, **cases}, (logits, temperature, top_k, top_p, uniforms)


def _prefill_kernel(group, head_dim):
    """The kernel tsa_varlen_prefill runs for bf16 rows of this GQA group and
    head_dim (varlen_prefill.hip: takes_w64, then takes_gqa)."""
    if head_dim == 128 and group % 4 == 0 and os.environ.get("TSA_PREFILL_W64", "1")[:1] != "0":
        return "varlen_prefill_w64"
    return "varlen_prefill_gqa" if group in (2, 4, 8) else "varlen_prefill_mfma"


def _graph_us_per_call(fn, steps, warmup, calls=20):
    """fn(i) for i < `calls` captured in one HIP graph, replayed: the GPU
    time per call without the host's enqueue cost."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(3):
            fn(i)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(calls):
            fn(i)
    reps = max(2, steps // calls)
    ms = time_region(lambda i: graph.replay(), reps, max(1, warmup // calls))[0]
    del graph
    return ms * 1e3 / calls


def clock_ramp(ms=200.0):
    """Device copies (not the measured path) for `ms` of wall time before the
    headline's warmup steps, so the shader clock has left its idle state as
    it has in a serving loop; returns the time spent."""
    x = torch.empty(1 << 27, dtype=torch.bfloat16, device="cuda")
    y = torch.empty_like(x)
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(8):
            y.copy_(x)
        torch.cuda.synchronize()
    del x, y
    return (time.perf_counter() - t0) * 1e3


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
    if isinstance(d, dict):
        return {k: _round(v) for k, v in d.items()}
    if isinstance(d, float):
        return round(d, 3)
    return d


def _free():
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def _fmt_cpu(cpu):
    """The CPU baselines of a result, as 'cpu(literal) 1.2e+06 us' pieces."""
    if not isinstance(cpu, dict):
        return ""
    parts = []
    for variant in ("literal", "vectorized"):
        c = cpu.get(variant)
        if isinstance(c, dict) and ("us_per_layer" in c or "us_per_call" in c):
            parts.append(f"cpu({variant}) {c.get('us_per_layer', c.get('us_per_call')):.0f} us")
    if "us_per_call" in cpu:
        parts.append(f"cpu {cpu['us_per_call']:.0f} us")
    return " ".join(parts)


def _summary(name, s):
    """One short line per workload: time per call, roofline fraction, CPU
    baseline time (the whole result is in the JSON line)."""
    bits = [name]
    if "roofline" in s and "us_per_call" in s:  # decode or prefill
        r = s["roofline"]
        bits.append(f"{s['us_per_call']:.1f} us {r['bound']} {r['frac']:.3f}")
        if "graph_us_per_call" in s:
            bits.append(f"graph {s['graph_us_per_call']:.1f} us")
        if "block_graph_us_per_call" in s:
            bits.append(f"block graph {s['block_graph_us_per_call']:.1f} us eager {s['block_us_per_call']:.1f} us")
        if "norm_rope_store_roofline" in s:
            bits.append(f"norm/rope/store {s['norm_rope_store_us']:.1f} us "
                        f"hbm {s['norm_rope_store_roofline']['frac']:.3f}")
    if "step_graph_us" in s:  # mixed step
        bits.append(f"step graph {s['step_graph_us']:.1f} us, one-store form {s['one_launch']['step_graph_us']:.1f} us")
        for k, v in s["launches"].items():
            bits.append(f"{k} {v['us']:.1f} us {v['roofline']['bound']} {v['roofline']['frac']:.3f}")
    for k, v in s.items():  # sampling cases
        if isinstance(v, dict) and "graph_us_per_call" in v and "roofline" in v:
            bits.append(f"{k} graph {v['graph_us_per_call']:.1f} us hbm {v['roofline']['frac']:.3f}")
    cpu = s.get("cpu_baseline")
    if isinstance(cpu, dict) and ("prefill" in cpu or "decode" in cpu):
        bits += [f"{half}: {_fmt_cpu(cpu[half])}" for half in ("prefill", "decode") if half in cpu]
    elif cpu:
        bits.append(_fmt_cpu(cpu))
    return " | ".join(b for b in bits if b)


def _progress(name, s):
    print(f"bench: {_summary(name, s)}", file=sys.stderr, flush=True)


def secondaries(steps, warmup, cpu, cpu_s):
    """Every secondary workload, each with its CPU baselines (cpu=True)."""
    global _MIN_WARM_MS
    _MIN_WARM_MS = 200.0
    sec = {}
    # the reference's CPU-runnable decode case
    s, w = bench_decode("qwen3-0.6b-decode-bs4", steps, warmup, with_block=True)
    if cpu:
        s["cpu_baseline"] = {"literal": cpu_decode_baseline(w, True, cpu_s),
                             "vectorized": cpu_decode_baseline(w, False, cpu_s)}
    sec["qwen3-0.6b-decode-bs4"] = _round(s)
    _progress("qwen3-0.6b-decode-bs4", sec["qwen3-0.6b-decode-bs4"])
    del w
    _free()
    # 32k-context decode (one pool copy: 4.3 GB, far past the MALL)
    s, w = bench_decode("qwen3-32b-decode-bs32", steps, min(warmup, 3), copies=1)
    if cpu:
        s["cpu_baseline"] = {"literal": cpu_decode_baseline(w, True, cpu_s),
                             "vectorized": cpu_decode_baseline(w, False, cpu_s)}
    sec["qwen3-32b-decode-bs32"] = _round(s)
    _progress("qwen3-32b-decode-bs32", sec["qwen3-32b-decode-bs32"])
    del w
    _free()
    # varlen prefill
    s, w = bench_prefill("qwen3-8b-prefill-16seq", steps, min(warmup, 3))
    if cpu:
        s["cpu_baseline"] = {
            "literal": {"skipped": "the block-diagonal mask over 17,794 packed tokens is a dense 17,794^2 matrix "
                                   "(606 MB in bf16) and its SDPA scores every pair: not a bounded sample"},
            "vectorized": cpu_prefill_baseline(w, False, cpu_s)}
    sec["qwen3-8b-prefill-16seq"] = _round(s)
    _progress("qwen3-8b-prefill-16seq", sec["qwen3-8b-prefill-16seq"])
    del w
    _free()
    # the continuous-batching step on one shared pool
    s, m = bench_mixed("qwen3-4b-mixed", steps, min(warmup, 3))
    if cpu:
        s["cpu_baseline"] = {
            "prefill": {"literal": cpu_prefill_baseline(m.prefill, True, cpu_s),
                        "vectorized": cpu_prefill_baseline(m.prefill, False, cpu_s)},
            "decode": {"literal": cpu_decode_baseline(m.decode, True, cpu_s),
                       "vectorized": cpu_decode_baseline(m.decode, False, cpu_s)}}
    sec["qwen3-4b-mixed"] = _round(s)
    _progress("qwen3-4b-mixed", sec["qwen3-4b-mixed"])
    del m
    _free()
    s, m = bench_mixed("qwen3-4b-mixed-chunk", steps, min(warmup, 3))
    sec["qwen3-4b-mixed-chunk"] = _round(s)
    _progress("qwen3-4b-mixed-chunk", sec["qwen3-4b-mixed-chunk"])
    del m
    _free()
    # the headline batch on the server's default 256-token pages
    s, w = bench_decode(HEADLINE, steps, min(warmup, 3), with_block=True, page=256)
    sec["qwen3-8b-decode-bs64-page256"] = _round(s)
    _progress("qwen3-8b-decode-bs64-page256", sec["qwen3-8b-decode-bs64-page256"])
    del w
    _free()
    # batched sampling
    s, args = bench_sampling(steps, min(warmup, 3))
    if cpu:
        s["cpu_baseline"] = cpu_sampling_baseline(*args, cpu_s)
    sec["sampling-qwen3-vocab-bs64"] = _round(s)
    _progress("sampling-qwen3-vocab-bs64", sec["sampling-qwen3-vocab-bs64"])
    return sec


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--num-workgroups", type=int, default=0)
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=4.0, help="CPU work per secondary CPU baseline")
    ap.add_argument("--copy-probe", action="store_true")
    ap.add_argument("--workload", default=None, help="run one workload of tinyserver_amd.workloads alone")
    ap.add_argument("--page", type=int, default=None, help="page size for --workload (decode workloads)")
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
    from tinyserver_amd import workloads as W

    _lib.load()
    if args.workload:
        global _MIN_WARM_MS
        _MIN_WARM_MS = 200.0
        kind = W.WORKLOADS[args.workload][0] if args.workload in W.WORKLOADS else None
        if args.workload == "sampling-qwen3-vocab-bs64":
            res, _ = bench_sampling(args.steps, args.warmup)
        elif kind == "prefill":
            res, _ = bench_prefill(args.workload, args.steps, args.warmup)
        elif kind == "mixed":
            res, _ = bench_mixed(args.workload, args.steps, args.warmup)
        else:
            kw = {"page": args.page} if args.page else {}
            res, _ = bench_decode(args.workload, args.steps, args.warmup, args.num_workgroups, with_block=True, **kw)
        print(json.dumps({"workload": args.workload, "steps": args.steps, "warmup": args.warmup, **_round(res)}),
              flush=True)
        return
    ramp_ms = clock_ramp()
    head, w = bench_decode(HEADLINE, args.steps, args.warmup, args.num_workgroups, with_block=True)
    traffic, traffic_src = measured_traffic()
    line = {
        "metric": METRIC,
        "value": round(head["achieved_gbs"] / 1000.0, 4),
        "unit": "TB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "clock_ramp_ms": round(ramp_ms, 1),
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
        "decode_norm_rope_store_us": round(head["norm_rope_store_us"], 2),
        "decode_block_us_per_layer": round(head["block_us_per_call"], 2),
        "decode_block_fused_us_per_layer": round(head["block_fused_us_per_call"], 2),
        "decode_graph_us_per_layer": {k: round(head[k], 2) for k in (
            "graph_us_per_call", "norm_rope_store_graph_us", "block_graph_us_per_call",
            "block_fused_graph_us_per_call") if head.get(k) is not None},
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
        lit = cpu_decode_baseline(w, True, 10.0)
        line["cpu_baseline"] = {**lit, "vectorized": cpu_decode_baseline(w, False, 5.0)}
    print(f"bench: {HEADLINE} (headline) {line['us_per_layer']:.1f} us hbm {line['roofline']['frac']:.3f} | wall "
          f"{line['ms_per_step'] * 1e3:.1f} us/step | graph {head['graph_us_per_call']:.1f} us | block graph "
          f"{head['block_graph_us_per_call']:.1f} us eager {head['block_us_per_call']:.1f} us"
          + (f" | cpu(literal) {line['cpu_baseline']['us_per_layer']:.0f} us cpu(vectorized) "
             f"{line['cpu_baseline']['vectorized']['us_per_layer']:.0f} us" if "cpu_baseline" in line else ""),
          file=sys.stderr, flush=True)
    del w
    _free()
    if not args.no_secondary:
        line["secondary"] = secondaries(max(10, args.steps // 5), 3, not args.no_cpu_baseline, args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
