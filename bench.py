#!/usr/bin/env python3
"""Benchmark of the MI355X attention hot path; prints ONE JSON line.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--only decode|decode_small|prefill|long|mixed|flash|cache]
                    [--no-cpu-baseline]

Headline (``value``): paged decode attention, bf16, Qwen3-0.6B attention
shape (16 query heads, 8 KV heads, head_dim 128, 16-token pages), 64
sequences with contexts U[256, 4096] scattered over a pool 1.2x the used
blocks.  One step = one ``femtovllm.ops.paged_attention_gemv`` call over the
batch.  ``value`` = algorithmic HBM bytes (K and V once per KV head, Q, O,
block-table entries, kv_lens) / mean kernel time, in GB/s.

Timing: every step is [cache flush][spin][start event][op][end event] on
torch's current stream, the stream the op launches its kernels on;
``ms_per_step`` is the mean start->end time over K steps after W warm-up
steps, bracketed by torch.cuda.synchronize().  Inputs are resident in HBM
before timing starts.  The flush *reads* a 1 GiB buffer, which evicts the
pool from L2 and the 256 MB MALL and leaves the caches clean; a flush that
writes 1 GiB instead leaves ~256 MB of dirty lines whose write-back then
competes with the measured kernel (that figure is reported alongside as
``ms_per_step_write_flush``).

``--only copy`` times a plain 1 GiB device copy (used to calibrate the
HBM byte counters of rocprofv3).  Also reported (``extra``): chunked prefill TFLOP/s (8 x 512-token
chunks, and four uneven sequences with and without the key split),
long-context prefill (Llama-3-8B shape, 16 x 2048-token chunks of a 32k
sequence, and one GPU's 4-head / 1-KV-head share of it under 8-way tensor
parallelism, with and without the key split), the unified mixed batch
(Qwen3-8B shape, both routes), the dense flash-attention latencies at the
reference benchmark shapes and its TFLOP/s at the long-context chunk shapes, and the
KV-cache write (new K/V of the 8 x 512 prefill and of a 64-sequence decode
step scattered into the pools) and the fused q/k RMSNorm + RoPE + cache write
of the same chunk, in GB/s of bytes read + written.
``cpu_baseline``: the reference's CPU attention path (per-sequence block
gather + torch SDPA, restated in oracle/sdpa_path.py) timed on the host in
the workload dtype.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "nano-vllm-practice_amd")
for _p in (ROOT, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
PROFILES = os.path.join(ROOT, "profiles")


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--only", default="all",
                    choices=["all", "decode", "decode_small", "prefill", "long", "mixed", "flash", "cache", "copy"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    return ap.parse_args()


class Timer:
    """Per-step kernel timing with HIP events on torch's current stream."""

    def __init__(self, torch, device):
        self.torch = torch
        self.rbuf = torch.ones(1 << 28, dtype=torch.float32, device=device)
        self.wbuf = torch.empty(1 << 30, dtype=torch.uint8, device=device)

    def run(self, fn, steps, warmup, write_flush=False):
        torch = self.torch
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        evs = []
        t0 = time.perf_counter()
        for _ in range(steps):
            if write_flush:
                self.wbuf.zero_()
            else:
                self.rbuf.sum()
            torch.cuda._sleep(1_000_000)
            s = torch.cuda.Event(enable_timing=True)
            e = torch.cuda.Event(enable_timing=True)
            s.record()
            fn()
            e.record()
            evs.append((s, e))
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        ms = [s.elapsed_time(e) for s, e in evs]
        return statistics.fmean(ms), statistics.median(ms), wall


# Sources of the decode kernels: the committed PMC summary's traffic figure is
# used only while these files are the ones it measured.
DECODE_SOURCES = ("csrc/paged_decode.hip", "csrc/decode_worker.h", "csrc/common.h", "csrc/launch.h")


def sources_sha16(rel_paths):
    import hashlib

    h = hashlib.sha256()
    for rel in rel_paths:
        with open(os.path.join(PKG, rel), "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def pmc_traffic(kernel_key, rel_paths):
    """HBM bytes per launch from a committed rocprofv3 --pmc summary, and where
    the figure comes from: null when the summary is missing or measured other
    kernel sources than the current ones."""
    path = os.path.join(PROFILES, f"{kernel_key}_pmc.json")
    if not os.path.exists(path):
        return None, "no committed --pmc summary"
    with open(path) as f:
        rec = json.load(f)
    want = sources_sha16(rel_paths)
    if rec.get("sources_sha16") != want:
        return None, f"stale: profiles/{kernel_key}_pmc.json measured sources {rec.get('sources_sha16')}, now {want}"
    return rec.get("hbm_bytes_per_launch"), f"profiles/{kernel_key}_pmc.json (sources {want}, {rec.get('head', '?')})"


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _timed_reps(fn, sample_s, min_reps=2, max_reps=50):
    fn()  # warm
    times = []
    t_end = time.perf_counter() + sample_s
    while len(times) < min_reps or (time.perf_counter() < t_end and len(times) < max_reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


def cpu_baseline_prefill(w, calls, flops, what, sample_s=12.0):
    """The reference CPU path (per-sequence gather + SDPA) on prefill calls, in the workload dtype."""
    import torch

    from oracle import sdpa_path

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)

    def run():
        for q, meta in calls:
            sdpa_path.paged_prefill(q, w.k_pool, w.v_pool, meta.raw_cu_seqlens, meta.raw_block_tables,
                                    meta.kv_lens.tolist(), meta.positions)

    t, reps = _timed_reps(run, sample_s)
    return {
        "value": round(flops / t / 1e12, 4),
        "unit": "TFLOP/s",
        "median_ms": round(t * 1e3, 2),
        "cores": threads,
        "kind": "port",
        "cpu_model": cpu_model(),
        "sample": f"{what}, {reps} reps, median {t * 1e3:.1f} ms; per-sequence block gather + torch SDPA, "
                  f"{str(w.dtype).replace('torch.', '')}",
    }


def cpu_baseline_decode(w, sample_s=12.0):
    """The reference CPU path on the decode batch, bf16, all host threads."""
    import torch

    from oracle import sdpa_path
    from femtovllm import workloads

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    q, meta = w.gemv_call(device="cpu")
    args = (q, w.k_pool, w.v_pool, meta.raw_block_tables, meta.kv_lens.tolist())
    sdpa_path.paged_decode(*args)  # warm
    times = []
    t_end = time.perf_counter() + sample_s
    while len(times) < 3 or (time.perf_counter() < t_end and len(times) < 50):
        t0 = time.perf_counter()
        sdpa_path.paged_decode(*args)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    nbytes = workloads.decode_bytes(w)
    return {
        "value": round(nbytes / t / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "cpu_model": cpu_model(),
        "sample": f"whole decode batch (64 seqs), {len(times)} reps, median {t * 1e3:.1f} ms; "
                  "per-sequence block gather + torch SDPA, bf16",
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(
            f"bench.py: --gpus {args.gpus} is not supported: the attention path is measured on one GPU "
            "(the reference engine is single-GPU; across GPUs the path shards by KV head or by sequence "
            "with no exchange inside attention).",
            file=sys.stderr,
        )
        sys.exit(2)

    import torch

    from femtovllm import ops, workloads
    from femtovllm import _C

    dev = torch.device("cuda:0")
    timer = Timer(torch, dev)
    K, W = args.steps, args.warmup
    extra = []
    result = None

    def want(name):
        return args.only in ("all", name)

    # ---------------- headline: decode ------------------------------------
    if want("decode"):
        w = workloads.decode_bf16_qwen3_0p6b(poison=False)
        wd = w.to(dev)
        q, meta = wd.gemv_call(device=dev)
        fn = lambda: ops.paged_attention_gemv(q, wd.k_pool, wd.v_pool, meta.block_tables, meta.kv_lens,
                                              meta.max_kv_len)
        out = fn()
        torch.cuda.synchronize()
        assert not torch.isnan(out.float()).any(), "decode produced NaN"
        mean_ms, med_ms, wall = timer.run(fn, K, W)
        wf_ms, _, _ = timer.run(fn, K, 1, write_flush=True)
        prev = _C._lib.femto_attn_set_decode_single_max_kv(1 << 30)
        try:
            one_launch_ms, _, _ = timer.run(fn, K, W)
        finally:
            _C._lib.femto_attn_set_decode_single_max_kv(prev)
        nbytes = workloads.decode_bytes(w)
        gbs = nbytes / (mean_ms * 1e-3) / 1e9
        traffic, traffic_source = pmc_traffic("paged_decode_bf16_qwen3_0.6b_b64", DECODE_SOURCES)
        result = {
            "metric": "paged decode attention HBM bandwidth (bf16, Qwen3-0.6B shape, B=64, ctx U[256,4096])",
            "value": round(gbs, 2),
            "unit": "GB/s",
            "n_gpus": 1,
            "steps": K,
            "warmup": W,
            "ms_per_step": round(mean_ms, 5),
            "higher_is_better": True,
            "scaling": "weak",
            "vs_baseline": None,
            "dtype": "bf16",
            "data": "synthetic (seeded N(0,1) q/k/v, random block placement)",
            "config": {
                "workload": "paged_decode_bf16_qwen3_0.6b_b64_ctx256-4096",
                "num_seqs": 64,
                "n_heads": 16,
                "n_kv_heads": 8,
                "head_dim": 128,
                "block_size": 16,
                "total_kv_tokens": int(meta.kv_lens.sum().item()),
                "pool_blocks": int(w.k_pool.shape[0]),
                "parallelism": "single GPU",
            },
            "roofline": {
                "bound": "hbm",
                "achieved": round(gbs, 2),
                "peak": HBM_PEAK_GBS,
                "unit": "GB/s",
                "frac": round(gbs / HBM_PEAK_GBS, 4),
                "traffic": traffic,
                "traffic_source": traffic_source,
                "algorithmic_bytes_per_launch": nbytes,
                "kernel": "paged_decode_kernel<BF16,2> + paged_decode_merge_kernel<BF16> (both inside the timed region)",
            },
            "median_ms_per_step": round(med_ms, 5),
            "ms_per_step_write_flush": round(wf_ms, 5),
            "ms_per_step_one_launch_route": round(one_launch_ms, 5),
            "wall_s_timed_region": round(wall, 3),
        }
        del wd
        if not args.no_cpu_baseline:
            result["cpu_baseline"] = cpu_baseline_decode(w)
        del w

    # ---------------- small decode calls (latency) ---------------------------
    if want("decode_small"):
        # The reference's CPU-runnable case: fp32, 4 sequences, contexts
        # {17, 64, 200, 511}, and a 64-sequence step of short contexts; both
        # launch-bound (a few MB), so reported as latency.  Each is timed on
        # both decode routes (one launch; split workers + merge) as well as
        # with the library's default choice, which picks the route by
        # max_kv_len.
        def route_ms(fn, limit):
            prev = _C._lib.femto_attn_set_decode_single_max_kv(limit)
            try:
                return timer.run(fn, K, W)[0]
            finally:
                _C._lib.femto_attn_set_decode_single_max_kv(prev)

        for name, make in (("paged_decode_fp32_4seqs_ctx17-511_h16_kv8", workloads.decode_fp32_small),
                           ("paged_decode_bf16_64seqs_ctx64-512_h16_kv8", workloads.decode_bf16_short)):
            w = make(poison=False)
            wd = w.to(dev)
            q, meta = wd.gemv_call(device=dev)
            fn = lambda: ops.paged_attention_gemv(q, wd.k_pool, wd.v_pool, meta.block_tables, meta.kv_lens,
                                                  meta.max_kv_len)
            mean_ms, med_ms, _ = timer.run(fn, K, W)
            nbytes = workloads.decode_bytes(w)
            gbs = nbytes / (mean_ms * 1e-3) / 1e9
            extra.append({
                "workload": name, "metric": "ms per call",
                "value": round(mean_ms, 5), "median_ms": round(med_ms, 5),
                "max_kv_len": int(meta.max_kv_len),
                "ms_one_launch": round(route_ms(fn, 1 << 30), 5), "ms_split_plus_merge": round(route_ms(fn, -1), 5),
                "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                             "frac": round(gbs / HBM_PEAK_GBS, 4), "algorithmic_bytes_per_launch": nbytes,
                             "note": "latency-bound: a few MB per call"},
            })
            del wd, w

    # ---------------- prefill: 8 x 512 chunks -----------------------------
    if want("prefill"):
        w = workloads.prefill_bf16_chunked(poison=False)
        wd = w.to(dev)
        q, meta = wd.gemm_call(device=dev)
        fn = lambda: ops.paged_attention_gemm(q, wd.k_pool, wd.v_pool, meta.cu_seqlens, meta.max_q_len,
                                              meta.Q_TILE_SIZE, meta.cu_q_tiles, meta.q_tile_to_seq_idx,
                                              meta.block_tables, meta.kv_lens, meta.positions)
        mean_ms, med_ms, _ = timer.run(fn, K, W)
        flops = workloads.prefill_flops(w.chunks, w.n_heads, w.head_dim)
        tf = flops / (mean_ms * 1e-3) / 1e12
        rec = {
            "workload": "chunked_prefill_bf16_8x512_prefix0-2048_h16_kv8",
            "metric": "TFLOP/s (causal-exact)", "value": round(tf, 2), "ms": round(mean_ms, 5),
            "roofline": {"bound": "mfma", "achieved": round(tf, 2), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(tf / BF16_PEAK_TFLOPS, 4), "algorithmic_flops_per_launch": flops},
        }
        del wd
        if not args.no_cpu_baseline:
            qc, mc = w.gemm_call(device="cpu")
            rec["cpu_baseline"] = cpu_baseline_prefill(w, [(qc, mc)], flops, "the whole 8 x 512 batch")
        extra.append(rec)
        del w

        # Uneven batch (fewer query tiles than resident workgroups): the key
        # split balances it; the same call without a workspace runs unsplit.
        w = workloads.prefill_bf16_uneven(poison=False)
        wd = w.to(dev)
        q, meta = wd.gemm_call(device=dev)
        fn = lambda: ops.paged_attention_gemm(q, wd.k_pool, wd.v_pool, meta.cu_seqlens, meta.max_q_len,
                                              meta.Q_TILE_SIZE, meta.cu_q_tiles, meta.q_tile_to_seq_idx,
                                              meta.block_tables, meta.kv_lens, meta.positions)
        mean_ms, med_ms, _ = timer.run(fn, K, W)
        with_ws = _C._prefill_workspace
        _C._prefill_workspace = lambda *args: (None, 0)
        try:
            mean_unsplit, _, _ = timer.run(fn, K, W)
        finally:
            _C._prefill_workspace = with_ws
        flops = workloads.prefill_flops(w.chunks, w.n_heads, w.head_dim)
        tf = flops / (mean_ms * 1e-3) / 1e12
        extra.append({
            "workload": "chunked_prefill_bf16_uneven4_h16_kv8",
            "metric": "TFLOP/s (causal-exact)", "value": round(tf, 2), "ms": round(mean_ms, 5),
            "ms_without_key_split": round(mean_unsplit, 5),
            "roofline": {"bound": "mfma", "achieved": round(tf, 2), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(tf / BF16_PEAK_TFLOPS, 4), "algorithmic_flops_per_launch": flops},
        })
        del wd, w

    # ---------------- long context: 16 x 2048 chunks ----------------------
    if want("long"):
        w = workloads.prefill_bf16_long_llama3_8b(poison=False)
        wd = w.to(dev)
        calls = []
        for c in range(16):
            q, meta = workloads.long_context_chunk(wd, c, device=dev)
            calls.append((q, meta))

        def fn():
            for q, meta in calls:
                ops.paged_attention_gemm(q, wd.k_pool, wd.v_pool, meta.cu_seqlens, meta.max_q_len, meta.Q_TILE_SIZE,
                                         meta.cu_q_tiles, meta.q_tile_to_seq_idx, meta.block_tables, meta.kv_lens,
                                         meta.positions)

        steps = max(1, K // 4)
        mean_ms, med_ms, _ = timer.run(fn, steps, max(1, W // 2))
        flops = workloads.prefill_flops([(2048 * c, 2048) for c in range(16)], 32, 128)
        tf = flops / (mean_ms * 1e-3) / 1e12
        rec = {
            "workload": "long_context_prefill_bf16_llama3_8b_32k_as_16x2048",
            "metric": "TFLOP/s (causal-exact, 16 calls)", "value": round(tf, 2), "ms": round(mean_ms, 4),
            "roofline": {"bound": "mfma", "achieved": round(tf, 2), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(tf / BF16_PEAK_TFLOPS, 4), "algorithmic_flops_per_step": flops},
        }
        del wd, calls
        if not args.no_cpu_baseline:
            # one chunk (2048 tokens after a 14336-token prefix), all 32 heads
            c = 7
            qc, mc = workloads.long_context_chunk(w, c, device="cpu")
            cflops = workloads.prefill_flops([(2048 * c, 2048)], 32, 128)
            rec["cpu_baseline"] = cpu_baseline_prefill(w, [(qc, mc)], cflops,
                                                       "chunk 7 of 16 (2048 tokens on a 14336-token prefix)",
                                                       sample_s=15.0)
        extra.append(rec)
        del w

        # One GPU's share of the same job under 8-way tensor parallelism (4 query
        # heads, 1 KV head): 64 query tiles per chunk for 512 resident workgroups,
        # the case the key split is for; also timed without it.
        w = workloads.prefill_bf16_long_tp8_share(poison=False)
        wd = w.to(dev)
        calls = [workloads.long_context_chunk(wd, c, device=dev) for c in range(16)]

        def fn():
            for q, meta in calls:
                ops.paged_attention_gemm(q, wd.k_pool, wd.v_pool, meta.cu_seqlens, meta.max_q_len, meta.Q_TILE_SIZE,
                                         meta.cu_q_tiles, meta.q_tile_to_seq_idx, meta.block_tables, meta.kv_lens,
                                         meta.positions)

        mean_ms, _, _ = timer.run(fn, steps, max(1, W // 2))
        with_ws = _C._prefill_workspace
        _C._prefill_workspace = lambda *args: (None, 0)
        try:
            mean_unsplit, _, _ = timer.run(fn, steps, max(1, W // 2))
        finally:
            _C._prefill_workspace = with_ws
        flops = workloads.prefill_flops([(2048 * c, 2048) for c in range(16)], 4, 128)
        tf = flops / (mean_ms * 1e-3) / 1e12
        extra.append({
            "workload": "long_context_prefill_bf16_llama3_8b_32k_tp8_share_h4_kv1",
            "metric": "TFLOP/s (causal-exact, 16 calls)", "value": round(tf, 2), "ms": round(mean_ms, 4),
            "ms_without_key_split": round(mean_unsplit, 4),
            "roofline": {"bound": "mfma", "achieved": round(tf, 2), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(tf / BF16_PEAK_TFLOPS, 4), "algorithmic_flops_per_step": flops},
        })
        del wd, w, calls

    # ---------------- unified mixed batch ---------------------------------
    if want("mixed"):
        def mixed_entry(w, name, cpu):
            """Both routes of a unified batch: sequence 0 a prefill chunk, the rest decode rows."""
            n = len(w.chunks)
            wd = w.to(dev)
            qp, mp = wd.gemm_call(seqs=[0], device=dev)
            qd, md = wd.gemv_call(seqs=range(1, n), device=dev)
            qa, ma = wd.gemm_call(device=dev)

            def route_split():
                ops.paged_attention_gemm(qp, wd.k_pool, wd.v_pool, mp.cu_seqlens, mp.max_q_len, mp.Q_TILE_SIZE,
                                         mp.cu_q_tiles, mp.q_tile_to_seq_idx, mp.block_tables, mp.kv_lens,
                                         mp.positions)
                ops.paged_attention_gemv(qd, wd.k_pool, wd.v_pool, md.block_tables, md.kv_lens, md.max_kv_len)

            def route_unified():
                ops.paged_attention_gemm(qa, wd.k_pool, wd.v_pool, ma.cu_seqlens, ma.max_q_len, ma.Q_TILE_SIZE,
                                         ma.cu_q_tiles, ma.q_tile_to_seq_idx, ma.block_tables, ma.kv_lens,
                                         ma.positions)

            ms_split, _, _ = timer.run(route_split, K, W)
            ms_uni, _, _ = timer.run(route_unified, K, W)
            dec_bytes = workloads.decode_bytes(w, seqs=range(1, n))
            dec_bytes_logical = workloads.decode_bytes(w, seqs=range(1, n), unique_blocks=False)
            flops = workloads.prefill_flops([w.chunks[0]], w.n_heads, w.head_dim)
            # Floors: the decode rows' unique bytes at 8 TB/s and the prefill
            # chunk's FLOPs at 2.5 PFLOP/s, overlapped (max) or one after the
            # other (sum).
            t_hbm = dec_bytes / (HBM_PEAK_GBS * 1e9) * 1e3
            t_mfma = flops / (BF16_PEAK_TFLOPS * 1e12) * 1e3

            def route(ms):
                gbs_u = dec_bytes / (ms * 1e-3) / 1e9
                gbs_l = dec_bytes_logical / (ms * 1e-3) / 1e9
                tf = flops / (ms * 1e-3) / 1e12
                return {"ms": round(ms, 4),
                        "roofline": {"bound": "hbm", "achieved": round(gbs_u, 1), "peak": HBM_PEAK_GBS,
                                     "unit": "GB/s", "frac": round(gbs_u / HBM_PEAK_GBS, 4),
                                     "achieved_logical_GBs": round(gbs_l, 1),
                                     "frac_logical": round(gbs_l / HBM_PEAK_GBS, 4),
                                     "prefill_tflops": round(tf, 1),
                                     "prefill_frac_mfma": round(tf / BF16_PEAK_TFLOPS, 4),
                                     "floor_ms_overlapped": round(max(t_hbm, t_mfma), 4),
                                     "floor_ms_serial": round(t_hbm + t_mfma, 4),
                                     "frac_of_overlapped_floor": round(max(t_hbm, t_mfma) / ms, 4)}}

            rec = {
                "workload": name,
                "metric": "ms per step (both routes)", "value": round(ms_uni, 4),
                "headline_route": "single_gemm_call" if ms_uni <= ms_split else "prefill_plus_decode",
                "routes": {
                    "single_gemm_call": {**route(ms_uni), "what": f"one paged_attention_gemm over all {n} sequences "
                                         "(the CUSTOM_GEMM route); decode rows on decode wave workers"},
                    "prefill_plus_decode": {**route(ms_split), "what": "paged_attention_gemm on sequence 0, then "
                                            f"paged_attention_gemv on sequences 1-{n - 1} (the default routed engine)"},
                },
                "prefill_flops": flops, "decode_unique_bytes": dec_bytes, "decode_logical_bytes": dec_bytes_logical,
            }
            del wd
            if cpu and not args.no_cpu_baseline:
                qc, mc = w.gemm_call(device="cpu")
                cb = cpu_baseline_prefill(w, [(qc, mc)], flops, f"the whole {n}-sequence batch in one call")
                t_cpu = cb["median_ms"] * 1e-3
                rec["cpu_baseline"] = {**cb, "value": cb["median_ms"], "unit": "ms per step",
                                       "prefill_tflops": cb["value"],
                                       "decode_unique_GBs": round(dec_bytes / t_cpu / 1e9, 3)}
            return rec

        w = workloads.mixed_bf16_qwen3_8b(poison=False)
        extra.append(mixed_entry(w, "mixed_bf16_qwen3_8b_1x1024on4096_plus_127_decode", cpu=True))
        del w
        # One GPU's share of the same batch under 8-way tensor parallelism.
        w = workloads.mixed_bf16_qwen3_8b_tp8_share(poison=False)
        extra.append(mixed_entry(w, "mixed_bf16_qwen3_8b_tp8_share_h4_kv1", cpu=False))
        del w

    # ---------------- dense flash attention (reference benchmark shapes) --
    if want("flash"):
        lat = {}
        for T in (16, 32, 64, 128, 256):
            g = torch.Generator().manual_seed(T)
            qkv = [torch.randn((2, 4, T, 128), generator=g).half().to(dev) for _ in range(3)]
            fn = lambda: _C.FlashAttentionWarpCuda(*qkv)
            mean_ms, _, _ = timer.run(fn, K, W)
            lat[str(T)] = round(mean_ms, 5)
        extra.append({"workload": "dense_flash_attention_fp16_B2_H4_D128_noncausal", "ms_by_seq_len": lat})

        # The dense entry at the long-context chunk shapes (q: 2048 tokens x 32
        # heads, k/v: 8 KV heads), bf16, non-causal: FLOPs = 4 B H Tq Tkv D.
        tf_by_kv = {}
        for tkv in (2048, 8192, 32768):
            g = torch.Generator().manual_seed(tkv)
            q = torch.randn((1, 32, 2048, 128), generator=g).to(torch.bfloat16).to(dev)
            k = torch.randn((1, 8, tkv, 128), generator=g).to(torch.bfloat16).to(dev)
            v = torch.randn((1, 8, tkv, 128), generator=g).to(torch.bfloat16).to(dev)
            fn = lambda: _C.FlashAttentionWarpCuda(q, k, v)
            mean_ms, _, _ = timer.run(fn, K, W)
            tf_by_kv[str(tkv)] = round(4 * 32 * 2048 * tkv * 128 / (mean_ms * 1e-3) / 1e12, 1)
            del q, k, v
        extra.append({"workload": "dense_flash_attention_bf16_B1_H32_KV8_Tq2048_noncausal",
                      "metric": "TFLOP/s by kv length", "tflops_by_kv_len": tf_by_kv,
                      "peak": BF16_PEAK_TFLOPS})

    # ---------------- KV-cache write (prefill chunk and decode step) --------
    if want("cache"):
        w = workloads.prefill_bf16_chunked(poison=False)
        wd = w.to(dev)
        _, meta = wd.gemm_call(device=dev)
        T = meta.positions.numel()
        g = torch.Generator().manual_seed(7)
        k_new = torch.randn((T, 8, 128), generator=g).to(torch.bfloat16).to(dev)
        v_new = torch.randn((T, 8, 128), generator=g).to(torch.bfloat16).to(dev)
        fn = lambda: ops.kv_cache_write(k_new, v_new, wd.k_pool, wd.v_pool, meta.positions, meta.block_tables,
                                        cu_seqlens=meta.cu_seqlens, max_q_len=meta.max_q_len)
        mean_ms, _, _ = timer.run(fn, K, W)
        nbytes = 2 * 2 * k_new.numel() * k_new.element_size()  # K and V, read once and written once
        gbs = nbytes / (mean_ms * 1e-3) / 1e9
        extra.append({
            "workload": "kv_cache_write_bf16_8x512_kv8_d128", "metric": "GB/s (read + write)",
            "value": round(gbs, 1), "ms": round(mean_ms, 5),
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4), "algorithmic_bytes_per_launch": nbytes},
        })
        del wd, w
        w = workloads.decode_bf16_qwen3_0p6b(poison=False)
        wd = w.to(dev)
        _, dmeta = wd.gemv_call(device=dev)
        B = dmeta.kv_lens.numel()
        pos = (dmeta.kv_lens - 1).contiguous()
        kd1, vd1 = k_new[:B].contiguous(), v_new[:B].contiguous()
        fn = lambda: ops.kv_cache_write(kd1, vd1, wd.k_pool, wd.v_pool, pos, dmeta.block_tables)
        mean_ms, _, _ = timer.run(fn, K, W)
        extra.append({"workload": f"kv_cache_write_bf16_decode_{B}seqs_kv8_d128", "ms": round(mean_ms, 5)})
        del wd, w

        # fused prologue: q/k RMSNorm + RoPE + cache write, same 8 x 512 chunk, 16 q heads
        from femtovllm.rope import rope_tables
        w = workloads.prefill_bf16_chunked(poison=False)
        wd = w.to(dev)
        _, meta = wd.gemm_call(device=dev)
        T = meta.positions.numel()
        q_new = torch.randn((T, 16, 128), generator=g).to(torch.bfloat16).to(dev)
        wq = (1 + 0.1 * torch.randn(128, generator=g)).to(torch.bfloat16).to(dev)
        wk = (1 + 0.1 * torch.randn(128, generator=g)).to(torch.bfloat16).to(dev)
        cos, sin = rope_tables(8192, 128, device=dev)
        q_out = torch.empty_like(q_new)
        fn = lambda: ops.qk_norm_rope_cache_write(q_new, k_new, v_new, wq, wk, 1e-6, cos, sin, meta.positions,
                                                  wd.k_pool, wd.v_pool, meta.block_tables,
                                                  cu_seqlens=meta.cu_seqlens, max_q_len=meta.max_q_len, out=q_out)
        mean_ms, _, _ = timer.run(fn, K, W)
        # q, k, v read once, the rope rows of every token read once, q out + k, v into the pools written once
        esz = q_new.element_size()
        nbytes = 2 * (q_new.numel() + 2 * k_new.numel()) * esz + 2 * T * 128 * 4
        gbs = nbytes / (mean_ms * 1e-3) / 1e9
        extra.append({
            "workload": "qk_norm_rope_cache_write_bf16_8x512_h16_kv8_d128", "metric": "GB/s (read + write)",
            "value": round(gbs, 1), "ms": round(mean_ms, 5),
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4), "algorithmic_bytes_per_launch": nbytes},
        })
        del wd, w

    # ---------------- plain device copy (counter calibration, not in "all") --
    if args.only == "copy":
        src = torch.ones(1 << 28, dtype=torch.float32, device=dev)  # 1 GiB
        dst = torch.empty_like(src)
        mean_ms, _, _ = timer.run(lambda: dst.copy_(src), K, W)
        extra.append({"workload": "device_copy_1GiB", "ms": round(mean_ms, 4),
                      "GBs_read_plus_write": round(2 * (1 << 30) / (mean_ms * 1e-3) / 1e9, 1)})

    if result is None:
        result = {"metric": f"bench subset '{args.only}'", "value": None, "unit": None, "n_gpus": 1, "steps": K,
                  "warmup": W}
    result["extra"] = extra
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
