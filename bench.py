#!/usr/bin/env python3
"""Benchmark of the PAL paged-attention path on one MI355X.

Default workload ("config 2"): Llama-3-8B-shaped
bf16 decode -- 64 sequences with context lengths drawn U[512, 4096], 32 query
heads / 8 KV heads, head_dim 128, 16-token pages, a randomly permuted page
table over a pool sized to the tokens plus 10 % free pages, N(0,1) values.
One step = fill_kv_pages of each sequence's newest token (64 tokens) followed
by paged_attention_decode of the 64 queries.

Prints one JSON line: value = algorithmic HBM bytes of the step / step time
(GB/s), plus tokens/s, the decode kernel's roofline fraction measured live
with HIP events, and a CPU baseline (the numpy oracle on the host cores, on a
bounded sample).  Several independent copies of the workload are rotated so
that consecutive steps never hit in the 256 MB last-level cache.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c2]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "proxy-attention-lab_amd"))

import proxy_attention_lab as pal  # noqa: E402

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
METRIC = json.loads((ROOT / "BASELINE.json").read_text())["metric"] if (ROOT / "BASELINE.json").exists() else \
    "decode HBM GB/s (% of peak) + tokens/s; prefill TFLOP/s (% MFMA peak)"


# ---------------------------------------------------------------------------
# workloads
# ---------------------------------------------------------------------------


class DecodeWorkload:
    """Config 2 (or a variant): pools, page table, queries and the fill step's inputs."""

    def __init__(self, seed: int, num_seqs=64, ctx_lo=512, ctx_hi=4096, hq=32, hkv=8, hd=128, tpp=16,
                 dtype=torch.bfloat16, device="cuda:0"):
        rng = np.random.default_rng(1000 + seed)
        lens = rng.integers(ctx_lo, ctx_hi + 1, size=num_seqs).astype(np.int32)
        pages_per_seq = (lens + tpp - 1) // tpp
        used = int(pages_per_seq.sum())
        num_pages = used + int(math.ceil(0.1 * used))
        perm = rng.permutation(num_pages).astype(np.int32)
        width = int(pages_per_seq.max())
        pt = np.zeros((num_seqs, width), np.int32)
        cur = 0
        for s, n in enumerate(pages_per_seq):
            pt[s, :n] = perm[cur:cur + n]
            cur += n
        g = torch.Generator(device=device)
        g.manual_seed(2000 + seed)
        self.lens_np, self.pt_np = lens, pt
        self.num_seqs, self.hq, self.hkv, self.hd, self.tpp = num_seqs, hq, hkv, hd, tpp
        self.dtype = dtype
        self.k_pool = torch.randn(pal.get_k_cache_shape(num_pages, hkv, hd, tpp, dtype), generator=g,
                                  device=device, dtype=torch.float32).to(dtype)
        self.v_pool = torch.randn(pal.get_v_cache_shape(num_pages, hkv, hd, tpp, dtype), generator=g,
                                  device=device, dtype=torch.float32).to(dtype)
        self.page_table = torch.from_numpy(pt).to(device)
        self.seq_lens = torch.from_numpy(lens).to(device)
        self.queries = torch.randn((num_seqs, hq, hd), generator=g, device=device, dtype=torch.float32).to(dtype)
        # fill step: the newest token (position len-1) of every sequence
        self.new_k = torch.randn((num_seqs, hkv, hd), generator=g, device=device, dtype=torch.float32).to(dtype)
        self.new_v = torch.randn((num_seqs, hkv, hd), generator=g, device=device, dtype=torch.float32).to(dtype)
        self.write_pos = torch.from_numpy(lens - 1).to(device)
        self.q2seq = torch.arange(num_seqs, dtype=torch.int32, device=device)

    def fill(self):
        pal.fill_kv_pages(self.new_k, self.new_v, self.k_pool, self.v_pool, self.page_table, self.write_pos,
                          self.q2seq)

    def decode(self, partition_size: int = 0):
        return pal.paged_attention_decode(self.queries, self.k_pool, self.v_pool, self.page_table, self.seq_lens,
                                          partition_size=partition_size)

    # algorithmic bytes (each byte the operation must move at least once)
    def decode_bytes(self) -> int:
        el = 2
        kv = int(self.lens_np.astype(np.int64).sum()) * 2 * self.hkv * self.hd * el
        qo = 2 * self.num_seqs * self.hq * self.hd * el
        return kv + qo

    def fill_bytes(self) -> int:
        return 2 * self.num_seqs * self.hkv * self.hd * 2 * 2  # K and V: read new rows + write pool slots


# ---------------------------------------------------------------------------
# CPU baseline: the numpy oracle on a bounded sample of the same workload
# ---------------------------------------------------------------------------


def cpu_baseline(w: DecodeWorkload, budget_s: float = 12.0) -> dict:
    from oracle import pal_oracle as orc  # the checker, used here only as the timed CPU baseline

    try:
        from threadpoolctl import threadpool_info

        cores = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
    except Exception:  # pragma: no cover
        cores = os.cpu_count() or 1
    dt = "bf16"
    q = w.queries.view(torch.int16).cpu().numpy().view(np.uint16)
    kb = w.k_pool.view(torch.int16).cpu().numpy().view(np.uint16)
    vb = w.v_pool.view(torch.int16).cpu().numpy().view(np.uint16)
    # sample: the first 8 sequences (their pages only), repeated until the time budget is used
    ns = 8
    lens = w.lens_np[:ns]
    used = np.concatenate([w.pt_np[s, : (int(n) + w.tpp - 1) // w.tpp] for s, n in enumerate(lens)])
    kb, vb = kb[used], vb[used]
    pt = np.zeros((ns, w.pt_np.shape[1]), np.int32)
    cur = 0
    for s, n in enumerate(lens):
        npg = (int(n) + w.tpp - 1) // w.tpp
        pt[s, :npg] = np.arange(cur, cur + npg)
        cur += npg
    t0 = time.perf_counter()
    reps = 0
    while True:
        orc.paged_attention_decode(q[:ns], kb, vb, pt, lens, dt)
        reps += 1
        if time.perf_counter() - t0 > budget_s:
            break
    el = (time.perf_counter() - t0) / reps
    kv_bytes = int(lens.astype(np.int64).sum()) * 2 * w.hkv * w.hd * 2 + 2 * ns * w.hq * w.hd * 2
    return {
        "value": round(kv_bytes / el / 1e9, 3),
        "unit": "GB/s",
        "tokens_per_s": round(ns / el, 2),
        "cores": int(cores),
        "kind": "port",
        "sample": f"numpy oracle (bf16->fp32 decode of the sample's pages, gather, fp32 softmax attention) on "
                  f"{ns} of the 64 config-2 sequences ({int(lens.sum())} context tokens), {reps} reps in "
                  f"{el * reps:.1f} s; fill step not included",
    }


# ---------------------------------------------------------------------------
# main
# ---------------------------------------------------------------------------


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--rotate", type=int, default=4, help="independent workload copies cycled per step")
    ap.add_argument("--partition", type=int, default=0, help="decode partition size (0 = library default)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=12.0)
    ap.add_argument("--calibrate-copy-mib", type=int, default=0,
                    help="before the timed loop, run one device-to-device copy of this many MiB (a kernel of "
                         "known traffic for scaling rocprof FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the operators shard by KV head or sequence with no exchange; see DESIGN.md)", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        return 1

    dev = torch.device("cuda:0")
    if args.calibrate_copy_mib > 0:
        n = args.calibrate_copy_mib * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    works = [DecodeWorkload(seed=i) for i in range(max(1, args.rotate))]
    w0 = works[0]
    torch.cuda.synchronize()

    def step(w):
        w.fill()
        return w.decode(args.partition)

    for i in range(args.warmup):
        step(works[i % len(works)])
    torch.cuda.synchronize()

    stream = torch.cuda.current_stream(dev)
    ev_start = torch.cuda.Event(enable_timing=True)
    ev_end = torch.cuda.Event(enable_timing=True)
    dec_ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev_start.record(stream)
    for i in range(args.steps):
        w = works[i % len(works)]
        w.fill()
        dec_ev[i][0].record(stream)
        w.decode(args.partition)
        dec_ev[i][1].record(stream)
    ev_end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = ev_start.elapsed_time(ev_end)
    ms_per_step = max(gpu_ms, wall * 1e3) / args.steps
    dec_ms = float(np.mean([a.elapsed_time(b) for a, b in dec_ev]))

    step_bytes = float(np.mean([w.decode_bytes() + w.fill_bytes() for w in works]))
    dec_bytes = float(np.mean([w.decode_bytes() for w in works]))
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    dec_gbs = dec_bytes / (dec_ms * 1e-3) / 1e9

    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "config 2: Llama-3-8B-shaped bf16 decode step (fill_kv_pages of 64 new tokens + "
                        "paged_attention_decode)",
            "num_seqs": w0.num_seqs, "ctx": "U[512,4096]", "num_q_heads": w0.hq, "num_kv_heads": w0.hkv,
            "head_dim": w0.hd, "tokens_per_page": w0.tpp, "rotated_copies": len(works),
            "partition_size": args.partition or 512,
        },
        "tokens_per_s": round(w0.num_seqs / (ms_per_step * 1e-3), 1),
        "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "roofline": {
            "kernel": "paged_attention_decode (split-K partition kernel + LSE merge kernel)",
            "bound": "hbm",
            "achieved": round(dec_gbs, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(dec_gbs / HBM_PEAK_GBS, 4),
            "traffic": None,
            "algorithmic_bytes_per_launch": int(dec_bytes),
            "avg_launch_ms": round(dec_ms, 5),
        },
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(w0, args.cpu_budget)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
