#!/usr/bin/env python3
"""Benchmark of the PAL paged-attention path on one MI355X.

Headline workload ("config 2"): Llama-3-8B-shaped
bf16 decode -- 64 sequences with context lengths drawn U[512, 4096], 32 query
heads / 8 KV heads, head_dim 128, 16-token pages, a randomly permuted page
table over a pool sized to the tokens plus 10 % free pages, N(0,1) values.
One step = fill_kv_pages of each sequence's newest token (64 tokens) followed
by paged_attention_decode of the 64 queries.  value = algorithmic HBM bytes
of the step / step time (GB/s); the roofline object is the decode operator's
(its algorithmic bytes / its average duration from HIP events).  Several
independent copies of the workload are rotated so that consecutive steps
never hit in the 256 MB last-level cache.

The other configs are reported beside it, each in its own object:
  c3  long-context split-K decode (8 x U[32768, 131072] tokens, 1 % of key
      rows x8, partition 512 + log-sum-exp merge, and the default split)
  c4  chunked causal prefill: fill_kv_pages of the new chunks, then causal
      attention of the new rows over cached + new (fused operator), TFLOP/s
      over causal-valid pairs only
  c5  fused mixed batch, fp16: 256 decode rows + 4 prefill chunks of 1024
      rows, interleaved in shuffled row blocks, one operator call
  lh  batch-1 decode over 131,072 / 524,288 / 1,048,576-token histories
      (the reference benchmark's range), 32/16 heads, HD 128, bf16
  pages  (not in the default run) config 2's decode at head dims 64, 128
      and 256 over 16- and 32-token pages, 16-bit and fp8 pools, both split
      forms, each over 4 rotated copies; config 4's attention at the same
      head dims and page sizes over 3 rotated copies
  shapes  (not in the default run) bf16 decode, HD 128, 16-token pages,
      across batch shapes and GQA groups, both split forms
The CPU baseline is the reference's equivalency computation (gather pages +
fp32 softmax attention) on torch CPU over the host cores: configs 1 and 2 in
full, configs 3-5 on a stated subsample scaled by its share of the work.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--configs c2,c3,c4,c5,lh]
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


def paged_pool(rng: np.random.Generator, g: torch.Generator, lens: np.ndarray, hkv: int, hd: int, tpp: int,
               dtype: torch.dtype, device, free_frac: float = 0.1):
    """Pools of N(0,1) values with room for `lens` tokens per sequence plus
    free pages, and a randomly permuted page table (numpy int32 [S, W])."""
    pages_per_seq = (lens.astype(np.int64) + tpp - 1) // tpp
    used = int(pages_per_seq.sum())
    num_pages = max(1, used + int(math.ceil(free_frac * used)))
    perm = rng.permutation(num_pages).astype(np.int32)
    pt = np.zeros((len(lens), max(1, int(pages_per_seq.max()))), np.int32)
    cur = 0
    for s, n in enumerate(pages_per_seq):
        pt[s, :n] = perm[cur:cur + n]
        cur += n
    k_pool = torch.randn(pal.get_k_cache_shape(num_pages, hkv, hd, tpp, dtype), generator=g, device=device,
                         dtype=torch.float32).to(dtype)
    v_pool = torch.randn(pal.get_v_cache_shape(num_pages, hkv, hd, tpp, dtype), generator=g, device=device,
                         dtype=torch.float32).to(dtype)
    return k_pool, v_pool, pt


def to_fp8_pages(pool: torch.Tensor, headroom: float = 1.5):
    """An fp8 e4m3 copy of a 16-bit pool ([pages, Hkv, ...]) with one scale per
    (page, kv head): amax x headroom / 448.  Returns (codes, scales float32)."""
    p_, h_ = pool.shape[0], pool.shape[1]
    amax = pool.float().abs().reshape(p_, h_, -1).amax(dim=2)
    scales = torch.where(amax > 0, amax * headroom / 448.0, torch.ones_like(amax)).contiguous()
    shape = (p_, h_) + (1,) * (pool.dim() - 2)
    return (pool.float() / scales.view(shape)).clamp(-448, 448).to(torch.float8_e4m3fn), scales


def to_fp8_k_layout(k_pool: torch.Tensor) -> torch.Tensor:
    """16-bit K pool [P, H, HD/8, TPP, 8] -> the fp8 stripe layout's element
    order [P, H, HD/16, TPP, 16] (same values)."""
    p_, h_, c_, t_, x_ = k_pool.shape
    tok = k_pool.permute(0, 1, 3, 2, 4).reshape(p_, h_, t_, c_ * x_)
    return tok.reshape(p_, h_, t_, c_ * x_ // 16, 16).permute(0, 1, 3, 2, 4).contiguous()


def traffic_bytes():
    """HBM bytes per decode call measured by the committed rocprofv3 counter
    passes (FETCH_SIZE scaled by 2, WRITE_SIZE by 1, calibrated on a 1 GiB
    copy) for this workload, or None when that record is absent."""
    f = ROOT / "profiles" / "decode_config2_traffic.json"
    try:
        return int(json.loads(f.read_text())["traffic_bytes_per_launch"])
    except (OSError, ValueError, KeyError):
        return None


def causal_flops(hq: int, hd: int, cached: np.ndarray, new: np.ndarray) -> float:
    """4 * Hq * HD * (causal-valid query/key pairs): QK^T and PV, 2 flops per MAC."""
    c = cached.astype(np.float64)
    n = new.astype(np.float64)
    return float(4.0 * hq * hd * np.sum(n * c + n * (n + 1) / 2))


def time_op(fn, steps: int, warmup: int, stream) -> tuple[float, float]:
    """(mean ms per call, wall ms per call): `steps` back-to-back calls between
    one pair of HIP events on `stream`.  (An event recorded between calls
    costs the GPU an idle gap of a few microseconds, so none is recorded
    inside the timed loop.)"""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    a.record(stream)
    for _ in range(steps):
        fn()
    b.record(stream)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    return a.elapsed_time(b) / steps, wall


class DecodeWorkload:
    """Config 2 (or a variant): pools, page table, queries and the fill step's inputs."""

    def __init__(self, seed: int, num_seqs=64, ctx_lo=512, ctx_hi=4096, hq=32, hkv=8, hd=128, tpp=16,
                 dtype=torch.bfloat16, device="cuda:0"):
        rng = np.random.default_rng(1000 + seed)
        lens = rng.integers(ctx_lo, ctx_hi + 1, size=num_seqs).astype(np.int32)
        g = torch.Generator(device=device)
        g.manual_seed(2000 + seed)
        self.k_pool, self.v_pool, pt = paged_pool(rng, g, lens, hkv, hd, tpp, dtype, device)
        self.lens_np, self.pt_np = lens, pt
        self.num_seqs, self.hq, self.hkv, self.hd, self.tpp = num_seqs, hq, hkv, hd, tpp
        self.dtype = dtype
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

    def make_fp8(self):
        """fp8 e4m3 pages of the same values (per-(page, kv head) scales), beside
        the 16-bit pools."""
        self.k8, self.ks = to_fp8_pages(to_fp8_k_layout(self.k_pool))
        self.v8, self.vs = to_fp8_pages(self.v_pool)

    def fill_fp8(self):
        pal.fill_kv_pages(self.new_k, self.new_v, self.k8, self.v8, self.page_table, self.write_pos, self.q2seq,
                          k_scales=self.ks, v_scales=self.vs)

    def decode_fp8(self, partition_size: int = 0):
        return pal.paged_attention_decode(self.queries, self.k8, self.v8, self.page_table, self.seq_lens,
                                          partition_size=partition_size, k_scales=self.ks, v_scales=self.vs)

    def decode_bytes_fp8(self) -> int:
        """fp8 K/V bytes (1 per element) + their scales + Q and O."""
        ctx = int(self.lens_np.astype(np.int64).sum())
        pages = int(((self.lens_np.astype(np.int64) + self.tpp - 1) // self.tpp).sum())
        return ctx * 2 * self.hkv * self.hd + pages * self.hkv * 2 * 4 + 2 * self.num_seqs * self.hq * self.hd * 2

    # algorithmic bytes (each byte the operation must move at least once)
    def decode_bytes(self) -> int:
        el = 2
        kv = int(self.lens_np.astype(np.int64).sum()) * 2 * self.hkv * self.hd * el
        qo = 2 * self.num_seqs * self.hq * self.hd * el
        return kv + qo

    def fill_bytes(self) -> int:
        return 2 * self.num_seqs * self.hkv * self.hd * 2 * 2  # K and V: read new rows + write pool slots


def long_context_workload(device, seed: int = 3) -> DecodeWorkload:
    """Config 3: 8 sequences x U[32768, 131072] tokens, 32/8 heads, HD 128,
    bf16; 1 % of key rows (token positions, all heads) scaled x8."""
    w = DecodeWorkload(seed, num_seqs=8, ctx_lo=32768, ctx_hi=131072, device=device)
    rng = np.random.default_rng(3000 + seed)
    pages, slots = [], []
    for s, n in enumerate(w.lens_np):
        pos = rng.choice(int(n), size=max(1, int(n) // 100), replace=False)
        pages.append(w.pt_np[s, pos // w.tpp])
        slots.append(pos % w.tpp)
    pi = torch.from_numpy(np.concatenate(pages).astype(np.int64)).to(device)
    si = torch.from_numpy(np.concatenate(slots).astype(np.int64)).to(device)
    w.k_pool[pi, :, :, si, :] = w.k_pool[pi, :, :, si, :] * 8
    return w


class PrefillWorkload:
    """Config 4: 16 sequences, new chunk U[512, 2048] on cached U[0, 2048],
    32/8 heads, HD 128, bf16.  Step 1 writes the new K/V through
    fill_kv_pages; step 2 runs causal attention of the new rows over cached +
    new (the fused operator: each sequence's rows form one run of tiles)."""

    def __init__(self, device, seed: int = 4, num_seqs=16, hq=32, hkv=8, hd=128, tpp=16, dtype=torch.bfloat16):
        rng = np.random.default_rng(4000 + seed)
        self.new = rng.integers(512, 2049, size=num_seqs).astype(np.int32)
        self.cached = rng.integers(0, 2049, size=num_seqs).astype(np.int32)
        lens = self.cached + self.new
        g = torch.Generator(device=device)
        g.manual_seed(5000 + seed)
        self.k_pool, self.v_pool, pt = paged_pool(rng, g, lens, hkv, hd, tpp, dtype, device)
        self.hq, self.hkv, self.hd = hq, hkv, hd
        n = int(self.new.sum())
        self.rows = n
        self.page_table = torch.from_numpy(pt).to(device)
        self.seq_lens = torch.from_numpy(lens).to(device)
        pos = np.concatenate([np.arange(c, c + k) for c, k in zip(self.cached, self.new)]).astype(np.int32)
        q2s = np.repeat(np.arange(num_seqs), self.new).astype(np.int32)
        self.write_pos = torch.from_numpy(pos).to(device)
        self.q2seq = torch.from_numpy(q2s).to(device)
        self.q_offset = torch.from_numpy(pos + 1).to(device)
        self.queries = torch.randn((n, hq, hd), generator=g, device=device, dtype=torch.float32).to(dtype)
        self.new_k = torch.randn((n, hkv, hd), generator=g, device=device, dtype=torch.float32).to(dtype)
        self.new_v = torch.randn((n, hkv, hd), generator=g, device=device, dtype=torch.float32).to(dtype)

    def fill(self):
        pal.fill_kv_pages(self.new_k, self.new_v, self.k_pool, self.v_pool, self.page_table, self.write_pos,
                          self.q2seq)

    def attend(self):
        return pal.paged_attention(self.queries, self.k_pool, self.v_pool, self.page_table, self.seq_lens,
                                   self.q2seq, self.q_offset)

    def flops(self) -> float:
        return causal_flops(self.hq, self.hd, self.cached, self.new)

    def fill_bytes(self) -> int:
        return 2 * self.rows * self.hkv * self.hd * 2 * 2


class FusedWorkload:
    """Config 5: 256 decode rows (ctx U[256, 8192]) + 4 prefill chunks of
    1024 new rows on U[0, 4096] cached tokens, 64/8 heads, HD 128, fp16; rows
    in shuffled blocks (each decode row one block, prefill chunks in blocks
    of 128 rows), one paged_attention call."""

    def __init__(self, device, seed: int = 5, hq=64, hkv=8, hd=128, tpp=16, dtype=torch.float16, block=128):
        rng = np.random.default_rng(6000 + seed)
        dec = rng.integers(256, 8193, size=256).astype(np.int32)
        cached = rng.integers(0, 4097, size=4).astype(np.int32)
        new = np.full(4, 1024, np.int32)
        lens = np.concatenate([dec, cached + new]).astype(np.int32)
        g = torch.Generator(device=device)
        g.manual_seed(7000 + seed)
        self.k_pool, self.v_pool, pt = paged_pool(rng, g, lens, hkv, hd, tpp, dtype, device)
        blocks = [(np.array([s], np.int32), np.array([dec[s]], np.int32)) for s in range(256)]
        for j in range(4):
            pos = np.arange(cached[j], cached[j] + new[j], dtype=np.int32)
            for b0 in range(0, len(pos), block):
                blocks.append((np.full(len(pos[b0:b0 + block]), 256 + j, np.int32), pos[b0:b0 + block] + 1))
        order = rng.permutation(len(blocks))
        q2s = np.concatenate([blocks[i][0] for i in order])
        off = np.concatenate([blocks[i][1] for i in order])
        self.rows = len(q2s)
        self.page_table = torch.from_numpy(pt).to(device)
        self.seq_lens = torch.from_numpy(lens).to(device)
        self.q2seq = torch.from_numpy(q2s).to(device)
        self.q_offset = torch.from_numpy(off).to(device)
        self.queries = torch.randn((self.rows, hq, hd), generator=g, device=device, dtype=torch.float32).to(dtype)
        self.decode_bytes = int(dec.astype(np.int64).sum()) * 2 * hkv * hd * 2 + 2 * 256 * hq * hd * 2
        self.prefill_flops = causal_flops(hq, hd, cached, new)
        # the same rows split by kind (sequences 0..255 are the decode ones),
        # for timing each half alone through the same operator
        self.parts = {}
        for name, sel in (("decode_rows", q2s < 256), ("prefill_rows", q2s >= 256)):
            idx = torch.from_numpy(np.nonzero(sel)[0]).to(device)
            self.parts[name] = (self.queries.index_select(0, idx).contiguous(), self.q2seq.index_select(0, idx),
                                self.q_offset.index_select(0, idx))

    def attend_part(self, name: str):
        q, q2s, off = self.parts[name]
        return pal.paged_attention(q, self.k_pool, self.v_pool, self.page_table, self.seq_lens, q2s, off)

    def attend(self):
        return pal.paged_attention(self.queries, self.k_pool, self.v_pool, self.page_table, self.seq_lens,
                                   self.q2seq, self.q_offset)


class PromptWorkload:
    """The reference prefill signature (paged_attention_prefill): 16 sequences
    x 1024 prompt rows on U[0,2048] cached history, 32/8 heads, HD 128, bf16;
    history keys from pages, prompt keys from the dense prompt K/V rows."""

    def __init__(self, device, seed: int = 11, num_seqs=16, prompt=1024, hq=32, hkv=8, hd=128, dtype=torch.bfloat16):
        rng = np.random.default_rng(6000 + seed)
        self.hist = rng.integers(0, 2049, size=num_seqs).astype(np.int32)
        g = torch.Generator(device=device)
        g.manual_seed(7000 + seed)
        self.k_pool, self.v_pool, pt = paged_pool(rng, g, np.maximum(self.hist, 1), hkv, hd, 16, dtype, device)
        self.page_table = torch.from_numpy(pt).to(device)
        self.context_lens = torch.from_numpy(self.hist).to(device)
        n = num_seqs * prompt
        self.prompt, self.hq, self.hd = prompt, hq, hd
        self.q = torch.randn((n, hq, hd), generator=g, device=device, dtype=torch.float32).to(dtype)
        self.k = torch.randn((n, hkv, hd), generator=g, device=device, dtype=torch.float32).to(dtype)
        self.v = torch.randn((n, hkv, hd), generator=g, device=device, dtype=torch.float32).to(dtype)

    def attend(self):
        return pal.paged_attention_prefill(self.q, self.k, self.v, self.k_pool, self.v_pool, self.page_table,
                                           self.context_lens)

    def flops(self) -> float:
        return causal_flops(self.hq, self.hd, self.hist, np.full(len(self.hist), self.prompt, np.int32))


class RopeFill:
    """The fused RoPE + cast + scatter feeding a fill step: fp32 projection
    rows (K, V and the queries) of the workload's new tokens, NeoX rotation
    of K and Q over the whole head, cast to bf16, K/V scattered into the
    workload's 16-bit pools."""

    def __init__(self, w, device, seed: int = 9):
        g = torch.Generator(device=device)
        g.manual_seed(seed)
        n = int(w.write_pos.numel())
        self.n, self.hq, self.hkv, self.hd = n, w.hq, w.hkv, w.hd
        self.k = torch.randn((n, w.hkv, w.hd), generator=g, device=device)
        self.v = torch.randn((n, w.hkv, w.hd), generator=g, device=device)
        self.q = torch.randn((n, w.hq, w.hd), generator=g, device=device)
        self.pt, self.pos, self.q2s = w.page_table, w.write_pos, w.q2seq
        self.k_pool, self.v_pool = w.k_pool, w.v_pool
        self.table = pal.rope_cos_sin_cache(int(w.write_pos.max().item()) + 1, w.hd, 500000.0, device=device)

    def run(self):
        return pal.rope_fill_kv_pages(self.k, self.v, self.k_pool, self.v_pool, self.pt, self.pos, self.q2s,
                                      self.table, queries=self.q)

    def bytes(self) -> int:
        """fp32 K, V, Q read + bf16 K, V, Q written + one cos/sin row per token."""
        kv = 2 * self.n * self.hkv * self.hd
        qn = self.n * self.hq * self.hd
        return (kv + qn) * (4 + 2) + self.n * self.hd * 4

    def report(self, ms: float) -> dict:
        b = self.bytes()
        return {"workload": f"rope_fill_kv_pages of {self.n} tokens: fp32 K/V/Q rows, NeoX RoPE, cast to bf16, "
                            f"scatter (Hq {self.hq}, Hkv {self.hkv}, HD {self.hd})",
                "ms": round(ms, 5), "bytes": b, "GB/s": round(b / (ms * 1e-3) / 1e9, 1),
                "frac_of_hbm_peak": round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}


# ---------------------------------------------------------------------------
# CPU baseline: the reference's equivalency computation (gather pages + fp32
# softmax attention) on torch CPU, over the same inputs as the GPU run
# ---------------------------------------------------------------------------


def _host_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def host_subset(k_pool: torch.Tensor, v_pool: torch.Tensor, pt: np.ndarray, lens: np.ndarray, seqs,
                tpp: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Host bits of the pages sequences `seqs` use (their first lens[s]
    tokens) and their page table renumbered to that compacted pool."""
    used = []
    for s in seqs:
        used.extend(int(x) for x in pt[s, : (int(lens[s]) + tpp - 1) // tpp])
    uniq = np.unique(np.asarray(used, np.int64)) if used else np.zeros(1, np.int64)
    idx = torch.from_numpy(uniq).to(k_pool.device)
    kb, vb = _host_bits(k_pool.index_select(0, idx)), _host_bits(v_pool.index_select(0, idx))
    pos = {int(p): i for i, p in enumerate(uniq)}
    spt = np.zeros((len(seqs), max(1, max((int(lens[s]) + tpp - 1) // tpp for s in seqs))), np.uint32)
    for i, s in enumerate(seqs):
        for j in range((int(lens[s]) + tpp - 1) // tpp):
            spt[i, j] = pos[int(pt[s, j])]
    return kb, vb, spt


def config1_host() -> dict:
    """Config 1: 4 sequences, ctx {64, 100, 192, 256},
    Hq 4 / Hkv 1, HD 64, TPP 16, a 64-page pool assigned by a seeded random
    permutation, N(0,1) fp16 values."""
    rng = np.random.default_rng(100)
    lens = np.array([64, 100, 192, 256], np.int32)
    perm = rng.permutation(64)
    pt = np.zeros((4, 16), np.uint32)
    cur = 0
    for s, n in enumerate(lens):
        k = (int(n) + 15) // 16
        pt[s, :k] = perm[cur:cur + k]
        cur += k

    def bits(shape):
        return rng.standard_normal(shape).astype(np.float16).view(np.uint16)

    return {"q": bits((4, 4, 64)), "k": bits((64, 1, 8, 16, 8)), "v": bits((64, 1, 64, 16)), "pt": pt,
            "lens": lens, "dtype": "f16"}


def _cpu_time(fn, reps: int, warm: int) -> float:
    """Median wall seconds of `reps` calls after `warm` warm-up calls."""
    for _ in range(warm):
        fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts))


def cpu_baseline(samples: dict) -> dict:
    """The CPU restatement of PAL's equivalency path (the reference has no CPU
    kernels, paged_attention_decode_primitive.cpp:63-69, and MLX is not
    available offline) timed on the host cores: config 1 and config 2 in
    full, configs 3-5 on a stated subsample scaled to the whole workload by
    its share of the work.  torch CPU with one thread per core of the
    process's affinity; median of several calls after warm-up."""
    from oracle import pal_oracle as orc  # the checker, used here only as the timed CPU baseline

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    cpu_model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            cpu_model = next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")), cpu_model)
    except OSError:  # pragma: no cover
        pass
    t_start = time.perf_counter()
    res = {"unit": "GB/s", "cores": int(torch.get_num_threads()), "cpu_model": cpu_model,
           "affinity_cpus": cores, "kind": "port"}

    def run(sm, reps, warm):
        return _cpu_time(lambda: orc.torch_cpu_paged_attention(sm["q"], sm["k"], sm["v"], sm["pt"], sm["lens"],
                                                               sm["dtype"], sm.get("q2s"), sm.get("off")),
                         reps, warm)

    c1 = config1_host()
    t1 = run(c1, 20, 3)
    res["config1"] = {"ms": round(t1 * 1e3, 3), "sample": "config 1 in full (4 sequences)"}
    c2 = samples["c2"]
    t2 = run(c2, 40, 3)
    res["value"] = round(c2["bytes"] / t2 / 1e9, 3)
    res["tokens_per_s"] = round(len(c2["lens"]) / t2, 2)
    res["config2_ms"] = round(t2 * 1e3, 2)
    res["sample"] = (f"config 2 in full (64 sequences, {int(c2['lens'].sum())} context tokens, the same pools as "
                     f"the GPU run's first copy): decode by gather + torch fp32 scaled_dot_product_attention, "
                     f"median of 40 after 3 warm-up; the fill step not included")
    for key, name in (("c3", "config3"), ("c4", "config4"), ("c5d", "config5_decode_rows"),
                      ("c5p", "config5_prefill_rows")):
        sm = samples.get(key)
        if sm is None:
            continue
        t = run(sm, 8, 1)
        rec = {"sample": sm["what"], "ms_sample": round(t * 1e3, 2), "scale": round(sm["scale"], 3),
               "ms_scaled": round(t * sm["scale"] * 1e3, 1)}
        if "bytes" in sm:
            rec["GB/s"] = round(sm["bytes"] / (t * sm["scale"]) / 1e9, 3)
        if "flops" in sm:
            rec["TFLOP/s"] = round(sm["flops"] / (t * sm["scale"]) / 1e12, 4)
        res[name] = rec
    res["cpu_seconds"] = round(time.perf_counter() - t_start, 1)
    return res


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
    ap.add_argument("--configs", default="c2,c3,c4,c5,lh",
                    help="comma list of workloads to run (c2 is the headline; c3/c4/c5 and lh, the long-history "
                         "decode points, are reported beside it)")
    ap.add_argument("--extra-steps", type=int, default=20, help="timed calls per extra config")
    ap.add_argument("--calibrate-copy-mib", type=int, default=0,
                    help="before the timed loop, run one device-to-device copy of this many MiB (a kernel of "
                         "known traffic for scaling rocprof FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the operators would shard by KV head or sequence with no exchange)", file=sys.stderr)
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
    configs = {c.strip() for c in args.configs.split(",") if c.strip()}
    samples: dict = {}  # host copies of the CPU baseline's inputs, taken from the GPU run's workloads
    if "c2" not in configs:
        extra = run_extra(configs, dev, args, samples)
        print(json.dumps({"metric": METRIC, "configs": sorted(configs), **extra}), flush=True)
        return 0
    works = [DecodeWorkload(seed=i) for i in range(max(1, args.rotate))]
    w0 = works[0]
    torch.cuda.synchronize()

    def step(w):
        w.fill()
        return w.decode(args.partition)

    for i in range(args.warmup):
        step(works[i % len(works)])
    torch.cuda.synchronize()

    # the timed steps: fill + decode, back to back, one event pair around all
    stream = torch.cuda.current_stream(dev)
    ev_start = torch.cuda.Event(enable_timing=True)
    ev_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev_start.record(stream)
    for i in range(args.steps):
        w = works[i % len(works)]
        w.fill()
        w.decode(args.partition)
    ev_end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = ev_start.elapsed_time(ev_end)
    ms_per_step = max(gpu_ms, wall * 1e3) / args.steps
    # the decode operator alone (roofline of the dominant kernels): the same
    # number of calls over the rotated copies, one event pair around all
    rot = iter(range(1 << 30))
    dec_ms, _ = time_op(lambda: works[next(rot) % len(works)].decode(args.partition), args.steps, 2, stream)

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
            "partition_size": args.partition if args.partition else "0 (one equal share per resident worker)",
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
            "traffic": traffic_bytes(),
            "traffic_source": "profiles/decode_config2_traffic.md (rocprofv3 FETCH_SIZE x2 + WRITE_SIZE per call)",
            "algorithmic_bytes_per_launch": int(dec_bytes),
            "avg_launch_ms": round(dec_ms, 5),
            "timing": "HIP events around back-to-back decode calls on the launch stream (stream + merge kernels)",
        },
    }
    # the same step over fp8 pages (bytes counted at one byte per K/V element)
    # and the fused RoPE + cast + scatter feeding it (fp32 projection rows)
    for w in works:
        w.make_fp8()
    rot = iter(range(1 << 30))
    f8_dec_ms, _ = time_op(lambda: works[next(rot) % len(works)].decode_fp8(), args.steps, 3, stream)
    rot = iter(range(1 << 30))

    def fp8_step():
        w = works[next(rot) % len(works)]
        w.fill_fp8()
        w.decode_fp8()

    f8_step_ms, _ = time_op(fp8_step, args.steps, 3, stream)
    f8_bytes = float(np.mean([w.decode_bytes_fp8() for w in works]))
    rope = RopeFill(w0, dev)
    rope_ms, _ = time_op(rope.run, args.steps, 3, stream)
    result["fp8_pages"] = {
        "workload": "config 2 over fp8 e4m3 pages (per-(page, kv head) scales), bf16 queries/output",
        "decode_ms": round(f8_dec_ms, 5), "decode_bytes": int(f8_bytes),
        "decode_GB/s": round(f8_bytes / (f8_dec_ms * 1e-3) / 1e9, 1),
        "decode_frac_of_hbm_peak": round(f8_bytes / (f8_dec_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "speedup_vs_bf16_decode": round(dec_ms / f8_dec_ms, 3),
        "step_ms (fill_fp8 + decode)": round(f8_step_ms, 5),
        "tokens_per_s": round(w0.num_seqs / (f8_step_ms * 1e-3), 1),
    }
    result["rope_fill_config2"] = rope.report(rope_ms)
    if not args.no_cpu_baseline:
        samples["c2"] = {"q": _host_bits(w0.queries), "k": _host_bits(w0.k_pool), "v": _host_bits(w0.v_pool),
                         "pt": w0.pt_np.astype(np.uint32), "lens": w0.lens_np, "dtype": "bf16",
                         "bytes": w0.decode_bytes()}
    del works, rope, w0
    torch.cuda.empty_cache()
    result.update(run_extra(configs, dev, args, samples if not args.no_cpu_baseline else None))
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(samples)
    print(json.dumps(result), flush=True)
    return 0


def time_rotated(fns, steps: int, warm: int, stream) -> float:
    """time_op over calls that cycle through `fns` (independent copies of one
    workload), so consecutive calls share no data through L2 or MALL."""
    rot = iter(range(1 << 30))
    return time_op(lambda: fns[next(rot) % len(fns)](), steps, warm, stream)[0]


LONG_HISTORY = (131072, 524288, 1048576)


def run_long_history(dev, steps: int, warm: int, stream) -> dict:
    """Batch-1 decode over long histories, the reference's own benchmark
    range (benchmarks/paged_attention/cpp/seq_len_vs_latency.cpp:47-55,
    210-223 and python/test_paged_attention_python.py:140-141): 32 query / 16
    kv heads, HD 128, bf16, 16-token pages (get_optimal_page_size), randomly
    permuted pages; both split forms."""
    out = {"workload": "batch-1 decode, 32/16 heads, HD 128, bf16, TPP 16, permuted pages; history lengths as in "
                       "the reference's seq_len_vs_latency benchmark"}
    for hist in LONG_HISTORY:
        w = DecodeWorkload(30, num_seqs=1, ctx_lo=hist, ctx_hi=hist, hq=32, hkv=16, device=dev)
        nbytes = w.decode_bytes()
        rec = {"bytes": nbytes}
        for part in (0, 512):
            ms, _ = time_op(lambda: w.decode(part), steps, warm, stream)
            gbs = nbytes / (ms * 1e-3) / 1e9
            rec[f"partition_{part}"] = {"ms": round(ms, 4), "GB/s": round(gbs, 1),
                                        "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
                                        "tokens_per_s": round(1.0 / (ms * 1e-3), 1)}
        out[f"history_{hist}"] = rec
        del w
        torch.cuda.empty_cache()
    return out


def run_extra(configs: set[str], dev, args, samples: dict | None = None) -> dict:
    """Configs 3, 4 and 5 and the long-history points, each timed with HIP
    events around its operator calls.  With `samples`, host copies of a
    bounded subsample of each workload are kept for the CPU baseline."""
    out = {}
    stream = torch.cuda.current_stream(dev)
    steps, warm = max(1, args.extra_steps), 3
    if "c3" in configs:
        w = long_context_workload(dev)
        nbytes = w.decode_bytes()
        res = {"workload": "config 3: 8 x U[32768,131072] ctx, 32/8 heads, HD 128, bf16, 1% key rows x8",
               "context_tokens": int(w.lens_np.sum()), "algorithmic_bytes": nbytes}
        for part in (512, 0):
            ms, _ = time_op(lambda: w.decode(part), steps, warm, stream)
            gbs = nbytes / (ms * 1e-3) / 1e9
            res[f"partition_{part}"] = {"ms": round(ms, 4), "GB/s": round(gbs, 1),
                                        "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}
        if samples is not None:
            s0 = int(np.argmin(w.lens_np))
            kb, vb, spt = host_subset(w.k_pool, w.v_pool, w.pt_np, w.lens_np, [s0], w.tpp)
            samples["c3"] = {"q": _host_bits(w.queries)[[s0]], "k": kb, "v": vb, "pt": spt, "lens": w.lens_np[[s0]],
                             "dtype": "bf16", "bytes": nbytes,
                             "scale": float(w.lens_np.sum()) / float(w.lens_np[s0]),
                             "what": f"1 of 8 sequences ({int(w.lens_np[s0])} of {int(w.lens_np.sum())} context "
                                     f"tokens), scaled by the token ratio"}
        w.make_fp8()
        f8 = w.decode_bytes_fp8()
        for part in (512, 0):
            ms, _ = time_op(lambda: w.decode_fp8(part), steps, warm, stream)
            res[f"fp8_partition_{part}"] = {"ms": round(ms, 4), "bytes": f8, "GB/s": round(f8 / (ms * 1e-3) / 1e9, 1),
                                           "frac_of_hbm_peak": round(f8 / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        out["long_context_decode"] = res
        del w
        torch.cuda.empty_cache()
    if "c4" in configs:
        # three identical copies (same seed) in separate memory, cycled per
        # call: each call's 0.2-0.4 GB working set then comes from HBM, not
        # from the 256 MB last-level cache a repeated call would hit
        ws = [PrefillWorkload(dev) for _ in range(3)]
        w = ws[0]
        fill_ms = time_rotated([x.fill for x in ws], steps, warm, stream)
        att_ms = time_rotated([x.attend for x in ws], steps, warm, stream)
        fill_hot_ms, _ = time_op(w.fill, steps, warm, stream)
        fl = w.flops()
        tf = fl / (att_ms * 1e-3) / 1e12
        out["prefill"] = {
            "workload": "config 4: 16 seqs, new U[512,2048] on cached U[0,2048], 32/8 heads, HD 128, bf16; "
                        "fill_kv_pages of the new chunks, then causal attention (paged_attention, tile path); "
                        "timed over 3 rotated copies of the workload",
            "rows": w.rows, "causal_flops": fl,
            "attention_ms": round(att_ms, 4), "TFLOP/s": round(tf, 1),
            "frac_of_mfma_bf16_peak": round(tf / MFMA_BF16_PEAK_TFLOPS, 4),
            "fill_ms": round(fill_ms, 4), "fill_GB/s": round(w.fill_bytes() / (fill_ms * 1e-3) / 1e9, 1),
            "fill_frac_of_hbm_peak": round(w.fill_bytes() / (fill_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "fill_same_copy_ms": round(fill_hot_ms, 4),
            "step_ms": round(att_ms + fill_ms, 4),
        }
        if samples is not None:
            s0 = int(np.argsort(w.new)[len(w.new) // 2])  # the median new chunk
            lens = w.seq_lens.cpu().numpy()
            kb, vb, spt = host_subset(w.k_pool, w.v_pool, w.page_table.cpu().numpy(), lens, [s0], 16)
            rows = np.nonzero(w.q2seq.cpu().numpy() == s0)[0]
            sfl = causal_flops(w.hq, w.hd, w.cached[[s0]], w.new[[s0]])
            samples["c4"] = {"q": _host_bits(w.queries)[rows], "k": kb, "v": vb, "pt": spt, "lens": lens[[s0]],
                             "q2s": np.zeros(len(rows), np.uint32), "off": w.q_offset.cpu().numpy()[rows],
                             "dtype": "bf16", "flops": fl, "scale": fl / sfl,
                             "what": f"1 of 16 sequences ({int(w.new[s0])} new rows on {int(w.cached[s0])} cached), "
                                     f"scaled by the causal-flop ratio"}
        rope = RopeFill(w, dev)
        rope_ms, _ = time_op(rope.run, steps, warm, stream)
        out["prefill"]["rope_fill"] = rope.report(rope_ms)
        del rope, ws[1:]
        # the same attention over fp8 e4m3 pools (per-(page, kv head) scales)
        k8, ks = to_fp8_pages(to_fp8_k_layout(w.k_pool))
        v8, vs = to_fp8_pages(w.v_pool)
        f8_ms, _ = time_op(lambda: pal.paged_attention(w.queries, k8, v8, w.page_table, w.seq_lens, w.q2seq,
                                                       w.q_offset, k_scales=ks, v_scales=vs), steps, warm, stream)
        f8_tf = fl / (f8_ms * 1e-3) / 1e12
        out["prefill"]["fp8_pages"] = {"attention_ms": round(f8_ms, 4), "TFLOP/s": round(f8_tf, 1),
                                       "frac_of_mfma_bf16_peak": round(f8_tf / MFMA_BF16_PEAK_TFLOPS, 4)}
        del k8, v8, ks, vs
        del w, ws
        torch.cuda.empty_cache()
        pw = PromptWorkload(dev)
        p_ms, _ = time_op(pw.attend, steps, warm, stream)
        p_tf = pw.flops() / (p_ms * 1e-3) / 1e12
        out["prefill"]["reference_signature"] = {
            "workload": "paged_attention_prefill: 16 seqs x 1024 prompt rows on U[0,2048] cached history, "
                        "32/8 heads, HD 128, bf16 (history keys from pages, prompt keys from the prompt rows)",
            "causal_flops": pw.flops(), "ms": round(p_ms, 4), "TFLOP/s": round(p_tf, 1),
            "frac_of_mfma_bf16_peak": round(p_tf / MFMA_BF16_PEAK_TFLOPS, 4),
        }
        del pw
        torch.cuda.empty_cache()
    if "c5" in configs:
        w = FusedWorkload(dev)
        ms, _ = time_op(w.attend, steps, warm, stream)
        dec_ms, _ = time_op(lambda: w.attend_part("decode_rows"), steps, warm, stream)
        pre_ms, _ = time_op(lambda: w.attend_part("prefill_rows"), steps, warm, stream)
        t_roof_ms = (w.decode_bytes / (HBM_PEAK_GBS * 1e9) + w.prefill_flops / (MFMA_BF16_PEAK_TFLOPS * 1e12)) * 1e3
        out["fused"] = {
            "workload": "config 5: 256 decode rows ctx U[256,8192] + 4 x 1024 prefill rows on U[0,4096] cached, "
                        "64/8 heads, HD 128, fp16, shuffled row blocks, one paged_attention call",
            "rows": w.rows, "decode_bytes": w.decode_bytes, "prefill_flops": w.prefill_flops,
            "ms": round(ms, 4), "roofline_ms": round(t_roof_ms, 4), "frac_of_roofline": round(t_roof_ms / ms, 4),
            "decode_rows_alone_ms": round(dec_ms, 4), "prefill_rows_alone_ms": round(pre_ms, 4),
            "ms_over_sum_of_halves": round(ms / (dec_ms + pre_ms), 4),
        }
        if samples is not None:
            lens = w.seq_lens.cpu().numpy()
            q2s = w.q2seq.cpu().numpy()
            off = w.q_offset.cpu().numpy()
            pt = w.page_table.cpu().numpy()
            qb = _host_bits(w.queries)
            dec = list(range(0, 256, 16))  # 16 of the 256 decode sequences
            kb, vb, spt = host_subset(w.k_pool, w.v_pool, pt, lens, dec, 16)
            rows = np.nonzero(np.isin(q2s, dec))[0]
            local = {s: i for i, s in enumerate(dec)}
            dec_bytes = int(lens[dec].astype(np.int64).sum()) * 2 * 8 * 128 * 2
            samples["c5d"] = {"q": qb[rows], "k": kb, "v": vb, "pt": spt, "lens": lens[dec],
                              "q2s": np.array([local[int(x)] for x in q2s[rows]], np.uint32), "off": off[rows],
                              "dtype": "f16", "bytes": w.decode_bytes, "scale": w.decode_bytes / dec_bytes,
                              "what": "16 of the 256 decode rows, scaled by their share of the decode bytes"}
            ch = 256 + int(np.argmax(lens[256:]))  # the chunk on the largest cache
            kb, vb, spt = host_subset(w.k_pool, w.v_pool, pt, lens, [ch], 16)
            rows = np.nonzero(q2s == ch)[0]
            sfl = causal_flops(64, 128, np.array([lens[ch] - 1024]), np.array([1024]))
            samples["c5p"] = {"q": qb[rows], "k": kb, "v": vb, "pt": spt, "lens": lens[[ch]],
                              "q2s": np.zeros(len(rows), np.uint32), "off": off[rows], "dtype": "f16",
                              "flops": w.prefill_flops, "scale": w.prefill_flops / sfl,
                              "what": f"1 of the 4 prefill chunks (1024 rows on {int(lens[ch]) - 1024} cached), "
                                      f"scaled by the causal-flop ratio"}
        del w
        torch.cuda.empty_cache()
    if "lh" in configs:
        out["long_history_decode"] = run_long_history(dev, min(steps, 10), warm, stream)
    if "pages" in configs:
        out["decode_page_sizes"] = run_page_sizes(dev, steps, warm, stream)
    if "shapes" in configs:
        out["decode_shapes"] = run_decode_shapes(dev, steps, warm, stream)
    return out


DECODE_SHAPES = [  # (name, DecodeWorkload arguments)
    ("config 2: 64 seqs U[512,4096], 32/8 heads", {}),
    ("512 seqs U[64,512]", dict(num_seqs=512, ctx_lo=64, ctx_hi=512)),
    ("2048 seqs U[16,256]", dict(num_seqs=2048, ctx_lo=16, ctx_hi=256)),
    ("4096 seqs U[256,1024]", dict(num_seqs=4096, ctx_lo=256, ctx_hi=1024)),
    ("64 seqs, 32/32 heads (no GQA)", dict(hq=32, hkv=32)),
    ("64 seqs, 64/8 heads", dict(hq=64, hkv=8)),
    ("64 seqs, 8/8 heads", dict(hq=8, hkv=8)),
    ("8 seqs x 32768", dict(num_seqs=8, ctx_lo=32768, ctx_hi=32768)),
]


def run_decode_shapes(dev, steps: int, warm: int, stream) -> dict:
    """bf16 decode (HD 128, 16-token pages) across batch shapes and GQA
    groups, both split forms, each over 4 rotated copies."""
    out = {"workload": "bf16 decode, HD 128, 16-token pages, permuted pages; 4 rotated copies per shape"}
    for name, kw in DECODE_SHAPES:
        ws = [DecodeWorkload(seed=i, device=dev, **kw) for i in range(4)]
        nbytes = float(np.mean([w.decode_bytes() for w in ws]))
        rec = {"bytes": int(nbytes)}
        for part in (0, 512):
            ms = time_rotated([lambda w=w, part=part: w.decode(part) for w in ws], steps, warm, stream)
            rec[f"partition_{part}"] = {"us": round(ms * 1e3, 1),
                                        "frac_of_hbm_peak": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        out[name] = rec
        del ws
        torch.cuda.empty_cache()
    return out


def run_page_sizes(dev, steps: int, warm: int, stream) -> dict:
    """Config 2's decode (64 seqs, U[512,4096] ctx, 32/8 heads) at head dims
    64 / 128 / 256 over 16- and 32-token pages: bf16 pools in both split
    forms and fp8 pools, each timed over 4 rotated copies."""
    out = {"workload": "config 2's shape (64 seqs, U[512,4096] ctx, 32/8 heads, bf16 queries) at head dims 64, 128, "
                       "256 over 16- and 32-token pages, 4 rotated copies per point; config4_attention: config 4's "
                       "chunked prefill at the same head dim and page size, 3 rotated copies"}
    for hd in (64, 128, 256):
        for tpp in (16, 32):
            ws = [DecodeWorkload(seed=i, hd=hd, tpp=tpp, device=dev) for i in range(4)]
            nbytes = float(np.mean([w.decode_bytes() for w in ws]))
            rec = {}
            for part in (0, 512):
                ms = time_rotated([lambda w=w, part=part: w.decode(part) for w in ws], steps, warm, stream)
                rec[f"bf16_partition_{part}"] = {"us": round(ms * 1e3, 1),
                                                 "frac_of_hbm_peak": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
            for w in ws:
                w.make_fp8()
            f8 = float(np.mean([w.decode_bytes_fp8() for w in ws]))
            ms = time_rotated([w.decode_fp8 for w in ws], steps, warm, stream)
            rec["fp8_partition_0"] = {"us": round(ms * 1e3, 1),
                                      "frac_of_hbm_peak": round(f8 / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
            ps = [PrefillWorkload(dev, hd=hd, tpp=tpp) for _ in range(3)]
            ms = time_rotated([x.attend for x in ps], max(2, steps // 2), 2, stream)
            tf = ps[0].flops() / (ms * 1e-3) / 1e12
            rec["config4_attention"] = {"ms": round(ms, 4), "TFLOP/s": round(tf, 1),
                                        "frac_of_mfma_bf16_peak": round(tf / MFMA_BF16_PEAK_TFLOPS, 4)}
            out[f"hd{hd}_tpp{tpp}"] = rec
            del ws, ps
            torch.cuda.empty_cache()
    return out


if __name__ == "__main__":
    sys.exit(main())
