"""Seeded case builders and comparison helpers shared by the tests.

Cases are built in numpy (raw 16-bit patterns) so the CPU oracle and the GPU
path see identical inputs.  Page tables are randomly permuted and unused
page-table entries point at random valid pages, so an out-of-range read by a
kernel shows up as a wrong result rather than passing silently.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

from oracle import pal_oracle as orc

# Output tolerances for attention (the contract for this path).
TOL = {"bf16": dict(atol=2e-2, rtol=2e-2), "f16": dict(atol=5e-3, rtol=5e-3)}


def randn_bits(rng: np.random.Generator, shape, dtype: str, scale: float = 1.0) -> np.ndarray:
    x = rng.standard_normal(size=shape, dtype=np.float32)
    if scale != 1.0:
        x *= np.float32(scale)
    return orc.f32_to_bits(x, dtype)


def extreme_query_bits(rng: np.random.Generator, shape, dtype: str, tiles: bool = False) -> np.ndarray:
    """Queries [..., H >= 5, HD] whose first five heads span the dtype's
    range: zeros; tiny values (fp16: subnormals); huge values; a head with
    half its dims large and half small; values near the bottom of bf16's
    normal range, or near the fp16 maximum.  The other heads are N(0, 1).

    Decode takes its exponents as exp2(score - max) in log2 units, exact at
    any size, so the huge heads there reach scores past 2^31 (one-hot
    softmax).  The prefill tiles take one fma against the rounded max, exact
    while the scaled max stays below ~2^14; with tiles=True the large heads
    are held to magnitude 1e3 (scaled scores of a few thousand)."""
    x = rng.standard_normal(size=shape, dtype=np.float32)
    bf = dtype == "bf16"
    half = shape[-1] // 2
    big = 1e3 if tiles else (1e20 if bf else 3e3)
    x[..., 0, :] = 0.0
    x[..., 1, :] *= np.float32(1e-30 if bf else 1e-7)
    x[..., 2, :] *= np.float32(big)
    x[..., 3, :half] *= np.float32(1e3 if tiles else (1e6 if bf else 1e2))
    x[..., 3, half:] *= np.float32(1e-3 if tiles else (1e-6 if bf else 1e-2))
    if bf:
        x[..., 4, :] *= np.float32(1e-38)
    else:
        x[..., 4, :] = np.clip(x[..., 4, :] * (1e3 if tiles else 3e4), -65000, 65000)
    return orc.f32_to_bits(x, dtype)


@dataclass
class PagedCase:
    dtype: str
    num_q_heads: int
    num_kv_heads: int
    head_dim: int
    tokens_per_page: int
    seq_lens: np.ndarray  # int32 [S]
    page_table: np.ndarray  # uint32 [S, W]
    k_pool: np.ndarray  # uint16 [P, Hkv, HD/8, TPP, 8]
    v_pool: np.ndarray  # uint16 [P, Hkv, HD, TPP]
    extra: dict = field(default_factory=dict)

    @property
    def num_seqs(self) -> int:
        return int(self.page_table.shape[0])


def make_paged_case(seed: int, seq_lens, num_q_heads: int, num_kv_heads: int, head_dim: int,
                    tokens_per_page: int, dtype: str, *, extra_pages: int = 3, width: int | None = None,
                    outlier_frac: float = 0.0, outlier_scale: float = 8.0,
                    garbage_tail: bool = True) -> PagedCase:
    """Pools filled with N(0,1) values and a permuted page table.

    outlier_frac: fraction of key rows (token positions, the same for all KV
    heads) multiplied by outlier_scale, to stress softmax range.
    garbage_tail: fill the unused slots of each sequence's last page with
    NaN bit patterns; correct kernels never let them reach the output.
    """
    rng = np.random.default_rng(seed)
    lens = np.asarray(seq_lens, dtype=np.int32)
    tpp = tokens_per_page
    pages_per_seq = [(int(n) + tpp - 1) // tpp for n in lens]
    total = sum(pages_per_seq)
    num_pages = max(1, total + extra_pages)
    w = width if width is not None else max(1, max(pages_per_seq) if len(pages_per_seq) else 1)
    perm = rng.permutation(num_pages).astype(np.uint32)
    pt = rng.integers(0, num_pages, size=(len(lens), w), dtype=np.uint32)
    cur = 0
    for s, npg in enumerate(pages_per_seq):
        pt[s, :npg] = perm[cur : cur + npg]
        cur += npg
    x = 8
    k_pool = randn_bits(rng, (num_pages, num_kv_heads, head_dim // x, tpp, x), dtype)
    v_pool = randn_bits(rng, (num_pages, num_kv_heads, head_dim, tpp), dtype)
    if outlier_frac > 0:
        kf = orc.bits_to_f32(k_pool, dtype)
        for s, n in enumerate(lens):
            n = int(n)
            if n == 0:
                continue
            cnt = max(1, int(round(outlier_frac * n)))
            toks = rng.choice(n, size=cnt, replace=False)
            for t in toks:
                page, slot = pt[s, t // tpp], t % tpp
                kf[page, :, :, slot, :] *= np.float32(outlier_scale)
        k_pool = orc.f32_to_bits(kf, dtype)
    if garbage_tail:
        nan = np.uint16(0x7FC0 if dtype == "bf16" else 0x7E00)
        for s, n in enumerate(lens):
            n = int(n)
            if n % tpp:
                page = pt[s, n // tpp]
                k_pool[page, :, :, n % tpp :, :] = nan
                v_pool[page, :, :, n % tpp :] = nan
    return PagedCase(dtype, num_q_heads, num_kv_heads, head_dim, tpp, lens, pt, k_pool, v_pool)


def compact_subset(case: PagedCase, seqs) -> PagedCase:
    """Restrict a case to some sequences with a compacted pool (for the oracle)."""
    seqs = np.asarray(seqs)
    tpp = case.tokens_per_page
    lens = case.seq_lens[seqs]
    rows = case.page_table[seqs]
    used = []
    for r, n in zip(rows, lens):
        used.extend(int(p) for p in r[: (int(n) + tpp - 1) // tpp])
    uniq = np.unique(np.asarray(used, dtype=np.int64)) if used else np.zeros(1, np.int64)
    remap = {int(p): i for i, p in enumerate(uniq)}
    pt = np.zeros_like(rows)
    for i, (r, n) in enumerate(zip(rows, lens)):
        for j in range((int(n) + tpp - 1) // tpp):
            pt[i, j] = remap[int(r[j])]
    return PagedCase(case.dtype, case.num_q_heads, case.num_kv_heads, case.head_dim, tpp, lens, pt,
                     case.k_pool[uniq], case.v_pool[uniq])


def _log_margin(what: str, dtype: str, max_err: float, worst: float) -> None:
    """Record how close a comparison came to its tolerance: max |err| and the
    largest |err| / (atol + rtol |expected|) (below 1 passes).  Printed to the
    real stderr (outside pytest's capture) and, if PAL_MARGIN_LOG names a
    file, appended to it as one JSON line."""
    import json
    import os
    import sys

    tol = TOL[dtype]
    rec = {"case": what, "dtype": dtype, "atol": tol["atol"], "rtol": tol["rtol"], "max_abs_err": max_err,
           "worst_err_over_allowed": worst}
    print(f"[margin] {what} {dtype}: max|err| {max_err:.3g}, worst err/allowed {worst:.3f} "
          f"(atol {tol['atol']}, rtol {tol['rtol']})", file=sys.__stderr__, flush=True)
    path = os.environ.get("PAL_MARGIN_LOG")
    if path:
        with open(path, "a") as f:
            f.write(json.dumps(rec) + "\n")


def assert_close(actual_f32: np.ndarray, expected_f32: np.ndarray, dtype: str, what: str = "") -> None:
    tol = TOL[dtype]
    a = np.asarray(actual_f32, np.float32)
    e = np.asarray(expected_f32, np.float32)
    assert a.shape == e.shape, f"{what}: shape {a.shape} != {e.shape}"
    ok = np.isclose(a, e, atol=tol["atol"], rtol=tol["rtol"])
    diff = np.abs(a.astype(np.float64) - e.astype(np.float64))
    if a.size:
        with np.errstate(invalid="ignore"):
            ratio = diff / (tol["atol"] + tol["rtol"] * np.abs(e.astype(np.float64)))
        _log_margin(what, dtype, float(np.nanmax(diff)) if np.isfinite(diff).any() else float("inf"),
                    float(np.nanmax(ratio)) if np.isfinite(ratio).any() else float("inf"))
    if not ok.all():
        bad = np.argwhere(~ok)
        i = tuple(bad[0])
        raise AssertionError(
            f"{what}: {len(bad)} of {a.size} elements outside atol={tol['atol']} rtol={tol['rtol']}; "
            f"max |diff| {np.nanmax(diff):.4g}; first at {i}: got {a[i]!r}, want {e[i]!r}"
        )


def sdpa_prefill_case(seed, batch, hist, plen, hq, hkv, hd, dtype):
    """The reference's prefill equivalency construction (prefill/test_sdpa_equivalency.py:51-117):
    one causal SDPA over history + prompt, then keep the prompt rows."""
    rng = np.random.default_rng(seed)
    total = hist + plen
    q = orc.f32_to_bits(rng.standard_normal((batch, hq, total, hd)).astype(np.float32), dtype)
    k = orc.f32_to_bits(rng.standard_normal((batch, hkv, total, hd)).astype(np.float32), dtype)
    v = orc.f32_to_bits(rng.standard_normal((batch, hkv, total, hd)).astype(np.float32), dtype)
    qf, kf, vf = (torch.from_numpy(orc.bits_to_f32(a, dtype)) for a in (q, k, v))
    g = hq // hkv
    ref = torch.nn.functional.scaled_dot_product_attention(
        qf, kf.repeat_interleave(g, 1), vf.repeat_interleave(g, 1), is_causal=True)[:, :, hist:, :]
    ref = ref.permute(0, 2, 1, 3).reshape(batch * plen * hq, hd).numpy()
    q_prompt = q[:, :, hist:, :].transpose(0, 2, 1, 3).reshape(batch * plen, hq, hd)
    k_prompt = k[:, :, hist:, :].transpose(0, 2, 1, 3).reshape(batch * plen, hkv, hd)
    v_prompt = v[:, :, hist:, :].transpose(0, 2, 1, 3).reshape(batch * plen, hkv, hd)
    tpp = 16
    npg = (hist + tpp - 1) // tpp
    k_pool = np.zeros(orc.k_cache_shape(batch * npg + 2, hkv, hd, tpp, dtype), np.uint16)
    v_pool = np.zeros(orc.v_cache_shape(batch * npg + 2, hkv, hd, tpp, dtype), np.uint16)
    perm = rng.permutation(batch * npg + 2)
    pt = np.zeros((batch, max(npg, 1)), np.uint32)
    for b in range(batch):
        pt[b, :npg] = perm[b * npg:(b + 1) * npg]
        orc.scatter_contiguous(k[b, :, :hist, :].transpose(1, 0, 2), v[b, :, :hist, :].transpose(1, 0, 2),
                               k_pool, v_pool, pt[b])
    lens = np.full(batch, hist, np.int32)
    return q_prompt, k_prompt, v_prompt, k_pool, v_pool, pt, lens, ref


def make_prefill_case(seed: int, hist_lens, prompt_len: int, num_q_heads: int, num_kv_heads: int, head_dim: int,
                      tokens_per_page: int, dtype: str, **kw):
    """Paged history of hist_lens[s] tokens per sequence plus a uniform dense
    prompt (the reference prefill's inputs): (case, q_prompt, k_prompt, v_prompt)."""
    case = make_paged_case(seed, hist_lens, num_q_heads, num_kv_heads, head_dim, tokens_per_page, dtype, **kw)
    rng = np.random.default_rng(seed + 1000)
    rows = case.num_seqs * prompt_len
    q = randn_bits(rng, (rows, num_q_heads, head_dim), dtype)
    k = randn_bits(rng, (rows, num_kv_heads, head_dim), dtype)
    v = randn_bits(rng, (rows, num_kv_heads, head_dim), dtype)
    return case, q, k, v


@dataclass
class FusedCase:
    case: PagedCase
    queries: np.ndarray   # uint16 [R, Hq, HD]
    q2seq: np.ndarray     # uint32 [R]
    q_offset: np.ndarray  # int32 [R]


def make_fused_case(seed: int, decode_lens, chunks, num_q_heads: int, num_kv_heads: int, head_dim: int,
                    tokens_per_page: int, dtype: str, *, block: int = 64, extra_offset: bool = True,
                    **kw) -> FusedCase:
    """A mixed batch: one decode row per entry of decode_lens, and for each
    (cached, new) in chunks the `new` prompt rows at positions cached ..
    cached+new-1 (offset p + 1), all K/V already in the pages.  Sequences are
    the decode ones first, then one per chunk.  Rows are shuffled in blocks
    (each decode row is a block, each chunk is cut into blocks of `block`
    rows), so decode and prefill rows interleave.  With extra_offset, some
    decode rows pass offset len + 1 (clamped to len by the op), as the
    reference benchmark's history + 1 does."""
    rng = np.random.default_rng(seed)
    lens = list(int(x) for x in decode_lens) + [int(c) + int(n) for c, n in chunks]
    case = make_paged_case(seed, lens, num_q_heads, num_kv_heads, head_dim, tokens_per_page, dtype, **kw)
    blocks = []
    nd = len(decode_lens)
    for s in range(nd):
        off = lens[s] + (1 if extra_offset and rng.random() < 0.5 else 0)
        blocks.append((np.array([s], np.uint32), np.array([off], np.int32)))
    for j, (cached, new) in enumerate(chunks):
        s = nd + j
        pos = np.arange(int(cached), int(cached) + int(new), dtype=np.int32)
        for b0 in range(0, len(pos), block):
            pb = pos[b0:b0 + block]
            blocks.append((np.full(len(pb), s, np.uint32), pb + 1))
    order = rng.permutation(len(blocks))
    q2seq = np.concatenate([blocks[i][0] for i in order]) if blocks else np.zeros(0, np.uint32)
    q_off = np.concatenate([blocks[i][1] for i in order]) if blocks else np.zeros(0, np.int32)
    q = randn_bits(rng, (len(q2seq), num_q_heads, head_dim), dtype)
    return FusedCase(case, q, q2seq.astype(np.uint32), q_off.astype(np.int32))
