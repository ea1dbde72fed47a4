"""Seeded case builders and comparison helpers shared by the tests.

Cases are built in numpy (raw 16-bit patterns) so the CPU oracle and the GPU
path see identical inputs.  Page tables are randomly permuted and unused
page-table entries point at random valid pages, so an out-of-range read by a
kernel shows up as a wrong result rather than passing silently.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from oracle import pal_oracle as orc

# Output tolerances for attention (the contract for this path).
TOL = {"bf16": dict(atol=2e-2, rtol=2e-2), "f16": dict(atol=5e-3, rtol=5e-3)}


def randn_bits(rng: np.random.Generator, shape, dtype: str, scale: float = 1.0) -> np.ndarray:
    x = rng.standard_normal(size=shape, dtype=np.float32)
    if scale != 1.0:
        x *= np.float32(scale)
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


def assert_close(actual_f32: np.ndarray, expected_f32: np.ndarray, dtype: str, what: str = "") -> None:
    tol = TOL[dtype]
    a = np.asarray(actual_f32, np.float32)
    e = np.asarray(expected_f32, np.float32)
    assert a.shape == e.shape, f"{what}: shape {a.shape} != {e.shape}"
    ok = np.isclose(a, e, atol=tol["atol"], rtol=tol["rtol"])
    if not ok.all():
        bad = np.argwhere(~ok)
        i = tuple(bad[0])
        diff = np.abs(a - e)
        raise AssertionError(
            f"{what}: {len(bad)} of {a.size} elements outside atol={tol['atol']} rtol={tol['rtol']}; "
            f"max |diff| {np.nanmax(diff):.4g}; first at {i}: got {a[i]!r}, want {e[i]!r}"
        )
