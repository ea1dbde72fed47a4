"""Write the golden fixtures of this directory from the CPU oracle.

The reference ships no golden vectors for this path (its tests compare
against MLX SDPA at run time), so the fixtures are written by the oracle,
which is itself pinned by the reference's known-answer tests and by torch
SDPA (tests/test_oracle.py).  They freeze the expected outputs of:

  config1_decode_f16.npz  BASELINE config 1: 4 sequences, ctx {64,100,192,256},
                          4/1 heads, HD 64, 16-token pages, 64-page pool with a
                          seeded random page permutation, fp16 N(0,1) values
  prefill_small_bf16.npz  2 sequences, history {5, 40}, prompt 12, 8/2 heads,
                          HD 64, bf16
  fused_small_f16.npz     3 decode rows + one 20-row prefill run, 8/2 heads,
                          HD 64, fp16
  fill_small_bf16.npz     fill_kv_pages of 37 tokens into a 12-page pool

Arrays hold raw 16-bit patterns (uint16) and int32/uint32 indices; expected
attention outputs are float32.  Regenerate with
    python tests/golden/make_golden.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))
sys.path.insert(0, str(HERE.parent))

from oracle import pal_oracle as orc  # noqa: E402
from pal_cases import make_fused_case, make_paged_case, make_prefill_case, randn_bits  # noqa: E402


def config1():
    rng = np.random.default_rng(1)
    lens = np.array([64, 100, 192, 256], np.int32)
    hq, hkv, hd, tpp, n_pages = 4, 1, 64, 16, 64
    perm = rng.permutation(n_pages).astype(np.uint32)
    npg = (lens + tpp - 1) // tpp
    pt = np.zeros((4, int(npg.max())), np.uint32)
    cur = 0
    for s, n in enumerate(npg):
        pt[s, :n] = perm[cur:cur + n]
        cur += n
    k_pool = randn_bits(rng, orc.k_cache_shape(n_pages, hkv, hd, tpp, "f16"), "f16")
    v_pool = randn_bits(rng, orc.v_cache_shape(n_pages, hkv, hd, tpp, "f16"), "f16")
    q = randn_bits(rng, (4, hq, hd), "f16")
    out = orc.paged_attention_decode(q, k_pool, v_pool, pt, lens, "f16")
    np.savez_compressed(HERE / "config1_decode_f16.npz", queries=q, k_pool=k_pool, v_pool=v_pool, page_table=pt,
                        seq_lens=lens, expected=out)


def prefill_small():
    case, q, k, v = make_prefill_case(70, [5, 40], 12, 8, 2, 64, 16, "bf16", garbage_tail=False)
    out = orc.paged_attention_prefill(q, k, v, case.k_pool, case.v_pool, case.page_table, case.seq_lens, "bf16")
    np.savez_compressed(HERE / "prefill_small_bf16.npz", q_prompt=q, k_prompt=k, v_prompt=v, k_pool=case.k_pool,
                        v_pool=case.v_pool, page_table=case.page_table, context_lens=case.seq_lens, expected=out)


def fused_small():
    fc = make_fused_case(71, [30, 1, 77], [(9, 20)], 8, 2, 64, 16, "f16", block=20, garbage_tail=False)
    c = fc.case
    out = orc.paged_attention(fc.queries, c.k_pool, c.v_pool, c.page_table, c.seq_lens, fc.q2seq, fc.q_offset, "f16")
    np.savez_compressed(HERE / "fused_small_f16.npz", queries=fc.queries, k_pool=c.k_pool, v_pool=c.v_pool,
                        page_table=c.page_table, seq_lens=c.seq_lens, q2seq=fc.q2seq, q_offset=fc.q_offset,
                        expected=out)


def fill_small():
    rng = np.random.default_rng(72)
    hkv, hd, tpp, n_pages = 2, 32, 16, 12
    k_pool = randn_bits(rng, orc.k_cache_shape(n_pages, hkv, hd, tpp, "bf16"), "bf16")
    v_pool = randn_bits(rng, orc.v_cache_shape(n_pages, hkv, hd, tpp, "bf16"), "bf16")
    pt = rng.permutation(n_pages).astype(np.uint32).reshape(3, 4)
    q2seq = rng.integers(0, 3, size=37).astype(np.uint32)
    pos = np.zeros(37, np.int32)
    for s in range(3):  # distinct slots per sequence
        idx = np.nonzero(q2seq == s)[0]
        pos[idx] = rng.permutation(4 * tpp)[: len(idx)]
    nk = randn_bits(rng, (37, hkv, hd), "bf16")
    nv = randn_bits(rng, (37, hkv, hd), "bf16")
    ek, ev = orc.fill_kv_pages(nk, nv, k_pool, v_pool, pt, pos, q2seq)
    np.savez_compressed(HERE / "fill_small_bf16.npz", new_keys=nk, new_values=nv, k_pool=k_pool, v_pool=v_pool,
                        page_table=pt, write_pos=pos, q2seq=q2seq, expected_k=ek, expected_v=ev)


if __name__ == "__main__":
    config1()
    prefill_small()
    fused_small()
    fill_small()
    print("wrote", sorted(p.name for p in HERE.glob("*.npz")))
