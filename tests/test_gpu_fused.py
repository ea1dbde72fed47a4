"""GPU parity of the fused mixed-batch paged_attention against the CPU
oracle, and its agreement with the decode and prefill operators on the rows
they share.

Tolerances (the contract of this path): bf16 atol/rtol 2e-2, fp16 atol/rtol
5e-3, outputs compared in float32.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import proxy_attention_lab as pal
from gpu_util import announce, dev_bits, dev_index, host_bits, host_f32
from oracle import pal_oracle as orc
from pal_cases import assert_close, extreme_query_bits, make_fused_case, make_paged_case, make_prefill_case, randn_bits

pytestmark = pytest.mark.gpu
DTYPES = ["f16", "bf16"]


def _fused_gpu(case, q, q2seq, q_off, stream=None):
    out = pal.paged_attention(dev_bits(q, case.dtype), dev_bits(case.k_pool, case.dtype),
                              dev_bits(case.v_pool, case.dtype), dev_index(case.page_table, torch.uint32),
                              dev_index(case.seq_lens), dev_index(q2seq, torch.uint32), dev_index(q_off), stream)
    torch.cuda.synchronize()
    return out


def _check_fused(fc, what):
    c = fc.case
    announce(f"fused {what} R={len(fc.q2seq)} S={c.num_seqs} Hq={c.num_q_heads} Hkv={c.num_kv_heads} "
             f"HD={c.head_dim} TPP={c.tokens_per_page} {c.dtype}")
    out = host_f32(_fused_gpu(c, fc.queries, fc.q2seq, fc.q_offset))
    assert out.shape == fc.queries.shape
    ref = orc.paged_attention(fc.queries, c.k_pool, c.v_pool, c.page_table, c.seq_lens, fc.q2seq, fc.q_offset,
                              c.dtype)
    assert_close(out, ref, c.dtype, what)
    return out


@pytest.mark.parametrize("dtype", DTYPES)
def test_fused_mixed_small(dtype):
    """A config-5-like batch in miniature: GQA 8:1, decode rows interleaved
    with blocks of three prefill chunks."""
    rng = np.random.default_rng(50)
    dec = rng.integers(1, 900, size=40)
    fc = make_fused_case(50, dec, [(0, 100), (130, 64), (500, 257)], 64, 8, 128, 16, dtype, block=40)
    _check_fused(fc, "mixed")


@pytest.mark.parametrize("hd", [32, 64, 96, 128, 256])
def test_fused_head_dims(hd):
    fc = make_fused_case(hd, [17, 300, 1], [(20, 33), (0, 5)], 8, 2, hd, 32 if hd == 64 else 16, "bf16")
    _check_fused(fc, f"hd{hd}")


@pytest.mark.parametrize("heads", [(1, 1), (4, 1), (32, 8), (40, 2), (32, 32)])
def test_fused_gqa_groups(heads):
    hq, hkv = heads
    fc = make_fused_case(hq + hkv, [100, 2000, 0, 16], [(64, 70), (3, 140)], hq, hkv, 64, 16, "f16", block=32)
    _check_fused(fc, f"heads{heads}")


def test_fused_decode_rows_equal_decode_op():
    lens = [1, 15, 16, 17, 511, 3000, 0, 40]
    case = make_paged_case(60, lens, 32, 8, 128, 16, "bf16")
    q = randn_bits(np.random.default_rng(60), (len(lens), 32, 128), "bf16")
    announce("fused decode rows vs decode op")
    fused = host_f32(_fused_gpu(case, q, np.arange(len(lens), dtype=np.uint32), case.seq_lens.copy()))
    dec = pal.paged_attention_decode(dev_bits(q, "bf16"), dev_bits(case.k_pool, "bf16"), dev_bits(case.v_pool, "bf16"),
                                     dev_index(case.page_table, torch.uint32), dev_index(case.seq_lens))
    torch.cuda.synchronize()
    assert_close(fused, host_f32(dec), "bf16", "fused vs decode")
    ref = orc.paged_attention_decode(q, case.k_pool, case.v_pool, case.page_table, case.seq_lens, "bf16")
    assert_close(fused, ref, "bf16", "fused vs oracle")


def test_fused_after_fill_equals_prefill_op():
    """fill_kv_pages writes the prompt into the pages; the fused op over the
    prompt rows then matches the reference-signature prefill (dense prompt)."""
    hist, plen, hq, hkv, hd, tpp = [37, 0, 64], 48, 16, 4, 128, 16
    case, qp, kp, vp = make_prefill_case(61, hist, plen, hq, hkv, hd, tpp, "f16")
    S = case.num_seqs
    # room for the prompt: extend each page row with fresh pages
    need = [(h + plen + tpp - 1) // tpp for h in hist]
    width = max(need)
    base = case.k_pool.shape[0]
    extra = sum(n - (h + tpp - 1) // tpp for n, h in zip(need, hist))
    k_pool = np.concatenate([case.k_pool, np.zeros((extra,) + case.k_pool.shape[1:], np.uint16)])
    v_pool = np.concatenate([case.v_pool, np.zeros((extra,) + case.v_pool.shape[1:], np.uint16)])
    pt = np.zeros((S, width), np.uint32)
    nxt = base
    for s in range(S):
        have = (hist[s] + tpp - 1) // tpp
        pt[s, :have] = case.page_table[s, :have]
        for j in range(have, need[s]):
            pt[s, j] = nxt
            nxt += 1
    announce("fused after fill vs prefill op")
    kd, vd = dev_bits(k_pool, "f16"), dev_bits(v_pool, "f16")
    ptd = dev_index(pt, torch.uint32)
    pos = np.concatenate([h + np.arange(plen) for h in hist]).astype(np.int32)
    q2s = np.repeat(np.arange(S), plen).astype(np.uint32)
    pal.fill_kv_pages(dev_bits(kp, "f16"), dev_bits(vp, "f16"), kd, vd, ptd, dev_index(pos),
                      dev_index(q2s, torch.uint32))
    lens_total = np.array(hist, np.int32) + plen
    fused = pal.paged_attention(dev_bits(qp, "f16"), kd, vd, ptd, dev_index(lens_total),
                                dev_index(q2s, torch.uint32), dev_index(pos + 1))
    pre = pal.paged_attention_prefill(dev_bits(qp, "f16"), dev_bits(kp, "f16"), dev_bits(vp, "f16"),
                                      dev_bits(case.k_pool, "f16"), dev_bits(case.v_pool, "f16"),
                                      dev_index(case.page_table, torch.uint32), dev_index(case.seq_lens))
    torch.cuda.synchronize()
    fused = host_f32(fused).reshape(-1, hd)
    assert_close(fused, host_f32(pre), "f16", "fused vs prefill")
    ref = orc.paged_attention_prefill(qp, kp, vp, case.k_pool, case.v_pool, case.page_table, case.seq_lens, "f16")
    assert_close(fused, ref, "f16", "fused vs oracle")


def test_fused_edge_rows():
    """Offsets of 0, negative and past the length; a row naming no sequence;
    a run longer than a tile; runs of two rows."""
    case = make_paged_case(62, [50, 300, 7], 8, 2, 64, 16, "bf16")
    rng = np.random.default_rng(62)
    q2seq = np.array([0, 0, 1, 2, 9, 1, 1, 1] + [1] * 150 + [2, 0], np.uint32)
    off = np.array([0, -3, 1000, 7, 5, 1, 2, 3] + list(range(4, 154)) + [1, 50], np.int32)
    q = randn_bits(rng, (len(q2seq), 8, 64), "bf16")
    announce("fused edge rows")
    out = host_f32(_fused_gpu(case, q, q2seq, off))
    ref = orc.paged_attention(q, case.k_pool, case.v_pool, case.page_table, case.seq_lens, q2seq, off, "bf16")
    assert_close(out, ref, "bf16", "edge rows")
    assert np.all(out[[0, 1, 4]] == 0)


def test_fused_many_rows_planner_chunks():
    """More than 1024 rows (the decode workers' row scan carries runs across
    its passes of 4096 rows): 1100 decode rows plus a 1500-row prompt run."""
    rng = np.random.default_rng(63)
    dec = rng.integers(0, 80, size=1100)
    fc = make_fused_case(63, dec, [(200, 1500)], 8, 1, 64, 16, "f16", block=1500, garbage_tail=False)
    _check_fused(fc, "many rows")


def test_fused_lone_rows_beyond_the_list():
    """More lone (decode) rows with keys than the fused kernel's in-LDS list
    holds (2048): the decode workers claim batches of 64 rows and compute each
    lone row whole.  Rows without keys and a prompt run interleave."""
    rng = np.random.default_rng(65)
    dec = rng.integers(0, 400, size=2300)
    fc = make_fused_case(65, dec, [(50, 300)], 8, 2, 64, 16, "bf16", block=100)
    assert int(np.count_nonzero(dec)) > 2048
    _check_fused(fc, "claiming mode")


def test_fused_deterministic_and_empty():
    fc = make_fused_case(64, [900, 3], [(100, 300)], 32, 8, 128, 16, "bf16", block=100)
    c = fc.case
    announce("fused determinism")
    a = host_bits(_fused_gpu(c, fc.queries, fc.q2seq, fc.q_offset))
    b = host_bits(_fused_gpu(c, fc.queries, fc.q2seq, fc.q_offset))
    assert np.array_equal(a, b)
    empty = pal.paged_attention(dev_bits(fc.queries[:0], "bf16"), dev_bits(c.k_pool, "bf16"),
                                dev_bits(c.v_pool, "bf16"), dev_index(c.page_table), dev_index(c.seq_lens),
                                dev_index(fc.q2seq[:0]), dev_index(fc.q_offset[:0]))
    assert empty.shape == (0, 32, 128)


@pytest.mark.parametrize("tpp", [16, 32])
def test_fused_long_history_window(tpp):
    """A prefill run over a cache longer than 8192 keys (window mode stages
    its page ids in chunks of 512 entries and rotates them), beside decode
    rows of similar length."""
    fc = make_fused_case(70 + tpp, [100, 30000], [(26000 if tpp == 16 else 38000, 64), (9000, 40)], 32, 8, 128,
                         tpp, "bf16", block=64)
    _check_fused(fc, f"long history window tpp{tpp}")


@pytest.mark.parametrize("dtype", DTYPES)
def test_fused_query_magnitudes(dtype):
    """A mixed batch whose query heads span the dtype's range (zeros, tiny,
    large, mixed, near the range ends), in its decode rows and its tiles
    (the large heads held to the tiles' exact range)."""
    fc = make_fused_case(74, [5, 300, 1200], [(0, 70), (200, 130)], 16, 4, 128, 16, dtype)
    fc.queries = extreme_query_bits(np.random.default_rng(74), fc.queries.shape, dtype, tiles=True)
    out = _check_fused(fc, f"query magnitudes {dtype}")
    assert np.isfinite(out).all()
