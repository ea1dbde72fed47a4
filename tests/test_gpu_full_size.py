"""GPU parity at the benchmark's full sizes.

The workloads come from bench.py's own seeded generators (the exact inputs
the benchmark times).  Every output must be finite, and real-length
sequences are re-checked on the CPU oracle from a compacted copy of their
pages.  Tolerances (the contract of this path): bf16 atol/rtol 2e-2, fp16
atol/rtol 5e-3, outputs compared in float32; pools after fill_kv_pages
bit-exact.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import bench
from gpu_util import announce, host_bits, host_f32
from oracle import pal_oracle as orc
from pal_cases import assert_close

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _subset_pools(k_pool: torch.Tensor, v_pool: torch.Tensor, pt: np.ndarray, lens: np.ndarray, seqs, tpp: int):
    """Host bits of the pages that sequences `seqs` use (first lens[s] tokens),
    and their page table renumbered to the compacted pool."""
    used = []
    for s in seqs:
        used.extend(int(x) for x in pt[s, : (int(lens[s]) + tpp - 1) // tpp])
    uniq = np.unique(np.asarray(used, np.int64)) if used else np.zeros(1, np.int64)
    idx = torch.from_numpy(uniq).to(k_pool.device)
    kb = host_bits(k_pool.index_select(0, idx))
    vb = host_bits(v_pool.index_select(0, idx))
    remap = {int(p): i for i, p in enumerate(uniq)}
    width = max(1, max((int(lens[s]) + tpp - 1) // tpp for s in seqs))
    spt = np.zeros((len(seqs), width), np.uint32)
    for i, s in enumerate(seqs):
        for j in range((int(lens[s]) + tpp - 1) // tpp):
            spt[i, j] = remap[int(pt[s, j])]
    return kb, vb, spt


def _fused_oracle_rows(q_bits, kb, vb, spt, lens, q2s_local, offs, dtype, chunk=512):
    """Oracle of the fused op for rows of the compacted sequences, computed in
    row chunks (each row's result depends on its own limit only)."""
    out = np.zeros(q_bits.shape, np.float32)
    for r0 in range(0, len(q2s_local), chunk):
        sl = slice(r0, r0 + chunk)
        out[sl] = orc.paged_attention(q_bits[sl], kb, vb, spt, lens, q2s_local[sl], offs[sl], dtype)
    return out


def test_config4_full_size_fill_and_prefill():
    """Config 4 exactly as bench.py builds it: fill_kv_pages of the new chunks
    (bit-exact over the whole pool), then causal attention through the fused
    operator (finite everywhere; the longest chunk and the longest cache
    re-checked on the oracle)."""
    announce("config 4 full size: build")
    w = bench.PrefillWorkload(DEV)
    tpp = 16
    pt = w.page_table.cpu().numpy().astype(np.uint32)
    lens = w.seq_lens.cpu().numpy()
    k_before, v_before = host_bits(w.k_pool), host_bits(w.v_pool)
    announce(f"config 4 full size: fill {w.rows} tokens")
    w.fill()
    torch.cuda.synchronize()
    ek, ev = orc.fill_kv_pages(host_bits(w.new_k), host_bits(w.new_v), k_before, v_before, pt,
                               w.write_pos.cpu().numpy(), w.q2seq.cpu().numpy().astype(np.uint32))
    assert np.array_equal(host_bits(w.k_pool), ek), "K pool after fill differs from the oracle"
    assert np.array_equal(host_bits(w.v_pool), ev), "V pool after fill differs from the oracle"
    del k_before, v_before, ek, ev
    announce("config 4 full size: attention")
    out = w.attend()
    torch.cuda.synchronize()
    out_h = host_f32(out)
    assert out_h.shape == (w.rows, w.hq, w.hd)
    assert np.isfinite(out_h).all()
    longest_new = int(np.argmax(w.new))
    longest_cache = int(np.argmax(w.cached))
    seqs = sorted({longest_new, longest_cache})
    if len(seqs) == 1:
        seqs.append(int(np.argmin(w.new)))
    q2s = w.q2seq.cpu().numpy()
    offs = w.q_offset.cpu().numpy()
    kb, vb, spt = _subset_pools(w.k_pool, w.v_pool, pt, lens, seqs, tpp)
    q_bits = host_bits(w.queries)
    for i, s in enumerate(seqs):
        rows = np.nonzero(q2s == s)[0]
        ref = _fused_oracle_rows(q_bits[rows], kb, vb, spt, lens[seqs], np.full(len(rows), i, np.uint32),
                                 offs[rows], "bf16")
        assert_close(out_h[rows], ref, "bf16",
                     f"config 4 seq {s} (new {int(w.new[s])}, cached {int(w.cached[s])})")


def test_config5_full_size_fused():
    """Config 5 exactly as bench.py builds it (256 decode rows + 4 x 1024
    prefill rows, 64/8 heads, fp16, shuffled row blocks): finite everywhere;
    decode rows including the longest context, and the whole prefill chunk
    with the largest cache, re-checked on the oracle."""
    announce("config 5 full size: build")
    w = bench.FusedWorkload(DEV)
    tpp = 16
    pt = w.page_table.cpu().numpy().astype(np.uint32)
    lens = w.seq_lens.cpu().numpy()
    q2s = w.q2seq.cpu().numpy()
    offs = w.q_offset.cpu().numpy()
    announce("config 5 full size: fused call")
    out_h = host_f32(w.attend())
    assert out_h.shape == (w.rows, 64, 128)
    assert np.isfinite(out_h).all()
    dec_lens = lens[:256]
    pick_dec = sorted({int(np.argmax(dec_lens)), int(np.argmin(dec_lens)), 3, 77, 128, 200, 255})
    chunk_seq = 256 + int(np.argmax(lens[256:] - 1024))  # the prefill chunk on the largest cache
    seqs = pick_dec + [chunk_seq]
    kb, vb, spt = _subset_pools(w.k_pool, w.v_pool, pt, lens, seqs, tpp)
    q_bits = host_bits(w.queries)
    local = {s: i for i, s in enumerate(seqs)}
    rows = np.nonzero(np.isin(q2s, seqs))[0]
    ref = _fused_oracle_rows(q_bits[rows], kb, vb, spt, lens[seqs],
                             np.array([local[int(s)] for s in q2s[rows]], np.uint32), offs[rows], "f16")
    dec_rows = np.isin(q2s[rows], pick_dec)
    assert_close(out_h[rows][dec_rows], ref[dec_rows], "f16",
                 f"config 5 decode rows (ctx up to {int(dec_lens.max())})")
    assert_close(out_h[rows][~dec_rows], ref[~dec_rows], "f16",
                 f"config 5 prefill chunk on {int(lens[chunk_seq]) - 1024} cached")


@pytest.mark.parametrize("partition", [512, 0])
def test_config3_full_size_decode(partition):
    """Config 3 exactly as bench.py builds it (8 x U[32768, 131072] tokens,
    1 % of key rows x8), in the reference's two-pass form (partition 512) and
    the default equal-share form: finite everywhere, the longest and the
    shortest sequence re-checked on the oracle."""
    announce(f"config 3 full size partition {partition}: build")
    w = bench.long_context_workload(DEV)
    announce(f"config 3 full size partition {partition}: decode")
    out_h = host_f32(w.decode(partition))
    assert np.isfinite(out_h).all()
    seqs = sorted({int(np.argmax(w.lens_np)), int(np.argmin(w.lens_np))})
    kb, vb, spt = _subset_pools(w.k_pool, w.v_pool, w.pt_np.astype(np.uint32), w.lens_np, seqs, w.tpp)
    q_bits = host_bits(w.queries)[seqs]
    ref = orc.paged_attention_decode(q_bits, kb, vb, spt, w.lens_np[seqs], "bf16")
    assert_close(out_h[seqs], ref, "bf16", f"config 3 partition {partition} seqs {seqs} "
                                          f"(ctx {[int(w.lens_np[s]) for s in seqs]})")


def test_reference_signature_full_size():
    """The reference prefill signature as bench.py builds it (16 x 1024
    prompt rows on U[0,2048] cached history, 32/8 heads, HD 128, bf16):
    finite everywhere; the sequences with the longest and the shortest
    history re-checked on the oracle."""
    announce("reference-signature prefill full size: build")
    w = bench.PromptWorkload(DEV)
    announce("reference-signature prefill full size: run")
    out = w.attend()
    torch.cuda.synchronize()
    out_h = host_f32(out)
    P, hq, hd = w.prompt, w.hq, w.hd
    S = len(w.hist)
    assert out_h.shape == (S * P * hq, hd)
    assert np.isfinite(out_h).all()
    seqs = sorted({int(np.argmax(w.hist)), int(np.argmin(w.hist))})
    pt = w.page_table.cpu().numpy().astype(np.uint32)
    kb, vb, spt = _subset_pools(w.k_pool, w.v_pool, pt, np.maximum(w.hist, 1), seqs, 16)
    rows = np.concatenate([np.arange(s * P, (s + 1) * P) for s in seqs])
    q_bits, k_bits, v_bits = host_bits(w.q)[rows], host_bits(w.k)[rows], host_bits(w.v)[rows]
    ref = orc.paged_attention_prefill(q_bits, k_bits, v_bits, kb, vb, spt, w.hist[seqs], "bf16")
    for i, s in enumerate(seqs):
        got = out_h[s * P * hq:(s + 1) * P * hq]
        assert_close(got, ref[i * P * hq:(i + 1) * P * hq], "bf16", f"reference signature seq {s} (history {int(w.hist[s])})")


@pytest.mark.parametrize("partition", [512, 0])
def test_long_history_decode_524288(partition):
    """Batch-1 decode over a 524,288-token history, the top of the range the
    reference times (benchmarks/paged_attention/cpp/seq_len_vs_latency.cpp:
    210-223), at HD 128 bf16 with 4 query heads on 2 kv heads (the
    reference benchmark's 2:1 grouping, fewer heads so the oracle's fp32 copy
    of the pools fits host memory), 1 % of key rows x8.  Each segment is
    shared by hundreds (equal shares) or a thousand (partition 512)
    contributors, which the merge must combine."""
    announce(f"long-history decode 524288 tokens partition {partition}: build")
    w = bench.DecodeWorkload(21, num_seqs=1, ctx_lo=524288, ctx_hi=524288, hq=4, hkv=2, device=DEV)
    rng = np.random.default_rng(21)
    pos = rng.choice(524288, size=5242, replace=False)
    pi = torch.from_numpy(w.pt_np[0, pos // w.tpp].astype(np.int64)).to(DEV)
    si = torch.from_numpy((pos % w.tpp).astype(np.int64)).to(DEV)
    w.k_pool[pi, :, :, si, :] = w.k_pool[pi, :, :, si, :] * 8
    announce(f"long-history decode 524288 tokens partition {partition}: decode")
    out_h = host_f32(w.decode(partition))
    assert np.isfinite(out_h).all()
    ref = orc.paged_attention_decode(host_bits(w.queries), host_bits(w.k_pool), host_bits(w.v_pool),
                                     w.pt_np.astype(np.uint32), w.lens_np, "bf16")
    assert_close(out_h, ref, "bf16", f"long-history decode 524288 tokens, 4/2 heads, partition {partition}")
