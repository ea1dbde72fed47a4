"""GPU parity of fill_kv_pages: bit-exact against the CPU oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import kat_cases
import proxy_attention_lab as pal
from gpu_util import announce, dev_bits, dev_index, host_bits
from oracle import pal_oracle as orc

pytestmark = pytest.mark.gpu
DTYPES = ["f16", "bf16"]


def _run(kw, dtype, copy=False):
    k = dev_bits(kw["k_pool"], dtype)
    v = dev_bits(kw["v_pool"], dtype)
    k_out, v_out = pal.fill_kv_pages(
        dev_bits(kw["new_k"], dtype), dev_bits(kw["new_v"], dtype), k, v,
        dev_index(kw["page_table"], torch.uint32), dev_index(kw["write_pos"]),
        dev_index(kw["q2seq"], torch.uint32), copy=copy)
    torch.cuda.synchronize()
    return k, v, k_out, v_out


@pytest.mark.parametrize("dtype", DTYPES)
def test_fill_known_answers(dtype):
    for name, kw, ek, ev in kat_cases.fill_cases(dtype):
        announce(f"fill KAT {name} {dtype}")
        _, _, k_out, v_out = _run(kw, dtype)
        assert np.array_equal(host_bits(k_out), ek), name
        assert np.array_equal(host_bits(v_out), ev), name


def _random_fill_case(seed, n, hkv, hd, tpp, pages, seqs, width, consecutive=False):
    rng = np.random.default_rng(seed)
    pt = rng.permutation(pages)[: seqs * width].reshape(seqs, width).astype(np.uint32)
    if consecutive:  # prefill-like chunks: runs of consecutive positions per sequence
        q2s, pos = [], []
        per = n // seqs
        for s in range(seqs):
            start = int(rng.integers(0, width * tpp - per + 1))
            q2s += [s] * per
            pos += list(range(start, start + per))
        q2s, pos = np.asarray(q2s, np.uint32), np.asarray(pos, np.int32)
    else:
        pairs = rng.permutation(seqs * width * tpp)[:n]
        q2s = (pairs // (width * tpp)).astype(np.uint32)
        pos = (pairs % (width * tpp)).astype(np.int32)
    n = len(q2s)
    return dict(
        new_k=rng.integers(0, 65536, size=(n, hkv, hd), dtype=np.uint16),
        new_v=rng.integers(0, 65536, size=(n, hkv, hd), dtype=np.uint16),
        k_pool=rng.integers(0, 65536, size=(pages, hkv, hd // 8, tpp, 8), dtype=np.uint16),
        v_pool=rng.integers(0, 65536, size=(pages, hkv, hd, tpp), dtype=np.uint16),
        page_table=pt, write_pos=pos, q2seq=q2s,
    )


FILL_SHAPES = [  # (n, hkv, hd, tpp, pages, seqs, width)
    (1, 1, 64, 2, 4, 1, 2),
    (33, 2, 32, 4, 40, 3, 8),
    (64, 8, 128, 16, 300, 64, 4),
    (100, 4, 256, 32, 90, 5, 8),
    (257, 1, 80, 16, 80, 2, 30),
    (500, 8, 64, 8, 200, 10, 16),
]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", FILL_SHAPES)
def test_fill_random_bit_exact(shape, dtype):
    announce(f"fill random {shape} {dtype}")
    kw = _random_fill_case(sum(shape), *shape)
    _, _, k_out, v_out = _run(kw, dtype)
    ek, ev = orc.fill_kv_pages(**kw)
    assert np.array_equal(host_bits(k_out), ek)
    assert np.array_equal(host_bits(v_out), ev)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("hd,tpp", [(128, 16), (64, 32), (256, 16), (256, 32)])
def test_fill_prefill_chunks_bit_exact(dtype, hd, tpp):
    """Prefill-sized batches (4096 tokens in 4 runs of consecutive positions)
    take the windowed kernel: every head dim's window size and page size."""
    announce(f"fill consecutive chunks {dtype} hd={hd} tpp={tpp}")
    kw = _random_fill_case(5 + hd + tpp, 4096, 8, hd, tpp, 19200 // tpp, 4, 4096 // tpp, consecutive=True)
    _, _, k_out, v_out = _run(kw, dtype)
    ek, ev = orc.fill_kv_pages(**kw)
    assert np.array_equal(host_bits(k_out), ek)
    assert np.array_equal(host_bits(v_out), ev)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n", [256, 257])
def test_fill_small_batch_threshold_bit_exact(n, dtype):
    """Batches of up to 256 same-dtype tokens are written one 8-dim chunk per
    thread, larger ones through the windowed kernel: a run of n consecutive
    positions from a random start (partial pages at both ends) on both
    sides of the switch."""
    announce(f"fill small-batch threshold n={n} {dtype}")
    kw = _random_fill_case(n, n, 8, 128, 16, 240, 1, 40, consecutive=True)
    assert len(kw["q2seq"]) == n
    _, _, k_out, v_out = _run(kw, dtype)
    ek, ev = orc.fill_kv_pages(**kw)
    assert np.array_equal(host_bits(k_out), ek)
    assert np.array_equal(host_bits(v_out), ev)


def test_fill_in_place_and_copy_semantics():
    announce("fill in-place vs copy")
    kw = _random_fill_case(9, 20, 2, 64, 16, 12, 2, 4)
    k, v, k_out, v_out = _run(kw, "bf16")
    assert k_out is k and v_out is v  # in place by default
    ek, ev = orc.fill_kv_pages(**kw)
    k2, v2, k2_out, v2_out = _run(kw, "bf16", copy=True)
    assert k2_out is not k2
    assert np.array_equal(host_bits(k2), kw["k_pool"]) and np.array_equal(host_bits(v2), kw["v_pool"])
    assert np.array_equal(host_bits(k2_out), ek) and np.array_equal(host_bits(v2_out), ev)


def test_fill_zero_tokens_is_noop():
    announce("fill zero tokens")
    kw = _random_fill_case(10, 4, 2, 64, 16, 12, 2, 4)
    kw["new_k"] = kw["new_k"][:0]
    kw["new_v"] = kw["new_v"][:0]
    _, _, k_out, v_out = _run(kw, "f16")
    assert np.array_equal(host_bits(k_out), kw["k_pool"])
    assert np.array_equal(host_bits(v_out), kw["v_pool"])


def test_fill_skips_out_of_range_destinations():
    """Tokens pointing outside the page table or pool are dropped by the
    kernel's bounds checks; all other tokens land normally."""
    announce("fill out-of-range destinations")
    kw = _random_fill_case(11, 8, 2, 64, 16, 12, 2, 4)
    kw["q2seq"][1] = 5  # no such sequence
    kw["write_pos"][2] = -3  # negative position
    kw["write_pos"][3] = 4 * 16 + 1  # beyond the page-table width
    kw["page_table"][int(kw["q2seq"][4]), int(kw["write_pos"][4]) // 16] = 999  # page id beyond the pool
    _, _, k_out, v_out = _run(kw, "bf16")
    pt, q2s, pos = kw["page_table"], kw["q2seq"].astype(np.int64), kw["write_pos"].astype(np.int64)
    keep = np.array([
        q2s[t] < pt.shape[0] and 0 <= pos[t] < pt.shape[1] * 16 and pt[q2s[t], pos[t] // 16] < 12
        for t in range(8)
    ])
    assert not keep[[1, 2, 3, 4]].any() and keep.sum() >= 1
    sub = dict(kw, new_k=kw["new_k"][keep], new_v=kw["new_v"][keep], write_pos=kw["write_pos"][keep],
               q2seq=kw["q2seq"][keep])
    ek, ev = orc.fill_kv_pages(**sub)
    assert np.array_equal(host_bits(k_out), ek)
    assert np.array_equal(host_bits(v_out), ev)
