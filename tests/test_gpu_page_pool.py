"""GPU: page-pool compaction moves pages bit-exactly and leaves attention
unchanged.

A pool is fragmented by allocating pages for interleaved sequences and
freeing some of them; compaction then moves the live pages to [0, live) on
the GPU.  Checked: both pools (and fp8 scale rows) equal the oracle's moves
applied to the old pools, the page tables equal the oracle's remap, and
decode through the new tables returns the same bits as before.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import proxy_attention_lab as pal
from gpu_util import DEV, announce, dev_bits, dev_index, host_bits
from oracle import pal_oracle as orc
from pal_cases import randn_bits

pytestmark = pytest.mark.gpu


def _fragmented(pool, rng, n_seqs=24, tpp=16):
    """Allocate pages for n_seqs sequences a few pages at a time in turn,
    then free every third sequence.  Returns (lens, page lists) of the
    survivors."""
    lens = rng.integers(1, 600, n_seqs)
    need = [(int(l) + tpp - 1) // tpp for l in lens]
    pages = [[] for _ in range(n_seqs)]
    while any(len(pages[s]) < need[s] for s in range(n_seqs)):
        for s in range(n_seqs):
            k = min(int(rng.integers(1, 4)), need[s] - len(pages[s]))
            if k > 0:
                pages[s].extend(int(x) for x in pool.allocate(k))
    keep = [s for s in range(n_seqs) if s % 3 != 1]
    for s in range(n_seqs):
        if s % 3 == 1:
            pool.free(pages[s])
    return lens[keep].astype(np.int32), [pages[s] for s in keep]


@pytest.mark.parametrize("kv", ["bf16", "fp8"])
def test_compaction_moves_pages_and_keeps_decode(kv):
    rng = np.random.default_rng(40 if kv == "bf16" else 41)
    num_pages, hkv, hd, tpp, hq = 700, 4, 128, 16, 16
    pool = pal.PagePool(num_pages)
    lens, plist = _fragmented(pool, rng)
    S = len(lens)
    width = max(len(p) for p in plist)
    pt = np.zeros((S, width), np.uint32)
    for s, pg in enumerate(plist):
        pt[s, : len(pg)] = pg
    x = orc.stripe_size(kv)
    if kv == "fp8":
        k = orc.quantize_fp8(rng.standard_normal((num_pages, hkv, hd // x, tpp, x)).astype(np.float32), 1.0 / 64)
        v = orc.quantize_fp8(rng.standard_normal((num_pages, hkv, hd, tpp)).astype(np.float32), 1.0 / 64)
        ks = rng.uniform(0.01, 0.03, (num_pages, hkv)).astype(np.float32)
        vs = rng.uniform(0.01, 0.03, (num_pages, hkv)).astype(np.float32)
        kd = torch.from_numpy(k).to(DEV).view(torch.float8_e4m3fn)
        vd = torch.from_numpy(v).to(DEV).view(torch.float8_e4m3fn)
        ksd, vsd = torch.from_numpy(ks).to(DEV), torch.from_numpy(vs).to(DEV)
        extra = dict(k_scales=ksd, v_scales=vsd)
    else:
        k = randn_bits(rng, (num_pages, hkv, hd // x, tpp, x), "bf16")
        v = randn_bits(rng, (num_pages, hkv, hd, tpp), "bf16")
        kd, vd = dev_bits(k, "bf16"), dev_bits(v, "bf16")
        extra = {}
    q = dev_bits(randn_bits(rng, (S, hq, hd), "bf16"), "bf16")
    ptd = dev_index(pt, torch.uint32)
    lensd = dev_index(lens)
    announce(f"page-pool compaction {kv}: {pool.num_used} live of {num_pages}")
    before = host_bits(pal.paged_attention_decode(q, kd, vd, ptd, lensd, **extra))
    src, dst = pool.compaction_plan()
    assert src.size > 0
    pal.PagePool.apply_moves(src, dst, kd, vd, [ptd], **extra)
    torch.cuda.synchronize()
    # pools and tables against the oracle
    host = (lambda t: t.view(torch.uint8).cpu().numpy()) if kv == "fp8" else host_bits
    assert np.array_equal(host(kd), orc.apply_moves(k, src, dst))
    assert np.array_equal(host(vd), orc.apply_moves(v, src, dst))
    if kv == "fp8":
        assert np.array_equal(ksd.cpu().numpy(), orc.apply_moves(ks, src, dst))
        assert np.array_equal(vsd.cpu().numpy(), orc.apply_moves(vs, src, dst))
    new_pt = ptd.view(torch.int32).cpu().numpy().view(np.uint32)
    assert np.array_equal(new_pt, orc.remap_table(pt, src, dst, num_pages))
    live = np.concatenate([new_pt[s, : (int(l) + tpp - 1) // tpp] for s, l in enumerate(lens)])
    assert live.max() < pool.num_used  # the live pages are now [0, live)
    after = host_bits(pal.paged_attention_decode(q, kd, vd, ptd, lensd, **extra))
    assert np.array_equal(before, after), "decode changed across compaction"


def test_rejected_compact_leaves_allocator_and_tables():
    """An int64 page table, wrong-shaped scales or a pool of another size are
    rejected before the plan is recorded or any page moves."""
    num_pages, hkv, hd, tpp = 16, 2, 64, 16
    pool = pal.PagePool(num_pages)
    pool.allocate(10)
    pool.free([0, 3, 4])
    k = torch.arange(num_pages * hkv * hd * tpp, dtype=torch.float32, device=DEV).to(torch.bfloat16)
    k = k.view(num_pages, hkv, hd // 8, tpp, 8)
    v = k.clone().view(num_pages, hkv, hd, tpp)
    k0, v0 = k.clone(), v.clone()
    good = dev_index(np.array([[1, 2, 5, 6], [7, 8, 9, 0]], np.uint32), torch.uint32)
    bad64 = good.view(torch.int32).to(torch.int64)
    announce("page-pool compaction rejected before planning")
    with pytest.raises(ValueError, match="page tables"):
        pool.compact(k, v, [good, bad64])
    with pytest.raises(ValueError, match="k_scales"):
        pool.compact(k, v, [good], k_scales=torch.ones((num_pages, hkv + 1), device=DEV),
                     v_scales=torch.ones((num_pages, hkv), device=DEV))
    with pytest.raises(ValueError, match="pages"):
        pool.compact(k[:8], v[:8], [good])
    torch.cuda.synchronize()
    assert pool.num_free == 9
    assert torch.equal(k, k0) and torch.equal(v, v0)
    assert good.view(torch.int32).tolist() == [[1, 2, 5, 6], [7, 8, 9, 0]]
    assert bad64.tolist() == [[1, 2, 5, 6], [7, 8, 9, 0]]
    # the accepted call then compacts as planned: live pages 1,2,5..9 -> [0, 7)
    assert pool.compact(k, v, [good]) == 3
    torch.cuda.synchronize()
    src, dst = np.array([7, 8, 9], np.uint32), np.array([0, 3, 4], np.uint32)
    assert np.array_equal(good.view(torch.int32).cpu().numpy().view(np.uint32),
                          orc.remap_table(np.array([[1, 2, 5, 6], [7, 8, 9, 0]], np.uint32), src, dst, num_pages))
    assert torch.equal(k[0], k0[7]) and torch.equal(v[4], v0[9])
