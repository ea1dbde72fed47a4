"""Pools larger than 4 GiB: every kernel must address pages by 64-bit byte
offsets (an MI355X holds 288 GB, so a KV pool can span far more than 2^32
bytes).

Each case is built compact on the host, as the oracle takes it, and placed
on the device at page ids `base ..`, where `base` is chosen so that the
case's first page starts past 5 GiB of its pool (so K and V pools are more
than 5 GiB each).  The page table is shifted by the same base, so its
unused entries still name valid pages.  Attention results must match the
oracle on the compact case within the dtype's tolerance (bf16 atol/rtol 2e-2,
fp16 5e-3), and fills and page copies must be bit-exact.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import proxy_attention_lab as pal
from gpu_util import DEV, announce, dev_bits, dev_index, host_bits, host_f32
from oracle import pal_oracle as orc
from pal_cases import assert_close, make_fused_case, make_paged_case, make_prefill_case, randn_bits
from test_gpu_fill import _random_fill_case
from test_gpu_fp8_rope import dev_codes, fp8_case

pytestmark = pytest.mark.gpu
BASE_BYTES = 5 << 30  # the case's first page starts past this offset of its pool


@pytest.fixture(autouse=True)
def _release_pools():
    yield
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def _base(pool: np.ndarray) -> int:
    """First page id whose byte offset in a pool of these pages is >= BASE_BYTES."""
    page_bytes = pool[0].nbytes
    return -(-BASE_BYTES // page_bytes)


def _big(small: torch.Tensor, base: int) -> torch.Tensor:
    """A device tensor of base + len(small) pages (or scale rows) holding small
    at rows base ..; the rows below are left uninitialized."""
    raw = {1: torch.uint8, 2: torch.int16, 4: torch.int32}[small.element_size()]  # copied as bits
    big = torch.empty((base + small.shape[0], *small.shape[1:]), dtype=raw, device=DEV)
    big[base:].copy_(small.view(raw))
    big = big.view(small.dtype)
    assert big.numel() * big.element_size() > BASE_BYTES or small.element_size() == 4
    return big


def _shifted(page_table: np.ndarray, base: int) -> torch.Tensor:
    pt = page_table.astype(np.int64) + base
    assert pt.max() < 2**32
    return dev_index(pt.astype(np.uint32), torch.uint32)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("partition", [0, 512])
def test_large_pool_decode(dtype, partition):
    lens = [1, 17, 300, 2049, 5000, 0, 16]
    case = make_paged_case(91, lens, 32, 8, 128, 16, dtype)
    q = randn_bits(np.random.default_rng(91), (len(lens), 32, 128), dtype)
    base = _base(case.k_pool)
    announce(f"large pool decode {dtype} partition={partition} base page {base}")
    k = _big(dev_bits(case.k_pool, dtype), base)
    v = _big(dev_bits(case.v_pool, dtype), base)
    out = pal.paged_attention_decode(dev_bits(q, dtype), k, v, _shifted(case.page_table, base),
                                     dev_index(case.seq_lens), partition_size=partition)
    torch.cuda.synchronize()
    ref = orc.paged_attention_decode(q, case.k_pool, case.v_pool, case.page_table, case.seq_lens, dtype)
    assert_close(host_f32(out), ref, dtype, f"large pool decode {dtype} p{partition}")


@pytest.mark.parametrize("partition", [0, 512])
def test_large_pool_decode_fp8(partition):
    lens = [1, 17, 300, 2049, 5000, 0, 16]
    rng = np.random.default_rng(92)
    case = make_paged_case(92, lens, 32, 8, 128, 16, "bf16")
    kc, vc, ks, vs = fp8_case(case, rng)
    q = randn_bits(rng, (len(lens), 32, 128), "bf16")
    base = _base(kc)
    announce(f"large pool decode fp8 partition={partition} base page {base}")
    out = pal.paged_attention_decode(dev_bits(q, "bf16"), _big(dev_codes(kc), base), _big(dev_codes(vc), base),
                                     _shifted(case.page_table, base), dev_index(case.seq_lens),
                                     partition_size=partition, k_scales=_big(torch.from_numpy(ks).to(DEV), base),
                                     v_scales=_big(torch.from_numpy(vs).to(DEV), base))
    torch.cuda.synchronize()
    ref = orc.paged_attention_decode(q, kc, vc, case.page_table, case.seq_lens, "bf16", kv_scales=(ks, vs))
    assert_close(host_f32(out), ref, "bf16", f"large pool decode fp8 p{partition}")


@pytest.mark.parametrize("tpp", [16, 24])
def test_large_pool_prefill(tpp):
    """Pages of 16 tokens take the direct-to-LDS copies, 24 the register path."""
    case, q, k, v = make_prefill_case(93 + tpp, [0, 37, 300, 1000], 45, 16, 4, 128, tpp, "bf16")
    base = _base(case.k_pool)
    announce(f"large pool prefill tpp={tpp} base page {base}")
    out = pal.paged_attention_prefill(dev_bits(q, "bf16"), dev_bits(k, "bf16"), dev_bits(v, "bf16"),
                                      _big(dev_bits(case.k_pool, "bf16"), base),
                                      _big(dev_bits(case.v_pool, "bf16"), base),
                                      _shifted(case.page_table, base), dev_index(case.seq_lens))
    torch.cuda.synchronize()
    ref = orc.paged_attention_prefill(q, k, v, case.k_pool, case.v_pool, case.page_table, case.seq_lens, "bf16")
    assert_close(host_f32(out), ref, "bf16", f"large pool prefill tpp{tpp}")


@pytest.mark.parametrize("fp8", [False, True])
def test_large_pool_fused(fp8):
    rng = np.random.default_rng(94)
    fc = make_fused_case(94, [1, 17, 300, 2049, 0, 700], [(0, 70), (130, 64), (900, 129)], 32, 8, 128, 16, "bf16",
                         block=40)
    c = fc.case
    if fp8:
        kc, vc, ks, vs = fp8_case(c, rng)
        base = _base(kc)
        kp, vp = _big(dev_codes(kc), base), _big(dev_codes(vc), base)
        scales = dict(k_scales=_big(torch.from_numpy(ks).to(DEV), base),
                      v_scales=_big(torch.from_numpy(vs).to(DEV), base))
        ko, vo, kvs = kc, vc, (ks, vs)
    else:
        base = _base(c.k_pool)
        kp, vp = _big(dev_bits(c.k_pool, "bf16"), base), _big(dev_bits(c.v_pool, "bf16"), base)
        scales, ko, vo, kvs = {}, c.k_pool, c.v_pool, None
    announce(f"large pool fused fp8={fp8} base page {base}")
    out = pal.paged_attention(dev_bits(fc.queries, "bf16"), kp, vp, _shifted(c.page_table, base),
                              dev_index(c.seq_lens), dev_index(fc.q2seq, torch.uint32), dev_index(fc.q_offset),
                              **scales)
    torch.cuda.synchronize()
    ref = orc.paged_attention(fc.queries, ko, vo, c.page_table, c.seq_lens, fc.q2seq, fc.q_offset, "bf16",
                              kv_scales=kvs)
    assert_close(host_f32(out), ref, "bf16", f"large pool fused fp8={fp8}")


@pytest.mark.parametrize("shape,consecutive", [
    ((64, 8, 128, 16, 300, 64, 4), False),      # a decode step's tokens: the per-token kernel
    ((4096, 8, 128, 16, 1200, 4, 256), True),   # prefill chunks: the windowed kernel
])
def test_large_pool_fill(shape, consecutive):
    kw = _random_fill_case(95, *shape, consecutive=consecutive)
    base = _base(kw["k_pool"])
    announce(f"large pool fill {shape[0]} tokens base page {base}")
    k = _big(dev_bits(kw["k_pool"], "bf16"), base)
    v = _big(dev_bits(kw["v_pool"], "bf16"), base)
    pal.fill_kv_pages(dev_bits(kw["new_k"], "bf16"), dev_bits(kw["new_v"], "bf16"), k, v,
                      _shifted(kw["page_table"], base), dev_index(kw["write_pos"]),
                      dev_index(kw["q2seq"], torch.uint32))
    torch.cuda.synchronize()
    ek, ev = orc.fill_kv_pages(**kw)
    assert np.array_equal(host_bits(k[base:]), ek)
    assert np.array_equal(host_bits(v[base:]), ev)


def test_large_pool_copy_pages():
    """Page moves and page-table remapping between ids past the 4 GiB mark."""
    from proxy_attention_lab.page_pool import PagePool

    rng = np.random.default_rng(96)
    pages = 64
    kp = rng.integers(0, 65536, size=(pages, 8, 16, 16, 8), dtype=np.uint16)
    vp = rng.integers(0, 65536, size=(pages, 8, 128, 16), dtype=np.uint16)
    base = _base(kp)
    announce(f"large pool copy_pages base page {base}")
    k = _big(dev_bits(kp, "bf16"), base)
    v = _big(dev_bits(vp, "bf16"), base)
    src = np.arange(32, 48, dtype=np.uint32)
    dst = rng.permutation(np.arange(0, 32, dtype=np.uint32))[:16]
    table = rng.integers(0, pages, size=(4, 20), dtype=np.uint32)
    pt = _shifted(table, base)
    PagePool.apply_moves(src + base, dst + base, k, v, page_tables=(pt,))
    torch.cuda.synchronize()
    ek, ev = kp.copy(), vp.copy()
    ek[dst], ev[dst] = kp[src], vp[src]
    remap = np.arange(pages, dtype=np.uint32)
    remap[src] = dst
    assert np.array_equal(host_bits(k[base:]), ek)
    assert np.array_equal(host_bits(v[base:]), ev)
    assert np.array_equal(pt.view(torch.int32).cpu().numpy().view(np.uint32).astype(np.int64) - base, remap[table])


@pytest.mark.parametrize("kv", ["bf16", "fp8"])
def test_large_pool_rope_fill(kv):
    """The RoPE fill (fp32 rows, NeoX, queries rotated too) into pages past the
    5 GiB mark: pools and rotated queries bit-exact."""
    from test_gpu_fp8_rope import dev_f32, dev_pool, fill_layout, host_pool, src_values

    hkv, hq, hd, tpp = 4, 16, 128, 16
    k, v, pt, pos, q2s, (ks, vs) = fill_layout(97, hkv, hd, tpp, kv)
    rng = np.random.default_rng(97)
    n = len(pos)
    nk = src_values(rng, (n, hkv, hd), "f32", 2.0)
    nv = src_values(rng, (n, hkv, hd), "f32", 2.0)
    q = src_values(rng, (n, hq, hd), "f32", 2.0)
    table = pal.rope_cos_sin_cache(512, hd, 10000.0, device=DEV)
    base = _base(k)
    announce(f"large pool rope fill {kv} base page {base}")
    kd, vd = _big(dev_pool(k, kv), base), _big(dev_pool(v, kv), base)
    extra = {}
    if kv == "fp8":
        extra = dict(k_scales=_big(torch.from_numpy(ks).to(DEV), base),
                     v_scales=_big(torch.from_numpy(vs).to(DEV), base))
    _, _, qo = pal.rope_fill_kv_pages(dev_f32(nk, "f32"), dev_f32(nv, "f32"), kd, vd, _shifted(pt, base),
                                      dev_index(pos), dev_index(q2s, torch.uint32), table, queries=dev_f32(q, "f32"),
                                      rotary_dim=hd, style="neox", query_dtype=torch.bfloat16, **extra)
    torch.cuda.synchronize()
    ek, ev, eq = orc.fill_kv_pages_ex(nk, nv, k, v, kv, pt, pos, q2s, k_scales=ks if kv == "fp8" else None,
                                      v_scales=vs if kv == "fp8" else None, rope=(table.cpu().numpy(), hd, "neox"),
                                      queries=q, q_out_dtype="bf16")
    assert np.array_equal(host_pool(kd[base:], kv), ek), "K pool differs"
    assert np.array_equal(host_pool(vd[base:], kv), ev), "V pool differs"
    assert np.array_equal(host_bits(qo), eq), "rotated queries differ"
