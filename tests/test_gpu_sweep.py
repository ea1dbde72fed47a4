"""Seeded random sweeps of the attention operators against the CPU oracle.

Each case draws its shape from the supported space (dtype, head dim, page
size, GQA group, partition size, fp8 pools) and its sequence lengths from a
mix of block/page/partition boundaries (n*16 - 1, n*16, n*16 + 1, ...) and
uniform draws, with some cases carrying key outliers that move the softmax
max late in a sequence.  Case i uses seed i, so a failure names a case that
can be rebuilt on the CPU.

Tolerances (the contract of this path): bf16 atol/rtol 2e-2, fp16 atol/rtol
5e-3, outputs compared in float32.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import proxy_attention_lab as pal
from gpu_util import announce, dev_bits, dev_index, host_f32
from oracle import pal_oracle as orc
from pal_cases import assert_close, make_fused_case, make_paged_case, make_prefill_case, randn_bits
from test_gpu_fp8_rope import dev_codes, fp8_case

pytestmark = pytest.mark.gpu
DEV = "cuda:0"

EDGES = [0, 1, 2, 15, 16, 17, 31, 32, 33, 63, 64, 65, 127, 128, 129, 255, 256, 257, 511, 512, 513,
         1023, 1024, 1025, 2047, 2048, 2049, 4095, 4096, 4097]
# context work per case (sum of lengths x q heads x head dim) stays below this,
# so the oracle finishes each case in about a second
BUDGET = 6e7


def _lens(rng, n, cap):
    out = []
    for _ in range(n):
        out.append(int(rng.choice(EDGES)) if rng.random() < 0.6 else int(rng.integers(0, cap)))
    return out


def _heads(rng):
    hkv = int(rng.choice([1, 2, 4, 8]))
    group = int(rng.choice([1, 2, 3, 4, 5, 8, 16, 20, 32]))
    while hkv * group > 64:
        hkv //= 2
    return max(hkv, 1) * group, max(hkv, 1)


def _fit(lens, hq, hd):
    while sum(lens) * hq * hd > BUDGET and max(lens) > 1:
        i = int(np.argmax(lens))
        lens[i] //= 2
    return lens


def _pools(case, rng, fp8):
    """The case's pools on the device and as the oracle takes them: its 16-bit
    pools, or fp8 codes with per-(page, kv head) scales.  Returns (k_pool,
    v_pool, scale kwargs of the op, (k, v) for the oracle, kv_scales for the
    oracle)."""
    if not fp8:
        return (dev_bits(case.k_pool, case.dtype), dev_bits(case.v_pool, case.dtype), {},
                (case.k_pool, case.v_pool), None)
    kc, vc, ks, vs = fp8_case(case, rng)
    scales = dict(k_scales=torch.from_numpy(ks).to(DEV), v_scales=torch.from_numpy(vs).to(DEV))
    return dev_codes(kc), dev_codes(vc), scales, (kc, vc), (ks, vs)


def _decode_case(i):
    rng = np.random.default_rng(1000 + i)
    dtype = "bf16" if rng.random() < 0.6 else "f16"
    fp8 = rng.random() < 0.35
    hd = int(rng.choice([64, 128, 256] if fp8 else [32, 64, 80, 96, 128, 256]))
    tpp = int(rng.choice([16, 32]))
    hq, hkv = _heads(rng)
    lens = _fit(_lens(rng, int(rng.integers(1, 25)), 6000), hq, hd)
    partition = int(rng.choice([0, 0, 128, 256, 512]))
    outliers = rng.random() < 0.3
    return rng, dtype, fp8, hd, tpp, hq, hkv, lens, partition, outliers


@pytest.mark.parametrize("i", range(64))
def test_decode_sweep(i):
    rng, dtype, fp8, hd, tpp, hq, hkv, lens, partition, outliers = _decode_case(i)
    kw = dict(outlier_frac=0.02, outlier_scale=float(rng.choice([4.0, 8.0, 16.0]))) if outliers else {}
    case = make_paged_case(2000 + i, lens, hq, hkv, hd, tpp, dtype, **kw)
    q = randn_bits(rng, (len(lens), hq, hd), dtype)
    what = (f"decode sweep {i}: {dtype} fp8={fp8} Hq={hq} Hkv={hkv} HD={hd} TPP={tpp} part={partition} "
            f"outliers={outliers} lens={lens}")
    announce(what)
    if fp8:
        kc, vc, ks, vs = fp8_case(case, rng)
        out = pal.paged_attention_decode(dev_bits(q, dtype), dev_codes(kc), dev_codes(vc),
                                         dev_index(case.page_table, torch.uint32), dev_index(case.seq_lens),
                                         partition_size=partition, k_scales=torch.from_numpy(ks).to(DEV),
                                         v_scales=torch.from_numpy(vs).to(DEV))
        ref = orc.paged_attention_decode(q, kc, vc, case.page_table, case.seq_lens, dtype, kv_scales=(ks, vs))
    else:
        out = pal.paged_attention_decode(dev_bits(q, dtype), dev_bits(case.k_pool, dtype),
                                         dev_bits(case.v_pool, dtype), dev_index(case.page_table, torch.uint32),
                                         dev_index(case.seq_lens), partition_size=partition)
        ref = orc.paged_attention_decode(q, case.k_pool, case.v_pool, case.page_table, case.seq_lens, dtype)
    torch.cuda.synchronize()
    assert_close(host_f32(out), ref, dtype, what)


@pytest.mark.parametrize("i", range(32))
def test_prefill_sweep(i):
    rng = np.random.default_rng(3000 + i)
    dtype = "bf16" if rng.random() < 0.6 else "f16"
    hd = int(rng.choice([32, 64, 96, 128, 256]))
    tpp = int(rng.choice([16, 32])) if rng.random() < 0.7 else 8 * int(rng.integers(1, 17))
    hq, hkv = _heads(rng)
    plen = int(rng.choice([1, 2, 15, 16, 17, 63, 64, 65, 130, 200]))
    hist = _fit(_lens(rng, int(rng.integers(1, 6)), 3000), hq, hd)
    while len(hist) * plen * (max(hist) + plen) * hq * hd > 4 * BUDGET and plen > 1:
        plen //= 2
    fp8 = rng.random() < 0.5 and hd in (64, 128, 256) and tpp in (16, 32)
    case, q, k, v = make_prefill_case(4000 + i, hist, plen, hq, hkv, hd, tpp, dtype)
    what = f"prefill sweep {i}: {dtype} fp8={fp8} Hq={hq} Hkv={hkv} HD={hd} TPP={tpp} P={plen} hist={hist}"
    announce(what)
    kp, vp, scales, (ko, vo), kvs = _pools(case, rng, fp8)
    out = pal.paged_attention_prefill(dev_bits(q, dtype), dev_bits(k, dtype), dev_bits(v, dtype), kp, vp,
                                      dev_index(case.page_table, torch.uint32), dev_index(case.seq_lens), **scales)
    torch.cuda.synchronize()
    ref = orc.paged_attention_prefill(q, k, v, ko, vo, case.page_table, case.seq_lens, dtype, kv_scales=kvs)
    assert_close(host_f32(out), ref, dtype, what)


@pytest.mark.parametrize("i", range(32))
def test_fused_sweep(i):
    rng = np.random.default_rng(5000 + i)
    dtype = "bf16" if rng.random() < 0.6 else "f16"
    hd = int(rng.choice([32, 64, 96, 128, 256]))
    tpp = int(rng.choice([16, 32]))
    hq, hkv = _heads(rng)
    dec = _lens(rng, int(rng.integers(0, 30)), 4000)
    chunks = [(int(rng.choice(EDGES[:20])) if rng.random() < 0.5 else int(rng.integers(0, 1500)),
               int(rng.integers(1, 300))) for _ in range(int(rng.integers(0, 4)))]
    if not dec and not chunks:
        dec = [int(rng.integers(1, 2000))]
    dec = _fit(dec, hq, hd) if dec else dec
    block = int(rng.choice([16, 32, 64, 128]))
    fp8 = rng.random() < 0.5 and hd in (64, 128, 256)
    fc = make_fused_case(6000 + i, dec, chunks, hq, hkv, hd, tpp, dtype, block=block)
    c = fc.case
    what = (f"fused sweep {i}: {dtype} fp8={fp8} Hq={hq} Hkv={hkv} HD={hd} TPP={tpp} block={block} decode={dec} "
            f"chunks={chunks}")
    announce(what)
    kp, vp, scales, (ko, vo), kvs = _pools(c, rng, fp8)
    out = pal.paged_attention(dev_bits(fc.queries, dtype), kp, vp, dev_index(c.page_table, torch.uint32),
                              dev_index(c.seq_lens), dev_index(fc.q2seq, torch.uint32), dev_index(fc.q_offset),
                              **scales)
    torch.cuda.synchronize()
    ref = orc.paged_attention(fc.queries, ko, vo, c.page_table, c.seq_lens, fc.q2seq, fc.q_offset, dtype,
                              kv_scales=kvs)
    assert_close(host_f32(out), ref, dtype, what)
