"""GPU parity of paged_attention_decode against the CPU oracle.

Tolerances (written here, the contract of this path): bf16 atol/rtol 2e-2,
fp16 atol/rtol 5e-3, on outputs compared in float32.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import kat_cases
import proxy_attention_lab as pal
from gpu_util import announce, dev_bits, dev_index, host_bits, host_f32
from oracle import pal_oracle as orc
from pal_cases import assert_close, compact_subset, extreme_query_bits, make_paged_case, randn_bits

pytestmark = pytest.mark.gpu
DTYPES = ["f16", "bf16"]


def _decode_gpu(case, q_bits, partition_size=0, stream=None):
    out = pal.paged_attention_decode(
        dev_bits(q_bits, case.dtype), dev_bits(case.k_pool, case.dtype), dev_bits(case.v_pool, case.dtype),
        dev_index(case.page_table, torch.uint32), dev_index(case.seq_lens), stream,
        partition_size=partition_size)
    torch.cuda.synchronize()
    return out


def _check(case, q_bits, partition_size=0, what=""):
    announce(f"decode {what} lens={case.seq_lens.tolist()[:8]} Hq={case.num_q_heads} Hkv={case.num_kv_heads} "
             f"HD={case.head_dim} TPP={case.tokens_per_page} {case.dtype} part={partition_size}")
    out = _decode_gpu(case, q_bits, partition_size)
    assert out.shape == (case.num_seqs, case.num_q_heads, case.head_dim)
    assert out.dtype == {"f16": torch.float16, "bf16": torch.bfloat16}[case.dtype]
    ref = orc.paged_attention_decode(q_bits, case.k_pool, case.v_pool, case.page_table, case.seq_lens, case.dtype)
    assert_close(host_f32(out), ref, case.dtype, what)
    return out


@pytest.mark.parametrize("dtype", DTYPES)
def test_decode_known_answers(dtype):
    for name, inp, expected in kat_cases.decode_cases(dtype):
        announce(f"decode KAT {name} {dtype}")
        out = pal.paged_attention_decode(
            dev_bits(inp["queries"], dtype), dev_bits(inp["k_pool"], dtype), dev_bits(inp["v_pool"], dtype),
            dev_index(inp["page_table"], torch.uint32), dev_index(inp["seq_lens"]))
        torch.cuda.synchronize()
        # the reference tests' own tolerance for these cases
        np.testing.assert_allclose(host_f32(out), expected, atol=1e-2, rtol=1e-2, err_msg=name)


# decode/test_sdpa_equivalency.py:40-59 (contiguous page tables there; permuted here)
REF_CONFIGS = [
    (1, 16, (1, 1), 32), (1, 32, (1, 1), 32), (1, 16, (4, 1), 32), (1, 16, (4, 2), 32),
    (1, 16, (1, 1), 64), (1, 64, (2, 2), 32), (1, 64, (4, 2), 128), (1, 64, (32, 16), 128),
    (2, 32, (4, 4), 32), (2, 64, (32, 16), 128), (3, 128, (32, 16), 128), (16, 64, (4, 4), 32),
    (1, 1024, (32, 16), 128), (1, 4096, (32, 16), 128), (1, 8192, (32, 16), 128),
]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("cfg", REF_CONFIGS, ids=lambda c: f"b{c[0]}_h{c[1]}_q{c[2][0]}kv{c[2][1]}_d{c[3]}")
def test_decode_reference_configs(cfg, dtype):
    b, hist, (hq, hkv), hd = cfg
    case = make_paged_case(100 + hist, [hist] * b, hq, hkv, hd, 16, dtype)
    q = randn_bits(np.random.default_rng(hist), (b, hq, hd), dtype)
    _check(case, q, what=str(cfg))


RAGGED_LENS = [1, 15, 16, 17, 100, 0, 511, 512, 513, 1000, 2049, 37]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("hd", [32, 64, 80, 96, 128, 256])
def test_decode_head_dims_ragged(hd, dtype):
    case = make_paged_case(hd, RAGGED_LENS, 8, 2, hd, 16, dtype)
    q = randn_bits(np.random.default_rng(hd + 1), (len(RAGGED_LENS), 8, hd), dtype)
    _check(case, q, what=f"hd{hd}")


@pytest.mark.parametrize("tpp", [16, 32])
@pytest.mark.parametrize("heads", [(1, 1), (4, 1), (32, 8), (64, 8), (40, 2), (32, 32)])
@pytest.mark.parametrize("partition", [0, 128, 256])
def test_decode_gqa_pages_partitions(tpp, heads, partition):
    hq, hkv = heads
    case = make_paged_case(tpp + hq, RAGGED_LENS, hq, hkv, 128, tpp, "bf16")
    q = randn_bits(np.random.default_rng(hq * 7 + tpp), (len(RAGGED_LENS) + 3, hq, 128), "bf16")  # extra rows ignored
    _check(case, q, partition, what=f"tpp{tpp} heads{heads}")


def test_decode_two_dim_queries():
    case = make_paged_case(3, [40, 7], 1, 1, 64, 16, "f16")
    q = randn_bits(np.random.default_rng(3), (2, 64), "f16")
    announce("decode 2-D queries")
    out = pal.paged_attention_decode(dev_bits(q, "f16"), dev_bits(case.k_pool, "f16"), dev_bits(case.v_pool, "f16"),
                                     dev_index(case.page_table), dev_index(case.seq_lens))
    torch.cuda.synchronize()
    assert out.shape == (2, 1, 64)
    ref = orc.paged_attention_decode(q, case.k_pool, case.v_pool, case.page_table, case.seq_lens, "f16")
    assert_close(host_f32(out), ref, "f16")


@pytest.mark.parametrize("partition", [512, 0])
def test_decode_long_context_outliers(partition):
    """Config-3-like long contexts with 1% of key rows scaled x8: 512-token
    partitions merged by the log-sum-exp pass, and the default equal shares."""
    case = make_paged_case(77, [40000, 70001], 32, 8, 128, 16, "bf16", outlier_frac=0.01)
    q = randn_bits(np.random.default_rng(77), (2, 32, 128), "bf16")
    _check(case, q, partition, what=f"long-context partition {partition}")


@pytest.mark.parametrize("partition", [128, 512])
@pytest.mark.parametrize("hd,dtype,tpp", [(256, "bf16", 16), (256, "f16", 32), (128, "f16", 16), (64, "f16", 32),
                                          (80, "bf16", 16)])
def test_decode_partition_modes(hd, dtype, tpp, partition):
    """The fixed-chunk kernel instances: head_dim 256 (two blocks of
    prefetch), fp16, 32-token pages, head dims that are not multiples of 32."""
    lens = RAGGED_LENS + [5000, 1537]
    case = make_paged_case(hd + tpp + partition, lens, 16, 4, hd, tpp, dtype)
    q = randn_bits(np.random.default_rng(hd * 3 + partition), (len(lens), 16, hd), dtype)
    _check(case, q, partition, what=f"partition {partition} hd{hd}")


@pytest.mark.parametrize("partition", [128, 512])
def test_decode_partition_many_sequences(partition):
    """Fixed-chunk mode with more sequences than the in-kernel planner takes
    (the separate plan kernel of plain decode), zero lengths among them."""
    rng = np.random.default_rng(17 + partition)
    lens = rng.integers(0, 700, size=1300).astype(np.int32)
    lens[rng.choice(1300, 50, replace=False)] = 0
    case = make_paged_case(17, lens, 8, 2, 128, 16, "bf16")
    q = randn_bits(rng, (1300, 8, 128), "bf16")
    _check(case, q, partition, what=f"1300 sequences partition {partition}")


def test_decode_deterministic():
    case = make_paged_case(5, [3000, 100, 777], 32, 8, 128, 16, "bf16")
    q = randn_bits(np.random.default_rng(5), (3, 32, 128), "bf16")
    announce("decode determinism")
    a = host_bits(_decode_gpu(case, q))
    b = host_bits(_decode_gpu(case, q))
    assert np.array_equal(a, b)


def test_decode_explicit_stream_and_empty_batch():
    case = make_paged_case(6, [300, 20], 8, 2, 64, 16, "bf16")
    q = randn_bits(np.random.default_rng(6), (2, 8, 64), "bf16")
    announce("decode explicit stream")
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        pass
    out = _decode_gpu(case, q, stream=s)
    ref = orc.paged_attention_decode(q, case.k_pool, case.v_pool, case.page_table, case.seq_lens, "bf16")
    assert_close(host_f32(out), ref, "bf16")
    empty = pal.paged_attention_decode(dev_bits(q, "bf16"), dev_bits(case.k_pool, "bf16"),
                                       dev_bits(case.v_pool, "bf16"), dev_index(case.page_table[:0]),
                                       dev_index(case.seq_lens[:0]))
    assert empty.shape == (0, 8, 64)


def test_decode_llama3_8b_shape_subset():
    """Config 2 at full size (64 sequences, ctx U[512, 4096], 32/8 heads,
    HD 128, bf16); 8 sequences are re-checked on the CPU oracle, all must be
    finite."""
    rng = np.random.default_rng(2)
    lens = rng.integers(512, 4097, size=64).astype(np.int32)
    case = make_paged_case(2, lens, 32, 8, 128, 16, "bf16", extra_pages=int(0.1 * (lens // 16 + 1).sum()))
    q = randn_bits(rng, (64, 32, 128), "bf16")
    announce("decode config-2 full size")
    out = host_f32(_decode_gpu(case, q))
    assert np.isfinite(out).all()
    pick = np.array([0, 5, 17, 31, 40, 51, 62, 63])
    sub = compact_subset(case, pick)
    ref = orc.paged_attention_decode(q[pick], sub.k_pool, sub.v_pool, sub.page_table, sub.seq_lens, "bf16")
    assert_close(out[pick], ref, "bf16", "config-2 subset")


def test_decode_many_short_sequences():
    """More sequences than the in-kernel planner takes (1024): the plan comes
    from the separate plan kernel; lengths include zeros."""
    rng = np.random.default_rng(15)
    lens = rng.integers(0, 60, size=1500).astype(np.int32)
    case = make_paged_case(15, lens, 8, 2, 64, 16, "bf16", garbage_tail=False)
    q = randn_bits(rng, (1500, 8, 64), "bf16")
    _check(case, q, what="1500 sequences")


def test_decode_many_pieces_per_worker():
    """900 short sequences (the in-kernel planner's item table), zeros among
    them: every wavefront streams many segment pieces back to back, so the
    next piece's blocks load while the current piece finishes."""
    rng = np.random.default_rng(16)
    lens = rng.integers(0, 200, size=900).astype(np.int32)
    lens[rng.choice(900, 60, replace=False)] = 0
    case = make_paged_case(16, lens, 32, 8, 128, 16, "bf16", garbage_tail=True)
    q = randn_bits(rng, (900, 32, 128), "bf16")
    _check(case, q, what="900 sequences")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("partition", [0, 512])
def test_decode_query_magnitudes(dtype, partition):
    """Query heads across the dtype's range (zeros, tiny, huge, mixed,
    near the range ends): the softmax takes exp2(score - max) in log2 units,
    so even scores past 2^31 stay finite and match the oracle."""
    lens = [1, 17, 300, 1000, 2049]
    case = make_paged_case(72 + partition, lens, 16, 4, 128, 16, dtype)
    q = extreme_query_bits(np.random.default_rng(72), (len(lens), 16, 128), dtype)
    out = _check(case, q, partition, f"query magnitudes p{partition}")
    assert np.isfinite(host_f32(out)).all()
