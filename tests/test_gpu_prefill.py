"""GPU parity of paged_attention_prefill (the reference's uniform-prompt
signature) against the CPU oracle and the reference's own SDPA construction.

Tolerances (the contract of this path): bf16 atol/rtol 2e-2, fp16 atol/rtol
5e-3, outputs compared in float32.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import kat_cases
import proxy_attention_lab as pal
from gpu_util import announce, dev_bits, dev_index, host_bits, host_f32
from oracle import pal_oracle as orc
from pal_cases import assert_close, extreme_query_bits, make_prefill_case, sdpa_prefill_case

pytestmark = pytest.mark.gpu
DTYPES = ["f16", "bf16"]


def _prefill_gpu(q, k, v, k_pool, v_pool, pt, lens, dtype, stream=None):
    out = pal.paged_attention_prefill(dev_bits(q, dtype), dev_bits(k, dtype), dev_bits(v, dtype),
                                      dev_bits(k_pool, dtype), dev_bits(v_pool, dtype),
                                      dev_index(pt, torch.uint32), dev_index(lens), stream)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("dtype", DTYPES)
def test_prefill_known_answers(dtype):
    for name, inp, expected in kat_cases.prefill_cases(dtype):
        announce(f"prefill KAT {name} {dtype}")
        out = _prefill_gpu(inp["q_prompt"], inp["k_prompt"], inp["v_prompt"], inp["k_pool"], inp["v_pool"],
                           inp["page_table"], inp["context_lens"], dtype)
        # the reference tests' own tolerance for these cases
        np.testing.assert_allclose(host_f32(out), expected, atol=1e-2, rtol=1e-2, err_msg=name)


# prefill/test_sdpa_equivalency.py:18-27, with causal SDPA over history + prompt as the expected value
REF_CONFIGS = [(1, 0, 16, (4, 4), 64), (1, 128, 16, (4, 4), 64), (2, 64, 32, (8, 2), 128),
               (1, 256, 1, (32, 8), 128), (1, 0, 128, (32, 8), 128)]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("cfg", REF_CONFIGS, ids=lambda c: f"b{c[0]}_h{c[1]}_p{c[2]}_q{c[3][0]}kv{c[3][1]}_d{c[4]}")
def test_prefill_reference_configs(cfg, dtype):
    b, hist, plen, (hq, hkv), hd = cfg
    qp, kp, vp, k_pool, v_pool, pt, lens, ref = sdpa_prefill_case(21, b, hist, plen, hq, hkv, hd, dtype)
    announce(f"prefill ref config {cfg} {dtype}")
    out = host_f32(_prefill_gpu(qp, kp, vp, k_pool, v_pool, pt, lens, dtype))
    assert out.shape == (b * plen * hq, hd)
    assert_close(out, ref, dtype, str(cfg))


def _check(seed, hist, plen, hq, hkv, hd, tpp, dtype, what=""):
    case, q, k, v = make_prefill_case(seed, hist, plen, hq, hkv, hd, tpp, dtype)
    announce(f"prefill {what} hist={list(hist)[:8]} P={plen} Hq={hq} Hkv={hkv} HD={hd} TPP={tpp} {dtype}")
    out = host_f32(_prefill_gpu(q, k, v, case.k_pool, case.v_pool, case.page_table, case.seq_lens, dtype))
    ref = orc.paged_attention_prefill(q, k, v, case.k_pool, case.v_pool, case.page_table, case.seq_lens, dtype)
    assert_close(out, ref, dtype, what)


RAGGED_HIST = [0, 1, 15, 16, 17, 100, 257]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("plen", [1, 7, 33, 130])
def test_prefill_ragged_history(plen, dtype):
    _check(plen, RAGGED_HIST, plen, 32, 8, 128, 16, dtype, "ragged")


@pytest.mark.parametrize("hd", [32, 64, 96, 128, 256])
@pytest.mark.parametrize("tpp", [16, 32])
def test_prefill_head_dims_pages(hd, tpp):
    _check(hd + tpp, [5, 40, 0], 45, 8, 2, hd, tpp, "bf16", f"hd{hd}")


@pytest.mark.parametrize("heads", [(1, 1), (4, 4), (16, 1), (40, 2), (64, 8), (32, 32)])
def test_prefill_gqa_groups(heads):
    hq, hkv = heads
    _check(hq * 3 + hkv, [20, 3], 70, hq, hkv, 64, 16, "f16", f"heads{heads}")


def test_prefill_rows_not_multiple_of_sequences():
    """N = 11 rows over 2 sequences: P = 5, the last row is not covered and is zero."""
    case, q, k, v = make_prefill_case(9, [10, 4], 5, 4, 2, 64, 16, "bf16")
    q = np.concatenate([q, q[:1]])
    k = np.concatenate([k, k[:1]])
    v = np.concatenate([v, v[:1]])
    announce("prefill N % S != 0")
    out = host_f32(_prefill_gpu(q, k, v, case.k_pool, case.v_pool, case.page_table, case.seq_lens, "bf16"))
    assert out.shape == (11 * 4, 64)
    ref = orc.paged_attention_prefill(q[:10], k[:10], v[:10], case.k_pool, case.v_pool, case.page_table,
                                      case.seq_lens, "bf16")
    assert_close(out[:40], ref, "bf16")
    assert np.all(out[40:] == 0)


def test_prefill_two_dim_queries_and_stream():
    case, q, k, v = make_prefill_case(12, [33], 9, 1, 1, 64, 16, "f16")
    announce("prefill 2-D queries on a side stream")
    s = torch.cuda.Stream()
    out = host_f32(_prefill_gpu(q[:, 0, :], k, v, case.k_pool, case.v_pool, case.page_table, case.seq_lens,
                                "f16", stream=s))
    ref = orc.paged_attention_prefill(q, k, v, case.k_pool, case.v_pool, case.page_table, case.seq_lens, "f16")
    assert out.shape == (9, 64)
    assert_close(out, ref, "f16")


def test_prefill_deterministic():
    case, q, k, v = make_prefill_case(13, [300, 64], 200, 32, 8, 128, 16, "bf16")
    announce("prefill determinism")
    a = host_bits(_prefill_gpu(q, k, v, case.k_pool, case.v_pool, case.page_table, case.seq_lens, "bf16"))
    b = host_bits(_prefill_gpu(q, k, v, case.k_pool, case.v_pool, case.page_table, case.seq_lens, "bf16"))
    assert np.array_equal(a, b)


@pytest.mark.parametrize("tpp,hist", [(16, [26000, 9000]), (32, [40000, 300])])
def test_prefill_long_history_page_id_chunks(tpp, hist):
    """Histories longer than 8192 keys: the page ids of a tile are staged into
    LDS in chunks of 512 entries, two live at a time; these cases need three
    or four chunks, so the kernel stages later chunks over earlier ones while
    the key loop runs."""
    _check(31 + tpp, hist, 48, 32, 8, 128, tpp, "bf16", f"long history tpp{tpp}")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("hd", [32, 64, 96, 128, 256])
def test_prefill_dense_prompt_steps(hd, dtype):
    """Prompts long enough that most 32-key steps lie wholly in the prompt:
    those steps copy K/V straight from the prompt rows (V untransposed, read
    back with transposing LDS reads), after paged steps of histories that end
    on and off a step boundary."""
    _check(70 + hd, [0, 64, 96, 31, 33], 160, 16, 4, hd, 16, dtype, f"dense prompt steps hd{hd}")


# The reference prefill reads the page size at run time
# (paged_attention_prefill.h.metal:243-263); 16 and 32 have their own kernels,
# other multiples of 8 (including the 56 of the reference's C++ benchmark,
# seq_len_vs_latency.cpp:47-55) run the run-time page-size kernel.
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("tpp", [8, 24, 56, 64, 128])
def test_prefill_runtime_page_sizes(tpp, dtype):
    _check(tpp, [0, 1, 7, 8, 9, tpp - 1, tpp, tpp + 1, 300, 1000], 37, 16, 4, 128, tpp, dtype, f"tpp{tpp}")


@pytest.mark.parametrize("hd", [32, 64, 96, 256])
def test_prefill_runtime_page_size_head_dims(hd):
    _check(hd + 1, [5, 40, 0, 129], 45, 8, 2, hd, 8, "bf16", f"tpp8 hd{hd}")
    _check(hd + 2, [5, 40, 0, 129], 45, 8, 2, hd, 64, "f16", f"tpp64 hd{hd}")


@pytest.mark.parametrize("dtype", DTYPES)
def test_prefill_query_magnitudes(dtype):
    """Query heads across the dtype's range (zeros, tiny, large, mixed, near
    the range ends) through the tile path, the large heads held to the
    tiles' exact range (extreme_query_bits with tiles=True)."""
    case, q, k, v = make_prefill_case(73, [0, 40, 300], 70, 16, 4, 128, 16, dtype)
    q = extreme_query_bits(np.random.default_rng(73), q.shape, dtype, tiles=True)
    announce(f"prefill query magnitudes {dtype}")
    out = host_f32(_prefill_gpu(q, k, v, case.k_pool, case.v_pool, case.page_table, case.seq_lens, dtype))
    assert np.isfinite(out).all()
    ref = orc.paged_attention_prefill(q, k, v, case.k_pool, case.v_pool, case.page_table, case.seq_lens, dtype)
    assert_close(out, ref, dtype, f"prefill query magnitudes {dtype}")
