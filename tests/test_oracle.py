"""Pins the CPU oracle (oracle/pal_oracle.py) before it is trusted as the checker.

Each oracle function is checked against something independent of its own
formula: the reference tests' known answers, torch's
scaled_dot_product_attention in float32 on contiguous K/V, a scalar
brute-force loop on tiny shapes, and invariants (page-table permutation,
two-pass == single pass, fused == decode / prefill on the rows they share).
A planted mistake (wrong GQA map, dropped scale, off-by-one mask, swapped
stripe index) fails at least one of them -- see test_planted_mistakes_are_caught.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import kat_cases
from oracle import pal_oracle as orc
from pal_cases import assert_close, make_paged_case, sdpa_prefill_case

DTYPES = ["f16", "bf16"]


# ---------------------------------------------------------------------------
# fill
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("dtype", DTYPES)
def test_fill_known_answers(dtype):
    for name, kw, ek, ev in kat_cases.fill_cases(dtype):
        k0, v0 = kw["k_pool"].copy(), kw["v_pool"].copy()
        k, v = orc.fill_kv_pages(**kw)
        assert np.array_equal(k, ek), name
        assert np.array_equal(v, ev), name
        # functional semantics: inputs untouched (fill_kv_pages_primitive.cpp:91-92)
        assert np.array_equal(kw["k_pool"], k0) and np.array_equal(kw["v_pool"], v0), name


def test_fill_full_page_plus_one_layout():
    """test_fill_multiple_tokens_single_sequence.py:302-322: page 1 fully
    written, page 2 only slot 0, other slots of page 2 untouched."""
    name, kw, _, _ = [c for c in kat_cases.fill_cases("bf16") if c[0] == "full_page_plus_one"][0]
    k, v = orc.fill_kv_pages(**kw)
    for slot in range(16):
        assert (k[1, :, :, slot, :] != 0).any() and (v[1, :, :, slot] != 0).any()
    assert (k[2, :, :, 0, :] != 0).any() and (v[2, :, :, 0] != 0).any()
    assert (k[2, :, :, 1:, :] == 0).all() and (v[2, :, :, 1:] == 0).all()


def test_fill_random_matches_scalar_loop():
    rng = np.random.default_rng(3)
    n, hkv, hd, tpp, pages, seqs, w = 40, 3, 32, 4, 30, 5, 6
    new_k = rng.integers(0, 65535, size=(n, hkv, hd), dtype=np.uint16)
    new_v = rng.integers(0, 65535, size=(n, hkv, hd), dtype=np.uint16)
    pt = rng.permutation(pages)[: seqs * w].reshape(seqs, w).astype(np.uint32)
    # distinct destinations: (seq, pos) pairs without repetition
    pairs = rng.permutation(seqs * w * tpp)[:n]
    q2s = (pairs // (w * tpp)).astype(np.uint32)
    pos = (pairs % (w * tpp)).astype(np.int32)
    k0 = rng.integers(0, 65535, size=(pages, hkv, hd // 8, tpp, 8), dtype=np.uint16)
    v0 = rng.integers(0, 65535, size=(pages, hkv, hd, tpp), dtype=np.uint16)
    k, v = orc.fill_kv_pages(new_k, new_v, k0, v0, pt, pos, q2s)
    ek, ev = k0.copy(), v0.copy()
    for t in range(n):
        page = pt[q2s[t], pos[t] // tpp]
        slot = pos[t] % tpp
        for h in range(hkv):
            for d in range(hd):
                ek[page, h, d // 8, slot, d % 8] = new_k[t, h, d]
                ev[page, h, d, slot] = new_v[t, h, d]
    assert np.array_equal(k, ek) and np.array_equal(v, ev)


def test_bf16_rounding_matches_torch():
    x = np.random.default_rng(0).standard_normal(10000).astype(np.float32) * 100
    x[:4] = [0.0, -0.0, np.inf, -np.inf]
    ours = orc.f32_to_bits(x, "bf16")
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, ref)
    assert np.array_equal(orc.bits_to_f32(ours, "bf16"), torch.from_numpy(x).to(torch.bfloat16).float().numpy())


# ---------------------------------------------------------------------------
# decode
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("dtype", DTYPES)
def test_decode_known_answers(dtype):
    for name, inp, expected in kat_cases.decode_cases(dtype):
        out = orc.paged_attention_decode(inp["queries"], inp["k_pool"], inp["v_pool"],
                                         inp["page_table"], inp["seq_lens"], dtype)
        np.testing.assert_allclose(out, expected, atol=1e-2, rtol=1e-3, err_msg=name)


def _sdpa_decode(case, q_bits):
    """torch SDPA (float32) per sequence on contiguous K/V re-gathered with
    the reference tests' page arithmetic."""
    dt = case.dtype
    q = torch.from_numpy(orc.bits_to_f32(q_bits, dt))
    kf = orc.bits_to_f32(case.k_pool, dt)
    vf = orc.bits_to_f32(case.v_pool, dt)
    out = torch.zeros(case.num_seqs, case.num_q_heads, case.head_dim)
    g = case.num_q_heads // case.num_kv_heads
    tpp = case.tokens_per_page
    for s in range(case.num_seqs):
        n = int(case.seq_lens[s])
        if n == 0:
            continue
        ks, vs = [], []
        for t in range(n):  # scalar per-token gather, independent of the oracle's fancy indexing
            page, slot = int(case.page_table[s, t // tpp]), t % tpp
            ks.append(kf[page, :, :, slot, :].reshape(case.num_kv_heads, case.head_dim))
            vs.append(vf[page, :, :, slot])
        k = torch.from_numpy(np.stack(ks, 1)).repeat_interleave(g, 0)  # [Hq, n, HD]
        v = torch.from_numpy(np.stack(vs, 1)).repeat_interleave(g, 0)
        o = torch.nn.functional.scaled_dot_product_attention(q[s][:, None, :], k, v)
        out[s] = o[:, 0, :]
    return out.numpy()


# The reference's SDPA-equivalency configurations (decode/test_sdpa_equivalency.py:40-59)
# plus ragged and GQA-heavy ones.
DECODE_CONFIGS = [
    (1, 16, (1, 1), 32), (1, 32, (1, 1), 32), (1, 16, (4, 1), 32), (1, 16, (4, 2), 32),
    (1, 16, (1, 1), 64), (1, 64, (2, 2), 32), (1, 64, (4, 2), 128), (1, 64, (32, 16), 128),
    (2, 32, (4, 4), 32), (2, 64, (32, 16), 128), (3, 128, (32, 16), 128), (16, 64, (4, 4), 32),
    (1, 1024, (32, 16), 128),
]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("cfg", DECODE_CONFIGS[::2] + [DECODE_CONFIGS[-1]])
def test_decode_matches_torch_sdpa(cfg, dtype):
    b, hist, (hq, hkv), hd = cfg
    case = make_paged_case(11, [hist] * b, hq, hkv, hd, 16, dtype)
    q = orc.f32_to_bits(np.random.default_rng(5).standard_normal((b, hq, hd)).astype(np.float32), dtype)
    ours = orc.paged_attention_decode(q, case.k_pool, case.v_pool, case.page_table, case.seq_lens, dtype)
    ref = _sdpa_decode(case, q)
    np.testing.assert_allclose(ours, ref, atol=2e-5, rtol=2e-5)


def test_decode_ragged_gqa_matches_torch_sdpa():
    case = make_paged_case(12, [1, 15, 16, 17, 100, 0, 33], 8, 2, 64, 16, "bf16")
    q = orc.f32_to_bits(np.random.default_rng(6).standard_normal((7, 8, 64)).astype(np.float32), "bf16")
    ours = orc.paged_attention_decode(q, case.k_pool, case.v_pool, case.page_table, case.seq_lens, "bf16")
    np.testing.assert_allclose(ours, _sdpa_decode(case, q), atol=2e-5, rtol=2e-5)
    assert np.all(ours[5] == 0)  # empty sequence -> zeros


def test_decode_brute_force_tiny():
    """Pure-Python scalar loops on a tiny case: softmax(q.k / sqrt(d)) v."""
    case = make_paged_case(13, [5, 3], 2, 1, 8 * 2, 4, "f16")
    q = orc.f32_to_bits(np.random.default_rng(1).standard_normal((2, 2, 16)).astype(np.float32), "f16")
    qf = orc.bits_to_f32(q, "f16")
    kf = orc.bits_to_f32(case.k_pool, "f16")
    vf = orc.bits_to_f32(case.v_pool, "f16")
    ours = orc.paged_attention_decode(q, case.k_pool, case.v_pool, case.page_table, case.seq_lens, "f16")
    import math

    for s in range(2):
        for h in range(2):
            n = int(case.seq_lens[s])
            scores = []
            for t in range(n):
                page, slot = int(case.page_table[s, t // 4]), t % 4
                dot = 0.0
                for d in range(16):
                    dot += float(qf[s, h, d]) * float(kf[page, 0, d // 8, slot, d % 8])
                scores.append(dot / math.sqrt(16))
            mx = max(scores)
            w = [math.exp(x - mx) for x in scores]
            tot = sum(w)
            for d in range(16):
                acc = 0.0
                for t in range(n):
                    page, slot = int(case.page_table[s, t // 4]), t % 4
                    acc += w[t] * float(vf[page, 0, d, slot])
                assert abs(acc / tot - ours[s, h, d]) < 1e-5


def test_decode_invariant_under_page_permutation():
    case = make_paged_case(14, [70, 33], 4, 2, 32, 16, "bf16", extra_pages=5)
    q = orc.f32_to_bits(np.random.default_rng(2).standard_normal((2, 4, 32)).astype(np.float32), "bf16")
    base = orc.paged_attention_decode(q, case.k_pool, case.v_pool, case.page_table, case.seq_lens, "bf16")
    perm = np.random.default_rng(9).permutation(case.k_pool.shape[0])
    inv = np.argsort(perm)
    k2 = case.k_pool[perm]
    v2 = case.v_pool[perm]
    pt2 = inv[case.page_table].astype(np.uint32)
    moved = orc.paged_attention_decode(q, k2, v2, pt2, case.seq_lens, "bf16")
    np.testing.assert_allclose(moved, base, atol=1e-6, rtol=1e-6)


@pytest.mark.parametrize("chunk", [16, 128, 512])
def test_two_pass_equals_single_pass(chunk):
    case = make_paged_case(15, [1000, 513, 40], 8, 2, 64, 16, "bf16", outlier_frac=0.01)
    q = orc.f32_to_bits(np.random.default_rng(3).standard_normal((3, 8, 64)).astype(np.float32), "bf16")
    one = orc.paged_attention_decode(q, case.k_pool, case.v_pool, case.page_table, case.seq_lens, "bf16")
    two = orc.paged_attention_decode_two_pass(q, case.k_pool, case.v_pool, case.page_table, case.seq_lens,
                                              "bf16", chunk_size=chunk)
    np.testing.assert_allclose(two, one, atol=1e-5, rtol=1e-5)


# ---------------------------------------------------------------------------
# prefill and fused
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("dtype", DTYPES)
def test_prefill_known_answers(dtype):
    for name, inp, expected in kat_cases.prefill_cases(dtype):
        out = orc.paged_attention_prefill(inp["q_prompt"], inp["k_prompt"], inp["v_prompt"], inp["k_pool"],
                                          inp["v_pool"], inp["page_table"], inp["context_lens"], dtype)
        np.testing.assert_allclose(out, expected, atol=1e-2, rtol=1e-3, err_msg=name)


# prefill/test_sdpa_equivalency.py:18-27
PREFILL_CONFIGS = [(1, 0, 16, (4, 4), 64), (1, 128, 16, (4, 4), 64), (2, 64, 32, (8, 2), 128),
                   (1, 256, 1, (32, 8), 128), (1, 0, 128, (32, 8), 128)]


@pytest.mark.parametrize("cfg", PREFILL_CONFIGS)
def test_prefill_matches_torch_sdpa(cfg):
    b, hist, plen, (hq, hkv), hd = cfg
    qp, kp, vp, k_pool, v_pool, pt, lens, ref = sdpa_prefill_case(21, b, hist, plen, hq, hkv, hd, "bf16")
    ours = orc.paged_attention_prefill(qp, kp, vp, k_pool, v_pool, pt, lens, "bf16")
    np.testing.assert_allclose(ours, ref, atol=3e-5, rtol=3e-5)


def test_fused_matches_decode_and_prefill():
    """Fused rows reproduce decode rows and (prompt written to pages) prefill rows."""
    dtype = "bf16"
    hq, hkv, hd, tpp = 8, 2, 64, 16
    # decode part
    case = make_paged_case(31, [40, 77, 5], hq, hkv, hd, tpp, dtype)
    q = orc.f32_to_bits(np.random.default_rng(4).standard_normal((3, hq, hd)).astype(np.float32), dtype)
    dec = orc.paged_attention_decode(q, case.k_pool, case.v_pool, case.page_table, case.seq_lens, dtype)
    fused = orc.paged_attention(q, case.k_pool, case.v_pool, case.page_table, case.seq_lens,
                                np.arange(3, dtype=np.uint32), case.seq_lens.copy(), dtype)
    np.testing.assert_allclose(fused, dec, atol=1e-6)
    # prefill part: history 30, prompt 20 -> write the prompt into pages, run fused.
    hist, plen = 30, 20
    qp, kp, vp, k_pool, v_pool, pt, lens, ref = sdpa_prefill_case(22, 1, hist, plen, hq, hkv, hd, dtype)
    pre = orc.paged_attention_prefill(qp, kp, vp, k_pool, v_pool, pt, lens, dtype)
    npg = (hist + plen + tpp - 1) // tpp
    extra = npg - pt.shape[1]
    base = k_pool.shape[0]
    k_big = np.concatenate([k_pool, np.zeros((extra,) + k_pool.shape[1:], np.uint16)])
    v_big = np.concatenate([v_pool, np.zeros((extra,) + v_pool.shape[1:], np.uint16)])
    pt_big = np.concatenate([pt, (base + np.arange(extra, dtype=np.uint32))[None]], axis=1)
    k_big, v_big = orc.fill_kv_pages(kp, vp, k_big, v_big, pt_big, hist + np.arange(plen, dtype=np.int32),
                                     np.zeros(plen, np.uint32))
    fused = orc.paged_attention(qp, k_big, v_big, pt_big, np.array([hist + plen], np.int32),
                                np.zeros(plen, np.uint32), hist + 1 + np.arange(plen, dtype=np.int32), dtype)
    np.testing.assert_allclose(fused.reshape(-1, hd), pre, atol=1e-6)
    np.testing.assert_allclose(pre, ref, atol=3e-5, rtol=3e-5)


def test_torch_cpu_restatement_matches_oracle():
    """The CPU baseline's comparator (gather + torch SDPA on the CPU) equals
    the numpy oracle: config 1 decode, a ragged GQA decode with NaN bits in
    unused slots, and a fused batch of decode rows, prefill runs, an empty
    row and a row naming no sequence."""
    for dtype in DTYPES:
        case = make_paged_case(0, [64, 100, 192, 256], 4, 1, 64, 16, dtype, extra_pages=25)
        q = orc.f32_to_bits(np.random.default_rng(0).standard_normal((4, 4, 64)).astype(np.float32), dtype)
        want = orc.paged_attention_decode(q, case.k_pool, case.v_pool, case.page_table, case.seq_lens, dtype)
        got = orc.torch_cpu_paged_attention(q, case.k_pool, case.v_pool, case.page_table, case.seq_lens, dtype)
        np.testing.assert_allclose(got, want, atol=2e-6, rtol=2e-6)
    case = make_paged_case(5, [3, 700, 129, 1], 16, 4, 128, 32, "bf16")
    q = orc.f32_to_bits(np.random.default_rng(5).standard_normal((4, 16, 128)).astype(np.float32), "bf16")
    want = orc.paged_attention_decode(q, case.k_pool, case.v_pool, case.page_table, case.seq_lens, "bf16")
    got = orc.torch_cpu_paged_attention(q, case.k_pool, case.v_pool, case.page_table, case.seq_lens, "bf16")
    np.testing.assert_allclose(got, want, atol=2e-6, rtol=2e-6)
    q2s = np.array([1, 1, 1, 0, 2, 2, 3, 9, 1], np.uint32)
    off = np.array([5, 6, 7, 3, 100, 129, 0, 4, 700], np.int32)
    qf = orc.f32_to_bits(np.random.default_rng(6).standard_normal((9, 16, 128)).astype(np.float32), "bf16")
    want = orc.paged_attention(qf, case.k_pool, case.v_pool, case.page_table, case.seq_lens, q2s, off, "bf16")
    got = orc.torch_cpu_paged_attention(qf, case.k_pool, case.v_pool, case.page_table, case.seq_lens, "bf16",
                                        q2s, off)
    np.testing.assert_allclose(got, want, atol=2e-6, rtol=2e-6)
    assert not got[6].any() and not got[7].any()


# ---------------------------------------------------------------------------
# the checks above must catch plausible mistakes
# ---------------------------------------------------------------------------


def test_planted_mistakes_are_caught(monkeypatch):
    """Swap in broken variants of the oracle's pieces; a check must fail."""
    dtype = "bf16"
    case = make_paged_case(41, [37, 20], 8, 2, 32, 16, dtype)
    q = orc.f32_to_bits(np.random.default_rng(8).standard_normal((2, 8, 32)).astype(np.float32), dtype)
    ref = _sdpa_decode(case, q)
    good_attend = orc.attend
    good_gather = orc.gather_tokens

    def wrong_gqa(q_, k, v, limits, causal_pos=None):  # kv head h % Hkv instead of h // G
        hq, hkv = q_.shape[1], k.shape[1]
        idx = np.arange(hq) % hkv
        order = np.argsort(idx, kind="stable")
        return good_attend(q_[:, order], k, v, limits)[:, np.argsort(order)]

    def no_scale(q_, k, v, limits, causal_pos=None):
        return good_attend(q_ * np.sqrt(np.float32(q_.shape[-1])), k, v, limits)

    def off_by_one(q_, k, v, limits, causal_pos=None):
        return good_attend(q_, k, v, np.asarray(limits) - 1)

    def swapped_stripe(kp, vp, row, n):
        k, v = good_gather(kp, vp, row, n)
        hd = k.shape[-1]
        return k.reshape(n, k.shape[1], hd // 8, 8).transpose(0, 1, 3, 2).reshape(k.shape), v

    for name, fn, target in (("gqa", wrong_gqa, "attend"), ("scale", no_scale, "attend"),
                             ("mask", off_by_one, "attend"), ("stripe", swapped_stripe, "gather_tokens")):
        monkeypatch.setattr(orc, target, fn)
        bad = orc.paged_attention_decode(q, case.k_pool, case.v_pool, case.page_table, case.seq_lens, dtype)
        monkeypatch.setattr(orc, "attend", good_attend)
        monkeypatch.setattr(orc, "gather_tokens", good_gather)
        assert not np.allclose(bad, ref, atol=2e-5, rtol=2e-5), f"planted mistake '{name}' not caught"


def test_assert_close_helper_rejects_large_error():
    a = np.zeros(10, np.float32)
    with pytest.raises(AssertionError):
        assert_close(a + 0.1, a, "bf16")
    assert_close(a + 0.001, a, "f16")
