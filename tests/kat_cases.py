"""Known-answer cases restated from the reference's own tests.

Each builder returns numpy inputs (16-bit patterns for fp16/bf16 data) and
the expected result computed the way the reference test computes it (closed
form or the test's own scalar loops), so the CPU oracle and the GPU kernels
are checked against the same answers.  Reference test files are cited per
case; the reference tests compare with atol 1e-2 (attention) and 1e-3
(fill), the fill checks here are bit-exact.
"""

from __future__ import annotations

import numpy as np

from oracle import pal_oracle as orc

X = 8  # K stripe width for 2-byte dtypes


def _bits(vals, dtype):
    return orc.f32_to_bits(np.asarray(vals, np.float32), dtype)


def _f32(bits, dtype):
    return orc.bits_to_f32(bits, dtype)


def _put_k(k_pool, page, head, slot, vec):
    """Reference tests' scalar K write loop (e.g. decode/test_full_attention.py:84-88)."""
    for d in range(vec.shape[0]):
        k_pool[page, head, d // X, slot, d % X] = vec[d]


# ---------------------------------------------------------------------------
# fill_kv_pages
# ---------------------------------------------------------------------------


def _fill_expected(new_k, new_v, k_shape, v_shape, page_table, positions, q2seq, tpp):
    """Expected pools built with the reference tests' loops
    (fill_kv_pages/test_fill_multiple_tokens_single_sequence.py:97-106)."""
    ek = np.zeros(k_shape, np.uint16)
    ev = np.zeros(v_shape, np.uint16)
    n, hkv, hd = new_k.shape
    for t in range(n):
        page = int(page_table[int(q2seq[t]), int(positions[t]) // tpp])
        slot = int(positions[t]) % tpp
        for h in range(hkv):
            for d in range(hd):
                ev[page, h, d, slot] = new_v[t, h, d]
                ek[page, h, d // X, slot, d % X] = new_k[t, h, d]
    return ek, ev


def fill_cases(dtype):
    """All fill known-answer cases: list of (name, kwargs, expected_k, expected_v)."""
    cases = []

    def add(name, n, hkv, hd, tpp, pages, page_table, positions, q2seq, kvals, vvals):
        new_k = _bits(kvals, dtype).reshape(n, hkv, hd)
        new_v = _bits(vvals, dtype).reshape(n, hkv, hd)
        k_shape = (pages, hkv, hd // X, tpp, X)
        v_shape = (pages, hkv, hd, tpp)
        pt = np.asarray(page_table, np.uint32)
        pos = np.asarray(positions, np.int32)
        q2s = np.asarray(q2seq, np.uint32)
        ek, ev = _fill_expected(new_k, new_v, k_shape, v_shape, pt, pos, q2s, tpp)
        kw = dict(new_k=new_k, new_v=new_v, k_pool=np.zeros(k_shape, np.uint16),
                  v_pool=np.zeros(v_shape, np.uint16), page_table=pt, write_pos=pos, q2seq=q2s)
        cases.append((name, kw, ek, ev))

    # fill_kv_pages/test_fill_kv_pages_data.py:33-118 -- one token, TPP 2, HD 64.
    hd = 64
    add("single_token", 1, 1, hd, 2, 1, [[0]], [0], [0],
        np.arange(1, hd + 1), np.arange(hd + 1, 2 * hd + 1))

    # test_fill_single_token_multiple_sequences.py:32-125 -- seqs on pages 1 and 3.
    n, hkv, hd = 2, 2, 32
    kv = [[[(s * 100) + (h * 10) + d for d in range(hd)] for h in range(hkv)] for s in range(n)]
    add("multi_seq_distinct_pages", n, hkv, hd, 4, 4, [[1], [3]], [0, 1], [0, 1],
        kv, np.asarray(kv) + 1000)

    # :128-207 -- two sequences sharing page 2, slots 1 and 3.
    rng = np.random.default_rng(7)
    kr = rng.standard_normal((n, hkv, hd)).astype(np.float32)
    vr = rng.standard_normal((n, hkv, hd)).astype(np.float32)
    add("multi_seq_same_page", n, hkv, hd, 4, 4, [[2], [2]], [1, 3], [0, 1], kr, vr)

    # test_fill_multiple_tokens_single_sequence.py:33-116 -- 3 tokens in page 1.
    n, hkv, hd = 3, 2, 32
    kv = [[[(t * 1000) + (h * 100) + d for d in range(hd)] for h in range(hkv)] for t in range(n)]
    add("tokens_within_page", n, hkv, hd, 4, 2, [[1]], np.arange(n), np.zeros(n),
        kv, np.asarray(kv) + 5000)

    # :119-206 -- page boundary with page table [5, 10], start position 1, TPP 2.
    add("tokens_across_pages", n, hkv, hd, 2, 12, [[5, 10]], np.arange(1, 1 + n), np.zeros(n),
        kv, np.asarray(kv) + 5000)

    # :209-324 -- 17 tokens, TPP 16, Hkv 8, HD 128 (values beyond the fp16
    # range become inf and must be copied as such).
    n, hkv, hd = 17, 8, 128
    kv = [[[(t * 10000) + (h * 1000) + d for d in range(hd)] for h in range(hkv)] for t in range(n)]
    add("full_page_plus_one", n, hkv, hd, 16, 3, [[1, 2]], np.arange(n), np.zeros(n),
        kv, np.asarray(kv) + 50000)
    return cases


# ---------------------------------------------------------------------------
# decode
# ---------------------------------------------------------------------------


def decode_cases(dtype):
    """Decode known-answer cases: list of (name, inputs, expected_f32 [S, Hq, HD])."""
    cases = []
    tpp = 16

    # decode/test_core_functionality.py:36-183 -- one history token per
    # sequence, so the output is exactly that token's V.  Unused page-table
    # entries 99 / 88 lie outside the 2-page pool and must never be read.
    for hd in (32, 64, 128, 256):
        q = np.zeros((2, 1, hd), np.float32)
        q[0, 0, 0], q[1, 0, 0] = 100.0, 200.0
        k = np.zeros((2, 1, hd // X, tpp, X), np.uint16)
        for page, val in ((0, 11.0), (1, 22.0)):
            vec = np.zeros(hd, np.float32)
            vec[0] = val
            _put_k(k, page, 0, 0, _bits(vec, dtype))
        v = np.zeros((2, 1, hd, tpp), np.uint16)
        v[0, 0, :, 0] = _bits(np.arange(hd) * 10.0 + 10.0, dtype)
        v[1, 0, :, 0] = _bits(np.arange(hd) * 100.0 + 100.0, dtype)
        inputs = dict(queries=_bits(q, dtype), k_pool=k, v_pool=v,
                      page_table=np.array([[0, 99], [1, 88]], np.uint32),
                      seq_lens=np.array([1, 1], np.int32))
        expected = np.stack([_f32(v[0, 0, :, 0], dtype), _f32(v[1, 0, :, 0], dtype)])[:, None, :]
        cases.append((f"one_token_per_seq_hd{hd}", inputs, expected))

    # decode/test_softmax_and_value.py:36-131 -- single token, output = V.
    for hd in (32, 64, 128, 256):
        q = np.ones((1, 1, hd), np.float32)
        k = np.zeros((1, 1, hd // X, tpp, X), np.uint16)
        vec = np.zeros(hd, np.float32)
        vec[:4] = 1.0
        _put_k(k, 0, 0, 0, _bits(vec, dtype))
        v = np.zeros((1, 1, hd, tpp), np.uint16)
        v[0, 0, :4, 0] = _bits([10.0, 20.0, 30.0, 40.0], dtype)
        expected = np.zeros((1, 1, hd), np.float32)
        expected[0, 0, :4] = [10.0, 20.0, 30.0, 40.0]
        inputs = dict(queries=_bits(q, dtype), k_pool=k, v_pool=v,
                      page_table=np.array([[0]], np.uint32), seq_lens=np.array([1], np.int32))
        cases.append((f"single_token_value_hd{hd}", inputs, expected))

    # decode/test_softmax_and_value.py:134-241 -- three equal scores: 1/3 average.
    hd = 32
    q = np.ones((1, 1, hd), np.float32)
    k = np.zeros((1, 1, hd // X, tpp, X), np.uint16)
    for t, (a, b) in enumerate(((0, 2), (1, 3), (2, 4))):
        vec = np.zeros(hd, np.float32)
        vec[a:b] = 1.0
        _put_k(k, 0, 0, t, _bits(vec, dtype))
    v = np.zeros((1, 1, hd, tpp), np.uint16)
    for t in range(3):
        e = np.zeros(4, np.float32)
        e[t] = 1.0
        v[0, 0, :4, t] = _bits(e, dtype)
    expected = np.zeros((1, 1, hd), np.float32)
    expected[0, 0, :3] = 1.0 / 3.0
    inputs = dict(queries=_bits(q, dtype), k_pool=k, v_pool=v,
                  page_table=np.array([[0]], np.uint32), seq_lens=np.array([3], np.int32))
    cases.append(("three_equal_scores", inputs, expected))

    # decode/test_full_attention.py:36-204 -- K = ones * {1, 2, 0.5},
    # V rows arange(base, base + HD), q = arange(1, HD + 1) / 10; the test
    # computes the softmax itself in fp32 from the dtype-rounded inputs.
    for hd in (32, 64, 128, 256):
        qf = _f32(_bits(np.arange(1, hd + 1) / 10.0, dtype), dtype)
        k = np.zeros((1, 1, hd // X, tpp, X), np.uint16)
        kvecs = []
        for t, mult in enumerate((1.0, 2.0, 0.5)):
            kb = _bits(np.ones(hd) * mult, dtype)
            _put_k(k, 0, 0, t, kb)
            kvecs.append(_f32(kb, dtype))
        v = np.zeros((1, 1, hd, tpp), np.uint16)
        vvecs = []
        for t, base in enumerate((10.0, 20.0, 30.0)):
            vb = _bits(np.arange(base, base + hd), dtype)
            v[0, 0, :, t] = vb
            vvecs.append(_f32(vb, dtype))
        scale = 1.0 / np.sqrt(np.float32(hd))
        scores = np.array([np.sum(qf * kv) * scale for kv in kvecs], np.float32)
        probs = np.exp(scores - scores.max())
        probs /= probs.sum()
        expected = sum(p * vv for p, vv in zip(probs, vvecs)).astype(np.float32)[None, None, :]
        inputs = dict(queries=_bits(qf[None, None, :], dtype), k_pool=k, v_pool=v,
                      page_table=np.array([[0]], np.uint32), seq_lens=np.array([3], np.int32))
        cases.append((f"full_attention_one_block_hd{hd}", inputs, expected))
    return cases


# ---------------------------------------------------------------------------
# prefill
# ---------------------------------------------------------------------------


def prefill_cases(dtype):
    """Prefill known-answer cases: list of (name, inputs, expected_f32 [S*P*Hq, HD])."""
    cases = []
    tpp = 16

    # prefill/test_softmax_and_value.py:36-114 -- P = 1, no history: output = V.
    for hd in (32, 64, 128):
        qp = np.ones((1, 1, hd), np.float32)
        kp = np.ones((1, 1, hd), np.float32)
        kp[0, 0, :4] = [1.0, 1.0, 0.0, 0.0]
        vp = np.zeros((1, 1, hd), np.float32)
        vp[0, 0, :4] = [10.0, 20.0, 30.0, 40.0]
        expected = np.zeros((1, hd), np.float32)
        expected[0, :4] = [10.0, 20.0, 30.0, 40.0]
        inputs = dict(q_prompt=_bits(qp, dtype), k_prompt=_bits(kp, dtype), v_prompt=_bits(vp, dtype),
                      k_pool=np.zeros((0, 1, hd // X, tpp, X), np.uint16),
                      v_pool=np.zeros((0, 1, hd, tpp), np.uint16),
                      page_table=np.zeros((1, 0), np.uint32), context_lens=np.array([0], np.int32))
        cases.append((f"single_query_no_history_hd{hd}", inputs, expected))

    # :117-187 -- causal two-token prompt: [1, 0, ...] and [.5, .5, ...].
    hd = 32
    qp = np.ones((2, 1, hd), np.float32)
    kp = np.zeros((2, 1, hd), np.float32)
    kp[0, 0, :2] = 1.0
    kp[1, 0, 1:3] = 1.0
    vp = np.zeros((2, 1, hd), np.float32)
    vp[0, 0, :4] = [1.0, 0.0, 0.0, 0.0]
    vp[1, 0, :4] = [0.0, 1.0, 0.0, 0.0]
    expected = np.zeros((2, hd), np.float32)
    expected[0, :4] = [1.0, 0.0, 0.0, 0.0]
    expected[1, :4] = [0.5, 0.5, 0.0, 0.0]
    inputs = dict(q_prompt=_bits(qp, dtype), k_prompt=_bits(kp, dtype), v_prompt=_bits(vp, dtype),
                  k_pool=np.zeros((0, 1, hd // X, tpp, X), np.uint16),
                  v_pool=np.zeros((0, 1, hd, tpp), np.uint16),
                  page_table=np.zeros((1, 0), np.uint32), context_lens=np.array([0], np.int32))
    cases.append(("causal_two_tokens", inputs, expected))

    # :190-284 -- 2 history tokens + 2 prompt tokens: [1/3]*3 and [1/4]*4.
    kp = np.zeros((2, 1, hd), np.float32)
    kp[0, 0, 2:4] = 1.0
    kp[1, 0, 3:5] = 1.0
    vp = np.zeros((2, 1, hd), np.float32)
    vp[0, 0, :4] = [0.0, 0.0, 1.0, 0.0]
    vp[1, 0, :4] = [0.0, 0.0, 0.0, 1.0]
    k = np.zeros((1, 1, hd // X, tpp, X), np.uint16)
    h0 = np.zeros(hd, np.float32)
    h0[:2] = 1.0
    h1 = np.zeros(hd, np.float32)
    h1[1:3] = 1.0
    _put_k(k, 0, 0, 0, _bits(h0, dtype))
    _put_k(k, 0, 0, 1, _bits(h1, dtype))
    v = np.zeros((1, 1, hd, tpp), np.uint16)
    v[0, 0, :4, 0] = _bits([1.0, 0.0, 0.0, 0.0], dtype)
    v[0, 0, :4, 1] = _bits([0.0, 1.0, 0.0, 0.0], dtype)
    expected = np.zeros((2, hd), np.float32)
    expected[0, :4] = [1 / 3, 1 / 3, 1 / 3, 0.0]
    expected[1, :4] = [0.25, 0.25, 0.25, 0.25]
    inputs = dict(q_prompt=_bits(qp, dtype), k_prompt=_bits(kp, dtype), v_prompt=_bits(vp, dtype),
                  k_pool=k, v_pool=v, page_table=np.array([[0]], np.uint32),
                  context_lens=np.array([2], np.int32))
    cases.append(("history_plus_prompt", inputs, expected))
    return cases
