"""CPU oracle for PAL's paged-attention path -- TEST INFRASTRUCTURE ONLY.

This module is the checker, never the product.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  The shipped operators in ``proxy_attention_lab`` run exclusively on
the HIP library and fail loudly when it is missing.

It restates, in numpy, what the reference computes on the hot path:

* ``fill_kv_pages``        -- kernels/paged_attention/fill_kv_pages.h.metal:56-116
  (index math) and src/fill_kv_pages_primitive.cpp:91-92 (functional copy).
* ``paged_attention_decode`` -- kernels/paged_attention/decode/
  paged_attention_decode.h.metal:59-65 (GQA map), :106-116 (1/sqrt(HD) scale),
  :125-131 and :298-306 (length mask), :212-241 (softmax), output shape from
  src/paged_attention_decode_primitive.cpp:289-300.
* ``paged_attention_decode_two_pass`` -- the 512-token chunking of
  paged_attention_decode_primitive.cpp:100-102 and decode.h.metal:122-139,
  367-395, merged as in decode/paged_reduce_decode.h.metal:79-128.
* ``paged_attention_prefill`` -- prefill/paged_attention_prefill.h.metal:
  62-74 (row addressing), :147-234 (causal prompt part), :251-360 (paged
  history part), :368-388 (normalise / write); output shape from
  src/paged_attention_prefill_primitive.cpp:188-192, uniform prompt length
  from :115-116.
* ``paged_attention`` (fused mixed batch) has no reference function; its
  semantics are defined by this build: row r of sequence s = q2seq[r] attends
  to the keys [0, min(seq_lens[s], q_offset[r])) of s, all read from pages.
* ``fp8_e4m3_encode`` / ``fp8_e4m3_decode`` / ``quantize_fp8`` -- fp8 KV
  pages (no reference counterpart: the reference stores f16 / bf16 only,
  paged_attention_kernels.metal:41-42); OCP e4m3 "fn" (bias 7, 3 mantissa
  bits, max 448, no infinities), round to nearest even.
* ``torch_cpu_paged_attention`` -- the same decode / fused semantics as a
  gather + torch scaled_dot_product_attention on the CPU (the reference's
  equivalency path, decode/test_sdpa_equivalency.py:106-112), timed by
  bench.py as the CPU baseline; pinned against the numpy functions above.
* ``compaction_plan`` / ``apply_moves`` / ``remap_table`` -- the page-pool
  compaction (no reference counterpart); pinned by its invariants: the live
  set becomes [0, L), ids below L stay put, every page's bytes follow it,
  and attention through the remapped tables is unchanged.
* ``rope_cos_sin_cache`` / ``apply_rope`` / ``fill_kv_pages_ex`` -- the step
  feeding fill_kv_pages (RoPE of K and Q, cast to the pool dtype) fused with
  its scatter; the scatter is that of fill_kv_pages.h.metal:65-116 with the
  K stripe x = 16 / sizeof(T) (paged_attention_decode_primitive.cpp:384-397).

All pools and activations are handled as raw 16-bit patterns (uint16) plus a
dtype tag ("f16" or "bf16"), so bf16 needs no numpy dtype and fill parity can
be checked bit for bit.  Attention math runs in float32, the precision the
reference accumulates in.

Pinning (what checks this oracle, in tests/test_oracle.py):
  * fill index math: the reference tests' own expected-pool loops
    (fill_kv_pages/test_fill_*.py), restated as known-answer tests, plus an
    independent scalar loop;
  * decode / prefill / fused: torch.nn.functional.scaled_dot_product_attention
    in float32 on contiguous K/V (a library routine), the closed-form
    known-answer tests of decode/test_full_attention.py,
    decode/test_softmax_and_value.py, prefill/test_softmax_and_value.py,
    invariance under page-table permutation, and a brute-force scalar loop
    on tiny shapes;
  * two-pass: equality with the single-pass result (any chunk size);
  * fp8 encode / decode: torch.float8_e4m3fn on every finite value, on the
    midpoints between neighbours (ties to even) and on random values;
  * RoPE: position 0 is the identity, rotations preserve the norm of every
    rotated pair, rotating by p then q equals rotating by p + q (to fp32
    rounding), GPT-J and NeoX styles agree after the matching permutation of
    dims, and a torch fp32 restatement (same operation order) agrees bit for
    bit; the cos/sin table matches its closed form (row 0 = (1, 0)).
The reference's epsilon (+1e-6 in denominators) and -88 exp clamp are not
reproduced: their relative effect is below 1e-6.
"""

from __future__ import annotations

import numpy as np

MEMORY_ALIGNMENT_BYTES = 16  # include/kernels/paged_attention_types.h:37
CHUNK_SIZE = 512  # include/kernels/paged_attention_types.h:33

# ---------------------------------------------------------------------------
# 16-bit float helpers
# ---------------------------------------------------------------------------


def bits_to_f32(bits: np.ndarray, dtype: str) -> np.ndarray:
    """Decode raw fp16/bf16 bit patterns (uint16) into float32."""
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    if dtype == "f16":
        return bits.view(np.float16).astype(np.float32)
    if dtype == "bf16":
        return (bits.astype(np.uint32) << 16).view(np.float32)
    raise ValueError(f"unsupported dtype {dtype!r}")


def f32_to_bits(x: np.ndarray, dtype: str) -> np.ndarray:
    """Round float32 to fp16/bf16 (round to nearest even) and return the bits."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if dtype == "f16":
        with np.errstate(over="ignore"):  # out-of-range values become +-inf, as in a cast
            return x.astype(np.float16).view(np.uint16)
    if dtype == "bf16":
        u = x.view(np.uint32).astype(np.uint64)
        rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
        nan = np.isnan(x)
        if nan.any():
            rounded = rounded.copy()
            rounded[nan] = 0x7FC0
        return rounded
    raise ValueError(f"unsupported dtype {dtype!r}")


FP8_MAX = 448.0


def fp8_e4m3_decode(codes: np.ndarray) -> np.ndarray:
    """uint8 e4m3 codes -> float32.  Exponent field e (4 bits, bias 7),
    mantissa m (3 bits): e == 0 -> m * 2^-9 (subnormal); e == 15 and m == 7 ->
    NaN (the only non-finite codes, sign either way); else (1 + m/8) 2^(e-7)."""
    c = np.asarray(codes, dtype=np.uint8).astype(np.int32)
    sign = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 0x7
    mag = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * np.exp2(e.astype(np.float64) - 7.0))
    out = (sign * mag).astype(np.float32)
    out[(e == 15) & (m == 7)] = np.nan
    return out


def fp8_e4m3_encode(x: np.ndarray) -> np.ndarray:
    """float32 -> uint8 e4m3 code, round to nearest even, for |x| <= 448
    (larger magnitudes and NaN give the NaN code 0x7F / 0xFF; callers clamp
    first).  Works on the exact binary value: |x| = f * 2^k with f in [1, 2)
    (frexp), mantissa (f - 1) * 8 rounded half to even; below 2^-6 the value
    is a multiple of 2^-9 rounded half to even."""
    x = np.asarray(x, dtype=np.float32).astype(np.float64)
    neg = np.signbit(x)
    a = np.abs(x)
    sub = a < 2.0 ** -6
    # subnormal range: a multiple of 2^-9 (an exact scaling; rint rounds half
    # to even); 8 becomes 0b0001000, the smallest normal
    n_sub = np.rint(np.where(sub, a, 0.0) * 2.0 ** 9).astype(np.int64)
    fr, ex = np.frexp(np.where(sub | ~np.isfinite(a), 1.0, a))  # a = fr * 2^ex, fr in [0.5, 1)
    k = ex.astype(np.int64) - 1  # a = (2 fr) 2^k
    mant = np.rint((2.0 * fr - 1.0) * 8.0).astype(np.int64)
    k = np.where(mant == 8, k + 1, k)
    mant = np.where(mant == 8, 0, mant)
    normal = ((k + 7) << 3) | mant
    code = np.where(sub, n_sub, normal)
    bad = ~np.isfinite(a) | (a > FP8_MAX) | (~sub & (code > 0x7E))
    code = np.where(bad, 0x7F, code)
    code = code | np.where(neg, 0x80, 0)
    return code.astype(np.uint8)


def quantize_fp8(x: np.ndarray, scale) -> np.ndarray:
    """The fill's fp8 quantization: q = x / scale in float32 (correctly
    rounded), held to [-448, 448] with NaN kept, then e4m3 round to nearest
    even."""
    q = np.asarray(x, np.float32) / np.asarray(scale, np.float32)
    q = np.where(q > FP8_MAX, np.float32(FP8_MAX), q)
    q = np.where(q < -FP8_MAX, np.float32(-FP8_MAX), q)
    return fp8_e4m3_encode(q.astype(np.float32))


def pool_to_f32(pool: np.ndarray, kv_dtype: str, scales=None) -> np.ndarray:
    """A K or V pool as float32 values: 16-bit bits decoded, or fp8 codes
    decoded and multiplied by their (page, kv head) scale ([P, Hkv])."""
    if kv_dtype in ("f16", "bf16"):
        return bits_to_f32(pool, kv_dtype)
    if kv_dtype != "fp8":
        raise ValueError(f"unsupported pool dtype {kv_dtype!r}")
    vals = fp8_e4m3_decode(pool)
    sc = np.asarray(scales, np.float32).reshape(pool.shape[:2] + (1,) * (pool.ndim - 2))
    return (vals * sc).astype(np.float32)


def stripe_size(dtype: str) -> int:
    """K-cache stripe width x = 16 / sizeof(T) (bindings.cpp:44-48)."""
    if dtype in ("f16", "bf16"):
        return MEMORY_ALIGNMENT_BYTES // 2
    if dtype == "fp8":
        return MEMORY_ALIGNMENT_BYTES
    raise ValueError(f"unsupported dtype {dtype!r}")


# ---------------------------------------------------------------------------
# fill_kv_pages
# ---------------------------------------------------------------------------


def fill_kv_pages(new_k, new_v, k_pool, v_pool, page_table, write_pos, q2seq):
    """Scatter new K/V rows into copies of the pools (bit patterns, uint16).

    new_k/new_v: [N, Hkv, HD] uint16.  k_pool: [P, Hkv, HD/x, TPP, x];
    v_pool: [P, Hkv, HD, TPP].  Follows fill_kv_pages.h.metal:65-116:
    seq = q2seq[t], pos = write_pos[t], page = page_table[seq, pos // TPP],
    slot = pos % TPP, K[page, h, d // x, slot, d % x] = new_k[t, h, d],
    V[page, h, d, slot] = new_v[t, h, d].  Returns (k_out, v_out); the inputs
    are left untouched, like the reference's copy at
    fill_kv_pages_primitive.cpp:91-92.  Duplicate destinations are undefined
    in the reference (racing writes); here the last token wins.
    """
    k_out = np.array(k_pool, dtype=np.uint16, copy=True)
    v_out = np.array(v_pool, dtype=np.uint16, copy=True)
    n = int(new_k.shape[0])
    if n == 0:
        return k_out, v_out
    _, hkv, nstripe, tpp, x = k_out.shape
    hd = nstripe * x
    pt = np.asarray(page_table).astype(np.int64)
    seq = np.asarray(q2seq).astype(np.int64)
    pos = np.asarray(write_pos).astype(np.int64)
    page = pt[seq, pos // tpp]
    slot = pos % tpp
    nk = np.asarray(new_k, dtype=np.uint16).reshape(n, hkv, nstripe, x)
    nv = np.asarray(new_v, dtype=np.uint16).reshape(n, hkv, hd)
    for t in range(n):  # sequential order makes the "last writer wins" rule explicit
        k_out[page[t], :, :, slot[t], :] = nk[t]
        v_out[page[t], :, :, slot[t]] = nv[t]
    return k_out, v_out


# ---------------------------------------------------------------------------
# RoPE + cast + scatter (the step feeding fill_kv_pages, fused with it)
# ---------------------------------------------------------------------------


def rope_cos_sin_cache(max_position: int, rotary_dim: int, base: float = 10000.0) -> np.ndarray:
    """[max_position, rotary_dim] float32: cos(p w_f) for f < rotary_dim / 2,
    then sin(p w_f), with w_f = base^(-2f / rotary_dim), computed in float64
    and rounded once."""
    half = rotary_dim // 2
    inv_freq = base ** (-(2.0 * np.arange(half, dtype=np.float64)) / rotary_dim)
    ang = np.arange(max_position, dtype=np.float64)[:, None] * inv_freq[None, :]
    return np.concatenate([np.cos(ang), np.sin(ang)], axis=1).astype(np.float32)


def apply_rope(x: np.ndarray, positions, table: np.ndarray, rotary_dim: int, style: str) -> np.ndarray:
    """Rotate [N, H, HD] float32 rows by the angles of their positions.

    style "neox": dims (f, f + rot/2) form pair f; "gptj": dims (2f, 2f+1).
    x' = x cos - y sin, y' = y cos + x sin, each product and sum rounded to
    float32 separately (no fused multiply-add).  Dims >= rotary_dim pass
    through; rows whose position is outside the table pass through
    unrotated."""
    x = np.array(x, dtype=np.float32, copy=True)
    pos = np.asarray(positions, np.int64)
    half = rotary_dim // 2
    ok = (pos >= 0) & (pos < table.shape[0])
    rows = table[np.where(ok, pos, 0)]
    c = rows[:, None, :half]
    s_ = rows[:, None, half:rotary_dim]
    if style == "neox":
        a = x[:, :, :half].copy()
        b = x[:, :, half:rotary_dim].copy()
    elif style == "gptj":
        a = x[:, :, 0:rotary_dim:2].copy()
        b = x[:, :, 1:rotary_dim:2].copy()
    else:
        raise ValueError(f"unknown rope style {style!r}")
    na = (a * c).astype(np.float32) - (b * s_).astype(np.float32)
    nb = (b * c).astype(np.float32) + (a * s_).astype(np.float32)
    na = np.where(ok[:, None, None], na, a)
    nb = np.where(ok[:, None, None], nb, b)
    if style == "neox":
        x[:, :, :half] = na
        x[:, :, half:rotary_dim] = nb
    else:
        x[:, :, 0:rotary_dim:2] = na
        x[:, :, 1:rotary_dim:2] = nb
    return x


def cast_to_pool(x: np.ndarray, kv_dtype: str, scales=None) -> np.ndarray:
    """float32 values -> pool element codes: f16 / bf16 bits (round to nearest
    even), or fp8 codes quantized with one scale per row ([N, Hkv] scales
    broadcast over the last dim)."""
    if kv_dtype in ("f16", "bf16"):
        return f32_to_bits(x, kv_dtype)
    return quantize_fp8(x, np.asarray(scales, np.float32)[..., None])


def fill_kv_pages_ex(new_k, new_v, k_pool, v_pool, kv_dtype, page_table, write_pos, q2seq, *,
                     k_scales=None, v_scales=None, rope=None, queries=None, q_out_dtype=None):
    """fill_kv_pages generalised: float32 source rows (the projection output),
    optional RoPE of K (and Q), cast to the pool dtype, scatter.

    new_k / new_v: [N, Hkv, HD] float32 values.  Pools: element codes (uint16
    bits for f16 / bf16, uint8 fp8 codes), K [P, Hkv, HD/x, TPP, x] with
    x = stripe_size(kv_dtype).  fp8: k_scales / v_scales [P, Hkv]; the value
    stored is quantize_fp8(x, scale of the destination (page, head)).  rope:
    None or (table, rotary_dim, style); the position is write_pos.  Tokens
    with no valid destination (sequence, position, page out of range, or a
    position outside the table) are skipped, as the kernel does.  Returns
    (k_out, v_out, q_out): copies of the pools, and the rotated queries'
    bits in q_out_dtype (None without queries).  Index math of
    fill_kv_pages.h.metal:65-116.
    """
    k_out = np.array(k_pool, copy=True)
    v_out = np.array(v_pool, copy=True)
    n = int(new_k.shape[0])
    _, hkv, nstripe, tpp, x = k_out.shape
    hd = nstripe * x
    kf = np.asarray(new_k, np.float32)
    vf = np.asarray(new_v, np.float32)
    pos = np.asarray(write_pos, np.int64)
    q_out = None
    if rope is not None:
        table, rot, style = rope
        kf = apply_rope(kf, pos, table, rot, style)
        if queries is not None:
            q_out = f32_to_bits(apply_rope(np.asarray(queries, np.float32), pos, table, rot, style), q_out_dtype)
    pt = np.asarray(page_table).astype(np.int64)
    seq = np.asarray(q2seq).astype(np.int64)
    for t in range(n):
        s_, p_ = int(seq[t]), int(pos[t])
        if s_ >= pt.shape[0] or p_ < 0 or p_ // tpp >= pt.shape[1]:
            continue
        if rope is not None and p_ >= rope[0].shape[0]:
            continue
        page = int(pt[s_, p_ // tpp])
        if page >= k_out.shape[0]:
            continue
        slot = p_ % tpp
        ks = None if k_scales is None else np.asarray(k_scales)[page]
        vs = None if v_scales is None else np.asarray(v_scales)[page]
        kc = cast_to_pool(kf[t], kv_dtype, ks)  # [Hkv, HD]
        vc = cast_to_pool(vf[t], kv_dtype, vs)
        k_out[page, :, :, slot, :] = kc.reshape(hkv, nstripe, x)
        v_out[page, :, :, slot] = vc.reshape(hkv, hd)
    return k_out, v_out, q_out


# ---------------------------------------------------------------------------
# attention helpers
# ---------------------------------------------------------------------------


def gather_tokens(k_pool_f32, v_pool_f32, page_row, n_tokens):
    """Read tokens [0, n_tokens) of one sequence out of the pools.

    Inverse of the test-side scatter at decode/test_sdpa_equivalency.py:141-173
    and prefill/test_sdpa_equivalency.py:98-117; the addressing follows
    decode.h.metal:143-190 (K) and :249-295 (V).  Returns K, V as
    [n_tokens, Hkv, HD] float32.
    """
    _, hkv, nstripe, tpp, x = k_pool_f32.shape
    hd = nstripe * x
    if n_tokens <= 0:
        z = np.zeros((0, hkv, hd), np.float32)
        return z, z.copy()
    j = np.arange(n_tokens)
    pages = np.asarray(page_row).astype(np.int64)[j // tpp]
    slots = j % tpp
    # k_pool[page, h, c, slot, e] -> [n, h, c, e] -> [n, h, hd]
    k = k_pool_f32[pages, :, :, slots, :].reshape(n_tokens, hkv, hd)
    # v_pool[page, h, d, slot] -> [n, h, d]
    v = v_pool_f32[pages, :, :, slots]
    return np.ascontiguousarray(k), np.ascontiguousarray(v)


def attend(q, k, v, limits, causal_pos=None):
    """Softmax attention with GQA for one sequence.

    q: [R, Hq, HD]; k, v: [L, Hkv, HD]; limits: [R] -- row r attends to keys
    [0, limits[r]).  Scale is 1/sqrt(HD) (decode.h.metal:115,
    prefill.h.metal:178).  Query head h reads KV head h // (Hq // Hkv)
    (decode.h.metal:64-65).  Rows with no key produce zeros.
    Returns [R, Hq, HD] float32.
    """
    r_rows, hq, hd = q.shape
    l_keys, hkv, _ = k.shape
    g = hq // hkv
    out = np.zeros((r_rows, hq, hd), np.float32)
    if r_rows == 0 or l_keys == 0:
        return out
    scale = np.float32(1.0 / np.sqrt(np.float32(hd)))
    qg = q.reshape(r_rows, hkv, g, hd).transpose(1, 0, 2, 3).reshape(hkv, r_rows * g, hd)
    kt = k.transpose(1, 2, 0)  # [Hkv, HD, L]
    s = np.matmul(qg, kt) * scale  # [Hkv, R*G, L]
    lim = np.repeat(np.asarray(limits, np.int64), g)  # [R*G]
    mask = np.arange(l_keys)[None, :] >= lim[:, None]
    s = np.where(mask[None], -np.inf, s)
    m = s.max(axis=-1, keepdims=True)
    m = np.where(np.isfinite(m), m, 0.0)
    p = np.exp(s - m)
    den = p.sum(axis=-1, keepdims=True)
    o = np.matmul(p, v.transpose(1, 0, 2))  # [Hkv, R*G, HD]
    o = np.where(den > 0, o / np.where(den > 0, den, 1.0), 0.0)
    out[:] = o.reshape(hkv, r_rows, g, hd).transpose(1, 0, 2, 3).reshape(r_rows, hq, hd)
    return out


def _pools_f32(k_pool, v_pool, dtype, kv=None):
    """float32 pools: kv = None means 16-bit pools of the query dtype; else
    kv = (k_scales, v_scales) of fp8 pools."""
    if kv is None:
        return bits_to_f32(k_pool, dtype), bits_to_f32(v_pool, dtype)
    return pool_to_f32(k_pool, "fp8", kv[0]), pool_to_f32(v_pool, "fp8", kv[1])


# ---------------------------------------------------------------------------
# operators
# ---------------------------------------------------------------------------


def paged_attention_decode(queries, k_pool, v_pool, page_table, seq_lens, dtype, kv_scales=None):
    """Decode: one query row per sequence over its paged context.

    queries: [N, Hq, HD] (or [N, HD] meaning Hq = 1) uint16 bits, N >= S; row s
    serves sequence s and rows >= S are ignored (decode.h.metal:106-108).
    kv_scales: None for 16-bit pools of the query dtype, or (k_scales,
    v_scales) of fp8 pools.  Returns [S, Hq, HD] float32
    (decode_primitive.cpp:289-300).
    """
    q = bits_to_f32(queries, dtype)
    if q.ndim == 2:
        q = q[:, None, :]
    kf, vf = _pools_f32(k_pool, v_pool, dtype, kv_scales)
    s_count = int(np.asarray(page_table).shape[0])
    hq, hd = q.shape[1], q.shape[2]
    out = np.zeros((s_count, hq, hd), np.float32)
    lens = np.asarray(seq_lens).astype(np.int64)
    for s in range(s_count):
        n = int(lens[s])
        k, v = gather_tokens(kf, vf, np.asarray(page_table)[s], n)
        out[s] = attend(q[s : s + 1], k, v, [n])[0]
    return out


def paged_attention_decode_two_pass(queries, k_pool, v_pool, page_table, seq_lens, dtype,
                                    chunk_size=CHUNK_SIZE):
    """Decode computed chunk by chunk and merged with a log-sum-exp reduction.

    Pass 1 (decode.h.metal:122-139, 211-241, 367-395): chunk c covers tokens
    [c*chunk, (c+1)*chunk); it yields the chunk max m_c, the chunk exp-sum l_c
    and the chunk-normalised output o_c.  Pass 2 (paged_reduce_decode.h.metal:
    79-128): M = max_c m_c, w_c = l_c * exp(m_c - M),
    out = sum_c w_c * o_c / sum_c w_c.  Returns [S, Hq, HD] float32.
    """
    q = bits_to_f32(queries, dtype)
    if q.ndim == 2:
        q = q[:, None, :]
    kf, vf = _pools_f32(k_pool, v_pool, dtype)
    s_count = int(np.asarray(page_table).shape[0])
    hq, hd = q.shape[1], q.shape[2]
    hkv = kf.shape[1]
    g = hq // hkv
    scale = np.float32(1.0 / np.sqrt(np.float32(hd)))
    out = np.zeros((s_count, hq, hd), np.float32)
    lens = np.asarray(seq_lens).astype(np.int64)
    for s in range(s_count):
        n = int(lens[s])
        if n <= 0:
            continue
        k, v = gather_tokens(kf, vf, np.asarray(page_table)[s], n)
        qs = q[s].reshape(hkv, g, hd)
        ms, ls, os_ = [], [], []
        for c0 in range(0, n, chunk_size):
            kc = k[c0 : c0 + chunk_size].transpose(1, 2, 0)  # [Hkv, HD, Lc]
            vc = v[c0 : c0 + chunk_size].transpose(1, 0, 2)  # [Hkv, Lc, HD]
            sc = np.matmul(qs, kc) * scale  # [Hkv, G, Lc]
            m = sc.max(axis=-1, keepdims=True)
            p = np.exp(sc - m)
            l_c = p.sum(axis=-1, keepdims=True)
            ms.append(m)
            ls.append(l_c)
            os_.append(np.matmul(p, vc) / l_c)
        m_all = np.stack(ms)  # [C, Hkv, G, 1]
        big_m = m_all.max(axis=0)
        w = np.stack(ls) * np.exp(m_all - big_m)
        o = (w * np.stack(os_)).sum(axis=0) / w.sum(axis=0)
        out[s] = o.reshape(hq, hd)
    return out


def paged_attention_prefill(q_prompt, k_prompt, v_prompt, k_pool, v_pool, page_table,
                            context_lens, dtype, kv_scales=None):
    """Prefill over paged history plus a causal dense prompt.

    q_prompt: [S*P, Hq, HD]; k_prompt/v_prompt: [S*P, Hkv, HD]; P is uniform,
    P = q_prompt.shape[0] // S (prefill_primitive.cpp:115-116).  Prompt token
    i of sequence s (global row s*P + i) attends to all context_lens[s]
    history tokens read from pages (prefill.h.metal:251-360) and to prompt
    tokens j <= i (prefill.h.metal:147-165).  Returns [S*P*Hq, HD] float32
    with row (s*P + i)*Hq + h (prefill.h.metal:379-381).
    """
    q = bits_to_f32(q_prompt, dtype)
    kp = bits_to_f32(k_prompt, dtype)
    vp = bits_to_f32(v_prompt, dtype)
    kf, vf = _pools_f32(k_pool, v_pool, dtype, kv_scales)
    pt = np.asarray(page_table)
    s_count = int(pt.shape[0])
    rows, hq, hd = q.shape
    p_len = rows // s_count if s_count else 0
    out = np.zeros((rows, hq, hd), np.float32)
    hist = np.asarray(context_lens).astype(np.int64)
    for s in range(s_count):
        h_len = int(hist[s])
        kh, vh = gather_tokens(kf, vf, pt[s], h_len)
        sl = slice(s * p_len, (s + 1) * p_len)
        k = np.concatenate([kh, kp[sl]], axis=0)
        v = np.concatenate([vh, vp[sl]], axis=0)
        limits = h_len + np.arange(1, p_len + 1)
        out[sl] = attend(q[sl], k, v, limits)
    return out.reshape(rows * hq, hd)


def paged_attention(queries, k_pool, v_pool, page_table, seq_lens, q2seq, q_offset, dtype, kv_scales=None):
    """Fused mixed batch (build-defined; no reference function exists).

    Row r belongs to sequence s = q2seq[r] and attends to the keys
    [0, min(seq_lens[s], q_offset[r])) of s, all read from pages.  A decode
    row uses q_offset = seq_lens[s]; a prefill row at absolute position p uses
    q_offset = p + 1.  Rows with no visible key, or whose q2seq names no
    sequence, are zero.  Returns [R, Hq, HD] float32.
    """
    q = bits_to_f32(queries, dtype)
    kf, vf = _pools_f32(k_pool, v_pool, dtype, kv_scales)
    pt = np.asarray(page_table)
    lens = np.asarray(seq_lens).astype(np.int64)
    seqs = np.asarray(q2seq).astype(np.int64)
    offs = np.asarray(q_offset).astype(np.int64)
    out = np.zeros(q.shape, np.float32)
    for s in np.unique(seqs):
        if s >= pt.shape[0]:  # names no sequence: nothing to attend to
            continue
        rows = np.nonzero(seqs == s)[0]
        limits = np.minimum(lens[s], offs[rows])
        n = int(max(0, limits.max()))
        k, v = gather_tokens(kf, vf, pt[s], n)
        out[rows] = attend(q[rows], k, v, limits)
    return out


# ---------------------------------------------------------------------------
# the same computation on torch CPU (the CPU baseline's comparator)
# ---------------------------------------------------------------------------


def torch_cpu_paged_attention(queries, k_pool, v_pool, page_table, seq_lens, dtype, q2seq=None, q_offset=None):
    """The reference's equivalency computation on torch CPU: gather each
    sequence's pages (decode/test_sdpa_equivalency.py:141-173 inverted),
    widen to float32, then torch's scaled_dot_product_attention with the GQA
    map h -> h // (Hq / Hkv) and the row limits as a boolean mask.  Same
    semantics as ``paged_attention`` (q2seq / q_offset given) or
    ``paged_attention_decode`` (row s = sequence s, all its keys); returns
    [R, Hq, HD] float32.  Used as the timed CPU baseline: its inputs are
    raw 16-bit patterns already in host memory, as for the numpy oracle.
    """
    import torch

    tdt = torch.bfloat16 if dtype == "bf16" else torch.float16
    q = torch.from_numpy(np.ascontiguousarray(queries).view(np.int16)).view(tdt).float()
    if q.dim() == 2:
        q = q[:, None, :]
    kp = torch.from_numpy(np.ascontiguousarray(k_pool).view(np.int16)).view(tdt)
    vp = torch.from_numpy(np.ascontiguousarray(v_pool).view(np.int16)).view(tdt)
    _, hkv, nstripe, tpp, x = kp.shape
    hd = nstripe * x
    pt = torch.from_numpy(np.asarray(page_table).astype(np.int64))
    lens = np.asarray(seq_lens).astype(np.int64)
    rows_n, hq, _ = q.shape
    g = hq // hkv
    if q2seq is None:
        seqs = np.arange(pt.shape[0], dtype=np.int64)
        offs = lens[: pt.shape[0]]
    else:
        seqs = np.asarray(q2seq).astype(np.int64)
        offs = np.asarray(q_offset).astype(np.int64)
    out = torch.zeros((len(seqs), hq, hd), dtype=torch.float32)
    for s in np.unique(seqs):
        if s >= pt.shape[0]:
            continue
        rows = np.nonzero(seqs == s)[0]
        limits = np.minimum(lens[s], offs[rows])
        n = int(max(0, limits.max()))
        if n == 0:
            continue
        npg = (n + tpp - 1) // tpp
        ids = pt[s, :npg]
        # [pages, Hkv, HD/x, TPP, x] -> [tokens, Hkv, HD]; [pages, Hkv, HD, TPP] -> [tokens, Hkv, HD]
        k = kp.index_select(0, ids).permute(0, 3, 1, 2, 4).reshape(npg * tpp, hkv, hd)[:n].float()
        v = vp.index_select(0, ids).permute(0, 3, 1, 2).reshape(npg * tpp, hkv, hd)[:n].float()
        qs = q[torch.from_numpy(rows)]                                   # [r, Hq, HD]
        qh = qs.reshape(len(rows), hkv, g, hd).permute(1, 2, 0, 3).reshape(hkv, g * len(rows), hd)
        lim = torch.from_numpy(np.tile(limits, g))                       # row order (head in group, row)
        mask = torch.arange(n)[None, :] < lim[:, None]                   # [G*r, n]
        o = torch.nn.functional.scaled_dot_product_attention(
            qh[None], k.permute(1, 0, 2)[None], v.permute(1, 0, 2)[None], attn_mask=mask[None, None])[0]
        o = torch.where((lim > 0)[None, :, None], o, torch.zeros(()))
        out[torch.from_numpy(rows)] = o.reshape(hkv, g, len(rows), hd).permute(2, 0, 1, 3).reshape(len(rows), hq, hd)
    return out.numpy()


# ---------------------------------------------------------------------------
# page-pool compaction (no reference counterpart: the reference's page
# tables come from the caller, ops.py:61-63)
# ---------------------------------------------------------------------------


def compaction_plan(used: np.ndarray, num_pages: int):
    """Moves that make the allocated ids exactly [0, L), L = len(used): every
    allocated id >= L, ascending, goes to the free ids < L, ascending.
    Returns (src, dst) uint32 arrays."""
    used = np.unique(np.asarray(used, np.int64))
    live = len(used)
    is_used = np.zeros(num_pages, bool)
    is_used[used] = True
    movers = np.nonzero(is_used[live:])[0] + live
    holes = np.nonzero(~is_used[:live])[0]
    assert len(movers) == len(holes)
    return movers.astype(np.uint32), holes.astype(np.uint32)


def apply_moves(pool: np.ndarray, src, dst) -> np.ndarray:
    """A copy of a pool (pages along axis 0) with page src[m] copied to
    dst[m]; sources and destinations disjoint."""
    out = np.array(pool, copy=True)
    out[np.asarray(dst, np.int64)] = np.asarray(pool)[np.asarray(src, np.int64)]
    return out


def remap_table(table, src, dst, num_pages: int) -> np.ndarray:
    """Page table with id src[m] replaced by dst[m] (ids >= num_pages kept)."""
    remap = np.arange(num_pages, dtype=np.int64)
    remap[np.asarray(src, np.int64)] = np.asarray(dst, np.int64)
    t = np.asarray(table).astype(np.int64)
    return np.where(t < num_pages, remap[np.minimum(t, num_pages - 1)], t).astype(np.asarray(table).dtype)


# ---------------------------------------------------------------------------
# layout helpers (restated for the tests; the product has its own)
# ---------------------------------------------------------------------------


def k_cache_shape(num_pages, num_kv_heads, head_dim, tokens_per_page, dtype):
    """decode_primitive.cpp:384-397."""
    x = stripe_size(dtype)
    return (num_pages, num_kv_heads, head_dim // x, tokens_per_page, x)


def v_cache_shape(num_pages, num_kv_heads, head_dim, tokens_per_page, dtype):
    """decode_primitive.cpp:373-381."""
    stripe_size(dtype)
    return (num_pages, num_kv_heads, head_dim, tokens_per_page)


def scatter_contiguous(k_seq, v_seq, k_pool, v_pool, page_row):
    """Write contiguous per-sequence K/V [L, Hkv, HD] (bits) into pools in place.

    The reshape/transpose formulation of the reference tests
    (decode/test_sdpa_equivalency.py:141-173): K tokens of page p are
    reshaped to [count, HD/x, x] and transposed to [HD/x, count, x]; V is
    written transposed as [HD, count].
    """
    _, hkv, nstripe, tpp, x = k_pool.shape
    n = k_seq.shape[0]
    for lp in range((n + tpp - 1) // tpp):
        page = int(page_row[lp])
        t0, t1 = lp * tpp, min((lp + 1) * tpp, n)
        cnt = t1 - t0
        for h in range(hkv):
            ks = k_seq[t0:t1, h, :].reshape(cnt, nstripe, x).transpose(1, 0, 2)
            k_pool[page, h, :, :cnt, :] = ks
            v_pool[page, h, :, :cnt] = v_seq[t0:t1, h, :].T
