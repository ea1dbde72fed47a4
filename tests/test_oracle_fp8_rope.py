"""CPU pins of the oracle's fp8 e4m3 codec, RoPE and general fill.

fp8: torch.float8_e4m3fn (a library codec) on every finite code, on every
midpoint between neighbouring values (ties to even) and on random values
across the exponent range.  RoPE: closed forms (position 0 is the identity,
each rotated pair keeps its norm, rotating by p then q is rotating by p + q),
the two pairings agree after the matching permutation of dims, and a torch
fp32 restatement with the same operation order agrees bit for bit.  The
general fill: with no rotation and a 16-bit source it is the reference
fill's bit copy; fp8 pages hold each value where the reference layout puts
it (K stripe x = 16).  Planted mistakes (a flipped sign, a wrong pair) are
caught.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import proxy_attention_lab as pal
from oracle import pal_oracle as orc

RNG = np.random.default_rng(1234)


def _torch_e4m3(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_fp8_decode_every_code_matches_torch():
    codes = np.arange(256, dtype=np.uint8)
    ours = orc.fp8_e4m3_decode(codes)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(np.isnan(ours), np.isnan(ref))
    fin = ~np.isnan(ref)
    assert np.array_equal(ours[fin], ref[fin])
    assert np.nanmax(ours) == 448.0 and np.isnan(ours[0x7F]) and np.isnan(ours[0xFF])


def test_fp8_encode_matches_torch_values_midpoints_random():
    vals = np.unique(orc.fp8_e4m3_decode(np.arange(256, dtype=np.uint8)))
    vals = vals[np.isfinite(vals)]
    mids = ((vals[:-1].astype(np.float64) + vals[1:]) / 2).astype(np.float32)  # exact in fp32
    # just either side of every midpoint, too
    above = np.nextafter(mids, np.float32(np.inf))
    below = np.nextafter(mids, np.float32(-np.inf))
    rnd = np.concatenate([RNG.standard_normal(200_000).astype(np.float32) * np.float32(s)
                          for s in (1e-3, 0.02, 1.0, 30.0, 150.0)])
    rnd = np.clip(rnd, -448, 448)
    for x in (vals, mids, above, below, rnd, -rnd):
        assert np.array_equal(orc.fp8_e4m3_encode(x), _torch_e4m3(x))


def test_quantize_fp8_scales_and_holds_range():
    x = np.array([0.0, 1.0, -3.0, 1000.0, -1e6, 0.3, np.nan], np.float32)
    q = orc.quantize_fp8(x, np.float32(0.5))
    assert orc.fp8_e4m3_decode(q[:3]).tolist() == [0.0, 2.0, -6.0]
    assert orc.fp8_e4m3_decode(q[3:5]).tolist() == [448.0, -448.0]  # held, not NaN
    assert np.isnan(orc.fp8_e4m3_decode(q[6:7]))[0]
    # the division is float32 and correctly rounded, then e4m3 rounding
    s = np.float32(0.37)
    y = RNG.standard_normal(10_000).astype(np.float32)
    assert np.array_equal(orc.quantize_fp8(y, s), _torch_e4m3(np.clip(y / s, -448, 448)))


def test_pool_to_f32_applies_page_head_scales():
    codes = orc.fp8_e4m3_encode(np.full((3, 2, 4, 16, 16), 1.5, np.float32))
    sc = np.array([[1, 2], [3, 4], [0.5, 0.25]], np.float32)
    f = orc.pool_to_f32(codes, "fp8", sc)
    assert np.all(f[1, 1] == 6.0) and np.all(f[2, 0] == 0.75)


# ---------------------------------------------------------------------------
# RoPE
# ---------------------------------------------------------------------------


def test_cos_sin_table_closed_form_and_product_table():
    t = orc.rope_cos_sin_cache(4096, 128, 10000.0)
    assert t.shape == (4096, 128) and t.dtype == np.float32
    assert np.all(t[0, :64] == 1.0) and np.all(t[0, 64:] == 0.0)
    # frequency 0 turns by one radian per position
    np.testing.assert_allclose(t[:, 0], np.cos(np.arange(4096)).astype(np.float32), rtol=0, atol=1e-6)
    # the product's table (torch float64, rounded once) agrees to the last bit or one ulp
    prod = pal.rope_cos_sin_cache(4096, 128, 10000.0, device="cpu").numpy()
    np.testing.assert_array_max_ulp(prod, t, maxulp=1)


@pytest.mark.parametrize("style", ["neox", "gptj"])
def test_rope_closed_forms(style):
    table = orc.rope_cos_sin_cache(1000, 64)
    x = RNG.standard_normal((5, 3, 96)).astype(np.float32)
    # position 0 is the identity
    assert np.array_equal(orc.apply_rope(x, np.zeros(5, np.int64), table, 64, style), x)
    # dims past rotary_dim pass through; each rotated pair keeps its norm
    pos = np.array([1, 7, 100, 999, 500])
    y = orc.apply_rope(x, pos, table, 64, style)
    assert np.array_equal(y[..., 64:], x[..., 64:])
    if style == "neox":
        n0 = x[..., :32] ** 2 + x[..., 32:64] ** 2
        n1 = y[..., :32] ** 2 + y[..., 32:64] ** 2
    else:
        n0 = x[..., 0:64:2] ** 2 + x[..., 1:64:2] ** 2
        n1 = y[..., 0:64:2] ** 2 + y[..., 1:64:2] ** 2
    np.testing.assert_allclose(n1, n0, rtol=1e-5, atol=1e-6)
    # rotating by p then q is rotating by p + q (to float32 rounding)
    p_ = np.array([3, 10, 200, 400, 1])
    q_ = np.array([5, 20, 300, 500, 998])
    two = orc.apply_rope(orc.apply_rope(x, p_, table, 64, style), q_, table, 64, style)
    one = orc.apply_rope(x, p_ + q_, table, 64, style)
    np.testing.assert_allclose(two, one, rtol=1e-4, atol=1e-4)
    # a position outside the table leaves the row unrotated
    assert np.array_equal(orc.apply_rope(x[:1], np.array([1000]), table, 64, style), x[:1])


def test_rope_styles_agree_after_permutation():
    table = orc.rope_cos_sin_cache(300, 64)
    x = RNG.standard_normal((4, 2, 64)).astype(np.float32)
    pos = np.array([0, 17, 150, 299])
    # gptj pair f = dims (2f, 2f+1); neox pair f = dims (f, f + 32)
    perm = np.concatenate([np.arange(0, 64, 2), np.arange(1, 64, 2)])
    neox = orc.apply_rope(x[..., perm], pos, table, 64, "neox")
    gptj = orc.apply_rope(x, pos, table, 64, "gptj")
    assert np.array_equal(neox, gptj[..., perm])


def _torch_rope(x, pos, table, rot, style):
    """torch float32 restatement: each product and sum a separate op."""
    xt = torch.from_numpy(x.copy())
    tt = torch.from_numpy(table)[torch.from_numpy(pos)]
    half = rot // 2
    c, s = tt[:, None, :half], tt[:, None, half:rot]
    if style == "neox":
        a, b = xt[..., :half].clone(), xt[..., half:rot].clone()
    else:
        a, b = xt[..., 0:rot:2].clone(), xt[..., 1:rot:2].clone()
    na = torch.sub(torch.mul(a, c), torch.mul(b, s))
    nb = torch.add(torch.mul(b, c), torch.mul(a, s))
    if style == "neox":
        xt[..., :half], xt[..., half:rot] = na, nb
    else:
        xt[..., 0:rot:2], xt[..., 1:rot:2] = na, nb
    return xt.numpy()


@pytest.mark.parametrize("style,rot", [("neox", 128), ("neox", 64), ("gptj", 128), ("gptj", 40)])
def test_rope_matches_torch_fp32_bitwise(style, rot):
    table = orc.rope_cos_sin_cache(2048, rot)
    x = RNG.standard_normal((64, 4, 128)).astype(np.float32) * np.float32(3)
    pos = RNG.integers(0, 2048, 64)
    assert np.array_equal(orc.apply_rope(x, pos, table, rot, style), _torch_rope(x, pos, table, rot, style))


def test_rope_planted_mistakes_are_caught():
    table = orc.rope_cos_sin_cache(500, 64)
    x = RNG.standard_normal((8, 2, 64)).astype(np.float32)
    pos = RNG.integers(1, 250, 8)
    good = orc.apply_rope(x, pos, table, 64, "neox")
    # a flipped sine (rotation the other way) breaks the composition law with the torch restatement
    flipped = table.copy()
    flipped[:, 32:] *= -1
    bad = orc.apply_rope(x, pos, flipped, 64, "neox")
    assert not np.array_equal(bad, _torch_rope(x, pos, table, 64, "neox"))
    # the wrong pairing (gptj applied to neox data) fails the torch check
    assert not np.array_equal(orc.apply_rope(x, pos, table, 64, "gptj"), good)


# ---------------------------------------------------------------------------
# the general fill
# ---------------------------------------------------------------------------


def _case(n_pages=12, hkv=2, hd=64, tpp=16, kv="bf16"):
    x = orc.stripe_size(kv)
    dt = np.uint8 if kv == "fp8" else np.uint16
    k = RNG.integers(0, 255 if kv == "fp8" else 65535, size=(n_pages, hkv, hd // x, tpp, x)).astype(dt)
    v = RNG.integers(0, 255 if kv == "fp8" else 65535, size=(n_pages, hkv, hd, tpp)).astype(dt)
    pt = np.array([[3, 7, 1], [9, 0, 4]], np.uint32)
    return k, v, pt


def test_fill_ex_without_rope_is_the_reference_copy():
    k, v, pt = _case()
    n = 20
    nk = RNG.standard_normal((n, 2, 64)).astype(np.float32)
    nv = RNG.standard_normal((n, 2, 64)).astype(np.float32)
    nk_b, nv_b = orc.f32_to_bits(nk, "bf16"), orc.f32_to_bits(nv, "bf16")
    pos = np.concatenate([np.arange(10, 20), np.arange(30, 40)]).astype(np.int32)
    q2s = np.repeat([0, 1], 10).astype(np.uint32)
    ek, ev = orc.fill_kv_pages(nk_b, nv_b, k, v, pt, pos, q2s)
    # float32 rows of bf16 values: the cast is exact, so the result is the bit copy
    gk, gv, _ = orc.fill_kv_pages_ex(orc.bits_to_f32(nk_b, "bf16"), orc.bits_to_f32(nv_b, "bf16"), k, v, "bf16",
                                     pt, pos, q2s)
    assert np.array_equal(gk, ek) and np.array_equal(gv, ev)


def test_fill_ex_fp8_layout_known_answer():
    """One token at position 21 of sequence 0 (page pt[0,1] = 7, slot 5):
    value d of head h is (d % 7) * 0.5 + h with scale 0.5 -> code of
    (d % 7) + 2h.  K stripe x = 16: K[7, h, d // 16, 5, d % 16]; V[7, h, d, 5]."""
    k, v, pt = _case(kv="fp8")
    hd = 64
    d = np.arange(hd)
    vals = np.stack([(d % 7) * 0.5 + h for h in range(2)]).astype(np.float32)[None]  # [1, 2, 64]
    sc = np.full((12, 2), 0.5, np.float32)
    gk, gv, _ = orc.fill_kv_pages_ex(vals, vals, k, v, "fp8", pt, np.array([21], np.int32),
                                     np.array([0], np.uint32), k_scales=sc, v_scales=sc)
    for h in range(2):
        want = orc.fp8_e4m3_encode((d % 7) + 2.0 * h)
        assert np.array_equal(gk[7, h, d // 16, 5, d % 16], want)
        assert np.array_equal(gv[7, h, d, 5], want)
    # nothing else moved
    mask = np.ones(k.shape, bool)
    mask[7, :, :, 5, :] = False
    assert np.array_equal(gk[mask], k[mask])


def test_fill_ex_rope_rotates_keys_and_queries_only():
    k, v, pt = _case(kv="f16")
    table = orc.rope_cos_sin_cache(64, 64)
    n = 5
    nk = RNG.standard_normal((n, 2, 64)).astype(np.float32)
    nv = RNG.standard_normal((n, 2, 64)).astype(np.float32)
    q = RNG.standard_normal((n, 4, 64)).astype(np.float32)
    pos = np.array([0, 1, 2, 40, 47], np.int32)
    q2s = np.zeros(n, np.uint32)
    gk, gv, qo = orc.fill_kv_pages_ex(nk, nv, k, v, "f16", pt, pos, q2s, rope=(table, 64, "neox"), queries=q,
                                      q_out_dtype="bf16")
    rk = orc.apply_rope(nk, pos, table, 64, "neox")
    ek, ev, _ = orc.fill_kv_pages_ex(rk, nv, k, v, "f16", pt, pos, q2s)
    assert np.array_equal(gk, ek) and np.array_equal(gv, ev)  # V unrotated
    assert np.array_equal(qo, orc.f32_to_bits(orc.apply_rope(q, pos, table, 64, "neox"), "bf16"))
    assert np.array_equal(qo[0], orc.f32_to_bits(q[0], "bf16"))  # position 0
