"""GPU parity of the fp8 KV pages and the fused RoPE + cast + scatter.

Pools after fill_kv_pages (fp8, or 16-bit from fp32 / other-dtype rows) and
after rope_fill_kv_pages, and the rotated queries, must be bit-exact against
the oracle (oracle.fill_kv_pages_ex).  Decode, prefill and the fused mixed
batch over fp8 pools are compared with the oracle on the dequantized pools
(code x scale of its (page, kv head)) at the query dtype's attention
tolerance: bf16 atol/rtol 2e-2, fp16 5e-3.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import proxy_attention_lab as pal
from gpu_util import DEV, announce, dev_bits, dev_index, host_bits, host_f32
from oracle import pal_oracle as orc
from pal_cases import assert_close, compact_subset, extreme_query_bits, make_paged_case, randn_bits

pytestmark = pytest.mark.gpu
TD = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}


def dev_codes(codes: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(codes, np.uint8)).to(DEV).view(torch.float8_e4m3fn)


def host_codes(t: torch.Tensor) -> np.ndarray:
    return t.view(torch.uint8).cpu().numpy()


def dev_pool(codes: np.ndarray, kv: str) -> torch.Tensor:
    return dev_codes(codes) if kv == "fp8" else dev_bits(codes, kv)


def host_pool(t: torch.Tensor, kv: str) -> np.ndarray:
    return host_codes(t) if kv == "fp8" else host_bits(t)


def dev_f32(x: np.ndarray, dt: str) -> torch.Tensor:
    """Source rows on the device in dtype dt holding exactly the values x
    (x must be representable: pass values already rounded to dt)."""
    t = torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(DEV)
    return t.to(TD[dt])


def src_values(rng, shape, dt: str, scale: float = 1.0) -> np.ndarray:
    """N(0, scale) values exactly representable in dt."""
    x = rng.standard_normal(shape).astype(np.float32) * np.float32(scale)
    if dt in ("f16", "bf16"):
        x = orc.bits_to_f32(orc.f32_to_bits(x, dt), dt)
    return x


def fill_layout(seed, hkv, hd, tpp, kv, n_decode=9, chunks=((37, 70), (0, 33), (5, 1))):
    """Pools of random codes and a permuted page table; new tokens: one per
    decode sequence at a random position, plus prefill runs (start, length)
    of consecutive positions.  Returns (k, v, pt, pos, q2seq, scales)."""
    rng = np.random.default_rng(seed)
    lens = [int(x) for x in rng.integers(1, 300, n_decode)] + [s + n for s, n in chunks]
    w = max((l + tpp - 1) // tpp for l in lens)
    n_pages = sum((l + tpp - 1) // tpp for l in lens) + 5
    perm = rng.permutation(n_pages).astype(np.uint32)
    pt = rng.integers(0, n_pages, size=(len(lens), w)).astype(np.uint32)
    cur = 0
    for s, l in enumerate(lens):
        npg = (l + tpp - 1) // tpp
        pt[s, :npg] = perm[cur:cur + npg]
        cur += npg
    x = orc.stripe_size(kv)
    hi = 255 if kv == "fp8" else 65535
    dt = np.uint8 if kv == "fp8" else np.uint16
    k = rng.integers(0, hi, size=(n_pages, hkv, hd // x, tpp, x)).astype(dt)
    v = rng.integers(0, hi, size=(n_pages, hkv, hd, tpp)).astype(dt)
    pos = [int(rng.integers(0, lens[s])) for s in range(n_decode)]
    q2s = list(range(n_decode))
    for j, (st, n) in enumerate(chunks):
        pos += list(range(st, st + n))
        q2s += [n_decode + j] * n
    order = rng.permutation(n_decode)  # decode tokens in shuffled order, runs kept consecutive
    pos = np.array([pos[i] for i in order] + pos[n_decode:], np.int32)
    q2s = np.array([q2s[i] for i in order] + q2s[n_decode:], np.uint32)
    scales = (rng.uniform(0.004, 0.03, size=(n_pages, hkv)).astype(np.float32),
              rng.uniform(0.004, 0.03, size=(n_pages, hkv)).astype(np.float32))
    return k, v, pt, pos, q2s, scales


@pytest.mark.parametrize("src", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("hd,tpp", [(128, 16), (64, 32), (256, 16)])
def test_fill_fp8_bit_exact(src, hd, tpp):
    k, v, pt, pos, q2s, (ks, vs) = fill_layout(hd + tpp, 4, hd, tpp, "fp8")
    rng = np.random.default_rng(hd)
    n = len(pos)
    nk = src_values(rng, (n, 4, hd), src, 2.0)
    nv = src_values(rng, (n, 4, hd), src, 2.0)
    announce(f"fill fp8 src={src} hd={hd} tpp={tpp} n={n}")
    kd, vd = dev_codes(k), dev_codes(v)
    pal.fill_kv_pages(dev_f32(nk, src), dev_f32(nv, src), kd, vd, dev_index(pt, torch.uint32), dev_index(pos),
                      dev_index(q2s, torch.uint32), k_scales=torch.from_numpy(ks).to(DEV),
                      v_scales=torch.from_numpy(vs).to(DEV))
    torch.cuda.synchronize()
    ek, ev, _ = orc.fill_kv_pages_ex(nk, nv, k, v, "fp8", pt, pos, q2s, k_scales=ks, v_scales=vs)
    assert np.array_equal(host_codes(kd), ek), "fp8 K pool differs"
    assert np.array_equal(host_codes(vd), ev), "fp8 V pool differs"


@pytest.mark.parametrize("src,kv", [("f32", "bf16"), ("f32", "f16"), ("bf16", "f16"), ("f16", "bf16")])
def test_fill_cast_bit_exact(src, kv):
    k, v, pt, pos, q2s, _ = fill_layout(7, 8, 128, 16, kv)
    rng = np.random.default_rng(8)
    n = len(pos)
    nk = src_values(rng, (n, 8, 128), src, 3.0)
    nv = src_values(rng, (n, 8, 128), src, 3.0)
    announce(f"fill cast {src}->{kv}")
    kd, vd = dev_bits(k, kv), dev_bits(v, kv)
    pal.fill_kv_pages(dev_f32(nk, src), dev_f32(nv, src), kd, vd, dev_index(pt, torch.uint32), dev_index(pos),
                      dev_index(q2s, torch.uint32))
    torch.cuda.synchronize()
    ek, ev, _ = orc.fill_kv_pages_ex(nk, nv, k, v, kv, pt, pos, q2s)
    assert np.array_equal(host_bits(kd), ek) and np.array_equal(host_bits(vd), ev)


@pytest.mark.parametrize("style,rot", [("neox", 128), ("neox", 64), ("gptj", 128), ("gptj", 40)])
@pytest.mark.parametrize("src,kv", [("f32", "bf16"), ("bf16", "bf16"), ("f32", "fp8"), ("f16", "f16")])
def test_rope_fill_bit_exact(style, rot, src, kv):
    hkv, hq, hd, tpp = 4, 16, 128, 16
    k, v, pt, pos, q2s, (ks, vs) = fill_layout(rot + len(src), hkv, hd, tpp, kv)
    rng = np.random.default_rng(rot)
    n = len(pos)
    nk = src_values(rng, (n, hkv, hd), src, 2.0)
    nv = src_values(rng, (n, hkv, hd), src, 2.0)
    q = src_values(rng, (n, hq, hd), src, 2.0)
    table = pal.rope_cos_sin_cache(512, rot, 10000.0, device=DEV)
    qdt = "f16" if kv == "f16" else "bf16"
    announce(f"rope fill {style} rot={rot} {src}->{kv}")
    kd, vd = dev_pool(k, kv), dev_pool(v, kv)
    extra = {}
    if kv == "fp8":
        extra = dict(k_scales=torch.from_numpy(ks).to(DEV), v_scales=torch.from_numpy(vs).to(DEV))
    _, _, qo = pal.rope_fill_kv_pages(dev_f32(nk, src), dev_f32(nv, src), kd, vd, dev_index(pt, torch.uint32),
                                      dev_index(pos), dev_index(q2s, torch.uint32), table, queries=dev_f32(q, src),
                                      rotary_dim=rot, style=style, query_dtype=TD[qdt], **extra)
    torch.cuda.synchronize()
    tab = table.cpu().numpy()
    ek, ev, eq = orc.fill_kv_pages_ex(nk, nv, k, v, kv, pt, pos, q2s, k_scales=ks if kv == "fp8" else None,
                                      v_scales=vs if kv == "fp8" else None, rope=(tab, rot, style), queries=q,
                                      q_out_dtype=qdt)
    assert np.array_equal(host_pool(kd, kv), ek), "K pool differs"
    assert np.array_equal(host_pool(vd, kv), ev), "V pool differs"
    assert np.array_equal(host_bits(qo), eq), "rotated queries differ"


@pytest.mark.parametrize("hd", [32, 64, 96, 256])
@pytest.mark.parametrize("style,rot_frac", [("neox", 1), ("gptj", 2)])
def test_rope_fill_head_dims(hd, style, rot_frac):
    """fp32 rows into bf16 pools at other head dims: the query rows and the
    K/V rows move in 16-byte pieces (lanes per token hd/4 and hd/8, a token
    straddling wavefronts at HD 96), NeoX over the whole head, GPT-J over half
    of it; pools and rotated queries bit-exact."""
    hkv, hq, tpp = 2, 8, 16
    rot = hd // rot_frac
    k, v, pt, pos, q2s, _ = fill_layout(hd + rot_frac, hkv, hd, tpp, "bf16")
    rng = np.random.default_rng(hd * 10 + rot_frac)
    n = len(pos)
    nk = src_values(rng, (n, hkv, hd), "f32", 2.0)
    nv = src_values(rng, (n, hkv, hd), "f32", 2.0)
    q = src_values(rng, (n, hq, hd), "f32", 2.0)
    table = pal.rope_cos_sin_cache(512, rot, 10000.0, device=DEV)
    announce(f"rope fill head dim {hd} {style} rot={rot}")
    kd, vd = dev_pool(k, "bf16"), dev_pool(v, "bf16")
    _, _, qo = pal.rope_fill_kv_pages(dev_f32(nk, "f32"), dev_f32(nv, "f32"), kd, vd, dev_index(pt, torch.uint32),
                                      dev_index(pos), dev_index(q2s, torch.uint32), table, queries=dev_f32(q, "f32"),
                                      rotary_dim=rot, style=style, query_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    ek, ev, eq = orc.fill_kv_pages_ex(nk, nv, k, v, "bf16", pt, pos, q2s, rope=(table.cpu().numpy(), rot, style),
                                      queries=q, q_out_dtype="bf16")
    assert np.array_equal(host_pool(kd, "bf16"), ek), "K pool differs"
    assert np.array_equal(host_pool(vd, "bf16"), ev), "V pool differs"
    assert np.array_equal(host_bits(qo), eq), "rotated queries differ"


@pytest.mark.parametrize("hd", [128, 256])
def test_rope_fill_large_batch(hd):
    """A prefill-sized RoPE fill (more than 2048 tokens: the 64-token windows,
    1024 threads per workgroup above head dim 128): pools and rotated queries
    bit-exact."""
    hkv, hq, tpp = 4, 8, 16
    k, v, pt, pos, q2s, _ = fill_layout(hd + 5, hkv, hd, tpp, "bf16", chunks=((0, 1500), (100, 700)))
    rng = np.random.default_rng(hd + 6)
    n = len(pos)
    assert n >= 2048
    nk = src_values(rng, (n, hkv, hd), "f32", 2.0)
    nv = src_values(rng, (n, hkv, hd), "f32", 2.0)
    q = src_values(rng, (n, hq, hd), "f32", 2.0)
    table = pal.rope_cos_sin_cache(2048, hd, 10000.0, device=DEV)
    announce(f"rope fill large batch head dim {hd} ({n} tokens)")
    kd, vd = dev_pool(k, "bf16"), dev_pool(v, "bf16")
    _, _, qo = pal.rope_fill_kv_pages(dev_f32(nk, "f32"), dev_f32(nv, "f32"), kd, vd, dev_index(pt, torch.uint32),
                                      dev_index(pos), dev_index(q2s, torch.uint32), table, queries=dev_f32(q, "f32"),
                                      rotary_dim=hd, style="neox", query_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    ek, ev, eq = orc.fill_kv_pages_ex(nk, nv, k, v, "bf16", pt, pos, q2s, rope=(table.cpu().numpy(), hd, "neox"),
                                      queries=q, q_out_dtype="bf16")
    assert np.array_equal(host_pool(kd, "bf16"), ek), "K pool differs"
    assert np.array_equal(host_pool(vd, "bf16"), ev), "V pool differs"
    assert np.array_equal(host_bits(qo), eq), "rotated queries differ"


def test_rope_fill_positions_outside_table():
    """Tokens whose position has no row in the cos/sin table leave the pools
    alone; their queries come back cast, unrotated."""
    k, v, pt, pos, q2s, _ = fill_layout(3, 2, 64, 16, "bf16", chunks=((0, 40),))
    rng = np.random.default_rng(3)
    n = len(pos)
    nk = src_values(rng, (n, 2, 64), "f32")
    nv = src_values(rng, (n, 2, 64), "f32")
    q = src_values(rng, (n, 4, 64), "f32")
    table = pal.rope_cos_sin_cache(30, 64, device=DEV)  # positions >= 30 have no row
    announce("rope fill positions outside the table")
    kd, vd = dev_bits(k, "bf16"), dev_bits(v, "bf16")
    _, _, qo = pal.rope_fill_kv_pages(dev_f32(nk, "f32"), dev_f32(nv, "f32"), kd, vd, dev_index(pt, torch.uint32),
                                      dev_index(pos), dev_index(q2s, torch.uint32), table, queries=dev_f32(q, "f32"))
    torch.cuda.synchronize()
    ek, ev, eq = orc.fill_kv_pages_ex(nk, nv, k, v, "bf16", pt, pos, q2s, rope=(table.cpu().numpy(), 64, "neox"),
                                      queries=q, q_out_dtype="bf16")
    assert np.array_equal(host_bits(kd), ek) and np.array_equal(host_bits(vd), ev)
    assert np.array_equal(host_bits(qo), eq)


# ---------------------------------------------------------------------------
# decode over fp8 pools
# ---------------------------------------------------------------------------


def fp8_case(case, rng, headroom=(1.0, 2.0)):
    """fp8 pools from a 16-bit case: per-(page, kv head) scale = amax / 448
    times a headroom in the given range (NaN garbage slots stay NaN codes)."""
    kf = orc.bits_to_f32(case.k_pool, case.dtype)
    vf = orc.bits_to_f32(case.v_pool, case.dtype)
    with np.errstate(all="ignore"):
        ka = np.nanmax(np.abs(kf).reshape(kf.shape[0], kf.shape[1], -1), axis=2)
        va = np.nanmax(np.abs(vf).reshape(vf.shape[0], vf.shape[1], -1), axis=2)
    hr = rng.uniform(*headroom, size=ka.shape).astype(np.float32)
    ks = np.where(ka > 0, ka / 448 * hr, 1.0).astype(np.float32)
    vs = np.where(va > 0, va / 448 * hr, 1.0).astype(np.float32)
    p_, h_, c_, t_, x_ = kf.shape
    # 16-bit K layout [P, H, HD/8, TPP, 8] -> fp8 layout [P, H, HD/16, TPP, 16]
    k_tok = kf.transpose(0, 1, 3, 2, 4).reshape(p_, h_, t_, c_ * x_)  # [P, H, TPP, HD]
    k8 = k_tok.reshape(p_, h_, t_, c_ * x_ // 16, 16).transpose(0, 1, 3, 2, 4)
    kc = orc.quantize_fp8(k8, ks[:, :, None, None, None])
    vc = orc.quantize_fp8(vf, vs[:, :, None, None])
    return kc, vc, ks, vs


def _decode_fp8(case, q, kc, vc, ks, vs, partition=0):
    out = pal.paged_attention_decode(dev_bits(q, case.dtype), dev_codes(kc), dev_codes(vc),
                                     dev_index(case.page_table, torch.uint32), dev_index(case.seq_lens),
                                     partition_size=partition, k_scales=torch.from_numpy(ks).to(DEV),
                                     v_scales=torch.from_numpy(vs).to(DEV))
    torch.cuda.synchronize()
    return host_f32(out)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("hd,tpp", [(128, 16), (64, 32), (256, 16), (128, 32), (256, 32)])
@pytest.mark.parametrize("partition", [0, 512])
def test_decode_fp8_pages(dtype, hd, tpp, partition):
    """fp8 pages against the oracle on dequantized pools.  The V codes are read
    as 16-byte rows (one per 64 dims) at the block's slot offset in its page
    (0, or 16 on 32-token pages) and transposed across the lane groups."""
    lens = [1, 15, 16, 17, 100, 0, 511, 512, 513, 1000, 2049, 37, 5000]
    rng = np.random.default_rng(hd + tpp + partition)
    case = make_paged_case(hd * 3 + tpp, lens, 16, 4, hd, tpp, dtype)
    kc, vc, ks, vs = fp8_case(case, rng)
    q = randn_bits(rng, (len(lens), 16, hd), dtype)
    announce(f"decode fp8 pages {dtype} hd={hd} tpp={tpp} partition={partition}")
    out = _decode_fp8(case, q, kc, vc, ks, vs, partition)
    ref = orc.paged_attention_decode(q, kc, vc, case.page_table, case.seq_lens, dtype, kv_scales=(ks, vs))
    assert_close(out, ref, dtype, f"fp8 decode {dtype} hd{hd} tpp{tpp} p{partition}")


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("partition", [0, 512])
def test_decode_fp8_query_magnitudes(dtype, partition):
    """The fp8 decode turns each query head into fp8 terms scaled by a
    per-head power of two: heads across the dtype's range (extreme_query_bits)
    attend as the oracle does."""
    lens = [1, 17, 300, 1000, 2049]
    rng = np.random.default_rng(71 + partition)
    case = make_paged_case(71, lens, 16, 4, 128, 16, dtype)
    kc, vc, ks, vs = fp8_case(case, rng)
    q = extreme_query_bits(rng, (len(lens), 16, 128), dtype)
    announce(f"decode fp8 query magnitudes {dtype} partition={partition}")
    out = _decode_fp8(case, q, kc, vc, ks, vs, partition)
    ref = orc.paged_attention_decode(q, kc, vc, case.page_table, case.seq_lens, dtype, kv_scales=(ks, vs))
    assert np.isfinite(out).all()
    assert_close(out, ref, dtype, f"fp8 decode query magnitudes {dtype} p{partition}")


def test_decode_fp8_config2_shape_subset():
    """Config 2's shape (64 sequences, ctx U[512, 4096], 32/8 heads, HD 128)
    over fp8 pages with bf16 queries; 8 sequences re-checked on the oracle."""
    rng = np.random.default_rng(22)
    lens = rng.integers(512, 4097, size=64).astype(np.int32)
    case = make_paged_case(22, lens, 32, 8, 128, 16, "bf16")
    kc, vc, ks, vs = fp8_case(case, rng)
    q = randn_bits(rng, (64, 32, 128), "bf16")
    announce("decode fp8 config-2 shape")
    out = _decode_fp8(case, q, kc, vc, ks, vs)
    assert np.isfinite(out).all()
    pick = np.array([0, 9, 18, 27, 36, 45, 54, 63])
    sub = compact_subset(case, pick)
    used = []
    for s in pick:
        used.extend(int(x) for x in case.page_table[s, : (int(case.seq_lens[s]) + 15) // 16])
    uniq = np.unique(np.asarray(used))
    ref = orc.paged_attention_decode(q[pick], kc[uniq], vc[uniq], sub.page_table, sub.seq_lens, "bf16",
                                     kv_scales=(ks[uniq], vs[uniq]))
    assert_close(out[pick], ref, "bf16", "fp8 config-2 subset")


def test_fill_fp8_then_decode_round_trip():
    """fill_kv_pages writes each sequence's newest token into fp8 pages, then
    decode reads them: equal to the oracle decode over the oracle-filled pool."""
    rng = np.random.default_rng(31)
    lens = rng.integers(20, 700, size=12).astype(np.int32)
    case = make_paged_case(31, lens, 32, 8, 128, 16, "bf16", garbage_tail=False)
    kc, vc, ks, vs = fp8_case(case, rng, headroom=(2.0, 3.0))
    nk = src_values(rng, (12, 8, 128), "bf16")
    nv = src_values(rng, (12, 8, 128), "bf16")
    pos = lens - 1
    q2s = np.arange(12, dtype=np.uint32)
    q = randn_bits(rng, (12, 32, 128), "bf16")
    announce("fp8 fill then decode")
    kd, vd = dev_codes(kc), dev_codes(vc)
    ksd, vsd = torch.from_numpy(ks).to(DEV), torch.from_numpy(vs).to(DEV)
    pt = dev_index(case.page_table, torch.uint32)
    pal.fill_kv_pages(dev_f32(nk, "bf16"), dev_f32(nv, "bf16"), kd, vd, pt, dev_index(pos), dev_index(q2s, torch.uint32),
                      k_scales=ksd, v_scales=vsd)
    out = pal.paged_attention_decode(dev_bits(q, "bf16"), kd, vd, pt, dev_index(lens), k_scales=ksd, v_scales=vsd)
    torch.cuda.synchronize()
    ek, ev, _ = orc.fill_kv_pages_ex(nk, nv, kc, vc, "fp8", case.page_table, pos, q2s, k_scales=ks, v_scales=vs)
    assert np.array_equal(host_codes(kd), ek) and np.array_equal(host_codes(vd), ev)
    ref = orc.paged_attention_decode(q, ek, ev, case.page_table, lens, "bf16", kv_scales=(ks, vs))
    assert_close(host_f32(out), ref, "bf16", "fp8 fill + decode")


# ---------------------------------------------------------------------------
# prefill and the fused mixed batch over fp8 pools
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("hd,tpp", [(128, 16), (64, 32), (256, 16)])
def test_prefill_fp8_history(dtype, hd, tpp):
    """The reference prefill signature over an fp8 history (dense prompt in
    the query dtype): history keys straddling the prompt, ragged histories."""
    from pal_cases import make_prefill_case

    rng = np.random.default_rng(hd + tpp + 7)
    case, q, k, v = make_prefill_case(hd * 5 + tpp, [0, 37, 300, 1000], 45, 16, 4, hd, tpp, dtype)
    kc, vc, ks, vs = fp8_case(case, rng)
    announce(f"prefill fp8 history {dtype} hd={hd} tpp={tpp}")
    out = pal.paged_attention_prefill(dev_bits(q, dtype), dev_bits(k, dtype), dev_bits(v, dtype), dev_codes(kc),
                                      dev_codes(vc), dev_index(case.page_table, torch.uint32), dev_index(case.seq_lens),
                                      k_scales=torch.from_numpy(ks).to(DEV), v_scales=torch.from_numpy(vs).to(DEV))
    torch.cuda.synchronize()
    ref = orc.paged_attention_prefill(q, k, v, kc, vc, case.page_table, case.seq_lens, dtype, kv_scales=(ks, vs))
    assert_close(host_f32(out), ref, dtype, f"fp8 prefill {dtype} hd{hd} tpp{tpp}")


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("hd,tpp", [(128, 16), (64, 32), (256, 16)])
def test_fused_fp8_pages(dtype, hd, tpp):
    """A mixed batch over fp8 pages: decode rows (the fused kernel's decode
    workers, or the stream kernel at head_dim 256) and prefill runs."""
    from pal_cases import make_fused_case

    rng = np.random.default_rng(hd * 3 + tpp)
    fc = make_fused_case(hd + tpp + 11, [1, 17, 300, 2049, 0, 700], [(0, 70), (130, 64), (900, 129)], 32, 8, hd,
                         tpp, dtype, block=40)
    c = fc.case
    kc, vc, ks, vs = fp8_case(c, rng)
    announce(f"fused fp8 pages {dtype} hd={hd} tpp={tpp}")
    out = pal.paged_attention(dev_bits(fc.queries, dtype), dev_codes(kc), dev_codes(vc),
                              dev_index(c.page_table, torch.uint32), dev_index(c.seq_lens),
                              dev_index(fc.q2seq, torch.uint32), dev_index(fc.q_offset),
                              k_scales=torch.from_numpy(ks).to(DEV), v_scales=torch.from_numpy(vs).to(DEV))
    torch.cuda.synchronize()
    ref = orc.paged_attention(fc.queries, kc, vc, c.page_table, c.seq_lens, fc.q2seq, fc.q_offset, dtype,
                              kv_scales=(ks, vs))
    assert_close(host_f32(out), ref, dtype, f"fp8 fused {dtype} hd{hd} tpp{tpp}")


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_fused_fp8_query_magnitudes(dtype):
    """fp8 pages under the fused op with query heads across the dtype's range
    (zeros, tiny, large, mixed, near the range ends; the large heads held to
    the tiles' exact range), in its decode rows and its tiles."""
    from pal_cases import make_fused_case

    rng = np.random.default_rng(75)
    fc = make_fused_case(75, [5, 300, 1200], [(0, 70), (200, 130)], 16, 4, 128, 16, dtype)
    fc.queries = extreme_query_bits(rng, fc.queries.shape, dtype, tiles=True)
    c = fc.case
    kc, vc, ks, vs = fp8_case(c, rng)
    announce(f"fused fp8 pages, query magnitudes {dtype}")
    out = pal.paged_attention(dev_bits(fc.queries, dtype), dev_codes(kc), dev_codes(vc),
                              dev_index(c.page_table, torch.uint32), dev_index(c.seq_lens),
                              dev_index(fc.q2seq, torch.uint32), dev_index(fc.q_offset),
                              k_scales=torch.from_numpy(ks).to(DEV), v_scales=torch.from_numpy(vs).to(DEV))
    torch.cuda.synchronize()
    got = host_f32(out)
    ref = orc.paged_attention(fc.queries, kc, vc, c.page_table, c.seq_lens, fc.q2seq, fc.q_offset, dtype,
                              kv_scales=(ks, vs))
    assert np.isfinite(got).all()
    assert_close(got, ref, dtype, f"fp8 fused query magnitudes {dtype}")


def test_fused_fp8_claiming_mode():
    """More than 2048 lone rows with keys over fp8 pages at head_dim 128: the
    fused kernel's decode workers claim row batches and compute rows whole."""
    from pal_cases import make_fused_case

    rng = np.random.default_rng(71)
    dec = rng.integers(1, 200, size=2100)
    fc = make_fused_case(71, dec, [(20, 150)], 16, 4, 128, 16, "f16", block=50)
    c = fc.case
    kc, vc, ks, vs = fp8_case(c, rng)
    announce("fused fp8 pages, claiming mode (2100 lone rows)")
    out = pal.paged_attention(dev_bits(fc.queries, "f16"), dev_codes(kc), dev_codes(vc),
                              dev_index(c.page_table, torch.uint32), dev_index(c.seq_lens),
                              dev_index(fc.q2seq, torch.uint32), dev_index(fc.q_offset),
                              k_scales=torch.from_numpy(ks).to(DEV), v_scales=torch.from_numpy(vs).to(DEV))
    torch.cuda.synchronize()
    ref = orc.paged_attention(fc.queries, kc, vc, c.page_table, c.seq_lens, fc.q2seq, fc.q_offset, "f16",
                              kv_scales=(ks, vs))
    assert_close(host_f32(out), ref, "f16", "fp8 fused claiming mode")
