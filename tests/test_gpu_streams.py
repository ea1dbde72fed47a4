"""Operators launched on a stream other than torch's current one.

Every temporary an operator makes (int64 -> int32 index conversions,
contiguous copies of strided inputs, the output, the workspace) must be
written on the launch stream and owned by it in the caching allocator.
The inputs here are int64 index tensors and non-contiguous queries, made on
the current stream; the side stream waits for them (the caller's duty, as
for any torch op on another stream), then each operator runs there and the
current stream is kept busy meanwhile.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import proxy_attention_lab as pal
from gpu_util import DEV, announce, dev_bits, host_bits, host_f32
from oracle import pal_oracle as orc
from pal_cases import assert_close, make_fused_case, make_paged_case, make_prefill_case, randn_bits

pytestmark = pytest.mark.gpu


def _i64(a) -> torch.Tensor:
    return torch.from_numpy(np.asarray(a).astype(np.int64)).to(DEV)


def _strided(bits: np.ndarray, dtype: str) -> torch.Tensor:
    """The same values as a non-contiguous view (every other element of the
    last dimension of a buffer twice as wide)."""
    t = dev_bits(bits, dtype)
    big = torch.zeros(tuple(t.shape[:-1]) + (2 * t.shape[-1],), dtype=t.dtype, device=DEV)
    big[..., ::2] = t
    view = big[..., ::2]
    assert not view.is_contiguous()
    return view


def _busy_current_stream():
    """Queue a few ms of unrelated work on the current stream."""
    a = torch.randn(2048, 2048, device=DEV)
    for _ in range(8):
        a = a @ a
        a = a / a.norm()
    return a


def test_decode_on_side_stream_int64_strided():
    case = make_paged_case(80, [300, 1, 2000, 77], 16, 4, 128, 16, "bf16")
    q = randn_bits(np.random.default_rng(80), (4, 16, 128), "bf16")
    announce("decode on a side stream, int64 indices, strided queries")
    qd, kd, vd = _strided(q, "bf16"), dev_bits(case.k_pool, "bf16"), dev_bits(case.v_pool, "bf16")
    pt, lens = _i64(case.page_table), _i64(case.seq_lens)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    _busy_current_stream()
    outs = [pal.paged_attention_decode(qd, kd, vd, pt, lens, stream=side) for _ in range(3)]
    torch.cuda.synchronize()
    ref = orc.paged_attention_decode(q, case.k_pool, case.v_pool, case.page_table, case.seq_lens, "bf16")
    for o in outs:
        assert_close(host_f32(o), ref, "bf16", "decode side stream")


def test_fused_and_fill_on_side_stream_int64():
    fc = make_fused_case(81, [40, 900], [(30, 100)], 32, 8, 64, 16, "f16", block=50)
    c = fc.case
    announce("fill + fused on a side stream, int64 indices, strided queries")
    kd, vd = dev_bits(c.k_pool, "f16"), dev_bits(c.v_pool, "f16")
    rng = np.random.default_rng(81)
    # rewrite the last token of the first decode sequence through fill_kv_pages
    nk = randn_bits(rng, (1, 8, 64), "f16")
    nv = randn_bits(rng, (1, 8, 64), "f16")
    pos = np.array([c.seq_lens[0] - 1])
    nkd, nvd, qd = _strided(nk, "f16"), _strided(nv, "f16"), _strided(fc.queries, "f16")
    pt, lens, q2s, off, posd, seq0 = (_i64(a) for a in (c.page_table, c.seq_lens, fc.q2seq, fc.q_offset, pos, [0]))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    _busy_current_stream()
    pal.fill_kv_pages(nkd, nvd, kd, vd, pt, posd, seq0, stream=side)
    out = pal.paged_attention(qd, kd, vd, pt, lens, q2s, off, stream=side)
    torch.cuda.synchronize()
    ek, ev = orc.fill_kv_pages(nk, nv, c.k_pool, c.v_pool, c.page_table, pos, np.array([0], np.uint32))
    assert np.array_equal(host_bits(kd), ek) and np.array_equal(host_bits(vd), ev)
    ref = orc.paged_attention(fc.queries, ek, ev, c.page_table, c.seq_lens, fc.q2seq, fc.q_offset, "f16")
    assert_close(host_f32(out), ref, "f16", "fused side stream")


def test_prefill_on_side_stream_int64_strided():
    case, q, k, v = make_prefill_case(82, [40, 0, 130], 21, 8, 2, 64, 16, "bf16")
    announce("prefill on a side stream, int64 indices, strided inputs")
    side = torch.cuda.Stream()
    qd, kd, vd = _strided(q, "bf16"), _strided(k, "bf16"), _strided(v, "bf16")
    kp, vp = dev_bits(case.k_pool, "bf16"), dev_bits(case.v_pool, "bf16")
    pt, lens = _i64(case.page_table), _i64(case.seq_lens)
    side.wait_stream(torch.cuda.current_stream())
    _busy_current_stream()
    out = pal.paged_attention_prefill(qd, kd, vd, kp, vp, pt, lens, stream=side)
    torch.cuda.synchronize()
    ref = orc.paged_attention_prefill(q, k, v, case.k_pool, case.v_pool, case.page_table, case.seq_lens, "bf16")
    assert_close(host_f32(out), ref, "bf16", "prefill side stream")


def test_workspace_cache_is_bounded_and_releasable():
    """Calls on many streams keep workspaces for the most recent few only,
    results stay right on every stream, and release_workspaces drops them."""
    from proxy_attention_lab import ops as pal_ops

    case = make_paged_case(81, [700, 33, 2500], 8, 2, 64, 16, "f16")
    q = randn_bits(np.random.default_rng(81), (3, 8, 64), "f16")
    qd, kd, vd = dev_bits(q, "f16"), dev_bits(case.k_pool, "f16"), dev_bits(case.v_pool, "f16")
    pt, lens = _i64(case.page_table), _i64(case.seq_lens)
    ref = orc.paged_attention_decode(q, case.k_pool, case.v_pool, case.page_table, case.seq_lens, "f16")
    announce("decode on 7 streams: bounded workspace cache")
    pal.release_workspaces()
    streams = [torch.cuda.Stream() for _ in range(7)]
    outs = []
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
        outs.append(pal.paged_attention_decode(qd, kd, vd, pt, lens, stream=s))
    torch.cuda.synchronize()
    kept = [k for k in pal_ops._WORKSPACES if k[0] == "decode"]
    assert len(kept) == pal_ops._WORKSPACES_PER_DEVICE
    assert {k[2] for k in kept} == {s.cuda_stream for s in streams[-pal_ops._WORKSPACES_PER_DEVICE:]}
    for o in outs:
        assert_close(host_f32(o), ref, "f16", "decode on a side stream (bounded cache)")
    assert pal.release_workspaces() >= len(kept)
    assert not pal_ops._WORKSPACES
    out = pal.paged_attention_decode(qd, kd, vd, pt, lens)
    torch.cuda.synchronize()
    assert_close(host_f32(out), ref, "f16", "decode after release_workspaces")
