"""The bounds-checked library variant (libpal_hip_debug.so, PAL_DEBUG_CHECKS)
records inputs the kernels tolerate but the caller most likely did not mean;
the release library records nothing and says so.

Run through the C ABI of the debug library (loaded beside the release one):
a clean decode, prefill and fill leave the flags at zero and give the same
bits as the release library; a page table naming a page past the pool, a
length past the page table and a fill token with no destination each set
their bit, while the outputs stay those of the documented tolerant
behaviour (invalid pages read as zeros, lengths clamped, tokens skipped).
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np
import pytest
import torch

import proxy_attention_lab as pal
from gpu_util import announce, dev_bits, dev_index, host_bits
from pal_cases import make_paged_case, randn_bits
from proxy_attention_lab import _lib

pytestmark = pytest.mark.gpu
DEBUG_LIB = Path(_lib.__file__).resolve().parent / "libpal_hip_debug.so"


@pytest.fixture(scope="module")
def dbg():
    if not DEBUG_LIB.exists():
        pytest.skip("libpal_hip_debug.so not built (build_lib.py --debug-checks)")
    handle = ctypes.CDLL(str(DEBUG_LIB))
    for name, (restype, argtypes) in _lib._SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype, fn.argtypes = restype, argtypes
    return handle


def _flags(lib, reset=True) -> int:
    out = ctypes.c_uint32(0)
    assert lib.pal_debug_flags(1 if reset else 0, ctypes.byref(out)) == 0
    return out.value


def _decode(lib, case, q_bits, pt=None, lens=None):
    dt = case.dtype
    pt = case.page_table if pt is None else pt
    lens = case.seq_lens if lens is None else lens
    q = dev_bits(q_bits, dt)
    k, v = dev_bits(case.k_pool, dt), dev_bits(case.v_pool, dt)
    ptd, lensd = dev_index(pt, torch.uint32), dev_index(lens)
    S, W = pt.shape
    out = torch.empty((S, case.num_q_heads, case.head_dim), dtype=q.dtype, device=q.device)
    code = _lib.DTYPE_BFLOAT16 if dt == "bf16" else _lib.DTYPE_FLOAT16
    ws_bytes = lib.pal_paged_attention_decode_workspace_size(code, S, case.num_q_heads, case.num_kv_heads,
                                                             case.head_dim, case.tokens_per_page, W, 0)
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=q.device)
    torch.cuda.synchronize()
    st = lib.pal_paged_attention_decode(q.data_ptr(), k.data_ptr(), v.data_ptr(), ptd.data_ptr(), lensd.data_ptr(),
                                        out.data_ptr(), code, S, S, case.num_q_heads, case.num_kv_heads, case.head_dim,
                                        case.tokens_per_page, int(case.k_pool.shape[0]), W, 0, ws.data_ptr(),
                                        ws_bytes, torch.cuda.current_stream().cuda_stream)
    assert st == 0, lib.pal_last_error()
    torch.cuda.synchronize()
    return host_bits(out)


def test_release_library_reports_no_checks():
    out = ctypes.c_uint32(7)
    assert _lib.lib().pal_debug_flags(1, ctypes.byref(out)) == _lib.PAL_ERR_RUNTIME
    assert out.value == 0 and "PAL_DEBUG_CHECKS" in _lib.last_error()


def test_clean_calls_set_no_flags_and_match_release(dbg):
    case = make_paged_case(95, [300, 17, 1000], 16, 4, 128, 16, "bf16")
    q = randn_bits(np.random.default_rng(95), (3, 16, 128), "bf16")
    announce("debug checks: clean decode")
    _flags(dbg)
    got = _decode(dbg, case, q)
    assert _flags(dbg) == 0
    ref = host_bits(pal.paged_attention_decode(dev_bits(q, "bf16"), dev_bits(case.k_pool, "bf16"),
                                               dev_bits(case.v_pool, "bf16"), dev_index(case.page_table, torch.uint32),
                                               dev_index(case.seq_lens)))
    assert np.array_equal(got, ref)


def test_bad_page_id_and_length_are_flagged(dbg):
    case = make_paged_case(96, [300, 17, 1000], 16, 4, 128, 16, "bf16")
    q = randn_bits(np.random.default_rng(96), (3, 16, 128), "bf16")
    num_pages = int(case.k_pool.shape[0])
    announce("debug checks: page id past the pool")
    _flags(dbg)
    pt = case.page_table.copy()
    pt[0, 3] = num_pages + 5  # a page the first sequence reads
    _decode(dbg, case, q, pt=pt)
    f = _flags(dbg)
    assert f & 1 and not f & 4
    announce("debug checks: length past the page table")
    lens = case.seq_lens.copy()
    lens[1] = case.page_table.shape[1] * 16 + 40
    _decode(dbg, case, q, lens=lens)
    assert _flags(dbg) & 2


def test_fill_without_destination_is_flagged(dbg):
    announce("debug checks: fill destination out of range")
    case = make_paged_case(97, [40, 20], 4, 2, 64, 16, "bf16")
    rng = np.random.default_rng(97)
    nk = dev_bits(randn_bits(rng, (3, 2, 64), "bf16"), "bf16")
    nv = dev_bits(randn_bits(rng, (3, 2, 64), "bf16"), "bf16")
    k, v = dev_bits(case.k_pool, "bf16"), dev_bits(case.v_pool, "bf16")
    pt = dev_index(case.page_table, torch.uint32)
    pos = dev_index(np.array([5, 9999, 3], np.int32))  # the second token has no page
    q2s = dev_index(np.array([0, 1, 1], np.uint32), torch.uint32)
    torch.cuda.synchronize()
    _flags(dbg)
    st = dbg.pal_fill_kv_pages(nk.data_ptr(), nv.data_ptr(), k.data_ptr(), v.data_ptr(), pt.data_ptr(), pos.data_ptr(),
                               q2s.data_ptr(), _lib.DTYPE_BFLOAT16, 3, 2, 64, 16, int(case.k_pool.shape[0]), 2,
                               int(case.page_table.shape[1]), torch.cuda.current_stream().cuda_stream)
    assert st == 0
    torch.cuda.synchronize()
    assert _flags(dbg) == 4
