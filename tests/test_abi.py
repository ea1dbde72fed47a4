"""CPU checks of the C ABI: the library loads, exports every entry point the
header declares, and rejects bad arguments before touching a device."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

import proxy_attention_lab as pal
from proxy_attention_lab import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "pal_hip.h"


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pal_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    names = declared_functions()
    assert names, "no declarations parsed from include/pal_hip.h"
    for name in names:
        assert hasattr(lib, name), f"{name} declared in pal_hip.h but not exported"
    # the Python binding covers exactly the declared surface
    assert sorted(_lib.exported_symbols()) == names


def test_version_and_layout_helpers():
    lib = _lib.lib()
    assert lib.pal_version().decode().startswith("2025.06.4")
    assert lib.pal_get_optimal_page_size() == pal.get_optimal_page_size() == 16
    for dt, code in ((torch.float16, 0), (torch.bfloat16, 1)):
        assert lib.pal_get_k_cache_stripe_size(code) == pal.get_k_cache_stripe_size(dt) == 8
        shape = (ctypes.c_int64 * 5)()
        assert lib.pal_get_k_cache_shape(10, 4, 128, 16, code, shape) == 0
        assert tuple(shape) == pal.get_k_cache_shape(10, 4, 128, 16, dt) == (10, 4, 16, 16, 8)
        vshape = (ctypes.c_int64 * 4)()
        assert lib.pal_get_v_cache_shape(10, 4, 128, 16, code, vshape) == 0
        assert tuple(vshape) == pal.get_v_cache_shape(10, 4, 128, 16, dt) == (10, 4, 128, 16)
    assert lib.pal_get_k_cache_stripe_size(7) == _lib.PAL_ERR_INVALID_ARGUMENT
    assert "dtype" in _lib.last_error()


def test_fill_rejects_bad_arguments_without_launch():
    lib = _lib.lib()
    # head_dim not a multiple of 8 -> invalid argument, nothing launched
    st = lib.pal_fill_kv_pages(None, None, None, None, None, None, None, 1, 4, 2, 12, 16, 8, 1, 1, None)
    assert st == _lib.PAL_ERR_INVALID_ARGUMENT and "multiple of 8" in _lib.last_error()
    # zero tokens is a no-op
    assert lib.pal_fill_kv_pages(None, None, None, None, None, None, None, 1, 0, 2, 64, 16, 8, 1, 1, None) == 0
    # fp8 pools only at head dims an fp8 attention kernel reads (64, 128, 256)
    for hd in (16, 48, 80, 96, 192):
        st = lib.pal_fill_kv_pages_fp8(None, None, 1, None, None, None, None, None, None, None, 4, 2, hd, 16, 8, 1, 1,
                                       None)
        assert st == _lib.PAL_ERR_INVALID_ARGUMENT and "no attention kernel" in _lib.last_error()
    with pytest.raises(ValueError):
        _lib.check(_lib.PAL_ERR_INVALID_ARGUMENT)


def test_decode_rejects_bad_arguments_without_launch():
    lib = _lib.lib()
    args = dict(dtype=1, rows=4, seqs=4, hq=6, hkv=4, hd=128, tpp=16, pages=8, width=4, part=0)

    def call(**over):
        a = {**args, **over}
        return lib.pal_paged_attention_decode(None, None, None, None, None, None, a["dtype"], a["rows"], a["seqs"],
                                              a["hq"], a["hkv"], a["hd"], a["tpp"], a["pages"], a["width"],
                                              a["part"], None, 0, None)

    assert call() == _lib.PAL_ERR_RUNTIME and "divisible" in _lib.last_error()  # Hq % Hkv
    assert call(hq=8, hd=48) == _lib.PAL_ERR_RUNTIME  # no kernel for head_dim 48
    assert call(hq=8, tpp=8) == _lib.PAL_ERR_RUNTIME  # no kernel for TPP 8
    assert call(hq=8, part=100) == _lib.PAL_ERR_INVALID_ARGUMENT
    assert call(hq=8, rows=2) == _lib.PAL_ERR_INVALID_ARGUMENT  # fewer query rows than sequences
    assert call(hq=8, dtype=9) == _lib.PAL_ERR_INVALID_ARGUMENT
    with pytest.raises(RuntimeError):
        _lib.check(_lib.PAL_ERR_RUNTIME)


def test_decode_workspace_size_rejects_bad_arguments():
    lib = _lib.lib()
    # unsupported arguments report 0 bytes (no device is touched for them)
    assert lib.pal_paged_attention_decode_workspace_size(5, 64, 32, 8, 128, 16, 256, 0) == 0  # dtype
    assert lib.pal_paged_attention_decode_workspace_size(1, 64, 30, 8, 128, 16, 256, 0) == 0  # Hq % Hkv
    assert lib.pal_paged_attention_decode_workspace_size(1, 64, 32, 8, 48, 16, 256, 0) == 0  # head_dim
    assert lib.pal_paged_attention_decode_workspace_size(1, 64, 32, 8, 128, 16, 256, 100) == 0  # partition


def test_ops_reject_host_tensors_and_bad_ranks():
    q = torch.zeros(2, 4, 64, dtype=torch.bfloat16)
    k = torch.zeros(3, 1, 8, 16, 8, dtype=torch.bfloat16)
    v = torch.zeros(3, 1, 64, 16, dtype=torch.bfloat16)
    pt = torch.zeros(2, 1, dtype=torch.int32)
    lens = torch.ones(2, dtype=torch.int32)
    with pytest.raises(ValueError, match="HIP device"):
        pal.paged_attention_decode(q, k, v, pt, lens)
    with pytest.raises(ValueError, match="5D"):
        pal.fill_kv_pages(q, q, v, v, pt, lens, lens)
    with pytest.raises(ValueError, match="4D"):
        pal.fill_kv_pages(q, q, k, k, pt, lens, lens)


def test_prefill_rejects_bad_arguments_without_launch():
    lib = _lib.lib()
    args = dict(dtype=1, rows=8, seqs=2, hq=8, hkv=2, hd=128, tpp=16, pages=8, width=4)

    def call(**over):
        a = {**args, **over}
        return lib.pal_paged_attention_prefill(None, None, None, None, None, None, None, None, a["dtype"], a["rows"],
                                               a["seqs"], a["hq"], a["hkv"], a["hd"], a["tpp"], a["pages"],
                                               a["width"], None)

    assert call(hq=6, hkv=4) == _lib.PAL_ERR_RUNTIME and "divisible" in _lib.last_error()
    assert call(hd=80) == _lib.PAL_ERR_RUNTIME and "32" in _lib.last_error()  # prefill_primitive.cpp:91-93
    assert call(hd=160) == _lib.PAL_ERR_RUNTIME  # no kernel
    # any page size that is a multiple of 8 (up to 1024) passes the checks
    # (here it then stops at the null pointers); others have no kernel
    for tpp in (8, 24, 56, 64, 1024):
        assert call(tpp=tpp) == _lib.PAL_ERR_INVALID_ARGUMENT and "null" in _lib.last_error()
    for tpp in (4, 12, 20, 1032):
        assert call(tpp=tpp) == _lib.PAL_ERR_RUNTIME and "multiples of 8" in _lib.last_error()
    assert call(dtype=7) == _lib.PAL_ERR_INVALID_ARGUMENT
    assert call() == _lib.PAL_ERR_INVALID_ARGUMENT and "null" in _lib.last_error()
    assert call(seqs=0) == 0  # nothing to do
    assert call(rows=1, seqs=2) == 0  # prompt length 0


def test_fused_rejects_bad_arguments_without_launch():
    lib = _lib.lib()
    args = dict(dtype=0, rows=8, seqs=2, hq=8, hkv=2, hd=128, tpp=16, pages=8, width=4)

    def call(**over):
        a = {**args, **over}
        return lib.pal_paged_attention(None, None, None, None, None, None, None, None, a["dtype"], a["rows"],
                                       a["seqs"], a["hq"], a["hkv"], a["hd"], a["tpp"], a["pages"], a["width"],
                                       None, 0, None)

    assert call(hq=6, hkv=4) == _lib.PAL_ERR_RUNTIME
    assert call(hd=80) == _lib.PAL_ERR_RUNTIME
    assert call(tpp=64) == _lib.PAL_ERR_RUNTIME
    assert call(dtype=3) == _lib.PAL_ERR_INVALID_ARGUMENT
    assert call(rows=-1) == _lib.PAL_ERR_INVALID_ARGUMENT
    assert call() == _lib.PAL_ERR_INVALID_ARGUMENT and "null" in _lib.last_error()
    assert call(rows=0) == 0
    assert lib.pal_paged_attention_workspace_size(1, 64, 30, 8, 128, 16) == 0  # Hq % Hkv
    assert lib.pal_paged_attention_workspace_size(1, 64, 32, 8, 80, 16) == 0  # head_dim
    assert lib.pal_paged_attention_workspace_size(1, 0, 32, 8, 128, 16) == 0  # no rows


def test_new_ops_reject_host_tensors_and_shapes():
    q = torch.zeros(4, 4, 64, dtype=torch.float16)
    k = torch.zeros(3, 1, 8, 16, 8, dtype=torch.float16)
    v = torch.zeros(3, 1, 64, 16, dtype=torch.float16)
    kd = torch.zeros(4, 1, 64, dtype=torch.float16)
    pt = torch.zeros(2, 1, dtype=torch.int32)
    lens = torch.ones(2, dtype=torch.int32)
    rows = torch.zeros(4, dtype=torch.int32)
    with pytest.raises(ValueError, match="HIP device"):
        pal.paged_attention_prefill(q, kd, kd, k, v, pt, lens)
    with pytest.raises(ValueError, match="HIP device"):
        pal.paged_attention(q, k, v, pt, lens, rows, rows)
