"""Pool-layout helpers.

Reference: get_k_cache_stripe_size (bindings.cpp:44-48, ops.py:33-39),
get_k_cache_shape / get_v_cache_shape
(paged_attention_decode_primitive.cpp:373-397, bindings.cpp:50-64) and
get_optimal_page_size (constants.hpp:7-11).  The shape arithmetic is plain
integer math and is answered in Python; the C ABI exports the same helpers
for non-Python callers.

  K pool: [num_pages, num_kv_heads, head_dim / x, tokens_per_page, x]
  V pool: [num_pages, num_kv_heads, head_dim, tokens_per_page]
  x = 16 / sizeof(element)  (16-byte stripes; 8 for fp16 / bf16, 16 for fp8)
"""

from __future__ import annotations

import torch

from . import _lib

MEMORY_ALIGNMENT_BYTES = 16  # include/kernels/paged_attention_types.h:37
PAGE_SIZE = 16  # include/pal_core/constants.hpp:7

_DTYPE_CODES = {torch.float16: _lib.DTYPE_FLOAT16, torch.bfloat16: _lib.DTYPE_BFLOAT16}
FP8_DTYPE = torch.float8_e4m3fn  # fp8 KV pages (OCP e4m3: max 448, no infinities)
_POOL_CODES = {**_DTYPE_CODES, FP8_DTYPE: _lib.DTYPE_FP8_E4M3}
_SOURCE_CODES = {**_DTYPE_CODES, torch.float32: _lib.DTYPE_FLOAT32}


def dtype_code(dtype: torch.dtype) -> int:
    """C-ABI dtype code of queries / outputs; the attention kernels compute
    in float16 and bfloat16 (paged_attention_kernels.metal:41-42,111-130,
    142-214)."""
    try:
        return _DTYPE_CODES[dtype]
    except KeyError:
        raise RuntimeError(f"no paged-attention kernel for dtype {dtype} (float16 and bfloat16 only)") from None


def pool_dtype_code(dtype: torch.dtype) -> int:
    """C-ABI code of a KV pool dtype: float16, bfloat16 or fp8 e4m3
    (torch.float8_e4m3fn, with per-(page, kv head) scales)."""
    try:
        return _POOL_CODES[dtype]
    except KeyError:
        raise RuntimeError(f"no KV pool of dtype {dtype} (float16, bfloat16, float8_e4m3fn)") from None


def source_dtype_code(dtype: torch.dtype) -> int:
    """C-ABI code of new K/V rows written by fill_kv_pages: float16, bfloat16
    or float32 (cast to the pool dtype on the way)."""
    try:
        return _SOURCE_CODES[dtype]
    except KeyError:
        raise ValueError(f"new keys/values of dtype {dtype} (float16, bfloat16, float32 supported)") from None


def get_k_cache_stripe_size(dtype: torch.dtype) -> int:
    """Elements per 16-byte K stripe: 16 / sizeof(dtype) (16 for fp8)."""
    return MEMORY_ALIGNMENT_BYTES // torch.empty((), dtype=dtype).element_size()


def get_optimal_page_size() -> int:
    """Tokens per page the kernels are tuned for (16)."""
    return PAGE_SIZE


def get_k_cache_shape(num_total_pages: int, num_kv_heads: int, head_dim: int, tokens_per_page: int,
                      dtype: torch.dtype) -> tuple[int, int, int, int, int]:
    x = get_k_cache_stripe_size(dtype)
    return (int(num_total_pages), int(num_kv_heads), int(head_dim) // x, int(tokens_per_page), x)


def get_v_cache_shape(num_total_pages: int, num_kv_heads: int, head_dim: int, tokens_per_page: int,
                      dtype: torch.dtype) -> tuple[int, int, int, int]:
    return (int(num_total_pages), int(num_kv_heads), int(head_dim), int(tokens_per_page))
