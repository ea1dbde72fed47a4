"""Proxy Attention Lab paged-attention operators for AMD MI355X (gfx950).

Same public names as the reference package (src/proxy_attention_lab/
__init__.py:17-37), over torch tensors, backed by hand-written HIP kernels
in libpal_hip.so.  ``paged_attention`` (fused mixed batch) is an addition.
"""

from proxy_attention_lab.layout import (
    get_k_cache_shape,
    get_k_cache_stripe_size,
    get_optimal_page_size,
    get_v_cache_shape,
)
from proxy_attention_lab.layout import FP8_DTYPE
from proxy_attention_lab.page_pool import PagePool
from proxy_attention_lab.ops import (
    fill_kv_pages,
    paged_attention,
    paged_attention_decode,
    paged_attention_prefill,
    release_workspaces,
    rope_cos_sin_cache,
    rope_fill_kv_pages,
)

__version__ = "2025.06.4+gfx950"

__all__ = [
    "fill_kv_pages",
    "get_k_cache_shape",
    "get_k_cache_stripe_size",
    "get_optimal_page_size",
    "get_v_cache_shape",
    "paged_attention",
    "paged_attention_decode",
    "paged_attention_prefill",
    "release_workspaces",
    "rope_cos_sin_cache",
    "rope_fill_kv_pages",
    "FP8_DTYPE",
    "PagePool",
]
