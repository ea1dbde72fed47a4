"""Page-pool allocator and compaction for the paged K/V pools.

The reference takes page tables from its caller and keeps no allocator
(src/proxy_attention_lab/ops.py:61-63).  ``PagePool`` is the allocator an
engine keeps beside the pools: it hands out page ids lowest-first, takes
them back, and compacts the pools so the live pages become ids
[0, live) -- the moves run on the GPU (whole-page copies of both pools and,
for fp8 pools, their scale rows) and the page tables are rewritten in place.
The bookkeeping is the native allocator in libpal_hip.so
(``pal_page_pool_*``); this class owns one such pool.
"""

from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _lib

__all__ = ["PagePool"]


class PagePool:
    """Free-list allocator of ``num_pages`` page ids.

    ``allocate(n)`` returns the n lowest free ids (uint32 numpy array) or
    raises RuntimeError when fewer are free (nothing is allocated then);
    ``free(ids)`` raises ValueError for an id out of range, not allocated or
    listed twice (nothing is freed then).  ``compact(...)`` moves the live
    pages to ids [0, live) and rewrites the given page tables.
    """

    def __init__(self, num_pages: int):
        self._lib = _lib.lib()
        handle = ctypes.c_void_p()
        _lib.check(self._lib.pal_page_pool_create(int(num_pages), ctypes.byref(handle)))
        self._h = handle
        self.num_pages = int(num_pages)

    def close(self) -> None:
        if getattr(self, "_h", None) is not None and self._h.value:
            self._lib.pal_page_pool_destroy(self._h)
            self._h = None

    def __del__(self):  # pragma: no cover - interpreter shutdown order
        try:
            self.close()
        except Exception:
            pass

    @property
    def num_free(self) -> int:
        n = self._lib.pal_page_pool_num_free(self._h)
        if n < 0:
            _lib.check(int(n))
        return int(n)

    @property
    def num_used(self) -> int:
        return self.num_pages - self.num_free

    def allocate(self, n: int) -> np.ndarray:
        out = np.zeros(max(int(n), 0), np.uint32)
        _lib.check(self._lib.pal_page_pool_alloc(self._h, int(n), out.ctypes.data if n > 0 else None))
        return out

    def free(self, ids) -> None:
        arr = np.ascontiguousarray(np.asarray(ids).reshape(-1), dtype=np.uint32)
        _lib.check(self._lib.pal_page_pool_free(self._h, arr.ctypes.data if arr.size else None, int(arr.size)))

    def compaction_plan(self) -> tuple[np.ndarray, np.ndarray]:
        """Plan (and record in the allocator) the moves that make the live
        ids [0, live): returns (src, dst) uint32 arrays; the data must then be
        moved with ``apply_moves`` and the page tables rewritten."""
        n = ctypes.c_int64(0)
        _lib.check(self._lib.pal_page_pool_compaction_plan(self._h, None, None, 0, ctypes.byref(n)))
        src = np.zeros(n.value, np.uint32)
        dst = np.zeros(n.value, np.uint32)
        if n.value:
            _lib.check(self._lib.pal_page_pool_compaction_plan(self._h, src.ctypes.data, dst.ctypes.data, n.value,
                                                               ctypes.byref(n)))
        return src, dst

    @staticmethod
    def _check_targets(k_pool: torch.Tensor, v_pool: torch.Tensor, page_tables, k_scales, v_scales) -> None:
        """Everything a compaction writes, checked before anything is planned
        or launched: a rejected call leaves the allocator, the pools and the
        page tables as they were."""
        for name, t in (("k_pool", k_pool), ("v_pool", v_pool)):
            if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
                raise ValueError(f"[compact] {name} must be a tensor on a HIP device")
        device = k_pool.device
        for name, t in (("k_pool", k_pool), ("v_pool", v_pool)):
            if not t.is_contiguous() or t.device != device or t.dim() < 2:
                raise ValueError(f"[compact] {name} must be contiguous on {device}")
        num_pages, hkv = int(k_pool.shape[0]), int(k_pool.shape[1])
        page_bytes = k_pool[0].numel() * k_pool.element_size()
        if v_pool[0].numel() * v_pool.element_size() != page_bytes or int(v_pool.shape[0]) != num_pages:
            raise ValueError("[compact] K and V pools must hold the same pages of the same size")
        if (k_scales is None) != (v_scales is None):
            raise ValueError("[compact] give both k_scales and v_scales, or neither")
        for name, t in (("k_scales", k_scales), ("v_scales", v_scales)):
            if t is not None and (not isinstance(t, torch.Tensor) or t.dtype != torch.float32 or
                                  tuple(t.shape) != (num_pages, hkv) or not t.is_contiguous() or t.device != device):
                raise ValueError(f"[compact] {name} must be contiguous float32 [{num_pages}, {hkv}] on {device}")
        for pt in page_tables:
            # rewritten in place by the kernel, so only 32-bit tables qualify
            # (an int64 table would need a copy the caller never sees)
            if not isinstance(pt, torch.Tensor) or pt.dtype not in (torch.int32, torch.uint32) or \
                    not pt.is_contiguous() or pt.device != device:
                raise ValueError("[compact] page tables must be contiguous int32 / uint32 device tensors")

    @staticmethod
    def apply_moves(src: np.ndarray, dst: np.ndarray, k_pool: torch.Tensor, v_pool: torch.Tensor,
                    page_tables=(), k_scales: torch.Tensor | None = None, v_scales: torch.Tensor | None = None,
                    stream=None) -> None:
        """Copy pages src[m] -> dst[m] of both pools (and fp8 scale rows) on
        the GPU, then rewrite every page table in ``page_tables`` (uint32 /
        int32 device tensors, updated in place) through the same map.  Every
        argument is checked before the first launch."""
        from .ops import _launch_stream, _on_stream

        page_tables = tuple(page_tables)
        PagePool._check_targets(k_pool, v_pool, page_tables, k_scales, v_scales)
        device = k_pool.device
        num_pages = int(k_pool.shape[0])
        page_bytes = k_pool[0].numel() * k_pool.element_size()
        src = np.ascontiguousarray(src, np.uint32)
        dst = np.ascontiguousarray(dst, np.uint32)
        if src.shape != dst.shape or len(np.intersect1d(src, dst)):
            raise ValueError("[compact] move sources and destinations must be disjoint lists of one length")
        if src.size == 0:
            return
        hkv = int(k_pool.shape[1])
        remap = np.arange(num_pages, dtype=np.uint32)
        remap[src[src < num_pages]] = dst[src < num_pages]
        L = _lib.lib()
        sh, sh_current = _launch_stream(stream, device)
        with _on_stream(sh, device, sh_current):
            s_d = torch.from_numpy(src.view(np.int32)).to(device, non_blocking=False)
            d_d = torch.from_numpy(dst.view(np.int32)).to(device, non_blocking=False)
            r_d = torch.from_numpy(remap.view(np.int32)).to(device, non_blocking=False)
            _lib.check(L.pal_copy_pages(k_pool.data_ptr(), v_pool.data_ptr(),
                                        k_scales.data_ptr() if k_scales is not None else None,
                                        v_scales.data_ptr() if v_scales is not None else None,
                                        num_pages, hkv, page_bytes, s_d.data_ptr(), d_d.data_ptr(), int(src.size), sh))
            for pt in page_tables:
                _lib.check(L.pal_remap_pages(pt.data_ptr(), pt.numel(), r_d.data_ptr(), num_pages, sh))

    def compact(self, k_pool: torch.Tensor, v_pool: torch.Tensor, page_tables=(),
                k_scales: torch.Tensor | None = None, v_scales: torch.Tensor | None = None, stream=None) -> int:
        """Compaction in one call: plan, move the pages, rewrite the page
        tables.  Returns the number of pages moved.  The pools, scales and
        page tables are checked first (and the pools must hold this
        allocator's ``num_pages``): a ValueError leaves the allocator and
        every tensor unchanged."""
        page_tables = tuple(page_tables)
        self._check_targets(k_pool, v_pool, page_tables, k_scales, v_scales)
        if int(k_pool.shape[0]) != self.num_pages:
            raise ValueError(f"[compact] the pools hold {int(k_pool.shape[0])} pages, the allocator {self.num_pages}")
        src, dst = self.compaction_plan()
        self.apply_moves(src, dst, k_pool, v_pool, page_tables, k_scales, v_scales, stream)
        return int(src.size)
