"""Paged-attention operators over torch tensors on an MI355X (gfx950) device.

Drop-in counterparts of the reference's ``proxy_attention_lab.ops``
(src/proxy_attention_lab/ops.py:33-171): same function names, the same
positional arguments in the same order and the same output shapes, with
``torch.Tensor`` in place of ``mlx.core.array``.  Every operator runs on the
HIP library libpal_hip.so through its C ABI; there is no CPU path.

Differences from the reference, all deliberate:
  * ``fill_kv_pages`` updates the pools in place and returns the same tensor
    objects (the reference copies both whole pools on every call,
    fill_kv_pages_primitive.cpp:91-92).  ``copy=True`` restores the
    functional behaviour.
  * ``stream`` takes ``None`` (current torch stream), a ``torch.cuda.Stream``
    or a raw ``hipStream_t`` integer.
  * ``paged_attention`` (fused mixed batch) is an addition; the reference has
    no such function.
"""

from __future__ import annotations

import collections
import contextlib

import torch

from . import _lib
from .layout import (  # noqa: F401  (get_k_cache_stripe_size re-exported)
    FP8_DTYPE,
    dtype_code,
    get_k_cache_stripe_size,
    pool_dtype_code,
    source_dtype_code,
)

__all__ = [
    "fill_kv_pages",
    "get_k_cache_stripe_size",
    "rope_cos_sin_cache",
    "rope_fill_kv_pages",
    "paged_attention",
    "paged_attention_decode",
    "paged_attention_prefill",
    "release_workspaces",
]


# ---------------------------------------------------------------------------
# argument plumbing
# ---------------------------------------------------------------------------


def _stream_handle(stream, device: torch.device) -> int:
    if stream is None:
        return torch.cuda.current_stream(device).cuda_stream
    if isinstance(stream, torch.cuda.Stream):
        return stream.cuda_stream
    if isinstance(stream, int):
        return stream
    raise TypeError(f"stream must be None, a torch.cuda.Stream or an int handle, got {type(stream)!r}")


def _launch_stream(stream, device: torch.device) -> tuple[int, bool]:
    """The launch stream's handle, and whether it is torch's current stream
    (always so for the default ``stream=None``, which then needs no second
    query in ``_on_stream``)."""
    if stream is None:
        return torch.cuda.current_stream(device).cuda_stream, True
    return _stream_handle(stream, device), False


def _on_stream(stream_handle: int, device: torch.device, current: bool = False):
    """Context in which torch work (index conversions, contiguous copies,
    output and workspace allocation) is ordered on the launch stream.

    The kernels run on ``stream_handle``; any temporary the call makes must
    be written on that same stream, and the caching allocator must see it as
    that stream's memory, or a kernel could read a half-written buffer or a
    block freed and reused by another stream.  When the launch stream is
    torch's current stream this is a no-op.
    """
    if current or stream_handle == torch.cuda.current_stream(device).cuda_stream:
        return contextlib.nullcontext()
    return torch.cuda.stream(torch.cuda.ExternalStream(stream_handle, device=device))


def _require_device(name: str, t: torch.Tensor, device: torch.device | None = None) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor, got {type(t)!r}")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must live on a HIP device (got {t.device})")
    if device is not None and t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")


def _index_tensor(name: str, t: torch.Tensor, device: torch.device) -> torch.Tensor:
    """Return a contiguous 32-bit view/copy of an index tensor (u32/i32 bits)."""
    _require_device(name, t, device)
    if t.dtype in (torch.int32,):
        return t.contiguous()
    if t.dtype == torch.uint32:
        return t.contiguous().view(torch.int32)
    if t.dtype in (torch.int64, torch.int16, torch.uint8, torch.int8):
        return t.to(torch.int32).contiguous()
    raise ValueError(f"{name} must be an integer tensor, got {t.dtype}")


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


_WORKSPACES: "collections.OrderedDict[tuple[str, int, int], torch.Tensor]" = collections.OrderedDict()
_WORKSPACES_PER_DEVICE = 4  # streams whose workspaces are kept per (operator, device), most recent first


def _workspace(kind: str, nbytes: int, device: torch.device, stream_handle: int) -> torch.Tensor | None:
    """Zero-initialised workspace per (operator, device, stream), kept for the
    streams used most recently.

    The decode kernels keep a work-claim counter in it that must read zero
    when a call starts; every call leaves it zero again, so the buffer is
    reused as is by the next call of the same operator on the same stream
    (calls on one stream never overlap).  A larger request replaces it with a
    new zeroed buffer.  At most ``_WORKSPACES_PER_DEVICE`` streams keep one
    per (operator, device); the least recently used is dropped beyond that.
    Dropping is safe while kernels on that stream still read it: the
    buffer was allocated on that stream, so torch's caching allocator
    hands its memory out again only to later work of the same stream.
    ``release_workspaces`` drops them all.
    """
    if nbytes <= 0:
        return None
    dev_index = device.index if device.index is not None else torch.cuda.current_device()
    key = (kind, dev_index, stream_handle)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        # allocated and zero-filled on the launch stream (the caller holds
        # _on_stream), so the buffer it replaces, still in use by kernels
        # queued on that stream, is only reused after them
        ws = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    _WORKSPACES.move_to_end(key)
    same = [k for k in _WORKSPACES if k[0] == kind and k[1] == dev_index]
    for k in same[:-_WORKSPACES_PER_DEVICE]:
        del _WORKSPACES[k]
    return ws


def release_workspaces(device: torch.device | int | None = None) -> int:
    """Drop the operators' cached workspaces (of one device, or all); returns
    how many were dropped.  Their memory goes back to torch's caching
    allocator (``torch.cuda.empty_cache`` returns it to the device).  The
    next call on a stream allocates a fresh zeroed workspace."""
    if device is not None:
        device = torch.device("cuda", device) if isinstance(device, int) else torch.device(device)
    idx = None if device is None else (device.index if device.index is not None else torch.cuda.current_device())
    drop = [k for k in _WORKSPACES if idx is None or k[1] == idx]
    for k in drop:
        del _WORKSPACES[k]
    return len(drop)


def _pools(op: str, k_pool: torch.Tensor, v_pool: torch.Tensor, device: torch.device, dtype: torch.dtype):
    """Validate the paged pools; return (num_pages, Hkv, HD, TPP).  Pools hold
    the query dtype, or fp8 e4m3 (torch.float8_e4m3fn, K stripe of 16)."""
    for name, t in (("k_cache_pool", k_pool), ("v_cache_pool", v_pool)):
        _require_device(name, t, device)
    if v_pool.dim() != 4:
        raise ValueError(f"[{op}] v_cache_pool must be 4D [pages, kv_heads, head_dim, tokens_per_page]")
    if k_pool.dim() != 5:
        raise ValueError(f"[{op}] k_cache_pool must be 5D [pages, kv_heads, head_dim/x, tokens_per_page, x]")
    num_pages, num_kv_heads, head_dim, tpp = (int(x) for x in v_pool.shape)
    if k_pool.dtype != v_pool.dtype or k_pool.dtype not in (dtype, FP8_DTYPE):
        raise ValueError(f"[{op}] pools must share one dtype: the queries' or float8_e4m3fn")
    x = get_k_cache_stripe_size(k_pool.dtype)
    expect_k = (num_pages, num_kv_heads, head_dim // x, tpp, x)
    if tuple(k_pool.shape) != expect_k:
        raise ValueError(f"[{op}] k_cache_pool shape {tuple(k_pool.shape)} != {expect_k}")
    return num_pages, num_kv_heads, head_dim, tpp


def _scales(op: str, k_pool: torch.Tensor, k_scales, v_scales, num_pages: int, num_kv_heads: int,
            device: torch.device):
    """(k_scales, v_scales) for fp8 pools (validated), (None, None) for
    16-bit pools (where giving scales is an error)."""
    if k_pool.dtype != FP8_DTYPE:
        if k_scales is not None or v_scales is not None:
            raise ValueError(f"[{op}] k_scales / v_scales apply to fp8 pools only")
        return None, None
    for name, t in (("k_scales", k_scales), ("v_scales", v_scales)):
        if t is None:
            raise ValueError(f"[{op}] fp8 pools need k_scales and v_scales ([num_pages, num_kv_heads] float32)")
        _require_device(name, t, device)
        if t.dtype != torch.float32 or tuple(t.shape) != (num_pages, num_kv_heads):
            raise ValueError(f"[{op}] {name} must be float32 [{num_pages}, {num_kv_heads}]")
    return k_scales, v_scales


def _query_dims(op: str, queries: torch.Tensor, head_dim: int):
    """(rows, Hq) of 3-D [N, Hq, HD] or 2-D [N, HD] (one head) queries."""
    if queries.dim() == 3:
        num_rows, num_q_heads, q_hd = (int(x) for x in queries.shape)
    elif queries.dim() == 2:
        num_rows, q_hd = (int(x) for x in queries.shape)
        num_q_heads = 1
    else:
        raise ValueError(f"[{op}] queries must be 2D [N, HD] or 3D [N, Hq, HD]")
    if q_hd != head_dim:
        raise ValueError(f"[{op}] query head_dim {q_hd} != cache head_dim {head_dim}")
    return num_rows, num_q_heads


# ---------------------------------------------------------------------------
# operators
# ---------------------------------------------------------------------------


def paged_attention_decode(
    queries: torch.Tensor,
    k_cache_pool: torch.Tensor,
    v_cache_pool: torch.Tensor,
    page_table: torch.Tensor,
    sequence_lengths: torch.Tensor,
    stream=None,
    *,
    partition_size: int = 0,
    k_scales: torch.Tensor | None = None,
    v_scales: torch.Tensor | None = None,
) -> torch.Tensor:
    """Decode attention: one query row per sequence over its paged context.

    Reference: ops.py:42-84 -> bindings.cpp:125-180 -> ops.cpp:36-108 ->
    paged_attention_decode_primitive.cpp:71-266.

    queries: [N, Hq, HD] (or [N, HD], meaning one query head); row s is the
    query of sequence s and rows >= num_seqs are ignored.
    k_cache_pool: [P, Hkv, HD/x, TPP, x]; v_cache_pool: [P, Hkv, HD, TPP].
    page_table: [S, W] uint32/int32; sequence_lengths: [S] int32.
    Returns [S, Hq, HD] in the query dtype (decode_primitive.cpp:289-300;
    the "[N*Hq, HD]" in the reference docstring does not match its code).
    ``partition_size`` (keyword-only): 0 shares the KV blocks of the batch
    out to the workers the GPU keeps resident, one equal share each; 128, 256
    or 512 splits the KV stream into fixed chunks of that many tokens instead
    (each worker streams an equal run of consecutive chunks, every chunk its
    own partial); partials are merged by log-sum-exp as in the reference's
    two-pass mode.  fp8 pools (torch.float8_e4m3fn, an addition) need
    ``k_scales`` / ``v_scales`` (float32 [num_pages, Hkv]): a key or value
    is its code times the scale of its (page, kv head); head_dim 64, 128 or
    256.
    """
    op = "paged_attention_decode"
    _require_device("queries", queries)
    device = queries.device
    code = dtype_code(queries.dtype)
    num_pages, num_kv_heads, head_dim, tpp = _pools(op, k_cache_pool, v_cache_pool, device, queries.dtype)
    num_rows, num_q_heads = _query_dims(op, queries, head_dim)
    ks, vs = _scales(op, k_cache_pool, k_scales, v_scales, num_pages, num_kv_heads, device)
    if page_table.dim() != 2:
        raise ValueError("[paged_attention_decode] page_table must be 2D [num_seqs, max_pages_per_seq]")
    num_seqs, width = (int(x) for x in page_table.shape)
    _require_device("sequence_lengths", sequence_lengths, device)
    if sequence_lengths.numel() < num_seqs:
        raise ValueError(
            f"[paged_attention_decode] {sequence_lengths.numel()} sequence lengths for {num_seqs} sequences")
    L = _lib.lib()
    sh, sh_current = _launch_stream(stream, device)
    with _on_stream(sh, device, sh_current):
        pt = _index_tensor("page_table", page_table, device)
        lens = _index_tensor("sequence_lengths", sequence_lengths, device)
        q = queries.contiguous()
        kp = k_cache_pool.contiguous()
        vp = v_cache_pool.contiguous()
        out = torch.empty((num_seqs, num_q_heads, head_dim), dtype=queries.dtype, device=device)
        ws = None
        fp8 = ks is not None
        if num_seqs > 0:
            size_fn = L.pal_paged_attention_decode_fp8_workspace_size if fp8 else \
                L.pal_paged_attention_decode_workspace_size
            with torch.cuda.device(device):
                ws_bytes = size_fn(code, num_seqs, num_q_heads, num_kv_heads, head_dim, tpp, width,
                                   int(partition_size))
            ws = _workspace("decode", ws_bytes, device, sh)
        if fp8:
            status = L.pal_paged_attention_decode_fp8(
                _ptr(q), _ptr(kp), _ptr(vp), _ptr(ks.contiguous()), _ptr(vs.contiguous()), _ptr(pt), _ptr(lens),
                _ptr(out), code, num_rows, num_seqs, num_q_heads, num_kv_heads, head_dim, tpp, num_pages, width,
                int(partition_size), _ptr(ws), ws.numel() if ws is not None else 0, sh)
        else:
            status = L.pal_paged_attention_decode(
                _ptr(q), _ptr(kp), _ptr(vp), _ptr(pt), _ptr(lens), _ptr(out),
                code, num_rows, num_seqs, num_q_heads, num_kv_heads, head_dim, tpp,
                num_pages, width, int(partition_size),
                _ptr(ws), ws.numel() if ws is not None else 0, sh,
            )
    _lib.check(status)
    return out


def _fill_common(op: str, new_keys, new_values, k_pool, v_pool, page_table, write_positions, query_to_seq_map,
                 k_scales, v_scales):
    """Validation shared by fill_kv_pages and rope_fill_kv_pages; returns
    (device, num_tokens, num_pages, Hkv, HD, TPP, width, num_seqs, pool code,
    source code)."""
    # ops.cpp:204-211: the same rank checks, first, raised as ValueError.
    if k_pool.dim() != 5:
        raise ValueError(f"[{op}] global_key_pool must be 5D.")
    if v_pool.dim() != 4:
        raise ValueError(f"[{op}] global_value_pool must be 4D.")
    _require_device("new_keys", new_keys)
    device = new_keys.device
    for name, t in (("new_values", new_values), ("global_key_pool", k_pool), ("global_value_pool", v_pool)):
        _require_device(name, t, device)
    num_pages, num_kv_heads, head_dim, tpp = (int(x) for x in v_pool.shape)
    pool_code = pool_dtype_code(k_pool.dtype)
    if v_pool.dtype != k_pool.dtype:
        raise ValueError(f"[{op}] key and value pools must share one dtype")
    src_code = source_dtype_code(new_keys.dtype)
    if new_values.dtype != new_keys.dtype:
        raise ValueError(f"[{op}] new keys and values must share one dtype")
    x = get_k_cache_stripe_size(k_pool.dtype)
    expect_k = (num_pages, num_kv_heads, head_dim // x, tpp, x)
    if tuple(k_pool.shape) != expect_k:
        raise ValueError(f"[{op}] global_key_pool shape {tuple(k_pool.shape)} != {expect_k}")
    if not k_pool.is_contiguous() or not v_pool.is_contiguous():
        raise ValueError(f"[{op}] pools must be contiguous (they are updated in place)")
    if pool_code == _lib.DTYPE_FP8_E4M3:
        for name, t in (("k_scales", k_scales), ("v_scales", v_scales)):
            if t is None:
                raise ValueError(f"[{op}] fp8 pools need k_scales and v_scales ([num_pages, num_kv_heads] float32)")
            _require_device(name, t, device)
            if t.dtype != torch.float32 or tuple(t.shape) != (num_pages, num_kv_heads) or not t.is_contiguous():
                raise ValueError(f"[{op}] {name} must be contiguous float32 [{num_pages}, {num_kv_heads}]")
    n = int(new_keys.shape[0]) if new_keys.dim() > 0 else 0
    if n and (tuple(new_keys.shape) != (n, num_kv_heads, head_dim) or
              tuple(new_values.shape) != (n, num_kv_heads, head_dim)):
        raise ValueError(
            f"[{op}] new_keys/new_values must be [{n}, {num_kv_heads}, {head_dim}], got "
            f"{tuple(new_keys.shape)} / {tuple(new_values.shape)}"
        )
    if page_table.dim() != 2:
        raise ValueError(f"[{op}] page_table must be 2D")
    num_seqs, width = (int(x) for x in page_table.shape)
    if write_positions.numel() < n or query_to_seq_map.numel() < n:
        raise ValueError(f"[{op}] write positions and query_to_seq_map need one entry per new token")
    return device, n, num_pages, num_kv_heads, head_dim, tpp, width, num_seqs, pool_code, src_code


def fill_kv_pages(
    new_keys: torch.Tensor,
    new_values: torch.Tensor,
    global_key_pool: torch.Tensor,
    global_value_pool: torch.Tensor,
    page_table: torch.Tensor,
    current_token_write_positions: torch.Tensor,
    query_to_seq_map: torch.Tensor,
    stream=None,
    *,
    copy: bool = False,
    k_scales: torch.Tensor | None = None,
    v_scales: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Scatter new K/V rows into their page slots.

    Reference: ops.py:133-171 -> bindings.cpp:182-222 -> ops.cpp:188-239 ->
    fill_kv_pages_primitive.cpp:70-170 -> fill_kv_pages.h.metal:56-116.

    new_keys / new_values: [N, Hkv, HD]; pools as for decode;
    current_token_write_positions: [N] int32; query_to_seq_map: [N] uint32.
    Token t goes to page page_table[q2seq[t], pos // TPP], slot pos % TPP.
    With new rows in the pool dtype this is a bit-exact copy, as in the
    reference.  Additions: float32 rows (or 16-bit rows of the other
    dtype) are cast to the pool dtype (round to nearest even), and fp8 pools
    (torch.float8_e4m3fn, K stripe of 16) are written quantized with the
    keyword-only ``k_scales`` / ``v_scales`` (float32 [num_pages, Hkv]):
    q = x / scale held to [-448, 448], rounded to nearest even.
    Updates the pools in place and returns them; with ``copy=True`` the
    inputs are left untouched and fresh pools are returned, as in the
    reference.
    """
    op = "fill_kv_pages"
    device, n, num_pages, hkv, hd, tpp, width, num_seqs, pool_code, src_code = _fill_common(
        op, new_keys, new_values, global_key_pool, global_value_pool, page_table, current_token_write_positions,
        query_to_seq_map, k_scales, v_scales)
    sh, sh_current = _launch_stream(stream, device)
    if copy:
        with _on_stream(sh, device, sh_current):
            global_key_pool = global_key_pool.clone()
            global_value_pool = global_value_pool.clone()
    if n == 0 or new_keys.numel() == 0:
        return global_key_pool, global_value_pool
    L = _lib.lib()
    with _on_stream(sh, device, sh_current):
        pt = _index_tensor("page_table", page_table, device)
        pos = _index_tensor("current_token_write_positions", current_token_write_positions, device)
        q2s = _index_tensor("query_to_seq_map", query_to_seq_map, device)
        nk = new_keys.contiguous()
        nv = new_values.contiguous()
        if pool_code == _lib.DTYPE_FP8_E4M3:
            status = L.pal_fill_kv_pages_fp8(
                _ptr(nk), _ptr(nv), src_code, _ptr(global_key_pool), _ptr(global_value_pool), _ptr(k_scales),
                _ptr(v_scales), _ptr(pt), _ptr(pos), _ptr(q2s), n, hkv, hd, tpp, num_pages, num_seqs, width, sh)
        elif src_code == pool_code:
            status = L.pal_fill_kv_pages(
                _ptr(nk), _ptr(nv), _ptr(global_key_pool), _ptr(global_value_pool), _ptr(pt), _ptr(pos), _ptr(q2s),
                pool_code, n, hkv, hd, tpp, num_pages, num_seqs, width, sh)
        else:  # a cast on the way: the fused entry without rotation
            status = L.pal_rope_fill_kv_pages(
                _ptr(nk), _ptr(nv), src_code, _ptr(global_key_pool), _ptr(global_value_pool), pool_code, None, None,
                _ptr(pt), _ptr(pos), _ptr(q2s), n, hkv, hd, tpp, num_pages, num_seqs, width, None, 0, 0,
                _lib.ROPE_NONE, None, None, 0, _lib.DTYPE_BFLOAT16, sh)
    _lib.check(status)
    return global_key_pool, global_value_pool


_ROPE_STYLES = {"neox": _lib.ROPE_NEOX, "gptj": _lib.ROPE_GPTJ}
_COS_SIN: dict[tuple, torch.Tensor] = {}


def rope_cos_sin_cache(max_position: int, rotary_dim: int, base: float = 10000.0,
                       device: torch.device | str = "cuda") -> torch.Tensor:
    """The cos/sin table rope_fill_kv_pages reads: [max_position, rotary_dim]
    float32, cos(p w_f) for the rotary_dim / 2 frequencies w_f =
    base^(-2f / rotary_dim), then sin(p w_f), computed in float64 and rounded
    once.  Cached per (arguments, device)."""
    device = torch.device(device)
    key = (int(max_position), int(rotary_dim), float(base), str(device))
    t = _COS_SIN.get(key)
    if t is None:
        half = rotary_dim // 2
        inv_freq = float(base) ** (-(2.0 * torch.arange(half, dtype=torch.float64)) / rotary_dim)
        ang = torch.arange(max_position, dtype=torch.float64)[:, None] * inv_freq[None, :]
        t = torch.cat([torch.cos(ang), torch.sin(ang)], dim=1).to(torch.float32).to(device)
        _COS_SIN[key] = t
    return t


def rope_fill_kv_pages(
    new_keys: torch.Tensor,
    new_values: torch.Tensor,
    global_key_pool: torch.Tensor,
    global_value_pool: torch.Tensor,
    page_table: torch.Tensor,
    current_token_write_positions: torch.Tensor,
    query_to_seq_map: torch.Tensor,
    cos_sin_cache: torch.Tensor,
    stream=None,
    *,
    queries: torch.Tensor | None = None,
    rotary_dim: int | None = None,
    style: str = "neox",
    query_dtype: torch.dtype | None = None,
    k_scales: torch.Tensor | None = None,
    v_scales: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor | None]:
    """RoPE + cast + KV scatter in one pass: the step that produces
    fill_kv_pages' inputs from the QKV projection, fused with it (no
    reference counterpart; the scatter is fill_kv_pages', ops.py:133-171).

    new_keys / new_values: [N, Hkv, HD] float32, float16 or bfloat16 (the
    projection's output); the position of token t is
    current_token_write_positions[t].  K is rotated by row `pos` of
    ``cos_sin_cache`` ([rows, rotary_dim] float32, see rope_cos_sin_cache):
    style "neox" pairs dims (f, f + rotary_dim/2), "gptj" pairs (2f, 2f+1);
    dims past rotary_dim (default: the whole head) pass through.  K and V
    are then cast to the pool dtype (fp8 pools: with ``k_scales`` /
    ``v_scales``) and scattered like fill_kv_pages, in place.  ``queries``
    ([N, Hq, HD], same dtype as new_keys), if given, are rotated the same way
    and returned cast to ``query_dtype`` (default: the pool dtype, or
    bfloat16 for fp8 pools).  Tokens whose position has no row in the table
    are not written to the pools; their queries are cast unrotated.
    Returns (key_pool, value_pool, rotated queries or None).
    """
    op = "rope_fill_kv_pages"
    device, n, num_pages, hkv, hd, tpp, width, num_seqs, pool_code, src_code = _fill_common(
        op, new_keys, new_values, global_key_pool, global_value_pool, page_table, current_token_write_positions,
        query_to_seq_map, k_scales, v_scales)
    if style not in _ROPE_STYLES:
        raise ValueError(f"[{op}] style must be 'neox' or 'gptj', got {style!r}")
    rot = hd if rotary_dim is None else int(rotary_dim)
    _require_device("cos_sin_cache", cos_sin_cache, device)
    if cos_sin_cache.dim() != 2 or int(cos_sin_cache.shape[1]) != rot or cos_sin_cache.dtype != torch.float32:
        raise ValueError(f"[{op}] cos_sin_cache must be float32 [rows, {rot}]")
    q_out = None
    hq = 0
    if queries is not None:
        _require_device("queries", queries, device)
        if queries.dtype != new_keys.dtype or queries.dim() != 3 or int(queries.shape[0]) != n or \
                int(queries.shape[2]) != hd:
            raise ValueError(f"[{op}] queries must be [{n}, Hq, {hd}] in the dtype of new_keys")
        hq = int(queries.shape[1])
        if query_dtype is None:
            query_dtype = global_key_pool.dtype if pool_code != _lib.DTYPE_FP8_E4M3 else torch.bfloat16
        q_code = dtype_code(query_dtype)
    else:
        q_code = _lib.DTYPE_BFLOAT16
    sh, sh_current = _launch_stream(stream, device)
    with _on_stream(sh, device, sh_current):
        if queries is not None:
            q_out = torch.empty((n, hq, hd), dtype=query_dtype, device=device)
        if n == 0:
            return global_key_pool, global_value_pool, q_out
        pt = _index_tensor("page_table", page_table, device)
        pos = _index_tensor("current_token_write_positions", current_token_write_positions, device)
        q2s = _index_tensor("query_to_seq_map", query_to_seq_map, device)
        nk = new_keys.contiguous()
        nv = new_values.contiguous()
        cs = cos_sin_cache.contiguous()
        qi = queries.contiguous() if queries is not None else None
        status = _lib.lib().pal_rope_fill_kv_pages(
            _ptr(nk), _ptr(nv), src_code, _ptr(global_key_pool), _ptr(global_value_pool), pool_code,
            _ptr(k_scales), _ptr(v_scales), _ptr(pt), _ptr(pos), _ptr(q2s), n, hkv, hd, tpp, num_pages, num_seqs,
            width, _ptr(cs), int(cs.shape[0]), rot, _ROPE_STYLES[style], _ptr(qi), _ptr(q_out), hq, q_code, sh)
    _lib.check(status)
    return global_key_pool, global_value_pool, q_out


def paged_attention_prefill(
    q_prompt: torch.Tensor,
    k_prompt: torch.Tensor,
    v_prompt: torch.Tensor,
    k_cache_paged: torch.Tensor,
    v_cache_paged: torch.Tensor,
    page_table: torch.Tensor,
    context_len_arr: torch.Tensor,
    stream=None,
    *,
    k_scales: torch.Tensor | None = None,
    v_scales: torch.Tensor | None = None,
) -> torch.Tensor:
    """Causal prefill of a uniform prompt per sequence over a paged history.

    Reference: ops.py:87-130 -> bindings.cpp:74-124 -> ops.cpp:110-186 ->
    paged_attention_prefill_primitive.cpp:63-167 -> prefill.h.metal:28-389.

    S = page_table.shape[0] sequences, prompt length P = N // S (primitive
    :115-116).  q_prompt: [N, Hq, HD] (or [N, HD]); k_prompt / v_prompt:
    [N, Hkv, HD], rows s*P .. s*P+P-1 holding the prompt of sequence s.
    Prompt token i of sequence s attends to the cached tokens
    [0, context_len_arr[s]) of its pages and to prompt tokens 0..i.
    Returns [N * Hq, HD], row (s*P + i) * Hq + h; rows past S*P (when N is
    not a multiple of S) are zero.  HD % 32 == 0.  The page size may be any
    multiple of 8 up to 1024, as in the reference (prefill.h.metal:243-263);
    16 and 32 have dedicated kernels, other sizes read the history through
    registers (slower).  The prompt's K/V need not be in the pages.  fp8
    history pools (an addition) need ``k_scales`` / ``v_scales`` (float32
    [num_pages, Hkv]); head_dim 64, 128 or 256, page size 16 or 32.
    """
    op = "paged_attention_prefill"
    _require_device("q_prompt", q_prompt)
    device = q_prompt.device
    code = dtype_code(q_prompt.dtype)
    num_pages, num_kv_heads, head_dim, tpp = _pools(op, k_cache_paged, v_cache_paged, device, q_prompt.dtype)
    ks, vs = _scales(op, k_cache_paged, k_scales, v_scales, num_pages, num_kv_heads, device)
    num_rows, num_q_heads = _query_dims(op, q_prompt, head_dim)
    for name, t in (("k_prompt", k_prompt), ("v_prompt", v_prompt)):
        _require_device(name, t, device)
        if t.dtype != q_prompt.dtype:
            raise ValueError(f"[{op}] {name} must have the query dtype")
        if tuple(t.shape) != (num_rows, num_kv_heads, head_dim):
            raise ValueError(f"[{op}] {name} must be [{num_rows}, {num_kv_heads}, {head_dim}], got {tuple(t.shape)}")
    if page_table.dim() != 2:
        raise ValueError(f"[{op}] page_table must be 2D [num_seqs, max_pages_per_seq]")
    num_seqs, width = (int(x) for x in page_table.shape)
    _require_device("context_len_arr", context_len_arr, device)
    if context_len_arr.numel() < num_seqs:
        raise ValueError(f"[{op}] {context_len_arr.numel()} context lengths for {num_seqs} sequences")
    covered = num_seqs * (num_rows // num_seqs) if num_seqs > 0 else 0
    sh, sh_current = _launch_stream(stream, device)
    with _on_stream(sh, device, sh_current):
        pt = _index_tensor("page_table", page_table, device)
        ctx = _index_tensor("context_len_arr", context_len_arr, device)
        q = q_prompt.contiguous()
        kd = k_prompt.contiguous()
        vd = v_prompt.contiguous()
        kp = k_cache_paged.contiguous()
        vp = v_cache_paged.contiguous()
        out = torch.empty((num_rows * num_q_heads, head_dim), dtype=q_prompt.dtype, device=device)
        if covered < num_rows:
            out[covered * num_q_heads:].zero_()
        if ks is not None:
            status = _lib.lib().pal_paged_attention_prefill_fp8(
                _ptr(q), _ptr(kd), _ptr(vd), _ptr(kp), _ptr(vp), _ptr(ks.contiguous()), _ptr(vs.contiguous()),
                _ptr(pt), _ptr(ctx), _ptr(out), code, num_rows, num_seqs, num_q_heads, num_kv_heads, head_dim, tpp,
                num_pages, width, sh)
        else:
            status = _lib.lib().pal_paged_attention_prefill(
                _ptr(q), _ptr(kd), _ptr(vd), _ptr(kp), _ptr(vp), _ptr(pt), _ptr(ctx), _ptr(out),
                code, num_rows, num_seqs, num_q_heads, num_kv_heads, head_dim, tpp, num_pages, width, sh,
            )
    _lib.check(status)
    return out


def paged_attention(
    queries: torch.Tensor,
    k_cache_pool: torch.Tensor,
    v_cache_pool: torch.Tensor,
    page_table: torch.Tensor,
    sequence_lengths: torch.Tensor,
    query_to_seq_map: torch.Tensor,
    query_token_offset: torch.Tensor,
    stream=None,
    *,
    k_scales: torch.Tensor | None = None,
    v_scales: torch.Tensor | None = None,
) -> torch.Tensor:
    """Fused mixed batch: decode rows and prefill rows in one call.

    No reference function exists; the arguments are those the reference
    benchmark prepares (batch_latency_vs_num_sequences.cpp:124-131).
    queries: [R, Hq, HD] (or [R, HD]); query_to_seq_map: [R] (u32/i32);
    query_token_offset: [R] int32.  Row r of sequence s = query_to_seq_map[r]
    attends to tokens [0, min(sequence_lengths[s], query_token_offset[r]))
    of s's pages: a decode row passes an offset >= the length, the prompt
    token at absolute position p passes p + 1 (its K/V already written by
    fill_kv_pages).  Returns [R, Hq, HD]; rows that see no token, or name no
    sequence, are zero.  Runs of consecutive rows of one sequence run as MFMA
    prefill tiles, single rows on the split-K decode path.  fp8 pools need
    ``k_scales`` / ``v_scales`` (float32 [num_pages, Hkv]).
    """
    op = "paged_attention"
    _require_device("queries", queries)
    device = queries.device
    code = dtype_code(queries.dtype)
    num_pages, num_kv_heads, head_dim, tpp = _pools(op, k_cache_pool, v_cache_pool, device, queries.dtype)
    ks, vs = _scales(op, k_cache_pool, k_scales, v_scales, num_pages, num_kv_heads, device)
    num_rows, num_q_heads = _query_dims(op, queries, head_dim)
    if page_table.dim() != 2:
        raise ValueError(f"[{op}] page_table must be 2D [num_seqs, max_pages_per_seq]")
    num_seqs, width = (int(x) for x in page_table.shape)
    for name, t in (("sequence_lengths", sequence_lengths), ("query_to_seq_map", query_to_seq_map),
                    ("query_token_offset", query_token_offset)):
        _require_device(name, t, device)
    if sequence_lengths.numel() < num_seqs:
        raise ValueError(f"[{op}] {sequence_lengths.numel()} sequence lengths for {num_seqs} sequences")
    if query_to_seq_map.numel() != num_rows or query_token_offset.numel() != num_rows:
        raise ValueError(f"[{op}] query_to_seq_map and query_token_offset need one entry per query row ({num_rows})")
    L = _lib.lib()
    sh, sh_current = _launch_stream(stream, device)
    with _on_stream(sh, device, sh_current):
        pt = _index_tensor("page_table", page_table, device)
        lens = _index_tensor("sequence_lengths", sequence_lengths, device)
        q2s = _index_tensor("query_to_seq_map", query_to_seq_map, device)
        off = _index_tensor("query_token_offset", query_token_offset, device)
        q = queries.contiguous()
        kp = k_cache_pool.contiguous()
        vp = v_cache_pool.contiguous()
        out = torch.empty((num_rows, num_q_heads, head_dim), dtype=queries.dtype, device=device)
        ws = None
        if num_rows > 0:
            size_fn = L.pal_paged_attention_fp8_workspace_size if ks is not None else \
                L.pal_paged_attention_workspace_size
            with torch.cuda.device(device):
                ws_bytes = size_fn(code, num_rows, num_q_heads, num_kv_heads, head_dim, tpp)
            ws = _workspace("fused", ws_bytes, device, sh)
        if ks is not None:
            status = L.pal_paged_attention_fp8(
                _ptr(q), _ptr(kp), _ptr(vp), _ptr(ks.contiguous()), _ptr(vs.contiguous()), _ptr(pt), _ptr(lens),
                _ptr(q2s), _ptr(off), _ptr(out), code, num_rows, num_seqs, num_q_heads, num_kv_heads, head_dim, tpp,
                num_pages, width, _ptr(ws), ws.numel() if ws is not None else 0, sh)
        else:
            status = L.pal_paged_attention(
                _ptr(q), _ptr(kp), _ptr(vp), _ptr(pt), _ptr(lens), _ptr(q2s), _ptr(off), _ptr(out),
                code, num_rows, num_seqs, num_q_heads, num_kv_heads, head_dim, tpp, num_pages, width,
                _ptr(ws), ws.numel() if ws is not None else 0, sh,
            )
    _lib.check(status)
    return out
