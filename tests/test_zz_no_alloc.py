"""pal_paged_attention_decode_noalloc: the decode entry point that allocates
nothing, its scratch being a library-held device array.

Called through the C ABI and checked against pal_paged_attention_decode (the
entry point with a caller workspace) on the same inputs -- the two share
their kernels, so the outputs must be bit-identical -- and against the CPU
oracle (bf16 atol/rtol 2e-2), on two calls in a row, the second smaller
(the array keeps the first call's contents).  A shape whose workspace
exceeds the array is rejected before any launch.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import proxy_attention_lab as pal
from gpu_util import announce, dev_bits, dev_index, host_bits, host_f32
from oracle import pal_oracle as orc
from pal_cases import assert_close, make_paged_case, randn_bits
from proxy_attention_lab import _lib

pytestmark = pytest.mark.gpu


def _noalloc(case, q_dev, partition=0):
    dt = case.dtype
    out = torch.empty((case.num_seqs, case.num_q_heads, case.head_dim), dtype=q_dev.dtype, device=q_dev.device)
    k, v = dev_bits(case.k_pool, dt), dev_bits(case.v_pool, dt)
    pt, lens = dev_index(case.page_table, torch.uint32), dev_index(case.seq_lens)
    torch.cuda.synchronize()  # inputs are ready before the launch stream (the current one) runs the call
    st = _lib.lib().pal_paged_attention_decode_noalloc(
        q_dev.data_ptr(), k.data_ptr(), v.data_ptr(), pt.data_ptr(), lens.data_ptr(), out.data_ptr(),
        _lib.DTYPE_BFLOAT16 if dt == "bf16" else _lib.DTYPE_FLOAT16, int(q_dev.shape[0]), case.num_seqs,
        case.num_q_heads, case.num_kv_heads, case.head_dim, case.tokens_per_page, int(case.k_pool.shape[0]),
        int(case.page_table.shape[1]), partition, torch.cuda.current_stream().cuda_stream)
    _lib.check(st)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("partition", [0, 512])
def test_noalloc_matches_workspace_entry_two_calls(partition):
    cases = [
        (make_paged_case(90, [3000, 17, 512, 4096, 1, 900, 2222, 64], 32, 8, 128, 16, "bf16"), "first"),
        (make_paged_case(91, [100, 33, 700], 32, 8, 128, 16, "bf16"), "second (smaller)"),
    ]
    for case, what in cases:
        q = randn_bits(np.random.default_rng(case.num_seqs), (case.num_seqs, 32, 128), "bf16")
        announce(f"noalloc decode {what} partition {partition}")
        qd = dev_bits(q, "bf16")
        got = _noalloc(case, qd, partition)
        ref_dev = pal.paged_attention_decode(qd, dev_bits(case.k_pool, "bf16"), dev_bits(case.v_pool, "bf16"),
                                             dev_index(case.page_table, torch.uint32), dev_index(case.seq_lens),
                                             partition_size=partition)
        torch.cuda.synchronize()
        assert np.array_equal(host_bits(got), host_bits(ref_dev)), f"{what}: differs from the workspace entry"
        ref = orc.paged_attention_decode(q, case.k_pool, case.v_pool, case.page_table, case.seq_lens, "bf16")
        assert_close(host_f32(got), ref, "bf16", f"noalloc {what} partition {partition}")


def test_noalloc_under_graph_capture():
    """The callers the entry is for: captured into a HIP graph (after one
    eager call, which reads the scratch array's address) and replayed with
    new queries between replays; every replay equals the workspace entry's
    eager output bit for bit."""
    case = make_paged_case(92, [3000, 17, 512, 4096, 1, 900], 32, 8, 128, 16, "bf16")
    rng = np.random.default_rng(92)
    k, v = dev_bits(case.k_pool, "bf16"), dev_bits(case.v_pool, "bf16")
    pt, lens = dev_index(case.page_table, torch.uint32), dev_index(case.seq_lens)
    q = dev_bits(randn_bits(rng, (case.num_seqs, 32, 128), "bf16"), "bf16")
    out = torch.empty_like(q)
    L = _lib.lib()

    def call():
        _lib.check(L.pal_paged_attention_decode_noalloc(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), pt.data_ptr(), lens.data_ptr(), out.data_ptr(),
            _lib.DTYPE_BFLOAT16, case.num_seqs, case.num_seqs, 32, 8, 128, 16, int(case.k_pool.shape[0]),
            int(case.page_table.shape[1]), 0, torch.cuda.current_stream().cuda_stream))

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    announce("noalloc decode under graph capture")
    with torch.cuda.graph(g, stream=side):
        call()
    torch.cuda.synchronize()
    for r in range(3):
        q.copy_(dev_bits(randn_bits(rng, (case.num_seqs, 32, 128), "bf16"), "bf16"))
        torch.cuda.synchronize()
        announce(f"noalloc graph replay {r}")
        g.replay()
        torch.cuda.synchronize()
        eager = pal.paged_attention_decode(q, k, v, pt, lens)
        torch.cuda.synchronize()
        assert np.array_equal(host_bits(out), host_bits(eager)), f"replay {r} differs from the workspace entry"


def test_noalloc_rejects_shapes_beyond_scratch():
    """A partition-128 call over 4096 sequences with 8192-page tables needs
    far more than the 64 MiB array: rejected with a clear error.  The
    pointers are null, so even a call that got past the size check would be
    refused by the null-pointer check that follows it; nothing is launched."""
    L = _lib.lib()
    need = L.pal_paged_attention_decode_workspace_size(_lib.DTYPE_BFLOAT16, 4096, 32, 8, 128, 16, 8192, 128)
    assert need > 64 << 20
    st = L.pal_paged_attention_decode_noalloc(None, None, None, None, None, None, _lib.DTYPE_BFLOAT16, 4096, 4096,
                                              32, 8, 128, 16, 1 << 20, 8192, 128, None)
    assert st == _lib.PAL_ERR_INVALID_ARGUMENT
    assert "scratch" in _lib.last_error()
