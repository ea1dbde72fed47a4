"""The operators captured into a HIP graph (torch.cuda.CUDAGraph) and replayed.

A decode step (fill_kv_pages of each sequence's newest token, then
paged_attention_decode) and a chunked-prefill step (fill_kv_pages of new
chunks, then the fused paged_attention) are captured once on a side stream
after an eager warm-up there (so the per-stream workspace exists before the
capture), then replayed several times.  Between replays the inputs change by
eager copies, with synchronisations around each replay; every replay must
equal the eager call on the same inputs bit for bit and the oracle within the
dtype's tolerance (bf16 atol/rtol 2e-2), and the pools must equal the
oracle's fill bit for bit.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import proxy_attention_lab as pal
from gpu_util import announce, dev_bits, dev_index, host_bits
from oracle import pal_oracle as orc
from pal_cases import assert_close, make_fused_case, make_paged_case, randn_bits

pytestmark = pytest.mark.gpu
REPLAYS = 4


def _decode_step(t, partition):
    pal.fill_kv_pages(t["new_k"], t["new_v"], t["k"], t["v"], t["pt"], t["pos"], t["q2s"])
    return pal.paged_attention_decode(t["q"], t["k"], t["v"], t["pt"], t["lens"], partition_size=partition)


@pytest.mark.parametrize("partition", [0, 512])
def test_graph_decode_step(partition):
    rng = np.random.default_rng(120 + partition)
    lens = [int(x) for x in rng.integers(1, 3000, size=24)]
    case = make_paged_case(120, lens, 32, 8, 128, 16, "bf16", garbage_tail=False)
    n = len(lens)
    pos = np.asarray(lens, np.int32) - 1
    q2s = np.arange(n, dtype=np.uint32)
    t = dict(k=dev_bits(case.k_pool, "bf16"), v=dev_bits(case.v_pool, "bf16"),
             pt=dev_index(case.page_table, torch.uint32), lens=dev_index(case.seq_lens), pos=dev_index(pos),
             q2s=dev_index(q2s, torch.uint32), q=dev_bits(randn_bits(rng, (n, 32, 128), "bf16"), "bf16"),
             new_k=dev_bits(randn_bits(rng, (n, 8, 128), "bf16"), "bf16"),
             new_v=dev_bits(randn_bits(rng, (n, 8, 128), "bf16"), "bf16"))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            _decode_step(t, partition)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    announce(f"graph capture: fill + decode, partition {partition}")
    with torch.cuda.graph(g, stream=side):
        out = _decode_step(t, partition)
    torch.cuda.synchronize()
    for r in range(REPLAYS):
        q = randn_bits(rng, (n, 32, 128), "bf16")
        nk = randn_bits(rng, (n, 8, 128), "bf16")
        nv = randn_bits(rng, (n, 8, 128), "bf16")
        t["q"].copy_(dev_bits(q, "bf16"))
        t["new_k"].copy_(dev_bits(nk, "bf16"))
        t["new_v"].copy_(dev_bits(nv, "bf16"))
        k0, v0 = host_bits(t["k"]), host_bits(t["v"])
        torch.cuda.synchronize()
        announce(f"graph replay {r}: fill + decode, partition {partition}")
        g.replay()
        torch.cuda.synchronize()
        got, k1, v1 = host_bits(out), host_bits(t["k"]), host_bits(t["v"])
        ek, ev = orc.fill_kv_pages(nk, nv, k0, v0, case.page_table, pos, q2s)
        assert np.array_equal(k1, ek) and np.array_equal(v1, ev), f"replay {r}: pools differ from the oracle fill"
        # the eager call on the same inputs (pools already hold this replay's tokens)
        eager = host_bits(pal.paged_attention_decode(t["q"], t["k"], t["v"], t["pt"], t["lens"],
                                                     partition_size=partition))
        torch.cuda.synchronize()
        assert np.array_equal(got, eager), f"replay {r} differs from the eager call"
        ref = orc.paged_attention_decode(q, ek, ev, case.page_table, case.seq_lens, "bf16")
        assert_close(orc.bits_to_f32(got, "bf16"), ref, "bf16", f"graph replay {r} decode p{partition}")


def test_graph_chunked_prefill_step():
    rng = np.random.default_rng(130)
    fc = make_fused_case(130, [], [(0, 200), (300, 150), (40, 257)], 32, 8, 128, 16, "bf16", block=64,
                         garbage_tail=False)
    c = fc.case
    rows = len(fc.q2seq)
    pos = (fc.q_offset - 1).astype(np.int32)  # each prompt row's own position
    t = dict(k=dev_bits(c.k_pool, "bf16"), v=dev_bits(c.v_pool, "bf16"),
             pt=dev_index(c.page_table, torch.uint32), lens=dev_index(c.seq_lens), pos=dev_index(pos),
             q2s=dev_index(fc.q2seq, torch.uint32), off=dev_index(fc.q_offset),
             q=dev_bits(fc.queries, "bf16"), new_k=dev_bits(randn_bits(rng, (rows, 8, 128), "bf16"), "bf16"),
             new_v=dev_bits(randn_bits(rng, (rows, 8, 128), "bf16"), "bf16"))

    def step():
        pal.fill_kv_pages(t["new_k"], t["new_v"], t["k"], t["v"], t["pt"], t["pos"], t["q2s"])
        return pal.paged_attention(t["q"], t["k"], t["v"], t["pt"], t["lens"], t["q2s"], t["off"])

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    announce("graph capture: fill of prefill chunks + fused paged_attention")
    with torch.cuda.graph(g, stream=side):
        out = step()
    torch.cuda.synchronize()
    for r in range(REPLAYS):
        q = randn_bits(rng, (rows, 32, 128), "bf16")
        nk = randn_bits(rng, (rows, 8, 128), "bf16")
        nv = randn_bits(rng, (rows, 8, 128), "bf16")
        t["q"].copy_(dev_bits(q, "bf16"))
        t["new_k"].copy_(dev_bits(nk, "bf16"))
        t["new_v"].copy_(dev_bits(nv, "bf16"))
        k0, v0 = host_bits(t["k"]), host_bits(t["v"])
        torch.cuda.synchronize()
        announce(f"graph replay {r}: chunked prefill")
        g.replay()
        torch.cuda.synchronize()
        got, k1, v1 = host_bits(out), host_bits(t["k"]), host_bits(t["v"])
        ek, ev = orc.fill_kv_pages(nk, nv, k0, v0, c.page_table, pos, fc.q2seq)
        assert np.array_equal(k1, ek) and np.array_equal(v1, ev), f"replay {r}: pools differ from the oracle fill"
        eager = host_bits(pal.paged_attention(t["q"], t["k"], t["v"], t["pt"], t["lens"], t["q2s"], t["off"]))
        torch.cuda.synchronize()
        assert np.array_equal(got, eager), f"replay {r} differs from the eager call"
        ref = orc.paged_attention(q, ek, ev, c.page_table, c.seq_lens, fc.q2seq, fc.q_offset, "bf16")
        assert_close(orc.bits_to_f32(got, "bf16"), ref, "bf16", f"graph replay {r} chunked prefill")
