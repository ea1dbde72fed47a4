"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py):
the oracle must still reproduce them (CPU), and the HIP operators must match
them (GPU) -- bit-exact for fill, within the attention tolerances otherwise."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import pal_oracle as orc
from pal_cases import assert_close

GOLDEN = Path(__file__).resolve().parent / "golden"


def _load(name):
    with np.load(GOLDEN / name, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def test_oracle_reproduces_golden():
    g = _load("config1_decode_f16.npz")
    out = orc.paged_attention_decode(g["queries"], g["k_pool"], g["v_pool"], g["page_table"], g["seq_lens"], "f16")
    np.testing.assert_array_equal(out, g["expected"])
    g = _load("prefill_small_bf16.npz")
    out = orc.paged_attention_prefill(g["q_prompt"], g["k_prompt"], g["v_prompt"], g["k_pool"], g["v_pool"],
                                      g["page_table"], g["context_lens"], "bf16")
    np.testing.assert_array_equal(out, g["expected"])
    g = _load("fused_small_f16.npz")
    out = orc.paged_attention(g["queries"], g["k_pool"], g["v_pool"], g["page_table"], g["seq_lens"], g["q2seq"],
                              g["q_offset"], "f16")
    np.testing.assert_array_equal(out, g["expected"])
    g = _load("fill_small_bf16.npz")
    k, v = orc.fill_kv_pages(g["new_keys"], g["new_values"], g["k_pool"], g["v_pool"], g["page_table"],
                             g["write_pos"], g["q2seq"])
    np.testing.assert_array_equal(k, g["expected_k"])
    np.testing.assert_array_equal(v, g["expected_v"])


@pytest.mark.gpu
def test_hip_operators_match_golden():
    import proxy_attention_lab as pal
    from gpu_util import announce, dev_bits, dev_index, host_bits, host_f32

    announce("golden config 1 decode")
    g = _load("config1_decode_f16.npz")
    out = pal.paged_attention_decode(dev_bits(g["queries"], "f16"), dev_bits(g["k_pool"], "f16"),
                                     dev_bits(g["v_pool"], "f16"), dev_index(g["page_table"], torch.uint32),
                                     dev_index(g["seq_lens"]))
    torch.cuda.synchronize()
    assert_close(host_f32(out), g["expected"], "f16", "config 1")
    announce("golden prefill")
    g = _load("prefill_small_bf16.npz")
    out = pal.paged_attention_prefill(dev_bits(g["q_prompt"], "bf16"), dev_bits(g["k_prompt"], "bf16"),
                                      dev_bits(g["v_prompt"], "bf16"), dev_bits(g["k_pool"], "bf16"),
                                      dev_bits(g["v_pool"], "bf16"), dev_index(g["page_table"], torch.uint32),
                                      dev_index(g["context_lens"]))
    torch.cuda.synchronize()
    assert_close(host_f32(out), g["expected"], "bf16", "prefill")
    announce("golden fused")
    g = _load("fused_small_f16.npz")
    out = pal.paged_attention(dev_bits(g["queries"], "f16"), dev_bits(g["k_pool"], "f16"),
                              dev_bits(g["v_pool"], "f16"), dev_index(g["page_table"], torch.uint32),
                              dev_index(g["seq_lens"]), dev_index(g["q2seq"], torch.uint32), dev_index(g["q_offset"]))
    torch.cuda.synchronize()
    assert_close(host_f32(out), g["expected"], "f16", "fused")
    announce("golden fill")
    g = _load("fill_small_bf16.npz")
    kd, vd = dev_bits(g["k_pool"], "bf16"), dev_bits(g["v_pool"], "bf16")
    pal.fill_kv_pages(dev_bits(g["new_keys"], "bf16"), dev_bits(g["new_values"], "bf16"), kd, vd,
                      dev_index(g["page_table"], torch.uint32), dev_index(g["write_pos"]),
                      dev_index(g["q2seq"], torch.uint32))
    torch.cuda.synchronize()
    assert np.array_equal(host_bits(kd), g["expected_k"])
    assert np.array_equal(host_bits(vd), g["expected_v"])
