"""bench.py's host-side parts on the CPU: the config-1 builder and the CPU
baseline (torch CPU restatement of the equivalency path) over small samples
shaped like the ones the GPU run hands it."""

from __future__ import annotations

import numpy as np

import bench
from oracle import pal_oracle as orc


def _sample(seed, lens, hq, hkv, hd, dtype):
    rng = np.random.default_rng(seed)
    lens = np.asarray(lens, np.int32)
    npg = (lens + 15) // 16
    pages = int(npg.sum()) + 2
    perm = rng.permutation(pages)
    pt = np.zeros((len(lens), int(npg.max())), np.uint32)
    cur = 0
    for s, n in enumerate(npg):
        pt[s, :n] = perm[cur:cur + n]
        cur += n
    def bits(shape):
        return orc.f32_to_bits(rng.standard_normal(shape).astype(np.float32), dtype)
    return {"q": bits((len(lens), hq, hd)), "k": bits((pages, hkv, hd // 8, 16, 8)),
            "v": bits((pages, hkv, hd, 16)), "pt": pt, "lens": lens, "dtype": dtype}


def test_config1_host_shape():
    c1 = bench.config1_host()
    assert c1["k"].shape == (64, 1, 8, 16, 8) and c1["v"].shape == (64, 1, 64, 16)
    used = np.concatenate([c1["pt"][s, : (int(n) + 15) // 16] for s, n in enumerate(c1["lens"])])
    assert len(used) == 39 and len(np.unique(used)) == 39  # 39 distinct pages of the 64


def test_cpu_baseline_reports_every_config():
    c2 = _sample(1, [300, 40, 129], 8, 2, 64, "bf16")
    c2["bytes"] = int(c2["lens"].sum()) * 2 * 2 * 64 * 2
    c3 = dict(_sample(2, [500], 8, 2, 64, "bf16"), bytes=10**6, scale=4.0, what="1 of 4")
    c4 = dict(_sample(3, [70], 8, 2, 64, "bf16"), flops=1e9, scale=3.0, what="1 of 3",
              q2s=np.zeros(70, np.uint32), off=np.arange(1, 71, dtype=np.int32))
    c4["q"] = np.resize(c4["q"], (70, 8, 64))
    res = bench.cpu_baseline({"c2": c2, "c3": c3, "c4": c4})
    assert res["kind"] == "port" and res["unit"] == "GB/s" and res["value"] > 0
    assert res["cores"] >= 1 and "config1" in res and "config3" in res and "config4" in res
    assert res["config3"]["ms_scaled"] >= res["config3"]["ms_sample"]
    assert res["config4"]["TFLOP/s"] > 0
