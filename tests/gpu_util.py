"""Host <-> device helpers for the GPU parity tests (numpy bit patterns <-> torch)."""

from __future__ import annotations

import sys

import numpy as np
import torch

TORCH_DTYPE = {"f16": torch.float16, "bf16": torch.bfloat16}
DEV = "cuda:0"


def announce(msg: str) -> None:
    """Print a case name straight to the real stderr before a GPU step."""
    print(f"[gpu-case] {msg}", file=sys.__stderr__, flush=True)


def dev_bits(bits: np.ndarray, dtype: str) -> torch.Tensor:
    arr = np.ascontiguousarray(bits, dtype=np.uint16).view(np.int16)
    return torch.from_numpy(arr).to(DEV).view(TORCH_DTYPE[dtype])


def dev_index(a: np.ndarray, dtype=torch.int32) -> torch.Tensor:
    arr = np.ascontiguousarray(a)
    if arr.dtype == np.uint32:
        arr = arr.view(np.int32)
    return torch.from_numpy(arr.astype(np.int32, copy=False)).to(DEV).to(dtype)


def host_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def host_f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()
