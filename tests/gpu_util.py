"""numpy <-> device helpers for the GPU parity tests."""
from __future__ import annotations

import sys

import numpy as np
import torch

_VIEW = {np.dtype(np.uint16): np.int16, np.dtype(np.uint32): np.int32}


def to_dev(a: np.ndarray, device) -> torch.Tensor:
    a = np.ascontiguousarray(a)
    v = a.view(_VIEW.get(a.dtype, a.dtype))
    return torch.from_numpy(v).to(device)


def to_np(t: torch.Tensor, dtype=np.uint16) -> np.ndarray:
    t = t.detach().contiguous().cpu()
    if t.dtype == torch.bfloat16:
        t = t.view(torch.int16)
    return t.numpy().view(dtype)


def announce(msg: str) -> None:
    """Name the case on stdout before a GPU step, flushed, so a fault names it."""
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()
