"""Helpers for GPU parity tests: numpy int16 <-> device tensors, oracle threads."""
from __future__ import annotations

import os
import sys

import numpy as np


def dev(a: np.ndarray):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def host(t) -> np.ndarray:
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def empty_dev(shape, fill: int = 0x5A5A):
    """Device int16 buffer pre-filled with a marker so unwritten outputs show."""
    import torch
    t = torch.empty(shape, dtype=torch.int16, device="cuda")
    t.fill_(np.int16(np.uint16(fill).view(np.int16)))
    return t


def oracle_threads() -> int:
    """CPU threads for the oracle on this host (at most 16, one GPU host's CPU share)."""
    n = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    return n if n > 0 else min(os.cpu_count() or 1, 16)


def say(msg: str) -> None:
    """Flush a progress line so a GPU fault still leaves the case name behind."""
    sys.stdout.write(msg + "\n")
    sys.stdout.flush()
