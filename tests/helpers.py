"""Test helpers shared by the GPU and CPU suites."""
from __future__ import annotations

import numpy as np


def bf16_bits(orc, a: np.ndarray) -> np.ndarray:
    return orc.f32_to_bf16(np.ascontiguousarray(a, dtype=np.float32))


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


def to_dev_bf16(bits: np.ndarray, dev):
    import torch

    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(dev).view(torch.bfloat16)


def from_dev(t) -> np.ndarray:
    import torch

    if t.dtype == torch.bfloat16:
        return bf16_to_f32(t.view(torch.int16).cpu().numpy().view(np.uint16))
    return t.float().cpu().numpy()


def max_rel(a: np.ndarray, b: np.ndarray) -> float:
    """max|a - b| / max|b| (the bf16 / Q8_0 parity metric)."""
    den = float(np.abs(b).max())
    return float(np.abs(a.astype(np.float64) - b.astype(np.float64)).max() / max(den, 1e-30))


def row_subset(token_major: np.ndarray, n: int, rows: np.ndarray, ntaps: int = 27) -> np.ndarray:
    """Token-major sub-table of the given output rows (sources keep their ids)."""
    t = token_major.reshape(-1, ntaps)
    return np.ascontiguousarray(t[rows]).reshape(-1)
