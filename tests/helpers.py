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


def oracle_threads() -> int:
    """Host threads for the oracle's checks: the process's CPU affinity, at
    most 16 (the host cores a one-GPU machine gives a process)."""
    import oracle

    return max(1, min(oracle.cpu_threads(), 16))


def check_16bit(name: str, got: np.ndarray, ref: np.ndarray, maxrel: float = 2e-2,
                elementwise: bool = True, roundings: int = 1) -> float:
    """The bf16 / f16 parity bar: max|a - b| / max|b| <= maxrel (printed).
    With `elementwise`, also |a - b| <= roundings * 2^-8 |b| + 2^-12 max|b|
    per element: the GPU accumulates the same F32 terms in another order and
    rounds once to bf16 (half an ulp, 2^-9 |b|), so anything beyond that
    bound -- a dropped or doubled tap, a wrong weight -- fails even where its
    share of max|b| is small.  `roundings` = 2 for outputs rounded twice
    (f16, then bf16)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.isfinite(got).all(), f"{name}: non-finite outputs"
    den = float(np.abs(ref).max())
    err = np.abs(got - ref)
    mr = float(err.max() / max(den, 1e-30))
    print(f"[parity] {name}: rows={ref.shape[0]} max_rel={mr:.3e}", flush=True)
    assert mr <= maxrel, f"{name}: max-rel {mr:.3e} > {maxrel}"
    if elementwise:
        bad = err > np.abs(ref) * (roundings * 2.0 ** -8) + den * 2.0 ** -12
        assert not bad.any(), (f"{name}: {int(bad.sum())} elements beyond one bf16 rounding, "
                               f"first at {np.argwhere(bad)[0]}")
    return mr


def row_subset(token_major: np.ndarray, n: int, rows: np.ndarray, ntaps: int = 27) -> np.ndarray:
    """Token-major sub-table of the given output rows (sources keep their ids)."""
    t = token_major.reshape(-1, ntaps)
    return np.ascontiguousarray(t[rows]).reshape(-1)
