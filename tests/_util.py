"""Shared helpers for the parity tests."""
from __future__ import annotations

import numpy as np

# Parity bar: max-abs per component and max angular error vs the CPU oracle.
TOL_ABS = 1e-5
TOL_DEG = 0.01


def angular_error_deg(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Per-pixel angle between vectors a and b, shaped (..., 3, N) -> (..., N),
    via atan2(|a x b|, a.b); two zero vectors count as 0."""
    a = a.astype(np.float64)
    b = b.astype(np.float64)
    cr = np.cross(a, b, axis=-2)
    s = np.sqrt((cr * cr).sum(axis=-2))
    c = (a * b).sum(axis=-2)
    ang = np.degrees(np.arctan2(s, c))
    both_zero = ((a == 0).all(axis=-2)) & ((b == 0).all(axis=-2))
    return np.where(both_zero, 0.0, ang)


def compare(got: np.ndarray, want: np.ndarray, mask=None):
    """(max-abs over components, max angular error in degrees, NaN-pattern
    mismatch count); arrays shaped (B, 3, HW) or (3, HW)."""
    got = np.asarray(got, dtype=np.float32)
    want = np.asarray(want, dtype=np.float32)
    if got.ndim == 2:
        got, want = got[None], want[None]
    nan_g, nan_w = np.isnan(got), np.isnan(want)
    nan_mismatch = int((nan_g != nan_w).sum())
    fin = ~(nan_g | nan_w)
    if mask is not None:
        fin &= mask
    d = np.abs(got.astype(np.float64) - want.astype(np.float64))
    max_abs = float(d[fin].max()) if fin.any() else 0.0
    pix_ok = fin.all(axis=1)
    ang = angular_error_deg(got, want)
    max_deg = float(ang[pix_ok].max()) if pix_ok.any() else 0.0
    return max_abs, max_deg, nan_mismatch


def to_dev(a, device):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


# Out-of-bounds guards: outputs live inside a larger buffer whose head and
# tail hold a canary bit pattern (a NaN no kernel produces); a write past
# either end of the output changes it.
GUARD = 4096                    # floats on each side (16 KiB)
CANARY = 0x7FBADBAD


class Guarded:
    """A contiguous float32 view of n elements inside a canary-filled buffer,
    `shift` floats past a 16 KiB boundary (shift=1 misaligns it by 4 bytes)."""

    def __init__(self, n: int, device, shift: int = 0, fill=None):
        import torch
        self.n, self.lo = n, GUARD + shift
        self.buf = torch.full((n + 2 * GUARD + shift,), CANARY, dtype=torch.int32, device=device)
        if fill is not None:
            self.buf[self.lo:self.lo + n] = torch.as_tensor(
                np.ascontiguousarray(fill, dtype=np.float32).reshape(-1)).view(torch.int32).to(device)
        self.out = self.buf.view(torch.float32)[self.lo:self.lo + n]

    def intact(self) -> bool:
        b = self.buf.cpu().numpy()
        return bool((b[:self.lo] == CANARY).all() and (b[self.lo + self.n:] == CANARY).all())
