"""Shared test helpers: seeded inputs, torch <-> oracle conversions and the
tolerance rule.

Tolerance: 1e-5 relative for fp32, 2e-2 for bf16.  An
element passes when |got - want| <= rtol * max(|want|, FLOOR * rms(want)):
the pure relative bound for every element of at least FLOOR times the
tensor's RMS, and for the elements below that (results of cancellation, where
a relative bound measures only the rounding of the terms that cancelled) the
same relative bound on FLOOR * rms.  FLOOR is 1/16 (SANDY_TEST_FLOOR
overrides it).  Integer and index outputs are compared exactly.
"""
from __future__ import annotations

import os

import numpy as np
import torch

from oracle import oracle as O

RTOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2}
FLOOR = float(os.environ.get("SANDY_TEST_FLOOR", 1.0 / 16))


def rng(seed):
    return np.random.default_rng(seed)


def normal(r, shape, scale=1.0):
    return (r.standard_normal(shape) * scale).astype(np.float32)


def to_oracle(t: torch.Tensor) -> np.ndarray:
    """GPU/CPU torch tensor -> numpy in the oracle's encoding (bf16 as uint16)."""
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16).copy()
    return t.numpy().copy()


def from_f32(a: np.ndarray, dtype: torch.dtype, device="cuda") -> torch.Tensor:
    """float32 numpy -> torch tensor of dtype, rounding to bf16 with RNE exactly like the oracle."""
    if dtype == torch.bfloat16:
        bits = O.f32_to_bf16(a)
        return torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16).to(device)
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(device)


def from_oracle(a: np.ndarray, device="cuda") -> torch.Tensor:
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16).to(device)
    return torch.from_numpy(a.copy()).to(device)


def as_f32(a: np.ndarray) -> np.ndarray:
    return O.to_f32(a)


def assert_close(got, want, dtype, what="", rtol=None, floor=None):
    """got: torch tensor or oracle-encoded numpy; want: oracle-encoded numpy.
    `floor` overrides FLOOR for comparisons of multi-op chains (whole model
    steps), whose float roundings compound across dozens of ops."""
    if isinstance(got, torch.Tensor):
        got = to_oracle(got)
    g = as_f32(got).astype(np.float64)
    w = as_f32(want).astype(np.float64)
    assert g.shape == w.shape, f"{what}: shape {g.shape} != {w.shape}"
    rtol = rtol if rtol is not None else RTOL[dtype]
    finite = np.isfinite(w)
    assert np.array_equal(np.isfinite(g), finite), f"{what}: non-finite pattern differs"
    if not finite.any():
        return
    scale = float(np.sqrt(np.mean(w[finite] ** 2))) if finite.any() else 0.0
    err = np.abs(g - w)
    bound = rtol * np.maximum(np.abs(w), (FLOOR if floor is None else floor) * scale)
    bad = finite & (err > bound)
    if bad.any():
        i = np.unravel_index(np.argmax(np.where(finite, err - bound, -np.inf)), err.shape)
        raise AssertionError(
            f"{what}: {bad.sum()} of {w.size} elements outside tolerance (rtol {rtol}); "
            f"worst at {i}: got {g[i]!r} want {w[i]!r}")


def assert_equal(got, want, what=""):
    if isinstance(got, torch.Tensor):
        got = to_oracle(got)
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    if not np.array_equal(got, want):
        idx = np.argwhere(got != want)[0]
        raise AssertionError(f"{what}: differs at {tuple(idx)}: got {got[tuple(idx)]} want {want[tuple(idx)]}")
