"""Shared helpers for the tests: seeded inputs, tolerances, comparisons."""
from __future__ import annotations

import math
import sys

import numpy as np

# Tolerances of the parity bar (stated per mode, outputs and gradients):
#   fp32-MFMA: max-abs 1e-4
#   bf16-MFMA: |got - ref| <= 2e-2 + 1e-2 * |ref|   (max-abs 2e-2, relative 1e-2)
TOL = {"fp32": (1e-4, 0.0), "bf16": (2e-2, 1e-2)}


def randn(shape, seed, dtype=np.float32):
    """N(0,1) from numpy's PCG64 seeded generator, rounded to `dtype`."""
    return np.random.default_rng(seed).standard_normal(shape).astype(dtype)


def bf16_round(x):
    """Round float32 values to bfloat16 (nearest even) and back to float32."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def assert_close(got, ref, mode, what, mask=None):
    atol, rtol = TOL[mode]
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    if mask is not None:
        got, ref = got[mask], ref[mask]
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    err = np.abs(got - ref)
    bound = atol + rtol * np.abs(ref)
    worst = int(np.argmax(err - bound))
    ok = bool(np.all(err <= bound))
    print(f"[{what}] mode={mode} max_abs={err.max():.3e} atol={atol} rtol={rtol}", flush=True)
    assert ok, (f"{what}: max_abs={err.max():.3e} at {np.unravel_index(worst, err.shape)} "
                f"got={got.flat[worst]:.6g} ref={ref.flat[worst]:.6g}")
    return float(err.max())


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()
