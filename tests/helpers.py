"""Shared helpers for the parity tests: seeded inputs, bf16 rounding, error metrics."""

from __future__ import annotations

import numpy as np

import oracle


def randn(rng: np.random.Generator, shape, scale: float = 1.0) -> np.ndarray:
    return (rng.standard_normal(shape) * scale).astype(np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    return oracle.round_bf16(x)


def round_f16(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


def max_abs(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b))) if a.size else 0.0


# Tolerances stated by the task for this path: max-abs 1e-4 (f32), 2e-2 (bf16/f16).
TOL_F32 = 1e-4
TOL_BF16 = 2e-2
