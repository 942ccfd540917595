"""The 16-bit encoder kernel's choice of reference max, emulated on the CPU.

When every row max of a wave's first 32 keys lies in a window around 0 (log2 units), the kernel
takes 0 as each row's reference max and a weight is exp2 of the score itself, rounded to the
16-bit type for the second product (the row sum adds exactly those rounded weights). Otherwise
the reference max is the first subtile's row max. This emulation (numpy exp2, round to nearest
even into f16 or bf16) shows why the window must depend on the type: with the bf16 window
[-64, 32], an f16 row whose scores all sit near -40 log2 units gets weights that flush to zero,
so its sum is 0 and the kernel would write 0 instead of the softmax average. The window
constants are read from the kernel source, so the emulation checks the values the kernel uses.
"""

from __future__ import annotations

import os
import re

import numpy as np
import pytest

from tests.helpers import round_bf16

SRC = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "ffai_amd",
                   "csrc", "attn_common.cuh")


def window(name_lo: str, name_hi: str) -> tuple[float, float]:
    text = open(SRC).read()
    val = lambda n: float(re.search(rf"constexpr float {n} = (-?[0-9.]+)f;", text).group(1))
    return val(name_lo), val(name_hi)


def _round(w: np.ndarray, dtype: str) -> np.ndarray:
    with np.errstate(over="ignore"):
        return w.astype(np.float16).astype(np.float32) if dtype == "f16" else round_bf16(w)


def kernel_row(s_log2: np.ndarray, v: np.ndarray, dtype: str, win: tuple[float, float]):
    """One query row as the kernel computes it: reference max m from the first 32 keys (0 when
    it lies in `win`), then per 32-key subtile weights exp2(s - m) rounded to `dtype`; a subtile
    whose rounded weights overflow or sum above 2^64 is redone against its own max, the earlier
    sum and accumulator rescaled. Returns the normalised output and the weight sum."""
    m1 = float(s_log2[:32].max())
    m = 0.0 if win[0] <= m1 <= win[1] else m1
    l, acc = 0.0, np.zeros(v.shape[1])
    for j in range(0, s_log2.size, 32):
        sj, vj = s_log2[j:j + 32], v[j:j + 32]
        w = _round(np.exp2((sj - m).astype(np.float32)), dtype).astype(np.float64)
        if not np.isfinite(w).all() or w.sum() > 2.0 ** 64:
            m_new = max(m, float(sj.max()))
            corr = 2.0 ** (m - m_new)
            l, acc, m = l * corr, acc * corr, m_new
            w = _round(np.exp2((sj - m).astype(np.float32)), dtype).astype(np.float64)
        l += w.sum()
        acc += w @ vj
    out = acc / l if l > 0 else np.zeros(v.shape[1])
    return out, l


def exact_row(s_log2: np.ndarray, v: np.ndarray) -> np.ndarray:
    p = np.exp2(s_log2.astype(np.float64) - s_log2.max())
    return (p / p.sum()) @ v


def _row(seed: int, row_max: float, keys: int = 300):
    rng = np.random.default_rng(seed)
    s = rng.standard_normal(keys) * 1.44
    s = s - s[:32].max() + row_max  # the first subtile's max sits at row_max
    v = rng.standard_normal((keys, 64))
    return s.astype(np.float32), v


def test_bf16_window_in_f16_loses_rows_far_below_zero():
    """The failure the f16 window prevents: f16 weights of a row near -40 all flush to 0."""
    s, v = _row(1, -40.0)
    out, l = kernel_row(s, v, "f16", window("kFastMaxLo", "kFastMaxHi"))
    assert l == 0.0 and not out.any()
    # at -24 the largest weights are f16 subnormals with a few significant bits
    s, v = _row(2, -24.0)
    out, _ = kernel_row(s, v, "f16", window("kFastMaxLo", "kFastMaxHi"))
    assert np.abs(out - exact_row(s, v)).max() > 2e-2


@pytest.mark.parametrize("row_max", [-63.0, -40.0, -20.0, -5.0, -4.0, 0.0, 10.0, 15.0, 20.0])
def test_each_type_keeps_its_rows(row_max):
    """With the type's own window every row stays within the 16-bit bar of the exact softmax."""
    s, v = _row(int(100 + row_max), row_max)
    want = exact_row(s, v)
    for dtype, names in (("f16", ("kFastMaxLoF16", "kFastMaxHiF16")),
                         ("bf16", ("kFastMaxLo", "kFastMaxHi"))):
        out, l = kernel_row(s, v, dtype, window(*names))
        assert np.isfinite(l) and l > 0, (dtype, row_max)
        assert np.abs(out - want).max() < 2e-2, (dtype, row_max)


def test_f16_window_keeps_the_largest_weight_normal():
    lo, hi = window("kFastMaxLoF16", "kFastMaxHiF16")
    assert 2.0 ** lo >= 2.0 ** -14 * 2 ** 10  # keys 10 log2 units below the max stay normal
    assert 2.0 ** hi <= 65504.0                # the first subtile's weights are finite


@pytest.mark.parametrize("dtype,inf_bits", [("bf16", 0x7F80), ("f16", 0x7C00)])
def test_fold_overflow_test_is_exact_for_every_16_bit_pair(dtype, inf_bits):
    """The Q fold keeps Q unscaled when a scaled half is inf or NaN. The kernels test that with
    vector integer operations per packed pair: OR over the pairs of (y & inf_bits * 0x10001) +
    (0x8000 - inf_bits) * 0x10001, then bits 15 and 31. Over every 16-bit value in each half,
    that flags exactly the halves whose magnitude is at least inf_bits (an all-ones exponent),
    and a carry never crosses from the low half into the high one."""
    h = np.arange(1 << 16, dtype=np.uint64)
    k2, c2 = inf_bits * 0x10001, (0x8000 - inf_bits) * 0x10001
    for hi_vals in (h, h[::-1]):
        y = (hi_vals << 16) | h
        t = ((y & k2) + c2) & 0xFFFFFFFF
        assert np.array_equal((t & 0x8000) != 0, (h & 0x7FFF) >= inf_bits), dtype
        assert np.array_equal((t & 0x80000000) != 0, (hi_vals & 0x7FFF) >= inf_bits), dtype


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_fold_by_at_most_one_keeps_every_finite_element_finite(dtype):
    """The kernels test the folded Q for inf/NaN only when scale * log2(e) exceeds 1: below,
    every finite 16-bit value times the factor (an f32 product, rounded to nearest-even to the
    16-bit type) stays finite. Checked for every finite value of the type and factors up to 1."""
    from tests.helpers import round_f16

    bits = np.arange(1 << 16, dtype=np.uint32)
    if dtype == "bf16":
        vals = (bits << 16).view(np.float32)
        rnd = round_bf16
    else:
        vals = bits.astype(np.uint16).view(np.float16).astype(np.float32)
        rnd = round_f16
    vals = vals[np.isfinite(vals)]
    for f in (1.0, np.nextafter(np.float32(1.0), np.float32(0.0)), 0.5, 0.18033688, 1e-3):
        with np.errstate(over="ignore"):
            out = rnd(vals * np.float32(f))
        assert np.isfinite(out).all(), (dtype, f)
    with np.errstate(over="ignore"):  # and just above 1 a finite value can overflow
        assert not np.isfinite(rnd(vals * np.float32(1.0078125))).all()
