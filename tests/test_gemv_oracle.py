"""The decoder-GEMV oracle (oracle/gemv.py) against the properties the reference's arithmetic
fixes (CPU only)."""

from __future__ import annotations

import numpy as np

from oracle import gemv as og


def test_rust_round_is_half_away_from_zero():
    v = np.array([0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 0.49999997, -0.49999997, 126.5, 3.0],
                 np.float32)
    np.testing.assert_array_equal(og.rust_round(v),
                                  np.array([1, -1, 2, -2, 3, -3, 0, 0, 127, 3], np.float32))


def test_quantize_bounds_and_correction():
    """|q| <= 127, each block's largest magnitude maps to +-127, every weight is within half a
    step of q * scale, and corr is 64 * sum_b scale_b * blocksum_b (checked in float64)."""
    rng = np.random.default_rng(0)
    w = rng.standard_normal((257, 384)).astype(np.float32)
    w[3, 32:64] = 0.0  # an all-zero block takes scale 1
    q, sc, corr = og.vocab_quantize(w, 32)
    assert q.dtype == np.int8 and np.abs(q.astype(np.int32)).max() <= 127
    blocks = w.reshape(257, 12, 32)
    qb = q.reshape(257, 12, 32).astype(np.float64)
    assert sc[3, 1] == 1.0 and not qb[3, 1].any()
    nz = sc != 1.0
    assert (np.abs(qb).max(axis=2)[nz] == 127).all()
    assert (np.abs(blocks - qb * sc[:, :, None]) <= sc[:, :, None] / 2 * (1 + 1e-6)).all()
    want = 64.0 * (sc.astype(np.float64) * qb.sum(axis=2)).sum(axis=1)
    np.testing.assert_allclose(corr, want, rtol=1e-5, atol=1e-3)


def test_logits_equal_the_dequantized_dot():
    """(acc - corr) * sx = sx * sum_b scale_b * sum_k (x_u - 64) q: the offset trick cancels
    exactly in real arithmetic, so the f32 result matches the float64 dequantized dot to f32
    rounding; and the row it selects is within quantization error of the exact best (the
    reference's own test, vocab_int8.rs:383-420: 4096 x 384, shortfall < 2% of full scale)."""
    rng = np.random.default_rng(1)
    vocab, d = 4096, 384
    w = rng.standard_normal((vocab, d)).astype(np.float32)
    x = rng.standard_normal((3, d)).astype(np.float32)
    q, sc, corr = og.vocab_quantize(w, 32)
    got = og.vocab_logits(q, sc, corr, x, 32)
    xu, sx = og.act_quantize(x)
    xs = (xu.astype(np.float64) - 64.0) * sx[:, None].astype(np.float64)
    deq = (q.reshape(vocab, 12, 32).astype(np.float64) * sc[:, :, None]).reshape(vocab, d)
    want = xs @ deq.T
    scale = np.abs(want).max()
    assert np.abs(got - want).max() < 1e-5 * scale
    exact = x.astype(np.float64) @ w.astype(np.float64).T
    for r in range(3):
        picked, best = int(np.argmax(got[r])), int(np.argmax(exact[r]))
        assert (exact[r, best] - exact[r, picked]) / np.abs(exact[r]).max() < 0.02


def test_gemv_f16_exact_matches_the_reference_test_bound():
    """f16_gemv.rs:203-229: against the f32-weight matmul the f16 GEMV agrees to 5e-3 of full
    scale at 1536 x 384."""
    rng = np.random.default_rng(2)
    w = rng.standard_normal((1536, 384)).astype(np.float32)
    x = rng.standard_normal((1, 384)).astype(np.float32)
    got = og.gemv_f16_exact(w.astype(np.float16), x)
    want = x.astype(np.float64) @ w.astype(np.float64).T
    assert np.abs(got - want).max() / np.abs(want).max() < 5e-3
