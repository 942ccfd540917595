"""The encoder-block oracle (oracle/encoder.py) against independent restatements (CPU only)."""

from __future__ import annotations

import numpy as np

from oracle import encoder as oenc
from oracle import kvcache as okv


def _weights(rng, n):
    w = lambda: (rng.standard_normal((n, n)) / np.sqrt(n)).astype(np.float32)
    b = lambda: rng.standard_normal(n).astype(np.float32)
    return w(), b(), w(), w(), b(), w(), b()


def test_prescaled_key_equals_the_decoder_formula():
    """Folding head_dim^-0.5 into Wk (EncoderAttention::load) gives Attention::attend's
    softmax(q s^2 k^T) v (text_decoder.rs:832-841), computed independently: heads split with
    split_heads, scores by the three-op restatement, heads merged, then the out-projection."""
    rng = np.random.default_rng(0)
    b, t, n, h = 2, 7, 16, 2
    x = rng.standard_normal((b, t, n)).astype(np.float32)
    wq, bq, wk, wv, bv, wo, bo = _weights(rng, n)
    got = oenc.encoder_attention(x, wq, bq, oenc.prescale_key(wk, h), wv, bv, wo, bo, h)
    q = x.astype(np.float64) @ wq.T + bq
    k = x.astype(np.float64) @ wk.T
    v = x.astype(np.float64) @ wv.T + bv
    att = okv.three_op_attend(okv.split_heads(q, h), okv.split_heads(k, h), okv.split_heads(v, h),
                              (n // h) ** -0.5)
    want = att.transpose(0, 2, 1, 3).reshape(b, t, n) @ wo.T.astype(np.float64) + bo
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)


def test_brute_force_loops():
    rng = np.random.default_rng(1)
    b, t, n, h = 1, 3, 4, 2
    hd = n // h
    x = rng.standard_normal((b, t, n)).astype(np.float32)
    wq, bq, wk, wv, bv, wo, bo = _weights(rng, n)
    got = oenc.encoder_attention(x, wq, bq, wk, wv, bv, wo, bo, h)
    for i in range(t):
        merged = []
        for hh in range(h):
            cols = range(hh * hd, (hh + 1) * hd)
            q = [sum(x[0, i, c] * wq[o, c] for c in range(n)) + bq[o] for o in cols]
            scores = [sum(q[a] * sum(wk[o, c] * x[0, j, c] for c in range(n))
                          for a, o in enumerate(cols)) for j in range(t)]
            mx = max(scores)
            e = [np.exp(s - mx) for s in scores]
            z = sum(e)
            for o in cols:
                merged.append(sum(e[j] / z * (sum(x[0, j, c] * wv[o, c] for c in range(n)) + bv[o])
                                  for j in range(t)))
        for o in range(n):
            want = sum(merged[c] * wo[o, c] for c in range(n)) + bo[o]
            assert abs(got[0, i, o] - want) < 1e-5


def test_batch_items_are_independent():
    rng = np.random.default_rng(2)
    b, t, n, h = 3, 5, 8, 2
    x = rng.standard_normal((b, t, n)).astype(np.float32)
    ws = _weights(rng, n)
    all_ = oenc.encoder_attention(x, *ws, h)
    for i in range(b):
        np.testing.assert_allclose(all_[i:i + 1], oenc.encoder_attention(x[i:i + 1], *ws, h),
                                   rtol=1e-6, atol=1e-6)
