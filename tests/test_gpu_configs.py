"""GPU parity at the full sizes the benchmark runs, through the launch shapes it runs.

Each test builds one workload of the benchmark at its full size (same shapes, dtypes, K layout,
scale and output dtype as its bench leg), states the launch plan ffai_attn_fwd takes for it
(kernel, workgroup shape, key splits), and checks the whole output against the oracle on the
same seeded, rounded inputs (f32 math on the rounded values), plus sampled rows against the
float64 closed form. Bars: 1e-4 max-abs for f32, 2e-2 for bf16.

Workloads:
* whisper-tiny encoder, B1 H6 T1500 D64, f32 (four-wave blocks, keys split);
* whisper-small encoder, B8 H12 T1500 D64, K x 2, in f32 (one workgroup per 128 rows, no key
  split: the f32 kernel's direct epilogue) and bf16 (four waves x 64 rows, the last round's
  items in key pieces);
* whisper-large-v3 encoder, B16 H20 T1500 D64, bf16 (one layer of the headline run);
* Qwen2-VL-2B-shape causal prefill, Hq12 Hkv2 D128 S4096, bf16, Q and K rotated per position
  by random 2-D rotations of dimension pairs (norm preserving), as rotary embedding leaves them
  (longest query blocks in two key pieces);
* the beam-5 whisper-medium decode step: self-attention over ragged bf16 caches (lengths
  U{1..448}) and cross-attention of 5 beams over 1500 shared frames.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from oracle import textbook
from ffai_amd import flash_attn as fa
from tests.helpers import TOL_BF16, TOL_F32, max_abs, round_bf16

pytestmark = pytest.mark.gpu

THREADS = 16


def _dev(x: np.ndarray, dtype, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(x)).to(device=device, dtype=dtype)


def _encoder_case(seed, b, h, t, d, dtype, k_mult=1.0):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((b, h, t, d), dtype=np.float32)
    kt = rng.standard_normal((b, h, d, t), dtype=np.float32) * np.float32(k_mult)
    v = rng.standard_normal((b, h, t, d), dtype=np.float32)
    if dtype == torch.bfloat16:
        q, kt, v = round_bf16(q), round_bf16(kt), round_bf16(v)
    return q, kt, v


def _run_encoder(gpu, q, kt, v, dtype, out_dtype, expect_plan):
    d = q.shape[3]
    scale = d ** -0.5
    qd, kd, vd = _dev(q, dtype, gpu), _dev(kt, dtype, gpu), _dev(v, dtype, gpu)
    out = torch.empty(q.shape, dtype=out_dtype, device=gpu)
    plan = fa.plan(qd, kd, vd, out, k_transposed=True, scale=scale)
    print("plan", plan)
    for key, val in expect_plan.items():
        if key == "shape" and val == "wave4x2":  # either kernel of the four-wave x 64-row shape
            assert plan[key] in ("wave4x2", "wave4x2x16"), plan
        else:
            assert plan[key] == val, (key, plan)
    assert fa.attention(qd, kd, vd, k_transposed=True, scale=scale, out=out) is not None
    got = out.float().cpu().numpy()
    want = oracle.attend_general(q, kt, v, k_transposed=True, scale=scale, threads=THREADS)
    tol = TOL_F32 if dtype == torch.float32 else TOL_BF16
    err = max_abs(got, want)
    # sampled rows against the float64 closed form: first and last rows, a 64-key tile edge, a
    # 256-row block edge, in the first and last (batch, head)
    rows = np.array([0, 1, 63, 64, 255, 256, 1023, 1024, 1499])
    b1, h1 = q.shape[0] - 1, q.shape[1] - 1
    cf = textbook.attention(q[[0, b1]][:, [0, h1]], kt[[0, b1]][:, [0, h1]],
                            v[[0, b1]][:, [0, h1]], k_transposed=True, scale=scale, rows=rows)
    err_cf = max_abs(got[[0, b1]][:, [0, h1]][:, :, rows], cf)
    print(f"{tuple(q.shape)} {dtype}: vs oracle {err:.3e}, sampled rows vs closed form {err_cf:.3e}")
    assert err < tol
    assert err_cf < tol


def test_whisper_tiny_f32_full_size(gpu):
    q, kt, v = _encoder_case(1, 1, 6, 1500, 64, torch.float32)
    _run_encoder(gpu, q, kt, v, torch.float32, torch.float32,
                 {"kernel": "fwd", "shape": "wave4", "splits": 6, "split_items": (0, 72)})


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_whisper_small_full_size(gpu, dtype):
    """B8 H12 T1500 with K x 2. f32: 1152 workgroups of 128 rows, keys whole (the direct store
    of the f32 kernel's epilogue); bf16: four waves x 64 rows, 576 items of which the last 64
    (the round past the 512 resident workgroups) run in 4 key pieces merged in the launch."""
    q, kt, v = _encoder_case(2, 8, 12, 1500, 64, dtype, k_mult=2.0)
    if dtype == torch.float32:
        expect = {"kernel": "fwd", "shape": "wave4", "splits": 1}
    else:
        expect = {"kernel": "fwd", "shape": "wave4x2", "splits": 4, "split_items": (512, 576)}
    _run_encoder(gpu, q, kt, v, dtype, dtype, expect)


def test_whisper_large_v3_full_size(gpu):
    q, kt, v = _encoder_case(4, 16, 20, 1500, 64, torch.bfloat16)
    _run_encoder(gpu, q, kt, v, torch.bfloat16, torch.bfloat16,
                 {"kernel": "fwd", "shape": "wave4x2", "splits": 2, "workgroups": 2048,
                  "split_items": (1792, 1920)})


def _rotate_pairs(x: np.ndarray, rng) -> np.ndarray:
    """Rotate dimension pairs (2i, 2i+1) of every position by an angle ~ U[0, 2 pi), one angle
    per (position, pair), shared by the heads: norm-preserving, as rotary embedding is."""
    t, d = x.shape[2], x.shape[3]
    ang = rng.uniform(0.0, 2.0 * np.pi, (t, d // 2))
    c, s = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    y = np.empty_like(x)
    y[..., 0::2] = x[..., 0::2] * c - x[..., 1::2] * s
    y[..., 1::2] = x[..., 0::2] * s + x[..., 1::2] * c
    return y


def test_qwen2_vl_causal_prefill_full_size(gpu):
    """Hq12 over Hkv2, head_dim 128, S4096, causal, K as rows (a decoder cache's layout)."""
    rng = np.random.default_rng(5)
    s, d = 4096, 128
    q = rng.standard_normal((1, 12, s, d), dtype=np.float32)
    k = rng.standard_normal((1, 2, s, d), dtype=np.float32)
    v = rng.standard_normal((1, 2, s, d), dtype=np.float32)
    rot = np.random.default_rng(55)
    q, k = _rotate_pairs(q, rot), _rotate_pairs(k, rot)
    np.testing.assert_allclose(np.linalg.norm(q, axis=-1),
                               np.linalg.norm(_rotate_pairs(q, np.random.default_rng(7)), axis=-1),
                               rtol=1e-5)
    q, k, v = round_bf16(q), round_bf16(k), round_bf16(v)
    scale = d ** -0.5
    bf = torch.bfloat16
    qd, kd, vd = _dev(q, bf, gpu), _dev(k, bf, gpu), _dev(v, bf, gpu)
    out = torch.empty(1, 12, s, d, dtype=bf, device=gpu)
    plan = fa.plan(qd, kd, vd, out, scale=scale, causal=True)
    print("plan", plan)
    # 384 items (12 heads x 32 query blocks of 128 rows) dispatched longest first; the 192
    # longest (more than half the longest's keys) in 2 pieces merged in the launch
    assert plan["kernel"] == "fwd" and plan["shape"] == "wave4" and plan["splits"] == 2
    assert plan["split_items"] == (0, 192)
    assert fa.attention(qd, kd, vd, scale=scale, causal=True, out=out) is not None
    got = out.float().cpu().numpy()
    want = oracle.attend_general(q, k, v, k_transposed=False, scale=scale, causal=True,
                                 threads=THREADS)
    err = max_abs(got, want)
    # the first row sees one key; rows at block edges; the last row sees all 4096
    rows = np.array([0, 1, 127, 128, 2047, 2048, 4095])
    cf = textbook.attention(q, k, v, scale=scale, causal=True, rows=rows)
    err_cf = max_abs(got[:, :, rows], cf)
    assert max_abs(got[:, :, 0], v[:, np.arange(12) // 6, 0]) < TOL_BF16  # row 0 = value 0
    print(f"qwen2-vl prefill: vs oracle {err:.3e}, sampled rows vs closed form {err_cf:.3e}")
    assert err < TOL_BF16
    assert err_cf < TOL_BF16


def test_beam5_decode_step_shapes(gpu):
    """One layer of the bench's beam-5 step: self-attention (5 beams x 16 heads over ragged bf16
    caches of capacity 448, lengths U{1..448}) and cross-attention (the 5 beams as the query rows
    of one 16-head unit each over 1500 shared frames, K transposed and as rows), f32 outputs."""
    rng = np.random.default_rng(3)
    beams, h, d, cap, frames = 5, 16, 64, 448, 1500
    scale = d ** -0.5
    bf = torch.bfloat16
    lens = rng.integers(1, cap + 1, beams).astype(np.int32)
    lens[0] = cap  # one full cache
    q = round_bf16(rng.standard_normal((beams, h, 1, d), dtype=np.float32))
    k = round_bf16(rng.standard_normal((beams, h, cap, d), dtype=np.float32))
    v = round_bf16(rng.standard_normal((beams, h, cap, d), dtype=np.float32))
    qd, kd, vd = _dev(q, bf, gpu), _dev(k, bf, gpu), _dev(v, bf, gpu)
    ld = torch.from_numpy(lens).to(gpu)
    out = torch.empty(beams, h, 1, d, device=gpu)
    plan = fa.plan(qd, kd, vd, out, scale=scale, kv_lens=ld)
    print("self plan", plan)
    assert plan["kernel"] == "decode"
    assert fa.attention(qd, kd, vd, scale=scale, kv_lens=ld, out=out) is not None
    want = oracle.attend_general(q, k, v, k_transposed=False, scale=scale, kv_lens=lens)
    err = max_abs(out.cpu().numpy(), want)
    print(f"beam-5 self-attention: {err:.3e}")
    assert err < TOL_BF16

    qx = round_bf16(rng.standard_normal((1, h, beams, d), dtype=np.float32))
    kt = round_bf16(rng.standard_normal((1, h, d, frames), dtype=np.float32))
    vx = round_bf16(rng.standard_normal((1, h, frames, d), dtype=np.float32))
    want = oracle.attend_general(qx, kt, vx, k_transposed=True, scale=scale)
    # the cache's K either transposed (the reference's layout) or as rows (the bench's); both
    # layouts feed the MFMAs the same operands in the same order, so their outputs are equal
    outs = []
    for k_transposed in (True, False):
        kk = kt if k_transposed else np.ascontiguousarray(np.swapaxes(kt, 2, 3))
        qd, kd, vd = _dev(qx, bf, gpu), _dev(kk, bf, gpu), _dev(vx, bf, gpu)
        ox = torch.empty(1, h, beams, d, device=gpu)
        plan = fa.plan(qd, kd, vd, ox, k_transposed=k_transposed, scale=scale)
        print("cross plan", plan)
        assert plan["kernel"] == "decode" and plan["splits"] > 1
        assert fa.attention(qd, kd, vd, k_transposed=k_transposed, scale=scale, out=ox) is not None
        err = max_abs(ox.cpu().numpy(), want)
        print(f"beam-5 cross-attention (k_transposed={k_transposed}): {err:.3e}")
        assert err < TOL_BF16
        outs.append(ox)
    assert torch.equal(outs[0], outs[1])
