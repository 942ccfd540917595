"""GPU parity: the HIP kernels, called through the C ABI, against the CPU oracle.

Tolerances (max-abs): 1e-4 for f32, 2e-2 for bf16/f16 -- the bar stated for this path.
bf16/f16 cases feed the oracle the SAME rounded values (upcast to f32), so the comparison
measures the kernel's arithmetic, not the input rounding.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from oracle import textbook
from ffai_amd import flash_attn as fa
from tests.helpers import TOL_BF16, TOL_F32, max_abs, randn, round_bf16, round_f16

pytestmark = pytest.mark.gpu


def _dev(x: np.ndarray, dtype, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(x)).to(device=device, dtype=dtype)


def _host(t: torch.Tensor) -> np.ndarray:
    return t.float().cpu().numpy()


# ---------------------------------------------------------------------------------------------
# Reference-surface mirrors (f32, batch 1, head_dim 64)
# ---------------------------------------------------------------------------------------------

def test_attend_matches_reference_unit_test_shape(gpu):
    """flash_attn.rs:1005-1021 matches_three_op_path: H=4, T=512, f32, unscaled, < 1e-4."""
    rng = np.random.default_rng(1005)
    q, kt, v = randn(rng, (1, 4, 512, 64)), randn(rng, (1, 4, 64, 512)), randn(rng, (1, 4, 512, 64))
    out = fa.attend(_dev(q, torch.float32, gpu), _dev(kt, torch.float32, gpu),
                    _dev(v, torch.float32, gpu))
    assert out is not None
    got = _host(out)
    want = oracle.attend_f32(q, kt, v)
    three_op = textbook.attention(q, kt, v, k_transposed=True)
    print("attend 4x512 f32: vs oracle", max_abs(got, want), "vs closed form", max_abs(got, three_op))
    assert max_abs(got, want) < TOL_F32
    assert max_abs(got, three_op) < TOL_F32


@pytest.mark.parametrize("seq", [256, 300, 1500])
def test_attend_merged_tiny_encoder(gpu, seq):
    """MergedAttnOp at the whisper-tiny shape (6 heads) with scale 1/8 folded into q, as the
    reference probe does (examples/flash_probe.rs:375-405); ragged tails at 300 and 1500."""
    rng = np.random.default_rng(seq)
    h = 6
    q = randn(rng, (1, h, seq, 64)) * np.float32(1 / 8)
    kt, v = randn(rng, (1, h, 64, seq)), randn(rng, (1, h, seq, 64))
    out = fa.attend_merged(_dev(q, torch.float32, gpu), _dev(kt, torch.float32, gpu),
                           _dev(v, torch.float32, gpu))
    assert out is not None and tuple(out.shape) == (1, seq, h * 64)
    got = _host(out)
    want = oracle.attend_merged(q, kt, v)
    err = max_abs(got, want)
    print(f"attend_merged H6 T{seq}: {err:.3e}")
    assert err < TOL_F32


@pytest.mark.parametrize("keys", [8, 37, 448, 1500])
def test_attend_decode_f32(gpu, keys):
    """FlashAttnOp f32 decode arm (qlen == 1), xattn_head: 6 heads."""
    rng = np.random.default_rng(keys)
    q = randn(rng, (1, 6, 1, 64)) * np.float32(0.125)
    kt, v = randn(rng, (1, 6, 64, keys)), randn(rng, (1, 6, keys, 64))
    out = fa.attend(_dev(q, torch.float32, gpu), _dev(kt, torch.float32, gpu),
                    _dev(v, torch.float32, gpu))
    assert out is not None
    err = max_abs(_host(out), oracle.attend_f32(q, kt, v))
    print(f"decode f32 K{keys}: {err:.3e}")
    assert err < TOL_F32


@pytest.mark.parametrize("keys", [37, 1500])
def test_attend_decode_f16_kv(gpu, keys):
    """FlashAttnOp f16-K/V decode arm (xattn_head_f16): q f32, K/V f16, f32 math."""
    rng = np.random.default_rng(100 + keys)
    q = randn(rng, (1, 6, 1, 64)) * np.float32(0.125)
    kt = randn(rng, (1, 6, 64, keys)).astype(np.float16)
    v = randn(rng, (1, 6, keys, 64)).astype(np.float16)
    out = fa.attend(_dev(q, torch.float32, gpu), _dev(kt, torch.float16, gpu),
                    _dev(v, torch.float16, gpu))
    assert out is not None
    err = max_abs(_host(out), oracle.attend_f16kv(q, kt, v))
    print(f"decode f16kv K{keys}: {err:.3e}")
    assert err < TOL_F32


# ---------------------------------------------------------------------------------------------
# General descriptor path (extension of the reference: batch, bf16/f16, GQA, D=128, causal)
# ---------------------------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("k_transposed", [True, False])
@pytest.mark.parametrize("out_f32", [True, False])
def test_encoder_16bit(gpu, dtype, k_transposed, out_f32):
    """Encoder shape in bf16/f16 with K x 2 (the whisper-small stress case), ragged T=300."""
    rng = np.random.default_rng(2)
    b, h, t, d = 2, 3, 300, 64
    rnd = round_bf16 if dtype == torch.bfloat16 else round_f16
    q = rnd(randn(rng, (b, h, t, d)))
    k = rnd(randn(rng, (b, h, t, d)) * np.float32(2.0))
    v = rnd(randn(rng, (b, h, t, d)))
    scale = d ** -0.5
    kk = np.ascontiguousarray(np.swapaxes(k, 2, 3)) if k_transposed else k
    out = fa.attention(_dev(q, dtype, gpu), _dev(kk, dtype, gpu), _dev(v, dtype, gpu),
                       k_transposed=k_transposed, scale=scale,
                       out_dtype=torch.float32 if out_f32 else dtype)
    assert out is not None
    want = oracle.attend_general(q, k, v, k_transposed=False, scale=scale)
    err = max_abs(_host(out), want)
    print(f"encoder {dtype} kt={k_transposed} f32out={out_f32}: {err:.3e}")
    assert err < TOL_BF16


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("k_transposed", [True, False])
def test_scores_far_above_the_first_subtile(gpu, dtype, k_transposed):
    """The 16-bit kernel takes its reference max from each row's first 32 keys and raises it
    only when a subtile's weights would leave [0, 2^64]. Scores here jump twice: by ~58 log2
    units at keys 200-259 (weights near 2^58, accepted as they are) and by ~173 at keys 640-699
    (weights past f32's range, so that subtile is redone against its exact max and the
    accumulator rescaled). Without the redo the second jump gives inf and then NaN."""
    rng = np.random.default_rng(77)
    b, h, t, d = 1, 2, 1000, 64
    rnd = round_bf16 if dtype == torch.bfloat16 else round_f16
    u = np.zeros(d, np.float32)
    u[3] = 1.0
    q = rnd(8.0 * u + 0.05 * randn(rng, (b, h, t, d)))
    amp = np.full(t, 0.1, np.float32)
    amp[200:260] = 40.0
    amp[640:700] = 120.0
    k = rnd(amp[None, None, :, None] * u + 0.05 * randn(rng, (b, h, t, d)))
    v = rnd(randn(rng, (b, h, t, d)))
    scale = 0.125
    kk = np.ascontiguousarray(np.swapaxes(k, 2, 3)) if k_transposed else k
    out = fa.attention(_dev(q, dtype, gpu), _dev(kk, dtype, gpu), _dev(v, dtype, gpu),
                       k_transposed=k_transposed, scale=scale, out_dtype=torch.float32)
    got = _host(out)
    assert np.isfinite(got).all()
    want = oracle.attend_general(q, k, v, k_transposed=False, scale=scale)
    err = max_abs(got, want)
    print(f"score jumps {dtype} kt={k_transposed}: {err:.3e}")
    assert err < TOL_BF16


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("sign", [1.0, -1.0])
def test_first_subtile_outside_the_fast_window(gpu, dtype, sign):
    """A wave takes 0 as its reference max only when every row max of its first 32 keys lies
    in [-64, 32] log2 units. Here every score sits near +-87 log2 units, so the wave keeps the
    first subtile's max instead (well above: weights would overflow; well below: they would
    underflow to 0 and the rows would come out empty)."""
    rng = np.random.default_rng(31)
    b, h, t, d = 1, 2, 700, 64
    rnd = round_bf16 if dtype == torch.bfloat16 else round_f16
    u = np.zeros(d, np.float32)
    u[5] = 1.0
    q = rnd(8.0 * u + 0.05 * randn(rng, (b, h, t, d)))
    k = rnd(np.float32(sign * 60.0) * u + randn(rng, (b, h, t, d)))
    v = rnd(randn(rng, (b, h, t, d)))
    scale = 0.125
    out = fa.attention(_dev(q, dtype, gpu), _dev(k, dtype, gpu), _dev(v, dtype, gpu),
                       scale=scale, out_dtype=torch.float32)
    got = _host(out)
    assert np.isfinite(got).all()
    want = oracle.attend_general(q, k, v, k_transposed=False, scale=scale)
    err = max_abs(got, want)
    print(f"outside the fast window {dtype} sign={sign}: {err:.3e}")
    assert err < TOL_BF16


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("row_max", [-40.0, -20.0])
@pytest.mark.parametrize("shape", [(2, 64, 300), (1, 2, 300), (1, 16, 200)])
def test_scores_shifted_far_below_zero(gpu, dtype, row_max, shape):
    """Softmax ignores a shift shared by every score of a row. Q's dimension 0 is set to c and
    K's dimension 0 to -1 for every key, which moves every score of every row by -c * scale;
    c puts the row maxima near `row_max` log2 units, where exp2 of a raw score is below f16's
    normal range (2^-14) or flushes to 0 (2^-24). The output must still equal the oracle on the
    unshifted inputs (dimension 0 zero in both), in both 16-bit types and in the three launch
    shapes: four waves x 64 rows (2 x 64 heads), four waves x 32 rows with split keys, one wave
    x 32 rows (200 rows)."""
    rng = np.random.default_rng(33)
    b, h, t = shape
    d = 64
    rnd = round_bf16 if dtype == torch.bfloat16 else round_f16
    scale = 0.125
    q = rnd(randn(rng, (b, h, t, d)))
    k = rnd(randn(rng, (b, h, t, d)))
    v = rnd(randn(rng, (b, h, t, d)))
    q[..., 0] = 0.0
    k[..., 0] = 0.0
    # unshifted row maxima are a few log2 units above 0: shift them to about row_max
    c = np.float32((3.0 - row_max) / (scale * np.log2(np.e)))
    qs, ks = q.copy(), k.copy()
    qs[..., 0] = rnd(np.full(q.shape[:3], c, np.float32))
    ks[..., 0] = -1.0
    shifted = textbook.attention(qs, ks, v, scale=scale, rows=np.arange(32))
    unshifted = textbook.attention(q, k, v, scale=scale, rows=np.arange(32))
    assert max_abs(shifted, unshifted) < 1e-9  # the identity itself, in float64
    s_max = (np.einsum("bhtd,bhsd->bhts", qs[:, :, :32], ks[:, :, :32]).max(-1) * scale *
             np.log2(np.e))
    assert np.all(s_max < row_max + 6) and np.all(s_max > row_max - 6), (s_max.min(), s_max.max())
    out = fa.attention(_dev(qs, dtype, gpu), _dev(ks, dtype, gpu), _dev(v, dtype, gpu),
                       scale=scale, out_dtype=torch.float32)
    got = _host(out)
    assert np.isfinite(got).all()
    want = oracle.attend_general(q, k, v, k_transposed=False, scale=scale)
    err = max_abs(got, want)
    print(f"shifted scores {dtype} row max ~{row_max} shape {shape}: {err:.3e}")
    assert err < TOL_BF16


@pytest.mark.parametrize("k_transposed", [True, False])
def test_f16_query_beyond_the_folding_range(gpu, k_transposed):
    """The 16-bit kernel folds scale * log2(e) into Q. With scale 1, f16 query elements above
    65504 / log2(e) ~ 45400 would overflow once folded, so such a wave keeps Q as given and
    scales every score instead."""
    rng = np.random.default_rng(32)
    b, h, t, d = 1, 2, 400, 64
    u = np.zeros(d, np.float32)
    u[7] = 1.0
    q = round_f16(50000.0 * u + randn(rng, (b, h, t, d)))
    k = round_f16(np.float32(2e-4) * randn(rng, (b, h, t, d)))  # scores ~ N(0, 10)
    v = round_f16(randn(rng, (b, h, t, d)))
    assert np.abs(q).max() * 1.4426950408889634 > 65504.0
    kk = np.ascontiguousarray(np.swapaxes(k, 2, 3)) if k_transposed else k
    out = fa.attention(_dev(q, torch.float16, gpu), _dev(kk, torch.float16, gpu),
                       _dev(v, torch.float16, gpu), k_transposed=k_transposed, scale=1.0,
                       out_dtype=torch.float32)
    got = _host(out)
    assert np.isfinite(got).all()
    want = oracle.attend_general(q, k, v, k_transposed=False, scale=1.0)
    err = max_abs(got, want)
    print(f"f16 q beyond the folding range kt={k_transposed}: {err:.3e}")
    assert err < TOL_BF16


def _views_with_high_low_word(gpu, arrays, dtype):
    """Device copies of `arrays` placed in one buffer at an address whose low 32 bits have bit
    31 set (the DMA path builds its 64-bit scalar base from two 32-bit halves)."""
    esz = torch.tensor([], dtype=dtype).element_size()
    sizes = [((a.size * esz + 255) // 256) * 256 for a in arrays]
    # start exactly at 2^31 (mod 2^32): the whole region then keeps bit 31 of the low word
    buf = torch.empty(2 ** 32 + sum(sizes) + 4096, dtype=torch.uint8, device=gpu)
    lo = buf.data_ptr() & 0xFFFFFFFF
    off = (2 ** 31 - lo) % (2 ** 32)
    assert off % 256 == 0  # allocations are at least 256-byte aligned
    out = []
    for a, n in zip(arrays, sizes):
        t = buf[off:off + a.size * esz].view(dtype).view(a.shape)
        t.copy_(torch.from_numpy(np.ascontiguousarray(a)).to(dtype))
        assert t.data_ptr() & 0x80000000
        out.append(t)
        off += n
    return buf, out


@pytest.mark.parametrize("shape", [(2, 3, 300), (8, 16, 512)])
def test_operands_at_high_addresses(gpu, shape):
    """Regression: operands whose addresses have bit 31 of the low word set, through the
    one-wave (B2 H3 T300) and the 4-wave x 2-block (B8 H16 T512) encoder variants."""
    rng = np.random.default_rng(31)
    b, h, t = shape
    d = 64
    q = round_bf16(randn(rng, (b, h, t, d)))
    kt = round_bf16(randn(rng, (b, h, d, t)))
    v = round_bf16(randn(rng, (b, h, t, d)))
    buf, (qd, ktd, vd) = _views_with_high_low_word(gpu, [q, kt, v], torch.bfloat16)
    out = fa.attention(qd, ktd, vd, k_transposed=True, scale=0.125, out_dtype=torch.float32)
    torch.cuda.synchronize()
    del buf
    want = oracle.attend_general(q, kt, v, k_transposed=True, scale=0.125)
    err = max_abs(_host(out), want)
    print(f"high addresses {shape}: {err:.3e}")
    assert err < TOL_BF16


def test_encoder_f32_batched_rows_layout(gpu):
    rng = np.random.default_rng(3)
    b, h, t, d = 2, 2, 700, 64
    q, k, v = randn(rng, (b, h, t, d)), randn(rng, (b, h, t, d)), randn(rng, (b, h, t, d))
    out = fa.attention(_dev(q, torch.float32, gpu), _dev(k, torch.float32, gpu),
                       _dev(v, torch.float32, gpu), scale=0.125)
    err = max_abs(_host(out), oracle.attend_general(q, k, v, k_transposed=False, scale=0.125))
    print(f"encoder f32 rows: {err:.3e}")
    assert err < TOL_F32


@pytest.mark.parametrize("d", [64, 128])
def test_causal_gqa(gpu, d):
    """Causal prefill with grouped K/V heads (Hq=4, Hkv=2), S=130 (ragged), bf16."""
    rng = np.random.default_rng(5 + d)
    b, hq, hkv, s = 1, 4, 2, 130
    q = round_bf16(randn(rng, (b, hq, s, d)))
    k = round_bf16(randn(rng, (b, hkv, s, d)))
    v = round_bf16(randn(rng, (b, hkv, s, d)))
    scale = d ** -0.5
    out = fa.attention(_dev(q, torch.bfloat16, gpu), _dev(k, torch.bfloat16, gpu),
                       _dev(v, torch.bfloat16, gpu), scale=scale, causal=True,
                       out_dtype=torch.float32)
    want = oracle.attend_general(q, k, v, k_transposed=False, scale=scale, causal=True)
    err = max_abs(_host(out), want)
    print(f"causal gqa d{d}: {err:.3e}")
    assert err < TOL_BF16


def test_causal_with_offset(gpu):
    """Prompt-continuation shape: 40 new queries at absolute offset 90 over 130 keys."""
    rng = np.random.default_rng(9)
    b, h, tq, tk, d = 2, 2, 40, 130, 64
    q = round_bf16(randn(rng, (b, h, tq, d)))
    k = round_bf16(randn(rng, (b, h, tk, d)))
    v = round_bf16(randn(rng, (b, h, tk, d)))
    out = fa.attention(_dev(q, torch.bfloat16, gpu), _dev(k, torch.bfloat16, gpu),
                       _dev(v, torch.bfloat16, gpu), scale=0.125, causal=True, q_offset=90,
                       out_dtype=torch.float32)
    want = textbook.attention(q, k, v, scale=0.125, causal=True, q_offset=90)
    err = max_abs(_host(out), want)
    print(f"causal offset: {err:.3e}")
    assert err < TOL_BF16


def test_beam_cross_attention_shared_kv(gpu):
    """Beam-search cross-attention: 5 beams read ONE K/V of 1500 frames; the beams are the query
    rows of a single batch item, so K/V streams once (whisper-medium: 16 heads)."""
    rng = np.random.default_rng(3)
    beams, h, t, d = 5, 16, 1500, 64
    q = round_bf16(randn(rng, (beams, h, 1, d)))
    kt = round_bf16(randn(rng, (1, h, d, t)))
    v = round_bf16(randn(rng, (1, h, t, d)))
    qd = _dev(q, torch.bfloat16, gpu)
    out = torch.empty(beams, h, 1, d, dtype=torch.float32, device=gpu)
    # (beams, H, 1, D) viewed as (1, H, beams, D): beam rows H*D apart
    res = fa.attention(qd.permute(2, 1, 0, 3), _dev(kt, torch.bfloat16, gpu),
                       _dev(v, torch.bfloat16, gpu), k_transposed=True, scale=0.125,
                       out=out.permute(2, 1, 0, 3))
    assert res is not None
    want = oracle.attend_general(np.swapaxes(q, 0, 2), kt, v, k_transposed=True, scale=0.125)
    err = max_abs(_host(out), np.swapaxes(want, 0, 2))
    print(f"beam cross-attn: {err:.3e}")
    assert err < TOL_BF16


def test_beam_self_attention_ragged(gpu):
    """Decoder self-attention: 5 beams, each with its own cache of L_b keys (capacity 448)."""
    rng = np.random.default_rng(33)
    beams, h, cap, d = 5, 16, 448, 64
    lens = np.array([1, 9, 200, 447, 448], np.int32)
    q = round_bf16(randn(rng, (beams, h, 1, d)))
    k = round_bf16(randn(rng, (beams, h, cap, d)))
    v = round_bf16(randn(rng, (beams, h, cap, d)))
    out = fa.attention(_dev(q, torch.bfloat16, gpu), _dev(k, torch.bfloat16, gpu),
                       _dev(v, torch.bfloat16, gpu), scale=0.125,
                       kv_lens=torch.from_numpy(lens).to(gpu), out_dtype=torch.float32)
    want = oracle.attend_general(q, k, v, k_transposed=False, scale=0.125, kv_lens=lens)
    err = max_abs(_host(out), want)
    print(f"beam self-attn ragged: {err:.3e}")
    assert err < TOL_BF16


def test_whisper_large_shape_sampled_rows(gpu):
    """Full whisper-large-v3 layer shape (B16 H20 T1500 bf16): every row computed on the GPU,
    sampled rows checked against the float64 closed form on the same rounded inputs."""
    rng = np.random.default_rng(4)
    b, h, t, d = 16, 20, 1500, 64
    g = torch.Generator(device="cpu").manual_seed(4)
    q = torch.randn(b, h, t, d, generator=g).to(torch.bfloat16)
    kt = torch.randn(b, h, d, t, generator=g).to(torch.bfloat16)
    v = torch.randn(b, h, t, d, generator=g).to(torch.bfloat16)
    out = fa.attention(q.to(gpu), kt.to(gpu), v.to(gpu), k_transposed=True, scale=0.125,
                       out_dtype=torch.bfloat16)
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    rows = np.sort(rng.choice(t, size=24, replace=False))
    rows[0], rows[-1] = 0, t - 1
    bi = [0, 7, 15]
    want = textbook.attention(q[bi].float().numpy(), kt[bi].float().numpy(),
                              v[bi].float().numpy(), k_transposed=True, scale=0.125, rows=rows)
    err = max_abs(got[bi][:, :, rows], want)
    print(f"large-v3 sampled rows: {err:.3e}")
    assert err < TOL_BF16


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("k_transposed", [True, False])
@pytest.mark.parametrize("b,h", [(2, 3), (8, 32)])  # one-wave / four-wave x 32, four-wave x 64
def test_16bit_output_rows_paired_and_unpaired(gpu, dtype, k_transposed, b, h):
    """Head_dim 64 with a 16-bit output: rows that admit 16-byte stores are written by lane
    pairs exchanging halves (whole 8-element runs); rows that do not (here a row stride of 68
    elements: 8-byte but not 16-byte aligned) by each lane's own 4-element runs. Both carry the
    same values, so the two outputs must agree bit for bit, and both match the oracle. 300
    query rows: the last 32-row block is partly past the end (rows 288-299 written, 300-319
    not)."""
    rng = np.random.default_rng(64)
    rnd = round_bf16 if dtype == torch.bfloat16 else round_f16
    t, tk, d = 300, 333, 64
    q = rnd(randn(rng, (b, h, t, d)))
    k = rnd(randn(rng, (b, h, tk, d)))
    v = rnd(randn(rng, (b, h, tk, d)))
    kk = np.swapaxes(k, 2, 3) if k_transposed else k
    qd, kd, vd = _dev(q, dtype, gpu), _dev(kk, dtype, gpu), _dev(v, dtype, gpu)
    paired = torch.empty(b, h, t, d, dtype=dtype, device=gpu)
    wide = torch.full((b, h, t, 68), 7.0, dtype=dtype, device=gpu)  # 68: 136-byte rows
    unpaired = wide[..., :d]
    if b == 8:
        assert fa.plan(qd, kd, vd, paired, k_transposed=k_transposed,
                       scale=0.125)["shape"] == "wave4x2"
    for out in (paired, unpaired):
        fa.attention(qd, kd, vd, k_transposed=k_transposed, scale=0.125, out=out)
    assert torch.equal(paired.view(torch.int16), unpaired.contiguous().view(torch.int16))
    assert torch.all(wide[..., d:] == 7.0)  # nothing written past each row's 64 elements
    want = oracle.attend_general(q, k, v, k_transposed=False, scale=0.125)
    err = max_abs(_host(paired), want)
    print(f"16-bit output rows {dtype} kt={k_transposed}: {err:.3e}")
    assert err < TOL_BF16
