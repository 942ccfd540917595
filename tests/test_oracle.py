"""Pins for the CPU oracle (CPU only).

The reference (Rust) cannot be built here and ships no attention fixtures, so each oracle
function is pinned by checks whose answers the mathematics fixes:

* the closed form softmax(Q K^T) V in float64 -- the reference's own test oracle
  (flash_attn.rs:1005-1021, < 1e-4) -- on seeded inputs, including ragged tails;
* the exp polynomial against math.exp with the truncation bound of its series;
* invariants: uniform scores give the mean of V, one dominant key gives its V row, key
  permutation does nothing, the output is linear in V, the merged layout is a pure relayout;
* brute force in plain Python loops on tiny inputs;
* the committed golden vectors (tests/golden/);
* planted mistakes (oracle.plant_fault): each one must make at least one check fail.
"""

from __future__ import annotations

import glob
import math
import os

import numpy as np
import pytest

import oracle
from oracle import textbook
from tests.helpers import max_abs, randn

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(autouse=True)
def _faithful_oracle():
    oracle.plant_fault(0)
    yield
    oracle.plant_fault(0)


# ---------------------------------------------------------------------------------------------
# exp polynomial (flash_attn.rs:553-571)
# ---------------------------------------------------------------------------------------------

def _exp_bound() -> float:
    # Degree-5 Taylor series of 2^f on |f| <= 1/2: remainder <= (ln2/2)^6/6! * 2^(1/2), relative
    # to 2^f >= 2^(-1/2); plus a few f32 roundings.
    r = (math.log(2) / 2) ** 6 / math.factorial(6) * math.sqrt(2) / (2 ** -0.5)
    return r + 8 * 2.0 ** -24


def test_exp_poly_within_series_bound():
    x = np.concatenate([np.linspace(-87.0, 0.0, 400_001, dtype=np.float32),
                        np.linspace(-2.0, 2.0, 100_001, dtype=np.float32)])
    y = oracle.exp_poly(x).astype(np.float64)
    rel = np.abs(y / np.exp(x.astype(np.float64)) - 1.0)
    assert rel.max() < _exp_bound(), rel.max()
    # the bound is nearly attained at the series' edge (f = +-1/2), so a lost term shows
    assert rel.max() > 0.25 * _exp_bound()


def test_exp_poly_exact_points_and_clamp():
    assert oracle.exp_poly(np.array([0.0], np.float32))[0] == 1.0
    y = oracle.exp_poly(np.array([-87.0, -100.0, -1e30], np.float32))
    assert y[0] == y[1] == y[2] > 0.0  # clamped at -87 (flash_attn.rs:554), never 0 or denormal


# ---------------------------------------------------------------------------------------------
# encoder tiling (flash_head_strided and its callees)
# ---------------------------------------------------------------------------------------------

@pytest.mark.parametrize("h,t,scale", [(4, 512, 1.0), (2, 300, 0.125), (1, 257, 0.125),
                                       (3, 64, 1.0), (1, 5, 0.5)])
def test_encoder_matches_closed_form(h, t, scale):
    rng = np.random.default_rng(t)
    q = randn(rng, (1, h, t, 64)) * np.float32(scale)
    kt, v = randn(rng, (1, h, 64, t)), randn(rng, (1, h, t, 64))
    got = oracle.attend_f32(q, kt, v)
    want = textbook.attention(q, kt, v, k_transposed=True)
    assert max_abs(got, want) < 3e-5  # the reference's test bar is 1e-4


def test_encoder_whisper_tiny_full_layer():
    rng = np.random.default_rng(1500)
    h, t = 6, 1500
    q = randn(rng, (1, h, t, 64)) * np.float32(0.125)
    kt, v = randn(rng, (1, h, 64, t)), randn(rng, (1, h, t, 64))
    got = oracle.attend_f32(q, kt, v)
    rows = np.array([0, 1, 63, 64, 255, 256, 1023, 1024, 1279, 1280, 1499])
    want = textbook.attention(q, kt, v, k_transposed=True, rows=rows)
    assert max_abs(got[:, :, rows], want) < 1e-5


def test_merged_is_a_relayout():
    """MergedAttnOp writes head h into columns h*64..h*64+63 of each row (proofs.rs:205-248)."""
    rng = np.random.default_rng(7)
    q, kt, v = randn(rng, (1, 3, 300, 64)), randn(rng, (1, 3, 64, 300)), randn(rng, (1, 3, 300, 64))
    merged = oracle.attend_merged(q, kt, v)
    plain = oracle.attend_f32(q, kt, v)
    assert np.array_equal(merged.reshape(1, 300, 3, 64).transpose(0, 2, 1, 3), plain)


def test_uniform_scores_average_v():
    rng = np.random.default_rng(8)
    q = randn(rng, (1, 2, 300, 64))
    kt = np.zeros((1, 2, 64, 300), np.float32)
    v = randn(rng, (1, 2, 300, 64))
    got = oracle.attend_f32(q, kt, v)
    assert max_abs(got, np.broadcast_to(v.mean(axis=2, keepdims=True), got.shape)) < 1e-5


def test_dominant_key_selects_its_value():
    rng = np.random.default_rng(9)
    t = 300
    q = np.zeros((1, 1, t, 64), np.float32)
    q[..., 0] = 1.0
    kt = np.zeros((1, 1, 64, t), np.float32)
    kt[0, 0, 0, 271] = 200.0  # every query scores key 271 at 200, the rest at 0
    v = randn(rng, (1, 1, t, 64))
    got = oracle.attend_f32(q, kt, v)
    assert max_abs(got[0, 0], np.broadcast_to(v[0, 0, 271], (t, 64))) < 1e-6


def test_key_permutation_invariance_and_linearity():
    rng = np.random.default_rng(10)
    t = 300
    q = randn(rng, (1, 2, t, 64)) * np.float32(0.125)
    kt, v, v2 = randn(rng, (1, 2, 64, t)), randn(rng, (1, 2, t, 64)), randn(rng, (1, 2, t, 64))
    base = oracle.attend_f32(q, kt, v)
    perm = rng.permutation(t)
    got = oracle.attend_f32(q, np.ascontiguousarray(kt[..., perm]),
                            np.ascontiguousarray(v[:, :, perm]))
    assert max_abs(got, base) < 1e-5
    lin = oracle.attend_f32(q, kt, v + 2 * v2)
    assert max_abs(lin, base + 2 * oracle.attend_f32(q, kt, v2)) < 1e-5


def test_brute_force_tiny():
    """Plain Python loops, no numpy math, on H=1, T=5."""
    rng = np.random.default_rng(11)
    t = 5
    q = randn(rng, (1, 1, t, 64)) * np.float32(0.25)
    kt, v = randn(rng, (1, 1, 64, t)), randn(rng, (1, 1, t, 64))
    got = oracle.attend_f32(q, kt, v)
    for i in range(t):
        s = [sum(float(q[0, 0, i, d]) * float(kt[0, 0, d, j]) for d in range(64)) for j in range(t)]
        m = max(s)
        w = [math.exp(x - m) for x in s]
        z = sum(w)
        for d in range(64):
            o = sum(w[j] * float(v[0, 0, j, d]) for j in range(t)) / z
            assert abs(o - float(got[0, 0, i, d])) < 1e-5


# ---------------------------------------------------------------------------------------------
# decode kernels (xattn_head, xattn_head_f16)
# ---------------------------------------------------------------------------------------------

@pytest.mark.parametrize("keys", [1, 7, 8, 37, 448, 1500])
def test_decode_f32_matches_closed_form(keys):
    rng = np.random.default_rng(keys)
    q = randn(rng, (1, 6, 1, 64)) * np.float32(0.125)
    kt, v = randn(rng, (1, 6, 64, keys)), randn(rng, (1, 6, keys, 64))
    got = oracle.attend_f32(q, kt, v)
    assert max_abs(got, textbook.attention(q, kt, v, k_transposed=True)) < 1e-5
    assert np.array_equal(got, oracle.attend_f32(q, kt, v, par_heads=True))


@pytest.mark.parametrize("keys", [3, 300, 1500])
def test_decode_f16kv_matches_closed_form(keys):
    rng = np.random.default_rng(50 + keys)
    q = randn(rng, (1, 6, 1, 64)) * np.float32(0.125)
    kt = randn(rng, (1, 6, 64, keys)).astype(np.float16)
    v = randn(rng, (1, 6, keys, 64)).astype(np.float16)
    got = oracle.attend_f16kv(q, kt, v)
    want = textbook.attention(q, kt.astype(np.float32), v.astype(np.float32), k_transposed=True)
    assert max_abs(got, want) < 1e-5


def test_decline_shape_qlen_between():
    rng = np.random.default_rng(12)
    q, kt, v = randn(rng, (1, 2, 7, 64)), randn(rng, (1, 2, 64, 300)), randn(rng, (1, 2, 300, 64))
    assert oracle.attend_f32(q, kt, v) is None  # qlen not in {1, keys}: flash_attn.rs:254-258


# ---------------------------------------------------------------------------------------------
# extension (not reference): batch, GQA, D=128, causal with offset, ragged, K rows/transposed
# ---------------------------------------------------------------------------------------------

def test_general_reduces_to_reference_path():
    rng = np.random.default_rng(13)
    q = randn(rng, (1, 3, 300, 64)) * np.float32(0.125)
    kt, v = randn(rng, (1, 3, 64, 300)), randn(rng, (1, 3, 300, 64))
    gen = oracle.attend_general(q, kt, v, k_transposed=True)
    assert max_abs(gen, oracle.attend_f32(q, kt, v)) < 1e-6
    rows = oracle.attend_general(q, np.ascontiguousarray(np.swapaxes(kt, 2, 3)), v,
                                 k_transposed=False)
    assert max_abs(rows, gen) < 1e-6


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("causal,q_offset,tq,tk", [(False, 0, 70, 300), (True, 0, 130, 130),
                                                  (True, 90, 40, 130), (True, 0, 300, 300)])
def test_general_matches_closed_form(d, causal, q_offset, tq, tk):
    rng = np.random.default_rng(d + tq)
    b, hq, hkv = 2, 4, 2
    q, k, v = randn(rng, (b, hq, tq, d)), randn(rng, (b, hkv, tk, d)), randn(rng, (b, hkv, tk, d))
    sc = d ** -0.5
    got = oracle.attend_general(q, k, v, k_transposed=False, scale=sc, causal=causal,
                                q_offset=q_offset)
    want = textbook.attention(q, k, v, scale=sc, causal=causal, q_offset=q_offset)
    assert max_abs(got, want) < 1e-5


def test_general_ragged_lengths():
    rng = np.random.default_rng(14)
    q, k, v = randn(rng, (4, 2, 1, 64)), randn(rng, (4, 2, 448, 64)), randn(rng, (4, 2, 448, 64))
    lens = np.array([1, 8, 300, 448], np.int32)
    got = oracle.attend_general(q, k, v, k_transposed=False, scale=0.125, kv_lens=lens)
    assert max_abs(got, textbook.attention(q, k, v, scale=0.125, kv_lens=lens)) < 1e-5
    # a single visible key returns exactly its value row
    assert max_abs(got[0, :, 0], v[0, :, 0]) < 1e-6


def test_causal_first_row_sees_one_key():
    rng = np.random.default_rng(15)
    q, k, v = randn(rng, (1, 1, 64, 64)), randn(rng, (1, 1, 64, 64)), randn(rng, (1, 1, 64, 64))
    got = oracle.attend_general(q, k, v, k_transposed=False, scale=0.125, causal=True)
    assert max_abs(got[0, 0, 0], v[0, 0, 0]) < 1e-6


# ---------------------------------------------------------------------------------------------
# golden vectors
# ---------------------------------------------------------------------------------------------

def _bf16(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "*.npz"))),
                         ids=lambda p: os.path.basename(p))
def test_golden_vectors(path):
    z = np.load(path, allow_pickle=False)
    name = os.path.basename(path)
    if name.startswith("encoder_f32"):
        got = oracle.attend_f32(z["q"], z["kt"], z["v"])
    elif name.startswith("decode_f32"):
        got = oracle.attend_f32(z["q"], z["kt"], z["v"])
    elif name.startswith("decode_f16kv"):
        got = oracle.attend_f16kv(z["q"], z["kt16"], z["v16"])
    elif name.startswith("causal_gqa"):
        got = oracle.attend_general(_bf16(z["q_bf16"]), _bf16(z["k_bf16"]), _bf16(z["v_bf16"]),
                                    k_transposed=False, scale=float(z["scale"]), causal=True)
    elif name.startswith("encoder_bf16"):
        full = oracle.attend_general(_bf16(z["q_bf16"]), _bf16(z["kt_bf16"]), _bf16(z["v_bf16"]),
                                     k_transposed=True, scale=float(z["scale"]))
        got = full[:, :, z["rows"]]
    elif name.startswith("ragged_beams"):
        got = oracle.attend_general(_bf16(z["q_bf16"]), _bf16(z["k_bf16"]), _bf16(z["v_bf16"]),
                                    k_transposed=False, scale=float(z["scale"]),
                                    kv_lens=z["lens"])
    else:
        pytest.fail(f"unknown fixture {name}")
    # the oracle reproduces its committed output bit for bit (heads are independent, so the
    # thread count does not change any sum's order)
    assert np.array_equal(got, z["out"]), max_abs(got, z["out"])
    assert max_abs(z["out"], z["f64"]) < 3e-5  # which agrees with the closed form


# ---------------------------------------------------------------------------------------------
# planted mistakes: every one must be caught by a check above
# ---------------------------------------------------------------------------------------------

def _encoder_error(t: int = 300) -> float:
    rng = np.random.default_rng(16)
    q = randn(rng, (1, 2, t, 64))  # unscaled: sharp rows, so the running max moves per tile
    kt, v = randn(rng, (1, 2, 64, t)), randn(rng, (1, 2, t, 64))
    return max_abs(oracle.attend_f32(q, kt, v), textbook.attention(q, kt, v, k_transposed=True))


@pytest.mark.parametrize("fault", [1, 3, 4])
def test_planted_fault_fails_closed_form(fault):
    assert _encoder_error() < 3e-5
    oracle.plant_fault(fault)
    t = 64 if fault == 4 else 300  # the transposed index is only addressable on a square tile
    assert _encoder_error(t) > 1e-3


def test_planted_exp_fault_fails_series_bound():
    oracle.plant_fault(2)
    x = np.linspace(-5.0, 0.0, 10_001, dtype=np.float32)
    rel = np.abs(oracle.exp_poly(x) / np.exp(x.astype(np.float64)) - 1.0)
    assert rel.max() > _exp_bound()
