"""GPU parity of the fused kernel's key-split pieces: items that run as several workgroups over
contiguous key ranges, merged by the item's last piece in the same launch.

The split layout is forced with ffai_set_fwd_split_override so that every arrangement runs at
sizes the oracle finishes in seconds: the tail of a non-causal grid (a second dispatch section
after the whole items), the longest items of a causal grid, every item, ragged items whose later
pieces hold no keys. Each case checks the output against the oracle (1e-4 f32, 2e-2 16-bit),
the plan's split ranks, and that the counters at the workspace's start are zero again.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from ffai_amd import _lib as L
from ffai_amd import flash_attn as fa
from tests.helpers import TOL_BF16, TOL_F32, max_abs, randn, round_bf16, round_f16

pytestmark = pytest.mark.gpu

COUNTER_BYTES = 4096


@pytest.fixture
def split_override():
    prev = L.get_fwd_split_override()
    yield L.set_fwd_split_override
    L.set_fwd_split_override(*prev)


def _dev(x, dtype, device):
    return torch.from_numpy(np.ascontiguousarray(x)).to(device=device, dtype=dtype)


def _run(q, k, v, *, out_dtype, **kw):
    """One call with an explicit zeroed workspace; returns (out, plan, workspace)."""
    out = torch.empty(q.shape[0], q.shape[1], q.shape[2], v.shape[3], dtype=out_dtype,
                      device=q.device)
    n = fa.workspace_bytes(q, k, v, out, **kw)
    ws = torch.zeros(max(n, 1), dtype=torch.uint8, device=q.device)
    plan = fa.plan(q, k, v, out, **kw)
    res = fa.attention(q, k, v, out=out, workspace=ws, **kw)
    assert res is not None
    torch.cuda.synchronize()
    return out, plan, ws


def _counters_zero(ws):
    return int(ws[:COUNTER_BYTES].count_nonzero().item()) == 0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("k_transposed", [True, False])
def test_tail_items_in_pieces(gpu, split_override, dtype, k_transposed):
    """Non-causal, four waves x 32 rows: the last 37 of 90 items in 4 pieces each, dispatched as
    a second section after the 53 whole items."""
    rng = np.random.default_rng(37)
    b, h, t, d = 3, 5, 700, 64
    rnd = round_bf16 if dtype == torch.bfloat16 else round_f16
    q = rnd(randn(rng, (b, h, t, d)))
    k = rnd(randn(rng, (b, h, d, t) if k_transposed else (b, h, t, d)))
    v = rnd(randn(rng, (b, h, t, d)))
    split_override(37, 4)
    out, plan, ws = _run(_dev(q, dtype, gpu), _dev(k, dtype, gpu), _dev(v, dtype, gpu),
                         out_dtype=torch.float32, k_transposed=k_transposed, scale=0.125)
    assert plan["kernel"] == "fwd" and plan["shape"] == "wave4"
    assert plan["items"] == 90 and plan["split_items"] == (53, 90) and plan["splits"] == 4
    want = oracle.attend_general(q, k, v, k_transposed=k_transposed, scale=0.125)
    err = max_abs(out.cpu().numpy(), want)
    print(f"tail pieces {dtype} kt={k_transposed}: {err:.3e}")
    assert err < TOL_BF16
    assert _counters_zero(ws)


def test_tail_items_in_pieces_two_column_blocks(gpu, split_override):
    """The encoder's launch shape (four waves x 64 rows, K transposed): 512 items, the last 100
    in 3 pieces."""
    rng = np.random.default_rng(512)
    b, h, t, d = 16, 16, 512, 64
    q = round_bf16(randn(rng, (b, h, t, d)))
    kt = round_bf16(randn(rng, (b, h, d, t)))
    v = round_bf16(randn(rng, (b, h, t, d)))
    split_override(100, 3)
    out, plan, ws = _run(_dev(q, torch.bfloat16, gpu), _dev(kt, torch.bfloat16, gpu),
                         _dev(v, torch.bfloat16, gpu), out_dtype=torch.bfloat16,
                         k_transposed=True, scale=0.125)
    assert plan["shape"] in ("wave4x2", "wave4x2x16") and plan["items"] == 512
    assert plan["split_items"] == (412, 512) and plan["splits"] == 3
    want = oracle.attend_general(q, kt, v, k_transposed=True, scale=0.125)
    err = max_abs(out.float().cpu().numpy(), want)
    print(f"tail pieces 4x2: {err:.3e}")
    assert err < TOL_BF16
    assert _counters_zero(ws)


@pytest.mark.parametrize("d", [64, 128])
def test_longest_causal_items_in_pieces(gpu, split_override, d):
    """Causal GQA (Hq 4, Hkv 2, S 700): the 5 longest items in 3 pieces, dispatched first."""
    rng = np.random.default_rng(700 + d)
    b, hq, hkv, s = 1, 4, 2, 700
    q = round_bf16(randn(rng, (b, hq, s, d)))
    k = round_bf16(randn(rng, (b, hkv, s, d)))
    v = round_bf16(randn(rng, (b, hkv, s, d)))
    split_override(5, 3)
    out, plan, ws = _run(_dev(q, torch.bfloat16, gpu), _dev(k, torch.bfloat16, gpu),
                         _dev(v, torch.bfloat16, gpu), out_dtype=torch.float32,
                         scale=d ** -0.5, causal=True)
    assert plan["split_items"] == (0, 5) and plan["splits"] == 3
    want = oracle.attend_general(q, k, v, k_transposed=False, scale=d ** -0.5, causal=True)
    err = max_abs(out.cpu().numpy(), want)
    print(f"causal longest pieces d{d}: {err:.3e}")
    assert err < TOL_BF16
    assert _counters_zero(ws)


@pytest.mark.parametrize("items,pieces", [(-1, 7), (3, 2)])
def test_f32_items_in_pieces(gpu, split_override, items, pieces):
    """The f32 kernel (whisper-tiny heads) with every item in 7 pieces, and with the last 3
    items in 2."""
    rng = np.random.default_rng(600 + pieces)
    h, t, d = 6, 600, 64
    q = randn(rng, (1, h, t, d)) * np.float32(0.125)
    kt, v = randn(rng, (1, h, d, t)), randn(rng, (1, h, t, d))
    split_override(items, pieces)
    out, plan, ws = _run(_dev(q, torch.float32, gpu), _dev(kt, torch.float32, gpu),
                         _dev(v, torch.float32, gpu), out_dtype=torch.float32,
                         k_transposed=True, scale=1.0)
    n = plan["items"]
    assert plan["split_items"] == ((0, n) if items < 0 else (n - items, n))
    assert plan["splits"] == pieces
    want = oracle.attend_general(q, kt, v, k_transposed=True, scale=1.0)
    err = max_abs(out.cpu().numpy(), want)
    print(f"f32 pieces {items}x{pieces}: {err:.3e}")
    assert err < TOL_F32
    assert _counters_zero(ws)


def test_ragged_items_with_empty_pieces(gpu, split_override):
    """Per-batch key counts 300, 1, 65, 200 with every item in 5 pieces: the short items' later
    pieces hold no keys and must count as empty in the merge."""
    rng = np.random.default_rng(5)
    b, h, t, tk, d = 4, 2, 300, 300, 64
    lens = np.array([300, 1, 65, 200], np.int32)
    q = round_bf16(randn(rng, (b, h, t, d)))
    k = round_bf16(randn(rng, (b, h, tk, d)))
    v = round_bf16(randn(rng, (b, h, tk, d)))
    split_override(-1, 5)
    out, plan, ws = _run(_dev(q, torch.bfloat16, gpu), _dev(k, torch.bfloat16, gpu),
                         _dev(v, torch.bfloat16, gpu), out_dtype=torch.float32, scale=0.125,
                         kv_lens=torch.from_numpy(lens).to(gpu))
    assert plan["splits"] == 5
    want = oracle.attend_general(q, k, v, k_transposed=False, scale=0.125, kv_lens=lens)
    err = max_abs(out.cpu().numpy(), want)
    print(f"ragged empty pieces: {err:.3e}")
    assert err < TOL_BF16
    assert _counters_zero(ws)


def test_one_workspace_across_split_layouts(gpu, split_override):
    """A workspace zeroed once serves calls of different split layouts in a row (every call
    leaves its counters zero); each result matches the oracle."""
    rng = np.random.default_rng(11)
    b, h, t, d = 2, 4, 900, 64
    q = _dev(round_bf16(randn(rng, (b, h, t, d))), torch.bfloat16, gpu)
    k = _dev(round_bf16(randn(rng, (b, h, t, d))), torch.bfloat16, gpu)
    v = _dev(round_bf16(randn(rng, (b, h, t, d))), torch.bfloat16, gpu)
    want = oracle.attend_general(q.float().cpu().numpy(), k.float().cpu().numpy(),
                                 v.float().cpu().numpy(), k_transposed=False, scale=0.125)
    sizes = []
    for items, pieces in [(-1, 8), (10, 3), (20, 2), (-1, 4)]:
        split_override(items, pieces)
        sizes.append(fa.workspace_bytes(q, k, v, torch.empty_like(q, dtype=torch.float32),
                                        scale=0.125))
    ws = torch.zeros(max(sizes), dtype=torch.uint8, device=gpu)
    for items, pieces in [(-1, 8), (10, 3), (20, 2), (-1, 4)]:
        split_override(items, pieces)
        out = torch.empty(b, h, t, d, dtype=torch.float32, device=gpu)
        assert fa.attention(q, k, v, scale=0.125, out=out, workspace=ws) is not None
        torch.cuda.synchronize()
        err = max_abs(out.cpu().numpy(), want)
        print(f"layout {items}x{pieces}: {err:.3e}")
        assert err < TOL_BF16
        assert _counters_zero(ws)


@pytest.mark.parametrize("layout", ["forced", "prompt_cross"])
def test_pieces_in_graph_replays(gpu, split_override, layout):
    """A launch with split items captured in a HIP graph: every replay (with eager work and
    synchronisation between replays, new inputs copied in) equals the eager call on the same
    inputs bit for bit, and leaves the counters zero. Past the counters the workspace starts as
    garbage (0xFF): partials are written before they are read. Layouts: 9 of 12 four-wave items
    forced into 3 pieces (K transposed), and the planner's own layout for a prompt step's
    cross-attention (228 queries x 16 heads over 1500 keys as rows: one-wave items in 6 pieces,
    768 workgroups)."""
    rng = np.random.default_rng(77)
    if layout == "forced":
        b, h, tq, tk, d, kt = 2, 3, 700, 700, 64, True
        split_override(9, 3)
    else:
        b, h, tq, tk, d, kt = 1, 16, 228, 1500, 64, False
    q = torch.empty(b, h, tq, d, dtype=torch.bfloat16, device=gpu)
    k = torch.empty((b, h, d, tk) if kt else (b, h, tk, d), dtype=torch.bfloat16, device=gpu)
    v = torch.empty(b, h, tk, d, dtype=torch.bfloat16, device=gpu)
    out = torch.empty(b, h, tq, d, dtype=torch.float32, device=gpu)
    args = dict(k_transposed=kt, scale=0.125)
    plan = fa.plan(q, k, v, out, **args)
    if layout == "forced":
        assert plan["splits"] == 3 and plan["split_items"][1] - plan["split_items"][0] == 9
    else:
        assert plan["splits"] == 6 and plan["workgroups"] == 768, plan
    nbytes = fa.workspace_bytes(q, k, v, out, **args)
    ws = torch.full((nbytes,), 0xFF, dtype=torch.uint8, device=gpu)
    ws[:COUNTER_BYTES].zero_()
    inputs = [tuple(_dev(round_bf16(randn(rng, x.shape)), torch.bfloat16, gpu) for x in (q, k, v))
              for _ in range(3)]

    def call():
        fa.attention(q, k, v, out=out, workspace=ws, **args)

    eager = []
    for qi, ki, vi in inputs:
        q.copy_(qi); k.copy_(ki); v.copy_(vi)
        call()
        torch.cuda.synchronize()
        eager.append(out.clone())
        assert _counters_zero(ws)
    want = oracle.attend_general(inputs[0][0].float().cpu().numpy(),
                                 inputs[0][1].float().cpu().numpy(),
                                 inputs[0][2].float().cpu().numpy(), k_transposed=kt,
                                 scale=0.125)
    assert max_abs(eager[0].cpu().numpy(), want) < TOL_BF16
    graph = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        call()
    for i in range(6):
        qi, ki, vi = inputs[i % 3]
        q.copy_(qi); k.copy_(ki); v.copy_(vi)
        out.fill_(float(i + 1))     # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager[i % 3]), f"replay {i} differs"
        assert _counters_zero(ws), f"replay {i} left a counter set"


def _seeded_cases(n=24, seed=2026):
    """Small random shapes over every launch layout the planner and the override can make."""
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        d = int(rng.choice([64, 128]))
        dtype = ["bf16", "f16", "f32"][i % 3] if d == 64 else ["bf16", "f16"][i % 2]
        hkv = int(rng.integers(1, 4))
        hq = hkv * int(rng.integers(1, 4)) if dtype != "f32" else hkv
        b = int(rng.integers(1, 4))
        causal = bool(rng.integers(0, 2)) and dtype != "f32"
        tk = int(rng.integers(40, 700))
        tq = int(rng.integers(1, 400)) if not causal else int(rng.integers(1, tk + 1))
        q_offset = tk - tq if causal else 0
        ragged = bool(rng.integers(0, 2))
        items = int(rng.choice([0, -1, 1, 3, 7]))
        pieces = int(rng.integers(2, 6))
        k_transposed = bool(rng.integers(0, 2))
        cases.append((i, b, hq, hkv, tq, tk, d, dtype, causal, q_offset, ragged, items, pieces,
                      k_transposed))
    return cases


@pytest.mark.parametrize("case", _seeded_cases(), ids=lambda c: f"case{c[0]}")
def test_seeded_layouts_against_the_oracle(gpu, split_override, case):
    """Seeded random shapes (batch, grouped heads, head_dim 64/128, 16-bit and f32, causal with
    the queries at the end of the keys, ragged key counts including empty ones, K rows or K
    transposed) under the planner's layout or a forced one (the last / longest 1, 3 or 7 items or
    every item in 2-5 pieces), against the oracle. Query counts up to 32 take the decode kernel."""
    i, b, hq, hkv, tq, tk, d, dtype, causal, q_offset, ragged, items, pieces, k_transposed = case
    rng = np.random.default_rng(1000 + i)
    tdt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[dtype]
    rnd = {"bf16": round_bf16, "f16": round_f16, "f32": lambda x: x}[dtype]
    q = rnd(randn(rng, (b, hq, tq, d)))
    k = rnd(randn(rng, (b, hkv, d, tk) if k_transposed else (b, hkv, tk, d)))
    v = rnd(randn(rng, (b, hkv, tk, d)))
    lens = rng.integers(0, tk + 1, size=b).astype(np.int32) if ragged else None
    if items:
        split_override(items, pieces)
    scale = d ** -0.5
    kw = dict(scale=scale, causal=causal, q_offset=q_offset, k_transposed=k_transposed)
    if lens is not None:
        kw["kv_lens"] = torch.from_numpy(lens).to(gpu)
    out, plan, ws = _run(_dev(q, tdt, gpu), _dev(k, tdt, gpu), _dev(v, tdt, gpu),
                         out_dtype=torch.float32, **kw)
    want = oracle.attend_general(q, k, v, k_transposed=k_transposed, scale=scale, causal=causal,
                                 q_offset=q_offset, kv_lens=lens)
    err = max_abs(out.cpu().numpy(), want)
    print(f"case {case}: plan {plan}, err {err:.3e}")
    assert err < (TOL_F32 if dtype == "f32" else TOL_BF16)
    assert _counters_zero(ws)


def _dev_at(x, dtype, device, off):
    """x on the device as a view starting `off` elements into a larger buffer."""
    t = _dev(x, dtype, device)
    if off == 0:
        return t
    buf = torch.empty(t.numel() + off, dtype=dtype, device=device)
    view = buf[off:].view(t.shape)
    view.copy_(t)
    return view


def _broad_cases(seed, n):
    """Random shapes up to whisper-window size: 1-1700 keys, 1-1600 queries (a quarter of them
    decode-sized, at most 32), ragged or not, causal with the queries at the end of the keys,
    grouped heads, head_dim 64/128, K rows or transposed, f32 or 16-bit outputs, and the
    planner's layout or a forced split."""
    rng = np.random.default_rng(seed)
    for i in range(n):
        d = int(rng.choice([64, 128]))
        dtype = str(rng.choice(["bf16", "f16", "f32"] if d == 64 else ["bf16", "f16"]))
        hkv = int(rng.integers(1, 4))
        hq = hkv * int(rng.integers(1, 5)) if dtype != "f32" else hkv
        b = int(rng.integers(1, 4))
        causal = bool(rng.integers(0, 2)) and dtype != "f32"
        tk = int(rng.integers(1, 1700))
        tq = int(rng.integers(1, 33)) if rng.integers(0, 4) == 0 else int(rng.integers(1, 1600))
        if causal:
            tq = min(tq, tk)
        ragged = bool(rng.integers(0, 2))
        items = int(rng.choice([0, 0, 0, -1, 1, 3, 7]))
        pieces = int(rng.integers(2, 6))
        kt = bool(rng.integers(0, 2))
        out16 = bool(rng.integers(0, 2)) and dtype != "f32"
        yield i, b, hq, hkv, tq, tk, d, dtype, causal, ragged, items, pieces, kt, out16


def test_broad_seeded_sweep_against_the_oracle(gpu, split_override):
    """400 seeded random calls (see _broad_cases) against the oracle, one process, every fourth
    with misaligned inputs: every output within tolerance and every split counter zero again
    afterwards."""
    worst, kernels = {}, {}
    for case in _broad_cases(7, 400):
        i, b, hq, hkv, tq, tk, d, dtype, causal, ragged, items, pieces, kt, out16 = case
        rng = np.random.default_rng(7000 + i)
        tdt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[dtype]
        rnd = {"bf16": round_bf16, "f16": round_f16, "f32": lambda x: x}[dtype]
        q = rnd(randn(rng, (b, hq, tq, d)))
        k = rnd(randn(rng, (b, hkv, d, tk) if kt else (b, hkv, tk, d)))
        v = rnd(randn(rng, (b, hkv, tk, d)))
        lens = rng.integers(0, tk + 1, size=b).astype(np.int32) if ragged else None
        split_override(items, pieces) if items else split_override(0, 0)
        q_offset = tk - tq if causal else 0
        kw = dict(scale=d ** -0.5, causal=causal, q_offset=q_offset, k_transposed=kt)
        if lens is not None:
            kw["kv_lens"] = torch.from_numpy(lens).to(gpu)
        # every fourth call takes its inputs at 0-7 elements past 16-byte alignment (register
        # staging instead of the DMA)
        off = int(rng.integers(0, 8)) if i % 4 == 0 else 0
        out, plan, ws = _run(_dev_at(q, tdt, gpu, off), _dev_at(k, tdt, gpu, off),
                             _dev_at(v, tdt, gpu, off),
                             out_dtype=tdt if out16 else torch.float32, **kw)
        want = oracle.attend_general(q, k, v, k_transposed=kt, scale=kw["scale"], causal=causal,
                                     q_offset=q_offset, kv_lens=lens)
        err = max_abs(out.float().cpu().numpy(), want)
        tag = dtype + ("/out16" if out16 else "")
        worst[tag] = max(worst.get(tag, 0.0), err)
        kernels[plan["kernel"]] = kernels.get(plan["kernel"], 0) + 1
        assert err < (TOL_F32 if dtype == "f32" else TOL_BF16), (case, plan, err)
        assert _counters_zero(ws), (case, plan)
    print("kernels", kernels, "worst", {t: f"{e:.2e}" for t, e in worst.items()})
    assert set(kernels) == {"fwd", "decode"}
