"""Launch planning over the device's geometry (CPU; no GPU calls).

The planner balances grids over the device's CUs and deals workgroups to its XCDs
(hipDeviceAttributeMultiprocessorCount / NumberOfXccs). An MI355X in single-partition mode has
256 CUs in 8 XCDs; a partitioned one (DPX, QPX, CPX) shows each partition as a device with a
share of them. These tests plan under forced geometries and check that the plans follow the
CU count and that the fused kernel's workgroup -> work map (restated from attn_kernels.cuh)
stays a bijection for every XCD count.
"""

from __future__ import annotations

import ctypes

import pytest

from ffai_amd import _lib as L


@pytest.fixture
def lib():
    lib = L.load()
    yield lib
    L.set_geometry_override(0, 0)


def _desc(lib, qd, kvd, od, b, hq, hkv, tq, tk, hd, layout, causal=0):
    d = L.AttnDesc()
    lib.ffai_attn_desc_init(ctypes.byref(d), qd, kvd, od, b, hq, hkv, tq, tk, hd, layout)
    d.causal = causal
    return d


LARGE_V3 = (L.BF16, L.BF16, L.BF16, 16, 20, 20, 1500, 1500, 64, L.K_TRANSPOSED)
SMALL = (L.BF16, L.BF16, L.BF16, 8, 12, 12, 1500, 1500, 64, L.K_TRANSPOSED)
PREFILL = (L.BF16, L.BF16, L.BF16, 1, 12, 2, 4096, 4096, 128, L.K_ROWS, 1)
CROSS5 = (L.BF16, L.BF16, L.F32, 1, 16, 16, 5, 1500, 64, L.K_ROWS)  # 5 beams as rows
TINY32 = (L.F32, L.F32, L.F32, 1, 6, 6, 1500, 1500, 64, L.K_TRANSPOSED)


def test_no_device_plans_for_the_full_chip(lib):
    """Without a visible device the plans are those of 256 CUs in 8 XCDs."""
    for args in (LARGE_V3, SMALL, PREFILL, CROSS5, TINY32):
        default = L.plan_info(_desc(lib, *args))
        L.set_geometry_override(256, 8)
        assert L.plan_info(_desc(lib, *args)) == default, args
        L.set_geometry_override(0, 0)


def test_large_v3_last_round_follows_the_cus(lib):
    """1920 items of 256 rows, two per CU: 256 CUs leave a last round of 384 of 512 slots (its
    last 128 items in 2 pieces); 128 CUs (a half partition) leave 128 of 256 (again 128 in 2
    pieces, a different share); 320 CUs would take it in exact rounds (no pieces)."""
    d = _desc(lib, *LARGE_V3)
    L.set_geometry_override(256, 8)
    p = L.plan_info(d)
    assert p["split_items"] == (1792, 1920) and p["splits"] == 2
    L.set_geometry_override(128, 4)
    p = L.plan_info(d)
    assert p["split_items"] == (1792, 1920) and p["splits"] == 2
    L.set_geometry_override(160, 4)  # 320 slots: 1920 = 6 whole rounds
    p = L.plan_info(d)
    assert p["split_items"][0] == p["split_items"][1] and p["splits"] == 1


def test_short_grids_split_towards_the_cus(lib):
    """whisper-tiny f32 (72 items, 24 key tiles each) fills the 2 x CUs four-wave slots of 256
    CUs in 6 pieces (7 wanted, 6 cover the tiles); on 32 CUs it aims at 16 waves per CU: 2
    pieces. The beam-5 cross-attention (16 units x 24 tiles) splits towards CUs / 2
    workgroups."""
    d = _desc(lib, *TINY32)
    L.set_geometry_override(256, 8)
    full = L.plan_info(d)
    L.set_geometry_override(32, 1)
    cpx = L.plan_info(d)
    assert full["splits"] == 6 and cpx["splits"] == 2
    d = _desc(lib, *CROSS5)
    L.set_geometry_override(256, 8)
    full = L.plan_info(d)
    L.set_geometry_override(32, 1)
    cpx = L.plan_info(d)
    assert full["kernel"] == cpx["kernel"] == "decode"
    assert full["workgroups"] > cpx["workgroups"] and cpx["workgroups"] >= 16


def _work_map(n_work, sec1_work, xs, remap):
    """The fused kernel's workgroup -> work map (attn_kernels.cuh, top of fwd_kernel)."""
    X = 1 << xs
    sec1_wgs = -(-sec1_work // X) * X
    grid = sec1_wgs + -(-(n_work - sec1_work) // X) * X
    works = []
    for hw in range(grid):
        if hw < sec1_wgs:
            w = (hw & (X - 1)) * (sec1_wgs >> xs) + (hw >> xs) if remap else hw
            if w >= sec1_work:
                continue
        else:
            x, n = hw - sec1_wgs, grid - sec1_wgs
            w = sec1_work + ((x & (X - 1)) * (n >> xs) + (x >> xs) if remap else x)
            if w >= n_work:
                continue
        works.append(w)
    return works


@pytest.mark.parametrize("xcds", [1, 2, 4, 8])
@pytest.mark.parametrize("args", [LARGE_V3, SMALL, PREFILL])
def test_every_work_runs_once_for_every_xcd_count(lib, xcds, args):
    L.set_geometry_override(32 * xcds, xcds)
    d = _desc(lib, *args)
    p = L.plan_info(d)
    lo, hi = p["split_items"]
    sec1 = lo if hi > lo and lo > 0 else p["workgroups"]
    causal = len(args) > 10 and args[10]
    works = _work_map(p["workgroups"], sec1, xcds.bit_length() - 1, not causal)
    assert sorted(works) == list(range(p["workgroups"]))
