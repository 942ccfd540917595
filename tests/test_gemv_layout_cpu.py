"""CPU audit of the matrix-core f16 GEMV (ffai_amd/csrc/gemv.hip, gemv_f16_kernel).

The launch shape comes from the library itself (ffai_gemv_f16_plan_info); the kernel's index
formulas are restated here and checked over a sweep of shapes:

* every x, W and LDS access stays inside x (rows x in_dim), W (out_dim x in_dim) and the
  dynamic LDS the launch provides, and a workgroup fits a CU (<= 1024 lanes, <= 160 KB LDS);
* every weight element of a row meets the same element of each beam's x exactly once: the
  MFMA contraction index (pass, part, wave, block, lane group, element) enumerates [0, in_dim)
  once, the dense x load writes each (column, element) of the wave's LDS rows (QN * rows of
  them, column (part, beam) at row part * rows + beam) from the x element the B read of MFMA
  column part TR + beam expects there, and the reduction reads C[q TR + r][q TR + b] from the
  lane and register where the 16x16 D layout holds it;
* a numpy emulation of the whole tiling, the scaled hi/lo split of x included, equals the exact
  float64 product to the f32 summation bound the GPU test uses.
"""

from __future__ import annotations

import numpy as np
import pytest

from ffai_amd import _lib as L

SHAPES = [
    (1024, 1024, 5), (3072, 1024, 5), (4096, 1024, 5), (1024, 4096, 5),  # whisper-medium beam 5
    (1280, 1280, 5), (3840, 1280, 5), (5120, 1280, 5), (1280, 5120, 5),  # whisper-large beam 5
    (1024, 4096, 9), (1536, 384, 1), (1023, 1280, 16), (384, 384, 1), (1024, 1024, 1),
    (51, 40, 3), (7, 8, 1), (100, 5120, 2), (4096, 4096, 16), (17, 8200, 7), (33, 264, 4),
    (1280, 8192, 5), (64, 20000, 16), (1024, 2560, 3), (1280, 6144, 5), (1024, 20000, 9),
]


def geometry(out_dim, in_dim, rows):
    p = L.gemv_plan_info(out_dim, in_dim, rows)
    tr, nw, nj = p["tile_rows"], p["waves"], p["blocks_per_wave"]
    qn, rs, lpc = 16 // tr, 32 * nj + 8, 8 * nj
    ncol = qn * rows
    g = dict(p, tr=tr, tl=tr.bit_length() - 1, qn=qn, nw=nw, nj=nj, kw=32 * nj, rs=rs, lpc=lpc,
             ni_all=2 * nj, ncol=ncol, ni=(ncol * lpc + 63) // 64,
             reg=max(2 * ncol * rs, 608), kp=nw * 32 * nj, tiles=-(-out_dim // tr))
    return g


@pytest.mark.parametrize("out_dim,in_dim,rows", SHAPES)
def test_launch_shape_fits(out_dim, in_dim, rows):
    g = geometry(out_dim, in_dim, rows)
    assert g["tr"] in (1, 2, 4, 8, 16) and g["tr"] >= rows
    assert g["nj"] in (1, 2, 4, 8) and 1 <= g["nw"] <= 16
    assert g["nw"] * 64 <= 1024
    # per wave: the hi and lo rows of the QN * rows columns (16-byte aligned), at least the
    # partial tile (64 lanes x 4 floats at word 4 l + 16 (l / 16): 304 words)
    assert g["reg"] % 8 == 0
    assert 2 * (4 * 63 + 3 + 16 * 3 + 1) <= g["reg"]
    assert g["lds_bytes"] == g["nw"] * g["reg"] * 2 <= 160 * 1024
    # the passes cover in_dim
    assert g["passes"] * g["qn"] * g["kp"] >= in_dim
    assert (g["passes"] - 1) * g["qn"] * g["kp"] < in_dim
    # all the dense x loads cover the 16 slots exactly; those a launch makes hold every beam
    assert g["ni_all"] * 64 == 16 * g["lpc"]
    assert g["ncol"] <= 16 and g["ni"] <= g["ni_all"] and g["ni"] * 64 >= g["ncol"] * g["lpc"]


@pytest.mark.parametrize("out_dim,in_dim,rows", SHAPES)
def test_addresses_in_range_and_contraction_pairs_elements(out_dim, in_dim, rows):
    g = geometry(out_dim, in_dim, rows)
    tr, tl, qn, kw, rs, lpc, kp = g["tr"], g["tl"], g["qn"], g["kw"], g["rs"], g["lpc"], g["kp"]
    ncol, reg = g["ncol"], g["reg"]
    lane = np.arange(64)
    m, grp = lane & 15, lane >> 4
    q, r = m >> tl, m & (tr - 1)
    seen = np.zeros(in_dim, np.int64)
    for tile in {0, g["tiles"] - 1}:
        row = np.minimum(tile * tr + r, out_dim - 1)
        assert (row >= 0).all() and (row < out_dim).all()
    for ps in range(g["passes"]):
        for wave in range(g["nw"]):
            kb = ps * qn * kp + wave * kw
            # dense x loads (slot v = beam v / QN over part v % QN) and the LDS rows the slots of
            # beams < rows fill: (LDS column, element) -> (beam, x element)
            written = {}
            for i in range(g["ni"]):
                f = 64 * i + lane
                v = f // lpc
                assert (v < 16).all()
                b_raw, part = v >> (4 - tl), v & (qn - 1)
                b = np.minimum(b_raw, rows - 1)
                k = np.minimum(kb + part * kp + 4 * (f % lpc), in_dim - 4)
                assert (b >= 0).all() and (k >= 0).all() and (k + 4 <= in_dim).all()
                c4 = f % lpc
                for L_ in range(64):
                    if b_raw[L_] >= rows:  # a slot past the beams: loaded, not kept
                        continue
                    n = part[L_] * rows + b_raw[L_]
                    assert n < ncol and 4 * c4[L_] + 4 <= kw
                    assert (ncol + n) * rs + 4 * c4[L_] + 4 <= reg and n * rs + kw < reg
                    for e in range(4):
                        key = (n, 4 * c4[L_] + e)
                        assert key not in written
                        written[key] = (b_raw[L_], kb + part[L_] * kp + 4 * c4[L_] + e)
            # every column is fully written
            for n in range(ncol):
                assert all((n, off) in written for off in range(kw))
            for j in range(g["nj"]):
                kw_ = kb + q * kp + 32 * j + 8 * grp
                kc = np.minimum(kw_, in_dim - 8)
                assert (kc >= 0).all() and (kc + 8 <= in_dim).all()
                for L_ in range(64):
                    n_col = m[L_]  # B column of this lane; its A row is m too
                    for e in range(8):
                        k = kw_[L_] + e
                        if r[L_] == 0 and k < in_dim:  # count each (part, k) once per tile row
                            seen[k] += 1
                        if (n_col & (tr - 1)) < rows:
                            off = 32 * j + 8 * grp[L_] + e
                            ncm = (n_col >> tl) * rows + (n_col & (tr - 1))
                            assert off < kw and (ncol + ncm) * rs + off < reg
                            bb, kx = written[(ncm, off)]
                            # B column n = q' TR + b holds beam b over part q' = n >> tl, at the
                            # element the A rows of the same part contract with
                            assert bb == (n_col & (tr - 1))
                            assert kx == kb + (n_col >> tl) * kp + 32 * j + 8 * grp[L_] + e
    # rows r = 0 of each part over all passes and waves: each element exactly once
    assert (seen == 1).all()
    # the reduction reads C[q TR + rr][q TR + b] where the 16x16 D layout keeps it
    for rr in range(tr):
        for b in range(rows):
            for qq in range(qn):
                mm, nn = (qq << tl) + rr, (qq << tl) + b
                lidx, e = nn + 16 * (mm >> 2), mm & 3
                assert lidx < 64 and lidx % 16 == nn and 4 * (lidx // 16) + e == mm


def emulate(w16, x, g):
    """The kernel's arithmetic in numpy: per tile, pass and wave the MFMA products of the A rows
    with the split x columns, unscaled per column, summed over waves and parts."""
    out_dim, in_dim = w16.shape
    rows = x.shape[0]
    tr, tl, qn, kw, kp = g["tr"], g["tl"], g["qn"], g["kw"], g["kp"]
    y = np.zeros((rows, out_dim))
    wd = w16.astype(np.float64)
    for tile in range(g["tiles"]):
        acc_parts = np.zeros((16, 16))
        for ps in range(g["passes"]):
            for wave in range(g["nw"]):
                kb = ps * qn * kp + wave * kw
                A = np.zeros((16, kw))
                B = np.zeros((kw, 16))
                for mm in range(16):
                    q, r = mm >> tl, mm & (tr - 1)
                    row = min(tile * tr + r, out_dim - 1)
                    k = kb + q * kp + np.arange(kw)
                    ok = k < in_dim
                    A[mm, ok] = wd[row, k[ok]]
                inv = np.ones(16)
                for n in range(16):
                    qq, b = n >> tl, n & (tr - 1)
                    if b >= rows:
                        continue
                    k = kb + qq * kp + np.arange(kw)
                    ok = k < in_dim
                    xs = np.zeros(kw, np.float32)
                    xs[ok] = x[b, k[ok]]
                    mx = np.float32(np.abs(xs).max())
                    e = int(mx.view(np.uint32) >> 23)
                    sb = min(max(268 - e, 1), 253)
                    sc = np.uint32(sb << 23).view(np.float32)
                    inv[n] = np.uint32((254 - sb) << 23).view(np.float32)
                    v = xs * sc
                    hi = v.astype(np.float16)
                    lo = (v - hi.astype(np.float32)).astype(np.float16)
                    B[:, n] = hi.astype(np.float64) + lo.astype(np.float64)
                acc_parts += (A @ B) * inv[None, :]
        for rr in range(tr):
            o = tile * tr + rr
            if o >= out_dim:
                continue
            for b in range(rows):
                y[b, o] = sum(acc_parts[(qq << tl) + rr, (qq << tl) + b] for qq in range(qn))
    return y


@pytest.mark.parametrize("out_dim,in_dim,rows", [(51, 40, 3), (33, 264, 4), (7, 8, 1),
                                                 (40, 1032, 5), (24, 600, 16), (70, 136, 2)])
def test_emulated_tiling_matches_exact_product(out_dim, in_dim, rows):
    rng = np.random.default_rng(out_dim * 7 + in_dim)
    w16 = rng.standard_normal((out_dim, in_dim)).astype(np.float16)
    x = rng.standard_normal((rows, in_dim)).astype(np.float32)
    x[0, : min(5, in_dim)] *= 1e3  # a wide range within one column
    if rows > 1:
        x[1] *= 1e-6
    g = geometry(out_dim, in_dim, rows)
    got = emulate(w16, x, g)
    exact = x.astype(np.float64) @ w16.astype(np.float64).T
    bound = 1e-5 * (np.abs(x.astype(np.float64)) @ np.abs(w16.astype(np.float64)).T) + 1e-30
    assert (np.abs(got - exact) <= bound).all()
