"""Address-range audit of the encoder attention block at 16 whisper-large-v3 windows in ONE pass
(24000 rows), on the CPU: every byte range the projections, the fused kernel (Q loads, K/V
tiles by DMA and through registers, output stores) and its workspace can touch, checked
against the workspace regions of ffai_amd/csrc/encoder_attn.cpp.

The library runs at most 1500 rows per pass (one window); a first design ran all 16 windows in
one call and faulted the GPU. This audit restates the block's layout (sizes_of, run_pass,
attn_desc in encoder_attn.cpp) and the fused kernel's index bounds (attn_kernels.cuh: rows
clamped below q_len, keys clamped below kv_len, whole tiles by DMA only) and shows that at
B = 16 every access of the current design stays inside its region, the regions are disjoint,
and every 32-bit offset the kernel forms fits. The layout mirror is pinned against the
library's own ffai_encoder_attn_workspace_bytes at the sizes the library accepts.
"""

from __future__ import annotations

import ctypes

import pytest

from ffai_amd import _lib as L

ES = 2  # bf16 / f16 bytes
GEMM_SCRATCH = 32 << 20
COUNTER_BYTES = 4096
BN = 64  # keys per tile


def align256(n: int) -> int:
    return (n + 255) // 256 * 256


def attn_ws_bytes(lib, b, s, n, h, packed) -> int:
    """ffai_attn_workspace_bytes of the block's attention descriptor (attn_desc)."""
    hd = n // h
    d = L.AttnDesc()
    lib.ffai_attn_desc_init(ctypes.byref(d), L.BF16, L.BF16, L.BF16, b, h, h, s, s, hd,
                            L.K_ROWS if packed else L.K_TRANSPOSED)
    d.scale = 1.0
    q_st = [s * 3 * n, hd, 3 * n, 1] if packed else [s * n, hd, n, 1]
    k_st = q_st if packed else [s, hd * b * s, b * s, 1]
    o_st = [s * n, hd, n, 1]
    for i in range(4):
        d.q_strides[i], d.v_strides[i] = q_st[i], q_st[i]
        d.k_strides[i], d.o_strides[i] = k_st[i], o_st[i]
    out = ctypes.c_size_t(0)
    assert lib.ffai_attn_workspace_bytes(ctypes.byref(d), ctypes.byref(out)) == L.FFAI_OK
    return out.value


def layout(lib, b, s, n, h) -> dict:
    """Regions of one pass of b windows (sizes_of / run_pass): attention workspace first (at
    least the split counters), then q, kt, v, merged, hipBLASLt scratch."""
    act = align256(b * s * n * ES)
    aw = max(attn_ws_bytes(lib, b, s, n, h, p) for p in (False, True))
    sizes = [("attn", align256(max(aw, COUNTER_BYTES))), ("q", act), ("kt", act), ("v", act),
             ("merged", act), ("gemm", GEMM_SCRATCH)]
    regions, off = {}, 0
    for name, size in sizes:
        regions[name] = (off, off + size)
        off += size
    regions["total"] = (0, off)
    return regions


def extent(base: int, dims, strides) -> tuple:
    """[first, last + 1) element range of a strided box (every index in range)."""
    last = base + sum((d - 1) * st for d, st in zip(dims, strides))
    return base, last + 1


def inside(rng_bytes, region) -> bool:
    return region[0] <= rng_bytes[0] and rng_bytes[1] <= region[1]


@pytest.mark.parametrize("b,s,n,h", [(1, 1500, 1280, 20), (5, 300, 384, 6), (1, 1500, 384, 6)])
def test_layout_mirror_matches_the_library(b, s, n, h):
    """The mirror's total equals the library's workspace size at shapes it accepts."""
    lib = L.load()
    d = L.EncoderAttnDesc()
    d.dtype, d.batch, d.seq, d.n_state, d.n_head = L.BF16, b, s, n, h
    got = ctypes.c_size_t(0)
    assert lib.ffai_encoder_attn_workspace_bytes(ctypes.byref(d), ctypes.byref(got)) == L.FFAI_OK
    assert layout(lib, b, s, n, h)["total"][1] == got.value


@pytest.mark.parametrize("packed", [False, True])
def test_sixteen_windows_in_one_pass_stay_in_bounds(packed):
    lib = L.load()
    b, s, n, h = 16, 1500, 1280, 20
    hd = n // h
    bs = b * s
    z = layout(lib, b, s, n, h)
    names = ["attn", "q", "kt", "v", "merged", "gemm"]
    for x, y in zip(names, names[1:]):  # disjoint and in order
        assert z[x][1] <= z[y][0]

    def by(region_name, elem_range, base_elem=0):
        r0 = z[region_name][0] + (base_elem + elem_range[0]) * ES
        return r0, z[region_name][0] + (base_elem + elem_range[1]) * ES

    writes, reads = [], []
    if packed:
        # qkv GEMM: D^T (3N x BS) column-major, ldd 3N, from the start of q over q, kt, v
        writes.append(("qkv", (z["q"][0], z["q"][0] + (bs - 1) * 3 * n * ES + 3 * n * ES),
                       (z["q"][0], z["v"][1])))
        st = [s * 3 * n, hd, 3 * n, 1]
        for name, col in (("Q", 0), ("K rows", n), ("V", 2 * n)):
            e = extent(col, (b, h, s, hd), st)
            reads.append((name, by("q", e), (z["q"][0], z["v"][1])))
    else:
        for name in ("q", "v"):  # D^T (N x BS), ldd N
            writes.append((name, (z[name][0], z[name][0] + (bs - 1) * n * ES + n * ES), z[name]))
        # kt: column-major (BS x N), ldd BS
        writes.append(("kt", (z["kt"][0], z["kt"][0] + (n - 1) * bs * ES + bs * ES), z["kt"]))
        st = [s * n, hd, n, 1]
        reads.append(("Q", by("q", extent(0, (b, h, s, hd), st)), z["q"]))
        reads.append(("V", by("v", extent(0, (b, h, s, hd), st)), z["v"]))
        # K^T (b, h, d, key) with strides (S, hd B S, B S, 1); keys < kv_len: tiles whole by
        # DMA only when all 64 keys are valid, tails clamped to the last key
        reads.append(("K^T", by("kt", extent(0, (b, h, hd, s), [s, hd * bs, bs, 1])), z["kt"]))
    # the merged output (B, S, N) written by the kernel, read by the out-projection
    writes.append(("merged", by("merged", extent(0, (b, h, s, hd), [s * n, hd, n, 1])),
                   z["merged"]))
    for what, rng, region in writes + reads:
        assert inside(rng, region), (what, rng, region)
        assert rng[1] <= z["total"][1]

    # the kernel's 32-bit quantities: DMA lane offsets within a tile (K^T: 64 d-rows of k_st
    # elements; rows: 64 key rows), the flag that keeps them on the DMA path, workgroup counts
    k_st = 3 * n if packed else bs
    v_st = 3 * n if packed else n
    k_rows = BN if packed else hd
    assert k_rows * k_st * ES < 2 ** 31 and BN * v_st * ES < 2 ** 31
    assert 2 * ((k_rows - 1) * k_st + 8 * 7 + 7) < 2 ** 32
    items = b * h * -(-s // 256)
    assert items < 2 ** 31 and items * -(-s // BN) < 2 ** 30
    # the attention's own workspace at this size (1920 items, a last round of 384 of 512
    # resident: the last 128 items in 2 pieces) is the split counters plus 256 partials, which
    # fit the region reserved for it and the kernel's 32-bit buffer offsets
    ws = attn_ws_bytes(lib, b, s, n, h, packed)
    assert ws == COUNTER_BYTES + 128 * 2 * 256 * (hd + 2) * 4
    assert ws <= z["attn"][1] - z["attn"][0] and ws < 2 ** 31


def test_one_pass_above_1500_rows_is_refused():
    """The library still refuses a single pass of more than 1500 rows (passes of whole windows
    otherwise)."""
    lib = L.load()
    d = L.EncoderAttnDesc()
    d.dtype, d.batch, d.seq, d.n_state, d.n_head = L.BF16, 1, 1501, 1280, 20
    got = ctypes.c_size_t(0)
    assert lib.ffai_encoder_attn_workspace_bytes(ctypes.byref(d), ctypes.byref(got)) == \
        L.FFAI_ERR_INVALID


@pytest.mark.parametrize("b,s,n,h", [(6, 300, 1280, 20), (4, 500, 768, 12), (3, 700, 1024, 16)])
def test_a_shorter_last_pass_fits_the_attention_region(b, s, n, h):
    """A call whose last pass holds fewer windows: that pass's smaller grid splits its keys into
    more pieces and can need more attention workspace than a full pass. The call's attention
    region must hold the largest need of any pass (large-v3, small and medium widths)."""
    lib = L.load()
    wpp = max(1, min(b, 1500 // s))
    rem = b % wpp
    assert rem, "each shape ends with a shorter pass"
    need_full = max(attn_ws_bytes(lib, wpp, s, n, h, p) for p in (False, True))
    need_rem = max(attn_ws_bytes(lib, rem, s, n, h, p) for p in (False, True))
    assert need_rem > need_full  # the case a region sized by the first pass alone misses
    d = L.EncoderAttnDesc()
    d.dtype, d.batch, d.seq, d.n_state, d.n_head = L.BF16, b, s, n, h
    got = ctypes.c_size_t(0)
    assert lib.ffai_encoder_attn_workspace_bytes(ctypes.byref(d), ctypes.byref(got)) == L.FFAI_OK
    full = layout(lib, wpp, s, n, h)
    others = full["total"][1] - (full["attn"][1] - full["attn"][0])  # q, kt, v, merged, gemm
    attn_region = got.value - others
    assert attn_region == align256(max(need_full, need_rem, COUNTER_BYTES))
