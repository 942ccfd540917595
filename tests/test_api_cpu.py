"""C ABI and host logic on the CPU (no GPU calls): the library loads and exports every symbol the
header declares, descriptors initialise as documented, the serves predicate and the decline
contract of the reference's attend / attend_merged / serves hold (flash_attn.rs:103-264,
1024-1039)."""

from __future__ import annotations

import ctypes

import pytest

from ffai_amd import _lib as L

FAKE = 0x10000  # a non-null "device" address: no test below reaches a HIP call


@pytest.fixture(scope="module")
def lib():
    return L.load()


def view(dims, dtype=L.F32, on_device=1, strides=None, data=FAKE):
    v = L.TensorView()
    v.data = data
    v.dtype = dtype
    v.on_device = on_device
    dims = list(dims) + [1] * (4 - len(dims))
    if strides is None:
        strides = [0] * 4
        acc = 1
        for i in range(3, -1, -1):
            strides[i] = acc
            acc *= dims[i]
    for i in range(4):
        v.dims[i] = dims[i]
        v.strides[i] = strides[i]
    return v


def attend_rc(lib, q, kt, v, masked=0, out=None):
    out = out or view((q.dims[0], q.dims[1], q.dims[2], 64))
    return lib.ffai_attend(ctypes.byref(q), ctypes.byref(kt), ctypes.byref(v), masked,
                           ctypes.byref(out), None, 0, None)


def test_exports_every_header_symbol(lib):
    names = L.header_functions()
    assert len(names) >= 12
    for n in names:
        assert hasattr(lib, n), n
    assert lib.ffai_attn_abi_version() == L.ABI_VERSION


def test_desc_init_packed_strides(lib):
    d = L.AttnDesc()
    lib.ffai_attn_desc_init(ctypes.byref(d), L.BF16, L.BF16, L.BF16, 2, 12, 2, 100, 300, 128,
                            L.K_TRANSPOSED)
    assert list(d.q_strides) == [12 * 100 * 128, 100 * 128, 128, 1]
    assert list(d.k_strides) == [2 * 128 * 300, 128 * 300, 300, 1]
    assert list(d.v_strides) == [2 * 300 * 128, 300 * 128, 128, 1]
    assert list(d.o_strides) == [12 * 100 * 128, 100 * 128, 128, 1]
    assert d.scale == 1.0 and d.causal == 0 and not d.kv_lens
    lib.ffai_attn_desc_init(ctypes.byref(d), L.F32, L.F32, L.F32, 1, 1, 1, 5, 7, 64, L.K_ROWS)
    assert list(d.k_strides) == [7 * 64, 7 * 64, 64, 1]


def desc(lib, qd, kvd, od, b, hq, hkv, tq, tk, d, layout=L.K_ROWS):
    x = L.AttnDesc()
    lib.ffai_attn_desc_init(ctypes.byref(x), qd, kvd, od, b, hq, hkv, tq, tk, d, layout)
    return x


@pytest.mark.parametrize("args,served", [
    ((L.BF16, L.BF16, L.BF16, 16, 20, 20, 1500, 1500, 64), True),
    ((L.BF16, L.BF16, L.F32, 1, 12, 2, 4096, 4096, 128), True),
    ((L.F16, L.F16, L.F16, 1, 4, 4, 10, 10, 64), True),
    ((L.F32, L.F32, L.F32, 1, 6, 6, 1500, 1500, 64), True),
    ((L.F32, L.F16, L.F32, 1, 6, 6, 1, 1500, 64), True),   # reference f16-K/V decode arm
    ((L.F32, L.BF16, L.F32, 5, 16, 16, 1, 448, 64), True),
    ((L.F32, L.F32, L.F32, 1, 6, 6, 100, 100, 128), False),  # f32 serves head_dim 64 only
    ((L.BF16, L.F32, L.BF16, 1, 6, 6, 100, 100, 64), False),  # mixed 16-bit/f32
    ((L.BF16, L.BF16, L.F16, 1, 6, 6, 100, 100, 64), False),  # bf16 in, f16 out
    ((L.BF16, L.BF16, L.BF16, 1, 6, 6, 100, 100, 96), False),  # head_dim 96
])
def test_serves_predicate(lib, args, served):
    d = desc(lib, *args)
    assert lib.ffai_attn_serves(ctypes.byref(d)) == int(served)
    n = ctypes.c_size_t(0)
    rc = lib.ffai_attn_workspace_bytes(ctypes.byref(d), ctypes.byref(n))
    assert rc == (L.FFAI_OK if served else L.FFAI_DECLINED)


def test_fwd_declines_and_rejects_without_touching_the_gpu(lib):
    d = desc(lib, L.BF16, L.BF16, L.BF16, 1, 6, 6, 100, 100, 96)
    assert lib.ffai_attn_fwd(ctypes.byref(d), FAKE, FAKE, FAKE, FAKE, None, 0, None) == L.FFAI_DECLINED
    d = desc(lib, L.BF16, L.BF16, L.BF16, 1, 6, 4, 100, 100, 64)  # 6 % 4 != 0
    assert lib.ffai_attn_fwd(ctypes.byref(d), FAKE, FAKE, FAKE, FAKE, None, 0, None) == L.FFAI_ERR_INVALID
    d = desc(lib, L.BF16, L.BF16, L.BF16, 1, 6, 6, 100, 100, 64)
    d.scale = -1.0
    assert lib.ffai_attn_fwd(ctypes.byref(d), FAKE, FAKE, FAKE, FAKE, None, 0, None) == L.FFAI_ERR_INVALID
    assert "scale" in L.last_error()
    d = desc(lib, L.BF16, L.BF16, L.BF16, 1, 6, 6, 100, 100, 64)
    d.q_strides[3] = 2
    assert lib.ffai_attn_fwd(ctypes.byref(d), FAKE, FAKE, FAKE, FAKE, None, 0, None) == L.FFAI_ERR_INVALID
    d = desc(lib, L.BF16, L.BF16, L.BF16, 1, 6, 6, 100, 100, 64)
    assert lib.ffai_attn_fwd(ctypes.byref(d), None, FAKE, FAKE, FAKE, None, 0, None) == L.FFAI_ERR_INVALID


@pytest.mark.parametrize("bad", [float("nan"), -float("nan"), float("inf"), -float("inf"), 0.0,
                                 -0.0])
def test_non_finite_or_non_positive_scale_is_an_error(lib, bad):
    """The descriptor check rejects a NaN, infinite or non-positive scale before any launch (the
    host code is built with IEEE NaN semantics; only device code assumes no NaNs)."""
    d = desc(lib, L.BF16, L.BF16, L.BF16, 1, 6, 6, 100, 100, 64)
    d.scale = bad
    assert lib.ffai_attn_serves(ctypes.byref(d)) == 0
    assert lib.ffai_attn_fwd(ctypes.byref(d), FAKE, FAKE, FAKE, FAKE, None, 0, None) == L.FFAI_ERR_INVALID
    assert "scale" in L.last_error()
    n = ctypes.c_size_t(0)
    assert lib.ffai_attn_workspace_bytes(ctypes.byref(d), ctypes.byref(n)) == L.FFAI_ERR_INVALID


def test_workspace_only_for_split_shapes(lib):
    n = ctypes.c_size_t(0)
    # 1024 items of 256 rows: two whole rounds of the 512 resident slots, nothing split
    whole = desc(lib, L.BF16, L.BF16, L.BF16, 16, 16, 16, 1024, 1024, 64, L.K_TRANSPOSED)
    assert lib.ffai_attn_workspace_bytes(ctypes.byref(whole), ctypes.byref(n)) == L.FFAI_OK
    assert n.value == 0
    # whisper-large-v3: the last 128 of 1920 items in 2 pieces -> the counters plus 128 x 2
    # partials of 256 rows x (64 + 2) floats
    big = desc(lib, L.BF16, L.BF16, L.BF16, 16, 20, 20, 1500, 1500, 64, L.K_TRANSPOSED)
    assert lib.ffai_attn_workspace_bytes(ctypes.byref(big), ctypes.byref(n)) == L.FFAI_OK
    assert n.value == 4096 + 128 * 2 * 256 * 66 * 4
    beam = desc(lib, L.BF16, L.BF16, L.F32, 1, 16, 16, 5, 1500, 64, L.K_TRANSPOSED)
    assert lib.ffai_attn_workspace_bytes(ctypes.byref(beam), ctypes.byref(n)) == L.FFAI_OK
    # decode shape: per-split partials (O and (m, l) for 5 rows x 16 heads) plus counters
    assert n.value > 0 and n.value % 16 == 0 and n.value >= 2 * 5 * 16 * 66 * 4


# ---------------------------------------------------------------------------------------------
# the reference's decline contract (flash_attn.rs:218-264, 1024-1039)
# ---------------------------------------------------------------------------------------------

def test_declines_unsupported_shapes_like_the_reference(lib):
    """flash_attn.rs:1024-1039: qlen 1 with 1 key, and masked attention, both decline."""
    q, kt, v = view((1, 4, 1, 64)), view((1, 4, 64, 1)), view((1, 4, 1, 64))
    assert attend_rc(lib, q, kt, v) == L.FFAI_DECLINED
    q, kt, v = view((1, 4, 512, 64)), view((1, 4, 64, 512)), view((1, 4, 512, 64))
    assert attend_rc(lib, q, kt, v, masked=1) == L.FFAI_DECLINED


@pytest.mark.parametrize("case", ["q_f16", "batch2", "hd128", "short_encoder", "qlen_between",
                                  "host", "k_f16_v_f32", "heads_mismatch"])
def test_attend_decline_rules(lib, case):
    q, kt, v = view((1, 4, 512, 64)), view((1, 4, 64, 512)), view((1, 4, 512, 64))
    if case == "q_f16":
        q = view((1, 4, 512, 64), dtype=L.F16)
    elif case == "batch2":
        q = view((2, 4, 512, 64))
    elif case == "hd128":
        q = view((1, 4, 512, 128))
    elif case == "short_encoder":  # qlen == keys < MIN_SEQ (256)
        q, kt, v = view((1, 4, 200, 64)), view((1, 4, 64, 200)), view((1, 4, 200, 64))
    elif case == "qlen_between":
        q = view((1, 4, 7, 64))
    elif case == "host":
        q = view((1, 4, 512, 64), on_device=0)
    elif case == "k_f16_v_f32":
        kt = view((1, 4, 64, 512), dtype=L.F16)
    elif case == "heads_mismatch":
        kt = view((1, 3, 64, 512))
    assert attend_rc(lib, q, kt, v) == L.FFAI_DECLINED


def test_attend_errors_match_cpu_fwd_bails(lib):
    # f16 K/V at the encoder shape passes attend's checks but bails in cpu_fwd
    # (flash_attn.rs:289-296 then 357-359): an error, not a decline
    q = view((1, 4, 512, 64))
    kt, v = view((1, 4, 64, 512), dtype=L.F16), view((1, 4, 512, 64), dtype=L.F16)
    assert attend_rc(lib, q, kt, v) == L.FFAI_ERR_INVALID
    # non-contiguous operands bail (flash_attn.rs:360-363)
    q = view((1, 4, 512, 64), strides=[4 * 512 * 128, 512 * 128, 128, 1])
    kt, v = view((1, 4, 64, 512)), view((1, 4, 512, 64))
    assert attend_rc(lib, q, kt, v) == L.FFAI_ERR_INVALID


def test_attend_merged_decline_rules(lib):
    out = view((1, 300, 4 * 64))

    def rc(q, kt, v):
        return lib.ffai_attend_merged(ctypes.byref(q), ctypes.byref(kt), ctypes.byref(v),
                                      ctypes.byref(out), None, 0, None)

    ok = (view((1, 4, 300, 64)), view((1, 4, 64, 300)), view((1, 4, 300, 64)))
    assert rc(view((1, 4, 300, 64), dtype=L.BF16), ok[1], ok[2]) == L.FFAI_DECLINED
    assert rc(view((1, 4, 1, 64)), ok[1], ok[2]) == L.FFAI_DECLINED     # qlen != keys
    short = (view((1, 4, 255, 64)), view((1, 4, 64, 255)), view((1, 4, 255, 64)))
    assert rc(*short) == L.FFAI_DECLINED                                 # keys < 256
    assert rc(view((1, 4, 300, 64), on_device=0), ok[1], ok[2]) == L.FFAI_DECLINED


def test_serves_tracks_the_decode_floor_knob(lib):
    """The A1 lesson (flash_attn.rs:113-125): serves must apply the same floor the decode path
    applies, so raising DECODE_MIN_KEYS above the key count turns serves off."""
    kt, v = view((1, 16, 64, 1500)), view((1, 16, 1500, 64))
    saved = lib.ffai_get_decode_min_keys()
    try:
        assert lib.ffai_serves(ctypes.byref(kt), ctypes.byref(v)) == 1
        lib.ffai_set_decode_min_keys(2000)
        assert lib.ffai_serves(ctypes.byref(kt), ctypes.byref(v)) == 0
        q = view((1, 16, 1, 64))
        assert attend_rc(lib, q, kt, v) == L.FFAI_DECLINED  # and the kernel declines too
    finally:
        lib.ffai_set_decode_min_keys(saved)
    short_kt, short_v = view((1, 16, 64, 200)), view((1, 16, 200, 64))
    assert lib.ffai_serves(ctypes.byref(short_kt), ctypes.byref(short_v)) == 0  # < MIN_SEQ
    assert lib.ffai_serves(ctypes.byref(view((1, 16, 64, 1500), on_device=0)),
                           ctypes.byref(v)) == 0


def test_python_mirror_declines_host_tensors():
    import torch

    from ffai_amd import flash_attn as fa

    q = torch.zeros(1, 4, 512, 64)
    kt = torch.zeros(1, 4, 64, 512)
    v = torch.zeros(1, 4, 512, 64)
    assert fa.attend(q, kt, v) is None
    assert fa.attend_merged(q, kt, v) is None
    assert fa.serves(kt, v) is False


# ---------------------------------------------------------------------------------------------
# decode-state entry points (include/ffai_kv.h): argument checks happen before any HIP call
# ---------------------------------------------------------------------------------------------

def _cache(dtype=L.BF16, slots=5, heads=16, cap=448, d=64, data=FAKE):
    c = L.KVCacheView()
    c.k, c.v, c.lens = data, data + 0x100000, data + 0x200000
    c.dtype, c.slots, c.heads, c.capacity, c.head_dim = dtype, slots, heads, cap, d
    c.strides[0], c.strides[1], c.strides[2] = heads * cap * d, cap * d, d
    return c


def test_kv_append_rejects_bad_arguments(lib):
    c = _cache()
    ok = dict(src=FAKE, dt=L.F32, t=1, ss=16 * 64, rs=16 * 64)

    def rc(cache=c, **kw):
        a = {**ok, **kw}
        return lib.ffai_kv_append(ctypes.byref(cache), a["src"], a["src"], a["dt"], a["t"],
                                  a["ss"], a["rs"], None)

    assert rc(dt=7) == L.FFAI_ERR_INVALID
    assert rc(src=None) == L.FFAI_ERR_INVALID
    assert rc(t=-1) == L.FFAI_ERR_INVALID
    assert rc(rs=10) == L.FFAI_ERR_INVALID          # shorter than heads * head_dim
    assert rc(cache=_cache(d=60)) == L.FFAI_ERR_INVALID  # head_dim not a multiple of 8
    assert rc(cache=_cache(data=0)) == L.FFAI_ERR_INVALID
    assert rc(t=0) == L.FFAI_OK                      # nothing to do, nothing launched


def test_kv_gather_rejects_bad_arguments(lib):
    a, b = _cache(), _cache(data=FAKE + 0x1000000)

    def rc(dst=a, src=b, parent=FAKE, layers=1, ls=0, lls=0):
        return lib.ffai_kv_gather(ctypes.byref(dst), ctypes.byref(src), parent, layers, ls, lls,
                                  None)

    assert rc(src=a) == L.FFAI_ERR_INVALID           # in place
    assert rc(parent=None) == L.FFAI_ERR_INVALID
    assert rc(src=_cache(dtype=L.F16, data=FAKE + 0x2000000)) == L.FFAI_ERR_INVALID
    assert "dtype" in L.last_error()
    assert rc(layers=0) == L.FFAI_ERR_INVALID
    assert rc(layers=24, ls=0, lls=5) == L.FFAI_ERR_INVALID   # layers would overlap
    assert rc(layers=24, ls=1 << 20, lls=2) == L.FFAI_ERR_INVALID  # lens rows overlap
    assert "layer strides" in L.last_error()


def test_kv_advance_rejects_bad_arguments(lib):
    c = _cache()

    def rc(cache=c, t=1, layers=24, lls=5):
        return lib.ffai_kv_advance(ctypes.byref(cache), t, layers, lls, None)

    assert rc(t=-1) == L.FFAI_ERR_INVALID
    assert rc(layers=0) == L.FFAI_ERR_INVALID
    assert rc(layers=65536) == L.FFAI_ERR_INVALID
    assert rc(lls=4) == L.FFAI_ERR_INVALID             # the layers' lengths would overlap
    assert "lens_layer_stride" in L.last_error()
    assert rc(cache=_cache(data=0)) == L.FFAI_ERR_INVALID
    assert rc(t=0) == L.FFAI_OK                        # nothing to do, nothing launched


def test_gemv_qkv_cache_rejects_bad_arguments(lib):
    c = _cache()   # 5 slots, 16 heads x 64: out_dim 3 x 1024

    def rc(w=FAKE, bias=None, in_dim=1024, x=FAKE, rows=5, xs=1024, q=FAKE, qs=1024, cache=c):
        return lib.ffai_gemv_f16_qkv_cache(w, bias, in_dim, x, rows, xs, q, qs,
                                           ctypes.byref(cache), None)

    assert rc(w=None) == L.FFAI_ERR_INVALID
    assert rc(q=None) == L.FFAI_ERR_INVALID
    assert rc(in_dim=1020) == L.FFAI_ERR_INVALID       # f16_gemv.rs:101-103's rule
    assert rc(rows=6) == L.FFAI_ERR_INVALID            # more beams than cache slots
    assert "slots" in L.last_error()
    assert rc(rows=17, cache=_cache(slots=20)) == L.FFAI_ERR_INVALID
    assert rc(qs=1000) == L.FFAI_ERR_INVALID           # q rows shorter than heads * head_dim
    assert rc(xs=1000) == L.FFAI_ERR_INVALID
    assert rc(bias=FAKE + 2) == L.FFAI_ERR_INVALID     # misaligned bias
    assert rc(cache=_cache(dtype=7)) == L.FFAI_ERR_INVALID
    assert rc(cache=_cache(d=60)) == L.FFAI_ERR_INVALID
    assert rc(cache=_cache(data=0)) == L.FFAI_ERR_INVALID


def test_cross_kv_build_rejects_bad_arguments(lib):
    def rc(t=1500, heads=16, d=64, rs=1024, layout=L.K_TRANSPOSED, odt=L.BF16):
        return lib.ffai_cross_kv_build(FAKE, FAKE, L.F32, t, heads, d, rs, FAKE, FAKE, odt, layout,
                                       None)
    assert rc(t=0) == L.FFAI_ERR_INVALID
    assert rc(d=256) == L.FFAI_ERR_INVALID
    assert rc(rs=1000) == L.FFAI_ERR_INVALID
    assert rc(layout=9) == L.FFAI_ERR_INVALID
    assert rc(odt=5) == L.FFAI_ERR_INVALID


def test_encoder_attn_rejects_bad_arguments(lib):
    def desc(dtype=L.BF16, batch=1, seq=1500, n_state=1280, n_head=20):
        d = L.EncoderAttnDesc()
        d.dtype, d.batch, d.seq, d.n_state, d.n_head = dtype, batch, seq, n_state, n_head
        return d

    n = ctypes.c_size_t(0)
    assert lib.ffai_encoder_attn_workspace_bytes(ctypes.byref(desc()), ctypes.byref(n)) == L.FFAI_OK
    act = 1500 * 1280 * 2
    assert n.value >= 4 * act  # q, k^T, v and the merged output at least
    for bad in (desc(dtype=L.F32), desc(n_head=7), desc(n_state=640, n_head=20), desc(seq=0),
                desc(seq=1501)):  # one window of more than 1500 frames: a pass above 1500 rows
        assert lib.ffai_encoder_attn_workspace_bytes(ctypes.byref(bad), ctypes.byref(n)) == \
            L.FFAI_ERR_INVALID
    # the large-v3 batch of 16 windows runs as 16 passes of one window through one window's
    # workspace; 5 windows of 300 frames fit one pass
    one = ctypes.c_size_t(0)
    assert lib.ffai_encoder_attn_workspace_bytes(ctypes.byref(desc()), ctypes.byref(one)) == L.FFAI_OK
    assert lib.ffai_encoder_attn_workspace_bytes(ctypes.byref(desc(batch=16)), ctypes.byref(n)) == L.FFAI_OK
    assert n.value == one.value
    five = ctypes.c_size_t(0)
    assert lib.ffai_encoder_attn_workspace_bytes(ctypes.byref(desc(batch=5, seq=300)),
                                                 ctypes.byref(five)) == L.FFAI_OK
    assert lib.ffai_encoder_attn_workspace_bytes(ctypes.byref(desc(batch=10, seq=300)),
                                                 ctypes.byref(n)) == L.FFAI_OK
    assert n.value == five.value  # two full passes
    # eleven: a last pass of one window, whose smaller grid splits its keys and needs more
    # attention workspace than a full pass; the call's workspace holds both
    assert lib.ffai_encoder_attn_workspace_bytes(ctypes.byref(desc(batch=11, seq=300)),
                                                 ctypes.byref(n)) == L.FFAI_OK
    assert n.value > five.value
    w = L.EncoderAttnWeights()  # all null
    assert lib.ffai_encoder_attn_fwd(ctypes.byref(desc()), FAKE, ctypes.byref(w), FAKE, FAKE,
                                     1 << 40, None) == L.FFAI_ERR_INVALID
    assert "null" in L.last_error()
    # a packed projection weight without its packed bias, and no separate weights either
    w = L.EncoderAttnWeights(wqkv=FAKE, wo=FAKE, bo=FAKE)
    assert lib.ffai_encoder_attn_fwd(ctypes.byref(desc()), FAKE, ctypes.byref(w), FAKE, FAKE,
                                     1 << 40, None) == L.FFAI_ERR_INVALID
    assert "wqkv" in L.last_error()


def test_gemv_entry_points_reject_bad_arguments(lib):
    assert lib.ffai_gemv_f16(FAKE, 1024, 1020, FAKE, 5, 1020, FAKE, 1024, None) == L.FFAI_ERR_INVALID
    assert lib.ffai_gemv_f16(FAKE, 1024, 1024, FAKE, 17, 1024, FAKE, 1024, None) == L.FFAI_ERR_INVALID
    assert lib.ffai_gemv_f16(None, 1024, 1024, FAKE, 5, 1024, FAKE, 1024, None) == L.FFAI_ERR_INVALID
    # f16_gemv.rs:101-103 declines in_dim not a multiple of 8; vocab_int8.rs:131-133 needs a
    # block a multiple of 32 that tiles d
    assert lib.ffai_vocab_int8_quantize(FAKE, L.F32, 100, 384, 48, FAKE, FAKE, FAKE, None) == L.FFAI_ERR_INVALID
    assert lib.ffai_vocab_int8_quantize(FAKE, L.F32, 100, 400, 32, FAKE, FAKE, FAKE, None) == L.FFAI_ERR_INVALID
    n = ctypes.c_size_t(0)
    assert lib.ffai_vocab_int8_workspace_bytes(1024, 5, ctypes.byref(n)) == L.FFAI_OK
    assert n.value >= 5 * 1024 + 5 * 4
    assert lib.ffai_vocab_int8_logits(FAKE, FAKE, FAKE, 51865, 1024, 32, FAKE, 5, 1024, FAKE,
                                      51865, FAKE, 1, None) == L.FFAI_ERR_WORKSPACE


# ---------------------------------------------------------------------------------------------
# launch plans of the benchmarked workloads (host logic only)
# ---------------------------------------------------------------------------------------------

def _plan(lib, *args, causal=0):
    d = desc(lib, *args)
    d.causal = causal
    info = (ctypes.c_int32 * 5)()
    assert lib.ffai_attn_plan_info(ctypes.byref(d), info) == L.FFAI_OK
    sp = (ctypes.c_int32 * 3)()
    assert lib.ffai_attn_plan_splits(ctypes.byref(d), sp) == L.FFAI_OK
    return list(info), list(sp)


@pytest.mark.parametrize("args,causal,info,splits", [
    # whisper-large-v3 encoder: 1920 items of 256 rows, a last round of 384 of 512 slots: the
    # last 128 items in 2 pieces, so that the last round holds 256 whole items + 256 pieces
    ((L.BF16, L.BF16, L.BF16, 16, 20, 20, 1500, 1500, 64, L.K_TRANSPOSED), 0,
     [0, 2, 2, 12, 2048], [1920, 1792, 1920]),
    # whisper-small: 576 items on 512 resident, the last 64 in 4 pieces
    ((L.BF16, L.BF16, L.BF16, 8, 12, 12, 1500, 1500, 64, L.K_TRANSPOSED), 0,
     [0, 2, 4, 6, 768], [576, 512, 576]),
    # whisper-tiny f32: 72 items in 6 pieces (512 resident two-per-CU slots)
    ((L.F32, L.F32, L.F32, 1, 6, 6, 1500, 1500, 64, L.K_TRANSPOSED), 0,
     [0, 1, 6, 4, 432], [72, 0, 72]),
    # Qwen2-VL-2B prefill: 384 items longest first, the 192 longest in 2 pieces
    ((L.BF16, L.BF16, L.BF16, 1, 12, 2, 4096, 4096, 128, L.K_ROWS), 1,
     [0, 1, 2, 32, 576], [384, 0, 192]),
    # the same at batch 4: the longest item is below a slot's share, nothing split
    ((L.BF16, L.BF16, L.BF16, 4, 12, 2, 4096, 4096, 128, L.K_ROWS), 1,
     [0, 1, 1, 64, 1536], [1536, 0, 0]),
    # a whisper-large-v3 window (encoder block): 240 items, whole
    ((L.BF16, L.BF16, L.BF16, 1, 20, 20, 1500, 1500, 64, L.K_ROWS), 0,
     [0, 1, 1, 24, 240], [240, 0, 0]),
    # prompt step cross-attention: 228 tokens x 16 heads, one-wave items in 6 pieces (768
    # workgroups, three per CU)
    ((L.BF16, L.BF16, L.F32, 1, 16, 16, 228, 1500, 64, L.K_TRANSPOSED), 0,
     [0, 0, 6, 4, 768], [128, 0, 128]),
    # beam-5 cross-attention: the decode kernel, 8 pieces of 3 tiles per head (128 workgroups)
    ((L.BF16, L.BF16, L.F32, 1, 16, 16, 5, 1500, 64, L.K_TRANSPOSED), 0,
     [1, 4, 8, 3, 128], [0, 0, 0]),
    # the reference's cross-attention arm (one beam: f32 q, f16 K^T/V, 1500 frames, 16 heads):
    # the f32 decode kernel, 8 pieces of 3 tiles per head
    ((L.F32, L.F16, L.F32, 1, 16, 16, 1, 1500, 64, L.K_TRANSPOSED), 0,
     [1, 4, 8, 3, 128], [0, 0, 0]),
    # its self-attention arm (f32 q and K^T/V, 448 cached positions): one workgroup of 8 waves per
    # head covers the 7 tiles in one round of loads, unsplit
    ((L.F32, L.F32, L.F32, 1, 16, 16, 1, 448, 64, L.K_TRANSPOSED), 0,
     [1, 8, 1, 7, 16], [0, 0, 0]),
    # five beams' f32 self-attention in one call (80 units)
    ((L.F32, L.F32, L.F32, 5, 16, 16, 1, 448, 64, L.K_ROWS), 0,
     [1, 8, 1, 7, 80], [0, 0, 0]),
])
def test_plans_of_the_benchmarked_workloads(lib, args, causal, info, splits):
    got_info, got_splits = _plan(lib, *args, causal=causal)
    assert (got_info, got_splits) == (info, splits)


def test_split_override_and_its_workspace(lib):
    """The override forces the layout and the workspace follows it; (0, 0) restores the plan."""
    prev = L.get_fwd_split_override()
    try:
        args = (L.BF16, L.BF16, L.BF16, 16, 20, 20, 1500, 1500, 64, L.K_TRANSPOSED)
        L.set_fwd_split_override(100, 3)
        info, sp = _plan(lib, *args)
        assert info[2] == 3 and sp == [1920, 1820, 1920] and info[4] == 1820 + 300
        d = desc(lib, *args)
        n = ctypes.c_size_t(0)
        assert lib.ffai_attn_workspace_bytes(ctypes.byref(d), ctypes.byref(n)) == L.FFAI_OK
        assert n.value == 4096 + 100 * 3 * 256 * 66 * 4   # counters + partials of 300 pieces
        L.set_fwd_split_override(-1, 1)                     # nothing split
        assert _plan(lib, *args)[1] == [1920, 0, 0]
        L.set_fwd_split_override(0, 0)                      # the planner's own layout
        assert _plan(lib, *args)[1] == [1920, 1792, 1920]
        assert L.get_fwd_split_override() == (0, 0)
    finally:
        L.set_fwd_split_override(*prev)


def test_one_wave_grids_stay_within_one_round(lib):
    """One-wave 16-bit grids (query runs under 256 rows) are split towards the 768 slots of three
    workgroups per CU and never past them: a 769th workgroup would start a second round."""
    n = 0
    for tq in (33, 64, 100, 228):
        for heads in (1, 2, 5, 16, 24):
            for b in (1, 3):
                for tk in (64, 700, 1500, 3000):
                    for dt in (L.BF16, L.F16):
                        info, _ = _plan(lib, dt, dt, L.F32, b, heads, heads, tq, tk, 64, L.K_ROWS)
                        if info[0] != 0 or info[1] != 0:  # the fused kernel's one-wave shape only
                            continue
                        n += 1
                        items = b * heads * ((tq + 31) // 32)
                        assert info[4] <= max(768, items), (dt, b, heads, tq, tk, info)
                        if items < 384 and tk >= 128:   # room for two pieces of a tile or more
                            assert info[2] >= 2, (dt, b, heads, tq, tk, info)
    assert n > 50
