"""Register budget of the built kernels (CPU; reads what the last build recorded).

The fused kernels run at their register budget: the 16-bit encoder kernel (four waves x 64 rows)
needs <= 256 VGPRs for two workgroups per CU, and a small change of its code can make the compiler
spill to scratch instead. The results stay correct, so no parity test notices; the kernel runs
several times slower (an index rewrite once cost the large-v3 encoder 3x). `ffai_amd/build.py`
writes the compiler's kernel-resource-usage remarks to `_build/resource_usage.json` at every
build; these tests read it. The diagnostic library's kernels (built with FFAI_STAMPS, recorded
under "stamps:" names) are held to the same budget, so that the phase times they record are
those of the kernels as they run without instrumentation.
"""

from __future__ import annotations

import json
import os

import pytest

from ffai_amd import build as native_build


@pytest.fixture(scope="module")
def usage():
    if not os.path.exists(native_build.RESOURCES_PATH):
        pytest.skip("the library has not been built here (no resource report)")
    with open(native_build.RESOURCES_PATH) as f:
        return json.load(f)


def _kernels(usage, needle):
    return {k: v for k, v in usage.items() if needle in k}


def test_report_covers_the_attention_kernels(usage):
    assert len(_kernels(usage, "fwd_kernel")) >= 40
    assert len(_kernels(usage, "stamps:")) >= 100
    assert len(_kernels(usage, "decode_kernel")) >= 80
    for name, v in usage.items():
        assert {"vgprs", "scratch", "occupancy", "vgpr_spill"} <= set(v), name


@pytest.mark.parametrize("needle", ["fwd_kernel", "decode_kernel", "gemv", "kv_", "cross_",
                                    "vocab_"])
def test_no_vector_register_spills(usage, needle):
    spilled = {k: (v["vgpr_spill"], v["scratch"]) for k, v in _kernels(usage, needle).items()
               if v["vgpr_spill"] or v["scratch"]}
    assert not spilled, f"kernels spilling to scratch (VGPRs spilled, bytes per lane): {spilled}"


def test_encoder_kernels_keep_two_waves_per_simd(usage):
    # fwd_kernel<MODE, KV, OUT, 64, KT, 4 waves, 2 column blocks>: the encoder launch shape, two
    # four-wave workgroups per CU; head_dim 128 four-wave kernels likewise
    enc = {k: v for k, v in _kernels(usage, "fwd_kernel").items()
           if "ELi64ELb" in k and ("ELi4ELi2EEEvNS_9FwdParamsE" in k)}
    d128 = {k: v for k, v in _kernels(usage, "fwd_kernel").items()
            if "ELi128ELb" in k and "ELi4ELi1EEEvNS_9FwdParamsE" in k}
    assert enc and d128
    for k, v in {**enc, **d128}.items():
        assert v["occupancy"] >= 2 and v["vgprs"] + v["agprs"] <= 256, (k, v)


def test_no_scalar_register_spills(usage):
    """SGPR spills are parked in vector-register lanes (v_writelane / v_readlane), correct but a
    change of the code the kernels were measured with: the fused kernel has none. The decode
    kernel has none either, except its head_dim-128 K^T instantiations (no workload runs them:
    head_dim-128 decode caches keep K as rows), which park at most a few predicates of the
    register-staging tail path (checked in their ISA). The diagnostic library's kernels are
    exempt: their timers' scalar registers may be parked the same way (a few lane moves per
    tile), while their vector registers stay within budget (the test above)."""
    product = {k: v for k, v in usage.items() if not k.startswith("stamps:")}
    fwd = {k: v["sgpr_spill"] for k, v in _kernels(product, "fwd_kernel").items()
           if v.get("sgpr_spill")}
    assert not fwd, fwd
    dec = {k: v["sgpr_spill"] for k, v in _kernels(product, "decode_kernel").items()
           if v.get("sgpr_spill")}
    d128_kt = {k: n for k, n in dec.items() if "ELi128ELb1E" in k}
    assert dec.keys() == d128_kt.keys(), sorted(set(dec) - set(d128_kt))
    assert all(n <= 8 for n in d128_kt.values()), d128_kt


def test_phase_stamps_only_in_the_diagnostic_library():
    """The phase-timing instrumentation is compiled only into libffai_attn_stamps.so (bench.py
    --legs stamps); the product library has none of it."""
    import ctypes

    from ffai_amd import _lib

    if not os.path.exists(native_build.STAMPS_LIB_PATH):
        pytest.skip("the diagnostic library has not been built here")
    assert not hasattr(_lib.load(), "ffai_stamps_set")
    assert hasattr(ctypes.CDLL(native_build.STAMPS_LIB_PATH), "ffai_stamps_set")
