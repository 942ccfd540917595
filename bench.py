#!/usr/bin/env python3
"""Benchmark of the fused attention path on one MI355X.

Headline (``value``): encoder self-attention throughput at the whisper-large-v3 shape -- batch 16,
20 heads, T = 1500, head_dim 64, bf16, non-causal, K given transposed (the reference's layout),
scale 1/8 -- over the 32 encoder layers with distinct buffers per layer. One step = the 32 layer
calls. FLOP = 4 * B * H * T^2 * D per layer (flash_probe.rs:432's convention).

Also reported: the beam-5 decode step at the whisper-medium shape (24 layers of decoder
self-attention over ragged per-beam caches plus cross-attention over 1500 shared encoder frames,
bf16 K/V, f32 output), the device-resident decode state of that step (K/V append in place and
beam reorder, with and without the attention calls, and the per-window cross-attention cache
build), the whole whisper-large-v3 encoder self-attention block (hipBLASLt projections around
the fused kernel), the decoder GEMVs of a beam-5 step (f16 projections, int8 vocabulary),
the whisper-tiny f32 and whisper-small bf16 encoders, the
Qwen2-VL-2B-shape causal prefill (12 query heads over 2 K/V heads, head_dim 128, S = 4096), and
the CPU oracle (the reference's algorithm restated in C++/AVX2) timed on this host's cores on a
bounded sample.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--skip-cpu] [--skip-extras] [--eager]
                       [--layers L]
                       [--legs decode,decode_ref,state,block,gemv,tiny,small,prefill,floor,pipes,
                               stamps,keys | none | copy]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2516.6   # MI355X dense bf16 MFMA (256 CU x 2.4 GHz x 4096 FLOP/clk)
PEAK_F32_TFLOPS = 157.3     # MI355X fp32 matrix
PEAK_HBM_GBPS = 8000.0      # MI355X HBM3E


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--skip-extras", action="store_true")
    ap.add_argument("--eager", action="store_true",
                    help="decode leg without HIP graphs (for counter collection)")
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--legs",
                    default="decode,decode_ref,state,block,gemv,gemv_large,tiny,small,prefill,"
                            "floor,pipes,stamps,keys",
                    help="comma list of extra legs beside the headline encoder run: decode, "
                         "decode_ref, state, block, gemv, gemv_large (the decoder GEMVs at "
                         "whisper-large width), tiny, small, prefill, floor, pipes, stamps, keys, "
                         "or 'none'; 'gemv_probe' alone runs only a few decoder GEMV calls "
                         "for counter collection; "
                         "'copy' alone "
                         "runs only the copy calibration used to scale HBM byte counters")
    return ap.parse_args()


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ------------------------------------------------------------------------------------------
# Encoder (headline)
# ------------------------------------------------------------------------------------------

def encoder_bench(torch, fa, steps, warmup, layers, B=16, H=20, T=1500, D=64,
                  dtype="bf16", seed=4, causal=False, H_kv=None, k_mult=1.0):
    """Self-attention over `layers` distinct buffer sets. K is given transposed (B,Hkv,D,T) as
    the reference's encoder produces it, except for the causal prefill (rows, as a decoder's
    cache holds it). FLOP counts only the visible query-key pairs."""
    dev = torch.device("cuda:0")
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    H_kv = H_kv or H
    kt_layout = not causal
    g = torch.Generator(device=dev).manual_seed(seed)
    bufs = []
    for _ in range(layers):
        q = torch.randn(B, H, T, D, generator=g, device=dev).to(tdt)
        if kt_layout:
            k = (torch.randn(B, H_kv, D, T, generator=g, device=dev) * k_mult).to(tdt)
        else:
            k = (torch.randn(B, H_kv, T, D, generator=g, device=dev) * k_mult).to(tdt)
        v = torch.randn(B, H_kv, T, D, generator=g, device=dev).to(tdt)
        o = torch.empty(B, H, T, D, device=dev, dtype=tdt)
        bufs.append((q, k, v, o))
    scale = D ** -0.5
    ws = None
    nbytes = fa.workspace_bytes(*bufs[0], k_transposed=kt_layout, scale=scale, causal=causal)
    if nbytes:
        ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)

    def step():
        for q, k, v, o in bufs:
            r = fa.attention(q, k, v, k_transposed=kt_layout, scale=scale, causal=causal, out=o,
                             workspace=ws)
            assert r is not None

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = e0.elapsed_time(e1)
    pairs = T * (T + 1) / 2 if causal else T * T
    flop_layer = 4.0 * B * H * pairs * D
    launches = steps * layers
    avg_launch_s = gpu_ms * 1e-3 / launches
    esz = 2 if dtype == "bf16" else 4
    return {
        "elapsed_s": wall,
        "gpu_ms": gpu_ms,
        "ms_per_step": gpu_ms / steps,
        "tflops": flop_layer * launches / (gpu_ms * 1e-3) / 1e12,
        "flop_per_launch": flop_layer,
        "avg_launch_us": avg_launch_s * 1e6,
        "bytes_per_launch": float(B * T * D * esz * (2 * H + 2 * H_kv)),
    }


# ------------------------------------------------------------------------------------------
# Copy calibration: a plain device copy of known size, for scaling the HBM byte counters
# ------------------------------------------------------------------------------------------

def copy_bench(torch, steps, nbytes=1 << 30):
    """Copies `nbytes` between two device buffers `steps` times (torch's copy kernel). Under
    rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE each dispatch should read and write `nbytes`; the
    ratio of counted to known bytes is the scale applied to the attention kernels' counters."""
    dev = torch.device("cuda:0")
    src = torch.empty(nbytes // 4, dtype=torch.float32, device=dev).normal_()
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    return {"bytes_each_way": nbytes, "us_per_copy": ms * 1e3,
            "gbps": 2 * nbytes / (ms * 1e-3) / 1e9}


def gemv_probe(torch, calls=3, beams=5, n=1024, vocab=51865):
    """The whisper-medium decoder's GEMV shapes at `beams` beams and its int8 vocabulary
    projection, `calls` eager calls each with fresh weights per shape, untimed: a short program
    for rocprofv3 --pmc (the gemv leg's graphs are too many dispatches for counter collection).
    Returns the algorithmic bytes per call of each shape."""
    from ffai_amd.gemv import F16Gemv, Int8Vocab

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(9)
    out = {}
    for o, i in ((3 * n, n), (n, n), (4 * n, n), (n, 4 * n)):
        m = F16Gemv(torch.randn(o, i, generator=g, device=dev) / i ** 0.5)
        x = torch.randn(beams, i, generator=g, device=dev)
        for _ in range(calls):
            m(x)
        out[f"{o}x{i}"] = o * i * 2 + beams * (i + o) * 4
    iv = Int8Vocab(torch.randn(vocab, n, generator=g, device=dev) / n ** 0.5)
    ws = torch.empty(iv.workspace_bytes(beams), dtype=torch.uint8, device=dev)
    x = torch.randn(beams, n, generator=g, device=dev)
    for _ in range(calls):
        iv(x, workspace=ws)
    torch.cuda.synchronize()
    out[f"vocab {vocab}x{n}"] = vocab * n + vocab * (n // 32) * 4 + vocab * 4 + beams * (n + vocab) * 4
    return {"calls": calls, "beams": beams, "algorithmic_bytes_per_call": out}


# ------------------------------------------------------------------------------------------
# Launch floor: what one launch costs with nothing, or only a bare read, inside it
# ------------------------------------------------------------------------------------------

def floor_bench(torch, steps=50, launches=24, nbytes=6_175_744, sets=3, workgroups=(128, 256, 512)):
    """Per-launch time of an empty kernel and of a bare streaming read of `nbytes` (the
    cross-attention K/V of one whisper-medium layer), each in HIP graphs of `launches` launches
    as a decode step replays them. Reads rotate over `sets` x `launches` distinct regions
    (> 2 x the 256 MB MALL), so every launch reads HBM."""
    import ctypes
    from ffai_amd import _lib

    lib = _lib.load()
    dev = torch.device("cuda:0")
    regions = sets * launches
    buf = torch.zeros(regions * nbytes, dtype=torch.uint8, device=dev)
    out = torch.empty(1024, dtype=torch.float32, device=dev)

    def timed(body):
        graphs = []
        for st in range(sets):
            body(st)
            torch.cuda.synchronize()
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr):
                body(st)
            graphs.append(gr)
        for i in range(5):
            graphs[i % sets].replay()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(steps):
            graphs[i % sets].replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / (steps * launches)

    def stream():
        return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def empty(_st):
        for _ in range(launches):
            _lib.check(lib.ffai_probe_empty(128, stream()))

    res = {"launches_per_graph": launches, "bytes_per_read": nbytes,
           "empty_us": timed(empty), "read_us": {}, "read_gbps": {}}
    for wg in workgroups:
        def read(st, wg=wg):
            for i in range(launches):
                off = (st * launches + i) * nbytes
                _lib.check(lib.ffai_probe_read(buf.data_ptr() + off, nbytes, out.data_ptr(), wg,
                                               stream()))
        us = timed(read)
        res["read_us"][str(wg)] = us
        res["read_gbps"][str(wg)] = nbytes / (us * 1e-6) / 1e9
    return res


def pipes_bench(torch, iters=4096, waves_per_simd=(1, 2, 4)):
    """Pipe rates behind the fused kernel's per-tile budget (ffai_probe_pipes): per iteration
    and per SIMD, the time of 4 bf16 32x32x16 MFMAs, of 8 v_exp_f32, of 8 FMAs, and of the
    MFMAs with 8 (16) exp and 8 (16) FMA spread between them, at 1, 2 and 4 waves per SIMD.
    `mfma_tflops` is the chip rate the MFMA-only loop reaches; cycles are at 2.4 GHz."""
    import ctypes
    from ffai_amd import _lib

    lib = _lib.load()
    dev = torch.device("cuda:0")
    out = torch.empty(256 * 256 * max(waves_per_simd), dtype=torch.float32, device=dev)
    kinds = ("mfma4", "exp8", "fma8", "mfma4+exp8+fma8", "mfma4+exp16+fma16")
    res = {"iters": iters, "cycles_at_2p4ghz_per_iter_per_simd": {}, "mfma_tflops": {}}
    for w in waves_per_simd:
        wgs = 256 * w
        row = {}
        for k, name in enumerate(kinds):
            def launch():
                _lib.check(lib.ffai_probe_pipes(k, wgs, iters, out.data_ptr(),
                                                ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
            launch()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            launch()
            e1.record()
            torch.cuda.synchronize()
            ns = e0.elapsed_time(e1) * 1e6 / (iters * w)  # per iteration per SIMD
            row[name] = round(ns * 2.4, 1)
            if k == 0:
                res["mfma_tflops"][str(w)] = round(4 * 32768 * 1024 * w * iters / (e0.elapsed_time(e1) * 1e-3) / 1e12, 1)
        res["cycles_at_2p4ghz_per_iter_per_simd"][str(w)] = row
    return res


# ------------------------------------------------------------------------------------------
# Beam-5 decode step (whisper-medium: 24 layers, 16 heads, D=64)
# ------------------------------------------------------------------------------------------

# The decode step keeps the cross-attention cache's K as rows (heads, frames, head_dim): that
# cache is built once per window by ffai_cross_kv_build, which writes either layout, and rows are
# whole 128-byte lines per key where K^T rows (3000 bytes apart at 1500 frames) straddle lines
# (beam-5 cross-attention launch, graphs: 7.9 against 9.1 us).
CROSS_K_TRANSPOSED = False


def decode_bench(torch, fa, steps, warmup, beams=5, H=16, D=64, T_enc=1500, cap=448, layers=24,
                 sets=3, graphs=True):
    dev = torch.device("cuda:0")
    g = torch.Generator(device="cpu").manual_seed(3)
    lens_cpu = torch.randint(1, cap + 1, (layers, beams), generator=g, dtype=torch.int32)
    gd = torch.Generator(device=dev).manual_seed(3)
    scale = D ** -0.5
    bf = torch.bfloat16
    all_sets = []
    for _ in range(sets):   # > 2 x 256 MB: consecutive steps never find their K/V in the MALL
        layer_bufs = []
        for l in range(layers):
            q_self = torch.randn(beams, H, 1, D, generator=gd, device=dev).to(bf)
            k_self = torch.randn(beams, H, cap, D, generator=gd, device=dev).to(bf)
            v_self = torch.randn(beams, H, cap, D, generator=gd, device=dev).to(bf)
            lens = lens_cpu[l].to(dev)
            q_x = torch.randn(beams, H, 1, D, generator=gd, device=dev).to(bf)
            kt_x = torch.randn(*((1, H, D, T_enc) if CROSS_K_TRANSPOSED else (1, H, T_enc, D)),
                               generator=gd, device=dev).to(bf)
            v_x = torch.randn(1, H, T_enc, D, generator=gd, device=dev).to(bf)
            o_self = torch.empty(beams, H, 1, D, device=dev, dtype=torch.float32)
            o_x = torch.empty(beams, H, 1, D, device=dev, dtype=torch.float32)
            layer_bufs.append((q_self, k_self, v_self, lens, o_self, q_x, kt_x, v_x, o_x))
        all_sets.append(layer_bufs)
    # workspaces (one per call site, reused across layers: calls are stream-ordered)
    qs, ks, vs, ls, os_, qx, ktx, vx, ox = all_sets[0][0]
    ws_self = torch.zeros(max(1, fa.workspace_bytes(qs, ks, vs, os_, scale=scale, kv_lens=ls)),
                          dtype=torch.uint8, device=dev)
    ws_x = torch.zeros(max(1, fa.workspace_bytes(qx.permute(2, 1, 0, 3), ktx, vx,
                                                 ox.permute(2, 1, 0, 3),
                                                 k_transposed=CROSS_K_TRANSPOSED,
                                                 scale=scale)), dtype=torch.uint8, device=dev)

    def step(layer_bufs):
        for (q_self, k_self, v_self, lens, o_self, q_x, kt_x, v_x, o_x) in layer_bufs:
            fa.attention(q_self, k_self, v_self, scale=scale, kv_lens=lens, out=o_self,
                         workspace=ws_self)
            fa.attention(q_x.permute(2, 1, 0, 3), kt_x, v_x, k_transposed=CROSS_K_TRANSPOSED,
                         scale=scale, out=o_x.permute(2, 1, 0, 3), workspace=ws_x)

    # capture one HIP graph per buffer set: the step's 48 attention calls replay without
    # host-side dispatch (the kernels use no memset; the workspaces are preallocated). Without
    # graphs (counter collection, which serialises dispatches) every step is dispatched eagerly.
    step(all_sets[0])
    torch.cuda.synchronize()
    if graphs:
        captured = []
        for s in range(sets):
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr):
                step(all_sets[s])
            captured.append(gr)
        run_step = lambda i: captured[i % sets].replay()
    else:
        run_step = lambda i: step(all_sets[i % sets])
    torch.cuda.synchronize()
    for i in range(warmup):
        run_step(i)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(steps):
        run_step(i)
    e1.record(stream)
    torch.cuda.synchronize()
    gpu_ms = e0.elapsed_time(e1)
    us_step = gpu_ms * 1e3 / steps
    kv_row = H * D * 2 * 2  # K + V bytes per key (bf16)
    cross_bytes = layers * (H * T_enc * D * 2 * 2 + beams * H * D * 2 + beams * H * D * 4)
    self_bytes = int(lens_cpu.sum()) * kv_row + layers * (beams * H * D * 2 + beams * H * D * 4)
    step_bytes = cross_bytes + self_bytes
    return {
        "us_per_step": us_step,
        "bytes_per_step": step_bytes,
        "cross_bytes_per_layer": cross_bytes / layers,
        "self_bytes_per_step": self_bytes,
        "gbps": step_bytes / (us_step * 1e-6) / 1e9,
        "hbm_frac": step_bytes / (us_step * 1e-6) / 1e9 / PEAK_HBM_GBPS,
        "launches_per_step": 2 * layers,
        "cross_k_layout": "transposed" if CROSS_K_TRANSPOSED else "rows",
        "mean_self_len": float(lens_cpu.float().mean()),
        "buffer_sets": sets,
        "hip_graphs": graphs,
    }


def decode_ref_bench(torch, fa, steps, warmup, beams=5, H=16, D=64, T_enc=1500, cap=448,
                     layers=24, sets=3):
    """The beam-5 whisper-medium decode step as the reference calls its kernel: per layer and per
    beam, one after another (decoder.rs:542-596), the self-attention arm (f32 q over that beam's
    f32 K^T/V cache, flash_attn.rs:370-399) and the cross-attention arm (f32 q over the window's
    f16 K^T/V, :289-356; text_decoder.rs:771-793), each one call of ffai_attn_fwd on the f32
    decode kernel: 2 x 5 x 24 = 240 launches per step in HIP graphs, 3 buffer sets beyond the
    MALL. Cache lengths are the 16-bit decode leg's (seed 3). Besides the step, graphs of the
    cross-attention calls alone and of the self-attention calls alone give per-launch times, and
    one more times each layer's five self-attention calls as one call over the 5 beams (batch 5,
    ragged lengths), the comparison at the bytes per launch of the 16-bit beam kernel."""
    dev = torch.device("cuda:0")
    g = torch.Generator(device="cpu").manual_seed(3)
    lens_cpu = torch.randint(1, cap + 1, (layers, beams), generator=g, dtype=torch.int32)
    gd = torch.Generator(device=dev).manual_seed(31)
    scale = D ** -0.5
    all_sets = []
    for _ in range(sets):
        layer_bufs = []
        for l in range(layers):
            kt_s = torch.randn(beams, H, D, cap, generator=gd, device=dev)
            v_s = torch.randn(beams, H, cap, D, generator=gd, device=dev)
            q_s = torch.randn(beams, H, 1, D, generator=gd, device=dev)
            q_x = torch.randn(beams, H, 1, D, generator=gd, device=dev)
            kt_x = torch.randn(1, H, D, T_enc, generator=gd, device=dev).half()
            v_x = torch.randn(1, H, T_enc, D, generator=gd, device=dev).half()
            o_s = torch.empty(beams, H, 1, D, device=dev)
            o_x = torch.empty(beams, H, 1, D, device=dev)
            calls_s, calls_x = [], []
            for b in range(beams):
                n = int(lens_cpu[l, b])
                calls_s.append((q_s[b:b + 1], kt_s[b:b + 1, :, :, :n], v_s[b:b + 1, :, :n],
                                o_s[b:b + 1]))
                calls_x.append((q_x[b:b + 1], kt_x, v_x, o_x[b:b + 1]))
            # the same self-attention as one call over the 5 beams (ragged lengths)
            batched = (q_s, kt_s, v_s, o_s, lens_cpu[l].to(dev))
            layer_bufs.append((calls_s, calls_x, batched))
        all_sets.append(layer_bufs)
    # workspaces (one per call site, reused: calls are stream-ordered), for the largest need
    c_x = all_sets[0][0][1][0]
    ws_x = torch.zeros(max(16, fa.workspace_bytes(*c_x, k_transposed=True, scale=scale)),
                       dtype=torch.uint8, device=dev)
    ws_s = torch.zeros(max(16, max(fa.workspace_bytes(*c, k_transposed=True, scale=scale)
                                   for lb in all_sets[0] for c in lb[0])),
                       dtype=torch.uint8, device=dev)
    qb, ktb, vb, ob, lb0 = all_sets[0][0][2]
    ws_b = torch.zeros(max(16, fa.workspace_bytes(qb, ktb, vb, ob, k_transposed=True, scale=scale,
                                                  kv_lens=lb0)), dtype=torch.uint8, device=dev)
    longest = max((c for lb in all_sets[0] for c in lb[0]), key=lambda c: c[1].shape[3])
    plans = {"cross": fa.plan(*c_x, k_transposed=True, scale=scale),
             f"self_{longest[1].shape[3]}": fa.plan(*longest, k_transposed=True, scale=scale)}

    def step(layer_bufs, which):
        for calls_s, calls_x, (qb, ktb, vb, ob, lb) in layer_bufs:
            if which == "self_batched":
                fa.attention(qb, ktb, vb, k_transposed=True, scale=scale, kv_lens=lb, out=ob,
                             workspace=ws_b)
                continue
            for b in range(beams):
                if which in ("both", "self"):
                    q, kt, v, o = calls_s[b]
                    fa.attention(q, kt, v, k_transposed=True, scale=scale, out=o, workspace=ws_s)
                if which in ("both", "cross"):
                    q, kt, v, o = calls_x[b]
                    fa.attention(q, kt, v, k_transposed=True, scale=scale, out=o, workspace=ws_x)

    def timed(which):
        step(all_sets[0], which)
        torch.cuda.synchronize()
        captured = []
        for s_ in range(sets):
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr):
                step(all_sets[s_], which)
            captured.append(gr)
        torch.cuda.synchronize()
        for i in range(warmup):
            captured[i % sets].replay()
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for i in range(steps):
            captured[i % sets].replay()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / steps

    us_step = timed("both")
    us_cross = timed("cross")
    us_self = timed("self")
    us_self_b = timed("self_batched")
    n_calls = layers * beams
    qo = H * D * 4 * 2                                    # f32 q read, f32 out written
    cross_call = H * T_enc * D * 2 * 2 + qo               # f16 K^T + V of the window
    self_bytes = int(lens_cpu.sum()) * H * D * 4 * 2 + n_calls * qo
    step_bytes = n_calls * cross_call + self_bytes
    return {
        "us_per_step": us_step,
        "bytes_per_step": step_bytes,
        "gbps": step_bytes / (us_step * 1e-6) / 1e9,
        "hbm_frac": step_bytes / (us_step * 1e-6) / 1e9 / PEAK_HBM_GBPS,
        "launches_per_step": 2 * n_calls,
        "cross_us_per_launch": us_cross / n_calls,
        "cross_bytes_per_launch": cross_call,
        "cross_gbps_per_launch": cross_call / (us_cross / n_calls * 1e-6) / 1e9,
        "self_us_per_launch": us_self / n_calls,
        "self_mean_bytes_per_launch": self_bytes / n_calls,
        "self_gbps_per_launch": self_bytes / (us_self * 1e-6) / 1e9,
        "self_batched_us_per_launch": us_self_b / layers,
        "self_batched_gbps_per_launch": self_bytes / (us_self_b * 1e-6) / 1e9,
        "mean_self_len": float(lens_cpu.float().mean()),
        "plans": plans,
        "buffer_sets": sets,
        "hip_graphs": True,
        "note": ("bytes count each call's reads as the reference issues them: the cross K/V "
                 "once per beam"),
    }


def key_sweep_bench(torch, fa, B=16, H=20, sets=4, reps=20, key_lens=(1500, 3000, 4500, 6000)):
    """Fixed and per-key cost of the fused kernel on an encoder layer's items: B x H heads of
    1500 query rows (the large-v3 layer's 1920 items at B16 H20, whisper-small's 576 at B8 H12),
    bf16, K^T, with 1500 .. 6000 keys (the same items and launch shape; only the key loop
    grows). A least-squares line through the times gives the per-key rate the loops sustain and
    the time a launch spends outside them (prologues, epilogues, the tail of the last round)."""
    import numpy as np

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(4)
    T, D = 1500, 64
    pts = []
    for tk in key_lens:
        bufs = []
        for _ in range(sets):
            q = torch.randn(B, H, T, D, generator=g, device=dev).bfloat16()
            kt = torch.randn(B, H, D, tk, generator=g, device=dev).bfloat16()
            v = torch.randn(B, H, tk, D, generator=g, device=dev).bfloat16()
            bufs.append((q, kt, v, torch.empty_like(q)))
        nb = fa.workspace_bytes(*bufs[0], k_transposed=True, scale=0.125)
        ws = torch.zeros(max(nb, 16), dtype=torch.uint8, device=dev) if nb else None

        def once():
            for q, kt, v, o in bufs:
                fa.attention(q, kt, v, k_transposed=True, scale=0.125, out=o, workspace=ws)

        for _ in range(3):
            once()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            once()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / (reps * sets)
        pts.append((tk, us, 4.0 * B * H * T * tk * D / us / 1e6))
        del bufs, ws
        torch.cuda.empty_cache()
    x = np.array([p_[0] for p_ in pts], float)
    y = np.array([p_[1] for p_ in pts], float)
    slope, icpt = np.polyfit(x, y, 1)
    return {"points": [{"keys": k, "us": u, "tflops": f} for k, u, f in pts],
            "us_per_1500_keys": float(slope * 1500), "fixed_us": float(icpt),
            "loop_tflops": float(4.0 * B * H * T * 1500 * D / (slope * 1500) / 1e6),
            "fixed_share_at_1500": float(icpt / (icpt + slope * 1500))}


def workgroup_timeline(r):
    """Per-workgroup times of the fused kernel's record (stamps leg): medians in ns of the
    prologue (entry -> key loop; of it: entry -> Q loads issued, Q and tiles 0/1 issued -> landed,
    the barrier and the first product), the key loop, the epilogue (loop end -> last store
    issued -> acknowledged), the gap from a workgroup's exit to the next workgroup's entry on the
    same CU (the hardware slot each wave recorded), and the loops' share of the slot-time
    (2 workgroups per CU x the span from the first entry to the last exit)."""
    import numpy as np

    a = r.astype("int64")
    ran = a[:, 0, 6] > 0
    a = a[ran]
    base = a[:, :, 11].min()
    t = lambda k, f: (f(a[:, :, k], axis=1) - base) * 10  # 100 MHz real-time ticks -> ns
    e0, pre_q, issued, landed = t(11, np.min), t(18, np.max), t(15, np.max), t(16, np.max)
    bar, l0, l1 = t(17, np.max), t(8, np.min), t(10, np.max)
    wrote = a[:, 0, 12] > 0
    x1, x2 = t(12, np.max), t(13, np.max)
    med = lambda x: float(np.median(x)) if len(x) else None
    where = a[:, 0, 14]
    hwid, xcc = where & 0xffffffff, where >> 32
    cu = xcc * 1000 + ((hwid >> 13) & 7) * 100 + ((hwid >> 12) & 1) * 16 + ((hwid >> 8) & 15)
    end = np.where(wrote, x2, l1)
    span = float(end.max())
    # each CU's two slots: a workgroup takes the slot that freed first
    gaps, startup, loop_gaps, tail = [], [], [], []
    for c in np.unique(cu):
        idx = np.where(cu == c)[0]
        idx = idx[np.argsort(e0[idx])]
        slots = []
        for i in idx:
            if len(slots) < 2:
                slots.append([i])
                continue
            j = min(range(2), key=lambda k: end[slots[k][-1]])
            gaps.append(e0[i] - end[slots[j][-1]])
            slots[j].append(i)
        for sl in slots:
            startup.append(l0[sl[0]])
            tail.append(span - end[sl[-1]])
            loop_gaps.extend(l0[v_] - l1[u_] for u_, v_ in zip(sl[:-1], sl[1:]))
    n_slots = 2 * len(np.unique(cu))
    return {"workgroups": int(ran.sum()), "cus": int(len(np.unique(cu))),
            "prologue_ns": med(l0 - e0), "entry_to_q_issue_ns": med(pre_q - e0),
            "q_and_tiles_issue_ns": med(issued - pre_q), "loads_land_ns": med(landed - issued),
            "barrier_ns": med(bar - landed), "first_product_ns": med(l0 - bar),
            "loop_tiles_most": int(a[:, 0, 6].max()),
            "loop_ns_most_tiles": med((l1 - l0)[a[:, 0, 6] == a[:, 0, 6].max()]),
            "epilogue_issue_ns": med((x1 - l1)[wrote]), "store_ack_ns": med((x2 - x1)[wrote]),
            "exit_to_next_entry_ns": med(np.array(gaps)) if gaps else None,
            "span_ns": span,
            # per slot (mean): first entry -> first loop, loop end -> next loop start (summed),
            # last exit -> the launch's last exit, loops
            "slot_startup_ns": float(np.sum(startup) / n_slots),
            "slot_gaps_ns": float(np.sum(loop_gaps) / n_slots),
            "slot_tail_ns": float((np.sum(tail) + (n_slots - len(startup)) * span) / n_slots),
            "slot_loops_ns": float((l1 - l0).sum() / n_slots),
            "loop_share_of_slot_time": float((l1 - l0).sum() / (n_slots * span))}


def stamps_bench(torch, fa, calls=3):
    """Where the kernels' time goes, from the diagnostic library (libffai_attn_stamps.so: the same
    sources built with FFAI_STAMPS, whose kernels time their phases with s_memtime and write the
    results with vector stores; the product library has none of it). Two workloads:
      * the fused kernel on one whisper-large-v3 layer (B16 H20 T1500, bf16, K^T): per wave, the
        sums over its tiles of phase B (S^T of subtile 1 with subtile 0's exps), the settle check
        of subtile 0, phase C (PV of subtile 0 with subtile 1's exps), the settle check of
        subtile 1, the barrier (the DMA wait and the workgroup), and D (staging, PV of subtile 1,
        S^T of the next tile's subtile 0); shares of the loop and cycles per tile;
      * the 16-bit decode kernel on the beam-5 whisper-medium step's cross-attention (5 beams as
        rows, 16 heads x 1500 frames, K as rows: 8 key splits) and self-attention (5 ragged beam
        caches of <= 448 keys): each workgroup's event times from its entry (first K/V load
        issued, first tile landed, tiles done, LDS merge done, end), for the workgroups that
        wrote the output and those that only passed a split partial on.
    Besides, each fused-kernel workgroup's timeline (workgroup_timeline) on the large-v3 layer,
    the whisper-small layer (B8 H12 T1500) and the Qwen2-VL-2B prefill (Hq 12 over 2 K/V heads,
    S 4096, head_dim 128, causal, K as rows).
    Timing adds ~8% to the fused kernel on the large-v3 layer (0.240 against 0.221 ms); the
    shares, not the absolute times, are what this leg is for. Ticks are converted with the
    100 MHz real-time counter read beside them."""
    import ctypes
    import statistics as stats

    from ffai_amd import build as fbuild

    lib = ctypes.CDLL(fbuild.STAMPS_LIB_PATH)
    vp, sz = ctypes.c_void_p, ctypes.c_size_t
    lib.ffai_attn_fwd.argtypes = [ctypes.c_void_p, vp, vp, vp, vp, vp, sz, vp]
    lib.ffai_attn_fwd.restype = ctypes.c_int
    lib.ffai_attn_workspace_bytes.argtypes = [ctypes.c_void_p, ctypes.POINTER(sz)]
    lib.ffai_attn_workspace_bytes.restype = ctypes.c_int
    lib.ffai_stamps_set.argtypes = [vp, sz]
    lib.ffai_stamps_set.restype = ctypes.c_int
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()

    def run(q, k, v, out, rec_bytes, **kw):
        d = fa.make_desc(q, k, v, out, k_transposed=kw.get("k_transposed", False),
                         scale=kw.get("scale", 1.0), causal=kw.get("causal", False), q_offset=0,
                         kv_lens=kw.get("kv_lens"))
        n = ctypes.c_size_t(0)
        assert lib.ffai_attn_workspace_bytes(ctypes.byref(d), ctypes.byref(n)) == 0
        ws = torch.zeros(max(16, n.value), dtype=torch.uint8, device=dev)
        buf = torch.zeros(rec_bytes // 8, dtype=torch.int64, device=dev)
        for i in range(calls):  # the last call records
            lib.ffai_stamps_set(buf.data_ptr() if i == calls - 1 else None, rec_bytes)
            rc = lib.ffai_attn_fwd(ctypes.byref(d), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                   out.data_ptr(), ws.data_ptr(), ws.numel(), stream.cuda_stream)
            assert rc == 0, rc
        torch.cuda.synchronize()
        lib.ffai_stamps_set(None, 0)
        return buf.cpu().numpy().astype("uint64")

    g = torch.Generator(device=dev).manual_seed(4)
    # ---- fused kernel, one whisper-large-v3 layer
    B, H, T, D = 16, 20, 1500, 64
    q = torch.randn(B, H, T, D, generator=g, device=dev).bfloat16()
    kt = torch.randn(B, H, D, T, generator=g, device=dev).bfloat16()
    v = torch.randn(B, H, T, D, generator=g, device=dev).bfloat16()
    o = torch.empty_like(q)
    wgs = 2048
    r = run(q, kt, v, o, wgs * 1024, k_transposed=True, scale=0.125).reshape(wgs, 4, 32)
    rec = r[r[:, :, 6].astype("int64") > 0]      # waves that ran tiles
    names = ["B", "settle0", "C", "settle1", "barrier", "D"]
    sums = rec[:, :6].astype("float64").sum(axis=0)
    tiles = float(rec[:, 6].sum())
    ticks_per_ns = stats.median(((rec[:, 9] - rec[:, 7]) / ((rec[:, 10] - rec[:, 8]) * 10.0)).tolist())
    enc = {"waves": int(len(rec)), "tiles_per_wave": tiles / len(rec),
           "share": {n: float(x / sums.sum()) for n, x in zip(names, sums)},
           "ticks_per_tile": float(sums.sum() / tiles),
           "ns_per_tile": float(sums.sum() / tiles / ticks_per_ns),
           "clock_ticks_per_ns": float(ticks_per_ns)}
    enc.update(workgroup_timeline(r))
    out_timelines = {}
    for name, (B_, H_, Hk_, T_, D_, kt_, causal_) in (
            ("encoder_small_layer", (8, 12, 12, 1500, 64, True, False)),
            ("prefill_qwen2vl", (1, 12, 2, 4096, 128, False, True))):
        q_ = torch.randn(B_, H_, T_, D_, generator=g, device=dev).bfloat16()
        k_ = (torch.randn(B_, Hk_, D_, T_, generator=g, device=dev) if kt_ else
              torch.randn(B_, Hk_, T_, D_, generator=g, device=dev)).bfloat16()
        v_ = torch.randn(B_, Hk_, T_, D_, generator=g, device=dev).bfloat16()
        o_ = torch.empty_like(q_)
        nwg = 4096
        r_ = run(q_, k_, v_, o_, nwg * 1024, k_transposed=kt_, scale=D_ ** -0.5,
                 causal=causal_).reshape(nwg, 4, 32)
        out_timelines[name] = workgroup_timeline(r_)
        del q_, k_, v_, o_
    # ---- decode kernel, beam-5 cross- and self-attention of one whisper-medium layer
    Hd, beams, Te, cap = 16, 5, 1500, 448
    out = {"encoder_large_v3_layer": enc, **out_timelines}
    qx = torch.randn(1, Hd, beams, D, generator=g, device=dev).bfloat16()
    kx = torch.randn(1, Hd, Te, D, generator=g, device=dev).bfloat16()
    vx = torch.randn(1, Hd, Te, D, generator=g, device=dev).bfloat16()
    ox = torch.empty(1, Hd, beams, D, device=dev)
    gl = torch.Generator(device="cpu").manual_seed(3)
    lens = torch.randint(1, cap + 1, (beams,), generator=gl, dtype=torch.int32).to(dev)
    qs = torch.randn(beams, Hd, 1, D, generator=g, device=dev).bfloat16()
    ks = torch.randn(beams, Hd, cap, D, generator=g, device=dev).bfloat16()
    vs = torch.randn(beams, Hd, cap, D, generator=g, device=dev).bfloat16()
    os_ = torch.empty(beams, Hd, 1, D, device=dev)
    events = ["issued", "landed", "tiles_done", "lds_merged", "end"]
    for name, args, kw in (("decode_cross_beam5", (qx, kx, vx, ox), dict(scale=0.125)),
                           ("decode_self_beam5", (qs, ks, vs, os_),
                            dict(scale=0.125, kv_lens=lens))):
        nw = 1024
        r = run(*args, nw * 64, **kw).reshape(nw, 8)
        r = r[r[:, 0] > 0]
        rel = (r[:, 1:6].astype("int64") - r[:, :1].astype("int64")) / ticks_per_ns
        wrote = r[:, 6] == 1
        leg = {"workgroups": int(len(r))}
        for tag, m in (("writers", wrote), ("split_only", ~wrote)):
            if m.any():
                leg[tag] = {"count": int(m.sum()),
                            **{f"{e}_ns": float(stats.median(rel[m, i].tolist()))
                               for i, e in enumerate(events)}}
        out[name] = leg
    return out


# ------------------------------------------------------------------------------------------
# Device-resident decode state (whisper-medium: 24 layers, beam 5, 16 heads, D=64)
# ------------------------------------------------------------------------------------------

def decode_state_bench(torch, fa, steps, warmup, beams=5, H=16, D=64, T_enc=1500, cap=448,
                       layers=24, mid_len=224):
    """A beam step's state work on the device: per layer, append this step's K/V row of every
    beam (f32 projections -> bf16 cache), then reorder the beams of all layers by parent into
    the other cache of a ping-pong pair in one launch; then the same step with the attention calls between append and reorder
    (self-attention over the beams' caches, cross-attention over the window's shared cache).
    All beams of a step share one length, as in beam search; lengths start so that the timed
    steps are centred on `mid_len`. Also times the per-window cross-attention cache build of
    the 24 layers (f32 projections -> bf16 K and V, K as rows)."""
    from ffai_amd.kv_cache import KVCache, cross_kv_build

    dev = torch.device("cuda:0")
    gd = torch.Generator(device=dev).manual_seed(3)
    g = torch.Generator(device="cpu").manual_seed(3)
    scale = D ** -0.5
    bf = torch.bfloat16
    total = warmup + steps
    start_len = max(1, mid_len - total // 2)
    assert start_len + total <= cap
    caches = [KVCache(beams, H, cap, D, bf, dev, layers=layers) for _ in range(2)]
    caches[0].k.normal_(generator=gd)
    caches[0].v.normal_(generator=gd)
    projs, xs = [], []
    for _ in range(layers):
        projs.append((torch.randn(beams, 1, H * D, generator=gd, device=dev),
                      torch.randn(beams, 1, H * D, generator=gd, device=dev),
                      torch.randn(beams, H, 1, D, generator=gd, device=dev).to(bf),
                      torch.randn(beams, H, 1, D, generator=gd, device=dev).to(bf)))
        kp = torch.randn(T_enc, H * D, generator=gd, device=dev)
        vp = torch.randn(T_enc, H * D, generator=gd, device=dev)
        xs.append((kp, vp) + cross_kv_build(kp, vp, H, bf, k_transposed=CROSS_K_TRANSPOSED))
    parent = torch.randint(0, beams, (beams,), generator=g, dtype=torch.int32).to(dev)
    o_self = torch.empty(beams, H, 1, D, device=dev, dtype=torch.float32)
    o_x = torch.empty(beams, H, 1, D, device=dev, dtype=torch.float32)
    q0, k0 = projs[0][2], caches[0].layer(0)
    ws_self = torch.zeros(max(1, fa.workspace_bytes(q0, k0.k, k0.v, o_self, scale=scale,
                                                    kv_lens=k0.lens)), dtype=torch.uint8, device=dev)
    ws_x = torch.zeros(max(1, fa.workspace_bytes(projs[0][3].permute(2, 1, 0, 3), xs[0][2][None],
                                                 xs[0][3][None], o_x.permute(2, 1, 0, 3),
                                                 k_transposed=CROSS_K_TRANSPOSED, scale=scale)),
                       dtype=torch.uint8, device=dev)

    def step(phase, attend):
        cur, nxt = caches[phase], caches[1 - phase]
        for l in range(layers):
            c = cur.layer(l)
            nk, nv, qs, qx = projs[l]
            c.append(nk, nv)
            if attend:
                fa.attention(qs, c.k, c.v, scale=scale, kv_lens=c.lens, out=o_self,
                             workspace=ws_self)
                fa.attention(qx.permute(2, 1, 0, 3), xs[l][2][None], xs[l][3][None],
                             k_transposed=CROSS_K_TRANSPOSED, scale=scale,
                             out=o_x.permute(2, 1, 0, 3), workspace=ws_x)
        nxt.gather_from(cur, parent)   # every layer's reorder in one launch

    def timed(attend):
        caches[0].lens.fill_(start_len)
        torch.cuda.synchronize()
        graphs = []
        for phase in (0, 1):   # capture does not execute: the lengths stay at start_len
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr):
                step(phase, attend)
            graphs.append(gr)
        torch.cuda.synchronize()
        for i in range(warmup):
            graphs[i % 2].replay()
        stream = torch.cuda.current_stream()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for i in range(warmup, total):
            graphs[i % 2].replay()
        e1.record(stream)
        torch.cuda.synchronize()
        final = int(caches[total % 2].lens[0, 0])
        assert final == start_len + total, (final, start_len, total)
        return e0.elapsed_time(e1) * 1e3 / steps

    us_state = timed(False)
    us_full = timed(True)
    # the step's self-attention q/k/v projections with the appends: per layer the GEMV of the
    # packed (3n, n) f16 weights and the append of its k and v rows, against one all-layer
    # length advance and per layer the fused projection that writes the rows itself
    from ffai_amd.gemv import F16Gemv
    n = H * D
    wqkv = [F16Gemv(torch.randn(3 * n, n, generator=gd, device=dev) / n ** 0.5)
            for _ in range(layers)]
    xq = torch.randn(beams, n, generator=gd, device=dev)
    yq = torch.empty(beams, 3 * n, device=dev)
    qo = torch.empty(beams, n, device=dev)

    def proj_step(fused):
        c = caches[0]
        if fused:
            c.advance(1)
        for l in range(layers):
            if fused:
                wqkv[l].qkv_into_cache(xq, qo, c.layer(l))
            else:
                wqkv[l](xq, out=yq)
                c.layer(l).append(yq[:, None, n:2 * n], yq[:, None, 2 * n:])

    def timed_proj(fused):
        caches[0].lens.fill_(start_len)
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            proj_step(fused)
        torch.cuda.synchronize()
        for _ in range(warmup):
            gr.replay()
        stream = torch.cuda.current_stream()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            gr.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        final = int(caches[0].lens[0, 0])
        assert final == start_len + total, (final, start_len, total)
        return e0.elapsed_time(e1) * 1e3 / steps

    us_proj_append = timed_proj(False)
    us_proj_fused = timed_proj(True)
    # algorithmic bytes of the state work per step (lengths after the append, averaged over
    # the timed steps): append reads the f32 rows and writes bf16; the reorder reads and
    # writes every beam's valid prefix of K and V
    mean_len = start_len + warmup + (steps + 1) / 2.0
    row = H * D
    append_bytes = layers * beams * 2 * row * (4 + 2)
    gather_bytes = layers * beams * 2 * row * 2 * 2 * mean_len
    state_bytes = append_bytes + gather_bytes
    # per-window cross cache build, all layers
    reps = 20

    def build_all():
        for kp, vp, kx, vx in xs:
            cross_kv_build(kp, vp, H, bf, k_transposed=CROSS_K_TRANSPOSED, out=(kx, vx))

    build_all()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        build_all()
    e1.record()
    torch.cuda.synchronize()
    us_build = e0.elapsed_time(e1) * 1e3 / reps
    build_bytes = layers * 2 * T_enc * row * (4 + 2)
    # the prompt step (step 0 of a window): 228 tokens appended to a one-slot stack, causal
    # self-attention at offset 0 and cross-attention over the window's frames, every layer
    from ffai_amd.kv_cache import self_attention_step
    P = 228
    pstack = KVCache(1, H, cap, D, bf, dev, layers=layers)
    pk = torch.randn(1, P, H * D, generator=gd, device=dev)
    pv = torch.randn(1, P, H * D, generator=gd, device=dev)
    pq = torch.randn(1, H, P, D, generator=gd, device=dev).to(bf)
    po = torch.empty(1, H, P, D, device=dev, dtype=torch.float32)
    pws = torch.zeros(max(1, fa.workspace_bytes(pq, xs[0][2][None], xs[0][3][None], po,
                                                k_transposed=CROSS_K_TRANSPOSED, scale=scale)),
                      dtype=torch.uint8, device=dev)

    def prompt_step():
        for l in range(layers):
            self_attention_step(pstack.layer(l), pq, pk, pv, 0, scale, out=po, workspace=pws)
            fa.attention(pq, xs[l][2][None], xs[l][3][None], k_transposed=CROSS_K_TRANSPOSED,
                         scale=scale, out=po, workspace=pws)

    pstack.lens.zero_()
    torch.cuda.synchronize()
    pg = torch.cuda.CUDAGraph()
    with torch.cuda.graph(pg):
        prompt_step()
    torch.cuda.synchronize()
    preps = 20
    e0.record()
    for _ in range(preps):
        pstack.lens.zero_()
        pg.replay()
    e1.record()
    torch.cuda.synchronize()
    us_prompt = e0.elapsed_time(e1) * 1e3 / preps
    prompt_flop = layers * 4.0 * D * H * (P * (P + 1) / 2 + P * T_enc)
    return {
        "state_us_per_step": us_state,
        "state_bytes_per_step": state_bytes,
        "state_gbps": state_bytes / (us_state * 1e-6) / 1e9,
        "full_step_us": us_full,
        "mean_self_len": mean_len,
        "cross_build_us_per_window": us_build,
        "cross_build_gbps": build_bytes / (us_build * 1e-6) / 1e9,
        "prompt_step_us": us_prompt,
        "prompt_step_tflops": prompt_flop / (us_prompt * 1e-6) / 1e12,
        "prompt_tokens": P,
        "launches_per_step": layers + 1,
        "qkv_and_append_us_per_step": us_proj_append,
        "qkv_into_cache_us_per_step": us_proj_fused,
    }


# ------------------------------------------------------------------------------------------
# Encoder self-attention block (whisper-large-v3: projections + attention + out-projection)
# ------------------------------------------------------------------------------------------

def encoder_block_bench(torch, fa, steps, warmup, layers=4, windows=16, T=1500, n=1280, H=20):
    """The whole EncoderAttention::forward per layer through ffai_encoder_attn_fwd, one call per
    1500-frame window as the reference runs it (text_decoder.rs:1069-1076): the q, v, k^T and
    out projections on hipBLASLt (bf16, f32 accumulation, bias epilogues) around the fused
    attention, which reads the projections by stride. `windows` windows per layer (the
    large-v3 batch of 16), distinct weights and activations per layer. FLOP per window =
    4 GEMMs x 2 T n^2 + the attention's 4 H T^2 hd."""
    from ffai_amd.encoder import EncoderAttention

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(6)
    bf = torch.bfloat16
    blocks = []
    for _ in range(layers):
        w = [(torch.randn(n, n, generator=g, device=dev) / n ** 0.5).to(bf) for _ in range(4)]
        bias = [(0.1 * torch.randn(n, generator=g, device=dev)).to(bf) for _ in range(3)]
        ea = EncoderAttention.load(n, H, w[0], bias[0], w[1], w[2], bias[1], w[3], bias[2])
        xs = [torch.randn(1, T, n, generator=g, device=dev).to(bf) for _ in range(windows)]
        blocks.append((ea, xs, [torch.empty_like(x) for x in xs]))
    ws = torch.zeros(blocks[0][0].workspace_bytes(blocks[0][1][0]), dtype=torch.uint8, device=dev)

    def step():
        for ea, xs, outs in blocks:
            for x, out in zip(xs, outs):
                ea(x, out=out, workspace=ws)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms_window = e0.elapsed_time(e1) / (steps * layers * windows)
    gemm_flop = 4 * 2.0 * T * n * n
    attn_flop = 4.0 * H * T * T * (n // H)
    return {"ms_per_window": ms_window,
            "tflops": (gemm_flop + attn_flop) / (ms_window * 1e-3) / 1e12,
            "gemm_gflop_per_window": gemm_flop / 1e9, "attn_gflop_per_window": attn_flop / 1e9,
            "layers": layers, "windows": windows}


# ------------------------------------------------------------------------------------------
# Decoder GEMVs of a beam-5 whisper-medium step (f16 projections + int8 vocabulary)
# ------------------------------------------------------------------------------------------

def gemv_bench(torch, steps, warmup, beams=5, n=1024, layers=24, vocab=51865):
    """Every single-row projection of one decode step for all beams at once: per layer the
    self-attention q, k and v (one GEMV over the three weights packed as (3n, n), since all
    three project the same normed input), the self-attention out and cross-attention q and
    out (n x n), and the MLP (4n x n, n x 4n) as f16 GEMVs, then the block-scaled int8
    vocabulary projection. Captured in a HIP graph. Algorithmic bytes: every weight byte once
    (f16, int8 + block scales + corrections) plus the activations read and outputs written."""
    from ffai_amd.gemv import F16Gemv, Int8Vocab

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(8)
    shapes = [(3 * n, n)] + [(n, n)] * 3 + [(4 * n, n), (n, 4 * n)]
    mats = [[F16Gemv(torch.randn(o, i, generator=g, device=dev) / i ** 0.5) for o, i in shapes]
            for _ in range(layers)]
    xs = {i: torch.randn(beams, i, generator=g, device=dev) for i in (n, 4 * n)}
    ys = {o: torch.empty(beams, o, device=dev) for o in (n, 3 * n, 4 * n)}
    iv = Int8Vocab(torch.randn(vocab, n, generator=g, device=dev) / n ** 0.5)
    logits = torch.empty(beams, vocab, device=dev)
    ws = torch.empty(iv.workspace_bytes(beams), dtype=torch.uint8, device=dev)

    def step():
        for layer in mats:
            for m in layer:
                m(xs[m.in_dim], out=ys[m.out_dim])
        iv(xs[n], out=logits, workspace=ws)

    step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / steps
    f16_bytes = layers * sum(o * i * 2 + beams * (i + o) * 4 for o, i in shapes)
    vocab_bytes = vocab * n + vocab * (n // 32) * 4 + vocab * 4 + beams * (n + vocab) * 4
    # the vocabulary projection alone (activation quantization + logits): 20 calls per graph
    # (timing calls one by one, eager or one per replay, measured the host's launches), cycling
    # over 5 quantized copies (300 MB, beyond the 256 MB MALL)
    per_graph = 20
    ivs = [iv] + [Int8Vocab(torch.randn(vocab, n, generator=g, device=dev) / n ** 0.5)
                  for _ in range(4)]
    vgraph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(vgraph):
        for k in range(per_graph):
            ivs[k % len(ivs)](xs[n], out=logits, workspace=ws)
    vgraph.replay()
    torch.cuda.synchronize()
    e0.record()
    for _ in range(steps):
        vgraph.replay()
    e1.record()
    torch.cuda.synchronize()
    us_vocab = e0.elapsed_time(e1) * 1e3 / (steps * per_graph)
    del vgraph, ivs
    # per shape: graphs of `layers` dependent launches over distinct weights, two sets
    # alternating so that the weights replayed (2 x layers matrices) exceed the 256 MB MALL for
    # the larger shapes
    per_launch = {}
    for o, i in dict.fromkeys(shapes):  # the distinct shapes, in order
        si = shapes.index((o, i))
        extra = [F16Gemv(torch.randn(o, i, generator=g, device=dev) / i ** 0.5)
                 for _ in range(layers)]
        sets = [[layer[si] for layer in mats], extra]
        graphs = []
        for ms in sets:
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr):
                for m in ms:
                    m(xs[i], out=ys[o])
            graphs.append(gr)
        for k in range(4):
            graphs[k % 2].replay()
        torch.cuda.synchronize()
        e0.record()
        for k in range(2 * steps):
            graphs[k % 2].replay()
        e1.record()
        torch.cuda.synchronize()
        per_launch[f"{o}x{i}"] = e0.elapsed_time(e1) * 1e3 / (2 * steps) / layers
        del graphs, extra
    return {"us_per_step": us, "bytes_per_step": f16_bytes + vocab_bytes,
            "gbps": (f16_bytes + vocab_bytes) / (us * 1e-6) / 1e9,
            "vocab_us": us_vocab, "vocab_gbps": vocab_bytes / (us_vocab * 1e-6) / 1e9,
            "launches_per_step": layers * len(shapes) + 2, "beams": beams,
            "us_per_launch": per_launch}


# ------------------------------------------------------------------------------------------
# CPU baseline: the oracle (reference algorithm restated) on this host's cores
# ------------------------------------------------------------------------------------------

def host_info():
    """CPUs this process may run on (sched_getaffinity) and the CPU model."""
    cpus = len(os.sched_getaffinity(0))
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return cpus, model


def cpu_baselines(rounds=21):
    """The reference's kernel, restated by the oracle in C++/AVX2, timed on this host on each
    encoder-shaped workload, by the reference's own method (examples/flash_probe.rs:409-432):
    one warm-up, then `rounds` interleaved rounds (each round runs every workload once, the order
    reversed on odd rounds), the median per workload. Threads: one per head up to the host's
    CPUs, as rayon spreads the heads (flash_attn.rs:199,402); batch items run serially, as the
    reference loops them (text_decoder.rs:1069-1076). Inputs are bf16-rounded where the GPU leg
    is bf16 (the reference computes in f32 on those values). The causal GQA prefill has no
    reference path: it runs the oracle's extension of the same tiling (labelled so)."""
    import numpy as np

    import oracle

    oracle.build()
    cpus, model = host_info()
    rb = oracle.round_bf16

    def rnd(rng, shape, mult=1.0):
        return (rng.standard_normal(shape) * mult).astype(np.float32)

    work = {}
    # whisper-large-v3 (headline): one batch item of one layer, 20 heads
    rng = np.random.default_rng(4)
    q, kt, v = rb(rnd(rng, (1, 20, 1500, 64))) * np.float32(0.125), rb(rnd(rng, (1, 20, 64, 1500))), rb(rnd(rng, (1, 20, 1500, 64)))
    work["encoder_large_v3"] = dict(
        run=lambda q=q, kt=kt, v=v: oracle.attend_f32(q, kt, v, threads=min(cpus, 20)),
        flop=4.0 * 20 * 1500 ** 2 * 64, threads=min(cpus, 20), kind="port",
        sample="one batch item (20 heads x T=1500, D=64) of one whisper-large-v3 layer, bf16-rounded "
               "inputs in f32 math; the reference runs the 16 items serially, so this is the "
               "layer's rate")
    # whisper-tiny f32: the 4 layers, 6 heads each
    rng = np.random.default_rng(1)
    tiny = [(rnd(rng, (1, 6, 1500, 64)) * np.float32(0.125), rnd(rng, (1, 6, 64, 1500)),
             rnd(rng, (1, 6, 1500, 64))) for _ in range(4)]
    work["encoder_tiny_f32"] = dict(
        run=lambda: [oracle.attend_f32(a, b, c, threads=min(cpus, 6)) for a, b, c in tiny],
        flop=4 * 4.0 * 6 * 1500 ** 2 * 64, threads=min(cpus, 6), kind="port",
        sample="the 4 whisper-tiny encoder layers (6 heads x T=1500, D=64, f32)")
    # whisper-small f32: 8 items serially, 12 heads each, K x 2
    rng = np.random.default_rng(2)
    small = [(rnd(rng, (1, 12, 1500, 64)) * np.float32(0.125), rnd(rng, (1, 12, 64, 1500), 2.0),
              rnd(rng, (1, 12, 1500, 64))) for _ in range(8)]
    work["encoder_small_f32"] = dict(
        run=lambda: [oracle.attend_f32(a, b, c, threads=min(cpus, 12)) for a, b, c in small],
        flop=8 * 4.0 * 12 * 1500 ** 2 * 64, threads=min(cpus, 12), kind="port",
        sample="one whisper-small layer: 8 batch items serially, 12 heads x T=1500, D=64, f32, "
               "K x 2")
    # Qwen2-VL causal GQA prefill: the oracle's extension (no reference path)
    rng = np.random.default_rng(5)
    S = 4096
    pq, pk, pv = rb(rnd(rng, (1, 12, S, 128))), rb(rnd(rng, (1, 2, S, 128))), rb(rnd(rng, (1, 2, S, 128)))
    work["prefill_causal_gqa_d128"] = dict(
        run=lambda: oracle.attend_general(pq, pk, pv, k_transposed=False, scale=128 ** -0.5,
                                          causal=True, threads=min(cpus, 12)),
        flop=4.0 * 12 * 128 * S * (S + 1) / 2, threads=min(cpus, 12), kind="oracle, not reference",
        sample="causal GQA prefill Hq12 over Hkv2, D=128, S=4096, bf16-rounded inputs in f32 math; "
               "the reference has no such path, so this times the oracle's extension of its tiling")
    names = list(work)
    for n in names:  # warm-up
        work[n]["run"]()
    times = {n: [] for n in names}
    t_start = time.perf_counter()
    for r in range(rounds):
        for n in (names if r % 2 == 0 else names[::-1]):
            t0 = time.perf_counter()
            work[n]["run"]()
            times[n].append(time.perf_counter() - t0)
    total_s = time.perf_counter() - t_start
    out = {}
    for n in names:
        med = float(np.median(times[n]))
        w = work[n]
        out[n] = {"value": w["flop"] / med / 1e12, "unit": "TFLOP/s", "cores": w["threads"],
                  "host_cpus": cpus, "cpu_model": model, "kind": w["kind"], "ms": med * 1e3,
                  "sample": (f"{w['sample']}; median of {rounds} interleaved rounds after one "
                             f"warm-up ({med * 1e3:.1f} ms each; the {len(names)} workloads' "
                             f"rounds took {total_s:.1f} s); heads over {w['threads']} of the "
                             f"host's {cpus} CPUs; CPU: {model}")}
    return out


def cpu_decode_baseline(beams=5, H=16, D=64, T_enc=1500, cap=448, layers=24, reps=5):
    """The reference's beam-5 decode step on this host, through the oracle: per layer and beam,
    the shipped f16-K/V cross-attention arm over 1500 frames (flash_attn.rs:289-356) and the f32
    self-attention arm over that beam's cache (:370-399; fewer than 8 keys decline there and are
    skipped here), beams serially as decode_beam does (decoder.rs:542-596). Heads serial (the
    reference default) and heads over the host's cores (its FFAI_PAR_HEADS arm). One layer's
    cross-attention calls are timed and counted 24 times; every layer's self-attention is run."""
    import numpy as np
    import torch

    import oracle

    oracle.build()
    cpus, model = host_info()
    threads = min(cpus, H)  # the heads-parallel arm: one head per thread, up to the host's CPUs
    g = torch.Generator(device="cpu").manual_seed(3)  # the GPU decode leg's cache lengths
    lens = torch.randint(1, cap + 1, (layers, beams), generator=g, dtype=torch.int32).numpy()
    rng = np.random.default_rng(3)
    q = rng.standard_normal((1, H, 1, D)).astype(np.float32) * np.float32(D ** -0.5)
    kt16 = rng.standard_normal((1, H, D, T_enc)).astype(np.float16)
    v16 = rng.standard_normal((1, H, T_enc, D)).astype(np.float16)
    kt_self = rng.standard_normal((1, H, D, cap)).astype(np.float32)
    v_self = rng.standard_normal((1, H, cap, D)).astype(np.float32)
    selfs = [(np.ascontiguousarray(kt_self[..., :n]), np.ascontiguousarray(v_self[:, :, :n]))
             for n in sorted(set(int(x) for x in lens.ravel()))]
    by_len = {kt.shape[3]: (kt, v) for kt, v in selfs}
    out = {}
    for name, par in (("heads_serial", False), ("heads_parallel", True)):
        oracle.attend_f16kv(q, kt16, v16, par_heads=par, threads=threads)  # warm-up
        cross = []
        for _ in range(reps):
            t0 = time.perf_counter()
            for _b in range(beams):
                oracle.attend_f16kv(q, kt16, v16, par_heads=par, threads=threads)
            cross.append(time.perf_counter() - t0)
        t0 = time.perf_counter()
        for n in lens.ravel():
            if n >= 8:
                kt, v = by_len[int(n)]
                oracle.attend_f32(q, kt, v, par_heads=par, threads=threads)
        self_s = time.perf_counter() - t0
        out[f"us_per_step_{name}"] = (float(np.median(cross)) * layers + self_s) * 1e6
    out["threads"] = threads
    out["host_cpus"] = cpus
    out["cpu_model"] = model
    out["kind"] = "port"
    out["sample"] = (f"one layer's {beams} cross-attention calls (f16 K/V, {H} heads x {T_enc} "
                     f"frames), median of {reps}, x {layers} layers; plus all {layers * beams} "
                     f"self-attention calls (f32 caches, the GPU leg's lengths); heads-parallel "
                     f"arm on a persistent pool of {threads} threads, as rayon's")
    return out


def load_traffic(name: str):
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get(name)
    except (OSError, ValueError):
        return None


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: there is no multi-GPU path (asked for {args.gpus}). "
              f"The attention shards over (batch, head) with no exchange, so N GPUs would each "
              f"run this benchmark's kernels on their share of the heads.", file=sys.stderr)
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    from ffai_amd import flash_attn as fa
    from ffai_amd import _lib

    _lib.load()
    legs = set() if args.skip_extras else {x for x in args.legs.split(",") if x and x != "none"}
    if legs == {"copy"}:
        print(json.dumps({"copy_calibration": copy_bench(torch, max(args.steps, 1))}), flush=True)
        return
    if legs == {"gemv_probe"}:
        print(json.dumps({"gemv_probe": gemv_probe(torch)}), flush=True)
        return
    log("encoder: whisper-large-v3 bf16 ...")
    enc = encoder_bench(torch, fa, args.steps, args.warmup, args.layers)
    log(f"encoder: {enc['tflops']:.1f} TFLOP/s, {enc['ms_per_step']:.3f} ms/step")
    extras = {}
    if "decode" in legs:
        log("decode: beam-5 whisper-medium step ...")
        dec = decode_bench(torch, fa, max(args.steps * 10, 100), 10, graphs=not args.eager)
        log(f"decode: {dec['us_per_step']:.1f} us/step, {dec['gbps']:.0f} GB/s")
        extras["decode_beam5"] = dec
    if "decode_ref" in legs:
        log("decode, the reference's calls: per beam, f32 q over f32 self / f16 cross caches ...")
        dr = decode_ref_bench(torch, fa, max(args.steps * 2, 20), 3)
        log(f"decode (reference calls): {dr['us_per_step']:.1f} us/step ({dr['gbps']:.0f} GB/s); "
            f"cross {dr['cross_us_per_launch']:.2f} us/launch ({dr['cross_gbps_per_launch']:.0f} "
            f"GB/s), self {dr['self_us_per_launch']:.2f} us/launch "
            f"({dr['self_gbps_per_launch']:.0f} GB/s), self 5 beams per call "
            f"{dr['self_batched_us_per_launch']:.2f} us/launch "
            f"({dr['self_batched_gbps_per_launch']:.0f} GB/s)")
        extras["decode_ref_beam5"] = dr
    if "state" in legs:
        log("decode state: append + beam reorder, whisper-medium ...")
        st = decode_state_bench(torch, fa, 100, 10)
        log(f"decode state: {st['state_us_per_step']:.1f} us/step ({st['state_gbps']:.0f} GB/s), "
            f"full step {st['full_step_us']:.1f} us, cross build {st['cross_build_us_per_window']:.1f} us, "
            f"prompt step {st['prompt_step_us']:.1f} us ({st['prompt_step_tflops']:.1f} TFLOP/s), "
            f"q/k/v + append {st['qkv_and_append_us_per_step']:.1f} us, fused "
            f"{st['qkv_into_cache_us_per_step']:.1f} us")
        extras["decode_state_beam5"] = st
    if "block" in legs:
        log("encoder block: whisper-large-v3 projections + attention + out-projection ...")
        blk = encoder_block_bench(torch, fa, max(args.steps // 4, 3), 1)
        log(f"encoder block: {blk['ms_per_window']:.3f} ms per window-layer, "
            f"{blk['tflops']:.1f} TFLOP/s")
        extras["encoder_block_large_v3"] = blk
    if "gemv" in legs:
        log("decoder GEMVs: beam-5 whisper-medium step ...")
        gv = gemv_bench(torch, 50, 5)
        log(f"decoder GEMVs: {gv['us_per_step']:.1f} us/step ({gv['gbps']:.0f} GB/s); vocabulary "
            f"projection {gv['vocab_us']:.1f} us ({gv['vocab_gbps']:.0f} GB/s); per launch "
            + ", ".join(f"{k} {v:.2f} us" for k, v in gv["us_per_launch"].items()))
        extras["decoder_gemv_beam5"] = gv
    if "gemv_large" in legs:
        log("decoder GEMVs: beam-5 whisper-large step (d 1280, 32 layers) ...")
        gl = gemv_bench(torch, 50, 5, n=1280, layers=32, vocab=51866)
        log(f"decoder GEMVs large: {gl['us_per_step']:.1f} us/step ({gl['gbps']:.0f} GB/s); "
            f"vocabulary projection {gl['vocab_us']:.1f} us; per launch "
            + ", ".join(f"{k} {v:.2f} us" for k, v in gl["us_per_launch"].items()))
        extras["decoder_gemv_large_beam5"] = gl
    if "tiny" in legs:
        log("encoder: whisper-tiny f32 ...")
        tiny = encoder_bench(torch, fa, max(args.steps * 5, 50), args.warmup, 4, B=1, H=6,
                             dtype="f32", seed=1)
        tiny["frac_of_f32_peak"] = tiny["tflops"] / PEAK_F32_TFLOPS
        extras["encoder_tiny_f32"] = tiny
        log(f"tiny f32: {tiny['tflops']:.2f} TFLOP/s")
    if "small" in legs:
        log("encoder: whisper-small bf16 ...")
        small = encoder_bench(torch, fa, args.steps, args.warmup, 4, B=8, H=12, seed=2,
                              k_mult=2.0)
        small["frac_of_bf16_peak"] = small["tflops"] / PEAK_BF16_TFLOPS
        extras["encoder_small_bf16"] = small
        log(f"small bf16: {small['tflops']:.1f} TFLOP/s")
        log("encoder: whisper-small f32 ...")
        small32 = encoder_bench(torch, fa, args.steps, args.warmup, 4, B=8, H=12, seed=2,
                                k_mult=2.0, dtype="f32")
        small32["frac_of_f32_peak"] = small32["tflops"] / PEAK_F32_TFLOPS
        extras["encoder_small_f32"] = small32
        log(f"small f32: {small32['tflops']:.2f} TFLOP/s")
    if "prefill" in legs:
        log("prefill: qwen2-vl causal GQA bf16 ...")
        pre = encoder_bench(torch, fa, args.steps, args.warmup, 4, B=1, H=12, H_kv=2, T=4096,
                            D=128, seed=5, causal=True)
        pre["frac_of_bf16_peak"] = pre["tflops"] / PEAK_BF16_TFLOPS
        extras["prefill_causal_gqa_d128"] = pre
        log(f"prefill: {pre['tflops']:.1f} TFLOP/s")
    if "floor" in legs:
        log("launch floor: empty kernel and bare 6 MB reads in graphs ...")
        fl = floor_bench(torch)
        log(f"launch floor: empty {fl['empty_us']:.2f} us, 6 MB read "
            + ", ".join(f"{k} WGs {v:.2f} us" for k, v in fl["read_us"].items()))
        extras["launch_floor"] = fl
    if "keys" in legs:
        for name, bb, hh in (("large_v3", 16, 20), ("small", 8, 12)):
            log(f"key sweep: the {name} layer's items over 1500 .. 6000 keys ...")
            ks = key_sweep_bench(torch, fa, B=bb, H=hh)
            log(f"key sweep {name}: "
                + ", ".join(f"{p_['keys']} keys {p_['us']:.1f} us" for p_ in ks["points"])
                + f"; per 1500 keys {ks['us_per_1500_keys']:.1f} us ({ks['loop_tflops']:.0f} "
                f"TFLOP/s in the loops), fixed {ks['fixed_us']:.1f} us "
                f"({ks['fixed_share_at_1500']:.1%} of the 1500-key launch)")
            extras[f"key_sweep_{name}_items"] = ks
    if "stamps" in legs:
        log("phase stamps: fused kernel (large-v3 layer) and decode kernel (beam-5 layer) ...")
        stp = stamps_bench(torch, fa)
        e = stp["encoder_large_v3_layer"]
        log("phase stamps: encoder " + ", ".join(f"{k} {v:.1%}" for k, v in e["share"].items())
            + f"; {e['ns_per_tile']:.0f} ns per tile per wave")
        for name in ("encoder_large_v3_layer", "encoder_small_layer", "prefill_qwen2vl"):
            t = stp[name]
            log(f"phase stamps: {name} workgroups (median ns): prologue {t['prologue_ns']:.0f}, "
                f"loop of {t['loop_tiles_most']} tiles {t['loop_ns_most_tiles']:.0f}, epilogue "
                f"{t['epilogue_issue_ns']:.0f} + ack {t['store_ack_ns']:.0f}; per slot: startup "
                f"{t['slot_startup_ns']:.0f}, gaps {t['slot_gaps_ns']:.0f}, tail "
                f"{t['slot_tail_ns']:.0f}, loops {t['slot_loops_ns']:.0f} of {t['span_ns']:.0f}")
        for name in ("decode_cross_beam5", "decode_self_beam5"):
            log(f"phase stamps: {name} {stp[name]}")
        extras["phase_stamps"] = stp
    if "pipes" in legs:
        log("pipe rates: MFMA, v_exp_f32, FMA and mixes ...")
        pr = pipes_bench(torch)
        log(f"pipes: MFMA-only {pr['mfma_tflops']} TFLOP/s by waves per SIMD; cycles per "
            f"iteration per SIMD at 2.4 GHz {pr['cycles_at_2p4ghz_per_iter_per_simd']}")
        extras["pipe_rates"] = pr
    cpu = None
    if not args.skip_cpu:
        log("cpu baselines (oracle restating the reference's kernel) ...")
        cpus = cpu_baselines()
        cpu = cpus["encoder_large_v3"]
        log(f"cpu: {cpu['value'] * 1e3:.1f} GFLOP/s on {cpu['cores']} threads")
        for name, leg in (("encoder_tiny_f32", "encoder_tiny_f32"),
                          ("encoder_small_f32", "encoder_small_f32"),
                          ("prefill_causal_gqa_d128", "prefill_causal_gqa_d128")):
            extras.setdefault(leg, {})["cpu"] = cpus[name]
            log(f"cpu {name}: {cpus[name]['value'] * 1e3:.1f} GFLOP/s on {cpus[name]['cores']} "
                f"threads")
        if "decode_beam5" in extras:
            dcpu = cpu_decode_baseline()
            extras["decode_beam5"]["cpu"] = dcpu
            log(f"cpu decode step: {dcpu['us_per_step_heads_serial']:.0f} us heads serial, "
                f"{dcpu['us_per_step_heads_parallel']:.0f} us heads parallel")

    achieved = enc["flop_per_launch"] / (enc["avg_launch_us"] * 1e-6) / 1e12
    line = {
        "metric": "attention TFLOP/s + % MFMA peak (encoder); decode-step us + HBM GB/s (beam 5)",
        "value": round(enc["tflops"], 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(enc["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: Q/K/V ~ N(0,1) from seed 4, K given transposed (B,H,D,T)",
        "config": {"workload": "whisper-large-v3 encoder self-attention", "batch": 16,
                   "heads": 20, "seq": 1500, "head_dim": 64, "layers": args.layers,
                   "causal": False, "scale": 0.125, "k_layout": "transposed",
                   "out_dtype": "bf16"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2),
                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": load_traffic("encoder_large_v3_bf16")},
        "cpu_baseline": cpu,
    }
    if "decode_beam5" in extras:
        dec = extras["decode_beam5"]
        line["roofline_decode"] = {"bound": "hbm", "achieved": round(dec["gbps"], 1),
                                   "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                                   "frac": round(dec["gbps"] / PEAK_HBM_GBPS, 4),
                                   "us_per_step": round(dec["us_per_step"], 1),
                                   "traffic": load_traffic("decode_beam5")}
    if extras:
        line["extras"] = extras
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
