/*
 * ffai_probe.h -- launch-floor and pipe-rate probes, diagnostics with no counterpart in the
 * reference.
 *
 * The decode-step kernels move a few MB per launch, so their time is mostly launch and latency.
 * These two kernels measure that floor on the same device and stream: an empty kernel, and a
 * bare streaming read of `bytes` by `workgroups` workgroups of 256 threads (16-byte
 * non-temporal loads, one float per workgroup written to `out[workgroups]`).
 *
 * ffai_probe_pipes measures the pipe rates the fused kernel's per-tile budget rests on: each
 * of `workgroups` workgroups of 256 threads (one wave per SIMD of a CU per workgroup, so
 * workgroups = 256 x waves per SIMD) runs `iters` iterations of a fixed mix and writes one
 * float per thread to out[workgroups * 256]. kind 0: 4 bf16 32x32x16 MFMAs on independent
 * accumulators; 1: 8 v_exp_f32 on 8 independent chains; 2: 8 FMAs; 3: the 4 MFMAs with 8 exp
 * and 8 FMA spread between them; 4: the 4 MFMAs with 16 exp and 16 FMA.
 *
 * Asynchronous on `stream`; they return FFAI_OK or a negative ffai_status (ffai_attn.h).
 */
#ifndef FFAI_PROBE_H
#define FFAI_PROBE_H

#include <stddef.h>

#include "ffai_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

int ffai_probe_empty(int workgroups, void* stream);
int ffai_probe_read(const void* src, size_t bytes, float* out, int workgroups, void* stream);
int ffai_probe_pipes(int kind, int workgroups, int iters, float* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FFAI_PROBE_H */
