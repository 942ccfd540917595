/*
 * ffai_probe.h -- launch-floor probes, diagnostics with no counterpart in the reference.
 *
 * The decode-step kernels move a few MB per launch, so their time is mostly launch and latency.
 * These two kernels measure that floor on the same device and stream: an empty kernel, and a
 * bare streaming read of `bytes` by `workgroups` workgroups of 256 threads (16-byte
 * non-temporal loads, one float per workgroup written to `out[workgroups]`). Asynchronous on
 * `stream`; they return FFAI_OK or a negative ffai_status (ffai_attn.h).
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

#ifdef __cplusplus
}
#endif

#endif /* FFAI_PROBE_H */
