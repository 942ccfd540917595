// Probes (include/ffai_probe.h): an empty kernel and a bare streaming read, so that the
// per-launch floor under the decode kernels can be measured beside them; and pipe-rate loops
// (MFMA, v_exp_f32, FMA, and their mixes) behind the fused kernel's per-tile cycle budget.
#include "../../include/ffai_probe.h"

#include <hip/hip_runtime.h>

#include "attn_kernels.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void probe_empty_kernel() {}

// Workgroup w reads its contiguous share of the 16-byte chunks, each thread issuing up to 16
// independent loads before it uses any (as the decode kernel has its whole share in flight).
// Nothing is reduced across threads: a thread stores only if its XOR of the data equals a value
// the data never produces (all-zero input), which keeps the loads alive without adding a serial
// tail to the read.
__global__ __launch_bounds__(256) void probe_read_kernel(const u32x4* src, int64_t chunks,
                                                         int64_t per, float* out) {
  constexpr int kBatch = 16;
  const int tid = (int)__builtin_amdgcn_workitem_id_x();
  const int wg = (int)__builtin_amdgcn_workgroup_id_x();
  const int64_t begin = (int64_t)wg * per;
  const int64_t end = begin + per < chunks ? begin + per : chunks;
  uint32_t acc = 0;
  for (int64_t i0 = begin + tid; i0 < end; i0 += 256 * kBatch) {
    u32x4 x[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const int64_t i = i0 + (int64_t)j * 256;
      x[j] = __builtin_nontemporal_load(src + (i < end ? i : begin));
    }
#pragma unroll
    for (int j = 0; j < kBatch; ++j)
      if (i0 + (int64_t)j * 256 < end) acc ^= x[j][0] ^ x[j][1] ^ x[j][2] ^ x[j][3];
  }
  if (acc == 0x9e3779b9u) out[wg] = (float)acc;
}

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// Per iteration: NM bf16 32x32x16 MFMAs on NM independent accumulators, NE v_exp_f32 and NF FMAs
// on 8 independent chains (exp2(-e) and e * 0.5 + 0.25 stay bounded), the VALU share spread
// evenly between the MFMAs. Every thread writes one float so that nothing is dead code.
template <int NM, int NE, int NF>
__global__ __launch_bounds__(256) void probe_pipes_kernel(int iters, float seed, float* out) {
  bf16x8 x;
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = (__bf16)(seed + 0.01f * i + 1e-4f * threadIdx.x);
  f32x16 acc[NM > 0 ? NM : 1] = {};
  float e[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) e[j] = seed * (j + 1) * 1e-3f + threadIdx.x * 1e-6f;
  constexpr int G = NM > 0 ? NM : 1;  // VALU groups per iteration
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int m = 0; m < G; ++m) {
      if constexpr (NM > 0) acc[m] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x, x, acc[m], 0, 0, 0);
#pragma unroll
      for (int j = m * NE / G; j < (m + 1) * NE / G; ++j)
        e[j % 8] = __builtin_amdgcn_exp2f(-e[j % 8]);
#pragma unroll
      for (int j = m * NF / G; j < (m + 1) * NF / G; ++j)
        e[j % 8] = __builtin_fmaf(e[j % 8], 0.5f, 0.25f);
    }
  }
  float s = 0.f;
#pragma unroll
  for (int m = 0; m < G; ++m)
#pragma unroll
    for (int i = 0; i < 16; ++i) s += acc[m][i];
#pragma unroll
  for (int j = 0; j < 8; ++j) s += e[j];
  out[(int64_t)blockIdx.x * 256 + threadIdx.x] = s;
}

}  // namespace

extern "C" {

int ffai_probe_empty(int workgroups, void* stream) {
  if (workgroups < 1) return ffai::api_fail(FFAI_ERR_INVALID, "workgroups must be >= 1");
  hipLaunchKernelGGL(probe_empty_kernel, dim3((unsigned)workgroups), dim3(256), 0,
                     static_cast<hipStream_t>(stream));
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? FFAI_OK : ffai::api_fail(FFAI_ERR_HIP, hipGetErrorString(e));
}

int ffai_probe_read(const void* src, size_t bytes, float* out, int workgroups, void* stream) {
  if (!src || !out || workgroups < 1 || bytes < 16 || bytes % 16 || (uintptr_t)src % 16)
    return ffai::api_fail(FFAI_ERR_INVALID,
                          "src and out must be set, bytes a positive multiple of 16, src 16-byte "
                          "aligned, workgroups >= 1");
  const int64_t chunks = (int64_t)(bytes / 16);
  hipLaunchKernelGGL(probe_read_kernel, dim3((unsigned)workgroups), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const u32x4*>(src), chunks,
                     (chunks + workgroups - 1) / workgroups, out);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? FFAI_OK : ffai::api_fail(FFAI_ERR_HIP, hipGetErrorString(e));
}

int ffai_probe_pipes(int kind, int workgroups, int iters, float* out, void* stream) {
  if (!out || workgroups < 1 || iters < 1 || kind < 0 || kind > 4)
    return ffai::api_fail(FFAI_ERR_INVALID, "kind 0..4, workgroups >= 1, iters >= 1, out set");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 g((unsigned)workgroups), b(256);
  switch (kind) {
    case 0: hipLaunchKernelGGL((probe_pipes_kernel<4, 0, 0>), g, b, 0, s, iters, 1.f, out); break;
    case 1: hipLaunchKernelGGL((probe_pipes_kernel<0, 8, 0>), g, b, 0, s, iters, 1.f, out); break;
    case 2: hipLaunchKernelGGL((probe_pipes_kernel<0, 0, 8>), g, b, 0, s, iters, 1.f, out); break;
    case 3: hipLaunchKernelGGL((probe_pipes_kernel<4, 8, 8>), g, b, 0, s, iters, 1.f, out); break;
    default: hipLaunchKernelGGL((probe_pipes_kernel<4, 16, 16>), g, b, 0, s, iters, 1.f, out); break;
  }
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? FFAI_OK : ffai::api_fail(FFAI_ERR_HIP, hipGetErrorString(e));
}

}  // extern "C"
