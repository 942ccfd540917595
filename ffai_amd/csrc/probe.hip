// Launch-floor probes (include/ffai_probe.h): an empty kernel, and a bare streaming read, so
// that the per-launch floor under the decode kernels can be measured beside them.
#include "../../include/ffai_probe.h"

#include <hip/hip_runtime.h>

#include "attn_kernels.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void probe_empty_kernel() {}

// Workgroup w reads its contiguous share of the 16-byte chunks, each thread issuing up to 16
// independent loads before it uses any (as the decode kernel has its whole share in flight), and
// thread 0 writes the workgroup's XOR of them (it keeps the loads alive).
__global__ __launch_bounds__(256) void probe_read_kernel(const u32x4* src, int64_t chunks,
                                                         float* out) {
  constexpr int kBatch = 16;
  const int64_t per = (chunks + gridDim.x - 1) / gridDim.x;
  const int64_t begin = (int64_t)blockIdx.x * per;
  const int64_t end = begin + per < chunks ? begin + per : chunks;
  uint32_t acc = 0;
  for (int64_t i0 = begin + threadIdx.x; i0 < end; i0 += 256 * kBatch) {
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
  __shared__ uint32_t red[256];
  red[threadIdx.x] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t s = 0;
    for (int t = 0; t < 256; ++t) s ^= red[t];
    out[blockIdx.x] = (float)s;
  }
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
  hipLaunchKernelGGL(probe_read_kernel, dim3((unsigned)workgroups), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const u32x4*>(src),
                     (int64_t)(bytes / 16), out);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? FFAI_OK : ffai::api_fail(FFAI_ERR_HIP, hipGetErrorString(e));
}

}  // extern "C"
