// Launch dispatch by dtype and the split-key combine launch.
#include "attn_kernels.cuh"

namespace ffai {


hipError_t launch_fwd(const FwdParams& p, int mode, int kv_dtype, int out_dtype, int head_dim,
                      bool k_transposed, int variant, hipStream_t stream) {
  if (mode == kBF16)
    return kv_dtype == kBF16 ? launch_fwd_bf16(p, out_dtype, head_dim, k_transposed, variant, stream)
                             : hipErrorInvalidValue;
  if (mode == kF16)
    return kv_dtype == kF16 ? launch_fwd_f16(p, out_dtype, head_dim, k_transposed, variant, stream)
                            : hipErrorInvalidValue;
  if (mode == kF32 && out_dtype == kF32)
    return launch_fwd_f32(p, kv_dtype, head_dim, k_transposed, variant, stream);
  return hipErrorInvalidValue;
}

hipError_t launch_combine(const CombineParams& p, int out_dtype, int head_dim,
                          hipStream_t stream) {
  const int64_t rows = (int64_t)p.B * p.Hq * p.Tq;
#define FFAI_COMBINE(OT, DD)                                                                  \
  hipLaunchKernelGGL((combine_kernel<OT, DD>), dim3((unsigned)((rows + 1024 / DD - 1) / (1024 / DD))), \
                     dim3(256), 0, stream, p)
  if (head_dim == 64) {
    if (out_dtype == kF32) FFAI_COMBINE(kF32, 64);
    else if (out_dtype == kBF16) FFAI_COMBINE(kBF16, 64);
    else FFAI_COMBINE(kF16, 64);
  } else if (head_dim == 128) {
    if (out_dtype == kF32) FFAI_COMBINE(kF32, 128);
    else if (out_dtype == kBF16) FFAI_COMBINE(kBF16, 128);
    else FFAI_COMBINE(kF16, 128);
  } else {
    return hipErrorInvalidValue;
  }
#undef FFAI_COMBINE
  return hipGetLastError();
}

}  // namespace ffai
