// Launch dispatch by dtype.
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

}  // namespace ffai
