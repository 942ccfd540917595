// Instantiations of the forward kernel for one input dtype (compiled in parallel).
#include "attn_launch.cuh"

namespace ffai {

hipError_t launch_fwd_f16(const FwdParams& p, int out_dtype, int d, bool kt, int variant,
                           hipStream_t s) {
  if (out_dtype == kF16) return pick_dim<kF16, kF16, kF16>(p, d, kt, variant, s);
  if (out_dtype == kF32) return pick_dim<kF16, kF16, kF32>(p, d, kt, variant, s);
  return hipErrorInvalidValue;
}

}  // namespace ffai
