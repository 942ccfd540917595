// Instantiations of the forward kernel for one input dtype (compiled in parallel).
#include "attn_launch.cuh"

namespace ffai {

hipError_t launch_fwd_f32(const FwdParams& p, int kv_dtype, int d, bool kt, int variant,
                           hipStream_t s) {
  if (kv_dtype == kF32) return pick_dim<kF32, kF32, kF32>(p, d, kt, variant, s);
  if (kv_dtype == kF16) return pick_dim<kF32, kF16, kF32>(p, d, kt, variant, s);
  if (kv_dtype == kBF16) return pick_dim<kF32, kBF16, kF32>(p, d, kt, variant, s);
  return hipErrorInvalidValue;
}

}  // namespace ffai
