// bf16 instantiations of the decode kernel, and the dispatch on the input type (the f16 ones are
// in decode_f16.hip: two translation units compile in parallel).
#include "decode_launch.cuh"

namespace ffai {

hipError_t launch_decode(const DecodeParams& p, int mode, int out_dtype, int head_dim,
                         bool k_transposed, int waves, hipStream_t stream) {
  if (mode == kBF16)
    return launch_decode_mode<kBF16>(p, out_dtype, head_dim, k_transposed, waves, stream);
  if (mode == kF16) return launch_decode_f16(p, out_dtype, head_dim, k_transposed, waves, stream);
  return hipErrorInvalidValue;
}

}  // namespace ffai
