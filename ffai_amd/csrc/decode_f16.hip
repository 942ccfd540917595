// f16 instantiations of the decode kernel (bf16 and the dispatch: decode.hip).
#include "decode_launch.cuh"

namespace ffai {

hipError_t launch_decode_f16(const DecodeParams& p, int out_dtype, int head_dim,
                             bool k_transposed, int waves, hipStream_t stream) {
  return launch_decode_mode<kF16>(p, out_dtype, head_dim, k_transposed, waves, stream);
}

}  // namespace ffai
