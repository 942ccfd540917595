// Launch of the decode kernel for one input type (head_dim 64 with 1, 2, 4 or 8 waves, head_dim
// 128 with 1, 2 or 4; K given transposed or as rows; f32 or same-type output; one or two
// 16-column blocks of query rows), instantiated by decode.hip (bf16) and decode_f16.hip (f16).
// Split units merge inside the same launch (the unit's last workgroup), so a call is one launch.
#pragma once

#include "decode_kernels.cuh"

namespace ffai {
namespace {

template <int MODE, int OUTT, int D, bool KT, int NWD>
hipError_t launch_dec(const DecodeParams& p, hipStream_t s) {
  const dim3 grid((unsigned)p.n_split, (unsigned)p.Hkv, (unsigned)p.B);  // (split, kv-head, batch)
  // one 16-column block of query rows for units of at most 16 rows, two up to 32
  if (p.group * p.Tq <= 16)
    hipLaunchKernelGGL((decode_kernel<MODE, OUTT, D, KT, NWD, 1>), grid, dim3(NWD * 64), 0, s, p);
  else
    hipLaunchKernelGGL((decode_kernel<MODE, OUTT, D, KT, NWD, 2>), grid, dim3(NWD * 64), 0, s, p);
  return hipGetLastError();
}

template <int MODE, int OUTT, int D, bool KT>
hipError_t pick_waves(const DecodeParams& p, int waves, hipStream_t s) {
  if (waves == 1) return launch_dec<MODE, OUTT, D, KT, 1>(p, s);
  if (waves == 2) return launch_dec<MODE, OUTT, D, KT, 2>(p, s);
  if (waves == 4) return launch_dec<MODE, OUTT, D, KT, 4>(p, s);
  if constexpr (D == 64) {
    if (waves == 8) return launch_dec<MODE, OUTT, D, KT, 8>(p, s);
  }
  return hipErrorInvalidValue;
}

template <int MODE, int OUTT>
hipError_t pick(const DecodeParams& p, int d, bool kt, int waves, hipStream_t s) {
  if (d == 64) return kt ? pick_waves<MODE, OUTT, 64, true>(p, waves, s)
                         : pick_waves<MODE, OUTT, 64, false>(p, waves, s);
  if (d == 128) return kt ? pick_waves<MODE, OUTT, 128, true>(p, waves, s)
                          : pick_waves<MODE, OUTT, 128, false>(p, waves, s);
  return hipErrorInvalidValue;
}

template <int MODE>
hipError_t launch_decode_mode(const DecodeParams& p, int out_dtype, int head_dim,
                              bool k_transposed, int waves, hipStream_t stream) {
  if (out_dtype == kF32) return pick<MODE, kF32>(p, head_dim, k_transposed, waves, stream);
  if (out_dtype == MODE) return pick<MODE, MODE>(p, head_dim, k_transposed, waves, stream);
  return hipErrorInvalidValue;
}

}  // namespace
}  // namespace ffai
