// Launch helpers shared by the per-dtype translation units (fwd_*.hip).
#pragma once

#include "attn_kernels.cuh"

namespace ffai {
namespace {

template <int MODE, int KVT, int OUTT, int D, bool KT, int NW>
hipError_t launch_one(const FwdParams& p, hipStream_t s) {
  const unsigned grid = (unsigned)((p.n_work + 7) / 8 * 8);
  hipLaunchKernelGGL((fwd_kernel<MODE, KVT, OUTT, D, KT, NW>), dim3(grid), dim3(NW * 64), 0, s,
                     p);
  return hipGetLastError();
}

template <int MODE, int KVT, int OUTT, int D, bool KT>
hipError_t pick_waves(const FwdParams& p, int waves, hipStream_t s) {
  switch (waves) {
    case 1: return launch_one<MODE, KVT, OUTT, D, KT, 1>(p, s);
    case 4: return launch_one<MODE, KVT, OUTT, D, KT, 4>(p, s);
    default: return hipErrorInvalidValue;
  }
}

template <int MODE, int KVT, int OUTT, int D>
hipError_t pick_layout(const FwdParams& p, bool kt, int waves, hipStream_t s) {
  return kt ? pick_waves<MODE, KVT, OUTT, D, true>(p, waves, s)
            : pick_waves<MODE, KVT, OUTT, D, false>(p, waves, s);
}

template <int MODE, int KVT, int OUTT>
hipError_t pick_dim(const FwdParams& p, int d, bool kt, int waves, hipStream_t s) {
  if (d == 64) return pick_layout<MODE, KVT, OUTT, 64>(p, kt, waves, s);
  if constexpr (MODE != kF32) {
    if (d == 128) return pick_layout<MODE, KVT, OUTT, 128>(p, kt, waves, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace
}  // namespace ffai
