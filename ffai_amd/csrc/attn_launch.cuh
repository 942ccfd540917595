// Launch helpers shared by the per-dtype translation units (fwd_*.hip).
#pragma once

#include "attn_kernels.cuh"
#include "attn_kernels16.cuh"

namespace ffai {
namespace {

template <int MODE, int KVT, int OUTT, int D, bool KT, int NW, int QW>
hipError_t launch_one(const FwdParams& p, hipStream_t s) {
  // two dispatch sections, each in whole XCD rounds
  const int xr = 1 << p.xcd_shift;
  const unsigned grid = (unsigned)(p.sec1_wgs + (p.n_work - p.sec1_work + xr - 1) / xr * xr);
  // Head_dim 128, four waves: 80 KB of LDS and <= 256 VGPRs admit two workgroups per CU. A grid
  // of fewer than two per CU then piles pairs onto some CUs and leaves others idle; 16 KB of
  // unused dynamic LDS keeps such a grid at one per CU (Qwen2-VL prefill, 384 workgroups:
  // 446 TFLOP/s against 407 with pairs; with 1536 workgroups pairs win, 770 against 585).
  const size_t pad = (MODE != kF32 && D == 128 && NW == 4 && p.n_work < 2 * p.cus) ? 16384 : 0;
  hipLaunchKernelGGL((fwd_kernel<MODE, KVT, OUTT, D, KT, NW, QW>), dim3(grid), dim3(NW * 64), pad,
                     s, p);
  return hipGetLastError();
}

template <int MODE, int OUTT, bool KT>
hipError_t launch_x16(const FwdParams& p, hipStream_t s) {
  const int xr = 1 << p.xcd_shift;
  const unsigned grid = (unsigned)(p.sec1_wgs + (p.n_work - p.sec1_work + xr - 1) / xr * xr);
  hipLaunchKernelGGL((fwd16_kernel<MODE, OUTT, KT>), dim3(grid), dim3(256), 0, s, p);
  return hipGetLastError();
}

// Launch shapes instantiated per head_dim and dtype (see Variant in attn_kernels.h).
template <int MODE, int KVT, int OUTT, int D, bool KT>
hipError_t pick_variant(const FwdParams& p, int variant, hipStream_t s) {
  switch (variant) {
    case kWave1: return launch_one<MODE, KVT, OUTT, D, KT, 1, 1>(p, s);
    case kWave4: return launch_one<MODE, KVT, OUTT, D, KT, 4, 1>(p, s);
    case kWave4x2:
      if constexpr (MODE != kF32 && D == 64) return launch_one<MODE, KVT, OUTT, D, KT, 4, 2>(p, s);
      return hipErrorInvalidValue;
    case kWave4x2x16:
      if constexpr (MODE != kF32 && D == 64) return launch_x16<MODE, OUTT, KT>(p, s);
      return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
  }
}

template <int MODE, int KVT, int OUTT, int D>
hipError_t pick_layout(const FwdParams& p, bool kt, int variant, hipStream_t s) {
  return kt ? pick_variant<MODE, KVT, OUTT, D, true>(p, variant, s)
            : pick_variant<MODE, KVT, OUTT, D, false>(p, variant, s);
}

template <int MODE, int KVT, int OUTT>
hipError_t pick_dim(const FwdParams& p, int d, bool kt, int variant, hipStream_t s) {
  if (d == 64) return pick_layout<MODE, KVT, OUTT, 64>(p, kt, variant, s);
  if constexpr (MODE != kF32) {
    if (d == 128) return pick_layout<MODE, KVT, OUTT, 128>(p, kt, variant, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace
}  // namespace ffai
