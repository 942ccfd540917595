// Instantiations of the f32-query decode kernel (decode_vec_kernel, decode_kernels.cuh): K/V
// f32, f16 or bf16, K given transposed or as rows, 1, 2, 4 or 8 waves per workgroup.
#include "decode_kernels.cuh"

namespace ffai {
namespace {

template <int KVT, bool KT, int NWD>
hipError_t launch_vec(const DecodeParams& p, hipStream_t s) {
  const dim3 grid((unsigned)p.n_split, (unsigned)p.Hkv, (unsigned)p.B);  // (split, kv-head, batch)
  hipLaunchKernelGGL((decode_vec_kernel<KVT, KT, NWD>), grid, dim3(NWD * 64), 0, s, p);
  return hipGetLastError();
}

template <int KVT, bool KT>
hipError_t pick_vec_waves(const DecodeParams& p, int waves, hipStream_t s) {
  switch (waves) {
    case 1: return launch_vec<KVT, KT, 1>(p, s);
    case 2: return launch_vec<KVT, KT, 2>(p, s);
    case 4: return launch_vec<KVT, KT, 4>(p, s);
    case 8: return launch_vec<KVT, KT, 8>(p, s);
    default: return hipErrorInvalidValue;
  }
}

template <int KVT>
hipError_t pick_vec_layout(const DecodeParams& p, bool kt, int waves, hipStream_t s) {
  return kt ? pick_vec_waves<KVT, true>(p, waves, s) : pick_vec_waves<KVT, false>(p, waves, s);
}

}  // namespace

hipError_t launch_decode_vec(const DecodeParams& p, int kv_dtype, bool k_transposed, int waves,
                             hipStream_t stream) {
  if (p.group * p.Tq != 1) return hipErrorInvalidValue;
  if (kv_dtype == kF32) return pick_vec_layout<kF32>(p, k_transposed, waves, stream);
  if (kv_dtype == kF16) return pick_vec_layout<kF16>(p, k_transposed, waves, stream);
  if (kv_dtype == kBF16) return pick_vec_layout<kBF16>(p, k_transposed, waves, stream);
  return hipErrorInvalidValue;
}

}  // namespace ffai
