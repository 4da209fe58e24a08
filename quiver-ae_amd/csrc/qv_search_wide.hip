// qv_search_wide.hip -- the per-query-LUT search kernels for a top-k above 64
// (the reference's retset_push_32 path, gpu_primitives.cuh:99-138, for any
// k): entries 0 .. 63 in the wave's registers as in every other kernel,
// entries 64 .. k - 1 in LDS after the query's area.  Kept apart from the
// other kernels so theirs stay exactly as they are; every element type, PQ
// layout and neighbour-slot count, beams of Q = 2, 4, 7, 10 or 16 positions
// per lane.
#include "qv_search_kernels.hpp"

namespace {

template <class T, int Q, int NPL>
KernelFn wide_mc(int M) {
  if (M == 32) return search_kernel<T, Q, 32, NPL, true>;
  if (M == 48) return search_kernel<T, Q, 48, NPL, true>;
  return search_kernel<T, Q, 0, NPL, true>;
}

template <class T, int NPL>
KernelFn wide_q(int Q, int M) {
  switch (Q) {
    case 2: return wide_mc<T, 2, NPL>(M);
    case 4: return wide_mc<T, 4, NPL>(M);
    case 7: return wide_mc<T, 7, NPL>(M);
    case 10: return wide_mc<T, 10, NPL>(M);
    case 16: return wide_mc<T, 16, NPL>(M);
    default: return nullptr;
  }
}

template <class T>
KernelFn wide_npl(int Q, int M, int npl) {
  return npl > 1 ? wide_q<T, 2>(Q, M) : wide_q<T, 1>(Q, M);
}

}  // namespace

namespace qv {
namespace sk {

KernelFn pick_kernel_wide(int dtype, int Q, int M, int npl) {
  if (dtype == QV_UINT8) return wide_npl<uint8_t>(Q, M, npl);
  if (dtype == QV_INT8) return wide_npl<int8_t>(Q, M, npl);
  return wide_npl<float>(Q, M, npl);
}

}  // namespace sk
}  // namespace qv
