// qv_search_r128.hip -- the search kernels with two neighbour slots per lane
// (indexes of max degree 65..128, such as the reference's R = 128 layouts,
// ae/scripts/common.sh:118-121), for every element type and PQ layout.  The
// register beam holds Q = 1, 2, 4, 7, 10 or 16 positions per lane (a request
// for another Q gets the next larger one: the shared-pivot kernel's LDS beam
// is sized by ef, not by Q).
#include "qv_search_kernels.hpp"

namespace {

constexpr int round_q(int Q) { return Q <= 2 ? Q : (Q <= 4 ? 4 : (Q <= 7 ? 7 : (Q <= 10 ? 10 : 16))); }

template <class T, int Q>
KernelFn lut_mc(int M) {
  if (M == 32) return search_kernel<T, Q, 32, 2>;
  if (M == 48) return search_kernel<T, Q, 48, 2>;
  return search_kernel<T, Q, 0, 2>;
}

template <class T>
KernelFn lut_q(int Q, int M) {
  switch (round_q(Q)) {
    case 1: return lut_mc<T, 1>(M);
    case 2: return lut_mc<T, 2>(M);
    case 4: return lut_mc<T, 4>(M);
    case 7: return lut_mc<T, 7>(M);
    case 10: return lut_mc<T, 10>(M);
    default: return lut_mc<T, 16>(M);
  }
}

template <class T, int MC, int SC>
KernelFn sp_q(int Q) {
  switch (round_q(Q)) {
    case 1: return search_kernel_sp<T, 1, MC, SC, 2>;
    case 2: return search_kernel_sp<T, 2, MC, SC, 2>;
    case 4: return search_kernel_sp<T, 4, MC, SC, 2>;
    case 7: return search_kernel_sp<T, 7, MC, SC, 2>;
    case 10: return search_kernel_sp<T, 10, MC, SC, 2>;
    default: return search_kernel_sp<T, 16, MC, SC, 2>;
  }
}

template <class T>
KernelFn sp_m(int Q, int M) {
  if (M == 32) return sp_q<T, 32, 4>(Q);
  if (M == 48) return sp_q<T, 48, 2>(Q);
  return nullptr;
}

}  // namespace

namespace qv {
namespace sk {

KernelFn pick_kernel_r128(int dtype, int Q, int M) {
  if (Q < 1 || Q > 16) return nullptr;
  if (dtype == QV_UINT8) return lut_q<uint8_t>(Q, M);
  if (dtype == QV_INT8) return lut_q<int8_t>(Q, M);
  return lut_q<float>(Q, M);
}

KernelFn pick_kernel_sp_r128(int dtype, int Q, int M) {
  if (Q < 1 || Q > 16) return nullptr;
  if (dtype == QV_UINT8) return sp_m<uint8_t>(Q, M);
  if (dtype == QV_INT8) return sp_m<int8_t>(Q, M);
  return sp_m<float>(Q, M);
}

}  // namespace sk
}  // namespace qv
