// qv_search_deep.hip -- the search kernels for ef in (448, 1024]: one
// neighbour slot per lane and Q = 10 or 16 register beam positions per lane,
// for every element type and PQ layout.
#include "qv_search_kernels.hpp"

namespace {

template <class T, int Q>
KernelFn lut_mc(int M) {
  if (M == 32) return search_kernel<T, Q, 32, 1>;
  if (M == 48) return search_kernel<T, Q, 48, 1>;
  return search_kernel<T, Q, 0, 1>;
}

template <class T>
KernelFn lut_q(int Q, int M) {
  return Q <= 10 ? lut_mc<T, 10>(M) : lut_mc<T, 16>(M);
}

template <class T>
KernelFn sp_m(int Q, int M) {
  if (M == 32) return Q <= 10 ? search_kernel_sp<T, 10, 32, 4, 1> : search_kernel_sp<T, 16, 32, 4, 1>;
  if (M == 48) return Q <= 10 ? search_kernel_sp<T, 10, 48, 2, 1> : search_kernel_sp<T, 16, 48, 2, 1>;
  return nullptr;
}

}  // namespace

namespace qv {
namespace sk {

KernelFn pick_kernel_deep(int dtype, int Q, int M) {
  if (Q < 8 || Q > 16) return nullptr;
  if (dtype == QV_UINT8) return lut_q<uint8_t>(Q, M);
  if (dtype == QV_INT8) return lut_q<int8_t>(Q, M);
  return lut_q<float>(Q, M);
}

KernelFn pick_kernel_sp_deep(int dtype, int Q, int M) {
  if (Q < 8 || Q > 16) return nullptr;
  if (dtype == QV_UINT8) return sp_m<uint8_t>(Q, M);
  if (dtype == QV_INT8) return sp_m<int8_t>(Q, M);
  return sp_m<float>(Q, M);
}

}  // namespace sk
}  // namespace qv
