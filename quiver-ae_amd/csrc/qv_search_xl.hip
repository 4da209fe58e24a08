// qv_search_xl.hip -- the per-query-LUT search kernels for ef in (1024, 2048]:
// 32 register beam positions per lane (the unvisited-slot mask holds 32 bits),
// a 16 KB LDS beam, every element type, PQ layout and neighbour-slot count,
// with a top-k of up to 64 or above (entries past the 64th in LDS).  The
// shared-pivot kernel stops at ef = 1024: a beam of 2048 entries would leave
// its pivot table room for two queries per CU.
#include "qv_search_kernels.hpp"

namespace {

template <class T, int NPL, bool WK>
KernelFn xl_mc(int M) {
  if (M == 32) return search_kernel<T, 32, 32, NPL, WK>;
  if (M == 48) return search_kernel<T, 32, 48, NPL, WK>;
  return search_kernel<T, 32, 0, NPL, WK>;
}

template <class T>
KernelFn xl_t(int M, int npl, bool wide) {
  if (npl > 1) return wide ? xl_mc<T, 2, true>(M) : xl_mc<T, 2, false>(M);
  return wide ? xl_mc<T, 1, true>(M) : xl_mc<T, 1, false>(M);
}

}  // namespace

namespace qv {
namespace sk {

KernelFn pick_kernel_xl(int dtype, int M, int npl, bool wide) {
  if (dtype == QV_UINT8) return xl_t<uint8_t>(M, npl, wide);
  if (dtype == QV_INT8) return xl_t<int8_t>(M, npl, wide);
  return xl_t<float>(M, npl, wide);
}

}  // namespace sk
}  // namespace qv
