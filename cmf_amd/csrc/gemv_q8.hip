// q8 GEMV kernel instances (k_gemv_q8, gemv_kern.h).
#include "gemv_kern.h"

namespace cmf {
GemvKernel q8_kernel(int m, int xm, int ks) { return m <= 5 ? q8_by_xm<true>(xm, ks) : q8_by_xm<false>(xm, ks); }
GemvKernel q8_kernel_m1(int nk, bool resid, int* ks, size_t* lds) { return q8_m1_pick(nk, resid, ks, lds); }
}  // namespace cmf
