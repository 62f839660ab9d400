// q4t GEMV kernel instances (k_gemv_q4, gemv_kern.h).
#include "gemv_kern.h"

namespace cmf {
GemvKernel q4t_kernel(int m, int xm, int ks, int rb) { return q4_pick<DT_Q4T>(m, xm, ks, rb); }
GemvKernel q4t_kernel_g3(int m, int xm, bool one) { return q4_pick_g3<DT_Q4T>(m, xm, one); }
GemvKernel q4t_kernel_s6(int m, int xm) { return q4_pick_s6<DT_Q4T>(m, xm); }
GemvKernel q4t_kernel_m1(int nk, bool resid, int* ks, size_t* lds) { return q4t_m1_pick(nk, resid, ks, lds); }
GemvKernel q4t_kernel_m1x(int nk, bool resid, int* ks) { return q4t_m1x_pick(nk, resid, ks); }
}  // namespace cmf
