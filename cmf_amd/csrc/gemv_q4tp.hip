// q4tp GEMV kernel instances (k_gemv_q4, gemv_kern.h).
#include "gemv_kern.h"

namespace cmf {
GemvKernel q4tp_kernel(int m, int xm, int ks, int rb) { return q4_pick<DT_Q4TP>(m, xm, ks, rb); }
GemvKernel q4tp_kernel_g3(int m, int xm, bool one) { return q4_pick_g3<DT_Q4TP>(m, xm, one); }
GemvKernel q4tp_kernel_s6(int m, int xm) { return q4_pick_s6<DT_Q4TP>(m, xm); }
}  // namespace cmf
