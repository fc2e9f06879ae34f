// k_q40_kw4.hip -- q4_0 GEMV variants for long rows (>= 8192 columns): the
// four waves of a workgroup split the columns and reduce through LDS, so a
// single launch writes complete outputs.
#include "q40_kernel.h"

namespace q40k {
template <bool XLO, int EPI>
static bool kw4(const Cfg& c, const Launch& L) {
  if (c.lpr != 64) return false;
  return launch_b<64, 4, XLO, EPI>(c, L);
}
}  // namespace q40k

bool q40k::dispatch_kw4(const Cfg& c, const Launch& L, int epi) {
  if (epi == EPI_F32) return L.xl ? kw4<true, EPI_F32>(c, L) : kw4<false, EPI_F32>(c, L);
  if (epi == EPI_GEGLU) return kw4<false, EPI_GEGLU>(c, L);
  if (epi == EPI_GELU_MUL) return kw4<false, EPI_GELU_MUL>(c, L);
  return false;
}
