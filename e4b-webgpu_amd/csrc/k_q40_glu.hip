// k_q40_glu.hip -- q4_0 GEMV variants with a GELU epilogue (GeGLU over a
// gate|up matrix, or gelu(dot) * mul).
#include "q40_kernel.h"

bool q40k::dispatch_glu(const Cfg& c, const Launch& L, int epi) {
  if (epi == EPI_GEGLU) return launch_plain<false, EPI_GEGLU>(c, L);
  if (epi == EPI_GELU_MUL) return launch_plain<false, EPI_GELU_MUL>(c, L);
  return false;
}
