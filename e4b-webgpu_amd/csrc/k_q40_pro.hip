// k_q40_pro.hip -- q4_0 GEMV variants with the fused residual/norm prologue.
#include "q40_kernel.h"

bool q40k::dispatch_pro(const Cfg& c, const Launch& L, int epi) {
  if (L.pa.part_o) return epi == EPI_F32 && launch_pro_attn(c, L);
  if (L.pa.tail) return epi == EPI_F32 && launch_pro_tail(c, L);
  if (epi == EPI_F32 && L.pa.na == kMaxPartials) return launch_pro<EPI_F32, kMaxPartials>(c, L);
  // the gate/up GeGLU after a two-slice o projection: two partial vectors
  if (epi == EPI_GEGLU && L.pa.na == 2) return launch_pro<EPI_GEGLU, 2>(c, L);
  // other partial-vector inputs: the f32 epilogue with exactly kMaxPartials
  if (L.pa.na > 1) return false;
  if (epi == EPI_F32) return launch_pro<EPI_F32>(c, L);
  if (epi == EPI_GEGLU) return launch_pro<EPI_GEGLU>(c, L);
  if (epi == EPI_GELU_MUL) return launch_pro<EPI_GELU_MUL>(c, L);
  return false;
}
