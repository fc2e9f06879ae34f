// k_q40_f32.hip -- q4_0 GEMV variants: f16 input, f32 output.
#include "q40_kernel.h"

bool q40k::dispatch_f32(const Cfg& c, const Launch& L) { return launch_plain<false, EPI_F32>(c, L); }
