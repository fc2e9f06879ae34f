// k_q40_f32hl.hip -- q4_0 GEMV variants: f32 input as a hi/lo f16 pair
// (hi + lo within max(2^-22 |x|, 2^-25) of x).
#include "q40_kernel.h"

bool q40k::dispatch_f32_hl(const Cfg& c, const Launch& L) { return launch_plain<true, EPI_F32>(c, L); }
