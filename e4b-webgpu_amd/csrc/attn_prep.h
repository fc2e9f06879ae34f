// attn_prep.h -- the attention head prep shared by the decode attention
// kernel and the batched prefill head prep (kernels/headprep.wgsl:19-87).
#pragma once
#include "kernels.h"

// weighted head RMS over 256 dims held 4 per lane, then NeoX-half RoPE:
// dims p < 128 (lanes 0..31) pair with p + 128 (lanes 32..63).
// head prep on inputs that were loaded up front: x (4 dims per lane), the
// norm weights w (use_w) and, when `have_cs`, the (cos, sin) of this lane's
// 4 rotary dims; otherwise the angles are evaluated with sincosf
DEV void prep_head_regs(float (&x)[4], const float (&w)[4], bool use_w, const float2 (&cs)[4], bool have_cs,
                        const float* inv_freq, int angles, float eps, float fpos, bool rotate) {
  const int lane = threadIdx.x & 63;
  const float ss = wave_sum(x[0] * x[0] + x[1] * x[1] + x[2] * x[2] + x[3] * x[3]);
  const float inv = rms_inv(ss, 256, eps);  // head_dim 256
#pragma unroll
  for (int i = 0; i < 4; ++i) x[i] = x[i] * inv * (use_w ? w[i] : 1.f);
  if (!rotate) return;
  const bool hi = lane >= 32;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float a = x[i], b = x[i];
    swapx32(a, b);  // lo lanes: b = partner (dim p + 128); hi lanes: a = partner (dim p)
    const float partner = hi ? a : b;
    const int p = 4 * (lane & 31) + i;
    if (p < angles) {
      float sn, c;
      if (have_cs) {
        c = cs[i].x;
        sn = cs[i].y;
      } else {
        sincosf(fpos * inv_freq[p], &sn, &c);
      }
      x[i] = hi ? (partner * sn + x[i] * c) : (x[i] * c - partner * sn);
    }
  }
}

