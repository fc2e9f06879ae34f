// k_ple.hip -- the per-layer-embedding branch of one layer in one launch
// (src/engine.js:282-323: gate GEMV, gelu * per-layer input, projection
// GEMV; kernels/plegatemv.wgsl:20-60 for the gate).
//
// The projection's input has PD = 256 elements = 8 q4_0 blocks, so the
// branch splits by projection block: workgroup (w, q) computes gate rows
// [32w, 32w+32) (after the fused post-FFN residual prologue, which every
// workgroup repeats), keeps the 32 gated values in LDS, and multiplies them
// with block w of the projection rows in quarter q.  Workgroups (w, *) write
// the partial projection part[w][0..H); the consumer (the next layer's qkv
// prologue or the step tail) adds the 8 partials in a fixed order.  Up to
// eight row slices q put the branch on 64 CUs instead of 8 (each CU's share
// of the weight and vector traffic is what bounds this small launch); the
// gate rows are recomputed per slice.  The projection weights are stored
// block-transposed ([block][row]) so that a block-w column is one contiguous
// stream.
#include "../../include/e4b.h"
#include "q40_kernel.h"
#include "step.h"
#include "util.h"
#include "trace.h"

namespace {

constexpr float kTwo24 = 16777216.0f;

// PROK = H / 256: lanes per gate row LPR = H / 32 = 8 PROK, G = 8 / PROK
// groups per wave, R = PROK rows per group, 8 gate rows per wave; Q row
// quarters (blockIdx.y), PR = PROK / Q projection rows per thread.
//
// The leading scalar arguments repeat the pointers the first requests need
// (the prologue's hin, a, w1; the gate planes, the projection's nibbles and
// the per-layer input; the projection's scales, needed last, come from the
// struct after its one wait): the library
// is built with -amdgpu-kernarg-preload-count, so they arrive in SGPRs with
// the wave and no request waits for a kernel-argument load (struct
// arguments are not preloaded); H and the gate's blocks per row follow from
// PROK.
template <int PROK, int Q, int NA>
__global__ __launch_bounds__(256) void k_ple(const float* lhin, const float* la, const float* lw1,
                                             const uint4* lgnib, const uint16_t* lgsc, const uint4* lpnib,
                                             const float* lple, PleLaunch A, ProArgs pa) {
  E4B_TRACE_SCOPE(trace_tag(TR_PLE, 0));
  constexpr int H = 256 * PROK, LPR = H / 32, G = 64 / LPR, R = PROK, PR = PROK / Q;
  pa.hin = lhin;
  pa.a = la;
  pa.w1 = lw1;
  pa.H = H;
  A.gate.nib = lgnib;
  A.gate.sc = lgsc;
  A.gate.nb = H / 32;
  A.proj_nib = lpnib;
  A.ple = lple;
  static_assert(G * R == 8, "8 gate rows per wave");
  static_assert(PR * Q == PROK, "whole projection rows per thread");
  __shared__ __align__(16) uint16_t xs[H];
  __shared__ float red[4];
  __shared__ __align__(16) uint16_t gs[32];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane / LPR, l = lane - g * LPR;
  const int w = blockIdx.x;

  q40k::ProRegs<PROK, 256, NA> pr;
  q40k::pro_issue<PROK, NA, 256, false>(pa, pr);
  // gate rows of this lane group, block l
  const int row0 = 32 * w + 8 * wave + g * R;
  // the per-layer input of the gate row this lane finishes (lanes that
  // finish no row load a valid neighbour and drop it)
  const float ple_v = A.ple[row0 + min(l / (LPR / R), R - 1)];
  uint4 wq[R];
  uint32_t wsc[R], wodd = 0;  // aligned scale pairs (ld_scale_pair) and their half
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const uint32_t e = (uint32_t)(row0 + r) * (uint32_t)A.gate.nb + l;
    wq[r] = ld_nt_u4_off(A.gate.nib, e);
    wsc[r] = ld_scale_pair_off(A.gate.sc, e);
    wodd |= (uint32_t)(e & 1) << r;
  }
  // projection rows o = H/Q q + threadIdx.x + 256 i, block w (block-transposed planes)
  const int o0 = (H / Q) * blockIdx.y;
  uint4 pq[PR];
  uint32_t psc[PR], podd = 0;
#pragma unroll
  for (int i = 0; i < PR; ++i) {
    const uint32_t e = (uint32_t)(w * H + o0) + threadIdx.x + 256 * i;
    pq[i] = ld_nt_u4_off(A.proj_nib, e);
    podd |= (uint32_t)(e & 1) << i;
  }
  // the struct fields read after this point, in one wait (else the
  // prologue's LDS waits wait on them one kernel-argument round trip at a
  // time), then the projection's scales, requested last
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("" ::"s"(A.proj_sc), "s"(A.part), "s"(pa.hout), "s"(pa.hsnap), "s"(pa.scale), "s"(pa.eps));
#pragma unroll
  for (int i = 0; i < PR; ++i) psc[i] = ld_scale_pair_off(A.proj_sc, (uint32_t)(w * H + o0) + threadIdx.x + 256 * i);
  __builtin_amdgcn_sched_barrier(0);  // every load in flight before the prologue waits
  E4B_TRACE_MARK(0);
  q40k::pro_finish<PROK, 256, NA, false>(pa, pr, xs, red);
  E4B_TRACE_MARK(1);

  // gate: 32 columns of x per lane (block l), R rows per group
  {
    uint32_t xp[16];
    const uint4* v = reinterpret_cast<const uint4*>(xs) + (size_t)l * 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint4 t = v[i];
      xp[4 * i + 0] = t.x;
      xp[4 * i + 1] = t.y;
      xp[4 * i + 2] = t.z;
      xp[4 * i + 3] = t.w;
    }
    const float xs8 = -8.f * xsum16(xp);
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float a0 = 0.f, a1 = 0.f;
      q40_dot2(wq[r], xp, a0, a1);
      acc[r] = scale_of(wsc[r], (wodd >> r) & 1) * fmaf(a1, kTwo24 / 16.f, fmaf(a0, kTwo24, xs8));
    }
    const float vrow = reduce_rows<LPR, R>(acc);
    const int r = l / (LPR / R);
    if ((l % (LPR / R)) == 0) {
      const int row = row0 + r;
      gs[row - 32 * w] = f2h(gelu_tanh(vrow) * ple_v);
    }
  }
  lds_sync();
  E4B_TRACE_MARK(2);

  // projection partial: part[w][o] = d_{o,w} * sum_j (n_j - 8) g_j
  {
    uint32_t gp[16];
    const uint4* v = reinterpret_cast<const uint4*>(gs);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint4 t = v[i];
      gp[4 * i + 0] = t.x;
      gp[4 * i + 1] = t.y;
      gp[4 * i + 2] = t.z;
      gp[4 * i + 3] = t.w;
    }
    const float gs8 = -8.f * xsum16(gp);
#pragma unroll
    for (int i = 0; i < PR; ++i) {
      float a0 = 0.f, a1 = 0.f;
      q40_dot2(pq[i], gp, a0, a1);
      A.part[(int64_t)w * H + o0 + threadIdx.x + 256 * i] =
          scale_of(psc[i], (podd >> i) & 1) * fmaf(a1, kTwo24 / 16.f, fmaf(a0, kTwo24, gs8));
    }
  }
}

}  // namespace

#define PLE_LEAD(A, pa) pa.hin, pa.a, pa.w1, A.gate.nib, A.gate.sc, A.proj_nib, A.ple, A, pa
template <int NA>
static void launch_ple_na(const PleLaunch& A, const ProArgs& pa, hipStream_t st) {
  switch (A.H) {
    case 256: hipLaunchKernelGGL((k_ple<1, 1, NA>), dim3(A.PD / 32, 1), dim3(256), 0, st, PLE_LEAD(A, pa)); break;
    case 512: hipLaunchKernelGGL((k_ple<2, 2, NA>), dim3(A.PD / 32, 2), dim3(256), 0, st, PLE_LEAD(A, pa)); break;
    case 1024: hipLaunchKernelGGL((k_ple<4, 4, NA>), dim3(A.PD / 32, 4), dim3(256), 0, st, PLE_LEAD(A, pa)); break;
    case 2048: hipLaunchKernelGGL((k_ple<8, 8, NA>), dim3(A.PD / 32, 8), dim3(256), 0, st, PLE_LEAD(A, pa)); break;
  }
}

int launch_ple(const PleLaunch& A, const ProArgs& pa, hipStream_t st) {
  if (A.PD != 256 || A.gate.rows != A.PD || A.gate.nb * 32 != A.H || pa.H != A.H || !q40_prologue_supported(A.H))
    return e4b_fail(E4B_EINVAL, "PLE branch: needs ple_dim 256 and hidden 256/512/1024/2048 (got %d, %d)", A.PD, A.H);
  if (!pa.a || !pa.w1 || (pa.na > 2))
    return e4b_fail(E4B_EINVAL, "PLE branch: the residual prologue needs a (1 or 2 column slices) and w1");
  if (pa.na == 2)
    launch_ple_na<2>(A, pa, st);
  else
    launch_ple_na<1>(A, pa, st);
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}
