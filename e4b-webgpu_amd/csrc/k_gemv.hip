// k_gemv.hip -- q4_0 and Q6_K dequant-GEMV kernels for gfx950 (wave64).
//
// Design (HBM-bound, batch 1):
//  * every lane streams 16 B weight blocks with non-temporal dwordx4 loads;
//    all of a lane's loads for one pass are issued before any math, so each
//    lane keeps R*BPL loads in flight;
//  * dequant happens in registers: a repacked nibble pair is an f16
//    subnormal pair and one v_dot2_f32_f16 multiplies it with the natural
//    (x[2j], x[2j+1]) f16 pair, accumulating in f32 (layout in common.h);
//  * a wave is split into 64/LPR lane groups, one row per group, so short
//    rows (e.g. 22 or 8 blocks) do not idle most of the wave;
//  * the per-row partials are reduced with a butterfly inside the group.
// f32 activations are carried as an exact hi/lo f16 split (x = hi + lo), so
// the f32 path is as accurate as an f32 dot product.
#include "../../include/e4b.h"
#include "kernels.h"
#include "util.h"

namespace {

constexpr float kTwo24 = 16777216.0f;

DEV void load_x16(const uint32_t* __restrict__ x, int jb, uint32_t* xp) {
  const uint4* v = reinterpret_cast<const uint4*>(x) + (size_t)jb * 4;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint4 t = v[i];
    xp[4 * i + 0] = t.x;
    xp[4 * i + 1] = t.y;
    xp[4 * i + 2] = t.z;
    xp[4 * i + 3] = t.w;
  }
}

// y[row] = sum_b d(row,b) * sum_i (n_i - 8) x_i, one group of LPR lanes per row,
// R rows per group, BPL blocks per lane and row (jb = l + LPR*k).
template <int LPR, int BPL, int R, bool XLO>
__global__ __launch_bounds__(256) void k_q40_gemv(Q40Mat W, const uint32_t* __restrict__ xh,
                                                  const uint32_t* __restrict__ xl, float* __restrict__ y) {
  constexpr int G = 64 / LPR;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane / LPR, l = lane - g * LPR;
  const int64_t row0 = ((int64_t)blockIdx.x * 4 + wave) * (G * R) + (int64_t)g * R;
  const int nb = W.nb;

  uint4 wq[R][BPL];
  uint16_t ws[R][BPL];
#pragma unroll
  for (int r = 0; r < R; ++r) {
#pragma unroll
    for (int k = 0; k < BPL; ++k) {
      const int64_t row = row0 + r;
      const int jb = l + LPR * k;
      if (row < W.rows && jb < nb) {
        wq[r][k] = ld_nt_u4(W.nib + row * nb + jb);
        ws[r][k] = ld_nt_u16(W.sc + row * nb + jb);
      } else {
        wq[r][k] = make_uint4(0u, 0u, 0u, 0u);
        ws[r][k] = 0;
      }
    }
  }

  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;
#pragma unroll
  for (int k = 0; k < BPL; ++k) {
    const int jb = l + LPR * k;
    if (jb < nb) {
      uint32_t xp[16];
      load_x16(xh, jb, xp);
      float xs = xsum16(xp);
      uint32_t xq[XLO ? 16 : 1];
      if constexpr (XLO) {
        load_x16(xl, jb, xq);
        xs = xs + xsum16(xq);
      }
      const float xs8 = -8.f * xs;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float a = q40_dot(wq[r][k], xp, 0.f);
        if constexpr (XLO) a = q40_dot(wq[r][k], xq, a);
        acc[r] = fmaf(h2f(ws[r][k]), fmaf(a, kTwo24, xs8), acc[r]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const float v = group_sum(acc[r], LPR);
    if (l == 0 && row0 + r < W.rows) y[row0 + r] = v;
  }
}

__global__ __launch_bounds__(256) void k_split_f32(const float* __restrict__ x, int64_t n, uint16_t* __restrict__ hi,
                                                   uint16_t* __restrict__ lo) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) {
    const float v = x[i];
    const _Float16 h = (_Float16)v;
    hi[i] = __builtin_bit_cast(uint16_t, h);
    lo[i] = __builtin_bit_cast(uint16_t, (_Float16)(v - (float)h));
  }
}

// ---- argmax helpers (kernels/argmax2.wgsl semantics: lowest index among the
// maxima, NaN never taken, empty -> (0, -3e38)) --------------------------------
DEV void amax_take(float& bv, uint32_t& bi, float v, uint32_t i) {
  if (v > bv || (v == bv && i < bi)) {
    bv = v;
    bi = i;
  }
}

DEV void amax_wave(float& bv, uint32_t& bi) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(bv, off, 64);
    const uint32_t oi = __shfl_xor(bi, off, 64);
    amax_take(bv, bi, ov, oi);
  }
}

// Block reduce, publish the block's partial, and let the last block to finish
// fold all partials into amax.  The counter is returned to zero by that block.
DEV void amax_finish(float bv, uint32_t bi, uint2* part, uint32_t* counter, uint32_t* amax) {
  __shared__ float sv[4];
  __shared__ uint32_t si[4];
  __shared__ int is_last;
  amax_wave(bv, bi);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    sv[wave] = bv;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float v = sv[0];
    uint32_t i = si[0];
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w) amax_take(v, i, sv[w], si[w]);
    __hip_atomic_store(&part[blockIdx.x].x, i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&part[blockIdx.x].y, __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t prev = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    is_last = (prev == gridDim.x - 1);
  }
  __syncthreads();
  if (!is_last) return;
  float v = -3.0e38f;
  uint32_t i = 0;
  for (uint32_t b = threadIdx.x; b < gridDim.x; b += blockDim.x) {
    const uint32_t pi = __hip_atomic_load(&part[b].x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t pv = __hip_atomic_load(&part[b].y, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    amax_take(v, i, __uint_as_float(pv), pi);
  }
  amax_wave(v, i);
  __syncthreads();
  if (lane == 0) {
    sv[wave] = v;
    si[wave] = i;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w) amax_take(sv[0], si[0], sv[w], si[w]);
    amax[0] = si[0];
    amax[1] = __float_as_uint(sv[0]);
    __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Q6_K GEMV + softcap + argmax.  Lane <-> 32-element segment (s = lane + 64k),
// R rows per wave per tile, tiles strided over the grid.
template <int BPL, int R>
__global__ __launch_bounds__(256) void k_q6k_gemv_argmax(Q6Mat W, const uint32_t* __restrict__ xh,
                                                         const uint32_t* __restrict__ xl, float softcap,
                                                         float* __restrict__ logits, uint2* part,
                                                         uint32_t* counter, uint32_t* amax, int64_t ntiles) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nseg = W.nseg, nsb = nseg / 8, ngrp = nseg * 2;
  uint32_t xph[BPL][16], xpl[BPL][16];
  float gs[BPL][2];
#pragma unroll
  for (int k = 0; k < BPL; ++k) {
    const int s = lane + 64 * k;
    gs[k][0] = gs[k][1] = 0.f;
    if (s < nseg) {
      load_x16(xh, s, xph[k]);
      load_x16(xl, s, xpl[k]);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        gs[k][0] = fdot2u(xph[k][i], 0x3C003C00u, gs[k][0]);
        gs[k][0] = fdot2u(xpl[k][i], 0x3C003C00u, gs[k][0]);
        gs[k][1] = fdot2u(xph[k][8 + i], 0x3C003C00u, gs[k][1]);
        gs[k][1] = fdot2u(xpl[k][8 + i], 0x3C003C00u, gs[k][1]);
      }
    }
  }
  float bv = -3.0e38f;
  uint32_t bi = 0;
  for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    const int64_t row0 = (tile * 4 + wave) * R;
    uint4 qa[R][BPL];
    uint2 qb[R][BPL];
    uint16_t sc2[R][BPL], dh[R][BPL];
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
      for (int k = 0; k < BPL; ++k) {
        const int64_t row = row0 + r;
        const int s = lane + 64 * k;
        if (row < W.rows && s < nseg) {
          qa[r][k] = ld_nt_u4(W.qa + row * nseg + s);
          qb[r][k] = ld_nt_u2(W.qb + row * nseg + s);
          sc2[r][k] = ld_nt_u16(reinterpret_cast<const uint16_t*>(W.sc + row * ngrp) + s);
          dh[r][k] = W.d[row * nsb + (s >> 3)];
        } else {
          qa[r][k] = make_uint4(0u, 0u, 0u, 0u);
          qb[r][k] = make_uint2(0u, 0u);
          sc2[r][k] = 0;
          dh[r][k] = 0;
        }
      }
    }
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      acc[r] = 0.f;
#pragma unroll
      for (int k = 0; k < BPL; ++k) {
        uint32_t p[8];
        q6_pairs(qa[r][k].x, qa[r][k].y, qb[r][k].x, p);
        float a0 = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          a0 = fdot2u(p[i], xph[k][i], a0);
          a0 = fdot2u(p[i], xpl[k][i], a0);
        }
        q6_pairs(qa[r][k].z, qa[r][k].w, qb[r][k].y, p);
        float a1 = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          a1 = fdot2u(p[i], xph[k][8 + i], a1);
          a1 = fdot2u(p[i], xpl[k][8 + i], a1);
        }
        const float s0 = (float)(int8_t)(sc2[r][k] & 0xff), s1 = (float)(int8_t)(sc2[r][k] >> 8);
        const float t = s0 * fmaf(a0, kTwo24, -32.f * gs[k][0]) + s1 * fmaf(a1, kTwo24, -32.f * gs[k][1]);
        acc[r] = fmaf(h2f(dh[r][k]), t, acc[r]);
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t row = row0 + r;
      float v = group_sum(acc[r], 64);
      if (softcap != 0.f) v = softcap * tanhf(v / softcap);
      if (row < W.rows) {
        if (logits && lane == r) logits[row] = v;
        amax_take(bv, bi, v, (uint32_t)row);
      }
    }
  }
  amax_finish(bv, bi, part, counter, amax);
}

// one Q6_K row * mult -> f32 (kernels/q6k.wgsl:37-73); thread per segment
__global__ __launch_bounds__(256) void k_q6k_row(Q6Mat W, int64_t row, const uint32_t* __restrict__ row_dev,
                                                 float mult, float* __restrict__ out) {
  const int s = blockIdx.x * 256 + threadIdx.x;
  if (s >= W.nseg) return;
  const int64_t r = row_dev ? (int64_t)row_dev[0] : row;
  if (r < 0 || r >= W.rows) return;
  const uint4 a = W.qa[r * W.nseg + s];
  const uint2 b = W.qb[r * W.nseg + s];
  const float d = h2f(W.d[r * (W.nseg / 8) + (s >> 3)]);
  const int8_t* sc = W.sc + r * (W.nseg * 2) + 2 * s;
  uint32_t p[8];
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    q6_pairs(g ? a.z : a.x, g ? a.w : a.y, g ? b.y : b.x, p);
    const float ds = d * (float)sc[g];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      out[32 * s + 16 * g + 2 * i] = ds * (float)((int)(p[i] & 0x3f) - 32) * mult;
      out[32 * s + 16 * g + 2 * i + 1] = ds * (float)((int)((p[i] >> 16) & 0x3f) - 32) * mult;
    }
  }
}

__global__ __launch_bounds__(256) void k_argmax(const float* __restrict__ x, int64_t n, uint2* part,
                                                uint32_t* counter, uint32_t* amax) {
  float bv = -3.0e38f;
  uint32_t bi = 0;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    amax_take(bv, bi, x[i], (uint32_t)i);
  amax_finish(bv, bi, part, counter, amax);
}

// ---- q4_0 launch configuration ---------------------------------------------
struct Q40Cfg {
  int lpr, bpl, r;
};

static Q40Cfg pick_q40(int nb, int64_t rows) {
  Q40Cfg best = {64, 1, 1};
  double best_util = -1.0;
  const int lprs[4] = {64, 32, 16, 8};
  for (int i = 0; i < 4; ++i) {
    const int lpr = lprs[i];
    int bpl = (nb + lpr - 1) / lpr;
    if (bpl > 8) continue;
    if (bpl == 5) bpl = 6;
    if (bpl == 7) bpl = 8;
    const double util = (double)nb / (double)(lpr * bpl);
    if (util > best_util + 1e-9) {
      best_util = util;
      best = {lpr, bpl, 1};
    }
  }
  if (best_util < 0) best = {64, 8, 1};  // caller loops over column slices
  // rows per group: aim for ~4 loads in flight per lane while keeping >= 512 blocks
  const int G = 64 / best.lpr;
  int r = best.bpl >= 4 ? 1 : (best.bpl >= 2 ? 2 : 4);
  while (r > 1 && (rows + 4 * G * r - 1) / (4 * G * r) < 512) r >>= 1;
  best.r = r;
  return best;
}

template <int LPR, int BPL, int R, bool XLO>
static void launch_q40_t(const Q40Mat& W, const uint32_t* xh, const uint32_t* xl, float* y, hipStream_t st) {
  constexpr int G = 64 / LPR;
  const int64_t per = 4 * G * R;
  const unsigned grid = (unsigned)((W.rows + per - 1) / per);
  hipLaunchKernelGGL((k_q40_gemv<LPR, BPL, R, XLO>), dim3(grid), dim3(256), 0, st, W, xh, xl, y);
}

template <int LPR, int BPL, bool XLO>
static bool launch_q40_r(int r, const Q40Mat& W, const uint32_t* xh, const uint32_t* xl, float* y, hipStream_t st) {
  switch (r) {
    case 1: launch_q40_t<LPR, BPL, 1, XLO>(W, xh, xl, y, st); return true;
    case 2: launch_q40_t<LPR, BPL, 2, XLO>(W, xh, xl, y, st); return true;
    case 4: launch_q40_t<LPR, BPL, 4, XLO>(W, xh, xl, y, st); return true;
  }
  return false;
}

template <int LPR, bool XLO>
static bool launch_q40_b(int bpl, int r, const Q40Mat& W, const uint32_t* xh, const uint32_t* xl, float* y,
                         hipStream_t st) {
  switch (bpl) {
    case 1: return launch_q40_r<LPR, 1, XLO>(r, W, xh, xl, y, st);
    case 2: return launch_q40_r<LPR, 2, XLO>(r, W, xh, xl, y, st);
    case 3: return launch_q40_r<LPR, 3, XLO>(r, W, xh, xl, y, st);
    case 4: return launch_q40_r<LPR, 4, XLO>(r, W, xh, xl, y, st);
    case 6: return launch_q40_r<LPR, 6, XLO>(r, W, xh, xl, y, st);
    case 8: return launch_q40_r<LPR, 8, XLO>(r, W, xh, xl, y, st);
  }
  return false;
}

template <bool XLO>
static bool launch_q40_l(const Q40Cfg& c, const Q40Mat& W, const uint32_t* xh, const uint32_t* xl, float* y,
                         hipStream_t st) {
  switch (c.lpr) {
    case 64: return launch_q40_b<64, XLO>(c.bpl, c.r, W, xh, xl, y, st);
    case 32: return launch_q40_b<32, XLO>(c.bpl, c.r, W, xh, xl, y, st);
    case 16: return launch_q40_b<16, XLO>(c.bpl, c.r, W, xh, xl, y, st);
    case 8: return launch_q40_b<8, XLO>(c.bpl, c.r, W, xh, xl, y, st);
  }
  return false;
}

}  // namespace

int launch_q40_gemv(const Q40Mat& W, const uint32_t* xh, const uint32_t* xl, float* y, hipStream_t st) {
  if (W.nb > 64 * 8)
    return e4b_fail(E4B_EINVAL, "q4_0 GEMV: %d blocks per row exceeds the 512-block (16384-column) maximum", W.nb);
  const Q40Cfg c = pick_q40(W.nb, W.rows);
  const bool ok = xl ? launch_q40_l<true>(c, W, xh, xl, y, st) : launch_q40_l<false>(c, W, xh, xl, y, st);
  if (!ok) return e4b_fail(E4B_EINVAL, "q4_0 GEMV: no kernel for lpr=%d bpl=%d r=%d", c.lpr, c.bpl, c.r);
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}

int launch_split_f32(const float* x, int64_t n, uint16_t* hi, uint16_t* lo, hipStream_t st) {
  hipLaunchKernelGGL(k_split_f32, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, n, hi, lo);
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}

int launch_q6k_gemv_argmax(const Q6Mat& W, const uint32_t* xh, const uint32_t* xl, float softcap, float* logits,
                           uint32_t* amax, uint2* part, uint32_t* counter, hipStream_t st) {
  constexpr int R = 8;
  const int64_t ntiles = (W.rows + 4 * R - 1) / (4 * R);
  const unsigned grid = (unsigned)(ntiles < 2048 ? ntiles : 2048);
  if (W.nseg <= 64)
    hipLaunchKernelGGL((k_q6k_gemv_argmax<1, R>), dim3(grid), dim3(256), 0, st, W, xh, xl, softcap, logits, part,
                       counter, amax, ntiles);
  else if (W.nseg <= 128)
    hipLaunchKernelGGL((k_q6k_gemv_argmax<2, R>), dim3(grid), dim3(256), 0, st, W, xh, xl, softcap, logits, part,
                       counter, amax, ntiles);
  else
    return e4b_fail(E4B_EINVAL, "Q6_K GEMV: %d columns exceeds the 4096-column maximum", W.nseg * 32);
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}

int launch_q6k_row(const Q6Mat& W, int64_t row, const uint32_t* row_dev, float mult, float* out, hipStream_t st) {
  hipLaunchKernelGGL(k_q6k_row, dim3((unsigned)((W.nseg + 255) / 256)), dim3(256), 0, st, W, row, row_dev, mult, out);
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}

int launch_argmax(const float* x, int64_t n, uint32_t* amax, uint2* part, uint32_t* counter, hipStream_t st) {
  const int64_t want = (n + 255) / 256;
  const unsigned grid = (unsigned)(want < 1024 ? (want > 0 ? want : 1) : 1024);
  hipLaunchKernelGGL(k_argmax, dim3(grid), dim3(256), 0, st, x, n, part, counter, amax);
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}
