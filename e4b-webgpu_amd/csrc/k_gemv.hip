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
constexpr int kQ6Rows = 8;  // lm-head rows per wave tile

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

DEV float gelu_tanh(float g) {
  float t = 0.7978845608028654f * (g + 0.044715f * g * g * g);
  t = fminf(fmaxf(t, -20.f), 20.f);
  return 0.5f * g * (1.f + tanhf(t));
}

// Persistent q4_0 GEMV.  A wave splits into 64/LPR lane groups; a group owns
// R rows ("slots") of a tile and each lane covers blocks jb = l + LPR*k of
// them; the activation slice of those blocks stays in registers for the
// whole kernel while the wave strides over tiles.  blockIdx.y selects one of
// KS column slices (partial outputs).
template <int LPR, int BPL, int R, bool XLO, int EPI>
__global__ __launch_bounds__(256) void k_q40(Q40Mat W, const uint32_t* __restrict__ xh,
                                             const uint32_t* __restrict__ xl, GemvOut o, int64_t ntiles,
                                             int nbk) {
  constexpr int G = 64 / LPR, SPAN = LPR / R;
  static_assert(EPI != EPI_GEGLU || (R % 2 == 0), "GeGLU tiles hold (gate, up) pairs");
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane / LPR, l = lane - g * LPR;
  const int kslice = blockIdx.y, jb0 = kslice * nbk;
  const int nb = W.nb;

  uint32_t xp[BPL][16];
  uint32_t xq[BPL][XLO ? 16 : 1];
  float xs8[BPL];
#pragma unroll
  for (int k = 0; k < BPL; ++k) {
    const int jb = l + LPR * k;
#pragma unroll
    for (int i = 0; i < 16; ++i) xp[k][i] = 0u;
    if constexpr (XLO) {
#pragma unroll
      for (int i = 0; i < 16; ++i) xq[k][i] = 0u;
    }
    xs8[k] = 0.f;
    if (jb < nbk) {
      load_x16(xh, jb0 + jb, xp[k]);
      float xs = xsum16(xp[k]);
      if constexpr (XLO) {
        load_x16(xl, jb0 + jb, xq[k]);
        xs += xsum16(xq[k]);
      }
      xs8[k] = -8.f * xs;
    }
  }

  const int64_t units = (EPI == EPI_GEGLU) ? 2 * o.ff : W.rows;
  for (int64_t tile = (int64_t)blockIdx.x * 4 + wave; tile < ntiles; tile += (int64_t)gridDim.x * 4) {
    const int64_t slot0 = tile * (G * R) + (int64_t)g * R;
    int64_t rowof[R];
    bool ok[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if constexpr (EPI == EPI_GEGLU) {
        const int64_t u = slot0 / 2 + r / 2;
        rowof[r] = (r & 1) ? o.ff + u : u;
        ok[r] = u < o.ff;
      } else {
        rowof[r] = slot0 + r;
        ok[r] = slot0 + r < units;
      }
    }
    // loads always issue (row and block clamped into range); slots past the
    // end are computed on duplicate data and never stored, and blocks past
    // the slice end meet zeroed activations
    uint4 wq[R][BPL];
    uint16_t ws[R][BPL];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t row = ok[r] ? rowof[r] : (W.rows - 1);
      const uint4* nrow = W.nib + row * nb + jb0;
      const uint16_t* srow = W.sc + row * nb + jb0;
#pragma unroll
      for (int k = 0; k < BPL; ++k) {
        const int jb = min(l + LPR * k, nbk - 1);
        wq[r][k] = ld_nt_u4(nrow + jb);
        ws[r][k] = ld_nt_u16(srow + jb);
      }
    }
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      acc[r] = 0.f;
#pragma unroll
      for (int k = 0; k < BPL; ++k) {
        float a = q40_dot(wq[r][k], xp[k], 0.f);
        if constexpr (XLO) a = q40_dot(wq[r][k], xq[k], a);
        acc[r] = fmaf(h2f(ws[r][k]), fmaf(a, kTwo24, xs8[k]), acc[r]);
      }
    }
    float v = reduce_rows<LPR, R>(acc);
    const int r = l / SPAN;  // this lane now holds slot r of the tile
    if constexpr (EPI == EPI_GEGLU) {
      const float up = __shfl_xor(v, SPAN, 64);
      const int64_t u = slot0 / 2 + r / 2;
      if ((l % (2 * SPAN)) == 0 && u < o.ff) o.yh[u] = f2h(gelu_tanh(v) * up);
    } else {
      const int64_t row = slot0 + r;
      if ((l % SPAN) == 0 && row < W.rows) {
        if constexpr (EPI == EPI_F32) o.y[(int64_t)kslice * W.rows + row] = v;
        if constexpr (EPI == EPI_GELU_MUL) o.yh[row] = f2h(gelu_tanh(v) * o.mul[row]);
      }
    }
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

// Block-level argmax partial: reduce the block and store (index, value) to
// part[blockIdx.x] with a plain store.  The fold over blocks runs in
// k_amax_final on the same stream (the kernel boundary makes the partials
// visible); a per-block atomic counter costs ~12-25 ns per block on this part
// because same-address atomics serialise.
DEV void amax_block(float bv, uint32_t bi, uint2* part) {
  __shared__ float sv[4];
  __shared__ uint32_t si[4];
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
    part[blockIdx.x] = make_uint2(i, __float_as_uint(v));
  }
}

__global__ __launch_bounds__(256) void k_amax_final(const uint2* __restrict__ part, int nparts, uint32_t* amax) {
  __shared__ float sv[4];
  __shared__ uint32_t si[4];
  float v = -3.0e38f;
  uint32_t i = 0;
  for (int b = threadIdx.x; b < nparts; b += 256) {
    const uint2 p = part[b];
    amax_take(v, i, __uint_as_float(p.y), p.x);
  }
  amax_wave(v, i);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    sv[wave] = v;
    si[wave] = i;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 4; ++w) amax_take(sv[0], si[0], sv[w], si[w]);
    amax[0] = si[0];
    amax[1] = __float_as_uint(sv[0]);
  }
}

// Q6_K GEMV + softcap + argmax.  Lane <-> 32-element segment (s = lane +
// 64k); a wave owns R rows per tile and strides over tiles; after the
// transposed reduction lane l holds row l/(64/R), so the softcap and the
// argmax update run once per R rows.
template <int BPL, int R>
__global__ __launch_bounds__(256) void k_q6k_gemv_argmax(Q6Mat W, const uint32_t* __restrict__ xh,
                                                         const uint32_t* __restrict__ xl, float softcap,
                                                         float* __restrict__ logits, uint2* part,
                                                         int64_t ntiles) {
  constexpr int SPAN = 64 / R;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nseg = W.nseg, nsb = nseg / 8, ngrp = nseg * 2;
  uint32_t xph[BPL][16], xpl[BPL][16];
  float gs[BPL][2];
#pragma unroll
  for (int k = 0; k < BPL; ++k) {
    const int s = lane + 64 * k;
    gs[k][0] = gs[k][1] = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) xph[k][i] = xpl[k][i] = 0u;  // lanes past the row end contribute 0
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
      gs[k][0] *= -32.f;
      gs[k][1] *= -32.f;
    }
  }
  float bv = -3.0e38f;
  uint32_t bi = 0;
  for (int64_t tile = (int64_t)blockIdx.x * 4 + wave; tile < ntiles; tile += (int64_t)gridDim.x * 4) {
    const int64_t row0 = tile * R;
    const uint4* qa = W.qa + row0 * nseg;
    const uint2* qb = W.qb + row0 * nseg;
    const uint16_t* sc = reinterpret_cast<const uint16_t*>(W.sc + row0 * ngrp);
    const uint16_t* dd = W.d + row0 * nsb;
    uint4 a[R][BPL];
    uint2 b[R][BPL];
    uint16_t s2[R][BPL], dh[R][BPL];
    const int rlast = (int)min((int64_t)R - 1, W.rows - 1 - row0);  // clamp the tail tile
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
      for (int k = 0; k < BPL; ++k) {
        const int s = min(lane + 64 * k, nseg - 1);  // x is zero past the row end
        const uint32_t o = (uint32_t)(min(r, rlast) * nseg + s);
        a[r][k] = ld_nt_u4(qa + o);
        b[r][k] = ld_nt_u2(qb + o);
        s2[r][k] = ld_nt_u16(sc + o);
        dh[r][k] = dd[(uint32_t)(min(r, rlast) * nsb) + (s >> 3)];
      }
    }
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      acc[r] = 0.f;
#pragma unroll
      for (int k = 0; k < BPL; ++k) {
        uint32_t p[8];
        q6_pairs(a[r][k].x, a[r][k].y, b[r][k].x, p);
        float a0 = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          a0 = fdot2u(p[i], xph[k][i], a0);
          a0 = fdot2u(p[i], xpl[k][i], a0);
        }
        q6_pairs(a[r][k].z, a[r][k].w, b[r][k].y, p);
        float a1 = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          a1 = fdot2u(p[i], xph[k][8 + i], a1);
          a1 = fdot2u(p[i], xpl[k][8 + i], a1);
        }
        const float s0 = (float)(int8_t)(s2[r][k] & 0xff), s1 = (float)(int8_t)(s2[r][k] >> 8);
        const float t = s0 * fmaf(a0, kTwo24, gs[k][0]) + s1 * fmaf(a1, kTwo24, gs[k][1]);
        acc[r] = fmaf(h2f(dh[r][k]), t, acc[r]);
      }
    }
    float v = reduce_rows<64, R>(acc);
    const int64_t row = row0 + lane / SPAN;
    if (softcap != 0.f) v = softcap * tanhf(v / softcap);
    if (row < W.rows) {
      if (logits && (lane % SPAN) == 0) logits[row] = v;
      amax_take(bv, bi, v, (uint32_t)row);
    }
  }
  amax_block(bv, bi, part);
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

__global__ __launch_bounds__(256) void k_argmax(const float* __restrict__ x, int64_t n, uint2* part) {
  float bv = -3.0e38f;
  uint32_t bi = 0;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    amax_take(bv, bi, x[i], (uint32_t)i);
  amax_block(bv, bi, part);
}

// ---- q4_0 launch configuration ---------------------------------------------
struct Q40Cfg {
  int lpr, bpl, r;
};

static Q40Cfg pick_q40(int nbk, int64_t units, int epi) {
  Q40Cfg best = {64, 1, 1};
  double best_util = -1.0;
  const int lprs[4] = {64, 32, 16, 8};
  for (int i = 0; i < 4; ++i) {
    const int lpr = lprs[i];
    int bpl = (nbk + lpr - 1) / lpr;
    if (bpl > 8) continue;
    if (bpl == 5) bpl = 6;
    if (bpl == 7) bpl = 8;
    const double util = (double)nbk / (double)(lpr * bpl);
    if (util > best_util + 1e-9) {
      best_util = util;
      best = {lpr, bpl, 1};
    }
  }
  // rows per group: ~8 weight loads in flight per lane, but keep >= 512 workgroups
  const int G = 64 / best.lpr;
  int r = best.bpl == 1 ? 8 : best.bpl == 2 ? 4 : best.bpl <= 4 ? 2 : 1;
  if (r > best.lpr) r = best.lpr;
  const int rmin = (epi == EPI_GEGLU) ? 2 : 1;
  while (r > rmin && (units + 4 * G * r - 1) / (4 * G * r) < 512) r >>= 1;
  if (r < rmin) r = rmin;
  best.r = r;
  return best;
}

template <int LPR, int BPL, int R, bool XLO, int EPI>
static void launch_t(const Q40Mat& W, const uint32_t* xh, const uint32_t* xl, const GemvOut& o, int64_t units,
                     int ks, int nbk, hipStream_t st) {
  constexpr int G = 64 / LPR;
  const int64_t ntiles = (units + G * R - 1) / (G * R);
  int64_t wgs = (ntiles + 3) / 4;
  if (wgs > 2048) wgs = 2048;
  hipLaunchKernelGGL((k_q40<LPR, BPL, R, XLO, EPI>), dim3((unsigned)wgs, (unsigned)ks), dim3(256), 0, st, W, xh, xl, o,
                     ntiles, nbk);
}

template <int LPR, int BPL, bool XLO, int EPI>
static bool launch_r(int r, const Q40Mat& W, const uint32_t* xh, const uint32_t* xl, const GemvOut& o, int64_t units,
                     int ks, int nbk, hipStream_t st) {
  switch (r) {
    case 1:
      if constexpr (EPI != EPI_GEGLU) {
        launch_t<LPR, BPL, 1, XLO, EPI>(W, xh, xl, o, units, ks, nbk, st);
        return true;
      }
      return false;
    case 2: launch_t<LPR, BPL, 2, XLO, EPI>(W, xh, xl, o, units, ks, nbk, st); return true;
    case 4: launch_t<LPR, BPL, 4, XLO, EPI>(W, xh, xl, o, units, ks, nbk, st); return true;
    case 8: launch_t<LPR, BPL, 8, XLO, EPI>(W, xh, xl, o, units, ks, nbk, st); return true;
  }
  return false;
}

template <int LPR, bool XLO, int EPI>
static bool launch_b(const Q40Cfg& c, const Q40Mat& W, const uint32_t* xh, const uint32_t* xl, const GemvOut& o,
                     int64_t units, int ks, int nbk, hipStream_t st) {
  switch (c.bpl) {
    case 1: return launch_r<LPR, 1, XLO, EPI>(c.r, W, xh, xl, o, units, ks, nbk, st);
    case 2: return launch_r<LPR, 2, XLO, EPI>(c.r, W, xh, xl, o, units, ks, nbk, st);
    case 3: return launch_r<LPR, 3, XLO, EPI>(c.r, W, xh, xl, o, units, ks, nbk, st);
    case 4: return launch_r<LPR, 4, XLO, EPI>(c.r, W, xh, xl, o, units, ks, nbk, st);
    case 6: return launch_r<LPR, 6, XLO, EPI>(c.r, W, xh, xl, o, units, ks, nbk, st);
    case 8: return launch_r<LPR, 8, XLO, EPI>(c.r, W, xh, xl, o, units, ks, nbk, st);
  }
  return false;
}

template <bool XLO, int EPI>
static bool launch_l(const Q40Cfg& c, const Q40Mat& W, const uint32_t* xh, const uint32_t* xl, const GemvOut& o,
                     int64_t units, int ks, int nbk, hipStream_t st) {
  switch (c.lpr) {
    case 64: return launch_b<64, XLO, EPI>(c, W, xh, xl, o, units, ks, nbk, st);
    case 32: return launch_b<32, XLO, EPI>(c, W, xh, xl, o, units, ks, nbk, st);
    case 16: return launch_b<16, XLO, EPI>(c, W, xh, xl, o, units, ks, nbk, st);
    case 8: return launch_b<8, XLO, EPI>(c, W, xh, xl, o, units, ks, nbk, st);
  }
  return false;
}

}  // namespace

int launch_q40(const Q40Mat& W, const uint32_t* xh, const uint32_t* xl, int epi, const GemvOut& o, int ks,
               hipStream_t st) {
  if (ks < 1 || W.nb % ks) return e4b_fail(E4B_EINVAL, "q4_0 GEMV: %d blocks per row not divisible by ks=%d", W.nb, ks);
  if (ks > 1 && epi != EPI_F32) return e4b_fail(E4B_EINVAL, "q4_0 GEMV: column split needs the f32 epilogue");
  const int nbk = W.nb / ks;
  if (nbk > 64 * 8)
    return e4b_fail(E4B_EINVAL, "q4_0 GEMV: %d blocks per slice exceeds the 512-block (16384-column) maximum", nbk);
  const int64_t units = (epi == EPI_GEGLU) ? 2 * o.ff : W.rows;
  const Q40Cfg c = pick_q40(nbk, units, epi);
  bool ok = false;
  switch (epi) {
    case EPI_F32:
      ok = xl ? launch_l<true, EPI_F32>(c, W, xh, xl, o, units, ks, nbk, st)
              : launch_l<false, EPI_F32>(c, W, xh, xl, o, units, ks, nbk, st);
      break;
    case EPI_GEGLU: ok = !xl && launch_l<false, EPI_GEGLU>(c, W, xh, xl, o, units, ks, nbk, st); break;
    case EPI_GELU_MUL: ok = !xl && launch_l<false, EPI_GELU_MUL>(c, W, xh, xl, o, units, ks, nbk, st); break;
  }
  if (!ok) return e4b_fail(E4B_EINVAL, "q4_0 GEMV: no kernel for epi=%d lpr=%d bpl=%d r=%d", epi, c.lpr, c.bpl, c.r);
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}

int launch_q40_gemv(const Q40Mat& W, const uint32_t* xh, const uint32_t* xl, float* y, hipStream_t st) {
  GemvOut o = {y, nullptr, nullptr, 0};
  return launch_q40(W, xh, xl, EPI_F32, o, 1, st);
}

int launch_split_f32(const float* x, int64_t n, uint16_t* hi, uint16_t* lo, hipStream_t st) {
  hipLaunchKernelGGL(k_split_f32, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, n, hi, lo);
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}

int q6k_gemv_grid(int64_t rows) {
  const int64_t ntiles = (rows + kQ6Rows - 1) / kQ6Rows;
  const int64_t wgs = (ntiles + 3) / 4;
  return (int)(wgs < 2048 ? wgs : 2048);
}

int launch_q6k_gemv_argmax(const Q6Mat& W, const uint32_t* xh, const uint32_t* xl, float softcap, float* logits,
                           uint32_t* amax, uint2* part, hipStream_t st) {
  constexpr int R = kQ6Rows;
  const int64_t ntiles = (W.rows + R - 1) / R;
  const int64_t wgs = q6k_gemv_grid(W.rows);
  if (W.nseg <= 64)
    hipLaunchKernelGGL((k_q6k_gemv_argmax<1, R>), dim3((unsigned)wgs), dim3(256), 0, st, W, xh, xl, softcap, logits,
                       part, ntiles);
  else if (W.nseg <= 128)
    hipLaunchKernelGGL((k_q6k_gemv_argmax<2, R>), dim3((unsigned)wgs), dim3(256), 0, st, W, xh, xl, softcap, logits,
                       part, ntiles);
  else
    return e4b_fail(E4B_EINVAL, "Q6_K GEMV: %d columns exceeds the 4096-column maximum", W.nseg * 32);
  if (amax) hipLaunchKernelGGL(k_amax_final, dim3(1), dim3(256), 0, st, part, (int)wgs, amax);
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}

int launch_q6k_row(const Q6Mat& W, int64_t row, const uint32_t* row_dev, float mult, float* out, hipStream_t st) {
  hipLaunchKernelGGL(k_q6k_row, dim3((unsigned)((W.nseg + 255) / 256)), dim3(256), 0, st, W, row, row_dev, mult, out);
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}

int launch_argmax(const float* x, int64_t n, uint32_t* amax, uint2* part, hipStream_t st) {
  const int64_t want = (n + 255) / 256;
  const unsigned grid = (unsigned)(want < 1024 ? (want > 0 ? want : 1) : 1024);
  hipLaunchKernelGGL(k_argmax, dim3(grid), dim3(256), 0, st, x, n, part);
  hipLaunchKernelGGL(k_amax_final, dim3(1), dim3(256), 0, st, part, (int)grid, amax);
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}
