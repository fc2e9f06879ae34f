// q40_kernel.h -- the q4_0 dequant-GEMV kernel template (included by the
// translation units that instantiate it).
//
// Design (HBM-bound, batch 1):
//  * every lane streams 16 B weight blocks with non-temporal dwordx4 loads;
//    all loads of a tile are issued before any math;
//  * dequant in registers: a repacked nibble pair is an f16 subnormal pair, so
//    one v_dot2_f32_f16 against the natural (x[2j], x[2j+1]) pair gives
//    2^-24 (n0 x0 + n1 x1) exactly, accumulated in f32 (layout in common.h);
//  * a wave splits into 64/LPR lane groups, one row per group, so short rows
//    (8 or 22 blocks) do not idle most of the wave;
//  * KW = 4 splits the columns over the four waves of a workgroup (long rows,
//    e.g. the 16384-column down projection) and reduces through LDS;
//  * PROK > 0 computes the input vector in a fused residual/norm prologue
//    (H = 256 * PROK) whose loads are issued before the first tile's weight
//    loads, so both latencies overlap (vmcnt drains in issue order).
#pragma once
#include "kernels.h"

namespace q40k {

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

// registers of the prologue's inputs (element i = threadIdx.x + 256 k)
template <int PROK>
struct ProRegs {
  float h[PROK > 0 ? PROK : 1], a[PROK > 0 ? PROK : 1], w1[PROK > 0 ? PROK : 1], w2[PROK > 0 ? PROK : 1];
};

template <int PROK>
DEV void pro_issue(const ProArgs& p, ProRegs<PROK>& r) {
#pragma unroll
  for (int k = 0; k < PROK; ++k) {
    const int i = threadIdx.x + 256 * k;
    r.h[k] = p.hin[i];
    r.a[k] = p.a ? p.a[i] : 0.f;
    r.w1[k] = p.a ? p.w1[i] : 0.f;
    r.w2[k] = p.w2 ? p.w2[i] : 1.f;
  }
}

// h = (hin + rms(a) * w1) * scale; x = w2 ? f16(rms(h) * w2) : f16(h)
// (kernels/rmsacc3.wgsl:36-53, kernels/a4btail.wgsl:54-71,
// kernels/rmsacc.wgsl:10-26 folded into the consumer GEMV)
template <int PROK>
DEV void pro_finish(const ProArgs& p, ProRegs<PROK>& r, uint16_t* xs, float* red) {
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < PROK; ++k) ss = fmaf(r.a[k], r.a[k], ss);
  const float inv1 = p.a ? rms_inv(block_sum(ss, red), p.H, p.eps) : 0.f;
  float s2 = 0.f;
#pragma unroll
  for (int k = 0; k < PROK; ++k) {
    r.h[k] = (r.h[k] + r.a[k] * inv1 * r.w1[k]) * p.scale;
    s2 = fmaf(r.h[k], r.h[k], s2);
  }
  const float inv2 = p.w2 ? rms_inv(block_sum(s2, red), p.H, p.eps) : 1.f;
  const bool writer = p.hout && blockIdx.x == 0 && blockIdx.y == 0;
#pragma unroll
  for (int k = 0; k < PROK; ++k) {
    const int i = threadIdx.x + 256 * k;
    xs[i] = f2h(p.w2 ? r.h[k] * inv2 * r.w2[k] : r.h[k]);
    if (writer) p.hout[i] = r.h[k];
  }
  __syncthreads();
}

// A wave splits into G = 64/LPR lane groups; with KW = 1 a group owns R rows
// ("slots") of a wave tile, with KW = 4 the four waves share the tile's rows
// and each covers a quarter of the columns.  Lane l of a group covers blocks
// jb = l + LPR*k (k < BPL) of its column range; its activation slice stays in
// registers while the wave strides over tiles.  blockIdx.y selects one of KS
// column slices (partial outputs, EPI_F32 only).
template <int LPR, int BPL, int R, int KW, bool XLO, int EPI, int PROK>
__global__ __launch_bounds__(256) void k_q40(Q40Mat W, const uint32_t* __restrict__ xh,
                                             const uint32_t* __restrict__ xl, GemvOut o, int64_t ntiles,
                                             int nbk, ProArgs pa) {
  constexpr int G = 64 / LPR, SPAN = LPR / R, SLOTS = G * R;
  constexpr int WPT = (KW == 1) ? 4 : 1;  // wave tiles per workgroup step
  static_assert(KW == 1 || KW == 4, "KW is 1 or 4");
  static_assert(EPI != EPI_GEGLU || (R % 2 == 0), "GeGLU tiles hold (gate, up) pairs");
  static_assert(!(PROK && XLO), "the prologue produces f16 input");
  __shared__ __align__(16) uint16_t xs_lds[PROK ? 256 * PROK : 8];
  __shared__ float red[4];
  __shared__ float part[KW == 4 ? 4 * SLOTS : 1];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane / LPR, l = lane - g * LPR;
  const int kslice = blockIdx.y;
  const int nbw = nbk / KW;                               // blocks per wave
  const int jb0 = kslice * nbk + (KW == 4 ? wave * nbw : 0);
  const int nb = W.nb;
  const int64_t units = (EPI == EPI_GEGLU) ? 2 * o.ff : W.rows;

  ProRegs<PROK> pr;
  if constexpr (PROK > 0) pro_issue<PROK>(pa, pr);

  // two register buffers of weight tiles: the loads of tile t + 2*tstep are
  // issued as soon as tile t is consumed, so a wave always has one tile in
  // flight while it computes the other.  Loads always issue (row and block
  // clamped into range); slots past the end are computed on duplicate data
  // and never stored, and blocks past the range end meet zeroed activations.
  uint4 wq0[R][BPL], wq1[R][BPL];
  uint16_t ws0[R][BPL], ws1[R][BPL];
  auto load_tile = [&](int64_t tile, uint4 (&wq)[R][BPL], uint16_t (&ws)[R][BPL]) {
    const int64_t slot0 = tile * SLOTS + (int64_t)g * R;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      int64_t row;
      if constexpr (EPI == EPI_GEGLU) {
        const int64_t u = min(slot0 / 2 + r / 2, o.ff - 1);
        row = (r & 1) ? o.ff + u : u;
      } else {
        row = min(slot0 + r, units - 1);
      }
      const uint4* nrow = W.nib + row * nb + jb0;
      const uint16_t* srow = W.sc + row * nb + jb0;
#pragma unroll
      for (int k = 0; k < BPL; ++k) {
        const int jb = min(l + LPR * k, nbw - 1);
        wq[r][k] = ld_nt_u4(nrow + jb);
        ws[r][k] = ld_nt_u16(srow + jb);
      }
    }
  };

  const int64_t tile0 = (KW == 1) ? (int64_t)blockIdx.x * 4 + wave : (int64_t)blockIdx.x;
  const int64_t tstep = (int64_t)gridDim.x * WPT;
  if (tile0 < ntiles) load_tile(tile0, wq0, ws0);
  if (tile0 + tstep < ntiles) load_tile(tile0 + tstep, wq1, ws1);

  uint32_t xp[BPL][16];
  uint32_t xq[BPL][XLO ? 16 : 1];
  float xs8[BPL];
  if constexpr (PROK > 0) pro_finish<PROK>(pa, pr, xs_lds, red);
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
    if (jb < nbw) {
      if constexpr (PROK > 0) {
        const uint4* v = reinterpret_cast<const uint4*>(xs_lds) + (size_t)(jb0 + jb) * 4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint4 t = v[i];
          xp[k][4 * i + 0] = t.x;
          xp[k][4 * i + 1] = t.y;
          xp[k][4 * i + 2] = t.z;
          xp[k][4 * i + 3] = t.w;
        }
      } else {
        load_x16(xh, jb0 + jb, xp[k]);
      }
      float xs = xsum16(xp[k]);
      if constexpr (XLO) {
        load_x16(xl, jb0 + jb, xq[k]);
        xs += xsum16(xq[k]);
      }
      xs8[k] = -8.f * xs;
    }
  }

  // dot products, reduction and epilogue of one tile
  auto finish_tile = [&](int64_t tile, const uint4 (&wq)[R][BPL], const uint16_t (&ws)[R][BPL]) {
    const int64_t slot0 = tile * SLOTS + (int64_t)g * R;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      acc[r] = 0.f;
#pragma unroll
      for (int k = 0; k < BPL; ++k) {
        float a0 = 0.f, a1 = 0.f;
        q40_dot2(wq[r][k], xp[k], a0, a1);
        if constexpr (XLO) q40_dot2(wq[r][k], xq[k], a0, a1);
        acc[r] = fmaf(h2f(ws[r][k]), fmaf(a1, kTwo24 / 16.f, fmaf(a0, kTwo24, xs8[k])), acc[r]);
      }
    }
    float v = reduce_rows<LPR, R>(acc);
    const int r = l / SPAN;  // this lane now holds slot r of the group
    if constexpr (KW == 4) {
      // fold the four column quarters through LDS; wave 0 finishes
      if ((l % SPAN) == 0) part[wave * SLOTS + g * R + r] = v;
      __syncthreads();
      if (wave == 0) {
        const int sl = g * R + r;
        v = (part[sl] + part[SLOTS + sl]) + (part[2 * SLOTS + sl] + part[3 * SLOTS + sl]);
      }
      __syncthreads();
      if (wave != 0) return;
    }
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
  };

  // the loop body handles two tiles so that each register buffer keeps a
  // compile-time name (a runtime buffer index would spill to scratch)
  for (int64_t tile = tile0; tile < ntiles; tile += 2 * tstep) {
    finish_tile(tile, wq0, ws0);
    if (tile + 2 * tstep < ntiles) load_tile(tile + 2 * tstep, wq0, ws0);
    if (tile + tstep < ntiles) {
      finish_tile(tile + tstep, wq1, ws1);
      if (tile + 3 * tstep < ntiles) load_tile(tile + 3 * tstep, wq1, ws1);
    }
  }
}

// ---- launch configuration -----------------------------------------------------
struct Cfg {
  int lpr, bpl, r, kw;
};

// lanes per row and blocks per lane that maximise lane utilisation for nbw
// blocks per wave (ties keep the wider group)
inline void pick_lanes(int nbw, int* lpr_out, int* bpl_out, bool lpr64_only) {
  int lpr_best = 64, bpl_best = (nbw + 63) / 64;
  double best_util = -1.0;
  const int lprs[4] = {64, 32, 16, 8};
  for (int i = 0; i < (lpr64_only ? 1 : 4); ++i) {
    const int lpr = lprs[i];
    int bpl = (nbw + lpr - 1) / lpr;
    if (bpl > 8) continue;
    if (bpl == 5) bpl = 6;
    if (bpl == 7) bpl = 8;
    const double util = (double)nbw / (double)(lpr * bpl);
    if (util > best_util + 1e-9) {
      best_util = util;
      lpr_best = lpr;
      bpl_best = bpl;
    }
  }
  *lpr_out = lpr_best;
  *bpl_out = bpl_best;
}

// rows per lane group give ~8-16 weight loads in flight per lane while
// keeping enough workgroups to cover the chip; rows of >= 8192 columns split
// their columns over the four waves of a workgroup (KW = 4)
inline Cfg pick(int nbk, int64_t units, int epi, bool pro) {
  Cfg c;
  c.kw = (!pro && nbk >= 256 && nbk % 4 == 0) ? 4 : 1;
  pick_lanes(nbk / c.kw, &c.lpr, &c.bpl, c.kw == 4);
  const int G = 64 / c.lpr;
  int r = c.bpl == 1 ? 8 : c.bpl == 2 ? (c.kw == 4 ? 8 : 4) : c.bpl <= 4 ? 2 : 1;
  if (r > c.lpr) r = c.lpr;
  const int rmin = (epi == EPI_GEGLU) ? 2 : 1;
  const int per_wg = (c.kw == 1 ? 4 : 1) * G;
  // measured on MI355X at the E4B shapes: 256 workgroups (128 with the fused
  // prologue, which every workgroup repeats) keep enough loads in flight
  const int64_t min_wgs = pro ? 128 : 256;
  while (r > rmin && (units + per_wg * r - 1) / (per_wg * r) < min_wgs) r >>= 1;
  if (r < rmin) r = rmin;
  c.r = r;
  return c;
}

// everything a launch needs besides the template parameters
struct Launch {
  Q40Mat W;
  const uint32_t* xh;
  const uint32_t* xl;
  GemvOut o;
  int64_t units;
  int ks, nbk;
  int max_wgs;  // grid cap; waves stride over the remaining tiles
  ProArgs pa;
  hipStream_t st;
};

template <int LPR, int BPL, int R, int KW, bool XLO, int EPI, int PROK>
void launch(const Launch& L) {
  constexpr int G = 64 / LPR;
  const int64_t ntiles = (L.units + G * R - 1) / (G * R);
  int64_t wgs = KW == 1 ? (ntiles + 3) / 4 : ntiles;
  if (wgs > L.max_wgs) wgs = L.max_wgs;
  hipLaunchKernelGGL((k_q40<LPR, BPL, R, KW, XLO, EPI, PROK>), dim3((unsigned)wgs, (unsigned)L.ks), dim3(256), 0,
                     L.st, L.W, L.xh, L.xl, L.o, ntiles, L.nbk, L.pa);
}

template <int LPR, int BPL, int KW, bool XLO, int EPI, int PROK>
bool launch_r(const Cfg& c, const Launch& L) {
  switch (c.r) {
    case 1:
      if constexpr (EPI != EPI_GEGLU) {
        launch<LPR, BPL, 1, KW, XLO, EPI, PROK>(L);
        return true;
      }
      return false;
    case 2: launch<LPR, BPL, 2, KW, XLO, EPI, PROK>(L); return true;
    case 4: launch<LPR, BPL, 4, KW, XLO, EPI, PROK>(L); return true;
    case 8: launch<LPR, BPL, 8, KW, XLO, EPI, PROK>(L); return true;
  }
  return false;
}

template <int LPR, int KW, bool XLO, int EPI>
bool launch_b(const Cfg& c, const Launch& L) {
  switch (c.bpl) {
    case 1: return launch_r<LPR, 1, KW, XLO, EPI, 0>(c, L);
    case 2: return launch_r<LPR, 2, KW, XLO, EPI, 0>(c, L);
    case 3: return launch_r<LPR, 3, KW, XLO, EPI, 0>(c, L);
    case 4: return launch_r<LPR, 4, KW, XLO, EPI, 0>(c, L);
    case 6: return launch_r<LPR, 6, KW, XLO, EPI, 0>(c, L);
    case 8: return launch_r<LPR, 8, KW, XLO, EPI, 0>(c, L);
  }
  return false;
}

// no prologue, KW = 1: any lane split
template <bool XLO, int EPI>
bool launch_plain(const Cfg& c, const Launch& L) {
  switch (c.lpr) {
    case 64: return launch_b<64, 1, XLO, EPI>(c, L);
    case 32: return launch_b<32, 1, XLO, EPI>(c, L);
    case 16: return launch_b<16, 1, XLO, EPI>(c, L);
    case 8: return launch_b<8, 1, XLO, EPI>(c, L);
  }
  return false;
}

// fused prologue: H = 256 PROK, one block per lane (LPR = H / 32)
template <int EPI>
bool launch_pro(const Cfg& c, const Launch& L) {
  if (c.bpl != 1) return false;
  switch (c.lpr) {
    case 8: return launch_r<8, 1, 1, false, EPI, 1>(c, L);
    case 16: return launch_r<16, 1, 1, false, EPI, 2>(c, L);
    case 32: return launch_r<32, 1, 1, false, EPI, 4>(c, L);
    case 64: return launch_r<64, 1, 1, false, EPI, 8>(c, L);
  }
  return false;
}

// per-translation-unit dispatchers (k_q40_*.hip)
bool dispatch_f32(const Cfg& c, const Launch& L);     // f16 x, f32 out
bool dispatch_f32_hl(const Cfg& c, const Launch& L);  // hi/lo f16 x, f32 out
bool dispatch_glu(const Cfg& c, const Launch& L, int epi);
bool dispatch_kw4(const Cfg& c, const Launch& L, int epi);
bool dispatch_pro(const Cfg& c, const Launch& L, int epi);

}  // namespace q40k
