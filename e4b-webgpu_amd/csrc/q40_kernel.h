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
#include "trace.h"

// batches of the fused-prologue gate/up GeGLU tile and of the column-split
// f32 tile of 8 rows (the down projection) (compile-time, for A/B builds)
#ifndef E4B_TUNE_GEGLU_NB
#define E4B_TUNE_GEGLU_NB 4
#endif
#ifndef E4B_TUNE_KW4_NB
#define E4B_TUNE_KW4_NB 2
#endif
// batches requested before the prologue (PRE) and kept in flight ahead of
// the one being multiplied (LB) by k_q40b
#ifndef E4B_TUNE_GEGLU_PRE
#define E4B_TUNE_GEGLU_PRE 1
#endif
#ifndef E4B_TUNE_GEGLU_LB
#define E4B_TUNE_GEGLU_LB 1
#endif
#ifndef E4B_TUNE_KW4_PRE
#define E4B_TUNE_KW4_PRE 2
#endif
#ifndef E4B_TUNE_KW4_LB
#define E4B_TUNE_KW4_LB 2
#endif

// waves, batches and batches requested ahead of the plain f32 GEMV tile of
// 8 rows x 64 blocks (measured on MI355X for c0, 16384 x 2048 with f32 x:
// the whole tile requested up front and multiplied in 2 batches 5.23 us,
// against 6.21 unbatched, 5.34 with one batch ahead, 5.39 in 4 batches,
// 6.35 / 5.33 with 8-wave workgroups)
#ifndef E4B_TUNE_PLAIN_NWV
#define E4B_TUNE_PLAIN_NWV 4
#endif
#ifndef E4B_TUNE_PLAIN_NB
#define E4B_TUNE_PLAIN_NB 2
#endif
#ifndef E4B_TUNE_PLAIN_PRE
#define E4B_TUNE_PLAIN_PRE 2
#endif
#ifndef E4B_TUNE_PLAIN_LB
#define E4B_TUNE_PLAIN_LB 2
#endif

// batches of the qkv tile (norm prologue, 4 rows) and of the o tile
// (attention-combine prologue, 2 rows); 1 = unbatched.  Measured on MI355X
// at the E4B shape: the o tile requested whole and multiplied in 2 batches
// 853.1 tok/s against 851.3 unbatched and 840.3 with one batch ahead; the
// qkv tile 851.5 (whole, 2 batches) and 841.8 (one ahead): left unbatched
#ifndef E4B_TUNE_QKV_NB
#define E4B_TUNE_QKV_NB 1
#endif
#ifndef E4B_TUNE_QKV_PRE
#define E4B_TUNE_QKV_PRE 1
#endif
#ifndef E4B_TUNE_QKV_LB
#define E4B_TUNE_QKV_LB 1
#endif
#ifndef E4B_TUNE_O_NB
#define E4B_TUNE_O_NB 2
#endif
#ifndef E4B_TUNE_O_PRE
#define E4B_TUNE_O_PRE 2
#endif
#ifndef E4B_TUNE_O_LB
#define E4B_TUNE_O_LB 2
#endif

// rows per wave and waves per workgroup of the fused-prologue GeGLU tile
#ifndef E4B_TUNE_GEGLU_R
#define E4B_TUNE_GEGLU_R 8
#endif
#ifndef E4B_TUNE_GEGLU_NWV
#define E4B_TUNE_GEGLU_NWV 8
#endif

// fewest workgroups the row-tile choice keeps for a GEMV with the fused norm
// prologue and with the attention-combine prologue
#ifndef E4B_TUNE_PRO_MINWGS
#define E4B_TUNE_PRO_MINWGS 128
#endif
#ifndef E4B_TUNE_ATTN_MINWGS
#define E4B_TUNE_ATTN_MINWGS 256
#endif

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

// registers of the prologue's inputs: H = 256 PROK elements over TPB
// threads, thread t owning the N contiguous elements [N t, N t + N) so that
// each vector costs N/4 16-byte loads per thread (a wave can have at most 63
// loads outstanding; dword loads of 11 vectors would exceed that); NA
// partial vectors of a
template <int PROK, int TPB = 256, int NA = 1>
struct ProRegs {
  static constexpr int N = PROK > 0 ? 256 * PROK / TPB : 1;
  static_assert(PROK <= 0 || (256 * PROK % TPB == 0 && (N == 1 || N == 2 || N % 4 == 0)), "elements per thread");
  float h[N], a[NA][N], w1[N], w2[N];
};

// N contiguous floats at p (aligned to min(N, 4) floats) with the widest loads
template <int N>
DEV void ld_floats(const float* p, float (&v)[N]) {
  if constexpr (N == 1) {
    v[0] = p[0];
  } else if constexpr (N == 2) {
    const float2 t = *reinterpret_cast<const float2*>(p);
    v[0] = t.x;
    v[1] = t.y;
  } else {
#pragma unroll
    for (int q = 0; q < N / 4; ++q) {
      const float4 t = reinterpret_cast<const float4*>(p)[q];
      v[4 * q] = t.x;
      v[4 * q + 1] = t.y;
      v[4 * q + 2] = t.z;
      v[4 * q + 3] = t.w;
    }
  }
}

// N contiguous floats to p (aligned to min(N, 4) floats) with the widest stores
template <int N>
DEV void st_floats(float* p, const float (&v)[N]) {
  if constexpr (N == 1) {
    p[0] = v[0];
  } else if constexpr (N == 2) {
    *reinterpret_cast<float2*>(p) = make_float2(v[0], v[1]);
  } else {
#pragma unroll
    for (int q = 0; q < N / 4; ++q)
      reinterpret_cast<float4*>(p)[q] = make_float4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
  }
}

// sum over a block of NW waves; every thread gets the total (red: NW floats of LDS)
template <int NW>
DEV float block_sum_n(float v, float* red) {
  v = wave_sum(v);
  lds_sync();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  lds_sync();
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) t += red[w];
  return t;
}

// NA partial vectors a[s*H + i] (s < NA) are summed into a, in order, by
// pro_finish; pro_issue only issues the loads, so nothing between them and
// the weight loads waits for memory
// NORM2 = false: the prologue ends at h (x = f16(h), w2 unused and not read)
template <int PROK, int NA = 1, int TPB = 256, bool NORM2 = true>
DEV void pro_issue(const ProArgs& p, ProRegs<PROK, TPB, NA>& r) {
  constexpr int N = ProRegs<PROK, TPB, NA>::N;
  // absent vectors read hin instead (always valid) and are masked after the
  // load, so every load issues without a branch
  const bool has_a = p.a != nullptr, has_w2 = p.w2 != nullptr;
  const float* a = has_a ? p.a : p.hin;
  const float* w1 = has_a ? p.w1 : p.hin;
  const float* w2 = has_w2 ? p.w2 : p.hin;
  const int64_t sstride = has_a ? p.H : 0;
  const int i0 = threadIdx.x * N;
  ld_floats<N>(p.hin + i0, r.h);
#pragma unroll
  for (int s = 0; s < NA; ++s) ld_floats<N>(a + s * sstride + i0, r.a[s]);
  ld_floats<N>(w1 + i0, r.w1);
  if constexpr (NORM2) ld_floats<N>(w2 + i0, r.w2);
}

// attention-combine prologue of the o projection: x[h*HD + d] = f16 of the
// log-sum-exp merge of the live split-K chunks of head h (kernels/attcomb.wgsl
// :10-36).  With kProAttn the workgroup merges all 8 heads of 256 dims;
// with kProAttn2 (4 heads of 256) and kProAttn4w (4 heads of 512) the
// projection's columns are cut into slices of 4 heads (blockIdx.y) and a
// workgroup merges only its slice's heads, so each workgroup reads only
// their partials (the consumer's prologue sums the slices' partial
// outputs).  attn_issue requests, before the weight tile and without
// waiting for the position, the (max, sum) pairs of every allocated chunk
// of the slice's heads (one lane per chunk) and the partial outputs of the
// first U chunks; attn_finish reduces the pairs to normalised chunk weights
// e^(m_c - M) / sum_c l_c e^(m_c - M) in LDS and accumulates.  Chunks past
// the first U are read U at a time in further passes.  The merged slice
// lands in LDS at offset 0 (the dot products index it from the slice's
// first column).
constexpr int kProAttn = -1;
constexpr int kProAttn2 = -3;
constexpr int kProAttn4w = -4;
constexpr int kProAttnFirst = 8;
constexpr int kProAttnMaxCh = kProAttnMaxChunks;  // chunks per head the prologue supports (one lane each)
constexpr bool pro_attn(int k) { return k == kProAttn || k == kProAttn2 || k == kProAttn4w; }
// heads a workgroup merges, and their head dim
constexpr int attn_hs(int k) { return k == kProAttn ? 8 : 4; }
constexpr int attn_hd(int k) { return k == kProAttn4w ? 512 : 256; }
static_assert(kProAttnH == 8 * 256 && kProAttnH == 4 * 512, "the merged slice fits the 2048-column LDS stage");
// 256 threads over HS heads of HD dims: thread t merges local head
// t / (256 / HS), EPT = HS HD / 256 consecutive dims (one or two 16-byte
// loads per chunk); wave v owns the (max, sum) pairs of local heads HPW v ..
// HPW v + HPW - 1
template <int U, int HS, int HD = 256>
struct AttnRegs {
  static constexpr int HPW = HS / 4, TPH = 256 / HS, EPT = HD / TPH;
  uint32_t pos;
  float m[HPW], l[HPW];
  float v[U][EPT];
};

// pos_idx: params[pos_idx] is the token's slot (0 on sliding layers, kv_idx
// on counted full layers)
template <int U, int HS, int HD>
DEV void attn_issue(const ProArgs& p, AttnRegs<U, HS, HD>& r, int pos_idx) {
  using R = AttnRegs<U, HS, HD>;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int hb = HS * (int)blockIdx.y;  // the slice's first head
  r.pos = p.params[pos_idx];
  const int c = min(lane, p.gch - 1);
#pragma unroll
  for (int hh = 0; hh < R::HPW; ++hh) {
    const float* ml = p.part_ml + (int64_t)(hb + R::HPW * wv + hh) * p.gch * 2;
    r.m[hh] = ml[2 * c];
    r.l[hh] = ml[2 * c + 1];
  }
  const int h = hb + threadIdx.x / R::TPH, d0 = (threadIdx.x % R::TPH) * R::EPT;
#pragma unroll
  for (int u = 0; u < U; ++u)
    ld_floats<R::EPT>(p.part_o + ((int64_t)h * p.gch + min(u, p.gch - 1)) * HD + d0, r.v[u]);
}

template <int U, int HS, int HD>
DEV void attn_finish(const ProArgs& p, AttnRegs<U, HS, HD>& r, uint16_t* xs, float* wts) {
  using R = AttnRegs<U, HS, HD>;
  const int pos = (int)r.pos;
  const int lo = (p.window > 0 && pos + 1 > p.window) ? pos + 1 - p.window : 0;
  const int nch = (pos + 1 - lo + (1 << p.chunk_shift) - 1) >> p.chunk_shift;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int hb = HS * (int)blockIdx.y;
  const bool live = lane < nch;
#pragma unroll
  for (int hh = 0; hh < R::HPW; ++hh) {
    const float m = live ? r.m[hh] : -3.0e38f;
    const float M = wave_max(m);
    const float f = live ? __expf(m - M) : 0.f;
    const float den = wave_sum(live ? r.l[hh] * f : 0.f);
    wts[(R::HPW * wv + hh) * kProAttnMaxCh + lane] = f / den;
  }
  lds_sync();
  const int hl = threadIdx.x / R::TPH, h = hb + hl, d0 = (threadIdx.x % R::TPH) * R::EPT;
  const float* wh = wts + hl * kProAttnMaxCh;
  float acc[R::EPT];
#pragma unroll
  for (int j = 0; j < R::EPT; ++j) acc[j] = 0.f;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (u < nch) {  // chunks past the live ones may hold stale or unwritten values
      const float wu = wh[u];
#pragma unroll
      for (int j = 0; j < R::EPT; ++j) acc[j] = fmaf(r.v[u][j], wu, acc[j]);
    }
  }
  for (int c0 = U; c0 < nch; c0 += U) {
#pragma unroll
    for (int u = 0; u < U; ++u)
      ld_floats<R::EPT>(p.part_o + ((int64_t)h * p.gch + min(c0 + u, nch - 1)) * HD + d0, r.v[u]);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (c0 + u < nch) {
        const float wu = wh[c0 + u];
#pragma unroll
        for (int j = 0; j < R::EPT; ++j) acc[j] = fmaf(r.v[u][j], wu, acc[j]);
      }
    }
  }
  uint32_t pk[R::EPT / 2];
#pragma unroll
  for (int j = 0; j < R::EPT / 2; ++j) pk[j] = (uint32_t)f2h(acc[2 * j]) | ((uint32_t)f2h(acc[2 * j + 1]) << 16);
  uint16_t* dst = xs + hl * HD + d0;  // the slice at offset 0
#pragma unroll
  for (int q = 0; q < R::EPT / 8; ++q)
    reinterpret_cast<uint4*>(dst)[q] = make_uint4(pk[4 * q], pk[4 * q + 1], pk[4 * q + 2], pk[4 * q + 3]);
  if constexpr (R::EPT == 4) *reinterpret_cast<uint2*>(dst) = make_uint2(pk[0], pk[1]);
  lds_sync();
}

// A4B layer-boundary prologue (ProArgs.tail): the previous layer's MoE tail
// (kernels/a4btail.wgsl:26-71) and this layer's input norm
// (kernels/rmsnorm.wgsl:13-51), for any H <= 3072 divisible by 4:
//   comb = rms(a) w1 + rms(a2) w1b;  h = (hin + rms(comb) wp) * scale;
//   x = f16(rms(h) w2); block (0,0) writes h to hout
// with a == null (the first layer) h = hin * scale.  Thread t owns the
// float4 groups q = t + 256 k (k < 3); groups past H/4 read the last one and
// are masked to zero.
constexpr int kProTail = -2;
constexpr int kProTailK = 3;
constexpr int kProTailMaxH = 4 * 256 * kProTailK;

struct TailRegs {
  // element 4 k + c of each vector: component c of the thread's float4 group k
  float h[4 * kProTailK], a[4 * kProTailK], a2[4 * kProTailK], w1[4 * kProTailK], w1b[4 * kProTailK],
      wp[4 * kProTailK], w2[4 * kProTailK];
};

DEV void ld4(const float* p, int q, float* d) {
  const float4 t = reinterpret_cast<const float4*>(p)[q];
  d[0] = t.x;
  d[1] = t.y;
  d[2] = t.z;
  d[3] = t.w;
}

DEV void tail_issue(const ProArgs& p, TailRegs& r) {
  const int H4 = p.H >> 2;
  // absent vectors (the first layer) read hin instead and are masked
  const bool has_a = p.a != nullptr;
  const float* a = has_a ? p.a : p.hin;
  const float* a2 = has_a ? p.a2 : p.hin;
  // the vectors whose pointers arrive as preloaded arguments first, then
  // the three norm weights read from the argument struct
#pragma unroll
  for (int k = 0; k < kProTailK; ++k) {
    const int q = min((int)threadIdx.x + 256 * k, H4 - 1);
    ld4(p.hin, q, r.h + 4 * k);
    ld4(a, q, r.a + 4 * k);
    ld4(a2, q, r.a2 + 4 * k);
    ld4(p.w2, q, r.w2 + 4 * k);
  }
  __builtin_amdgcn_sched_barrier(0);
  const float* w1 = has_a ? p.w1 : p.hin;
  const float* w1b = has_a ? p.w1b : p.hin;
  const float* wp = has_a ? p.wp : p.hin;
#pragma unroll
  for (int k = 0; k < kProTailK; ++k) {
    const int q = min((int)threadIdx.x + 256 * k, H4 - 1);
    ld4(w1, q, r.w1 + 4 * k);
    ld4(w1b, q, r.w1b + 4 * k);
    ld4(wp, q, r.wp + 4 * k);
  }
}

DEV void tail_finish(const ProArgs& p, TailRegs& r, uint16_t* xs, float* red) {
  constexpr int NE = 4 * kProTailK;
  const int H4 = p.H >> 2;
  const bool has_a = p.a != nullptr;
#pragma unroll
  for (int e = 0; e < NE; ++e) {
    const bool in = (int)threadIdx.x + 256 * (e >> 2) < H4;
    r.h[e] = in ? r.h[e] : 0.f;
    r.a[e] = (in && has_a) ? r.a[e] : 0.f;
    r.a2[e] = (in && has_a) ? r.a2[e] : 0.f;
  }
  // rms of the two branch outputs, then of their normed sum (every reduction
  // runs, the first layer's on zeros: no branch between loads and use)
  float sa = 0.f, sb = 0.f;
#pragma unroll
  for (int e = 0; e < NE; ++e) {
    sa = fmaf(r.a[e], r.a[e], sa);
    sb = fmaf(r.a2[e], r.a2[e], sb);
  }
  const float ia = rms_inv(block_sum_n<4>(sa, red), p.H, p.eps);
  const float ib = rms_inv(block_sum_n<4>(sb, red), p.H, p.eps);
  float sc = 0.f;
#pragma unroll
  for (int e = 0; e < NE; ++e) {
    r.a[e] = fmaf(r.a[e] * ia, r.w1[e], r.a2[e] * ib * r.w1b[e]);  // comb
    sc = fmaf(r.a[e], r.a[e], sc);
  }
  const float ic = has_a ? rms_inv(block_sum_n<4>(sc, red), p.H, p.eps) : 0.f;
  float sh = 0.f;
#pragma unroll
  for (int e = 0; e < NE; ++e) {
    const float w = has_a ? r.wp[e] : 0.f;
    r.h[e] = (r.h[e] + r.a[e] * ic * w) * p.scale;
    sh = fmaf(r.h[e], r.h[e], sh);
  }
  const float ih = rms_inv(block_sum_n<4>(sh, red), p.H, p.eps);
  const bool writer = p.hout && blockIdx.x == 0 && blockIdx.y == 0;
#pragma unroll
  for (int k = 0; k < kProTailK; ++k) {
    const int q = (int)threadIdx.x + 256 * k;
    if (q < H4) {
      const float* h = r.h + 4 * k;
      const float* w = r.w2 + 4 * k;
      const uint2 pk = make_uint2((uint32_t)f2h(h[0] * ih * w[0]) | ((uint32_t)f2h(h[1] * ih * w[1]) << 16),
                                  (uint32_t)f2h(h[2] * ih * w[2]) | ((uint32_t)f2h(h[3] * ih * w[3]) << 16));
      *reinterpret_cast<uint2*>(xs + 4 * q) = pk;
      if (writer) reinterpret_cast<float4*>(p.hout)[q] = make_float4(h[0], h[1], h[2], h[3]);
      if (writer && p.hsnap) reinterpret_cast<float4*>(p.hsnap)[q] = make_float4(h[0], h[1], h[2], h[3]);
    }
  }
  lds_sync();
}

// h = (hin + rms(a) * w1) * scale; x = w2 ? f16(rms(h) * w2) : f16(h)
// (kernels/rmsacc3.wgsl:36-53, kernels/a4btail.wgsl:54-71,
// kernels/rmsacc.wgsl:10-26 folded into the consumer GEMV)
template <int PROK, int TPB = 256, int NA = 1, bool NORM2 = true>
DEV void pro_finish(const ProArgs& p, ProRegs<PROK, TPB, NA>& r, uint16_t* xs, float* red) {
  constexpr int N = ProRegs<PROK, TPB, NA>::N;
  static_assert(256 * PROK % TPB == 0, "whole elements per thread");
  const bool has_a = p.a != nullptr, has_w2 = p.w2 != nullptr;
  float av[N];
#pragma unroll
  for (int k = 0; k < N; ++k) {
    float sum = r.a[0][k];
#pragma unroll
    for (int s = 1; s < NA; ++s) sum += r.a[s][k];
    av[k] = has_a ? sum : 0.f;
    r.w1[k] = has_a ? r.w1[k] : 0.f;
    r.w2[k] = (NORM2 && has_w2) ? r.w2[k] : 1.f;
  }
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < N; ++k) ss = fmaf(av[k], av[k], ss);
  // both reductions run unconditionally: no branch between the weight loads
  // and their use, so the compiler's wait counts stay exact
  const float s1 = block_sum_n<TPB / 64>(ss, red);
  const float inv1 = p.a ? rms_inv(s1, p.H, p.eps) : 0.f;
  float s2 = 0.f;
#pragma unroll
  for (int k = 0; k < N; ++k) {
    r.h[k] = (r.h[k] + av[k] * inv1 * r.w1[k]) * p.scale;
    s2 = fmaf(r.h[k], r.h[k], s2);
  }
  float inv2 = 1.f;
  if constexpr (NORM2) inv2 = p.w2 ? rms_inv(block_sum_n<TPB / 64>(s2, red), p.H, p.eps) : 1.f;
  const bool writer = p.hout && blockIdx.x == 0 && blockIdx.y == 0;
  const int i0 = threadIdx.x * N;
#pragma unroll
  for (int k = 0; k < N; ++k) {
    xs[i0 + k] = f2h((NORM2 && p.w2) ? r.h[k] * inv2 * r.w2[k] : r.h[k]);
    if (writer) p.hout[i0 + k] = r.h[k];
  }
  if (writer && p.hsnap) st_floats<N>(p.hsnap + i0, r.h);  // the per-layer readout (rare: its own branch)
  lds_sync();
}

// Leading scalar kernel arguments.  The library is built with
// -amdgpu-kernarg-preload-count, so the dispatcher writes the first 14
// dwords of a kernel's arguments into SGPRs before its waves start; struct
// arguments are not preloaded.  Everything a wave needs to issue its first
// requests (the weight planes, their shape, the prologue's input pointers)
// therefore comes first, ahead of the structs, and overwrites the structs'
// copies of the same fields: no request waits for a kernel-argument load
// (0.24 us a wave measured on MI355X).  lp0..lp3 by prologue:
//   PROK > 0 (residual + norm): hin, a, w1, w2;
//   attention combine: params, part_ml, part_o, and gch | pos_idx << 32 as
//   lp3's bits;
//   layer boundary: hin, a, a2, w2 (H = 32 nb; w1, w1b and wp come from
//   the struct and are requested after these);
//   none: xh, xl (lp2, lp3 unused).
// (lp3 is pointer-typed so that w2 keeps the global address space of a
// kernel pointer argument; an integer cast back would make its load a flat
// one, which the compiler can only wait for with vmcnt(0).)
// ldims = nb | nbk << 16; lunits = rows (2 ff for EPI_GEGLU).
#define Q40_LEAD_PARAMS                                                                                   \
  const uint4 *__restrict__ lnib, const uint16_t *__restrict__ lsc, const void *lp0, const void *lp1,    \
      const void *lp2, const void *lp3, uint32_t ldims, uint32_t lunits

template <int PROK, int EPI>
DEV void take_lead(const uint4* lnib, const uint16_t* lsc, const void* lp0, const void* lp1, const void* lp2,
                   const void* lp3, uint32_t ldims, uint32_t lunits, Q40Mat& W, const uint32_t* __restrict__& xh,
                   const uint32_t* __restrict__& xl, GemvOut& o, ProArgs& pa, int& nbk, int& pos_idx) {
  W.nib = lnib;
  W.sc = lsc;
  W.nb = (int)(ldims & 0xffffu);
  nbk = (int)(ldims >> 16);
  if constexpr (EPI == EPI_GEGLU) o.ff = lunits >> 1; else W.rows = lunits;
  if constexpr (PROK > 0) {
    pa.hin = static_cast<const float*>(lp0);
    pa.a = static_cast<const float*>(lp1);
    pa.w1 = static_cast<const float*>(lp2);
    pa.w2 = static_cast<const float*>(lp3);
    pa.H = 256 * PROK;
  } else if constexpr (pro_attn(PROK)) {
    pa.params = static_cast<const uint32_t*>(lp0);
    pa.part_ml = static_cast<const float*>(lp1);
    pa.part_o = static_cast<const float*>(lp2);
    const uint64_t bits = (uint64_t)(uintptr_t)lp3;
    pa.gch = (int)(uint32_t)bits;
    pos_idx = (int)(bits >> 32);
  } else if constexpr (PROK == kProTail) {
    pa.hin = static_cast<const float*>(lp0);
    pa.a = static_cast<const float*>(lp1);
    pa.a2 = static_cast<const float*>(lp2);
    pa.w2 = static_cast<const float*>(lp3);
    pa.H = 32 * (int)(ldims & 0xffffu);
  } else if constexpr (PROK == 0) {
    xh = static_cast<const uint32_t*>(lp0);
    xl = static_cast<const uint32_t*>(lp1);
  }
}

// A wave splits into G = 64/LPR lane groups; with KW = 1 a group owns R rows
// ("slots") of the wave's tile, with KW = 4 the four waves share the tile's
// rows and each covers a quarter of the columns.  Lane l of a group covers
// blocks jb = l + LPR*k (k < BPL) of its column range.  blockIdx.y selects
// one of KS column slices (partial outputs, EPI_F32 only).
//
// One tile per wave (the grid covers the matrix): all of the tile's loads are
// issued up front, with no branch between them and their first use, so the
// compiler's wait counts stay exact and a fused prologue computes while the
// weight stream is in flight.
// The struct fields that the residual/tail prologue and the epilogue read
// after the loads are issued, read in one wait that overlaps those loads.
// Left to the compiler, each field was read where first used, and the
// prologue's LDS waits (lgkmcnt also counts scalar loads) then waited on a
// kernel-argument round trip each.
template <int PROK, int EPI>
DEV void read_late_fields(const ProArgs& pa, const GemvOut& o) {
  if constexpr (PROK > 0 || PROK == kProTail)
    asm volatile("" ::"s"(pa.eps), "s"(pa.scale), "s"(pa.hout), "s"(pa.hsnap));
  if constexpr (EPI == EPI_F32)
    asm volatile("" ::"s"(o.y));
  else
    asm volatile("" ::"s"(o.yh));
}

template <int LPR, int BPL, int R, int KW, bool XLO, int EPI, int PROK, int NA = 1, int NWV = 4>
__global__ __launch_bounds__(64 * NWV) void k_q40(Q40_LEAD_PARAMS, Q40Mat W, const uint32_t* __restrict__ xh,
                                                  const uint32_t* __restrict__ xl, GemvOut o, ProArgs pa) {
  constexpr int G = 64 / LPR, SPAN = LPR / R, SLOTS = G * R;
  constexpr int TPB = 64 * NWV;
  [[maybe_unused]] constexpr uint32_t kLog2R = R >= 16 ? 4 : R >= 8 ? 3 : R >= 4 ? 2 : R >= 2 ? 1 : 0;
  E4B_TRACE_SCOPE(trace_tag(TR_Q40, (uint32_t)(PROK + 8) | (uint32_t)EPI << 5 | kLog2R << 8 | (uint32_t)(KW == 4) << 12 |
                                        (uint32_t)(gridDim.y > 1) << 13));
  static_assert(KW == 1 || KW == 4, "KW is 1 or 4");
  static_assert(NWV == 4 || (KW == 1 && PROK >= 0), "wide workgroups: no column split, no attention prologue");
  static_assert(EPI != EPI_GEGLU || (R % 2 == 0), "GeGLU tiles hold (gate, up) pairs");
  static_assert(!(PROK && XLO), "the prologue produces f16 input");
  static_assert(PROK >= kProAttn4w, "prologue kind");
  static_assert(PROK >= 0 || (EPI == EPI_F32 && KW == 1 && NWV == 4), "attention / tail prologue: f32, KW = 1");
  static_assert(R * BPL <= 64, "scale parity bits");
  __shared__ __align__(16) uint16_t xs_lds[PROK > 0 ? 256 * PROK : pro_attn(PROK) ? kProAttnH
                                                                  : PROK == kProTail ? kProTailMaxH : 8];
  __shared__ float red[NWV];
  __shared__ float part[KW == 4 ? 4 * SLOTS : 1];
  __shared__ float mls[pro_attn(PROK) ? attn_hs(PROK) * kProAttnMaxCh : 1];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane / LPR, l = lane - g * LPR;
  int nbk = 0, pos_idx = 0;
  take_lead<PROK, EPI>(lnib, lsc, lp0, lp1, lp2, lp3, ldims, lunits, W, xh, xl, o, pa, nbk, pos_idx);
  const int64_t ntiles = ((int64_t)lunits + SLOTS - 1) / SLOTS;
  const int kslice = blockIdx.y;
  const int nbw = nbk / KW;  // blocks per wave
  const int jb0 = kslice * nbk + (KW == 4 ? wave * nbw : 0);
  const int nb = W.nb;
  const int64_t units = (EPI == EPI_GEGLU) ? 2 * o.ff : W.rows;
  const int64_t tile_id = (KW == 1) ? (int64_t)blockIdx.x * NWV + wave : (int64_t)blockIdx.x;
  const bool live = tile_id < ntiles;                 // the last workgroup may hold idle waves
  const int64_t tile = live ? tile_id : ntiles - 1;   // their loads repeat the last tile
  const int64_t slot0 = tile * SLOTS + (int64_t)g * R;

  ProRegs<PROK, TPB, NA> pr;
  if constexpr (PROK > 0) pro_issue<PROK, NA, TPB>(pa, pr);
  // the attention prologue requests its first UA chunks up front (NA names
  // UA for this prologue: 8 or 16)
  constexpr int UA = (pro_attn(PROK) && NA > 1) ? NA : kProAttnFirst;
  AttnRegs<UA, attn_hs(PROK), attn_hd(PROK)> ar;
  if constexpr (pro_attn(PROK)) attn_issue(pa, ar, pos_idx);
  TailRegs tr;
  if constexpr (PROK == kProTail) tail_issue(pa, tr);
  // the prologue's requests stay ahead of the weight requests (vmcnt drains in order)
  __builtin_amdgcn_sched_barrier(0);

  // weight tile: rows and blocks clamped into range (slots past the end are
  // computed on duplicate data and never stored; blocks past the range end
  // meet zeroed activations); scales as aligned pairs (ld_scale_pair)
  uint4 wq[R][BPL];
  uint32_t ws[R][BPL];
  uint64_t odd = 0;  // bit r*BPL+k: the scale is the odd half of its pair
#pragma unroll
  for (int r = 0; r < R; ++r) {
    int64_t row;
    if constexpr (EPI == EPI_GEGLU) {
      const int64_t u = min(slot0 / 2 + r / 2, o.ff - 1);
      row = (r & 1) ? o.ff + u : u;
    } else {
      row = min(slot0 + r, units - 1);
    }
#pragma unroll
    for (int k = 0; k < BPL; ++k) {
      const int jb = min(l + LPR * k, nbw - 1);
      const uint32_t e = (uint32_t)row * (uint32_t)nb + (uint32_t)(jb0 + jb);  // planes < 4 GiB (host check)
      wq[r][k] = ld_nt_u4_off(W.nib, e);
      ws[r][k] = ld_scale_pair_off(W.sc, e);
      odd |= (uint64_t)(e & 1) << (r * BPL + k);
    }
  }
  // the epilogue multiplier of the row this lane finishes (lanes that finish
  // no row read a valid neighbour), requested with the tile
  float mulv = 0.f;
  if constexpr (EPI == EPI_GELU_MUL) mulv = o.mul[min(slot0 + l / SPAN, units - 1)];
  // keep the scheduler from hoisting prologue math (and its waits) above
  // the weight loads: every load of the tile is in flight before any wait
  __builtin_amdgcn_sched_barrier(0);
  read_late_fields<PROK, EPI>(pa, o);
  E4B_TRACE_MARK(0);

  uint32_t xp[BPL][16];
  uint32_t xq[BPL][XLO ? 16 : 1];
  float xs8[BPL];
  if constexpr (PROK > 0) pro_finish<PROK, TPB, NA>(pa, pr, xs_lds, red);
  if constexpr (pro_attn(PROK)) attn_finish(pa, ar, xs_lds, mls);
  if constexpr (PROK == kProTail) tail_finish(pa, tr, xs_lds, red);
  E4B_TRACE_MARK(1);
#pragma unroll
  for (int k = 0; k < BPL; ++k) {
    const int jb = l + LPR * k;
    const bool in = jb < nbw;
    const int jc = in ? jb : 0;
    if constexpr (PROK != 0) {
      const uint4* v = reinterpret_cast<const uint4*>(xs_lds) + (size_t)((pro_attn(PROK) ? 0 : jb0) + jc) * 4;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint4 t = v[i];
        xp[k][4 * i + 0] = t.x;
        xp[k][4 * i + 1] = t.y;
        xp[k][4 * i + 2] = t.z;
        xp[k][4 * i + 3] = t.w;
      }
    } else {
      load_x16(xh, jb0 + jc, xp[k]);
    }
    if constexpr (XLO) load_x16(xl, jb0 + jc, xq[k]);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      xp[k][i] = in ? xp[k][i] : 0u;
      if constexpr (XLO) xq[k][i] = in ? xq[k][i] : 0u;
    }
    float xs = xsum16(xp[k]);
    if constexpr (XLO) xs += xsum16(xq[k]);
    xs8[k] = -8.f * xs;
  }

  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    acc[r] = 0.f;
#pragma unroll
    for (int k = 0; k < BPL; ++k) {
      float a0 = 0.f, a1 = 0.f;
      q40_dot2(wq[r][k], xp[k], a0, a1);
      if constexpr (XLO) q40_dot2(wq[r][k], xq[k], a0, a1);
      const float d = scale_of(ws[r][k], (uint32_t)(odd >> (r * BPL + k)) & 1u);
      acc[r] = fmaf(d, fmaf(a1, kTwo24 / 16.f, fmaf(a0, kTwo24, xs8[k])), acc[r]);
    }
  }
  E4B_TRACE_MARK(2);
  float v = reduce_rows<LPR, R>(acc);
  const int r = l / SPAN;  // this lane now holds slot r of the group
  if constexpr (KW == 4) {
    // fold the four column quarters through LDS; wave 0 finishes
    if ((l % SPAN) == 0) part[wave * SLOTS + g * R + r] = v;
    lds_sync();
    if (wave != 0) return;
    const int sl = g * R + r;
    v = (part[sl] + part[SLOTS + sl]) + (part[2 * SLOTS + sl] + part[3 * SLOTS + sl]);
  }
  E4B_TRACE_MARK(3);
  if (!live) return;
  if constexpr (EPI == EPI_GEGLU) {
    const float up = __shfl_xor(v, SPAN, 64);
    const int64_t u = slot0 / 2 + r / 2;
    if ((l % (2 * SPAN)) == 0 && u < o.ff) o.yh[u] = f2h(gelu_tanh(v) * up);
  } else {
    const int64_t row = slot0 + r;
    if ((l % SPAN) == 0 && row < W.rows) {
      if constexpr (EPI == EPI_F32) o.y[(int64_t)kslice * W.rows + row] = v;
      if constexpr (EPI == EPI_GELU_MUL) o.yh[row] = f2h(gelu_tanh(v) * mulv);
    }
  }
}

// k_q40b: the tile of k_q40 pipelined in NB batches of R / NB rows: the input vector (from global memory when
// there is no prologue) and batch 0 are requested first, and batch b + 1 is
// requested before batch b's dot products, so a wave's arithmetic starts
// while the chip is still accepting the rest of the stream (on a full chip
// the memory system takes the requests of a whole tile only over several
// microseconds) and a prologue's block barriers wait only for batch 0.
template <int LPR, int BPL, int R, int KW, bool XLO, int EPI, int PROK, int NA = 1, int NWV = 4, int NB = 2,
          int PRE = 1, int LB = 1>
__global__ __launch_bounds__(64 * NWV) void k_q40b(Q40_LEAD_PARAMS, Q40Mat W, const uint32_t* __restrict__ xh,
                                                  const uint32_t* __restrict__ xl, GemvOut o, ProArgs pa) {
  constexpr int G = 64 / LPR, SPAN = LPR / R, SLOTS = G * R;
  constexpr int TPB = 64 * NWV;
  constexpr int RB = R / NB;  // rows per batch
  [[maybe_unused]] constexpr uint32_t kLog2R = R >= 16 ? 4 : R >= 8 ? 3 : R >= 4 ? 2 : R >= 2 ? 1 : 0;
  E4B_TRACE_SCOPE(trace_tag(TR_Q40, (uint32_t)(PROK + 8) | (uint32_t)EPI << 5 | kLog2R << 8 | (uint32_t)(KW == 4) << 12 |
                                        (uint32_t)(gridDim.y > 1) << 13 | (uint32_t)(NB > 1) << 14));
  static_assert(KW == 1 || KW == 4, "KW is 1 or 4");
  static_assert(NWV == 4 || (KW == 1 && PROK >= 0), "wide workgroups: no column split, no attention prologue");
  static_assert(EPI != EPI_GEGLU || (R % 2 == 0), "GeGLU tiles hold (gate, up) pairs");
  static_assert(!(PROK && XLO), "the prologue produces f16 input");
  static_assert(PROK >= kProAttn4w, "prologue kind");
  static_assert(PROK >= 0 || (EPI == EPI_F32 && KW == 1 && NWV == 4), "attention / tail prologue: f32, KW = 1");
  static_assert(R * BPL <= 64, "scale parity bits");
  static_assert(R % NB == 0 && (EPI != EPI_GEGLU || RB % 2 == 0), "whole (gate, up) pairs per batch");
  __shared__ __align__(16) uint16_t xs_lds[PROK > 0 ? 256 * PROK : pro_attn(PROK) ? kProAttnH
                                                                  : PROK == kProTail ? kProTailMaxH : 8];
  __shared__ float red[NWV];
  __shared__ float part[KW == 4 ? 4 * SLOTS : 1];
  __shared__ float mls[pro_attn(PROK) ? attn_hs(PROK) * kProAttnMaxCh : 1];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane / LPR, l = lane - g * LPR;
  int nbk = 0, pos_idx = 0;
  take_lead<PROK, EPI>(lnib, lsc, lp0, lp1, lp2, lp3, ldims, lunits, W, xh, xl, o, pa, nbk, pos_idx);
  const int64_t ntiles = ((int64_t)lunits + SLOTS - 1) / SLOTS;
  const int kslice = blockIdx.y;
  const int nbw = nbk / KW;  // blocks per wave
  const int jb0 = kslice * nbk + (KW == 4 ? wave * nbw : 0);
  const int nb = W.nb;
  const int64_t units = (EPI == EPI_GEGLU) ? 2 * o.ff : W.rows;
  const int64_t tile_id = (KW == 1) ? (int64_t)blockIdx.x * NWV + wave : (int64_t)blockIdx.x;
  const bool live = tile_id < ntiles;                 // the last workgroup may hold idle waves
  const int64_t tile = live ? tile_id : ntiles - 1;   // their loads repeat the last tile
  const int64_t slot0 = tile * SLOTS + (int64_t)g * R;

  ProRegs<PROK, TPB, NA> pr;
  if constexpr (PROK > 0) pro_issue<PROK, NA, TPB>(pa, pr);
  // the attention prologue requests its first UA chunks up front (NA names
  // UA for this prologue: 8 or 16)
  constexpr int UA = (pro_attn(PROK) && NA > 1) ? NA : kProAttnFirst;
  AttnRegs<UA, attn_hs(PROK), attn_hd(PROK)> ar;
  if constexpr (pro_attn(PROK)) attn_issue(pa, ar, pos_idx);
  TailRegs tr;
  if constexpr (PROK == kProTail) tail_issue(pa, tr);

  // the input vector: staged in LDS by a prologue, else this lane's blocks
  // from global memory (requested ahead of the weights when NB > 1); blocks
  // past the range end meet zeroed activations; xs8 is the -8 offset term
  uint32_t xp[BPL][16];
  uint32_t xq[BPL][XLO ? 16 : 1];
  float xs8[BPL];
  auto load_x = [&]() {  // NB > 1 without a prologue: this lane's blocks from global memory
#pragma unroll
    for (int k = 0; k < BPL; ++k) {
      const int jb = l + LPR * k;
      const int jc = jb < nbw ? jb : 0;
      load_x16(xh, jb0 + jc, xp[k]);
      if constexpr (XLO) load_x16(xl, jb0 + jc, xq[k]);
    }
  };
  auto finish_x = [&]() {
#pragma unroll
    for (int k = 0; k < BPL; ++k) {
      const bool in = l + LPR * k < nbw;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        xp[k][i] = in ? xp[k][i] : 0u;
        if constexpr (XLO) xq[k][i] = in ? xq[k][i] : 0u;
      }
      float xs = xsum16(xp[k]);
      if constexpr (XLO) xs += xsum16(xq[k]);
      xs8[k] = -8.f * xs;
    }
  };
  if constexpr (PROK == 0 && NB > 1) load_x();
  // the input requests stay ahead of the weight requests (vmcnt drains in order)
  __builtin_amdgcn_sched_barrier(0);

  // weight tile: rows and blocks clamped into range (slots past the end are
  // computed on duplicate data and never stored); scales as aligned pairs
  // (ld_scale_pair)
  uint4 wq[R][BPL];
  uint32_t ws[R][BPL];
  uint64_t odd = 0;  // bit r*BPL+k: the scale is the odd half of its pair
  auto issue_rows = [&](int r0) {
#pragma unroll
    for (int r = r0; r < r0 + RB; ++r) {
      int64_t row;
      if constexpr (EPI == EPI_GEGLU) {
        const int64_t u = min(slot0 / 2 + r / 2, o.ff - 1);
        row = (r & 1) ? o.ff + u : u;
      } else {
        row = min(slot0 + r, units - 1);
      }
#pragma unroll
      for (int k = 0; k < BPL; ++k) {
        const int jb = min(l + LPR * k, nbw - 1);
        const uint32_t e = (uint32_t)row * (uint32_t)nb + (uint32_t)(jb0 + jb);  // planes < 4 GiB (host check)
        wq[r][k] = ld_nt_u4_off(W.nib, e);
        ws[r][k] = ld_scale_pair_off(W.sc, e);
        odd |= (uint64_t)(e & 1) << (r * BPL + k);
      }
    }
  };
  float acc[R];
  auto dot_rows = [&](int r0) {
#pragma unroll
    for (int r = r0; r < r0 + RB; ++r) {
      acc[r] = 0.f;
#pragma unroll
      for (int k = 0; k < BPL; ++k) {
        float a0 = 0.f, a1 = 0.f;
        q40_dot2(wq[r][k], xp[k], a0, a1);
        if constexpr (XLO) q40_dot2(wq[r][k], xq[k], a0, a1);
        const float d = scale_of(ws[r][k], (uint32_t)(odd >> (r * BPL + k)) & 1u);
        acc[r] = fmaf(d, fmaf(a1, kTwo24 / 16.f, fmaf(a0, kTwo24, xs8[k])), acc[r]);
      }
    }
  };
  static_assert(PRE >= 0 && PRE <= LB && LB >= 1 && LB <= NB, "batches requested ahead");
#pragma unroll
  for (int b = 0; b < PRE; ++b) issue_rows(b * RB);
  // the epilogue multiplier of the row this lane finishes (lanes that finish
  // no row read a valid neighbour), requested with the tile
  float mulv = 0.f;
  if constexpr (EPI == EPI_GELU_MUL) mulv = o.mul[min(slot0 + l / SPAN, units - 1)];
  // keep the scheduler from hoisting prologue math (and its waits) above
  // the weight loads: every load requested so far is in flight before any wait
  __builtin_amdgcn_sched_barrier(0);
  read_late_fields<PROK, EPI>(pa, o);
  E4B_TRACE_MARK(0);

  if constexpr (PROK > 0) pro_finish<PROK, TPB, NA>(pa, pr, xs_lds, red);
  if constexpr (pro_attn(PROK)) attn_finish(pa, ar, xs_lds, mls);
  if constexpr (PROK == kProTail) tail_finish(pa, tr, xs_lds, red);
  E4B_TRACE_MARK(1);
  if constexpr (PROK == 0 && NB > 1) {
    finish_x();
  } else {
#pragma unroll
    for (int k = 0; k < BPL; ++k) {
      const int jb = l + LPR * k;
      const bool in = jb < nbw;
      const int jc = in ? jb : 0;
      if constexpr (PROK != 0) {
        const uint4* v = reinterpret_cast<const uint4*>(xs_lds) + (size_t)((pro_attn(PROK) ? 0 : jb0) + jc) * 4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint4 t = v[i];
          xp[k][4 * i + 0] = t.x;
          xp[k][4 * i + 1] = t.y;
          xp[k][4 * i + 2] = t.z;
          xp[k][4 * i + 3] = t.w;
        }
      } else {
        load_x16(xh, jb0 + jc, xp[k]);
      }
      if constexpr (XLO) load_x16(xl, jb0 + jc, xq[k]);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        xp[k][i] = in ? xp[k][i] : 0u;
        if constexpr (XLO) xq[k][i] = in ? xq[k][i] : 0u;
      }
      float xs = xsum16(xp[k]);
      if constexpr (XLO) xs += xsum16(xq[k]);
      xs8[k] = -8.f * xs;
    }
  }

  if constexpr (NB == 1) {
    if constexpr (PRE == 0) issue_rows(0);
    dot_rows(0);
  } else {
    if constexpr (PRE < LB) {
#pragma unroll
      for (int b = PRE; b < LB; ++b) issue_rows(b * RB);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      if (b + LB < NB) {
        issue_rows((b + LB) * RB);
        __builtin_amdgcn_sched_barrier(0);
      }
      dot_rows(b * RB);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  E4B_TRACE_MARK(2);
  float v = reduce_rows<LPR, R>(acc);
  const int r = l / SPAN;  // this lane now holds slot r of the group
  if constexpr (KW == 4) {
    // fold the four column quarters through LDS; wave 0 finishes
    if ((l % SPAN) == 0) part[wave * SLOTS + g * R + r] = v;
    lds_sync();
    if (wave != 0) return;
    const int sl = g * R + r;
    v = (part[sl] + part[SLOTS + sl]) + (part[2 * SLOTS + sl] + part[3 * SLOTS + sl]);
  }
  E4B_TRACE_MARK(3);
  if (!live) return;
  if constexpr (EPI == EPI_GEGLU) {
    const float up = __shfl_xor(v, SPAN, 64);
    const int64_t u = slot0 / 2 + r / 2;
    if ((l % (2 * SPAN)) == 0 && u < o.ff) o.yh[u] = f2h(gelu_tanh(v) * up);
  } else {
    const int64_t row = slot0 + r;
    if ((l % SPAN) == 0 && row < W.rows) {
      if constexpr (EPI == EPI_F32) o.y[(int64_t)kslice * W.rows + row] = v;
      if constexpr (EPI == EPI_GELU_MUL) o.yh[row] = f2h(gelu_tanh(v) * mulv);
    }
  }
}

// ---- launch configuration -----------------------------------------------------
struct Cfg {
  int lpr, bpl, r, kw;
  int nwv = 4;  // waves per workgroup
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
inline Cfg pick(int nbk, int64_t units, int epi, bool pro, int ks = 1, bool attn = false) {
  Cfg c;
  c.kw = (!pro && nbk >= 256 && nbk % 4 == 0) ? 4 : 1;
  pick_lanes(nbk / c.kw, &c.lpr, &c.bpl, c.kw == 4);
  const int G = 64 / c.lpr;
  int r = c.bpl == 1 ? 8 : c.bpl == 2 ? 4 : c.bpl <= 4 ? 2 : 1;
  // the fused-prologue GeGLU reads the prologue's vectors once per
  // workgroup: 64 rows per workgroup (8 waves x 8 rows, 512 workgroups)
  // halve that on-chip traffic against 4-wave workgroups of 8 rows
  if (pro && epi == EPI_GEGLU && c.lpr == 64 && c.bpl == 1 && c.kw == 1 && units >= 16 * 4 * 256) r = E4B_TUNE_GEGLU_R;
  if (r > c.lpr) r = c.lpr;
  const int rmin = (epi == EPI_GEGLU) ? 2 : 1;
  const int per_wg = (c.kw == 1 ? 4 : 1) * G;
  // measured on MI355X at the E4B shapes: 256 workgroups (128 with the fused
  // norm prologue, which every workgroup repeats; 256 with the attention
  // prologue, whose per-workgroup partial reads favour short tiles; 512 for
  // the column-split down projection) keep enough loads in flight
  const int64_t min_wgs = attn ? E4B_TUNE_ATTN_MINWGS : pro ? E4B_TUNE_PRO_MINWGS : c.kw == 4 ? 512 : 256;
  while (r > rmin && ks * ((units + per_wg * r - 1) / (per_wg * r)) < min_wgs) r >>= 1;
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
  ProArgs pa;
  hipStream_t st;
};

template <int LPR, int BPL, int R, int KW, bool XLO, int EPI, int PROK, int NA = 1, int NWV = 4, int NB = 1,
          int PRE = 1, int LB = 1>
void launch(const Launch& L) {
  constexpr int G = 64 / LPR;
  const int64_t ntiles = (L.units + G * R - 1) / (G * R);
  const int64_t wgs = KW == 1 ? (ntiles + NWV - 1) / NWV : ntiles;  // one tile per wave
  // the leading scalar arguments (Q40_LEAD_PARAMS); k_q40.hip checks the
  // packed shape fields
  const void *p0 = nullptr, *p1 = nullptr, *p2 = nullptr, *p3 = nullptr;
  if constexpr (PROK > 0) {
    p0 = L.pa.hin; p1 = L.pa.a; p2 = L.pa.w1; p3 = L.pa.w2;
  } else if constexpr (pro_attn(PROK)) {
    p0 = L.pa.params; p1 = L.pa.part_ml; p2 = L.pa.part_o;
    p3 = (const void*)(uintptr_t)((uint64_t)(uint32_t)L.pa.gch |
                                  (uint64_t)(uint32_t)(L.pa.window > 0 ? 0 : L.pa.kv_idx) << 32);
  } else if constexpr (PROK == kProTail) {
    p0 = L.pa.hin; p1 = L.pa.a; p2 = L.pa.a2; p3 = L.pa.w2;
  } else if constexpr (PROK == 0) {
    p0 = L.xh; p1 = L.xl;
  }
  const uint32_t dims = (uint32_t)L.W.nb | (uint32_t)L.nbk << 16;
  if constexpr (NB == 1)
    hipLaunchKernelGGL((k_q40<LPR, BPL, R, KW, XLO, EPI, PROK, NA, NWV>), dim3((unsigned)wgs, (unsigned)L.ks),
                       dim3(64 * NWV), 0, L.st, L.W.nib, L.W.sc, p0, p1, p2, p3, dims, (uint32_t)L.units, L.W,
                       L.xh, L.xl, L.o, L.pa);
  else
    hipLaunchKernelGGL((k_q40b<LPR, BPL, R, KW, XLO, EPI, PROK, NA, NWV, NB, PRE, LB>), dim3((unsigned)wgs, (unsigned)L.ks),
                       dim3(64 * NWV), 0, L.st, L.W.nib, L.W.sc, p0, p1, p2, p3, dims, (uint32_t)L.units, L.W,
                       L.xh, L.xl, L.o, L.pa);
}

template <int LPR, int BPL, int KW, bool XLO, int EPI, int PROK, int NA = 1>
bool launch_r(const Cfg& c, const Launch& L) {
  switch (c.r) {
    case 1:
      if constexpr (EPI != EPI_GEGLU) {
        launch<LPR, BPL, 1, KW, XLO, EPI, PROK, NA>(L);
        return true;
      }
      return false;
    case 2:
      if constexpr (pro_attn(PROK)) {
        launch<LPR, BPL, 2, KW, XLO, EPI, PROK, NA, 4, E4B_TUNE_O_NB, E4B_TUNE_O_PRE, E4B_TUNE_O_LB>(L);
      } else {
        launch<LPR, BPL, 2, KW, XLO, EPI, PROK, NA>(L);
      }
      return true;
    case 4:
      if constexpr (PROK > 0 && EPI == EPI_F32) {
        launch<LPR, BPL, 4, KW, XLO, EPI, PROK, NA, 4, E4B_TUNE_QKV_NB, E4B_TUNE_QKV_PRE, E4B_TUNE_QKV_LB>(L);
      } else {
        launch<LPR, BPL, 4, KW, XLO, EPI, PROK, NA>(L);
      }
      return true;
    case 8:
      if constexpr (BPL == 1 && KW == 1 && LPR == 64 && EPI == EPI_GEGLU && PROK > 0 && E4B_TUNE_GEGLU_R == 8) {
        // the fused-prologue GeGLU: 8-wave workgroups, 4 batches of 2 rows,
        // one batch requested ahead (measured on MI355X at the E4B shape:
        // 825 tok/s against 821 for 4-wave workgroups of 16 rows in 8
        // batches and 797-808 for the other 8-row shapes tried)
        launch<LPR, BPL, 8, KW, XLO, EPI, PROK, NA, E4B_TUNE_GEGLU_NWV, E4B_TUNE_GEGLU_NB, E4B_TUNE_GEGLU_PRE,
               E4B_TUNE_GEGLU_LB>(L);
      } else if constexpr (KW == 4 && !XLO && EPI == EPI_F32 && PROK == 0) {
        // the column-split down projection: the whole tile requested up
        // front, multiplied in 2 batches of 4 rows (measured on MI355X at
        // the E4B shape: 798 tok/s against 796 with one batch ahead, 788
        // unbatched, 791-793 with 4 batches; batching the qkv and o tiles
        // measured slower)
        launch<LPR, BPL, 8, KW, XLO, EPI, PROK, NA, 4, E4B_TUNE_KW4_NB, E4B_TUNE_KW4_PRE, E4B_TUNE_KW4_LB>(L);
      } else if constexpr (KW == 1 && EPI == EPI_F32 && PROK == 0 && LPR == 64 && BPL == 1) {
        // the plain f32 GEMV of 64-block rows (c0, the PLE model projection)
        launch<LPR, BPL, 8, KW, XLO, EPI, PROK, NA, E4B_TUNE_PLAIN_NWV, E4B_TUNE_PLAIN_NB, E4B_TUNE_PLAIN_PRE,
               E4B_TUNE_PLAIN_LB>(L);
      } else {
        launch<LPR, BPL, 8, KW, XLO, EPI, PROK, NA>(L);
      }
      return true;
    case 16:
      if constexpr (BPL == 1 && KW == 1 && LPR == 64 && EPI == EPI_GEGLU && PROK > 0) {
        // the fused-prologue GeGLU with 16 rows per wave (the 8-row shape
        // above measured faster)
        launch<LPR, BPL, 16, KW, XLO, EPI, PROK, NA, E4B_TUNE_GEGLU_NWV, E4B_TUNE_GEGLU_NB, E4B_TUNE_GEGLU_PRE,
               E4B_TUNE_GEGLU_LB>(L);
        return true;
      }
      return false;
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

// attention-combine prologue: 1024 or 2048 columns a slice, one block per
// lane.  (Reading 16 chunks up front for layers that allocate more than 8
// measured slower than a second pass: the loads cannot be trimmed to the
// live chunks without waiting for the position first.)
inline bool launch_pro_attn(const Cfg& c, const Launch& L) {
  if (c.bpl != 1) return false;
  const int hd = L.pa.head_dim ? L.pa.head_dim : 256;
  if (L.ks == 1) {
    // all 8 heads of 256 dims
    if (c.lpr != 64 || hd != 256) return false;
    // 16 chunks (a sliding layer in 32-position chunks) in one pass
    if (L.pa.gch == 16) return launch_r<64, 1, 1, false, EPI_F32, kProAttn, 16>(c, L);
    return launch_r<64, 1, 1, false, EPI_F32, kProAttn>(c, L);
  }
  if (hd == 256) {
    // column slices of 4 heads of 256 (1024 columns: 32 lanes per row)
    if (c.lpr != 32) return false;
#ifndef E4B_TUNE_ATTN_U16_ANY
    if (L.pa.gch == 16 && L.pa.chunk_shift == 5) return launch_r<32, 1, 1, false, EPI_F32, kProAttn2, 16>(c, L);
#else
    if (L.pa.gch == 16) return launch_r<32, 1, 1, false, EPI_F32, kProAttn2, 16>(c, L);
#endif
    return launch_r<32, 1, 1, false, EPI_F32, kProAttn2>(c, L);
  }
  // column slices of 4 heads of 512 (2048 columns)
  if (c.lpr != 64) return false;
  return launch_r<64, 1, 1, false, EPI_F32, kProAttn4w>(c, L);
}

// A4B boundary prologue (the x vector comes from LDS): lane splits
// (8|16|32|64, 1) and (32, 2|3), 1, 2 or 4 rows per lane group
template <int LPR, int BPL>
bool launch_pro_tail_r(const Cfg& c, const Launch& L) {
  switch (c.r) {
    case 1: launch<LPR, BPL, 1, 1, false, EPI_F32, kProTail>(L); return true;
    case 2: launch<LPR, BPL, 2, 1, false, EPI_F32, kProTail>(L); return true;
    case 4: launch<LPR, BPL, 4, 1, false, EPI_F32, kProTail>(L); return true;
#ifdef E4B_TUNE_TAIL_R8
    case 8: launch<LPR, BPL, 8, 1, false, EPI_F32, kProTail>(L); return true;
#endif
  }
  return false;
}
inline bool launch_pro_tail(const Cfg& c, const Launch& L) {
  if (c.kw != 1 || c.nwv != 4) return false;
  if (c.bpl == 1) {
    switch (c.lpr) {
      case 8: return launch_pro_tail_r<8, 1>(c, L);
      case 16: return launch_pro_tail_r<16, 1>(c, L);
      case 32: return launch_pro_tail_r<32, 1>(c, L);
      case 64: return launch_pro_tail_r<64, 1>(c, L);
    }
    return false;
  }
  if (c.lpr != 32) return false;
  if (c.bpl == 2) return launch_pro_tail_r<32, 2>(c, L);
  if (c.bpl == 3) return launch_pro_tail_r<32, 3>(c, L);
  return false;
}

// fused prologue: H = 256 PROK, one block per lane (LPR = H / 32); NA
// partial vectors in the residual input
template <int EPI, int NA = 1>
bool launch_pro(const Cfg& c, const Launch& L) {
  if (c.bpl != 1 || c.nwv != 4) return false;
  switch (c.lpr) {
    case 8: return launch_r<8, 1, 1, false, EPI, 1, NA>(c, L);
    case 16: return launch_r<16, 1, 1, false, EPI, 2, NA>(c, L);
    case 32: return launch_r<32, 1, 1, false, EPI, 4, NA>(c, L);
    case 64: return launch_r<64, 1, 1, false, EPI, 8, NA>(c, L);
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
