// k_prefill.hip -- the per-token kernels of the batched prefill: M prompt
// tokens per launch, the same per-token arithmetic as the decode step
// (src/engine-a4b.js:465-585 encodeLayerPre: "per-token math identical to
// encodeLayer").  The GEMMs between them are k_gemm.hip.
//
//   k_embed_rows      token rows of the Q6_K table * sqrt(H), plus the
//                     f16 hi/lo pair for the PLE model projection
//                     (kernels/q6k.wgsl:37-73 per token)
//   k_ple_prep_rows   per-layer inputs of every token (kernels/pleprep.wgsl:15-46)
//   k_resnorm_rows    residual + RMSNorm, one workgroup per token
//                     (kernels/rmsacc3.wgsl:36-53, kernels/a4btail.wgsl:26-71)
//   k_headprep_rows   q/k head-RMS + RoPE, v RMS, K/V cache write at the
//                     token's slot (kernels/headprep.wgsl:19-87 per token)
//   k_attn_prefill    causal softmax attention of the chunk's queries over
//                     the cache (kernels/attnf32.wgsl:21-105 /
//                     kernels/attnos.wgsl:22-98 per query) on the matrix
//                     cores
#include <algorithm>

#include "../../include/e4b.h"
#include "attn_prep.h"
#include "kernels.h"
#include "step.h"
#include "util.h"

namespace {

constexpr int kMaxPer = 16;  // elements per thread of the row kernels (H <= 4096)

// h[m] = E[ids[m]] * mult (f32) and its split hi = f16(h), lo = f16(h - hi)
// into xhl[0][m] / xhl[1][m]; the expression order is k_embed's
__global__ __launch_bounds__(256) void k_embed_rows(Q6Mat E, const uint32_t* __restrict__ ids, int M, float mult,
                                                    float* __restrict__ h, uint16_t* __restrict__ xhl) {
  const int m = blockIdx.y;
  const int H = E.nseg * 32;
  const uint32_t tok = ids[m];  // range-checked by the host
  for (int s = blockIdx.x * 256 + threadIdx.x; s < E.nseg; s += gridDim.x * 256) {
    const uint4 a = E.qa[(int64_t)tok * E.nseg + s];
    const uint2 b = E.qb[(int64_t)tok * E.nseg + s];
    const float d = h2f(E.d[(int64_t)tok * (E.nseg / 8) + (s >> 3)]);
    const int8_t* scg = E.sc + (int64_t)tok * (E.nseg * 2) + 2 * s;
    uint32_t pr[8];
#pragma unroll
    for (int gi = 0; gi < 2; ++gi) {
      q6_pairs(gi ? a.z : a.x, gi ? a.w : a.y, gi ? b.y : b.x, pr);
      const float ds = d * (float)scg[gi];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int e = 32 * s + 16 * gi + 2 * i + u;
          const float v = ds * (float)((int)((pr[i] >> (16 * u)) & 0x3f) - 32) * mult;
          const int64_t o = (int64_t)m * H + e;
          h[o] = v;
          const _Float16 hi = (_Float16)v;
          xhl[o] = __builtin_bit_cast(uint16_t, hi);
          xhl[(int64_t)M * H + o] = __builtin_bit_cast(uint16_t, (_Float16)(v - (float)hi));
        }
      }
    }
  }
}

// ggml Q6_K element e (0..255) of one superblock (kernels/q6k.wgsl:44-71 order)
DEV float q6k_elem(const uint8_t* blk, int e) {
  const int half = e >> 7, r = e & 127, quad = r >> 5, l = r & 31;
  const uint8_t* ql = blk + 64 * half;
  const uint8_t* qh = blk + 128 + 32 * half;
  int q = (quad & 1) ? ql[l + 32] : ql[l];
  q = (quad >= 2) ? (q >> 4) : (q & 15);
  q |= ((qh[l] >> (2 * quad)) & 3) << 4;
  const int is = 8 * half + (l >> 4) + 2 * quad;
  const float d = h2f((uint16_t)(blk[208] | (blk[209] << 8)));
  return d * (float)(int8_t)blk[192 + is] * (float)(q - 32);
}

// block (b, m): ple[m][b] = (rms(proj_m,b * H^-1/2) * w_pn + table_row_b(ids[m])
// * sqrt(PD)) * 2^-1/2, PD = 256; proj holds two partial products (the hi
// and lo halves of the input) that are summed first
__global__ __launch_bounds__(256) void k_ple_prep_rows(const float* __restrict__ proj, int64_t slice,
                                                       const uint8_t* __restrict__ table,
                                                       const float* __restrict__ w_pn,
                                                       const uint32_t* __restrict__ ids, int L, float proj_scale,
                                                       float* __restrict__ ple, float eps) {
  __shared__ float red[4];
  const int b = blockIdx.x, m = blockIdx.y, t = threadIdx.x;
  const int64_t o = (int64_t)m * L * 256 + b * 256 + t;
  const float pv = (proj[o] + proj[slice + o]) * proj_scale;
  const float wn = w_pn[t];
  const uint8_t* blk = table + ((int64_t)ids[m] * L + b) * 210;
  const float idv = q6k_elem(blk, t) * 16.0f;  // sqrt(PD), PD = 256
  const float inv = rms_inv(block_sum(pv * pv, red), 256, eps);
  ple[o] = (pv * inv * wn + idv) * 0.70710678118654752f;
}

// N contiguous floats at p (aligned to min(N, 4) floats) with the widest loads
template <int N>
DEV void ld_row(const float* p, float (&v)[N]) {
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
template <int N>
DEV void st_row(float* p, const float (&v)[N]) {
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
// N f16 values (N >= 2: 4-byte aligned) in one store per 8
template <int N>
DEV void st_halves(uint16_t* p, const uint16_t (&v)[N]) {
  if constexpr (N == 1) {
    p[0] = v[0];
  } else {
    uint32_t w[N / 2];
#pragma unroll
    for (int i = 0; i < N / 2; ++i) w[i] = (uint32_t)v[2 * i] | ((uint32_t)v[2 * i + 1] << 16);
    if constexpr (N == 2) {
      *reinterpret_cast<uint32_t*>(p) = w[0];
    } else if constexpr (N == 4) {
      *reinterpret_cast<uint2*>(p) = make_uint2(w[0], w[1]);
    } else {
#pragma unroll
      for (int q = 0; q < N / 8; ++q)
        reinterpret_cast<uint4*>(p)[q] = make_uint4(w[4 * q], w[4 * q + 1], w[4 * q + 2], w[4 * q + 3]);
    }
  }
}

// one workgroup per token m:
//   h = (h + rms(a) * w1) * scale, a = sum of na partial slices (a may be null)
//   w2 != null: x = f16(rms(h) * w2), else x = f16(h); with xlo the value is
//   stored as the pair x = f16(y), xlo = f16(y - x), x + xlo within
//   max(2^-22 |y|, 2^-25) of y (the lm-head input)
// H = 256 PER; thread t owns elements [PER t, PER t + PER).  NAM = 0: no
// residual input; else na <= NAM slices, all requested before the first use
// (slice indices past na repeat the last one and are not added), summed in
// slice order.
template <int PER, int NAM>
__global__ __launch_bounds__(256) void k_resnorm_rows(float* __restrict__ h, const float* __restrict__ a, int na,
                                                      int64_t slice, const float* __restrict__ w1, float scale,
                                                      const float* __restrict__ w2, uint16_t* __restrict__ x,
                                                      uint16_t* __restrict__ xlo, int H, float eps) {
  __shared__ float red[4];
  const int m = blockIdx.x;
  const int i0 = threadIdx.x * PER;
  const int64_t row = (int64_t)m * H + i0;
  float hv[PER];
  ld_row<PER>(h + row, hv);
  float av[NAM > 0 ? NAM : 1][PER], w1v[PER];
  if constexpr (NAM > 0) {
#pragma unroll
    for (int z = 0; z < NAM; ++z) ld_row<PER>(a + (int64_t)min(z, na - 1) * slice + row, av[z]);
    ld_row<PER>(w1 + i0, w1v);
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      float s = av[0][k];
#pragma unroll
      for (int z = 1; z < NAM; ++z)
        if (z < na) s += av[z][k];
      av[0][k] = s;
      ss = fmaf(s, s, ss);
    }
    const float inv1 = rms_inv(block_sum(ss, red), H, eps);
#pragma unroll
    for (int k = 0; k < PER; ++k) hv[k] = hv[k] + av[0][k] * inv1 * w1v[k];
  }
  float s2 = 0.f;
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    hv[k] *= scale;
    s2 = fmaf(hv[k], hv[k], s2);
  }
  st_row<PER>(h + row, hv);
  uint16_t xv[PER], xl[PER];
  if (w2) {
    float w2v[PER];
    ld_row<PER>(w2 + i0, w2v);
    const float inv2 = rms_inv(block_sum(s2, red), H, eps);
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const float y = hv[k] * inv2 * w2v[k];
      const _Float16 yh = (_Float16)y;
      xv[k] = __builtin_bit_cast(uint16_t, yh);
      xl[k] = __builtin_bit_cast(uint16_t, (_Float16)(y - (float)yh));
    }
  } else {
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const _Float16 yh = (_Float16)hv[k];
      xv[k] = __builtin_bit_cast(uint16_t, yh);
      xl[k] = __builtin_bit_cast(uint16_t, (_Float16)(hv[k] - (float)yh));
    }
  }
  st_halves<PER>(x + row, xv);
  if (xlo) st_halves<PER>(xlo + row, xl);
}

// y[m][n] = f16(gelu(sum of ks partial slices) * mul[m mul_ld + n]) for the
// PLE gate of every token (kernels/plegatemv.wgsl:20-60 per token)
__global__ __launch_bounds__(256) void k_gelu_mul_rows(const float* __restrict__ part, int ks, int64_t slice,
                                                       int64_t n, const float* __restrict__ mul, int64_t mul_ld,
                                                       uint16_t* __restrict__ y) {
  const int m = blockIdx.y;
  for (int64_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    float v = part[(int64_t)m * n + i];
    for (int z = 1; z < ks; ++z) v += part[z * slice + (int64_t)m * n + i];
    y[(int64_t)m * n + i] = f2h(gelu_tanh(v) * mul[(int64_t)m * mul_ld + i]);
  }
}

// one wave per (head row hh, token m): the qkv row is the sum of ks partial
// slices; q heads -> q[m][hh] (f32), k heads -> key cache, v heads -> value
// cache, at the slot of position p0 + m (ring slot for a sliding layer)
__global__ __launch_bounds__(64) void k_headprep_rows(const float* __restrict__ qkv, int ks, int64_t slice,
                                                      const float* __restrict__ qw, const float* __restrict__ kw,
                                                      const float* __restrict__ inv_freq, int angles, uint16_t* kc,
                                                      uint16_t* vc, int slots, int ring, uint32_t p0,
                                                      float* __restrict__ q, int qh, int kvh, float eps) {
  const int hh = blockIdx.x, m = blockIdx.y, lane = threadIdx.x;
  const int rows = (qh + 2 * kvh) * 256;
  const float* src = qkv + (int64_t)m * rows + hh * 256 + 4 * lane;
  float4 v = *reinterpret_cast<const float4*>(src);
  for (int z = 1; z < ks; ++z) {
    const float4 t = *reinterpret_cast<const float4*>(src + z * slice);
    v.x += t.x;
    v.y += t.y;
    v.z += t.z;
    v.w += t.w;
  }
  float x[4] = {v.x, v.y, v.z, v.w};
  const bool isq = hh < qh, isk = !isq && hh < qh + kvh;
  const float* wsrc = isq ? qw : kw;
  const float4 wv = *reinterpret_cast<const float4*>(wsrc + 4 * lane);
  const float w[4] = {wv.x, wv.y, wv.z, wv.w};
  const float2 cs[4] = {};
  const uint32_t pos = p0 + (uint32_t)m;
  prep_head_regs(x, w, isq || isk, cs, false, inv_freq, angles, eps, (float)pos, isq || isk);
  if (isq) {
    *reinterpret_cast<float4*>(q + ((int64_t)m * qh + hh) * 256 + 4 * lane) = make_float4(x[0], x[1], x[2], x[3]);
    return;
  }
  const int g = isk ? hh - qh : hh - qh - kvh;
  const int64_t slot = ring ? (int64_t)(pos % (uint32_t)slots) : (int64_t)pos;
  uint16_t* dst = (isk ? kc : vc) + ((int64_t)g * slots + slot) * 256 + 4 * lane;
  *reinterpret_cast<uint2*>(dst) = make_uint2((uint32_t)f2h(x[0]) | ((uint32_t)f2h(x[1]) << 16),
                                             (uint32_t)f2h(x[2]) | ((uint32_t)f2h(x[3]) << 16));
}

// ---- causal attention of a prefill chunk on the matrix cores ----------------
//
// Workgroup (KV group g, tile of 16 QS queries, key split s), GQA q heads
// per KV group and QS = 4 / GQA: wave w takes q head GQA g + w % GQA for
// queries 16 (w / GQA) .. + 15 of the tile, so the four waves share each
// K/V tile staged in LDS.  Key tiles of 32 positions walk the union of the
// tile's windows; per query
// the live keys are (qp - W, qp] (sliding) or [0, qp] (global), scale 1.0.
// With ns > 1 splits the union is cut into runs of kspl keys (a multiple of
// the tile), one workgroup each, which write unnormalised partials (O, max,
// sum) that k_attn_prefill_combine merges by log-sum-exp: the causal tiles
// late in the chunk no longer serialise on one CU.
//
// v_mfma_f32_16x16x32_f16 (lane l: A[l % 16][8 (l / 16) + t], B[8 (l / 16) +
// t][l % 16], D[4 (l / 16) + r][l % 16]):
//   S^T (16 keys x 16 queries) = K . Q^T over 8 steps of 32 dims; Q (f32) is
//   an f16 pair hi + lo (within max(2^-22 |q|, 2^-25) of q), K is f16, so two MFMAs give q.k to ~2^-22.
//   After the online-softmax update each lane holds P^T for its query
//   (column l % 16) and 8 keys: 4 (l / 16) + r of sub-tile 0 and 16 + 4 (l /
//   16) + r of sub-tile 1 -- exactly a B operand of a 32-key MFMA when the A
//   operand (V^T, 16 dims x 32 keys, read from a transposed V tile in LDS)
//   uses the same key order.  O^T (dims x queries) accumulates P_hi and
//   P_lo (P = P_hi + P_lo) against V in f32, so every product is as exact
//   as the decode kernel's f32 arithmetic.
typedef _Float16 h8v __attribute__((ext_vector_type(8)));
typedef float f4v __attribute__((ext_vector_type(4)));

constexpr int kKT = 32;            // keys per tile
// halfs per K row in LDS: the head dim + 8
constexpr int kVtStride = kKT + 8; // halfs per transposed V row in LDS
constexpr int kPfAttnMaxSplits = 8;  // key splits per query tile
constexpr int kPfAttnMinSplit = 128; // keys per split at least (a multiple of kKT)

DEV void split8(const float (&v)[8], h8v& hi, h8v& lo) {
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const _Float16 a = (_Float16)v[t];
    hi[t] = a;
    lo[t] = (_Float16)(v[t] - (float)a);
  }
}

// Head dim 512 (GQA 8, the A4B full layers): blockIdx.x also picks one of
// the two sets of 4 heads and one of the two 256-dim halves of V, so a
// workgroup holds 4 heads' O for 256 dims; both V halves compute the scores.
template <int GQA, int HD = 256>
__global__ __launch_bounds__(256) void k_attn_prefill(PrefillAttnArgs A) {
  static_assert((HD == 256 && GQA <= 4) || (HD == 512 && GQA == 8), "head dim 256 (GQA <= 4) or 512 (GQA 8)");
  constexpr int QS = GQA >= 4 ? 1 : 4 / GQA;  // 16-query sub-tiles per workgroup
  constexpr int NVH = HD / 256;               // 256-dim V halves
  constexpr int NHS = GQA > 4 ? GQA / 4 : 1;  // sets of 4 heads
  constexpr int WG = GQA > 4 ? GQA : 4;       // partial units per (group, tile, split)
  constexpr int KST = HD + 8;                 // halfs per K row in LDS
  __shared__ __align__(16) uint16_t ks[kKT * KST];
  __shared__ __align__(16) uint16_t vt[256 * kVtStride];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = blockIdx.x / (NHS * NVH), hs = (blockIdx.x / NVH) % NHS, vh = blockIdx.x % NVH;
  const int t0 = blockIdx.y * 16 * QS, q0 = t0 + 16 * (GQA >= 4 ? 0 : wave / GQA);
  const int hg = GQA >= 4 ? 4 * hs + wave : wave % GQA;  // head within the group
  const int wid = GQA >= 4 ? hg : wave;                  // partial unit of this wave
  const int head = GQA * g + hg;
  const int j = lane & 15, qq = lane >> 4;
  const int M = A.M;
  const int qi = q0 + j;                      // this lane's query (column)
  const int qp = (int)A.p0 + min(qi, M - 1);  // its position
  // key range of the workgroup's queries t0 .. t0 + 16 QS - 1
  const int P0 = (int)A.p0 + t0, P1 = (int)A.p0 + min(t0 + 16 * QS, M) - 1;
  const int W = A.window;
  const int klo = W > 0 ? max(0, P0 - W + 1) : 0;
  const uint16_t* kc = A.kc + (int64_t)g * A.slots * HD;
  const uint16_t* vc = A.vc + (int64_t)g * A.slots * HD + 256 * vh;
  const int NS = gridDim.z, sp = blockIdx.z;
  const int kstart = NS > 1 ? klo + sp * A.kspl : klo;
  if (kstart > P1) return;  // this tile needs fewer splits (uniform per workgroup)
  const int kend = NS > 1 ? min(P1, kstart + A.kspl - 1) : P1;

  // Q^T as the B operand: step s covers dims 32 s + 8 qq .. + 8
  constexpr int QST = HD / 32;  // score steps
  h8v qh_[QST], ql_[QST];
  {
    const float* qrow = A.q + ((int64_t)min(qi, M - 1) * A.qh + head) * HD;
#pragma unroll
    for (int s = 0; s < QST; ++s) {
      const float4 a = *reinterpret_cast<const float4*>(qrow + 32 * s + 8 * qq);
      const float4 b = *reinterpret_cast<const float4*>(qrow + 32 * s + 8 * qq + 4);
      const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
      split8(v, qh_[s], ql_[s]);
    }
  }
  f4v o[16];
#pragma unroll
  for (int dt = 0; dt < 16; ++dt) o[dt] = f4v{0.f, 0.f, 0.f, 0.f};
  float mrun = -3.0e38f, lrun = 0.f;

  for (int kb = kstart; kb <= kend; kb += kKT) {
    // stage keys kb .. kb + 31 (rows past P1 repeat row P1; they are masked)
    lds_sync();
    {
      const int t = threadIdx.x;
      // K: 8 threads per row, HD / 8 halfs each
      const int kr = t >> 3, part = t & 7;
      const int kp = min(kb + kr, P1);
      const int64_t sk = W > 0 ? (int64_t)(kp % A.slots) : (int64_t)kp;
      const uint4* srck = reinterpret_cast<const uint4*>(kc + sk * HD + (HD / 8) * part);
      uint4* dstk = reinterpret_cast<uint4*>(ks + kr * KST + (HD / 8) * part);
#pragma unroll
      for (int i = 0; i < HD / 64; ++i) dstk[i] = srck[i];
      // V: thread (key pair kp2, dim chunk dc) transposes 2 keys x 16 dims
      const int kp2 = t >> 4, dc = t & 15;
      const int pa = min(kb + 2 * kp2, P1), pb = min(kb + 2 * kp2 + 1, P1);
      const int64_t sa = W > 0 ? (int64_t)(pa % A.slots) : (int64_t)pa;
      const int64_t sb = W > 0 ? (int64_t)(pb % A.slots) : (int64_t)pb;
      const uint4* va = reinterpret_cast<const uint4*>(vc + sa * HD + 16 * dc);
      const uint4* vb = reinterpret_cast<const uint4*>(vc + sb * HD + 16 * dc);
      const uint4 a0 = va[0], a1 = va[1], b0 = vb[0], b1 = vb[1];
      const uint32_t aw[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
      const uint32_t bw[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t lo2 = (aw[i] & 0xffffu) | (bw[i] << 16);
        const uint32_t hi2 = (aw[i] >> 16) | (bw[i] & 0xffff0000u);
        *reinterpret_cast<uint32_t*>(vt + (16 * dc + 2 * i) * kVtStride + 2 * kp2) = lo2;
        *reinterpret_cast<uint32_t*>(vt + (16 * dc + 2 * i + 1) * kVtStride + 2 * kp2) = hi2;
      }
    }
    lds_sync();
    // S^T for the two 16-key sub-tiles
    f4v sc[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      f4v d = {0.f, 0.f, 0.f, 0.f};
      const uint16_t* krow = ks + (16 * kt + j) * KST + 8 * qq;
#pragma unroll
      for (int s = 0; s < QST; ++s) {
        const h8v ka = __builtin_bit_cast(h8v, *reinterpret_cast<const uint4*>(krow + 32 * s));
        d = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qh_[s], d, 0, 0, 0);
        d = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, ql_[s], d, 0, 0, 0);
      }
      sc[kt] = d;
    }
    // mask, online softmax (per query column; its 32 scores sit in the four
    // lanes j, j + 16, j + 32, j + 48)
    float p[8];
    float mx = -3.0e38f;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int kp = kb + 16 * kt + 4 * qq + r;
        const bool live = qi < M && kp <= qp && kp <= P1 && (W == 0 || kp > qp - W);
        p[4 * kt + r] = live ? sc[kt][r] : -3.0e38f;
        mx = fmaxf(mx, p[4 * kt + r]);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float mnew = fmaxf(mrun, mx);
    const float alpha = __expf(mrun - mnew);
    float ps = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      p[i] = p[i] > -1.0e38f ? __expf(p[i] - mnew) : 0.f;
      ps += p[i];
    }
    ps += __shfl_xor(ps, 16, 64);
    ps += __shfl_xor(ps, 32, 64);
    lrun = lrun * alpha + ps;
    mrun = mnew;
#pragma unroll
    for (int dt = 0; dt < 16; ++dt) o[dt] *= alpha;
    h8v phi, plo;
    split8(p, phi, plo);
    // O^T += V^T P^T: A = V^T rows 16 dt + j, keys 4 qq .. +3 and 16 + 4 qq .. +3
#pragma unroll
    for (int dt = 0; dt < 16; ++dt) {
      const uint16_t* vrow = vt + (16 * dt + j) * kVtStride;
      const uint2 va = *reinterpret_cast<const uint2*>(vrow + 4 * qq);
      const uint2 vb = *reinterpret_cast<const uint2*>(vrow + 16 + 4 * qq);
      const h8v vv = __builtin_bit_cast(h8v, make_uint4(va.x, va.y, vb.x, vb.y));
      o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vv, phi, o[dt], 0, 0, 0);
      o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vv, plo, o[dt], 0, 0, 0);
    }
  }
  if (qi >= M) return;
  if (NS > 1) {
    // partials of unit (g, tile, split), wave unit wid, query j: O [HD] (this
    // workgroup's 256 V dims) and (max, sum)
    const int64_t u = ((int64_t)(g * gridDim.y + blockIdx.y) * NS + sp) * WG + wid;
    float* po = A.part + (u * 16 + j) * HD + 256 * vh + 4 * qq;
#pragma unroll
    for (int dt = 0; dt < 16; ++dt)
      *reinterpret_cast<float4*>(po + 16 * dt) = make_float4(o[dt][0], o[dt][1], o[dt][2], o[dt][3]);
    if (qq == 0 && vh == 0) {
      float* ml = A.part + (int64_t)(gridDim.x / (NHS * NVH)) * gridDim.y * NS * WG * 16 * HD;
      *reinterpret_cast<float2*>(ml + (u * 16 + j) * 2) = make_float2(mrun, lrun);
    }
    return;
  }
  const float inv = 1.f / lrun;
  uint16_t* dst = A.out + ((int64_t)qi * A.qh + head) * HD + 256 * vh + 4 * qq;
#pragma unroll
  for (int dt = 0; dt < 16; ++dt) {
    const uint32_t lo2 = (uint32_t)f2h(o[dt][0] * inv) | ((uint32_t)f2h(o[dt][1] * inv) << 16);
    const uint32_t hi2 = (uint32_t)f2h(o[dt][2] * inv) | ((uint32_t)f2h(o[dt][3] * inv) << 16);
    *reinterpret_cast<uint2*>(dst + 16 * dt) = make_uint2(lo2, hi2);
  }
}

// log-sum-exp merge of the key splits of one (head, query): block (h, m),
// thread t = dims 4t .. 4t + 3.  A split in which the query has no live key
// left max -3e38 and sum 0 and drops out (its weight underflows to 0); the
// split that holds the query's own position is always live.
// (HD / 4 threads: thread t = dims 4t .. 4t + 3)
template <int GQA, int HD = 256>
__global__ __launch_bounds__(128) void k_attn_prefill_combine(PrefillAttnArgs A) {
  constexpr int QS = GQA >= 4 ? 1 : 4 / GQA, TQ = 16 * QS, WG = GQA > 4 ? GQA : 4;
  const int h = blockIdx.x, qi = blockIdx.y, t = threadIdx.x;
  const int g = h / GQA, qt = qi / TQ, j = qi & 15;
  const int w = GQA >= 4 ? h % GQA : ((qi % TQ) >> 4) * GQA + h % GQA;
  const int nqt = (A.M + TQ - 1) / TQ;
  const int P0 = (int)A.p0 + TQ * qt, P1 = (int)A.p0 + min(TQ * qt + TQ, A.M) - 1;
  const int klo = A.window > 0 ? max(0, P0 - A.window + 1) : 0;
  const int nspl = (P1 - klo + A.kspl) / A.kspl;  // splits of this tile (<= ns)
  const int64_t u0 = (int64_t)(g * nqt + qt) * A.ns;
  const float* ml = A.part + (int64_t)A.kvh * nqt * A.ns * WG * 16 * HD;
  float m[kPfAttnMaxSplits], l[kPfAttnMaxSplits];
  float4 ov[kPfAttnMaxSplits];
#pragma unroll
  for (int s = 0; s < kPfAttnMaxSplits; ++s) {
    const int64_t u = ((u0 + min(s, nspl - 1)) * WG + w) * 16 + j;
    const float2 v = *reinterpret_cast<const float2*>(ml + u * 2);
    m[s] = v.x;
    l[s] = v.y;
    ov[s] = *reinterpret_cast<const float4*>(A.part + u * HD + 4 * t);
  }
  float M = m[0];
#pragma unroll
  for (int s = 1; s < kPfAttnMaxSplits; ++s)
    if (s < nspl) M = fmaxf(M, m[s]);
  float den = 0.f, a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
  for (int s = 0; s < kPfAttnMaxSplits; ++s) {
    if (s < nspl) {
      const float f = __expf(m[s] - M);
      den = fmaf(l[s], f, den);
      a0 = fmaf(ov[s].x, f, a0);
      a1 = fmaf(ov[s].y, f, a1);
      a2 = fmaf(ov[s].z, f, a2);
      a3 = fmaf(ov[s].w, f, a3);
    }
  }
  const float inv = 1.f / den;
  uint16_t* dst = A.out + ((int64_t)qi * A.qh + h) * HD + 4 * t;
  *reinterpret_cast<uint2*>(dst) = make_uint2((uint32_t)f2h(a0 * inv) | ((uint32_t)f2h(a1 * inv) << 16),
                                             (uint32_t)f2h(a2 * inv) | ((uint32_t)f2h(a3 * inv) << 16));
}

template <int PER>
void launch_resnorm_per(int M, float* h, const float* a, int na, int64_t slice, const float* w1, float scale,
                        const float* w2, uint16_t* x, uint16_t* xlo, int H, float eps, hipStream_t st) {
  const int nam = !a ? 0 : na == 1 ? 1 : na <= 2 ? 2 : na <= 4 ? 4 : 8;
  switch (nam) {
    case 0: hipLaunchKernelGGL((k_resnorm_rows<PER, 0>), dim3(M), dim3(256), 0, st, h, a, na, slice, w1, scale, w2, x, xlo, H, eps); break;
    case 1: hipLaunchKernelGGL((k_resnorm_rows<PER, 1>), dim3(M), dim3(256), 0, st, h, a, na, slice, w1, scale, w2, x, xlo, H, eps); break;
    case 2: hipLaunchKernelGGL((k_resnorm_rows<PER, 2>), dim3(M), dim3(256), 0, st, h, a, na, slice, w1, scale, w2, x, xlo, H, eps); break;
    case 4: hipLaunchKernelGGL((k_resnorm_rows<PER, 4>), dim3(M), dim3(256), 0, st, h, a, na, slice, w1, scale, w2, x, xlo, H, eps); break;
    default: hipLaunchKernelGGL((k_resnorm_rows<PER, 8>), dim3(M), dim3(256), 0, st, h, a, na, slice, w1, scale, w2, x, xlo, H, eps); break;
  }
}

}  // namespace

int launch_embed_rows(const Q6Mat& E, const uint32_t* ids, int M, float mult, float* h, uint16_t* xhl, hipStream_t st) {
  if (M < 1) return e4b_fail(E4B_EINVAL, "embed rows: M = %d", M);
  hipLaunchKernelGGL(k_embed_rows, dim3((E.nseg + 255) / 256, M), dim3(256), 0, st, E, ids, M, mult, h, xhl);
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}

int launch_ple_prep_rows(const float* proj, int64_t slice, const uint8_t* table, const float* w_pn,
                         const uint32_t* ids, int M, int L, float proj_scale, float* ple, float eps, hipStream_t st) {
  hipLaunchKernelGGL(k_ple_prep_rows, dim3(L, M), dim3(256), 0, st, proj, slice, table, w_pn, ids, L, proj_scale, ple,
                     eps);
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}

int launch_gelu_mul_rows(const float* part, int ks, int64_t slice, int M, int64_t n, const float* mul, int64_t mul_ld,
                         uint16_t* y, hipStream_t st) {
  const unsigned gx = (unsigned)((n + 255) / 256);
  hipLaunchKernelGGL(k_gelu_mul_rows, dim3(gx, M), dim3(256), 0, st, part, ks, slice, n, mul, mul_ld, y);
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}

int launch_resnorm_rows(int M, float* h, const float* a, int na, int64_t slice, const float* w1, float scale,
                        const float* w2, uint16_t* x, uint16_t* xlo, int H, float eps, hipStream_t st) {
  const int per = H / 256;
  if (H % 256 || (per != 1 && per != 2 && per != 4 && per != 8 && per != kMaxPer))
    return e4b_fail(E4B_EINVAL, "resnorm rows: hidden %d is not 256, 512, 1024, 2048 or 4096", H);
  if (M < 1) return e4b_fail(E4B_EINVAL, "resnorm rows: M = %d", M);
  if (a && (na < 1 || na > kMaxPartials || !w1)) return e4b_fail(E4B_EINVAL, "resnorm rows: %d residual slices", na);
  switch (per) {
    case 1: launch_resnorm_per<1>(M, h, a, na, slice, w1, scale, w2, x, xlo, H, eps, st); break;
    case 2: launch_resnorm_per<2>(M, h, a, na, slice, w1, scale, w2, x, xlo, H, eps, st); break;
    case 4: launch_resnorm_per<4>(M, h, a, na, slice, w1, scale, w2, x, xlo, H, eps, st); break;
    case 8: launch_resnorm_per<8>(M, h, a, na, slice, w1, scale, w2, x, xlo, H, eps, st); break;
    default: launch_resnorm_per<kMaxPer>(M, h, a, na, slice, w1, scale, w2, x, xlo, H, eps, st); break;
  }
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}

int launch_headprep_rows(const float* qkv, int ks, int64_t slice, const float* qw, const float* kw,
                         const float* inv_freq, int angles, uint16_t* kc, uint16_t* vc, int slots, bool ring,
                         uint32_t p0, int M, float* q, int qh, int kvh, float eps, hipStream_t st) {
  if (qh != 4 * kvh) return e4b_fail(E4B_EINVAL, "headprep rows: %d q heads for %d kv heads", qh, kvh);
  if (!ring && (int64_t)p0 + M > slots)
    return e4b_fail(E4B_ERANGE, "headprep rows: positions [%u, %lld) beyond %d slots", p0, (long long)p0 + M, slots);
  hipLaunchKernelGGL(k_headprep_rows, dim3(qh + 2 * kvh, M), dim3(64), 0, st, qkv, ks, slice, qw, kw, inv_freq, angles,
                     kc, vc, slots, ring ? 1 : 0, p0, q, qh, kvh, eps);
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}

size_t attn_prefill_part_bytes(int M, int kvh, int gqa, int hd) {
  const int tq = 16 * (gqa == 1 || gqa == 2 ? 4 / gqa : 1), units = gqa > 4 ? gqa : 4;
  return (size_t)kvh * (size_t)((M + tq - 1) / tq) * kPfAttnMaxSplits * units * 16 * (hd + 2) * sizeof(float);
}

int launch_attn_prefill(PrefillAttnArgs a, hipStream_t st) {
  const int gqa = a.kvh > 0 && a.qh % a.kvh == 0 ? a.qh / a.kvh : 0;
  if (!(a.hd == 256 && (gqa == 1 || gqa == 2 || gqa == 4)) && !(a.hd == 512 && gqa == 8))
    return e4b_fail(E4B_EINVAL,
                    "prefill attention: head dim %d with %d q heads for %d kv heads (256: 1, 2 or 4 per group; "
                    "512: 8)", a.hd, a.qh, a.kvh);
  if (a.M < 1) return e4b_fail(E4B_EINVAL, "prefill attention: M = %d", a.M);
  if (a.window > 0) {
    // every key a query of the chunk needs must still own its ring slot
    // after the chunk's own writes: slots >= window + M - 1 (the Complete
    // condition of specs/KVRing.tla with C = M)
    if ((int64_t)a.slots < (int64_t)a.window + a.M - 1)
      return e4b_fail(E4B_EINVAL, "prefill attention: %d ring slots < window %d + chunk %d - 1", a.slots, a.window,
                      a.M);
  } else if ((int64_t)a.p0 + a.M > a.slots) {
    return e4b_fail(E4B_ERANGE, "prefill attention: positions beyond %d slots", a.slots);
  }
  // the widest key range of a query tile sets the split length: at least
  // kPfAttnMinSplit keys, at most kPfAttnMaxSplits splits
  const int tq = 16 * (gqa < 4 ? 4 / gqa : 1);  // queries per workgroup
  const int nqt = (a.M + tq - 1) / tq;
  int maxspan = 0;
  for (int t = 0; t < nqt; ++t) {
    const int P0 = (int)a.p0 + tq * t, P1 = (int)a.p0 + std::min(tq * t + tq, a.M) - 1;
    const int klo = a.window > 0 ? std::max(0, P0 - a.window + 1) : 0;
    maxspan = std::max(maxspan, P1 - klo + 1);
  }
  int kspl = (maxspan + kPfAttnMaxSplits - 1) / kPfAttnMaxSplits;
  kspl = std::max(kPfAttnMinSplit, (kspl + kKT - 1) / kKT * kKT);
  int ns = (maxspan + kspl - 1) / kspl;
  if (!a.part) ns = 1;
  if (ns > 1) {
    const size_t need = (size_t)a.kvh * nqt * ns * (gqa > 4 ? gqa : 4) * 16 * (a.hd + 2) * sizeof(float);
    if (a.part_bytes < need)
      return e4b_fail(E4B_EINVAL, "prefill attention: %zu partial bytes, %zu needed", a.part_bytes, need);
  }
  a.kspl = kspl;
  a.ns = ns;
  const dim3 grid(a.kvh, nqt, ns), cgrid(a.qh, a.M);
  if (a.hd == 512) {
    // two sets of 4 heads x two 256-dim V halves per KV group
    hipLaunchKernelGGL((k_attn_prefill<8, 512>), dim3(4 * a.kvh, nqt, ns), dim3(256), 0, st, a);
    if (ns > 1) hipLaunchKernelGGL((k_attn_prefill_combine<8, 512>), cgrid, dim3(128), 0, st, a);
  } else if (gqa == 4) {
    hipLaunchKernelGGL(k_attn_prefill<4>, grid, dim3(256), 0, st, a);
    if (ns > 1) hipLaunchKernelGGL(k_attn_prefill_combine<4>, cgrid, dim3(64), 0, st, a);
  } else if (gqa == 2) {
    hipLaunchKernelGGL(k_attn_prefill<2>, grid, dim3(256), 0, st, a);
    if (ns > 1) hipLaunchKernelGGL(k_attn_prefill_combine<2>, cgrid, dim3(64), 0, st, a);
  } else {
    hipLaunchKernelGGL(k_attn_prefill<1>, grid, dim3(256), 0, st, a);
    if (ns > 1) hipLaunchKernelGGL(k_attn_prefill_combine<1>, cgrid, dim3(64), 0, st, a);
  }
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}
