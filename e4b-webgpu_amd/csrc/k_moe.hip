// k_moe.hip -- the MoE FFN half-layer of the A4B-style decode step
// (src/engine-a4b.js:438-462): router + top-8, dense and expert gate/up
// GeGLU, dense down and slot-combined expert down, and the fused tail, in
// four launches that read only the 8 active experts' weight rows.
//
//   k_moe_router  h -> rms -> router scores (one wave per expert), plus the
//                 f16 inputs of the dense (ffn_norm) and expert (pre_ffw2)
//                 branches                       (kernels/rmsacc3.wgsl:36-53,
//                                                 kernels/routertop.wgsl:19-35)
//   k_moe_gu      top-8 selection, redone by every wave from the 128 scores
//                 (no cross-block handshake), then gate/up + GeGLU for the
//                 dense branch and the 8 expert slots
//                                                (kernels/routertop.wgsl:48-71,
//                                                 kernels/q40gu.wgsl:62-119)
//   k_moe_down    dense down rows and, per output row, the 8 expert rows
//                 weighted by the router weights  (kernels/q40moedown.wgsl:42-75)
//   k_moe_tail    comb = rms(dense) w1 + rms(moe) w2; h = (h + rms(comb) wp) * s
//                                                (kernels/a4btail.wgsl:26-71)
//
// The selection is made on the f32 scores with a strict '>' scan in index
// order (ties -> lowest index), the order the reference's softmax scan gives
// since exp is monotonic; weights are p_k / sum(p) renormalised over the
// picks and scaled by the per-expert scale, in the reference's f32 order.
#include "../../include/e4b.h"
#include "kernels.h"
#include "moe.h"
#include "util.h"
#include "trace.h"

namespace {

constexpr float kTwo24 = 16777216.0f;
constexpr int K = kMoeTopK;

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

// ---- router ---------------------------------------------------------------
// grid ceil(E/2) x 128: wave w of block b scores expert 2b + w.  Every block
// computes the rms of h itself and stages x_r = h * inv * scale * mult in LDS
// once; each wave then streams only its expert's row.  Block b also writes
// its slice of the two f16 GEMV inputs.  With attn_o set, every block first
// forms the attention residual h1 = h + rms(attn_o) post_attn
// (kernels/rmsacc3.wgsl:36-53) from its own loads, stages it in LDS for the
// branch inputs, and block 0 writes it to h1.
//
// Every request goes out before the first wait: the vector loads from the
// leading (preloaded) pointers, then the struct fields the later steps use
// (eps, the multiplier, the output and norm pointers) are read in one wait
// that overlaps those loads, then this block's slice of the two branch
// norms.  Left to the compiler, the struct reads were issued at the second
// rms and waited on there, a kernel-argument round trip on the critical path.
constexpr int kRouterMaxH4 = 768;  // H <= 3072

DEV float4 f4_fma(float4 a, float s, float4 w, float4 b) {
  return make_float4(fmaf(a.x * s, w.x, b.x), fmaf(a.y * s, w.y, b.y), fmaf(a.z * s, w.z, b.z),
                     fmaf(a.w * s, w.w, b.w));
}
DEV float f4_ss(float4 v, float acc) {
  return fmaf(v.x, v.x, fmaf(v.y, v.y, fmaf(v.z, v.z, fmaf(v.w, v.w, acc))));
}

// The router's leading scalar arguments repeat the fields its first
// requests need (h, router_scale, attn_o, post_attn, router_w, H | E << 16):
// the library is built with -amdgpu-kernarg-preload-count, so they arrive in
// SGPRs with the wave and no request waits for a kernel-argument load
// (struct arguments are not preloaded).  Measured on MI355X at the A4B
// shape: 734 tok/s against 724 without.  With the struct fields read in
// one early wait and the branch norms prefetched, and leads for the down
// kernel's expert blocks: 776.2 tok/s against 765.2 (c3: 21.0 against
// 21.4 us per half-layer).
template <int NO>  // the o projection's column slices; 0: no attention residual
__global__ __launch_bounds__(128) void k_moe_router(const float* lh, const float* lrs, const float* lo,
                                                    const float* lpa, const float* lrw, uint32_t lhe, MoeArgs A) {
  A.h = lh;
  A.router_scale = lrs;
  A.attn_o = lo;
  A.post_attn = lpa;
  A.router_w = lrw;
  A.H = (int)(lhe & 0xffffu);
  A.E = (int)(lhe >> 16);
  E4B_TRACE_SCOPE(trace_tag(TR_MOE_ROUTER, 0));
  // token row y of a batch (the batched prefill); y = 0 in the decode step.
  // The outputs are offset where they are written, so that their struct
  // fields are not read before the loads below are issued.
  A.h += (int64_t)blockIdx.y * A.H;
  const int64_t ry = blockIdx.y;
  __shared__ __align__(16) float4 xr[kRouterMaxH4];
  __shared__ __align__(16) float4 h1s[kRouterMaxH4];
  __shared__ float red[2];
  constexpr int PT = kRouterMaxH4 / 128;  // float4 per thread
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int H = A.H, H4 = H / 4;
  constexpr bool res = NO > 0;
  const float4* h4 = reinterpret_cast<const float4*>(A.h);
  const float4* rs4 = reinterpret_cast<const float4*>(A.router_scale);
  const float4* o4 = reinterpret_cast<const float4*>(A.attn_o);
  const float4* pa4 = reinterpret_cast<const float4*>(A.post_attn);
  const int e = min((int)blockIdx.x * 2 + wave, A.E - 1);
  const float4* w4 = reinterpret_cast<const float4*>(A.router_w + (int64_t)e * H);
  // every load up front: h, the scale and the residual inputs
  // (thread-strided), the expert row
  float4 hv[PT], sv[PT], ov[PT], pv[PT], wv[kRouterMaxH4 / 64];
  float4 os[NO > 1 ? NO - 1 : 1][PT];  // the o projection's further column slices
#pragma unroll
  for (int k = 0; k < PT; ++k) {
    const int i = min((int)threadIdx.x + 128 * k, H4 - 1);
    hv[k] = h4[i];
    sv[k] = rs4[i];
    if (res) {
      ov[k] = o4[i];
#pragma unroll
      for (int q = 1; q < NO; ++q) os[q - 1][k] = o4[(int64_t)q * H4 + i];
      pv[k] = pa4[i];
    }
  }
#pragma unroll
  for (int k = 0; k < kRouterMaxH4 / 64; ++k) wv[k] = w4[min(lane + 64 * k, H4 - 1)];
  __builtin_amdgcn_sched_barrier(0);
  // the struct fields, in one wait while the loads above are in flight
  asm volatile("" ::"s"(A.eps), "s"(A.router_mult), "s"(A.scores), "s"(A.xd), "s"(A.xm), "s"(A.ffn_norm),
               "s"(A.pre_ffw2));
  if (res) asm volatile("" ::"s"(A.h1));
  // this block's slice of the branch inputs: the first element of each
  // thread's share of the two norms requested now
  const int nblk = (A.E + 1) / 2;  // gridDim.x, known without the hidden arguments
  const int per = (H + nblk - 1) / nblk;
  const int b_lo = (int)blockIdx.x * per, b_hi = min(H, b_lo + per);
  const int i0 = b_lo + (int)threadIdx.x;
  float fn0 = 0.f, p20 = 0.f;
  if (i0 < b_hi) {
    fn0 = A.ffn_norm[i0];
    p20 = A.pre_ffw2[i0];
  }
  E4B_TRACE_MARK(0);
  if (res) {
    // o = the slices' sum in slice order
#pragma unroll
    for (int q = 1; q < NO; ++q)
#pragma unroll
      for (int k = 0; k < PT; ++k)
        ov[k] = make_float4(ov[k].x + os[q - 1][k].x, ov[k].y + os[q - 1][k].y, ov[k].z + os[q - 1][k].z,
                            ov[k].w + os[q - 1][k].w);
    float so = 0.f;
#pragma unroll
    for (int k = 0; k < PT; ++k)
      if ((int)threadIdx.x + 128 * k < H4) so = f4_ss(ov[k], so);
    so = wave_sum(so);
    if (lane == 0) red[wave] = so;
    lds_sync();
    const float io = rms_inv(red[0] + red[1], H, A.eps);
    E4B_TRACE_MARK(1);
    lds_sync();  // red is reused below
    const bool writer = blockIdx.x == 0 && blockIdx.y == 0;
#pragma unroll
    for (int k = 0; k < PT; ++k) {
      const int i = (int)threadIdx.x + 128 * k;
      hv[k] = f4_fma(ov[k], io, pv[k], hv[k]);
      if (i < H4) {
        h1s[i] = hv[k];
        if (writer) reinterpret_cast<float4*>(A.h1)[i] = hv[k];
      }
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < PT; ++k)
    if ((int)threadIdx.x + 128 * k < H4)
      ss = fmaf(hv[k].x, hv[k].x, fmaf(hv[k].y, hv[k].y, fmaf(hv[k].z, hv[k].z, fmaf(hv[k].w, hv[k].w, ss))));
  ss = wave_sum(ss);
  if (lane == 0) red[wave] = ss;
  lds_sync();
  const float inv = rms_inv(red[0] + red[1], H, A.eps);
#pragma unroll
  for (int k = 0; k < PT; ++k) {
    const int i = (int)threadIdx.x + 128 * k;
    if (i < H4)
      xr[i] = make_float4(hv[k].x * inv * (sv[k].x * A.router_mult), hv[k].y * inv * (sv[k].y * A.router_mult),
                          hv[k].z * inv * (sv[k].z * A.router_mult), hv[k].w * inv * (sv[k].w * A.router_mult));
  }
  lds_sync();
  E4B_TRACE_MARK(2);
  float acc = 0.f;
#pragma unroll
  for (int k = 0; k < kRouterMaxH4 / 64; ++k) {
    const int i = lane + 64 * k;
    if (i < H4) {
      const float4 x = xr[i], w = wv[k];
      acc = fmaf(x.x, w.x, fmaf(x.y, w.y, fmaf(x.z, w.z, fmaf(x.w, w.w, acc))));
    }
  }
  acc = wave_sum(acc);
  if (lane == 0 && (int)blockIdx.x * 2 + wave < A.E) A.scores[ry * A.E + e] = acc;
  E4B_TRACE_MARK(3);
  // this block's slice of the f16 branch inputs
  const float* h1f = reinterpret_cast<const float*>(h1s);
  if (i0 < b_hi) {
    const float v = (res ? h1f[i0] : A.h[i0]) * inv;
    A.xd[ry * H + i0] = f2h(v * fn0);
    A.xm[ry * H + i0] = f2h(v * p20);
  }
  for (int i = i0 + 128; i < b_hi; i += 128) {
    const float v = (res ? h1f[i] : A.h[i]) * inv;
    A.xd[ry * H + i] = f2h(v * A.ffn_norm[i]);
    A.xm[ry * H + i] = f2h(v * A.pre_ffw2[i]);
  }
}

// ---- router over token rows (batched prefill) -------------------------------
// grid ceil(E / kRrE) x ceil(M / kRrT), 128 threads: block (bx, by) scores
// experts [kRrE bx, kRrE bx + kRrE) of token rows [kRrT by, kRrT by + kRrT).
// Each row's rms and x_r follow k_moe_router's arithmetic step for step (the
// same 128-thread element split, fmaf chains, wave sums and two-wave sum),
// so the scores, and the top-8 taken from them, equal the decode router's
// bit for bit.  An expert row is read once per kRrT token rows instead of
// once per row (the decode layout over rows re-read the whole router matrix
// and the row's vectors in every one of its E/2 blocks).  Rows without the
// attention residual only (the prefill forms h1 before the router).
// 2 rows x 16 experts per workgroup: 24 KB of LDS, 6 workgroups per CU
// (measured against 4 x 16, 4 x 8 and 2 x 8: 367.7 us for the c3 layer over
// 512 rows against 377.9, 375.5 and 372.7)
constexpr int kRrT = 2, kRrE = 16;
static_assert(kRrT * kRrE / 2 <= 64, "one score per lane");
__global__ __launch_bounds__(128) __attribute__((amdgpu_waves_per_eu(2))) void k_moe_router_rows(MoeArgs A, int M) {
  __shared__ __align__(16) float4 xr[kRrT][kRouterMaxH4];
  __shared__ float red[kRrT][2];
  constexpr int PT = kRouterMaxH4 / 128;  // float4 per thread and row
  constexpr int PW = kRouterMaxH4 / 64;   // float4 per lane of an expert row
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int H = A.H, H4 = H / 4, E = A.E;
  const int r0 = blockIdx.y * kRrT;
  const float4* rs4 = reinterpret_cast<const float4*>(A.router_scale);
  const float4* fn4 = reinterpret_cast<const float4*>(A.ffn_norm);
  const float4* pf4 = reinterpret_cast<const float4*>(A.pre_ffw2);
  // this block writes float4 [q0, q1) of each row's f16 branch inputs
  const int per4 = (H4 + gridDim.x - 1) / gridDim.x;
  const int q0 = blockIdx.x * per4, q1 = min(H4, q0 + per4);
  // every load up front (clamped, branch-free): the rows, the scale, the
  // two branch norms
  float4 hv[kRrT][PT], sv[PT], fv[PT], pv[PT];
#pragma unroll
  for (int k = 0; k < PT; ++k) {
    const int i = min((int)threadIdx.x + 128 * k, H4 - 1);
    sv[k] = rs4[i];
    fv[k] = fn4[i];
    pv[k] = pf4[i];
#pragma unroll
    for (int t = 0; t < kRrT; ++t)
      hv[t][k] = reinterpret_cast<const float4*>(A.h + (int64_t)min(r0 + t, M - 1) * H)[i];
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int t = 0; t < kRrT; ++t) {
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < PT; ++k) {
      const float4 v = hv[t][k];
      const float nx = fmaf(v.x, v.x, fmaf(v.y, v.y, fmaf(v.z, v.z, fmaf(v.w, v.w, ss))));
      ss = (int)threadIdx.x + 128 * k < H4 ? nx : ss;
    }
    ss = wave_sum(ss);
    if (lane == 0) red[t][wave] = ss;
  }
  lds_sync();
#pragma unroll
  for (int t = 0; t < kRrT; ++t) {
    const float inv = rms_inv(red[t][0] + red[t][1], H, A.eps);
    const int64_t ro = (int64_t)(r0 + t) * H;
#pragma unroll
    for (int k = 0; k < PT; ++k) {
      const int i = (int)threadIdx.x + 128 * k;
      const float4 v = hv[t][k];
      if (i < H4)
        xr[t][i] = make_float4(v.x * inv * (sv[k].x * A.router_mult), v.y * inv * (sv[k].y * A.router_mult),
                               v.z * inv * (sv[k].z * A.router_mult), v.w * inv * (sv[k].w * A.router_mult));
      if (i >= q0 && i < q1 && r0 + t < M) {
        const float4 n = make_float4(v.x * inv, v.y * inv, v.z * inv, v.w * inv);
        uint2 d, m;
        d.x = (uint32_t)f2h(n.x * fv[k].x) | ((uint32_t)f2h(n.y * fv[k].y) << 16);
        d.y = (uint32_t)f2h(n.z * fv[k].z) | ((uint32_t)f2h(n.w * fv[k].w) << 16);
        m.x = (uint32_t)f2h(n.x * pv[k].x) | ((uint32_t)f2h(n.y * pv[k].y) << 16);
        m.y = (uint32_t)f2h(n.z * pv[k].z) | ((uint32_t)f2h(n.w * pv[k].w) << 16);
        reinterpret_cast<uint2*>(A.xd + ro)[i] = d;
        reinterpret_cast<uint2*>(A.xm + ro)[i] = m;
      }
    }
  }
  lds_sync();
  // wave w scores experts e0 + w + 2 j (j < kRrE / 2); the next row is
  // requested before the current one's dot products; lane j kRrT + t keeps
  // the score of (expert j, row t) for one store at the end
  const int e0 = blockIdx.x * kRrE + wave;
  float4 wv[2][PW];
  auto load_row = [&](float4* dst, int j) {
    const float4* w4 = reinterpret_cast<const float4*>(A.router_w + (int64_t)min(e0 + 2 * j, E - 1) * H);
#pragma unroll
    for (int k = 0; k < PW; ++k) dst[k] = w4[min(lane + 64 * k, H4 - 1)];
  };
  load_row(wv[0], 0);
  float mine = 0.f;
#pragma unroll
  for (int j = 0; j < kRrE / 2; ++j) {
    // the staged rows are read from LDS again for every expert: held in
    // registers (4 x 12 float4) they leave none for the next row's loads
    asm volatile("" ::: "memory");
    if (j + 1 < kRrE / 2) load_row(wv[(j + 1) & 1], j + 1);
#pragma unroll
    for (int t = 0; t < kRrT; ++t) {
      float acc = 0.f;
#pragma unroll
      for (int k = 0; k < PW; ++k) {
        const int i = lane + 64 * k;
        const float4 x = xr[t][min(i, H4 - 1)], w = wv[j & 1][k];
        const float nx = fmaf(x.x, w.x, fmaf(x.y, w.y, fmaf(x.z, w.z, fmaf(x.w, w.w, acc))));
        acc = i < H4 ? nx : acc;
      }
      acc = wave_sum(acc);
      mine = lane == j * kRrT + t ? acc : mine;
    }
  }
  const int j = lane / kRrT, t = lane % kRrT, e = e0 + 2 * j;
  if (lane < kRrT * kRrE / 2 && e < E && r0 + t < M) A.scores[(int64_t)(r0 + t) * E + e] = mine;
}

// ---- top-8 in one wave ----------------------------------------------------
// lane l holds the scores of experts l + 64 j (j < 4, E <= 256); every lane
// returns the same 8 picks (and, with WEIGHTS, their weights).  As in
// kernels/routertop.wgsl:53-64 the ranking is on the f32 p = exp(s - max),
// not on the scores: scores whose p round equal (apart by less than p's
// spacing, or both far enough below the maximum that p is 0) tie and go to
// the lowest index.  Each pick is the wave maximum of a 64-bit key (p's bits,
// which order non-negative floats, plus one; then the complemented expert
// index, so ties go to the lowest index as the strict '>' scan in index
// order gives), reduced with lane swaps and DPP moves (six short steps, no
// LDS round trips); the picked entry's key drops to 0, below every live key.
struct TopK {
  int idx[K];
  float w[K];
};

// the value of lane l ^ M (bit-preserving)
template <int M>
DEV uint32_t lane_partner(uint32_t v) {
  if constexpr (M == 32) {
    float a = __uint_as_float(v), b = a;
    swapx32(a, b);  // lanes < 32: b holds lane l + 32; lanes >= 32: a holds lane l - 32
    return __float_as_uint((threadIdx.x & 32) ? a : b);
  } else if constexpr (M == 16) {
    float a = __uint_as_float(v), b = a;
    swapx16(a, b);  // even rows: b holds lane l + 16; odd rows: a holds lane l - 16
    return __float_as_uint((threadIdx.x & 16) ? a : b);
  } else {
    return __float_as_uint(lane_xor<M>(__uint_as_float(v)));
  }
}

template <int M>
DEV void key_max_step(uint32_t& hi, uint32_t& lo) {
  const uint32_t ohi = lane_partner<M>(hi), olo = lane_partner<M>(lo);
  const bool take = (ohi > hi) | ((ohi == hi) & (olo > lo));
  hi = take ? ohi : hi;
  lo = take ? olo : lo;
}

template <bool WEIGHTS>
DEV TopK select_topk(const float* __restrict__ scores, const float* __restrict__ pes, int E) {
  const int lane = threadIdx.x & 63;
  float s[4], pe[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = min(lane + 64 * j, E - 1);
    s[j] = scores[e];
    pe[j] = WEIGHTS ? pes[e] : 0.f;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) s[j] = lane + 64 * j < E ? s[j] : -3.0e38f;
  const float M = wave_max(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])));
  uint32_t kh[4];
  float p[4];
  float psum = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const bool live = lane + 64 * j < E;
    p[j] = live ? expf(s[j] - M) : 0.f;
    psum += p[j];
    kh[j] = live ? __float_as_uint(p[j]) + 1u : 0u;  // live keys are >= 1
  }
  const float S = WEIGHTS ? wave_sum(psum) : 1.f;
  TopK t;
  float wsum = 0.f;
  float pk[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    // lane candidate: j ascending is index ascending, so a strict '>' keeps
    // the lowest index of equal keys
    uint32_t bh = kh[0], bl = ~(uint32_t)lane;
#pragma unroll
    for (int j = 1; j < 4; ++j) {
      const bool take = kh[j] > bh;
      bh = take ? kh[j] : bh;
      bl = take ? ~(uint32_t)(lane + 64 * j) : bl;
    }
    key_max_step<32>(bh, bl);
    key_max_step<16>(bh, bl);
    key_max_step<8>(bh, bl);
    key_max_step<4>(bh, bl);
    key_max_step<2>(bh, bl);
    key_max_step<1>(bh, bl);
    const int bi = __builtin_amdgcn_readfirstlane((int)~bl);
    t.idx[k] = bi;
    const int bj = bi >> 6, bln = bi & 63;
    if constexpr (WEIGHTS) {
      float sv = p[0], pv = pe[0];
#pragma unroll
      for (int j = 1; j < 4; ++j) {
        sv = bj == j ? p[j] : sv;
        pv = bj == j ? pe[j] : pv;
      }
      const float bv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sv), bln));
      pk[k] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pv), bln));
      t.w[k] = bv / S;  // p_k / sum p, as the reference stores it
      wsum += t.w[k];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) kh[j] = lane + 64 * j == bi ? 0u : kh[j];
  }
  if constexpr (WEIGHTS) {
#pragma unroll
    for (int k = 0; k < K; ++k) t.w[k] = t.w[k] / wsum * pk[k];
  }
  return t;
}

__global__ __launch_bounds__(64) void k_moe_topk(MoeArgs A) {
  // token row blockIdx.x of a batch (one block in the decode step)
  A.scores += (int64_t)blockIdx.x * A.E;
  A.topk_idx += (int64_t)blockIdx.x * K;
  A.topk_w += (int64_t)blockIdx.x * K;
  const TopK t = select_topk<true>(A.scores, A.pes, A.E);
  const int lane = threadIdx.x;
#pragma unroll
  for (int k = 0; k < K; ++k)
    if (lane == k) {
      A.topk_idx[k] = (uint32_t)t.idx[k];
      A.topk_w[k] = t.w[k];
    }
}

// ---- gate/up + GeGLU, dense branch and 8 expert slots ------------------------
// 32 lanes per unit (a gate row and its up row), 3 blocks per lane (88-block
// rows of the 2816-wide input), GU_U units per lane group and 2 GU_U per
// wave tile (2 measured fastest at the A4B shape: c3 23.3 us per half-layer
// against 24.3 with 1 and 24.1 with 4).  Units [0, FF2) are
// dense, then slot k covers [FF2 + k FF, FF2 + (k+1) FF).  The block stages
// both f16 inputs in LDS once (a block can hold dense and expert waves):
// read per wave, the input would cost more on-chip traffic than the weights.
constexpr int GU_LPR = 32, GU_BPL = 3;
constexpr int GU_U = 2;  // units per lane group (a wave tile holds 2 GU_U units)
constexpr int kMoeMaxH = GU_LPR * GU_BPL * 32;  // 3072

//
// The leading scalar arguments repeat what the first requests need (the
// scores, both weight matrices, H | E << 16, FF | FF2 << 16): they arrive
// preloaded in SGPRs, so every block requests the scores and the dense
// blocks their rows at entry; the two inputs follow from the struct, whose
// read then waits behind those requests.
__global__ __launch_bounds__(256) void k_moe_gu(float* lsco, const uint4* ldn, const uint16_t* lds, const uint4* len,
                                                const uint16_t* les, uint32_t lhe, uint32_t lff, MoeArgs A) {
  A.scores = lsco;
  A.dense_gu.nib = ldn;
  A.dense_gu.sc = lds;
  A.exp_gu.nib = len;
  A.exp_gu.sc = les;
  A.H = (int)(lhe & 0xffffu);
  A.E = (int)(lhe >> 16);
  A.FF = (int)(lff & 0xffffu);
  A.FF2 = (int)(lff >> 16);
  const int64_t ntiles = (A.FF2 + (int64_t)K * A.FF) / (2 * GU_U);
  E4B_TRACE_SCOPE(trace_tag(TR_MOE_GU, 0));
  __shared__ __align__(16) uint16_t xs[2][kMoeMaxH];
  __shared__ int sel[K];
  __shared__ __align__(16) uint64_t skey[256];  // the expert blocks' ranking keys
  __shared__ float smax[4];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane / GU_LPR, l = lane % GU_LPR;
  const int nb = A.H / 32;
  // one tile (2 GU_U units) per wave; idle waves of the last workgroup
  // repeat the last tile and store nothing
  const int64_t tile_id = (int64_t)blockIdx.x * 4 + wave;
  const bool live = tile_id < ntiles;
  const int64_t tile = live ? tile_id : ntiles - 1;
  const int u = (int)(2 * GU_U * tile) + GU_U * g;  // this group's first unit
  const bool dense = 2 * GU_U * tile < A.FF2;        // wave-uniform: FF2 and FF are multiples of 2 GU_U

  // 1. the scores (the expert blocks rank them below), one per thread
  const int E = A.E;
  const float sv = (int)threadIdx.x < E ? A.scores[threadIdx.x] : -3.0e38f;

  // 2. weight rows: dense units are known now; expert units after the top-8
  //    selection, made once per workgroup by wave 0 from the 128 scores and
  //    handed over in LDS (wave 0 of block 0 also stores the picks and their
  //    weights for the down kernel)
  // rows 2i (gate) and 2i + 1 (up) of unit u + i
  uint4 wq[2 * GU_U][GU_BPL];
  uint32_t ws[2 * GU_U][GU_BPL], odd = 0;  // aligned scale pairs (ld_scale_pair)
  auto load_rows = [&](const Q40Mat& W, int64_t row_g, int64_t up_off) {
#pragma unroll
    for (int i = 0; i < GU_U; ++i)
#pragma unroll
      for (int b = 0; b < GU_BPL; ++b) {
        const int jb = min(l + GU_LPR * b, nb - 1);
        const int64_t eg = (row_g + i) * nb + jb, eu = (row_g + i + up_off) * nb + jb;
        wq[2 * i][b] = ld_nt_u4(W.nib + eg);
        ws[2 * i][b] = ld_scale_pair(W.sc, eg);
        wq[2 * i + 1][b] = ld_nt_u4(W.nib + eu);
        ws[2 * i + 1][b] = ld_scale_pair(W.sc, eu);
        odd |= (uint32_t)(eg & 1) << (2 * i * GU_BPL + b);
        odd |= (uint32_t)(eu & 1) << ((2 * i + 1) * GU_BPL + b);
      }
  };
  if (dense) load_rows(A.dense_gu, u, A.FF2);
  __builtin_amdgcn_sched_barrier(0);
  // 3. both inputs (independent of the routing), two 16-byte pieces per
  //    thread and input at most (H <= 3072)
  // (named registers: an array here is kept in scratch memory by the compiler)
  const int nv = A.H / 8;
  const int i0 = min((int)threadIdx.x, nv - 1), i1 = min((int)threadIdx.x + 256, nv - 1);
  const uint4 xd0 = reinterpret_cast<const uint4*>(A.xd)[i0], xd1 = reinterpret_cast<const uint4*>(A.xd)[i1];
  const uint4 xm0 = reinterpret_cast<const uint4*>(A.xm)[i0], xm1 = reinterpret_cast<const uint4*>(A.xm)[i1];
  E4B_TRACE_MARK(0);
  // the block holds expert waves iff its last (clamped) tile is an expert tile
  const bool blk_expert = 2 * GU_U * min((int64_t)blockIdx.x * 4 + 3, ntiles - 1) >= A.FF2;
  if (blockIdx.x == 0) {
    // block 0 also stores the picks and their weights for the down kernel
    if (wave == 0) {
      const TopK t = select_topk<true>(A.scores, A.pes, A.E);
#pragma unroll
      for (int k = 0; k < K; ++k)
        if (lane == k) {
          A.topk_idx[k] = (uint32_t)t.idx[k];
          A.topk_w[k] = t.w[k];
          sel[k] = t.idx[k];
        }
    }
  } else if (blk_expert) {
    // the block's 4 waves rank the experts together: expert e's rank is the
    // number of experts with a larger key, or an equal key and a lower
    // index -- the order of select_topk -- as 64-bit compares of (key,
    // 255 - index) words staged in LDS, two threads per expert (E <= 128)
    // or one (E <= 256); no dependent cross-lane chain, so the picks are in
    // LDS ~1 us after the scores arrive instead of ~3 us for one wave's
    // eight wave-maximum rounds
    const int t = threadIdx.x;
    const float wm = wave_max(sv);
    if (lane == 0) smax[wave] = wm;
    lds_sync();
    const float M = fmaxf(fmaxf(smax[0], smax[1]), fmaxf(smax[2], smax[3]));
    const uint32_t key = t < E ? __float_as_uint(expf(sv - M)) + 1u : 0u;  // live keys are >= 1
    skey[t] = (uint64_t)key << 8 | (uint64_t)(255 - t);
    lds_sync();
    if (E <= 128) {
      const int c = t >> 1, h = t & 1;  // expert c, keys [64 h, 64 h + 64)
      const uint64_t mine = skey[c];
      int r = 0;
#pragma unroll 8
      for (int e = 64 * h; e < 64 * h + 64; e += 2) {
        const ulonglong2 k2 = *reinterpret_cast<const ulonglong2*>(&skey[e]);
        r += (k2.x > mine ? 1 : 0) + (k2.y > mine ? 1 : 0);
      }
      r += __shfl_xor(r, 1, 64);
      if (h == 0 && c < E && r < K) sel[r] = c;
    } else {
      const uint64_t mine = skey[t];
      int r = 0;
#pragma unroll 8
      for (int e = 0; e < 256; e += 2) {
        const ulonglong2 k2 = *reinterpret_cast<const ulonglong2*>(&skey[e]);
        r += (k2.x > mine ? 1 : 0) + (k2.y > mine ? 1 : 0);
      }
      if (t < E && r < K) sel[r] = t;
    }
  }

  // 4. stage the inputs and the picks, then the expert rows and this lane's
  //    blocks from LDS
  if ((int)threadIdx.x < nv) {
    reinterpret_cast<uint4*>(xs[0])[threadIdx.x] = xd0;
    reinterpret_cast<uint4*>(xs[1])[threadIdx.x] = xm0;
  }
  if ((int)threadIdx.x + 256 < nv) {
    reinterpret_cast<uint4*>(xs[0])[threadIdx.x + 256] = xd1;
    reinterpret_cast<uint4*>(xs[1])[threadIdx.x + 256] = xm1;
  }
  lds_sync();
  E4B_TRACE_MARK(1);
  int slot = 0, j = u;
  if (!dense) {
    slot = (u - A.FF2) / A.FF;
    j = (u - A.FF2) - slot * A.FF;
    const int64_t row_g = (int64_t)sel[slot] * 2 * A.FF + j;
    load_rows(A.exp_gu, row_g, A.FF);
  }
  const uint32_t* x = reinterpret_cast<const uint32_t*>(xs[dense ? 0 : 1]);
  uint32_t xp[GU_BPL][16];
#pragma unroll
  for (int b = 0; b < GU_BPL; ++b) load_x16(x, min(l + GU_LPR * b, nb - 1), xp[b]);
  E4B_TRACE_MARK(2);

  // 5. dot products, GeGLU
  float acc[2 * GU_U];
#pragma unroll
  for (int r = 0; r < 2 * GU_U; ++r) acc[r] = 0.f;
#pragma unroll
  for (int b = 0; b < GU_BPL; ++b) {
    const bool in = l + GU_LPR * b < nb;
#pragma unroll
    for (int i = 0; i < 16; ++i) xp[b][i] = in ? xp[b][i] : 0u;
    const float xs8 = -8.f * xsum16(xp[b]);
#pragma unroll
    for (int r = 0; r < 2 * GU_U; ++r) {
      float a0 = 0.f, a1 = 0.f;
      q40_dot2(wq[r][b], xp[b], a0, a1);
      const float d = scale_of(ws[r][b], (odd >> (r * GU_BPL + b)) & 1);
      acc[r] = fmaf(d, fmaf(a1, kTwo24 / 16.f, fmaf(a0, kTwo24, xs8)), acc[r]);
    }
  }
  E4B_TRACE_MARK(3);
  // lanes [SPAN r, SPAN r + SPAN) of the group hold row r: gate of unit r / 2
  // for even r, its up row for odd r
  constexpr int SPAN = GU_LPR / (2 * GU_U);
  const float v = reduce_rows<GU_LPR, 2 * GU_U>(acc);
  const float up = __shfl_xor(v, SPAN, 64);
  const int i = l / (2 * SPAN);
  if (live && (l % (2 * SPAN)) == 0) {
    const uint16_t y = f2h(gelu_tanh(v) * up);
    if (dense)
      A.g_dense[u + i] = y;
    else
      A.g_slots[(int64_t)slot * A.FF + j + i] = y;
  }
}

// ---- down projections -------------------------------------------------------
// Blocks [0, nbd) run the dense down rows (32 lanes x 3 blocks per row of
// FF2/32 blocks, DD_R rows per group, 2 DD_R per wave tile); the rest run
// the expert rows: for output row o the 8 lane groups are the 8 slots (8
// lanes x 3 blocks of the FF/32 = 22-block rows), DE_R output rows per wave
// tile, and the slot results are combined with the router weights across
// the groups.  One tile per wave; the block's f16 input (the dense GeGLU
// output, or the 8 slots' outputs) is staged in LDS once.  One row per
// group and tile measured fastest at the A4B shape (c3: 22.5 us per
// half-layer against 23.3 with 2 / 4 rows and 26.0 with 4 / 8).
constexpr int DD_LPR = 32, DD_BPL = 3, DD_R = 1;
constexpr int DE_LPR = 8, DE_BPL = 3, DE_R = 1;
constexpr int kMoeMaxX = K * DE_LPR * DE_BPL * 32;  // 6144 >= FF2 and 8 FF

//
// The leading scalar arguments repeat what the expert blocks' first requests
// need (the picks, the expert down matrix, both inputs, H | FF << 16 and
// FF2 | nbd << 16): they arrive preloaded in SGPRs, so an expert block
// requests its picks at entry and its weight rows one global round trip
// later.  From the struct alone that took a kernel-argument read, a second
// one for the picks' pointer and then the picks' own read.
__global__ __launch_bounds__(256) void k_moe_down(uint32_t* ltk, const uint4* lnib, const uint16_t* lsc,
                                                  uint16_t* lgs, uint16_t* lgd, uint32_t lhf, uint32_t lfn,
                                                  MoeArgs A) {
  A.topk_idx = ltk;
  A.exp_down.nib = lnib;
  A.exp_down.sc = lsc;
  A.g_slots = lgs;
  A.g_dense = lgd;
  A.H = (int)(lhf & 0xffffu);
  A.FF = (int)(lhf >> 16);
  A.FF2 = (int)(lfn & 0xffffu);
  const int nbd = (int)(lfn >> 16);
  E4B_TRACE_SCOPE(trace_tag(TR_MOE_DOWN, 0));
  __shared__ __align__(16) uint16_t xs[kMoeMaxX];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const bool dense_blk = (int)blockIdx.x < nbd;  // block-uniform
  // the block's input: FF2 (dense) or 8 FF (experts) f16 values, three
  // 16-byte pieces per thread at most
  const int nx = (dense_blk ? A.FF2 : K * A.FF) / 8;
  const uint4* xsrc = reinterpret_cast<const uint4*>(dense_blk ? A.g_dense : A.g_slots);
  // (named registers: an array here is kept in scratch memory by the compiler)
  const uint4 xv0 = xsrc[min((int)threadIdx.x, nx - 1)];
  const uint4 xv1 = xsrc[min((int)threadIdx.x + 256, nx - 1)];
  const uint4 xv2 = xsrc[min((int)threadIdx.x + 512, nx - 1)];
  auto stage_x = [&]() {
    uint4* d = reinterpret_cast<uint4*>(xs);
    if ((int)threadIdx.x < nx) d[threadIdx.x] = xv0;
    if ((int)threadIdx.x + 256 < nx) d[threadIdx.x + 256] = xv1;
    if ((int)threadIdx.x + 512 < nx) d[threadIdx.x + 512] = xv2;
    lds_sync();
  };

  if (dense_blk) {
    const int g = lane / DD_LPR, l = lane % DD_LPR;
    const int nb = A.FF2 / 32;
    const Q40Mat& W = A.dense_down;
    const int64_t ntiles = (A.H + 2 * DD_R - 1) / (2 * DD_R);
    const int64_t tile = min((int64_t)blockIdx.x * 4 + wave, ntiles - 1);
    const int64_t r0 = tile * 2 * DD_R + g * DD_R;
    uint4 wq[DD_R][DD_BPL];
    uint32_t ws[DD_R][DD_BPL], odd = 0;
#pragma unroll
    for (int r = 0; r < DD_R; ++r) {
      const int64_t row = min(r0 + r, (int64_t)A.H - 1);
#pragma unroll
      for (int b = 0; b < DD_BPL; ++b) {
        const int jb = min(l + DD_LPR * b, nb - 1);
        const int64_t e = row * nb + jb;
        wq[r][b] = ld_nt_u4(W.nib + e);
        ws[r][b] = ld_scale_pair(W.sc, e);
        odd |= (uint32_t)(e & 1) << (r * DD_BPL + b);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    stage_x();
    const uint32_t* x = reinterpret_cast<const uint32_t*>(xs);
    uint32_t xp[DD_BPL][16];
    float xs8[DD_BPL];
#pragma unroll
    for (int b = 0; b < DD_BPL; ++b) {
      const int jb = l + DD_LPR * b;
      load_x16(x, min(jb, nb - 1), xp[b]);
#pragma unroll
      for (int i = 0; i < 16; ++i) xp[b][i] = jb < nb ? xp[b][i] : 0u;
      xs8[b] = -8.f * xsum16(xp[b]);
    }
    float acc[DD_R];
#pragma unroll
    for (int r = 0; r < DD_R; ++r) {
      acc[r] = 0.f;
#pragma unroll
      for (int b = 0; b < DD_BPL; ++b) {
        float a0 = 0.f, a1 = 0.f;
        q40_dot2(wq[r][b], xp[b], a0, a1);
        const float d = scale_of(ws[r][b], (odd >> (r * DD_BPL + b)) & 1);
        acc[r] = fmaf(d, fmaf(a1, kTwo24 / 16.f, fmaf(a0, kTwo24, xs8[b])), acc[r]);
      }
    }
    const float v = reduce_rows<DD_LPR, DD_R>(acc);
    const int64_t row = r0 + l / (DD_LPR / DD_R);
    if ((l % (DD_LPR / DD_R)) == 0 && row < A.H && (int64_t)blockIdx.x * 4 + wave < ntiles) A.dense_out[row] = v;
    return;
  }
  // expert rows
  const int g = lane / DE_LPR, l = lane % DE_LPR;  // g = slot
  const int nb = A.FF / 32;
  const Q40Mat& W = A.exp_down;
  const int e = (int)A.topk_idx[g];
  const int64_t ntiles = (A.H + DE_R - 1) / DE_R;
  const int64_t tile_id = (int64_t)(blockIdx.x - nbd) * 4 + wave;
  const int64_t o0 = min(tile_id, ntiles - 1) * DE_R;
  uint4 wq[DE_R][DE_BPL];
  uint32_t ws[DE_R][DE_BPL], odd = 0;
#pragma unroll
  for (int r = 0; r < DE_R; ++r) {
    const int64_t row = (int64_t)e * A.H + min(o0 + r, (int64_t)A.H - 1);
#pragma unroll
    for (int b = 0; b < DE_BPL; ++b) {
      const int jb = min(l + DE_LPR * b, nb - 1);
      const int64_t ei = row * nb + jb;
      wq[r][b] = ld_nt_u4(W.nib + ei);
      ws[r][b] = ld_scale_pair(W.sc, ei);
      odd |= (uint32_t)(ei & 1) << (r * DE_BPL + b);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  const float wk = A.topk_w[g];  // needed last: its struct read waits behind the rows
  E4B_TRACE_MARK(0);
  stage_x();
  E4B_TRACE_MARK(1);
  const uint32_t* x = reinterpret_cast<const uint32_t*>(xs + (int64_t)g * A.FF);
  uint32_t xp[DE_BPL][16];
  float xs8[DE_BPL];
#pragma unroll
  for (int b = 0; b < DE_BPL; ++b) {
    const int jb = l + DE_LPR * b;
    load_x16(x, min(jb, nb - 1), xp[b]);
#pragma unroll
    for (int i = 0; i < 16; ++i) xp[b][i] = jb < nb ? xp[b][i] : 0u;
    xs8[b] = -8.f * xsum16(xp[b]);
  }
  float acc[DE_R];
#pragma unroll
  for (int r = 0; r < DE_R; ++r) {
    acc[r] = 0.f;
#pragma unroll
    for (int b = 0; b < DE_BPL; ++b) {
      float a0 = 0.f, a1 = 0.f;
      q40_dot2(wq[r][b], xp[b], a0, a1);
      const float d = scale_of(ws[r][b], (odd >> (r * DE_BPL + b)) & 1);
      acc[r] = fmaf(d, fmaf(a1, kTwo24 / 16.f, fmaf(a0, kTwo24, xs8[b])), acc[r]);
    }
  }
  E4B_TRACE_MARK(2);
  // lane l of slot g holds y_g of row o0 + l / 2; weight it and sum the slots
  float v = reduce_rows<DE_LPR, DE_R>(acc) * wk;
  v = xsum_step<8>(v);
  v = xsum_step<16>(v);
  v = xsum_step<32>(v);
  const int64_t row = o0 + l / (DE_LPR / DE_R);
  if (g == 0 && (l % (DE_LPR / DE_R)) == 0 && row < A.H && tile_id < ntiles) A.moe_out[row] = v;
}

// ---- tail ----------------------------------------------------------------------
constexpr int kTailPer = 12;  // elements per thread, H <= 3072

__global__ __launch_bounds__(256) void k_moe_tail(MoeArgs A) {
  E4B_TRACE_SCOPE(trace_tag(TR_MOE_TAIL, 0));
  __shared__ float red[4];
  const int H = A.H;
  // token row blockIdx.x of a batch (one block in the decode step)
  const int64_t ro = (int64_t)blockIdx.x * H;
  A.h = (A.attn_o ? A.h1 : A.h) + ro;
  A.dense_out += ro;
  A.moe_out += ro;
  A.h_out += ro;
  // every input requested before the first reduction waits
  float d[kTailPer], m[kTailPer], w1[kTailPer], w2[kTailPer], hv[kTailPer], wp[kTailPer];
#pragma unroll
  for (int k = 0; k < kTailPer; ++k) {
    const int i = min((int)threadIdx.x + 256 * k, H - 1);
    d[k] = A.dense_out[i];
    m[k] = A.moe_out[i];
    w1[k] = A.post_ffw1[i];
    w2[k] = A.post_ffw2[i];
    hv[k] = A.h[i];
    wp[k] = A.post_ffw[i];
  }
  float s1 = 0.f, s2 = 0.f;
#pragma unroll
  for (int k = 0; k < kTailPer; ++k) {
    const bool in = (int)threadIdx.x + 256 * k < H;
    d[k] = in ? d[k] : 0.f;
    m[k] = in ? m[k] : 0.f;
    s1 = fmaf(d[k], d[k], s1);
    s2 = fmaf(m[k], m[k], s2);
  }
  const float i1 = rms_inv(block_sum(s1, red), H, A.eps);
  const float i2 = rms_inv(block_sum(s2, red), H, A.eps);
  float s3 = 0.f;
#pragma unroll
  for (int k = 0; k < kTailPer; ++k) {
    d[k] = d[k] * i1 * w1[k] + m[k] * i2 * w2[k];  // comb (0 past H)
    s3 = fmaf(d[k], d[k], s3);
  }
  const float i3 = rms_inv(block_sum(s3, red), H, A.eps);
#pragma unroll
  for (int k = 0; k < kTailPer; ++k) {
    const int i = threadIdx.x + 256 * k;
    if (i < H) A.h_out[i] = (hv[k] + d[k] * i3 * wp[k]) * A.layer_scale;
  }
}

}  // namespace

#define ROUTER_LEAD(A) A.h, A.router_scale, A.attn_o, A.post_attn, A.router_w, (uint32_t)A.H | (uint32_t)A.E << 16, A
int launch_moe_router(const MoeArgs& A, hipStream_t st) {
  if (A.H % 4 || A.H / 4 > kRouterMaxH4) return e4b_fail(E4B_EINVAL, "router: H=%d (multiple of 4, <= 3072)", A.H);
  if (A.E < 1 || A.E > 0xffff) return e4b_fail(E4B_EINVAL, "router: %d experts", A.E);
  switch (A.attn_o ? (A.attn_o_slices ? A.attn_o_slices : 1) : 0) {
    case 0: hipLaunchKernelGGL(k_moe_router<0>, dim3((A.E + 1) / 2), dim3(128), 0, st, ROUTER_LEAD(A)); break;
    case 1: hipLaunchKernelGGL(k_moe_router<1>, dim3((A.E + 1) / 2), dim3(128), 0, st, ROUTER_LEAD(A)); break;
    case 2: hipLaunchKernelGGL(k_moe_router<2>, dim3((A.E + 1) / 2), dim3(128), 0, st, ROUTER_LEAD(A)); break;
    case 4: hipLaunchKernelGGL(k_moe_router<4>, dim3((A.E + 1) / 2), dim3(128), 0, st, ROUTER_LEAD(A)); break;
    default: return e4b_fail(E4B_EINVAL, "MoE layer: %d o-projection slices (1, 2 or 4)", A.attn_o_slices);
  }
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}

int launch_moe_ffn(const MoeArgs& A, hipStream_t st) {
  if (A.H % 256 || A.H > kMoeMaxH || A.H > 256 * kTailPer || A.FF % 32 || A.FF2 % 32 || A.FF % (2 * GU_U) ||
      A.FF2 / 32 > DD_LPR * DD_BPL || A.FF / 32 > DE_LPR * DE_BPL || A.FF2 > kMoeMaxX || K * A.FF > kMoeMaxX ||
      A.FF2 > 3 * 256 * 8 || K * A.FF > 3 * 256 * 8 || A.E < K || A.E > 256)
    return e4b_fail(E4B_EINVAL,
                    "MoE layer: unsupported shape (H=%d multiple of 256 <= 3072, FF2=%d <= 3072, FF=%d <= 768, "
                    "8 <= E=%d <= 256)",
                    A.H, A.FF2, A.FF, A.E);
  if (A.attn_o && (!A.post_attn || !A.h1 || A.h1 == A.h))
    return e4b_fail(E4B_EINVAL, "MoE layer: the attention residual needs post_attn and an h1 buffer apart from h");
  int rc = launch_moe_router(A, st);
  if (rc) return rc;
  const int64_t gu_tiles = (A.FF2 + (int64_t)K * A.FF) / (2 * GU_U);
  const int64_t gu_wgs = (gu_tiles + 3) / 4;  // one tile per wave
  hipLaunchKernelGGL(k_moe_gu, dim3((unsigned)gu_wgs), dim3(256), 0, st, A.scores, A.dense_gu.nib, A.dense_gu.sc,
                     A.exp_gu.nib, A.exp_gu.sc, (uint32_t)A.H | (uint32_t)A.E << 16,
                     (uint32_t)A.FF | (uint32_t)A.FF2 << 16, A);
  const int dd_tiles = (A.H + 2 * DD_R - 1) / (2 * DD_R), de_tiles = (A.H + DE_R - 1) / DE_R;
  const int nbd = (dd_tiles + 3) / 4, nbe = (de_tiles + 3) / 4;
  hipLaunchKernelGGL(k_moe_down, dim3(nbd + nbe), dim3(256), 0, st, A.topk_idx, A.exp_down.nib, A.exp_down.sc,
                     A.g_slots, A.g_dense, (uint32_t)A.H | (uint32_t)A.FF << 16, (uint32_t)A.FF2 | (uint32_t)nbd << 16,
                     A);
  if (A.h_out) hipLaunchKernelGGL(k_moe_tail, dim3(1), dim3(256), 0, st, A);
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}

int launch_moe_router_rows(const MoeArgs& A, int M, hipStream_t st) {
  if (A.H % 4 || A.H / 4 > kRouterMaxH4 || M < 1 || A.E < 1 || A.attn_o)
    return e4b_fail(E4B_EINVAL, "router rows: H=%d M=%d E=%d (no attention residual over rows)", A.H, M, A.E);
  hipLaunchKernelGGL(k_moe_router_rows, dim3((A.E + kRrE - 1) / kRrE, (M + kRrT - 1) / kRrT), dim3(128), 0, st, A, M);
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}

int launch_moe_topk_rows(const MoeArgs& A, int M, hipStream_t st) {
  if (A.E < K || A.E > 256 || M < 1) return e4b_fail(E4B_EINVAL, "top-8 rows: E=%d M=%d", A.E, M);
  hipLaunchKernelGGL(k_moe_topk, dim3(M), dim3(64), 0, st, A);
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}

int launch_moe_tail_rows(const MoeArgs& A, int M, hipStream_t st) {
  if (A.H > 256 * kTailPer || M < 1) return e4b_fail(E4B_EINVAL, "MoE tail rows: H=%d M=%d", A.H, M);
  hipLaunchKernelGGL(k_moe_tail, dim3(M), dim3(256), 0, st, A);
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}

int launch_moe_topk(const MoeArgs& A, hipStream_t st) {
  if (A.H % 4 || A.E < K || A.E > 256) return e4b_fail(E4B_EINVAL, "router: H=%d E=%d", A.H, A.E);
  int rc = launch_moe_router(A, st);
  if (rc) return rc;
  hipLaunchKernelGGL(k_moe_topk, dim3(1), dim3(64), 0, st, A);
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}
