// k_attn.hip -- decode attention for one layer: head prep (q/k weighted
// head-RMS + NeoX-half RoPE, v scale-less RMS; kernels/headprep.wgsl:19-87)
// with the K/V cache write of the new position, split-K softmax partials over
// the live positions (kernels/attsplit.wgsl:16-76) in one launch, and the
// log-sum-exp combine (kernels/attcomb.wgsl:10-36) in a second.
//
// The combine is its own launch on purpose: on this part a kernel boundary
// (~2.5 us) is the cheapest grid-wide ordering.  A last-block combine needs
// an agent-scope release/acquire pair per block (L2 write-back and
// invalidate across the 8 XCDs), which measured 5-9 us for 16-36 blocks.
//
// Split-K: the live positions are cut into chunks of CS (32 or 64)
// positions, one 512-thread block per (KV group, chunk); the grid is sized
// for the most live positions a layer can have and blocks past the live
// chunks exit.  Every K and V row of a chunk is requested before the head
// prep starts, so the chunk costs one memory round trip.  Inside the block
// the split goes one level further: wave w owns positions w, w+8, ... of
// the chunk and keeps its own softmax statistics, so scores, exponentials
// and P.V never leave the wave; one LDS merge per block folds the 8 waves.
//
// Cache layout [kv_head][slot][256] f16.  Sliding layers keep a ring of
// `slots` entries: position p lives in slot p % slots, and the live window is
// (pos - W, pos]; since slots >= W every live position still owns its slot,
// which is the SoundRec/Complete property of specs/KVRing.tla for decode.
// Iterating positions (instead of the reference's slot scan with position
// recovery, kernels/attnf32.wgsl:30-53) visits exactly the live slots.
#include "../../include/e4b.h"
#include "kernels.h"
#include "step.h"
#include "util.h"
#include "attn_prep.h"
#include "trace.h"

namespace {

constexpr int HD = 256;
constexpr int GQA = 4;

struct AttnArgs {
  const float* qkv;
  const float* qw;
  const float* kw;
  const float* inv_freq;
  const float2* rope;  // per-step (cos, sin) table, or null to evaluate sincosf here
  uint16_t* kc;
  uint16_t* vc;
  const uint32_t* params;
  uint32_t pos;
  int kv_idx;          // full layers: params[kv_idx] = the slot of this token (entries before it)
  float* part_o;
  float* part_ml;
  float* raw;          // full layers, may be null: raw scores [qh][slots] of the live slots
  uint16_t* out;
  int qh, kvh, angles, slots, window;
  float eps;
};

DEV void unpack16(const uint4& a, const uint4& b, float* f) {
  const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    f[2 * i] = h2f((uint16_t)(w[i] & 0xffff));
    f[2 * i + 1] = h2f((uint16_t)(w[i] >> 16));
  }
}

DEV float xmax16(float v) {
  float t = v;
  swapx16(v, t);
  return fmaxf(v, t);
}
DEV float xmax32(float v) {
  float t = v;
  swapx32(v, t);
  return fmaxf(v, t);
}

// One block of NW waves (8 or 4) per (KV group g, chunk c of CS positions, V
// slice z); wave w owns the chunk's positions j = w + NW k (k < CS/NW).  K is
// read as 16 lanes per position, lane dl holding dims 8dl..8dl+7 and
// 128+8dl..128+8dl+7 (two 256-byte contiguous halves per row), 4 positions
// per pass (lane group `sub` takes k = 4s + sub).  With NS > 1 the block
// handles V dims [VD z, VD z + VD) only (VD = 256 / NS): every slice computes
// the same scores and reads 1/NS of V, which spreads a chunk's memory traffic
// over NS CUs (the grid puts a chunk's slices on one XCD, so its K rows are
// fetched into that XCD's L2 once).  V is read as 16 B per lane, 8 dims each,
// 64/LV positions per load (LV = lanes per position).  With NW = 8 waves 4
// and 5 prep the new k and v rows; with NW = 4 waves 0 and 1 prep them after
// their q heads, in the chunk that owns the token only.
//
// The leading scalar arguments repeat the fields the first requests need
// (params, qkv, qw, kw, rope; qh | kvh << 16; pos; the index of the token's
// slot in params: 0 on sliding layers, kv_idx on full ones): the library is built with
// -amdgpu-kernarg-preload-count, so they arrive in SGPRs with the wave and
// no request waits for a kernel-argument load (struct arguments are not
// preloaded).
template <int CS, int NS, int NW = 8, bool RAW = false>
__global__ __launch_bounds__(64 * NW) void k_attn_split(const uint32_t* lparams, const float* lqkv, const float* lqw,
                                                        const float* lkw, const float2* lrope, uint32_t lheads,
                                                        uint32_t lpos, uint32_t lcur_idx, AttnArgs A) {
  A.params = lparams;
  A.qkv = lqkv;
  A.qw = lqw;
  A.kw = lkw;
  A.rope = lrope;
  A.qh = (int)(lheads & 0xffffu);
  A.kvh = (int)(lheads >> 16);
  A.pos = lpos;
  E4B_TRACE_SCOPE(trace_tag(TR_ATTN, A.window > 0 ? 0 : 1));
  constexpr int KP = CS / (4 * NW);  // score passes per wave (4 positions each)
  constexpr int VS = CS / NW;        // positions per wave
  constexpr int VD = HD / NS;        // V dims per block
  constexpr int LV = VD / 8;         // lanes per V row
  constexpr int PPL = 64 / LV;       // positions per V load
  constexpr int VQ = VS / PPL;       // V loads per lane
  static_assert(NW == 8 || NW == 4, "8 or 4 waves");
  static_assert(NS == 1 || NS == 2 || NS == 4, "one, two or four V slices");
  static_assert(KP >= 1 && VQ >= 1 && VS == VQ * PPL && CS == KP * 4 * NW, "positions per wave");
  __shared__ float qs[GQA][HD];
  __shared__ __align__(16) uint16_t knew[HD];
  __shared__ __align__(16) uint16_t vnew[HD];
  __shared__ __align__(16) float po[NW][GQA][VD];
  __shared__ float wml[NW][GQA][2];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = blockIdx.x, c = blockIdx.y, zs = NS == 1 ? 0 : (int)blockIdx.z;
  // 32-bit position arithmetic throughout (positions < 2^31): a 64-bit
  // modulo is a long software sequence on this ISA
  // `pos` rotates q and k; `cur` is the token's index in the cache's own
  // numbering: the position for sliding rings, the entry count for full
  // layers (equal to the position until a compaction moves entries)
  const int pos = (int)(A.params ? A.params[0] : A.pos);
  const int cur_raw = (int)(A.params ? A.params[lcur_idx] : A.pos);
  // the cache pointers (kernel-argument loads) are requested here too and
  // consumed after the position wait below, so the K/V requests do not wait
  // for a second kernel-argument round trip
  uint16_t* const kc0 = A.kc;
  uint16_t* const vc0 = A.vc;
  __builtin_amdgcn_sched_barrier(0);
  // 0a. the head-prep inputs do not depend on the position: they are
  //     requested while the position is in flight (this wave's q/k/v row,
  //     its norm weights, the RoPE (cos, sin) of its lane's dims; with
  //     NW = 8 waves 6-7 repeat wave 5's row and drop it; with NW = 4 waves
  //     0 and 1 also read the k and v rows)
  const int prow = NW == 8 ? (wave < 4 ? g * GQA + wave : A.qh + (wave == 4 ? 0 : A.kvh) + g) : g * GQA + wave;
  const float4 xin = *reinterpret_cast<const float4*>(A.qkv + (int64_t)prow * HD + 4 * lane);
  const float4 win = *reinterpret_cast<const float4*>((NW == 8 && wave >= 4 ? A.kw : A.qw) + 4 * lane);
  const int krow2 = A.qh + (wave == 0 ? 0 : A.kvh) + g;  // NW = 4: the k (wave 0) or v (wave 1) row
  float4 xin2 = make_float4(0.f, 0.f, 0.f, 0.f), win2 = xin2;
  if constexpr (NW == 4) {
    xin2 = *reinterpret_cast<const float4*>(A.qkv + (int64_t)krow2 * HD + 4 * lane);
    win2 = *reinterpret_cast<const float4*>(A.kw + 4 * lane);
  }
  const bool have_cs = A.rope != nullptr;
  const float2* rsrc = have_cs ? A.rope : reinterpret_cast<const float2*>(A.qkv);  // any readable 1 KB
  const float4 rc0 = reinterpret_cast<const float4*>(rsrc + 4 * (lane & 31))[0];
  const float4 rc1 = reinterpret_cast<const float4*>(rsrc + 4 * (lane & 31))[1];
  // the outputs' fields and the grid's chunk count in the same wait as the
  // caches' (read where they are used, at the final stores, they cost a
  // kernel-argument round trip at the end of every workgroup)
  const int gch = gridDim.y;  // partial stride: chunks allocated per head
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("" ::"s"(kc0), "s"(vc0), "s"(A.part_o), "s"(A.part_ml), "s"(gch));
  const int cur = A.window > 0 ? pos : cur_raw;
  const int lo = (A.window > 0 && cur + 1 > A.window) ? cur + 1 - A.window : 0;
  const int n = cur + 1 - lo;
  const int nch = (n + CS - 1) / CS;  // live chunks; the rest of the grid idles
  if (c >= nch) return;
  const int c_lo = lo + c * CS;
  const int m = min(CS, n - c * CS);
  const float fpos = (float)pos;
  uint16_t* kc = kc0 + (int64_t)g * A.slots * HD;
  uint16_t* vc = vc0 + (int64_t)g * A.slots * HD;
  // slot of position c_lo + j: one modulo per block; j < m <= window <= slots
  // so the ring index wraps at most once inside a chunk
  const int s_lo = A.window > 0 ? c_lo % A.slots : c_lo;
  auto slot_at = [&](int j) -> int64_t {
    const int s = s_lo + j;
    return (A.window > 0 && s >= A.slots) ? s - A.slots : s;
  };
  const int sub = lane >> 4, dl = lane & 15;
  const int vsub = lane / LV, vl = lane % LV, vd0 = VD * zs + 8 * vl;
  const bool owner = cur < c_lo + m;  // the last live chunk holds cur, at j = m - 1

  // 0b. the wave's K and V rows (index clamped into the chunk; the row of
  //     `pos` is not written yet and is replaced from LDS below), all
  //     requested before any math
  uint4 kr[KP][2];
  uint4 vr[VQ];
#pragma unroll
  for (int s = 0; s < KP; ++s) {
    const int j = min(wave + NW * (4 * s + sub), m - 1);
    const uint16_t* row = kc + slot_at(j) * HD;
    kr[s][0] = *reinterpret_cast<const uint4*>(row + 8 * dl);
    kr[s][1] = *reinterpret_cast<const uint4*>(row + 128 + 8 * dl);
  }
#pragma unroll
  for (int q = 0; q < VQ; ++q) {
    const int j = min(wave + NW * (PPL * q + vsub), m - 1);
    vr[q] = *reinterpret_cast<const uint4*>(vc + slot_at(j) * HD + vd0);
  }
  __builtin_amdgcn_sched_barrier(0);  // all loads in flight before the first wait
  E4B_TRACE_MARK(0);

  // 1. head prep: q heads 4g..4g+3 (waves 0-3), the new k and v rows
  //    (f16-rounded, as stored; NW = 8: waves 4 and 5, NW = 4: waves 0 and 1
  //    of the owner chunk); the chunk owning `pos` stores them
  const float2 cs[4] = {make_float2(rc0.x, rc0.y), make_float2(rc0.z, rc0.w), make_float2(rc1.x, rc1.y),
                        make_float2(rc1.z, rc1.w)};
  auto prep_kv = [&](float4 xr, float4 wr, bool is_k) {
    float x[4] = {xr.x, xr.y, xr.z, xr.w};
    const float w[4] = {wr.x, wr.y, wr.z, wr.w};
    prep_head_regs(x, w, is_k, cs, have_cs, A.inv_freq, A.angles, A.eps, fpos, is_k);
    const uint2 pk = make_uint2((uint32_t)f2h(x[0]) | ((uint32_t)f2h(x[1]) << 16),
                                (uint32_t)f2h(x[2]) | ((uint32_t)f2h(x[3]) << 16));
    *reinterpret_cast<uint2*>((is_k ? knew : vnew) + 4 * lane) = pk;
    if (owner && zs == 0) *reinterpret_cast<uint2*>((is_k ? kc : vc) + slot_at(m - 1) * HD + 4 * lane) = pk;
  };
  if (wave < 4) {
    float x[4] = {xin.x, xin.y, xin.z, xin.w};
    const float w[4] = {win.x, win.y, win.z, win.w};
    prep_head_regs(x, w, true, cs, have_cs, A.inv_freq, A.angles, A.eps, fpos, true);
#pragma unroll
    for (int i = 0; i < 4; ++i) qs[wave][4 * lane + i] = x[i];
  } else if (NW == 8 && wave < 6) {
    prep_kv(xin, win, wave == 4);
  }
  if (NW == 4 && owner && wave < 2) prep_kv(xin2, win2, wave == 0);
  lds_sync();
  E4B_TRACE_MARK(1);

  // 2. scores of the wave's positions: 16 lanes per position (16 dims each);
  //    after the reduction lane (sub, dl) holds head dl/4 of position
  //    k = 4s + sub
  float sc[KP];
  {
    float q[GQA][16];
#pragma unroll
    for (int h = 0; h < GQA; ++h)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        q[h][i] = qs[h][8 * dl + i];
        q[h][8 + i] = qs[h][128 + 8 * dl + i];
      }
#pragma unroll
    for (int s = 0; s < KP; ++s) {
      const int j = wave + NW * (4 * s + sub);
      uint4 ka = kr[s][0], kb = kr[s][1];
      if (c_lo + j == cur) {
        ka = *reinterpret_cast<const uint4*>(knew + 8 * dl);
        kb = *reinterpret_cast<const uint4*>(knew + 128 + 8 * dl);
      }
      float kf[16];
      unpack16(ka, kb, kf);
      float t[GQA];
#pragma unroll
      for (int h = 0; h < GQA; ++h) {
        float a = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) a = fmaf(q[h][i], kf[i], a);
        t[h] = a;
      }
      sc[s] = j < m ? reduce_rows<16, GQA>(t) : -3.0e38f;
      // raw scores for the mass of a scored full layer (lane dl % 4 == 0 of
      // each head; one V slice writes them)
      if (RAW && zs == 0 && j < m && (dl & 3) == 0)
        A.raw[(int64_t)(g * GQA + (dl >> 2)) * A.slots + slot_at(j)] = sc[s];
    }
  }
  E4B_TRACE_MARK(2);
  // 3. the wave's softmax statistics per head (lanes with equal dl/4 share
  //    a head): max and sum over the passes and the four lane groups
  float mx = sc[0];
#pragma unroll
  for (int s = 1; s < KP; ++s) mx = fmaxf(mx, sc[s]);
  mx = xmax32(xmax16(mx));
  float e[KP], ls = 0.f;
#pragma unroll
  for (int s = 0; s < KP; ++s) {
    e[s] = sc[s] > -1.0e38f ? __expf(sc[s] - mx) : 0.f;
    ls += e[s];
  }
  ls = xsum_step<32>(xsum_step<16>(ls));

  // 4. P.V over the wave's positions: lane covers dims vd0..vd0+7 of
  //    position i = PPL q + vsub; the weight of position k = 4s + sub, head h
  //    sits in lane 16 sub + 4h of e[s]
  {
    float acc[GQA][8];
#pragma unroll
    for (int h = 0; h < GQA; ++h)
#pragma unroll
      for (int d = 0; d < 8; ++d) acc[h][d] = 0.f;
    const uint4 vn = *reinterpret_cast<const uint4*>(vnew + vd0);
#pragma unroll
    for (int q = 0; q < VQ; ++q) {
      const int i = PPL * q + vsub;
      const int j = wave + NW * i;
      // a position past m reads a clamped, possibly stale row: zero it, so
      // its zero weight cannot meet a non-finite value
      const uint4 vv = (c_lo + j == cur) ? vn : (j < m ? vr[q] : make_uint4(0u, 0u, 0u, 0u));
      float vf[8];
      const uint32_t w4[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        vf[2 * t] = h2f((uint16_t)(w4[t] & 0xffff));
        vf[2 * t + 1] = h2f((uint16_t)(w4[t] >> 16));
      }
#pragma unroll
      for (int h = 0; h < GQA; ++h) {
        // zero for positions past m (e = 0 there), so no branch
        float pf;
        if constexpr (PPL == 2) {
          const int i0 = 2 * q, i1 = 2 * q + 1;
          const float p0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e[i0 >> 2]), 16 * (i0 & 3) + 4 * h));
          const float p1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e[i1 >> 2]), 16 * (i1 & 3) + 4 * h));
          pf = vsub ? p1 : p0;
        } else if constexpr (PPL == 4) {
          // position 4q + vsub lives in pass q, lane group vsub
          pf = __shfl(e[q], 16 * vsub + 4 * h, 64);
        } else {
          // PPL = 8: position 8q + vsub lives in pass 2q + vsub / 4, lane group vsub % 4
          const float p0 = __shfl(e[2 * q], 16 * (vsub & 3) + 4 * h, 64);
          const float p1 = __shfl(e[2 * q + 1], 16 * (vsub & 3) + 4 * h, 64);
          pf = vsub < 4 ? p0 : p1;
        }
#pragma unroll
        for (int d = 0; d < 8; ++d) acc[h][d] = fmaf(pf, vf[d], acc[h][d]);
      }
    }
    // fold the position groups: lanes < 32 keep heads 0, 1, lanes >= 32
    // heads 2, 3; with four or eight groups, bit 16 then picks one of the
    // two, and with eight groups the lanes 8 apart are added
    float r[2][8];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int d = 0; d < 8; ++d) r[hh][d] = tstep<32>(acc[hh][d], acc[hh + 2][d]);
    if constexpr (PPL == 2) {
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        float4* dst = reinterpret_cast<float4*>(&po[wave][hh + 2 * (lane >> 5)][8 * vl]);
        dst[0] = make_float4(r[hh][0], r[hh][1], r[hh][2], r[hh][3]);
        dst[1] = make_float4(r[hh][4], r[hh][5], r[hh][6], r[hh][7]);
      }
    } else {
      float t[8];
#pragma unroll
      for (int d = 0; d < 8; ++d) t[d] = tstep<16>(r[0][d], r[1][d]);
      if constexpr (PPL == 8) {
#pragma unroll
        for (int d = 0; d < 8; ++d) t[d] = xsum_step<8>(t[d]);
      }
      if (PPL == 4 || (lane & 8) == 0) {
        float4* dst = reinterpret_cast<float4*>(&po[wave][2 * (lane >> 5) + ((lane >> 4) & 1)][8 * vl]);
        dst[0] = make_float4(t[0], t[1], t[2], t[3]);
        dst[1] = make_float4(t[4], t[5], t[6], t[7]);
      }
    }
#pragma unroll
    for (int h = 0; h < GQA; ++h)
      if (lane == 4 * h) {
        wml[wave][h][0] = mx;
        wml[wave][h][1] = ls;
      }
  }
  lds_sync();
  E4B_TRACE_MARK(3);

  // 5. fold the NW waves (log-sum-exp) into this chunk's partials
  //    ([head][chunk][dim], [head][chunk][max, sum]); GQA x VD outputs, one
  //    or two (adjacent dims) per thread
  {
    constexpr int OPT = GQA * VD / (NW * 64);  // outputs per thread
    static_assert(OPT == 1 || OPT == 2, "outputs per thread");
    const int h = threadIdx.x / (VD / OPT), d = OPT * (threadIdx.x % (VD / OPT));
    float M = wml[0][h][0];
#pragma unroll
    for (int w = 1; w < NW; ++w) M = fmaxf(M, wml[w][h][0]);
    float v[OPT], L = 0.f;
#pragma unroll
    for (int u = 0; u < OPT; ++u) v[u] = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float f = __expf(wml[w][h][0] - M);  // 0 for a wave without positions
#pragma unroll
      for (int u = 0; u < OPT; ++u) v[u] = fmaf(po[w][h][d + u], f, v[u]);
      L = fmaf(wml[w][h][1], f, L);
    }
    const int64_t base = (int64_t)(g * GQA + h) * gch + c;
    float* dst = A.part_o + base * HD + VD * zs + d;
    if constexpr (OPT == 2) *reinterpret_cast<float2*>(dst) = make_float2(v[0], v[1]);
    else dst[0] = v[0];
    if (d == 0 && zs == 0) {
      A.part_ml[base * 2] = M;
      A.part_ml[base * 2 + 1] = L;
    }
  }
}

// log-sum-exp merge of the live chunks (kernels/attcomb.wgsl:10-36): block
// (h, y) merges q head h's output dims [64 y, 64 y + 64); wave g of the block
// accumulates chunks g, g + 4, ... of its lane's dim (every chunk's partial
// requested before the first use), and the four wave sums are added in LDS.
template <int CS>
__global__ __launch_bounds__(256) void k_attn_combine(const float* __restrict__ part_o,
                                                      const float* __restrict__ part_ml, const uint32_t* params,
                                                      uint32_t pos_imm, int kv_idx, int window, int gch,
                                                      uint16_t* __restrict__ out) {
  __shared__ float wt[kAttnMaxChunks];
  __shared__ float red[4];
  __shared__ float sums[4][64];
  const int h = blockIdx.x, d = 64 * (int)blockIdx.y + (threadIdx.x & 63), grp = threadIdx.x >> 6;
  const int pos = (int)(params ? params[window > 0 ? 0 : kv_idx] : pos_imm);
  const int lo = (window > 0 && pos + 1 > window) ? pos + 1 - window : 0;
  const int nch = (pos + 1 - lo + CS - 1) / CS;
  const float* ml = part_ml + (int64_t)h * gch * 2;
  // chunk weights exp(m_c - M) and the denominator sum_c l_c exp(m_c - M)
  float M = -3.0e38f;
  for (int cc = threadIdx.x; cc < nch; cc += 256) M = fmaxf(M, ml[2 * cc]);
  M = block_max(M, red);
  float den = 0.f;
  for (int cc = threadIdx.x; cc < nch; cc += 256) {
    const float f = __expf(ml[2 * cc] - M);
    wt[cc] = f;
    den = fmaf(ml[2 * cc + 1], f, den);
  }
  den = block_sum(den, red);
  lds_sync();
  const float* po = part_o + (int64_t)h * gch * HD + d;
  float acc = 0.f;
#pragma unroll 16
  for (int cc = grp; cc < nch; cc += 4) acc = fmaf(po[(int64_t)cc * HD], wt[cc], acc);
  sums[grp][threadIdx.x & 63] = acc;
  lds_sync();
  if (grp == 0) {
    const int t = threadIdx.x;
    out[h * HD + d] = f2h((sums[0][t] + sums[1][t] + sums[2][t] + sums[3][t]) / den);
  }
}

// attention mass of a scored full layer (kernels/attnos.wgsl:78-92, SCORE =
// 1): score[h][t] += e^(s_t - M) / den for the live slots t <= cur, where M
// and den = sum_c l_c e^(m_c - M) merge the split-K statistics of head h --
// the normalisation the combine applies.  Block (h, b) covers slots [256 b,
// 256 b + 256); the grid is sized for the capacity and blocks past the live
// slots exit.
template <int CS>
__global__ __launch_bounds__(256) void k_attn_score(const float* __restrict__ part_ml, const float* __restrict__ raw,
                                                    const uint32_t* params, int kv_idx, int gch, int slots,
                                                    float* __restrict__ score) {
  __shared__ float red[4];
  const int h = blockIdx.x, t = blockIdx.y * 256 + threadIdx.x;
  const int cur = (int)params[kv_idx];
  if ((int)blockIdx.y * 256 > cur) return;
  const int nch = (cur + 1 + CS - 1) / CS;
  const float* ml = part_ml + (int64_t)h * gch * 2;
  float M = -3.0e38f;
  for (int c = threadIdx.x; c < nch; c += 256) M = fmaxf(M, ml[2 * c]);
  M = block_max(M, red);
  float den = 0.f;
  for (int c = threadIdx.x; c < nch; c += 256) den = fmaf(ml[2 * c + 1], __expf(ml[2 * c] - M), den);
  den = block_sum(den, red);
  if (t <= cur) {
    const int64_t o = (int64_t)h * slots + t;
    score[o] = score[o] + __expf(raw[o] - M) / den;
  }
}

// compaction gather (kernels/kvgather.wgsl): dst[g][i] = src[g][keep[i]] for
// K and V, block (i, g), 256 dims per row as 32 threads x 16 bytes
__global__ __launch_bounds__(64) void k_kv_gather(const uint32_t* __restrict__ keep, const uint16_t* __restrict__ kc,
                                                  const uint16_t* __restrict__ vc, int slots, uint16_t* __restrict__ dk,
                                                  uint16_t* __restrict__ dv, int dslots) {
  const int i = blockIdx.x, g = blockIdx.y, t = threadIdx.x & 31;
  const int64_t src = ((int64_t)g * slots + keep[i]) * HD + 8 * t;
  const int64_t dst = ((int64_t)g * dslots + i) * HD + 8 * t;
  if (threadIdx.x < 32)
    *reinterpret_cast<uint4*>(dk + dst) = *reinterpret_cast<const uint4*>(kc + src);
  else
    *reinterpret_cast<uint4*>(dv + dst) = *reinterpret_cast<const uint4*>(vc + src);
}

}  // namespace

int launch_attn_score(const float* part_ml, const float* raw, const uint32_t* params, int kv_idx, int qh, int slots,
                      int chunk, float* score, hipStream_t st) {
  if (chunk != 32 && chunk != 64) return e4b_fail(E4B_EINVAL, "attention score: chunk %d", chunk);
  const int gch = attn_chunks(slots, chunk);
  const dim3 grid(qh, (slots + 255) / 256);
  if (chunk == 64)
    hipLaunchKernelGGL(k_attn_score<64>, grid, dim3(256), 0, st, part_ml, raw, params, kv_idx, gch, slots, score);
  else
    hipLaunchKernelGGL(k_attn_score<32>, grid, dim3(256), 0, st, part_ml, raw, params, kv_idx, gch, slots, score);
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}

int launch_kv_gather(const uint32_t* keep, int n, const uint16_t* kc, const uint16_t* vc, int kvh, int slots,
                     uint16_t* dk, uint16_t* dv, int dslots, hipStream_t st) {
  if (n <= 0) return E4B_OK;
  if (n > dslots) return e4b_fail(E4B_EINVAL, "kv gather: %d rows into %d", n, dslots);
  hipLaunchKernelGGL(k_kv_gather, dim3(n, kvh), dim3(64), 0, st, keep, kc, vc, slots, dk, dv, dslots);
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}

int attn_chunks(int max_positions, int chunk) { return (max_positions + chunk - 1) / chunk; }

int launch_attn(const AttnLaunch& a, hipStream_t st) {
  if (a.hd != HD || a.qh != GQA * a.kvh)
    return e4b_fail(E4B_EINVAL, "attention kernel supports head_dim 256 and 4 q heads per kv head (got %d, %d/%d)", a.hd,
                    a.qh, a.kvh);
  if (a.chunk != 32 && a.chunk != 64) return e4b_fail(E4B_EINVAL, "attention: chunk %d is not 32 or 64", a.chunk);
  const int span = a.window > 0 ? a.window : a.slots;  // most live positions
  if (a.window > a.slots) return e4b_fail(E4B_EINVAL, "attention: window %d exceeds %d ring slots", a.window, a.slots);
  const int nch = attn_chunks(span, a.chunk);
  if (nch > kAttnMaxChunks)
    return e4b_fail(E4B_EINVAL, "attention: %d positions need %d chunks of %d (max %d)", span, nch, a.chunk,
                    kAttnMaxChunks);
  AttnArgs A;
  A.qkv = a.qkv;
  A.qw = a.qw;
  A.kw = a.kw;
  A.inv_freq = a.inv_freq;
  A.rope = a.rope;
  A.kc = a.kc;
  A.vc = a.vc;
  A.params = a.params;
  A.pos = a.pos;
  A.kv_idx = a.kv_idx;
  A.part_o = a.part_o;
  A.part_ml = a.part_ml;
  A.raw = a.window > 0 ? nullptr : a.raw;
  A.out = a.out;
  A.qh = a.qh;
  A.kvh = a.kvh;
  A.angles = a.angles;
  A.slots = a.slots;
  A.window = a.window;
  A.eps = a.eps;
  if (a.vslices != 2 && a.vslices != 4) return e4b_fail(E4B_EINVAL, "attention: %d V slices (2 or 4)", a.vslices);
  if (a.qh > 0xffff || a.kvh > 0xffff) return e4b_fail(E4B_EINVAL, "attention: %d q / %d KV heads", a.qh, a.kvh);
#define ATTN_LEAD(A) A.params, A.qkv, A.qw, A.kw, A.rope, (uint32_t)A.qh | (uint32_t)A.kvh << 16, A.pos, \
                     (uint32_t)(A.window > 0 ? 0 : A.kv_idx), A
  const dim3 grid(a.kvh, nch, a.vslices);
  if (a.vslices == 4) {
    // 4 waves a block, 64-dim V slices
    if (a.chunk == 64) {
      if (A.raw)
        hipLaunchKernelGGL((k_attn_split<64, 4, 4, true>), grid, dim3(256), 0, st, ATTN_LEAD(A));
      else
        hipLaunchKernelGGL((k_attn_split<64, 4, 4>), grid, dim3(256), 0, st, ATTN_LEAD(A));
    } else {
      if (A.raw)
        hipLaunchKernelGGL((k_attn_split<32, 4, 4, true>), grid, dim3(256), 0, st, ATTN_LEAD(A));
      else
        hipLaunchKernelGGL((k_attn_split<32, 4, 4>), grid, dim3(256), 0, st, ATTN_LEAD(A));
    }
  } else if (a.chunk == 64) {
    if (A.raw)
      hipLaunchKernelGGL((k_attn_split<64, 2, 8, true>), grid, dim3(512), 0, st, ATTN_LEAD(A));
    else
      hipLaunchKernelGGL((k_attn_split<64, 2, 8>), grid, dim3(512), 0, st, ATTN_LEAD(A));
  } else {
    if (A.raw)
      hipLaunchKernelGGL((k_attn_split<32, 2, 8, true>), grid, dim3(512), 0, st, ATTN_LEAD(A));
    else
      hipLaunchKernelGGL((k_attn_split<32, 2, 8>), grid, dim3(512), 0, st, ATTN_LEAD(A));
  }
  if (a.combine) {
    if (a.chunk == 64)
      hipLaunchKernelGGL(k_attn_combine<64>, dim3(a.qh, HD / 64), dim3(256), 0, st, a.part_o, a.part_ml, a.params, a.pos,
                         a.kv_idx, a.window, nch, a.out);
    else
      hipLaunchKernelGGL(k_attn_combine<32>, dim3(a.qh, HD / 64), dim3(256), 0, st, a.part_o, a.part_ml, a.params, a.pos,
                         a.kv_idx, a.window, nch, a.out);
  }
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}
