// k_a4b.hip -- step kernels of the A4B recipe (src/engine-a4b.js:424-463)
// that the E4B kernels do not cover:
//   k_rownorm      residual + RMSNorm of one vector, any hidden size up to
//                  4096 (kernels/rmsacc3.wgsl:36-53, kernels/rmsnorm.wgsl
//                  :13-51; one workgroup)
//   k_attn_gen     one layer's decode attention for head dim 256 or 512 and
//                  1-8 q heads per KV head: head prep (q/k weighted head-RMS +
//                  NeoX RoPE over the first `angles` pairs, scale-less v RMS,
//                  V from the raw K slice on KEQV layers; kernels/headprep.wgsl
//                  :19-87) with the K/V row write at the token's slot, then
//                  the split-K partials of one (KV group, chunk of 64
//                  positions, 128 V dims): scale-1.0 scores of every q head
//                  of the group, the chunk's max and exponential sum, the
//                  unnormalised P.V (kernels/attsplit.wgsl:16-76 over the
//                  ring of attnf32.wgsl:21-105 or the counted slots of
//                  attnos.wgsl:22-98)
//   k_attn_merge   log-sum-exp merge of a head's live chunks to f16
//                  (kernels/attcomb.wgsl:10-36)
#include "../../include/e4b.h"
#include "a4b.h"
#include "kernels.h"
#include "util.h"
#include "trace.h"

namespace {

constexpr int kRowMax = 16;  // elements per thread of k_rownorm: H <= 16 * 256
constexpr int kRowSlices = 4;  // split-K slices k_rownorm sums at most

// thread t owns the elements i = t + 256 k
__global__ __launch_bounds__(256) void k_rownorm(const float* __restrict__ h_in, float* __restrict__ h_out,
                                                 const float* __restrict__ a, const float* __restrict__ w1, float scale,
                                                 const float* __restrict__ w2, uint16_t* __restrict__ x,
                                                 uint16_t* __restrict__ xlo, int H, float eps, int na,
                                                 int64_t a_slice) {
  E4B_TRACE_SCOPE(trace_tag(TR_ROWNORM, 0));
  __shared__ float red[4];
  const int t = threadIdx.x;
  // row blockIdx.x of a batch (one row in the decode step)
  const int64_t ro = (int64_t)blockIdx.x * H;
  h_in += ro;
  if (h_out) h_out += ro;
  if (a) a += ro;
  if (x) x += ro;
  if (xlo) xlo += ro;
  float hv[kRowMax], av[kRowMax];
#pragma unroll
  for (int k = 0; k < kRowMax; ++k) {
    const int i = t + 256 * k;
    hv[k] = i < H ? h_in[i] : 0.f;
    av[k] = (a && i < H) ? a[i] : 0.f;
  }
  if (a && na > 1) {
    // slices 1 .. kRowSlices - 1 requested together (clamped to the last
    // slice, added only below na)
    float sv[kRowSlices - 1][kRowMax];
#pragma unroll
    for (int s = 1; s < kRowSlices; ++s)
#pragma unroll
      for (int k = 0; k < kRowMax; ++k) {
        const int i = min(t + 256 * k, H - 1);
        sv[s - 1][k] = a[min(s, na - 1) * a_slice + i];
      }
#pragma unroll
    for (int s = 1; s < kRowSlices; ++s)
#pragma unroll
      for (int k = 0; k < kRowMax; ++k)
        if (s < na && t + 256 * k < H) av[k] += sv[s - 1][k];
  }
  if (a) {
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < kRowMax; ++k) ss = fmaf(av[k], av[k], ss);
    const float inv1 = rms_inv(block_sum(ss, red), H, eps);
#pragma unroll
    for (int k = 0; k < kRowMax; ++k) {
      const int i = t + 256 * k;
      if (i < H) hv[k] = hv[k] + av[k] * inv1 * w1[i];
    }
  }
  float s2 = 0.f;
#pragma unroll
  for (int k = 0; k < kRowMax; ++k) {
    hv[k] *= scale;
    s2 = fmaf(hv[k], hv[k], s2);
  }
  if (h_out) {
    lds_sync();  // every thread has read h_in before any writes h_out (they may alias)
#pragma unroll
    for (int k = 0; k < kRowMax; ++k) {
      const int i = t + 256 * k;
      if (i < H) h_out[i] = hv[k];
    }
  }
  if (!x) return;
  const float inv2 = w2 ? rms_inv(block_sum(s2, red), H, eps) : 1.f;
#pragma unroll
  for (int k = 0; k < kRowMax; ++k) {
    const int i = t + 256 * k;
    if (i < H) {
      const float y = w2 ? hv[k] * inv2 * w2[i] : hv[k];
      const _Float16 yh = (_Float16)y;
      x[i] = __builtin_bit_cast(uint16_t, yh);
      if (xlo) xlo[i] = __builtin_bit_cast(uint16_t, (_Float16)(y - (float)yh));
    }
  }
}

// live positions of the layer at this step: (lo, n) with the token's index
// `cur` in the cache's own numbering (the position on a ring, the counted
// slot on a full layer)
struct Live {
  int cur, lo, n;
};
// (from the loaded position and slot word params[kv_idx])
DEV Live live_at(const AttnGen& A, int pos, int slot) {
  Live L;
  L.cur = A.window > 0 ? pos : slot;
  L.lo = (A.window > 0 && L.cur + 1 > A.window) ? L.cur + 1 - A.window : 0;
  L.n = L.cur + 1 - L.lo;
  return L;
}
DEV Live live_of(const AttnGen& A) { return live_at(A, (int)A.params[0], (int)A.params[A.kv_idx]); }

// Block (KV group g, chunk c, V slice z), 8 waves.  Every load is issued
// before any math: the head-prep rows of the wave (q heads g GQA + r, the k
// head, the v head; 10 rows at GQA 8 take two passes of the 8 waves), the
// K rows of the wave's positions j = w + 8 i (lane l: dims [PER l, PER l +
// PER)), and their V dims [128 z + 2 l, 128 z + 2 l + 2).  The row of the
// token itself is not in the cache yet: it comes from the head prep (LDS),
// and the chunk that owns it (the last live one, slice 0) stores it.
// Scores: per position GQA dot products reduced across the wave
// (reduce_rows), stored to LDS; softmax statistics of head h by wave h over
// the chunk's 64 positions; P.V with the weights broadcast from LDS, folded
// over the 8 waves.  A chunk's K is read by all HD / VD slices (from L2
// after the first); V is split across them.
//
// The leading scalar arguments repeat the fields the first requests need
// (params, qkv, qw, kw, rope; qh | kvh << 16 | keqv << 31; angles; the
// index of the token's slot word in params: 0 on sliding layers, kv_idx on
// full ones): the library is built with -amdgpu-kernarg-preload-count, so
// they arrive in SGPRs with the wave and no request waits for a
// kernel-argument load (struct arguments are not preloaded).  The head-prep
// rows and the RoPE table do not depend on the position: they are requested
// while the position is in flight.
// V dims per slice (blockIdx.z): 128 at head dim 256; at head dim 512 the
// V slice width is a build knob (128: 4 slices that each read the chunk's
// K rows; 256: 2 slices, half the K reads, twice the P.V work a block).
// Measured at the A4B shape: 256 gave 775.5 tok/s against 777.9 for 128,
// so 128 is the default.
#ifndef E4B_TUNE_GEN512_VD
#define E4B_TUNE_GEN512_VD 128
#endif
constexpr int gen_vd(int hd) { return hd == 512 ? E4B_TUNE_GEN512_VD : 128; }
static_assert(gen_vd(512) == 128 || gen_vd(512) == 256, "V slice width");

template <int HD, int GQA, bool RAW>
__global__ __launch_bounds__(512) void k_attn_gen(const uint32_t* lparams, const float* lqkv, const float* lqw,
                                                  const float* lkw, const float2* lrope, uint32_t lheads,
                                                  uint32_t langles, uint32_t lslot_idx, AttnGen A) {
  A.params = lparams;
  A.qkv = lqkv;
  A.qw = lqw;
  A.kw = lkw;
  A.rope = lrope;
  A.qh = (int)(lheads & 0x7fffu);
  A.kvh = (int)((lheads >> 16) & 0x7fffu);
  A.keqv = (lheads >> 31) != 0;
  A.angles = (int)langles;
  E4B_TRACE_SCOPE(trace_tag(TR_ATTN_GEN, HD));
  constexpr int NW = 8, CS = kAttnGenChunk, PER = HD / 64, PW = CS / NW, VD = gen_vd(HD);
  constexpr int VW = VD / 128;  // 32-bit words (f16 pairs) of V a lane holds per position
  constexpr int NR = GQA + 2, RPW = (NR + NW - 1) / NW, LPH = 64 / GQA;
  static_assert(CS == 64 && GQA <= NW && (GQA & (GQA - 1)) == 0, "64-position chunks, GQA 1/2/4/8");
  __shared__ __align__(16) float qs[GQA][HD];
  __shared__ __align__(16) uint16_t knew[HD];
  __shared__ __align__(16) uint16_t vnew[HD];
  __shared__ float es[GQA][CS];
  __shared__ float mls[GQA][2];
  __shared__ __align__(16) float po[NW][GQA][VD];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = blockIdx.x, c = blockIdx.y, zs = blockIdx.z;
  const uint32_t pos_w = A.params[0], slot_w = A.params[lslot_idx];
  // the cache pointers (kernel-argument loads) are requested here too and
  // consumed after the position wait below, so the K/V requests do not wait
  // for a second kernel-argument round trip
  uint16_t* kc0 = A.kc;
  uint16_t* vc0 = A.vc;
  __builtin_amdgcn_sched_barrier(0);

  // 0. loads: head-prep rows and weights and the RoPE table (while the
  //    position is in flight), then the wave's K rows and V dims
  float xin[RPW][PER], win[RPW][PER];
#pragma unroll
  for (int u = 0; u < RPW; ++u) {
    const int r = min(wave + NW * u, NR - 1);
    const int src = r < GQA ? g * GQA + r : r == GQA || A.keqv ? A.qh + g : A.qh + A.kvh + g;
    const float* xr = A.qkv + (int64_t)src * HD + PER * lane;
    const float* wr = (r == GQA ? A.kw : A.qw) + PER * lane;  // v rows use no weight
#pragma unroll
    for (int e = 0; e < PER; e += 4) {
      const float4 t = *reinterpret_cast<const float4*>(xr + e);
      const float4 w = *reinterpret_cast<const float4*>(wr + e);
      xin[u][e] = t.x, xin[u][e + 1] = t.y, xin[u][e + 2] = t.z, xin[u][e + 3] = t.w;
      win[u][e] = w.x, win[u][e + 1] = w.y, win[u][e + 2] = w.z, win[u][e + 3] = w.w;
    }
  }
  // the step's (cos, sin) of this lane's pairs (p = PER (l mod 32) + e),
  // index clamped into the rotated range (absent table: any readable row)
  const bool have_cs = A.rope != nullptr;
  const float2* rsrc = have_cs ? A.rope : reinterpret_cast<const float2*>(A.qkv);
  float2 rc[PER];
#pragma unroll
  for (int e = 0; e < PER; ++e) rc[e] = rsrc[min(PER * (lane & 31) + e, max(A.angles - 1, 0))];
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("" ::"s"(kc0), "s"(vc0));
  const Live L = live_at(A, (int)pos_w, (int)slot_w);
  const int nch = (L.n + CS - 1) / CS;
  if (c >= nch) return;
  const int c_lo = L.lo + c * CS;
  const int m = min(CS, L.n - c * CS);
  uint16_t* kc = kc0 + (int64_t)g * A.slots * HD;
  uint16_t* vc = vc0 + (int64_t)g * A.slots * HD;
  // one modulo per block: j < m <= window <= slots, the ring wraps at most once
  const int s_lo = A.window > 0 ? c_lo % A.slots : c_lo;
  auto slot_at = [&](int j) -> int64_t {
    const int s = s_lo + j;
    return (A.window > 0 && s >= A.slots) ? s - A.slots : s;
  };
  uint32_t kr[PW][PER / 2];
  uint32_t vr[PW][VW];
#pragma unroll
  for (int i = 0; i < PW; ++i) {
    const int64_t sl = slot_at(min(wave + NW * i, m - 1));
    const uint32_t* krow = reinterpret_cast<const uint32_t*>(kc + sl * HD + PER * lane);
    if constexpr (PER == 4) {
      const uint2 t = *reinterpret_cast<const uint2*>(krow);
      kr[i][0] = t.x, kr[i][1] = t.y;
    } else {
      const uint4 t = *reinterpret_cast<const uint4*>(krow);
      kr[i][0] = t.x, kr[i][1] = t.y, kr[i][2] = t.z, kr[i][3] = t.w;
    }
    const uint16_t* vp = vc + sl * HD + VD * zs + 2 * VW * lane;
    if constexpr (VW == 1) {
      vr[i][0] = *reinterpret_cast<const uint32_t*>(vp);
    } else {
      const uint2 t = *reinterpret_cast<const uint2*>(vp);
      vr[i][0] = t.x, vr[i][1] = t.y;
    }
  }
  __builtin_amdgcn_sched_barrier(0);  // every load in flight before the first wait

  // 1. head prep: weighted head-RMS (v: scale-less), RoPE on q and k over the
  //    first `angles` pairs (p, p + HD/2) -- dim p of lane l < 32 pairs with
  //    the same register of lane l + 32
  const bool owner = c == nch - 1;  // the last live chunk holds the token, at j = m - 1
  const float fpos = (float)pos_w;
#pragma unroll
  for (int u = 0; u < RPW; ++u) {
    const int r = wave + NW * u;
    if (r >= NR) break;
    float* x = xin[u];
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < PER; ++e) ss = fmaf(x[e], x[e], ss);
    const float inv = rms_inv(wave_sum(ss), HD, A.eps);
#pragma unroll
    for (int e = 0; e < PER; ++e) x[e] = x[e] * inv * (r <= GQA ? win[u][e] : 1.f);
    if (r <= GQA) {
      const bool hi = lane >= 32;
#pragma unroll
      for (int e = 0; e < PER; ++e) {
        float lo_v = x[e], hi_v = x[e];
        swapx32(lo_v, hi_v);  // lanes < 32: hi_v = dim p + HD/2; lanes >= 32: lo_v = dim p
        const float partner = hi ? lo_v : hi_v;
        const int p = PER * (lane & 31) + e;
        if (p < A.angles) {
          float sn = rc[e].y, cs = rc[e].x;
          if (!have_cs) sincosf(fpos * A.inv_freq[p], &sn, &cs);
          x[e] = hi ? (partner * sn + x[e] * cs) : (x[e] * cs - partner * sn);
        }
      }
    }
    if (r < GQA) {
#pragma unroll
      for (int e = 0; e < PER; ++e) qs[r][PER * lane + e] = x[e];
    } else {
      uint16_t* dst = r == GQA ? knew : vnew;
#pragma unroll
      for (int e = 0; e < PER; ++e) dst[PER * lane + e] = f2h(x[e]);
      if (owner && zs == 0) {
        uint16_t* cache = (r == GQA ? kc : vc) + slot_at(m - 1) * HD + PER * lane;
#pragma unroll
        for (int e = 0; e < PER; ++e) cache[e] = f2h(x[e]);
      }
    }
  }
  lds_sync();

  // 2. scores of the wave's positions, all GQA heads: lane l ends with head
  //    l / LPH of position j
  {
    float q[GQA][PER];
#pragma unroll
    for (int h = 0; h < GQA; ++h)
#pragma unroll
      for (int e = 0; e < PER; ++e) q[h][e] = qs[h][PER * lane + e];
#pragma unroll
    for (int i = 0; i < PW; ++i) {
      const int j = wave + NW * i;
      uint32_t kw[PER / 2];
#pragma unroll
      for (int e = 0; e < PER / 2; ++e)
        kw[e] = (c_lo + j == L.cur) ? reinterpret_cast<const uint32_t*>(knew)[PER / 2 * lane + e] : kr[i][e];
      float t[GQA];
#pragma unroll
      for (int h = 0; h < GQA; ++h) {
        float a = 0.f;
#pragma unroll
        for (int e = 0; e < PER / 2; ++e) {
          a = fmaf(q[h][2 * e], h2f((uint16_t)(kw[e] & 0xffffu)), a);
          a = fmaf(q[h][2 * e + 1], h2f((uint16_t)(kw[e] >> 16)), a);
        }
        t[h] = a;
      }
      const float sc = reduce_rows<64, GQA>(t);
      if ((lane % LPH) == 0 && j < m) {
        es[lane / LPH][j] = sc;
        // raw scores for the mass of a scored full layer (one V slice writes them)
        if (RAW && zs == 0) A.raw[(int64_t)(g * GQA + lane / LPH) * A.slots + slot_at(j)] = sc;
      }
    }
  }
  lds_sync();

  // 3. softmax statistics of head h (wave h, lane = position)
  if (wave < GQA) {
    const float sv = lane < m ? es[wave][lane] : -3.0e38f;
    const float M = wave_max(sv);
    const float e = lane < m ? __expf(sv - M) : 0.f;
    const float l = wave_sum(e);
    es[wave][lane] = e;
    if (lane == 0) {
      mls[wave][0] = M;
      mls[wave][1] = l;
    }
  }
  lds_sync();

  // 4. P.V over the wave's positions, V dims VD z + 2 VW l .. 2 VW l + 2 VW - 1
  {
    float acc[GQA][2 * VW];
#pragma unroll
    for (int h = 0; h < GQA; ++h)
#pragma unroll
      for (int u = 0; u < 2 * VW; ++u) acc[h][u] = 0.f;
    uint32_t vn[VW];
#pragma unroll
    for (int w = 0; w < VW; ++w) vn[w] = reinterpret_cast<const uint32_t*>(vnew)[VD / 2 * zs + VW * lane + w];
#pragma unroll
    for (int i = 0; i < PW; ++i) {
      const int j = wave + NW * i;
#pragma unroll
      for (int w = 0; w < VW; ++w) {
        // positions past m read a clamped row; their weight is 0 and the row is zeroed
        const uint32_t vv = (c_lo + j == L.cur) ? vn[w] : (j < m ? vr[i][w] : 0u);
        const float v0 = h2f((uint16_t)(vv & 0xffffu)), v1 = h2f((uint16_t)(vv >> 16));
#pragma unroll
        for (int h = 0; h < GQA; ++h) {
          const float p = es[h][j];
          acc[h][2 * w] = fmaf(p, v0, acc[h][2 * w]);
          acc[h][2 * w + 1] = fmaf(p, v1, acc[h][2 * w + 1]);
        }
      }
    }
#pragma unroll
    for (int h = 0; h < GQA; ++h)
#pragma unroll
      for (int w = 0; w < VW; ++w)
        *reinterpret_cast<float2*>(&po[wave][h][2 * VW * lane + 2 * w]) = make_float2(acc[h][2 * w], acc[h][2 * w + 1]);
  }
  lds_sync();

  // 5. fold the 8 waves into this chunk's partials ([q head][chunk][dim],
  //    [q head][chunk][max, sum])
  for (int o = threadIdx.x; o < GQA * VD; o += 64 * NW) {
    const int h = o / VD, d = o % VD;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) v += po[w][h][d];
    A.part_o[((int64_t)(g * GQA + h) * A.gch + c) * HD + VD * zs + d] = v;
  }
  if (zs == 0 && threadIdx.x < GQA) {
    const int64_t b = (int64_t)(g * GQA + threadIdx.x) * A.gch + c;
    A.part_ml[2 * b] = mls[threadIdx.x][0];
    A.part_ml[2 * b + 1] = mls[threadIdx.x][1];
  }
}

// one block per head: out = sum_c e^(m_c - M) part_o[c] / sum_c e^(m_c - M) l_c.
// Thread t: output dims t + 256 q, and the (max, sum) of chunk t.  The first
// U chunks' outputs are requested with the statistics, before the reductions
// wait; further chunks follow U at a time.
constexpr int kMergeMaxChunks = kAttnGenMaxChunks;

template <int HD>
__global__ __launch_bounds__(256) void k_attn_merge(AttnGen A) {
  E4B_TRACE_SCOPE(trace_tag(TR_ATTN_MERGE, 0));
  constexpr int CS = kAttnGenChunk, U = 16, DPT = HD / 256;
  __shared__ float wts[kMergeMaxChunks];
  __shared__ float red[4];
  const int h = blockIdx.x, t = threadIdx.x;
  const Live L = live_of(A);
  const int nch = (L.n + CS - 1) / CS;
  const float* ml = A.part_ml + (int64_t)h * A.gch * 2;
  const float* po = A.part_o + (int64_t)h * A.gch * HD + t;
  float v[U][DPT];
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int q = 0; q < DPT; ++q) v[u][q] = po[(int64_t)min(u, nch - 1) * HD + 256 * q];
  const int tc = min(t, nch - 1);
  const float mt = ml[2 * tc], lt = ml[2 * tc + 1];
  __builtin_amdgcn_sched_barrier(0);
  const float M = block_max(t < nch ? mt : -3.0e38f, red);
  const float f = t < nch ? __expf(mt - M) : 0.f;
  const float den = block_sum(t < nch ? lt * f : 0.f, red);
  wts[t] = f;
  lds_sync();
  float acc[DPT];
#pragma unroll
  for (int q = 0; q < DPT; ++q) acc[q] = 0.f;
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int q = 0; q < DPT; ++q) acc[q] = fmaf(wts[u], v[u][q], acc[q]);  // wts = 0 past nch
  for (int c0 = U; c0 < nch; c0 += U) {
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int q = 0; q < DPT; ++q) v[u][q] = po[(int64_t)min(c0 + u, nch - 1) * HD + 256 * q];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int q = 0; q < DPT; ++q) acc[q] = fmaf(c0 + u < nch ? wts[c0 + u] : 0.f, v[u][q], acc[q]);
  }
#pragma unroll
  for (int q = 0; q < DPT; ++q) A.out[(int64_t)h * HD + t + 256 * q] = f2h(acc[q] / den);
}

// ---- batched prefill ----------------------------------------------------------
// one wave per (head row r, token m): q heads [0, qh), k heads [qh, qh + kvh),
// v heads [qh + kvh, qh + 2 kvh) (V from the K slice on KEQV layers); lane l
// holds dims [PER l, PER l + PER), the RoPE partner of dim p < HD / 2 in lane
// l + 32 (kernels/headprep.wgsl:19-87 per token)
template <int HD>
__global__ __launch_bounds__(64) void k_headprep_rows_gen(HeadRowsGen A) {
  constexpr int PER = HD / 64;
  const int r = blockIdx.x, m = blockIdx.y, lane = threadIdx.x;
  const int QH = A.qh, KVH = A.kvh;
  const int kind = r < QH ? 0 : r < QH + KVH ? 1 : 2;  // q, k, v
  const int g = kind == 0 ? r : kind == 1 ? r - QH : r - QH - KVH;
  const int src = kind == 0 ? r : kind == 1 || A.keqv ? QH + g : QH + KVH + g;
  const float* xr = A.qkv + (int64_t)m * A.ld + (int64_t)src * HD + PER * lane;
  const float* wr = (kind == 1 ? A.kw : A.qw) + PER * lane;  // v rows use no weight
  float x[PER], w[PER];
#pragma unroll
  for (int e = 0; e < PER; e += 4) {
    const float4 t = *reinterpret_cast<const float4*>(xr + e);
    const float4 u = *reinterpret_cast<const float4*>(wr + e);
    x[e] = t.x, x[e + 1] = t.y, x[e + 2] = t.z, x[e + 3] = t.w;
    w[e] = u.x, w[e + 1] = u.y, w[e + 2] = u.z, w[e + 3] = u.w;
  }
  for (int s = 1; s < A.ks; ++s)  // the GEMM's K slices, in slice order
#pragma unroll
    for (int e = 0; e < PER; e += 4) {
      const float4 t = *reinterpret_cast<const float4*>(xr + s * A.slice + e);
      x[e] += t.x, x[e + 1] += t.y, x[e + 2] += t.z, x[e + 3] += t.w;
    }
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < PER; ++e) ss = fmaf(x[e], x[e], ss);
  const float inv = rms_inv(wave_sum(ss), HD, A.eps);
#pragma unroll
  for (int e = 0; e < PER; ++e) x[e] = x[e] * inv * (kind < 2 ? w[e] : 1.f);
  const uint32_t pos = A.p0 + (uint32_t)m;
  if (kind < 2) {
    const float fpos = (float)pos;
    const bool hi = lane >= 32;
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      float lo_v = x[e], hi_v = x[e];
      swapx32(lo_v, hi_v);  // lanes < 32: hi_v = dim p + HD/2; lanes >= 32: lo_v = dim p
      const float partner = hi ? lo_v : hi_v;
      const int p = PER * (lane & 31) + e;
      if (p < A.angles) {
        float sn, cs;
        sincosf(fpos * A.inv_freq[p], &sn, &cs);
        x[e] = hi ? (partner * sn + x[e] * cs) : (x[e] * cs - partner * sn);
      }
    }
  }
  if (kind == 0) {
    float* q = A.q + ((int64_t)m * QH + r) * HD + PER * lane;
#pragma unroll
    for (int e = 0; e < PER; e += 4) *reinterpret_cast<float4*>(q + e) = make_float4(x[e], x[e + 1], x[e + 2], x[e + 3]);
    return;
  }
  const uint32_t slot = A.window > 0 ? pos % (uint32_t)A.slots : pos;
  uint16_t* dst = (kind == 1 ? A.kc : A.vc) + ((int64_t)g * A.slots + slot) * HD + PER * lane;
#pragma unroll
  for (int e = 0; e < PER; ++e) dst[e] = f2h(x[e]);
}

// Workgroup (KV group g, token m), 4 waves.  Wave w walks the token's live
// positions lo + w, lo + w + 4, ... in tiles of T, with its own running max,
// sum and P.V per q head of the group (flash-style online softmax; after the
// cross-lane reduction lane l holds the score of head l / (64 / GQA), so the
// statistics are lane-local and the P.V weights are read out per head);
// the four waves are folded by log-sum-exp at the end.  K and V rows come
// from the caches, which hold every position of the chunk already.
template <int HD, int GQA>
__global__ __launch_bounds__(256) void k_attn_rows_gen(AttnRowsGen A) {
  constexpr int NW = 4, PER = HD / 64, LPH = 64 / GQA, T = HD == 512 ? 4 : 8;
  __shared__ float sml[NW][GQA][2];
  __shared__ __align__(16) float sacc[NW - 1][GQA][HD];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = blockIdx.x, m = blockIdx.y;
  const int cur = (int)A.p0 + m;
  const int lo = (A.window > 0 && cur + 1 > A.window) ? cur + 1 - A.window : 0;
  const int n = cur + 1 - lo;
  const uint16_t* kc = A.kc + (int64_t)g * A.slots * HD + PER * lane;
  const uint16_t* vc = A.vc + (int64_t)g * A.slots * HD + PER * lane;
  const int s_lo = A.window > 0 ? lo % A.slots : lo;
  auto slot_at = [&](int j) -> int64_t {  // j < n <= window <= slots: one wrap at most
    const int s = s_lo + j;
    return (A.window > 0 && s >= A.slots) ? s - A.slots : s;
  };
  float q[GQA][PER];
#pragma unroll
  for (int h = 0; h < GQA; ++h) {
    const float* qr = A.q + ((int64_t)m * A.qh + g * GQA + h) * HD + PER * lane;
#pragma unroll
    for (int e = 0; e < PER; e += 4) {
      const float4 t = *reinterpret_cast<const float4*>(qr + e);
      q[h][e] = t.x, q[h][e + 1] = t.y, q[h][e + 2] = t.z, q[h][e + 3] = t.w;
    }
  }
  float acc[GQA][PER];
#pragma unroll
  for (int h = 0; h < GQA; ++h)
#pragma unroll
    for (int e = 0; e < PER; ++e) acc[h][e] = 0.f;
  float mrun = -3.0e38f, lrun = 0.f;  // of head lane / LPH
  for (int base = wave; base < n; base += NW * T) {
    uint32_t kr[T][PER / 2], vr[T][PER / 2];
#pragma unroll
    for (int i = 0; i < T; ++i) {
      const int64_t sl = slot_at(min(base + NW * i, n - 1)) * HD;
#pragma unroll
      for (int e = 0; e < PER / 2; e += 2) {
        const uint2 a = *reinterpret_cast<const uint2*>(kc + sl + 2 * e);
        const uint2 b = *reinterpret_cast<const uint2*>(vc + sl + 2 * e);
        kr[i][e] = a.x, kr[i][e + 1] = a.y;
        vr[i][e] = b.x, vr[i][e + 1] = b.y;
      }
    }
    float sc[T];
#pragma unroll
    for (int i = 0; i < T; ++i) {
      float t[GQA];
#pragma unroll
      for (int h = 0; h < GQA; ++h) {
        float a = 0.f;
#pragma unroll
        for (int e = 0; e < PER / 2; ++e) {
          a = fmaf(q[h][2 * e], h2f((uint16_t)(kr[i][e] & 0xffffu)), a);
          a = fmaf(q[h][2 * e + 1], h2f((uint16_t)(kr[i][e] >> 16)), a);
        }
        t[h] = a;
      }
      const float s = reduce_rows<64, GQA>(t);
      sc[i] = base + NW * i < n ? s : -3.0e38f;
    }
    float mt = sc[0];
#pragma unroll
    for (int i = 1; i < T; ++i) mt = fmaxf(mt, sc[i]);
    const float mnew = fmaxf(mrun, mt);
    const float alpha = __expf(mrun - mnew);
    float p[T], ps = 0.f;
#pragma unroll
    for (int i = 0; i < T; ++i) {
      p[i] = sc[i] > -1.0e38f ? __expf(sc[i] - mnew) : 0.f;
      ps += p[i];
    }
    lrun = lrun * alpha + ps;
    mrun = mnew;
#pragma unroll
    for (int h = 0; h < GQA; ++h) {
      const float ah = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(alpha), h * LPH));
#pragma unroll
      for (int e = 0; e < PER; ++e) acc[h][e] *= ah;
    }
#pragma unroll
    for (int i = 0; i < T; ++i) {
      float vf[PER];
#pragma unroll
      for (int e = 0; e < PER / 2; ++e) {
        vf[2 * e] = h2f((uint16_t)(vr[i][e] & 0xffffu));
        vf[2 * e + 1] = h2f((uint16_t)(vr[i][e] >> 16));
      }
#pragma unroll
      for (int h = 0; h < GQA; ++h) {
        const float ph = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p[i]), h * LPH));
#pragma unroll
        for (int e = 0; e < PER; ++e) acc[h][e] = fmaf(ph, vf[e], acc[h][e]);
      }
    }
  }
  // fold the four waves
  if ((lane % LPH) == 0) {
    sml[wave][lane / LPH][0] = mrun;
    sml[wave][lane / LPH][1] = lrun;
  }
  if (wave > 0) {
#pragma unroll
    for (int h = 0; h < GQA; ++h)
#pragma unroll
      for (int e = 0; e < PER; ++e) sacc[wave - 1][h][PER * lane + e] = acc[h][e];
  }
  lds_sync();
  if (wave != 0) return;
#pragma unroll
  for (int h = 0; h < GQA; ++h) {
    float M = sml[0][h][0];
#pragma unroll
    for (int w = 1; w < NW; ++w) M = fmaxf(M, sml[w][h][0]);
    float f[NW], L = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      f[w] = __expf(sml[w][h][0] - M);  // 0 for a wave without positions
      L = fmaf(sml[w][h][1], f[w], L);
    }
    const float invL = 1.f / L;
    uint16_t* dst = A.out + (int64_t)m * A.qh * HD + (int64_t)(g * GQA + h) * HD + PER * lane;
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      float v = acc[h][e] * f[0];
#pragma unroll
      for (int w = 1; w < NW; ++w) v = fmaf(sacc[w - 1][h][PER * lane + e], f[w], v);
      dst[e] = f2h(v * invL);
    }
  }
}

// compaction gather (kernels/kvgather.wgsl): block (i, g) copies row keep[i]
// of head g to row i, K by threads [0, hd/8) and V by [hd/8, hd/4), 16 bytes each
__global__ __launch_bounds__(256) void k_kv_gather_gen(const uint32_t* __restrict__ keep,
                                                       const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc,
                                                       int slots, int hd, uint16_t* __restrict__ dk,
                                                       uint16_t* __restrict__ dv, int dslots) {
  const int i = blockIdx.x, g = blockIdx.y, t = threadIdx.x, nr = hd / 8;
  if (t >= 2 * nr) return;
  const int part = t < nr ? t : t - nr;
  const int64_t src = ((int64_t)g * slots + keep[i]) * hd + 8 * part;
  const int64_t dst = ((int64_t)g * dslots + i) * hd + 8 * part;
  if (t < nr)
    *reinterpret_cast<uint4*>(dk + dst) = *reinterpret_cast<const uint4*>(kc + src);
  else
    *reinterpret_cast<uint4*>(dv + dst) = *reinterpret_cast<const uint4*>(vc + src);
}

}  // namespace

int launch_rownorm(const float* h_in, float* h_out, const float* a, const float* w1, float scale, const float* w2,
                   uint16_t* x, uint16_t* xlo, int H, float eps, hipStream_t st, int M, int na, int64_t a_slice) {
  if (H <= 0 || H > 256 * kRowMax) return e4b_fail(E4B_EINVAL, "row norm: hidden %d outside 1..%d", H, 256 * kRowMax);
  if (a && !w1) return e4b_fail(E4B_EINVAL, "row norm: residual without its norm weight");
  if (M < 1 || na < 1 || na > kRowSlices || (na > 1 && (!a || a_slice < (int64_t)M * H)))
    return e4b_fail(E4B_EINVAL, "row norm: %d rows, %d slices", M, na);
  hipLaunchKernelGGL(k_rownorm, dim3(M), dim3(256), 0, st, h_in, h_out, a, w1, scale, w2, x, xlo, H, eps, na, a_slice);
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}

// k_attn_gen's leading scalar arguments (launch_attn_gen checks qh, kvh < 2^15)
#define ATTN_GEN_LEAD(a)                                                                                    \
  a.params, a.qkv, a.qw, a.kw, a.rope, (uint32_t)a.qh | (uint32_t)a.kvh << 16 | (uint32_t)a.keqv << 31,     \
      (uint32_t)a.angles, (uint32_t)(a.window > 0 ? 0 : a.kv_idx), a
template <int HD, bool RAW>
static void launch_attn_hd_raw(const AttnGen& a, hipStream_t st) {
  const dim3 grid(a.kvh, a.gch, HD / gen_vd(HD));
  switch (a.qh / a.kvh) {
    case 1: hipLaunchKernelGGL((k_attn_gen<HD, 1, RAW>), grid, dim3(512), 0, st, ATTN_GEN_LEAD(a)); break;
    case 2: hipLaunchKernelGGL((k_attn_gen<HD, 2, RAW>), grid, dim3(512), 0, st, ATTN_GEN_LEAD(a)); break;
    case 4: hipLaunchKernelGGL((k_attn_gen<HD, 4, RAW>), grid, dim3(512), 0, st, ATTN_GEN_LEAD(a)); break;
    case 8: hipLaunchKernelGGL((k_attn_gen<HD, 8, RAW>), grid, dim3(512), 0, st, ATTN_GEN_LEAD(a)); break;
  }
}
template <int HD>
static void launch_attn_hd(const AttnGen& a, hipStream_t st) {
  if (a.raw)
    launch_attn_hd_raw<HD, true>(a, st);
  else
    launch_attn_hd_raw<HD, false>(a, st);
  if (!a.no_merge) hipLaunchKernelGGL(k_attn_merge<HD>, dim3(a.qh), dim3(256), 0, st, a);
}

int launch_attn_gen(const AttnGen& a, hipStream_t st) {
  const int gqa = a.kvh > 0 ? a.qh / a.kvh : 0;
  if ((a.hd != 256 && a.hd != 512) || a.kvh <= 0 || a.qh > 0x7fff || a.qh % a.kvh || (gqa != 1 && gqa != 2 && gqa != 4 && gqa != 8) ||
      a.angles < 0 || a.angles > a.hd / 2 || a.slots <= 0 || a.gch <= 0 || (a.window > 0 && a.slots < a.window) ||
      (int64_t)a.gch * kAttnGenChunk < (a.window > 0 ? a.window : a.slots) || a.gch > kMergeMaxChunks ||
      (a.raw && a.window > 0))
    return e4b_fail(E4B_EINVAL, "attention: head_dim %d, %d/%d heads (1, 2, 4 or 8 per KV head), %d pairs, %d slots, "
                    "%d chunks", a.hd, a.qh, a.kvh, a.angles, a.slots, a.gch);
  if (a.hd == 256)
    launch_attn_hd<256>(a, st);
  else
    launch_attn_hd<512>(a, st);
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}

int launch_headprep_rows_gen(const HeadRowsGen& a, int M, hipStream_t st) {
  if ((a.hd != 256 && a.hd != 512) || a.kvh <= 0 || a.qh > 0x7fff || a.qh % a.kvh || a.angles < 0 || a.angles > a.hd / 2 ||
      a.slots <= 0 || (a.window > 0 && a.slots < a.window) || M < 1 || a.ld < (int64_t)(a.qh + a.kvh) * a.hd ||
      (a.window == 0 && (int64_t)a.p0 + M > a.slots))
    return e4b_fail(E4B_EINVAL, "head prep rows: head_dim %d, %d/%d heads, %d pairs, %d slots, %d tokens", a.hd, a.qh,
                    a.kvh, a.angles, a.slots, M);
  const dim3 grid(a.qh + 2 * a.kvh, M);
  if (a.hd == 256)
    hipLaunchKernelGGL(k_headprep_rows_gen<256>, grid, dim3(64), 0, st, a);
  else
    hipLaunchKernelGGL(k_headprep_rows_gen<512>, grid, dim3(64), 0, st, a);
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}

template <int HD>
static void launch_attn_rows_hd(const AttnRowsGen& a, int M, hipStream_t st) {
  const dim3 grid(a.kvh, M);
  switch (a.qh / a.kvh) {
    case 1: hipLaunchKernelGGL((k_attn_rows_gen<HD, 1>), grid, dim3(256), 0, st, a); break;
    case 2: hipLaunchKernelGGL((k_attn_rows_gen<HD, 2>), grid, dim3(256), 0, st, a); break;
    case 4: hipLaunchKernelGGL((k_attn_rows_gen<HD, 4>), grid, dim3(256), 0, st, a); break;
    case 8: hipLaunchKernelGGL((k_attn_rows_gen<HD, 8>), grid, dim3(256), 0, st, a); break;
  }
}

int launch_attn_rows_gen(const AttnRowsGen& a, int M, hipStream_t st) {
  const int gqa = a.kvh > 0 ? a.qh / a.kvh : 0;
  if ((a.hd != 256 && a.hd != 512) || a.kvh <= 0 || a.qh > 0x7fff || a.qh % a.kvh || (gqa != 1 && gqa != 2 && gqa != 4 && gqa != 8) ||
      a.slots <= 0 || (a.window > 0 && a.slots < a.window) || M < 1 ||
      (a.window == 0 && (int64_t)a.p0 + M > a.slots))
    return e4b_fail(E4B_EINVAL, "attention rows: head_dim %d, %d/%d heads, %d slots, %d tokens from %u", a.hd, a.qh,
                    a.kvh, a.slots, M, a.p0);
  if (a.hd == 256)
    launch_attn_rows_hd<256>(a, M, st);
  else
    launch_attn_rows_hd<512>(a, M, st);
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}

int launch_kv_gather_gen(const uint32_t* keep, int n, const uint16_t* kc, const uint16_t* vc, int kvh, int slots,
                         int hd, uint16_t* dk, uint16_t* dv, int dslots, hipStream_t st) {
  if (n <= 0) return E4B_OK;
  if (n > dslots || hd % 8 || hd > 1024 || kvh <= 0)
    return e4b_fail(E4B_EINVAL, "kv gather: %d rows into %d, head dim %d", n, dslots, hd);
  hipLaunchKernelGGL(k_kv_gather_gen, dim3(n, kvh), dim3(256), 0, st, keep, kc, vc, slots, hd, dk, dv, dslots);
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}
