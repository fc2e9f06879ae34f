// k_persist.hip -- the decode step's layer loop as ONE persistent kernel.
//
// The kernel-chain step (record_step) runs six dependent launches per layer;
// each waits for its predecessor to drain before it requests its weights,
// so much of a layer goes to launch gaps and first-load latency.  Here one
// cooperative launch (one 512-thread block per CU, all co-resident) walks
// every layer; the phases of a layer hand their output vectors to the next
// phase through tagged 64-bit words in device memory:
//
//   word = (tag << 32) | payload     (payload: one f32 or two f16)
//
// stored and loaded with agent-scope relaxed atomics (write-through `sc1`
// stores, and loads that bypass the per-XCD L2s, which are not coherent with
// each other).  A consumer polls the words it needs until each carries the
// tag of the current phase; data and readiness travel in one single-copy-
// atomic word, so no fences are needed.  Tags are epoch + 1 + layer * 8 +
// phase, with a per-step epoch base in params[8] that only grows (block 0
// advances it when the step is done), so a word from an earlier phase, layer
// or step never matches.  Two sets of buffers alternate by layer parity, so
// a buffer is rewritten two layers later, after phases in which every block
// waited on words of every block (each block publishes a row of the o and
// down projections): no block can overwrite a word another still has to
// read.
// Every phase requests its weights BEFORE it polls its input, so the weight
// stream overlaps the hand-off.
//
// Phases per layer (the E4B recipe of record_step / src/engine.js:292-323):
//   QKV  h = (h + rms(p) w_post_norm) scale (previous layer);
//        x = f16(rms(h) w_attn_norm); qkv rows            (kernels/q40mv.wgsl:56-89)
//   ATT  head prep + RoPE, K/V row write, split-K partials per (KV group,
//        chunk, V half)              (kernels/headprep.wgsl:19-87, kernels/attsplit.wgsl:16-76)
//   CMB  log-sum-exp merge of the chunks -> f16 [QH 256]  (kernels/attcomb.wgsl:10-36)
//   O    o projection
//   GU   h += rms(o) w_post_attn; x = f16(rms(h) w_ffn); gate/up + GeGLU
//                                                          (kernels/q40gu.wgsl:62-119)
//   DN   down projection
//   PG   h += rms(dn) w_post_ffw; x = f16(h); PLE gate, f16(gelu(.) ple_l)
//                                                          (kernels/plegatemv.wgsl:48-57)
//   PP   PLE projection -> p
// After the last layer block 0 applies the last residual and the final norm
// (the lm-head input as an f16 hi/lo pair, as k_tail does) and advances the
// epoch.  The residual stream h lives in LDS, updated identically by every
// block (same inputs, same order), so only branch outputs cross the chip.
//
// Every wait is bounded: a poll gives up after kSpinLimit rounds, or when
// another block raised the abort word, and then its block returns; the grid
// always drains, and the host reports a raised abort word as an error.
#include "../../include/e4b.h"
#include "attn_prep.h"
#include "kernels.h"
#include "persist.h"
#include "step.h"
#include "util.h"

namespace {

constexpr int NT = kPersistThreads;  // 512 threads = 8 waves per block
constexpr int NW = NT / 64;
constexpr int HD = 256;
constexpr int GQA = 4;
constexpr int REC = HD + 2;          // attention partial record: 256 outputs, max, sum
constexpr int kMaxH = 2048;          // hidden size the LDS residual holds
constexpr int kMaxXWords = 8192;     // GEMV input words (f16 pairs): FF / 2 of the down projection
constexpr uint32_t kSpinLimit = 1u << 20;
constexpr float kTwo24 = 16777216.0f;
typedef unsigned long long u64;

// Address-space views.  Every pointer here arrives through the layer table
// or the argument struct, so the compiler cannot tell it is global memory
// and would emit flat accesses, which count against the LDS counter too: an
// LDS read after a weight prefetch would then wait for the whole prefetch.
// Global views make them global_load/global_store (vector counter only); the
// layer table, written by the host before the launch, is read through the
// constant address space (scalar loads, which do not wait behind the vector
// memory queue).
// (The host pass of hipcc parses the kernel too; address spaces exist only in
// the device pass.)
#if defined(__HIP_DEVICE_COMPILE__)
#define GAS __attribute__((address_space(1)))
typedef const __attribute__((address_space(4))) PersistLayer CLayer;
#else
#define GAS
typedef const PersistLayer CLayer;
#endif
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
template <typename T>
DEV const GAS T* gc(const T* p) {
  return (const GAS T*)p;
}
template <typename T>
DEV GAS T* gm(T* p) {
  return (GAS T*)p;
}
DEV uint4 gld_nt_u4(const void* base, uint32_t byte_off) {
  const u32x4 v = __builtin_nontemporal_load((const GAS u32x4*)((const GAS char*)base + byte_off));
  return make_uint4(v.x, v.y, v.z, v.w);
}
DEV uint32_t gld_nt_u32(const void* base, uint32_t byte_off) {
  return __builtin_nontemporal_load((const GAS uint32_t*)((const GAS char*)base + byte_off));
}
DEV uint4 gld_u4(const void* p) {
  const u32x4 v = *(const GAS u32x4*)p;
  return make_uint4(v.x, v.y, v.z, v.w);
}
DEV float4 gld_f4(const void* p) { return *(const GAS float4*)p; }
typedef float f32x2 __attribute__((ext_vector_type(2)));
DEV float2 gld_f2(const void* p) {
  const f32x2 v = *(const GAS f32x2*)p;
  return make_float2(v.x, v.y);
}

enum Phase { PH_QKV = 0, PH_ATT, PH_CMB, PH_O, PH_GU, PH_DN, PH_PG, PH_PP, PH_N };
static_assert(PH_N == kPersistPhases, "phase count");

// threadIdx.x behind an opaque zero: values derived from it are recomputed in
// each phase instead of being computed once and held (and spilled) across the
// whole layer loop
DEV int fresh_tid() {
  int z;
  asm volatile("s_mov_b32 %0, 0" : "=s"(z));
  return (int)threadIdx.x + z;
}

DEV void ll_put(u64* buf, int i, uint32_t payload, uint32_t tag) {
  __hip_atomic_store(gm(buf) + i, ((u64)tag << 32) | payload, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
DEV u64 ll_get(const u64* buf, int i) {
  return __hip_atomic_load(gm(const_cast<u64*>(buf)) + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
DEV bool aborted(int* abort) { return __hip_atomic_load(gm(abort), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0; }
DEV void raise_abort(int* abort) { __hip_atomic_store(gm(abort), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

// s_waitcnt vmcnt(0): every vector memory load this wave issued is in.  Put
// after each poll: a thread with no word to poll skips the poll loop (and its
// waits), and the compiler's wait placement takes the minimum over such
// paths, so without it a tile requested after the poll would be waited for
// before the first use of a tile requested before it.
DEV void vm_drain() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// true in every thread of the block when every thread passed `ok`
DEV bool block_ok(bool ok, int* vote, int tid) {
  if (tid == 0) *vote = 0;
  lds_sync();
  if (!ok) *vote = 1;
  lds_sync();
  const bool all = *vote == 0;
  lds_sync();
  return all;
}

// Block-wide poll of n words: word i (i < n) lives at buf[idx(i)], thread t
// owns i = t + NT k (k < MAXW); sink(i, payload) receives each word once its
// tag matches.  Returns false, in every thread of the block, when the wait
// gave up (spin limit or another block's abort).
template <int MAXW, typename Idx, typename Sink>
DEV bool poll_block(const u64* buf, int n, uint32_t tag, int* abort, int* vote, int tid, Idx&& idx, Sink&& sink) {
  uint32_t pend = 0;
#pragma unroll
  for (int k = 0; k < MAXW; ++k)
    if (tid + NT * k < n) pend |= 1u << k;
  uint32_t spins = 0;
  bool bad = false;
  while (pend) {
    u64 v[MAXW];
#pragma unroll
    for (int k = 0; k < MAXW; ++k) v[k] = ((pend >> k) & 1u) ? ll_get(buf, idx(tid + NT * k)) : 0ull;
#pragma unroll
    for (int k = 0; k < MAXW; ++k)
      if (((pend >> k) & 1u) && (uint32_t)(v[k] >> 32) == tag) {
        sink(tid + NT * k, (uint32_t)v[k]);
        pend &= ~(1u << k);
      }
    if (pend) {
      ++spins;
      if (spins >= kSpinLimit || ((spins & 63u) == 0 && aborted(abort))) {
        bad = true;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
  }
  vm_drain();
  if (bad) raise_abort(abort);
  return block_ok(!bad, vote, tid);
}

// contiguous words [0, n) of buf
template <int MAXW, typename Sink>
DEV bool poll_range(const u64* buf, int n, uint32_t tag, int* abort, int* vote, int tid, Sink&& sink) {
  return poll_block<MAXW>(buf, n, tag, abort, vote, tid, [](int i) { return i; }, sink);
}

DEV float block_sum8(float v, float* red, int tid) {
  v = wave_sum(v);
  lds_sync();
  if ((tid & 63) == 0) red[tid >> 6] = v;
  lds_sync();
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) t += red[w];
  lds_sync();
  return t;
}

// ---- q4_0 GEMV tiles (the arithmetic of q40_kernel.h's k_q40) ---------------
// A wave splits into 64/LPR lane groups; a group owns R row slots; lane l of
// a group covers blocks l + LPR k (k < BPL); row_of(r) gives slot r's row.
template <int R, int BPL>
struct Tile {
  uint4 q[R][BPL];
  uint32_t s[R][BPL];
  uint64_t odd;
};

template <int LPR, int R, int BPL, typename RowOf>
DEV void tile_load(Tile<R, BPL>& t, const Q40Mat& W, int l, RowOf&& row_of) {
  static_assert(R * BPL <= 64, "scale parity bits");
  t.odd = 0;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t row = row_of(r);
#pragma unroll
    for (int k = 0; k < BPL; ++k) {
      const int jb = min(l + LPR * k, W.nb - 1);
      const uint32_t e = (uint32_t)row * (uint32_t)W.nb + (uint32_t)jb;  // planes < 4 GiB
      t.q[r][k] = gld_nt_u4(W.nib, e * 16u);
      t.s[r][k] = gld_nt_u32(W.sc, (e >> 1) * 4u);
      t.odd |= (uint64_t)(e & 1u) << (r * BPL + k);
    }
  }
}

// slot r of the tile . x (f16 pairs in LDS, 16 words per block); after the
// transposed reduction lane l holds slot l / (LPR / R) of its group
template <int LPR, int R, int BPL>
DEV float tile_dot(const Tile<R, BPL>& t, const uint32_t* xs, int nb, int l) {
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;
#pragma unroll
  for (int k = 0; k < BPL; ++k) {
    const int jb = l + LPR * k;
    const bool in = jb < nb;
    uint32_t xp[16];
    const uint4* v = reinterpret_cast<const uint4*>(xs) + (size_t)(in ? jb : 0) * 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint4 u = v[i];
      xp[4 * i + 0] = in ? u.x : 0u;
      xp[4 * i + 1] = in ? u.y : 0u;
      xp[4 * i + 2] = in ? u.z : 0u;
      xp[4 * i + 3] = in ? u.w : 0u;
    }
    const float xs8 = -8.f * xsum16(xp);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float a0 = 0.f, a1 = 0.f;
      q40_dot2(t.q[r][k], xp, a0, a1);
      const float d = scale_of(t.s[r][k], (uint32_t)(t.odd >> (r * BPL + k)) & 1u);
      acc[r] = fmaf(d, fmaf(a1, kTwo24 / 16.f, fmaf(a0, kTwo24, xs8)), acc[r]);
    }
  }
  return reduce_rows<LPR, R>(acc);
}

// ---- residual stream (every block holds all of it) -------------------------
// Norm weights held in registers (requested a phase ahead): thread t holds
// the elements i = t + NT k of a residual weight, and the pairs (2i, 2i + 1)
// of a norm weight.
struct ResW {
  float w[kMaxH / NT];
};
struct NormW {
  float2 w[kMaxH / 2 / NT];
};
DEV void load_resw(ResW& r, const float* w, int H, int tid) {
#pragma unroll
  for (int k = 0; k < kMaxH / NT; ++k) {
    const int i = tid + NT * k;
    r.w[k] = i < H ? gc(w)[i] : 0.f;
  }
}
DEV void load_normw(NormW& n, const float* w, int H, int tid) {
#pragma unroll
  for (int k = 0; k < kMaxH / 2 / NT; ++k) {
    const int i = tid + NT * k;
    n.w[k] = i < H / 2 ? gld_f2(w + 2 * i) : make_float2(0.f, 0.f);
  }
}
// h = (h + rms(v) w) * scale (v in LDS)
DEV void residual(float* hs, const float* vs, const ResW& w, float scale, int H, float eps, float* red, int tid) {
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < kMaxH / NT; ++k) {
    const int i = tid + NT * k;
    if (i < H) ss = fmaf(vs[i], vs[i], ss);
  }
  const float inv = rms_inv(block_sum8(ss, red, tid), H, eps);
#pragma unroll
  for (int k = 0; k < kMaxH / NT; ++k) {
    const int i = tid + NT * k;
    if (i < H) hs[i] = (hs[i] + vs[i] * inv * w.w[k]) * scale;
  }
  lds_sync();
}
// xs (f16 pairs) = f16(rms(h) w), or f16(h) when w is null
DEV void norm_to_x(const float* hs, const NormW* w, int H, float eps, uint32_t* xs, float* red, int tid) {
  float inv = 1.f;
  if (w) {
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < kMaxH / NT; ++k) {
      const int i = tid + NT * k;
      if (i < H) ss = fmaf(hs[i], hs[i], ss);
    }
    inv = rms_inv(block_sum8(ss, red, tid), H, eps);
  }
#pragma unroll
  for (int k = 0; k < kMaxH / 2 / NT; ++k) {
    const int i = tid + NT * k;
    if (i < H / 2) {
      const float a = w ? hs[2 * i] * inv * w->w[k].x : hs[2 * i];
      const float b = w ? hs[2 * i + 1] * inv * w->w[k].y : hs[2 * i + 1];
      xs[i] = (uint32_t)f2h(a) | ((uint32_t)f2h(b) << 16);
    }
  }
  lds_sync();
}

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

// LDS of one block; the attention scratch overlays the GEMV input
struct AttnLds {
  __align__(16) float qkv[6][HD];        // the group's 4 raw q heads, k and v
  float qs[GQA][HD];                     // prepped q
  __align__(16) uint16_t knew[HD];
  __align__(16) uint16_t vnew[HD];
  __align__(16) float po[NW][GQA][HD / 2];
  float wml[NW][GQA][2];
};
struct Lds {
  float hs[kMaxH];                       // residual stream
  float vs[kMaxH];                       // the polled branch vector
  union {
    __align__(16) uint32_t xs[kMaxXWords];  // GEMV input, f16 pairs
    AttnLds at;
  };
  float red[NW];
  int vote;
};

// One (KV group g, chunk c, V half zs) item of the split-K attention: the
// arithmetic of k_attn.hip's k_attn_split (wave w owns the chunk's positions
// w + 8k; K as two 256-byte halves per row, 16 lanes a position; V half as
// 16 bytes a lane), with q/k/v from LDS and the partials published as tagged
// words.  Returns false when a wait gave up.
template <int CS>
DEV bool attn_item(const PersistArgs& a, const PersistLayer& ly, Lds& S, int g, int c, int zs, int lo, int n_live,
                   int cur, int pos, uint32_t tag_in, uint32_t tag_out, u64* ready_mark, int tid) {
  constexpr int KP = CS / 32, VS = CS / 8, VD = HD / 2, LV = VD / 8, PPL = 64 / LV, VQ = VS / PPL;
  const int lane = tid & 63, wave = tid >> 6;
  const int QH = a.QH, KVH = a.KVH;
  const int window = ly.global ? 0 : a.window;
  const int c_lo = lo + c * CS;
  const int m = min(CS, n_live - c * CS);
  uint16_t* kc = ly.kc + (int64_t)g * ly.slots * HD;
  uint16_t* vc = ly.vc + (int64_t)g * ly.slots * HD;
  const int s_lo = window > 0 ? c_lo % ly.slots : c_lo;
  auto slot_at = [&](int j) -> int64_t {
    const int s = s_lo + j;
    return (window > 0 && s >= ly.slots) ? s - ly.slots : s;
  };
  const int sub = lane >> 4, dl = lane & 15;
  const int vsub = lane / LV, vl = lane % LV, vd0 = VD * zs + 8 * vl;
  // 0. the chunk's K and V rows (they do not depend on this step's qkv), the
  //    head-prep weights and RoPE (cos, sin), then the group's q/k/v rows
  const float4 win = gld_f4((wave < 4 ? ly.q_norm : ly.k_norm) + 4 * lane);
  const float2* rsrc = a.rope + (ly.global ? HD / 2 : 0);
  const float4 rc0 = gld_f4(rsrc + 4 * (lane & 31));
  const float4 rc1 = gld_f4(rsrc + 4 * (lane & 31) + 2);
  uint4 kr[KP][2];
  uint4 vr[VQ];
#pragma unroll
  for (int s = 0; s < KP; ++s) {
    const int j = min(wave + NW * (4 * s + sub), m - 1);
    const uint16_t* row = kc + slot_at(j) * HD;
    kr[s][0] = gld_u4(row + 8 * dl);
    kr[s][1] = gld_u4(row + 128 + 8 * dl);
  }
#pragma unroll
  for (int q = 0; q < VQ; ++q) {
    const int j = min(wave + NW * (PPL * q + vsub), m - 1);
    vr[q] = gld_u4(vc + slot_at(j) * HD + vd0);
  }
  __builtin_amdgcn_sched_barrier(0);
  if (!poll_block<(6 * HD + NT - 1) / NT>(
          ly.ll_qkv, 6 * HD, tag_in, a.abort, &S.vote, tid,
          [&](int i) {
            const int r = i / HD, d = i - r * HD;
            const int row = r < 4 ? g * GQA + r : (r == 4 ? QH + g : QH + KVH + g);
            return row * HD + d;
          },
          [&](int i, uint32_t p) { (&S.at.qkv[0][0])[i] = __uint_as_float(p); }))
    return false;
  if (ready_mark && tid == 0) *gm(ready_mark) = wall_clock64();
  lds_sync();

  // 1. head prep: waves 0-3 the q heads, wave 4 the new k, wave 5 the new v
  const bool owner = cur < c_lo + m;  // the chunk holding `cur` (at j = m - 1)
  const float fpos = (float)pos;
  if (wave < 6) {
    const float4 xin = *reinterpret_cast<const float4*>(&S.at.qkv[wave][4 * lane]);
    float x[4] = {xin.x, xin.y, xin.z, xin.w};
    const float w[4] = {win.x, win.y, win.z, win.w};
    const float2 cs[4] = {make_float2(rc0.x, rc0.y), make_float2(rc0.z, rc0.w), make_float2(rc1.x, rc1.y),
                          make_float2(rc1.z, rc1.w)};
    prep_head_regs(x, w, wave < 5, cs, true, nullptr, 128, a.eps, fpos, wave < 5);
    if (wave < 4) {
#pragma unroll
      for (int i = 0; i < 4; ++i) S.at.qs[wave][4 * lane + i] = x[i];
    } else {
      const uint2 pk = make_uint2((uint32_t)f2h(x[0]) | ((uint32_t)f2h(x[1]) << 16),
                                  (uint32_t)f2h(x[2]) | ((uint32_t)f2h(x[3]) << 16));
      *reinterpret_cast<uint2*>((wave == 4 ? S.at.knew : S.at.vnew) + 4 * lane) = pk;
      if (owner && zs == 0) *(GAS uint2*)((wave == 4 ? kc : vc) + slot_at(m - 1) * HD + 4 * lane) = pk;
    }
  }
  lds_sync();

  // 2. scores of the wave's positions (16 lanes a position, 16 dims a lane)
  float sc[KP];
  {
    float q[GQA][16];
#pragma unroll
    for (int h = 0; h < GQA; ++h)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        q[h][i] = S.at.qs[h][8 * dl + i];
        q[h][8 + i] = S.at.qs[h][128 + 8 * dl + i];
      }
#pragma unroll
    for (int s = 0; s < KP; ++s) {
      const int j = wave + NW * (4 * s + sub);
      uint4 ka = kr[s][0], kb = kr[s][1];
      if (c_lo + j == cur) {
        ka = *reinterpret_cast<const uint4*>(S.at.knew + 8 * dl);
        kb = *reinterpret_cast<const uint4*>(S.at.knew + 128 + 8 * dl);
      }
      float kf[16];
      unpack16(ka, kb, kf);
      float t[GQA];
#pragma unroll
      for (int h = 0; h < GQA; ++h) {
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) acc = fmaf(q[h][i], kf[i], acc);
        t[h] = acc;
      }
      sc[s] = j < m ? reduce_rows<16, GQA>(t) : -3.0e38f;
    }
  }

  // 3. the wave's softmax statistics per head
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

  // 4. P.V over the wave's positions
  {
    float acc[GQA][8];
#pragma unroll
    for (int h = 0; h < GQA; ++h)
#pragma unroll
      for (int d = 0; d < 8; ++d) acc[h][d] = 0.f;
    const uint4 vn = *reinterpret_cast<const uint4*>(S.at.vnew + vd0);
#pragma unroll
    for (int q = 0; q < VQ; ++q) {
      const int i = PPL * q + vsub;
      const int j = wave + NW * i;
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
        float pf;
        if constexpr (PPL == 2) {
          const int i0 = 2 * q, i1 = 2 * q + 1;
          const float p0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e[i0 >> 2]), 16 * (i0 & 3) + 4 * h));
          const float p1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e[i1 >> 2]), 16 * (i1 & 3) + 4 * h));
          pf = vsub ? p1 : p0;
        } else {
          pf = __shfl(e[q], 16 * vsub + 4 * h, 64);
        }
#pragma unroll
        for (int d = 0; d < 8; ++d) acc[h][d] = fmaf(pf, vf[d], acc[h][d]);
      }
    }
    float r[2][8];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int d = 0; d < 8; ++d) r[hh][d] = tstep<32>(acc[hh][d], acc[hh + 2][d]);
    if constexpr (PPL == 2) {
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        float4* dst = reinterpret_cast<float4*>(&S.at.po[wave][hh + 2 * (lane >> 5)][8 * vl]);
        dst[0] = make_float4(r[hh][0], r[hh][1], r[hh][2], r[hh][3]);
        dst[1] = make_float4(r[hh][4], r[hh][5], r[hh][6], r[hh][7]);
      }
    } else {
      float t[8];
#pragma unroll
      for (int d = 0; d < 8; ++d) t[d] = tstep<16>(r[0][d], r[1][d]);
      float4* dst = reinterpret_cast<float4*>(&S.at.po[wave][2 * (lane >> 5) + ((lane >> 4) & 1)][8 * vl]);
      dst[0] = make_float4(t[0], t[1], t[2], t[3]);
      dst[1] = make_float4(t[4], t[5], t[6], t[7]);
    }
#pragma unroll
    for (int h = 0; h < GQA; ++h)
      if (lane == 4 * h) {
        S.at.wml[wave][h][0] = mx;
        S.at.wml[wave][h][1] = ls;
      }
  }
  lds_sync();

  // 5. fold the 8 waves into the chunk's partials: thread -> (head, dim)
  {
    const int h = tid / VD, d = tid % VD;  // GQA x VD = 512 outputs
    float M = S.at.wml[0][h][0];
#pragma unroll
    for (int w = 1; w < NW; ++w) M = fmaxf(M, S.at.wml[w][h][0]);
    float v = 0.f, L = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float f = __expf(S.at.wml[w][h][0] - M);
      v = fmaf(S.at.po[w][h][d], f, v);
      L = fmaf(S.at.wml[w][h][1], f, L);
    }
    const int rec = ((g * GQA + h) * a.nch_max + c) * REC;
    ll_put(ly.ll_pm, rec + VD * zs + d, __float_as_uint(v), tag_out);
    if (zs == 0 && d == 0) {
      ll_put(ly.ll_pm, rec + HD, __float_as_uint(M), tag_out);
      ll_put(ly.ll_pm, rec + HD + 1, __float_as_uint(L), tag_out);
    }
  }
  lds_sync();
  return true;
}

// CMB for one wave: head h, dims [d0, d0 + 8): merges the live chunks 64 at a
// time (lane = chunk) with a running maximum; returns false when a wait gave up
DEV bool combine_wave(const PersistArgs& a, const PersistLayer& ly, int h, int d0, int nch, uint32_t tag_in,
                      uint32_t tag_out, int lane) {
  float M = -3.0e38f, den = 0.f, acc[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) acc[k] = 0.f;
  for (int c0 = 0; c0 < nch; c0 += 64) {
    const int c = c0 + lane;
    const bool live = c < nch;
    const int rec = (h * a.nch_max + (live ? c : 0)) * REC;
    uint32_t pend = live ? 0x3FFu : 0u;  // 8 outputs + max + sum
    uint32_t got[10] = {};
    uint32_t spins = 0;
    bool bad = false;
    while (__any(pend != 0)) {
      u64 v[10];
#pragma unroll
      for (int k = 0; k < 10; ++k) v[k] = ((pend >> k) & 1u) ? ll_get(ly.ll_pm, rec + (k < 8 ? d0 + k : HD + k - 8)) : 0ull;
#pragma unroll
      for (int k = 0; k < 10; ++k)
        if (((pend >> k) & 1u) && (uint32_t)(v[k] >> 32) == tag_in) {
          got[k] = (uint32_t)v[k];
          pend &= ~(1u << k);
        }
      if (__any(pend != 0)) {
        ++spins;
        if (spins >= kSpinLimit || ((spins & 63u) == 0 && aborted(a.abort))) {
          bad = true;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
    }
    vm_drain();
    if (__any(bad)) {
      raise_abort(a.abort);
      return false;
    }
    const float mc = live ? __uint_as_float(got[8]) : -3.0e38f;
    const float nM = fmaxf(M, wave_max(mc));
    const float fo = __expf(M - nM);
    const float f = live ? __expf(mc - nM) : 0.f;
    den = den * fo + wave_sum(live ? __uint_as_float(got[9]) * f : 0.f);
#pragma unroll
    for (int k = 0; k < 8; ++k) acc[k] = acc[k] * fo + wave_sum(live ? __uint_as_float(got[k]) * f : 0.f);
    M = nM;
  }
  if (lane < 4) {
    float a0 = acc[0], a1 = acc[1];  // acc[2 lane], acc[2 lane + 1] without a private-memory index
#pragma unroll
    for (int k = 1; k < 4; ++k)
      if (lane == k) {
        a0 = acc[2 * k];
        a1 = acc[2 * k + 1];
      }
    const float lo = a0 / den, hi = a1 / den;
    ll_put(ly.ll_att, (h * HD + d0) / 2 + lane, (uint32_t)f2h(lo) | ((uint32_t)f2h(hi) << 16), tag_out);
  }
  return true;
}

template <int CS, int BPLD>
__global__ __launch_bounds__(NT) void k_persist(PersistArgs a) {
  __shared__ Lds S;
  const int nblk = gridDim.x;
  const int nwaves = nblk * NW;
  const int H = a.H, FF = a.FF, QH = a.QH, KVH = a.KVH, PD = a.PD, QKV = (QH + 2 * KVH) * HD;
  const uint32_t ep = gc(a.params)[8];
  const int pos = (int)gc(a.params)[0];
  int* ab = a.abort;
  auto tag_of = [&](int l, int ph) -> uint32_t { return ep + 1u + (uint32_t)(l * PH_N + ph); };
  u64* const tr = a.trace;
  auto mark = [&](int l, int ph, int k) {
    if (tr && threadIdx.x == 0) gm(tr)[((size_t)blockIdx.x * a.layers + l) * kPersistTraceSlots + ph * 3 + k] = wall_clock64();
  };

  for (int i = threadIdx.x; i < H; i += NT) S.hs[i] = gc(a.h_in)[i];
  lds_sync();

  CLayer* const LT = (CLayer*)a.L;
  // Software pipeline: each GEMV tile and the norm weights a phase applies
  // (its first tile: a wave's further tiles, when a matrix has more rows than
  // the grid has waves, are loaded in place, into a tile of their own, so the
  // compiler's wait for them never covers the tiles requested ahead)
  // are requested right after the PREVIOUS phase's input arrived, so they
  // stream while that phase computes and hands its output over.  (A wave's
  // loads return in order: a poll issued behind a tile completes only once
  // the tile is in, so the next tile is issued after the poll, not before.)
  Tile<2, 1> Tq = {};   // qkv rows of layer l (requested in layer l - 1's PP phase)
  NormW nq = {};        // attn_norm of layer l
  ResW rq = {};         // post_norm of layer l - 1
  {
    const int tid = fresh_tid(), lane = tid & 63, gw = blockIdx.x * NW + (tid >> 6);
    const PersistLayer l0 = LT[0];
    if (gw < (QKV + 1) / 2) tile_load<64, 2, 1>(Tq, l0.qkv, lane, [&](int r) { return (int64_t)min(gw * 2 + r, QKV - 1); });
    load_normw(nq, l0.attn_norm, H, tid);
  }
  for (int l = 0; l < a.layers; ++l) {
    const PersistLayer ly = LT[l];
    // ---------------------------------------------------------------- QKV
    {
      mark(l, PH_QKV, 0);
      const int tid = fresh_tid(), lane = tid & 63, gw = blockIdx.x * NW + (tid >> 6);
      constexpr int R = 2;
      const int ntiles = (QKV + R - 1) / R;
      if (l > 0) {
        const PersistLayer pv = LT[l - 1];
        if (!poll_range<kMaxH / NT>(pv.ll_p, H, tag_of(l - 1, PH_PP), ab, &S.vote, tid,
                                    [&](int i, uint32_t p) { S.vs[i] = __uint_as_float(p); }))
          return;
        mark(l, PH_QKV, 1);
        residual(S.hs, S.vs, rq, pv.scale, H, a.eps, S.red, tid);
      } else {
        mark(l, PH_QKV, 1);
      }
      norm_to_x(S.hs, &nq, H, a.eps, S.xs, S.red, tid);
      auto rows = [&](int t) { return [=](int r) { return (int64_t)min(t * R + r, QKV - 1); }; };
      auto body = [&](const Tile<R, 1>& T, int t) {
        const float y = tile_dot<64, R, 1>(T, S.xs, ly.qkv.nb, lane);
        const int row = t * R + (lane >> 5);
        if ((lane & 31) == 0 && row < QKV) ll_put(ly.ll_qkv, row, __float_as_uint(y), tag_of(l, PH_QKV));
      };
      if (gw < ntiles) body(Tq, gw);
      for (int t = gw + nwaves; t < ntiles; t += nwaves) {
        Tile<R, 1> T = {};
        tile_load<64, R, 1>(T, ly.qkv, lane, rows(t));
        body(T, t);
      }
      lds_sync();
      mark(l, PH_QKV, 2);
    }
    // ---------------------------------------------------------------- ATT
    const int cur = ly.global ? (int)gc(a.params)[4] : pos;
    const int lo = (!ly.global && cur + 1 > a.window) ? cur + 1 - a.window : 0;
    const int n_live = cur + 1 - lo;
    const int nch = (n_live + CS - 1) / CS;
    {
      mark(l, PH_ATT, 0);
      const int tid = fresh_tid();
      const int nitems = KVH * nch * 2;
      for (int wi = blockIdx.x; wi < nitems; wi += nblk) {
        const int zs = wi & 1, c = (wi >> 1) % nch, g = (wi >> 1) / nch;
        u64* rm = (tr && wi == (int)blockIdx.x)
                      ? tr + ((size_t)blockIdx.x * a.layers + l) * kPersistTraceSlots + PH_ATT * 3 + 1
                      : nullptr;
        if (!attn_item<CS>(a, ly, S, g, c, zs, lo, n_live, cur, pos, tag_of(l, PH_QKV), tag_of(l, PH_ATT), rm, tid))
          return;
      }
      mark(l, PH_ATT, 2);
    }
    // ---------------------------------------------------------------- CMB
    {
      mark(l, PH_CMB, 0);
      const int tid = fresh_tid(), lane = tid & 63, gw = blockIdx.x * NW + (tid >> 6);
      const int nitems = QH * (HD / 8);
      bool ok = true;
      for (int it = gw; it < nitems && ok; it += nwaves)
        ok = combine_wave(a, ly, it / (HD / 8), 8 * (it % (HD / 8)), nch, tag_of(l, PH_ATT), tag_of(l, PH_CMB), lane);
      if (!block_ok(ok, &S.vote, tid)) return;
      mark(l, PH_CMB, 2);
    }
    // GU's tile (the largest of the layer) and norm weights, requested in O
    constexpr int RG = 16;  // 8 (gate, up) pairs a wave
    const int ntiles_gu = (2 * FF + RG - 1) / RG;
    auto gu_rows = [&](int t) {
      return [=](int r) -> int64_t {
        const int u = min(t * (RG / 2) + r / 2, FF - 1);
        return (r & 1) ? (int64_t)FF + u : (int64_t)u;
      };
    };
    Tile<RG, 1> Tg = {};  // zero on every path: an undefined tile would become a loop-carried value
    ResW rg = {};
    NormW ng = {};
    // ---------------------------------------------------------------- O
    {
      mark(l, PH_O, 0);
      const int tid = fresh_tid(), lane = tid & 63, gw = blockIdx.x * NW + (tid >> 6);
      const int ntiles = H;  // one row a wave
      const int nbo = ly.o.nb;
      Tile<1, 1> T = {};
      if (gw < ntiles) tile_load<64, 1, 1>(T, ly.o, lane, [&](int) { return (int64_t)gw; });
      __builtin_amdgcn_sched_barrier(0);
      if (!poll_range<(kMaxH / 2 + NT - 1) / NT>(ly.ll_att, QH * HD / 2, tag_of(l, PH_CMB), ab, &S.vote, tid,
                                                 [&](int i, uint32_t p) { S.xs[i] = p; }))
        return;
      mark(l, PH_O, 1);
      if (gw < ntiles_gu) tile_load<64, RG, 1>(Tg, ly.gu, lane, gu_rows(gw));
      load_resw(rg, ly.post_attn, H, tid);
      load_normw(ng, ly.ffn_norm, H, tid);
      __builtin_amdgcn_sched_barrier(0);
      auto body = [&](const Tile<1, 1>& T1, int t) {
        const float y = tile_dot<64, 1, 1>(T1, S.xs, nbo, lane);
        if (lane == 0) ll_put(ly.ll_o, t, __float_as_uint(y), tag_of(l, PH_O));
      };
      if (gw < ntiles) body(T, gw);
      for (int t = gw + nwaves; t < ntiles; t += nwaves) {
        Tile<1, 1> T1 = {};
        tile_load<64, 1, 1>(T1, ly.o, lane, [&](int) { return (int64_t)t; });
        body(T1, t);
      }
      lds_sync();
      mark(l, PH_O, 2);
    }
    Tile<1, BPLD> Td = {};
    // ---------------------------------------------------------------- GU
    {
      mark(l, PH_GU, 0);
      const int tid = fresh_tid(), lane = tid & 63, gw = blockIdx.x * NW + (tid >> 6);
      if (!poll_range<kMaxH / NT>(ly.ll_o, H, tag_of(l, PH_O), ab, &S.vote, tid,
                                  [&](int i, uint32_t p) { S.vs[i] = __uint_as_float(p); }))
        return;
      mark(l, PH_GU, 1);
      if (gw < H) tile_load<64, 1, BPLD>(Td, ly.down, lane, [&](int) { return (int64_t)gw; });
      __builtin_amdgcn_sched_barrier(0);
      residual(S.hs, S.vs, rg, 1.f, H, a.eps, S.red, tid);
      norm_to_x(S.hs, &ng, H, a.eps, S.xs, S.red, tid);
      auto body = [&](const Tile<RG, 1>& T, int t) {
        const float v = tile_dot<64, RG, 1>(T, S.xs, ly.gu.nb, lane);   // lane l: slot l / 4
        const float up = __shfl_xor(v, 4, 64);
        const float gg = gelu_tanh(v) * up;                               // valid in lanes with (l & 7) < 4
        const float gg_hi = __shfl_down(gg, 8, 64);                       // the next unit
        const int u = t * (RG / 2) + lane / 8;
        if ((lane & 15) == 0 && u < FF) {
          const uint32_t hi = u + 1 < FF ? (uint32_t)f2h(gg_hi) : 0u;
          ll_put(ly.ll_gg, u / 2, (uint32_t)f2h(gg) | (hi << 16), tag_of(l, PH_GU));
        }
      };
      if (gw < ntiles_gu) body(Tg, gw);
      for (int t = gw + nwaves; t < ntiles_gu; t += nwaves) {
        Tile<RG, 1> T = {};
        tile_load<64, RG, 1>(T, ly.gu, lane, gu_rows(t));
        body(T, t);
      }
      lds_sync();
      mark(l, PH_GU, 2);
    }
    constexpr int RP = 2;
    const int ntiles_pg = PD / RP;
    Tile<RP, 1> Tp = {};
    ResW rp = {};
    float plv = 0.f;  // the PLE input of the PLE-gate row this lane finishes
    // ---------------------------------------------------------------- DN
    {
      mark(l, PH_DN, 0);
      const int tid = fresh_tid(), lane = tid & 63, gw = blockIdx.x * NW + (tid >> 6);
      const int ntiles = H;
      const int nbd = ly.down.nb;
      if (!poll_range<kMaxXWords / NT>(ly.ll_gg, FF / 2, tag_of(l, PH_GU), ab, &S.vote, tid,
                                       [&](int i, uint32_t p) { S.xs[i] = p; }))
        return;
      mark(l, PH_DN, 1);
      if (gw < ntiles_pg) {
        tile_load<64, RP, 1>(Tp, ly.pg, lane, [&](int r) { return (int64_t)(gw * RP + r); });
        plv = gc(a.ple)[(int64_t)l * PD + gw * RP + (lane >> 5)];
      }
      load_resw(rp, ly.post_ffw, H, tid);
      __builtin_amdgcn_sched_barrier(0);
      auto body = [&](const Tile<1, BPLD>& T, int t) {
        const float y = tile_dot<64, 1, BPLD>(T, S.xs, nbd, lane);
        if (lane == 0) ll_put(ly.ll_dn, t, __float_as_uint(y), tag_of(l, PH_DN));
      };
      if (gw < ntiles) body(Td, gw);
      for (int t = gw + nwaves; t < ntiles; t += nwaves) {
        Tile<1, BPLD> T = {};
        tile_load<64, 1, BPLD>(T, ly.down, lane, [&](int) { return (int64_t)t; });
        body(T, t);
      }
      lds_sync();
      mark(l, PH_DN, 2);
    }
    constexpr int LPP = 8;  // PLE projection: 8 blocks (PD = 256) a row, 8 rows a wave
    const int ntiles_pp = (H + 7) / 8;
    Tile<1, 1> Tpp = {};
    // ---------------------------------------------------------------- PG
    {
      mark(l, PH_PG, 0);
      const int tid = fresh_tid(), lane = tid & 63, gw = blockIdx.x * NW + (tid >> 6);
      const int grp = lane / LPP, l8 = lane % LPP;
      if (!poll_range<kMaxH / NT>(ly.ll_dn, H, tag_of(l, PH_DN), ab, &S.vote, tid,
                                  [&](int i, uint32_t p) { S.vs[i] = __uint_as_float(p); }))
        return;
      mark(l, PH_PG, 1);
      if (gw < ntiles_pp) tile_load<LPP, 1, 1>(Tpp, ly.pp, l8, [&](int) { return (int64_t)min(gw * 8 + grp, H - 1); });
      __builtin_amdgcn_sched_barrier(0);
      residual(S.hs, S.vs, rp, 1.f, H, a.eps, S.red, tid);
      norm_to_x(S.hs, nullptr, H, a.eps, S.xs, S.red, tid);
      auto body = [&](const Tile<RP, 1>& T, float pl, int t) {
        const float v = tile_dot<64, RP, 1>(T, S.xs, ly.pg.nb, lane);   // lane l: row t RP + l / 32
        const float gv = gelu_tanh(v) * pl;
        const float g_hi = __shfl_down(gv, 32, 64);
        if (lane == 0) ll_put(ly.ll_g, t, (uint32_t)f2h(gv) | ((uint32_t)f2h(g_hi) << 16), tag_of(l, PH_PG));
      };
      if (gw < ntiles_pg) body(Tp, plv, gw);
      for (int t = gw + nwaves; t < ntiles_pg; t += nwaves) {
        Tile<RP, 1> T = {};
        tile_load<64, RP, 1>(T, ly.pg, lane, [&](int r) { return (int64_t)(t * RP + r); });
        body(T, gc(a.ple)[(int64_t)l * PD + t * RP + (lane >> 5)], t);
      }
      lds_sync();
      mark(l, PH_PG, 2);
    }
    // ---------------------------------------------------------------- PP
    {
      mark(l, PH_PP, 0);
      const int tid = fresh_tid(), lane = tid & 63, gw = blockIdx.x * NW + (tid >> 6);
      const int grp = lane / LPP, l8 = lane % LPP;
      if (!poll_range<1>(ly.ll_g, PD / 2, tag_of(l, PH_PG), ab, &S.vote, tid, [&](int i, uint32_t p) { S.xs[i] = p; }))
        return;
      mark(l, PH_PP, 1);
      // the next layer's qkv tile and norm weights
      load_resw(rq, ly.post_norm, H, tid);
      if (l + 1 < a.layers) {
        const PersistLayer nx = LT[l + 1];
        Tq = {};
        if (gw < (QKV + 1) / 2)
          tile_load<64, 2, 1>(Tq, nx.qkv, lane, [&](int r) { return (int64_t)min(gw * 2 + r, QKV - 1); });
        load_normw(nq, nx.attn_norm, H, tid);
      }
      __builtin_amdgcn_sched_barrier(0);
      auto body = [&](const Tile<1, 1>& T, int t) {
        const float y = tile_dot<LPP, 1, 1>(T, S.xs, ly.pp.nb, l8);
        const int row = t * 8 + grp;
        if (l8 == 0 && row < H) ll_put(ly.ll_p, row, __float_as_uint(y), tag_of(l, PH_PP));
      };
      if (gw < ntiles_pp) body(Tpp, gw);
      for (int t = gw + nwaves; t < ntiles_pp; t += nwaves) {
        Tile<1, 1> T = {};
        tile_load<LPP, 1, 1>(T, ly.pp, l8, [&](int) { return (int64_t)min(t * 8 + grp, H - 1); });
        body(T, t);
      }
      lds_sync();
      mark(l, PH_PP, 2);
    }
  }
  // ------------------------------------------------------------------ tail
  if (blockIdx.x != 0) return;
  const PersistLayer last = LT[a.layers - 1];
  const int tid = threadIdx.x;
  if (!poll_range<kMaxH / NT>(last.ll_p, H, tag_of(a.layers - 1, PH_PP), ab, &S.vote, tid,
                              [&](int i, uint32_t p) { S.vs[i] = __uint_as_float(p); }))
    return;
  residual(S.hs, S.vs, rq, last.scale, H, a.eps, S.red, tid);
  float ss = 0.f;
  for (int i = tid; i < H; i += NT) ss = fmaf(S.hs[i], S.hs[i], ss);
  const float inv = rms_inv(block_sum8(ss, S.red, tid), H, a.eps);
  for (int i = tid; i < H; i += NT) {
    a.h_out[i] = S.hs[i];
    const float y = S.hs[i] * inv * a.out_norm[i];
    const _Float16 hi = (_Float16)y;
    a.xo_hl[i] = __builtin_bit_cast(uint16_t, hi);
    a.xo_hl[H + i] = __builtin_bit_cast(uint16_t, (_Float16)(y - (float)hi));
  }
  if (tid == 0) *a.epoch = ep + (uint32_t)(a.layers * PH_N) + 1u;
}

}  // namespace

bool persist_supported(int H, int FF, int QH, int KVH, int PD) {
  return H >= 256 && H <= kMaxH && H % 256 == 0 && QH == GQA * KVH && QH * HD <= 2048 && PD == 256 && FF >= 32 &&
         FF % 32 == 0 && FF / 2 <= kMaxXWords;
}

template <int CS, int BPLD>
static const void* persist_fn() {
  return reinterpret_cast<const void*>(&k_persist<CS, BPLD>);
}

static const void* persist_pick(int FF, int chunk) {
  const int bpl = (FF / 32 + 63) / 64;
  if (chunk == 64) {
    if (bpl <= 1) return persist_fn<64, 1>();
    if (bpl <= 2) return persist_fn<64, 2>();
    if (bpl <= 4) return persist_fn<64, 4>();
    if (bpl <= 8) return persist_fn<64, 8>();
  } else if (chunk == 32) {
    if (bpl <= 1) return persist_fn<32, 1>();
    if (bpl <= 2) return persist_fn<32, 2>();
    if (bpl <= 4) return persist_fn<32, 4>();
    if (bpl <= 8) return persist_fn<32, 8>();
  }
  return nullptr;
}

// One block per CU, and at most H / 8 blocks: then every wave owns one row
// of the o and down projections, so every block publishes words in every
// layer that every block waits for.  That chain is what makes rewriting a
// hand-off buffer one layer later safe: no block can still be reading it.
static char g_persist_why[256];

int persist_blocks(int H, int FF, int chunk) {
  const void* fn = persist_pick(FF, chunk);
  if (!fn) return 0;
  // an error an earlier call left pending would be returned by the queries
  // below instead of their own status
  (void)hipGetLastError();
  int dev = 0, cus = 0, per = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e == hipSuccess) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, fn, NT, 0);
  if (e != hipSuccess) return -(int)e;
  const int want = H / NW;
  if (per >= 1 && want <= cus) return want;
  hipFuncAttributes at{};
  int lds = 0;
  (void)hipFuncGetAttributes(&at, fn);
  (void)hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev);
  snprintf(g_persist_why, sizeof(g_persist_why),
           "occupancy %d block(s) per CU of %d threads (%d registers, %zu B LDS of %d), %d of %d CUs wanted", per, NT,
           at.numRegs, at.sharedSizeBytes, lds, want, cus);
  return 0;
}

const char* persist_why() { return g_persist_why; }

int launch_persist(const PersistArgs& a, int blocks, int chunk, hipStream_t st) {
  const void* fn = persist_pick(a.FF, chunk);
  if (!fn || blocks <= 0) return e4b_fail(E4B_EINVAL, "persistent step: unsupported shape (ffn %d, chunk %d)", a.FF, chunk);
  PersistArgs args = a;
  void* kargs[] = {&args};
  E4B_HIP(hipLaunchCooperativeKernel(fn, dim3(blocks), dim3(NT), kargs, 0, st));
  return E4B_OK;
}
