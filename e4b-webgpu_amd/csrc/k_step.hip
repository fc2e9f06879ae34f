// k_step.hip -- decode-step kernels other than the GEMVs: head prep + split-K
// attention over the f16 KV cache (sliding ring or linear), the chunk
// combine, the residual/norm kernels, the token embedding and the
// per-layer-embedding (PLE) input prep.
//
// Position-dependent kernels read the current position from params[0] on the
// device, so one captured hipGraph serves every token.
#include "../../include/e4b.h"
#include "kernels.h"
#include "step.h"
#include "util.h"

namespace {

// ---- block-wide reductions (256 threads = 4 waves) ---------------------------
DEV float wave_sum(float v) {
  v = xsum_step<32>(v);
  v = xsum_step<16>(v);
  v = xsum_step<8>(v);
  v = xsum_step<4>(v);
  v = xsum_step<2>(v);
  return xsum_step<1>(v);
}
DEV float wave_max(float v) {
  float t = v;
  swapx32(v, t);
  v = fmaxf(v, t);
  t = v;
  swapx16(v, t);
  v = fmaxf(v, t);
  v = fmaxf(v, lane_xor<8>(v));
  v = fmaxf(v, lane_xor<4>(v));
  v = fmaxf(v, lane_xor<2>(v));
  return fmaxf(v, lane_xor<1>(v));
}
// sum over the block; every thread gets the total.  `red` is 4 floats of LDS.
DEV float block_sum(float v, float* red) {
  v = wave_sum(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

// rms scale (mean(x^2) + eps)^-1/2 from a sum of squares
DEV float rms_inv(float ss, int n, float eps) { return 1.0f / sqrtf(ss / (float)n + eps); }

constexpr int kMaxPer = 16;  // elements per thread in the one-block norm kernels (H <= 4096)

// ---------------------------------------------------------------------------
// attention: grid (KVH, NCH); block = 4 waves; the 4 q heads of one KV group
// (GQA 4:1), one chunk of live positions.
// ---------------------------------------------------------------------------
struct AttnArgs {
  const float* qkv;       // raw q | k | v of this token
  const float* qw;        // q head-norm weight [HD]
  const float* kw;        // k head-norm weight [HD]
  const float* inv_freq;  // RoPE inverse frequencies [angles]
  uint16_t* kc;           // [KVH][slots][HD] f16
  uint16_t* vc;
  const uint32_t* params; // [0] = position
  float* part_o;          // [QH][NCH][HD]
  float* part_ml;         // [QH][NCH][2]
  int qh, kvh, angles, slots, window, nch;
  float eps;
};
constexpr int HD = 256;
constexpr int GQA = 4;
constexpr int kMaxChunk = 1024;

// weighted head RMS over 256 dims held 4 per lane, then NeoX-half RoPE:
// dims p < 128 (lanes 0..31) pair with p + 128 (lanes 32..63).
DEV void prep_head(float (&x)[4], const float* w, const float* inv_freq, int angles, float eps, float fpos,
                   bool rotate) {
  const int lane = threadIdx.x & 63;
  float ss = x[0] * x[0] + x[1] * x[1] + x[2] * x[2] + x[3] * x[3];
  ss = wave_sum(ss);
  const float inv = rms_inv(ss, HD, eps);
#pragma unroll
  for (int i = 0; i < 4; ++i) x[i] = x[i] * inv * (w ? w[4 * lane + i] : 1.f);
  if (!rotate) return;
  const bool hi = lane >= 32;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float a = x[i], b = x[i];
    swapx32(a, b);  // a (lo lanes) = own, b (lo lanes) = partner's; reversed for hi lanes
    const float partner = hi ? a : b;
    const int p = 4 * (lane & 31) + i;
    if (p < angles) {
      const float th = fpos * inv_freq[p];
      float sn, cs;
      sincosf(th, &sn, &cs);
      // lo lane holds x0 (dim p), hi lane holds x1 (dim p+128)
      x[i] = hi ? (partner * sn + x[i] * cs) : (x[i] * cs - partner * sn);
    }
  }
}

__global__ __launch_bounds__(256) void k_attn(AttnArgs A) {
  __shared__ float qs[GQA][HD];
  __shared__ float sc[GQA][kMaxChunk];
  __shared__ float po[4][GQA][HD];
  __shared__ float mlx[GQA][2];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = blockIdx.x, c = blockIdx.y;
  const int64_t pos = A.params[0];
  const int64_t lo = (A.window > 0 && pos + 1 > A.window) ? pos + 1 - A.window : 0;
  const int64_t n = pos + 1 - lo;
  const int64_t cs = (n + A.nch - 1) / A.nch;
  const int64_t c_lo = lo + c * cs, c_hi = min(lo + (c + 1) * cs, pos + 1);
  const float fpos = (float)pos;
  uint16_t* kc = A.kc + (int64_t)g * A.slots * HD;
  uint16_t* vc = A.vc + (int64_t)g * A.slots * HD;

  // 1. head prep: wave j -> q head 4g+j; the chunk owning `pos` also preps k/v
  {
    float x[4];
    const float* qsrc = A.qkv + (int64_t)(g * GQA + wave) * HD + 4 * lane;
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = qsrc[i];
    prep_head(x, A.qw, A.inv_freq, A.angles, A.eps, fpos, true);
#pragma unroll
    for (int i = 0; i < 4; ++i) qs[wave][4 * lane + i] = x[i];
  }
  const bool owner = (pos >= c_lo && pos < c_hi);
  if (owner && wave < 2) {
    float x[4];
    const float* src = A.qkv + (int64_t)(A.qh + (wave == 0 ? 0 : A.kvh) + g) * HD + 4 * lane;
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = src[i];
    prep_head(x, wave == 0 ? A.kw : nullptr, A.inv_freq, A.angles, A.eps, fpos, wave == 0);
    const int64_t slot = A.window > 0 ? pos % A.slots : pos;
    uint16_t* dst = (wave == 0 ? kc : vc) + slot * HD + 4 * lane;
    const uint32_t lo2 = (uint32_t)f2h(x[0]) | ((uint32_t)f2h(x[1]) << 16);
    const uint32_t hi2 = (uint32_t)f2h(x[2]) | ((uint32_t)f2h(x[3]) << 16);
    *reinterpret_cast<uint2*>(dst) = make_uint2(lo2, hi2);
  }
  __syncthreads();  // q in LDS; this block's own cache write is visible to it

  const int m = (int)max((int64_t)0, c_hi - c_lo);
  if (m == 0) {
    for (int i = threadIdx.x; i < GQA * HD; i += 256) A.part_o[((int64_t)(g * GQA + i / HD) * A.nch + c) * HD + i % HD] = 0.f;
    if (threadIdx.x < GQA) {
      A.part_ml[((int64_t)(g * GQA + threadIdx.x) * A.nch + c) * 2 + 0] = -3.0e38f;
      A.part_ml[((int64_t)(g * GQA + threadIdx.x) * A.nch + c) * 2 + 1] = 0.f;
    }
    return;
  }

  // 2. scores: 16 lanes per position (16 dims each), 4 positions per wave-step
  {
    const int sub = lane >> 4, dl = lane & 15;
    float q[GQA][16];
#pragma unroll
    for (int h = 0; h < GQA; ++h)
#pragma unroll
      for (int i = 0; i < 16; ++i) q[h][i] = qs[h][16 * dl + i];
    for (int j0 = wave * 4; j0 < m; j0 += 16) {
      const int j = j0 + sub;
      const int jj = min(j, m - 1);
      const int64_t p = c_lo + jj;
      const int64_t slot = A.window > 0 ? p % A.slots : p;
      const uint4* kr = reinterpret_cast<const uint4*>(kc + slot * HD + 16 * dl);
      const uint4 k0 = kr[0], k1 = kr[1];
      const uint32_t kw8[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
      float kf[16];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        kf[2 * i] = h2f((uint16_t)(kw8[i] & 0xffff));
        kf[2 * i + 1] = h2f((uint16_t)(kw8[i] >> 16));
      }
      float s[GQA];
#pragma unroll
      for (int h = 0; h < GQA; ++h) {
        float a = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) a = fmaf(q[h][i], kf[i], a);
        s[h] = a;
      }
      const float v = reduce_rows<16, GQA>(s);  // lane dl holds head dl/4
      if ((dl & 3) == 0 && j < m) sc[dl >> 2][j] = v;
    }
  }
  __syncthreads();

  // 3. chunk softmax stats: wave h owns head h
  {
    float mx = -3.0e38f;
    for (int j = lane; j < m; j += 64) mx = fmaxf(mx, sc[wave][j]);
    mx = wave_max(mx);
    float sum = 0.f;
    for (int j = lane; j < m; j += 64) {
      const float e = __expf(sc[wave][j] - mx);
      sc[wave][j] = e;
      sum += e;
    }
    sum = wave_sum(sum);
    if (lane == 0) {
      mlx[wave][0] = mx;
      mlx[wave][1] = sum;
    }
  }
  __syncthreads();

  // 4. P.V: wave w takes positions j = w, w+4, ...; lane covers dims 4l..4l+3
  {
    float acc[GQA][4];
#pragma unroll
    for (int h = 0; h < GQA; ++h)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[h][i] = 0.f;
    for (int j = wave; j < m; j += 4) {
      const int64_t p = c_lo + j;
      const int64_t slot = A.window > 0 ? p % A.slots : p;
      const uint2 vv = *reinterpret_cast<const uint2*>(vc + slot * HD + 4 * lane);
      const float vf[4] = {h2f((uint16_t)(vv.x & 0xffff)), h2f((uint16_t)(vv.x >> 16)),
                           h2f((uint16_t)(vv.y & 0xffff)), h2f((uint16_t)(vv.y >> 16))};
#pragma unroll
      for (int h = 0; h < GQA; ++h) {
        const float pj = sc[h][j];
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[h][i] = fmaf(pj, vf[i], acc[h][i]);
      }
    }
#pragma unroll
    for (int h = 0; h < GQA; ++h)
#pragma unroll
      for (int i = 0; i < 4; ++i) po[wave][h][4 * lane + i] = acc[h][i];
  }
  __syncthreads();
  for (int i = threadIdx.x; i < GQA * HD; i += 256) {
    const int h = i / HD, d = i % HD;
    const float v = (po[0][h][d] + po[1][h][d]) + (po[2][h][d] + po[3][h][d]);
    A.part_o[((int64_t)(g * GQA + h) * A.nch + c) * HD + d] = v;
  }
  if (threadIdx.x < GQA) {
    A.part_ml[((int64_t)(g * GQA + threadIdx.x) * A.nch + c) * 2 + 0] = mlx[threadIdx.x][0];
    A.part_ml[((int64_t)(g * GQA + threadIdx.x) * A.nch + c) * 2 + 1] = mlx[threadIdx.x][1];
  }
}

// combine: one block per q head; o = sum_c partO_c e^{m_c - M} / sum_c l_c e^{m_c - M}
__global__ __launch_bounds__(256) void k_attn_combine(const float* __restrict__ part_o,
                                                      const float* __restrict__ part_ml, int nch,
                                                      uint16_t* __restrict__ out) {
  const int h = blockIdx.x, d = threadIdx.x;
  float M = -3.0e38f;
  for (int c = 0; c < nch; ++c) {
    const float l = part_ml[((int64_t)h * nch + c) * 2 + 1];
    if (l > 0.f) M = fmaxf(M, part_ml[((int64_t)h * nch + c) * 2]);
  }
  float den = 0.f, acc = 0.f;
  for (int c = 0; c < nch; ++c) {
    const float m = part_ml[((int64_t)h * nch + c) * 2], l = part_ml[((int64_t)h * nch + c) * 2 + 1];
    if (l > 0.f) {
      const float f = __expf(m - M);
      den = fmaf(l, f, den);
      acc = fmaf(part_o[((int64_t)h * nch + c) * HD + d], f, acc);
    }
  }
  out[h * HD + d] = f2h(acc / den);
}

// ---------------------------------------------------------------------------
// one-block residual / norm kernels (hidden size H <= 4096)
// ---------------------------------------------------------------------------

// h += rms(o) * w_pa;  xf = f16(rms(h) * w_ffn)       (kernels/rmsacc3.wgsl:36-53)
__global__ __launch_bounds__(256) void k_post_attn(float* __restrict__ h, const float* __restrict__ o,
                                                   const float* __restrict__ w_pa, const float* __restrict__ w_ffn,
                                                   uint16_t* __restrict__ xf, int H, float eps) {
  __shared__ float red[4];
  float ov[kMaxPer], hv[kMaxPer];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < kMaxPer; ++k) {
    const int i = threadIdx.x + 256 * k;
    ov[k] = i < H ? o[i] : 0.f;
    hv[k] = i < H ? h[i] : 0.f;
    ss = fmaf(ov[k], ov[k], ss);
  }
  const float inv1 = rms_inv(block_sum(ss, red), H, eps);
  float s2 = 0.f;
#pragma unroll
  for (int k = 0; k < kMaxPer; ++k) {
    const int i = threadIdx.x + 256 * k;
    if (i < H) hv[k] = hv[k] + ov[k] * inv1 * w_pa[i];
    s2 = fmaf(hv[k], hv[k], s2);
  }
  const float inv2 = rms_inv(block_sum(s2, red), H, eps);
#pragma unroll
  for (int k = 0; k < kMaxPer; ++k) {
    const int i = threadIdx.x + 256 * k;
    if (i < H) {
      h[i] = hv[k];
      xf[i] = f2h(hv[k] * inv2 * w_ffn[i]);
    }
  }
}

// dn = sum of ks partials; h += rms(dn) * w_pf; xg = f16(h)
__global__ __launch_bounds__(256) void k_post_ffn(float* __restrict__ h, const float* __restrict__ dn, int ks,
                                                  const float* __restrict__ w_pf, uint16_t* __restrict__ xg, int H,
                                                  float eps) {
  __shared__ float red[4];
  float dv[kMaxPer];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < kMaxPer; ++k) {
    const int i = threadIdx.x + 256 * k;
    float v = 0.f;
    if (i < H)
      for (int s = 0; s < ks; ++s) v += dn[(int64_t)s * H + i];
    dv[k] = v;
    ss = fmaf(v, v, ss);
  }
  const float inv = rms_inv(block_sum(ss, red), H, eps);
#pragma unroll
  for (int k = 0; k < kMaxPer; ++k) {
    const int i = threadIdx.x + 256 * k;
    if (i < H) {
      const float hn = h[i] + dv[k] * inv * w_pf[i];
      h[i] = hn;
      xg[i] = f2h(hn);
    }
  }
}

// h = (h + rms(p) * w_post) * scale (p may be null: h *= scale); then the next
// layer's input norm xn = f16(rms(h) * w_next), or for the last layer the
// final norm xo = rms(h) * w_out stored as an exact f16 hi/lo split.
__global__ __launch_bounds__(256) void k_tail(float* __restrict__ h, const float* __restrict__ p,
                                              const float* __restrict__ w_post, float scale,
                                              const float* __restrict__ w_next, uint16_t* __restrict__ xn,
                                              uint16_t* __restrict__ xo_hl, int H, float eps) {
  __shared__ float red[4];
  float hv[kMaxPer];
  float inv = 0.f;
  if (p) {
    float pv[kMaxPer];
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < kMaxPer; ++k) {
      const int i = threadIdx.x + 256 * k;
      pv[k] = i < H ? p[i] : 0.f;
      ss = fmaf(pv[k], pv[k], ss);
    }
    inv = rms_inv(block_sum(ss, red), H, eps);
#pragma unroll
    for (int k = 0; k < kMaxPer; ++k) {
      const int i = threadIdx.x + 256 * k;
      hv[k] = i < H ? (h[i] + pv[k] * inv * w_post[i]) * scale : 0.f;
    }
  } else {
#pragma unroll
    for (int k = 0; k < kMaxPer; ++k) {
      const int i = threadIdx.x + 256 * k;
      hv[k] = i < H ? h[i] * scale : 0.f;
    }
  }
  float s2 = 0.f;
#pragma unroll
  for (int k = 0; k < kMaxPer; ++k) s2 = fmaf(hv[k], hv[k], s2);
  const float inv2 = rms_inv(block_sum(s2, red), H, eps);
#pragma unroll
  for (int k = 0; k < kMaxPer; ++k) {
    const int i = threadIdx.x + 256 * k;
    if (i < H) {
      h[i] = hv[k];
      const float y = hv[k] * inv2 * w_next[i];
      if (xn) {
        xn[i] = f2h(y);
      } else {
        const _Float16 hi = (_Float16)y;
        xo_hl[i] = __builtin_bit_cast(uint16_t, hi);
        xo_hl[H + i] = __builtin_bit_cast(uint16_t, (_Float16)(y - (float)hi));
      }
    }
  }
}

// ---------------------------------------------------------------------------
// token embedding: h = E[token] * sqrt(H) from the packed Q6_K lm-head planes
// (kernels/q6k.wgsl:37-73 with TOKSRC feedback folded in); also the exact
// hi/lo split of h for the PLE model projection.  The token is prompt[pos]
// while pos < params[3], else params[1] (GPU-fed greedy decode).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_embed(Q6Mat E, const uint32_t* __restrict__ params,
                                               const uint32_t* __restrict__ prompt, float mult,
                                               float* __restrict__ h, uint16_t* __restrict__ h_hl,
                                               uint32_t* __restrict__ status) {
  const uint32_t pos = params[0];
  uint32_t tok = pos < params[3] ? prompt[pos] : params[1];
  if (tok >= (uint32_t)E.rows) {
    if (threadIdx.x == 0 && blockIdx.x == 0) status[0] = 1u;  // reported by the host as E4B_ERANGE
    tok = 0;
  }
  const int H = E.nseg * 32;
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
          h[e] = v;
          const _Float16 hi = (_Float16)v;
          h_hl[e] = __builtin_bit_cast(uint16_t, hi);
          h_hl[H + e] = __builtin_bit_cast(uint16_t, (_Float16)(v - (float)hi));
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

// PLE input prep (kernels/pleprep.wgsl:15-46, src/engine.js:282-323): block b
// < L builds ple[b] = (rms(proj_b * H^-1/2) * w_pn + table_row_b(token) *
// sqrt(PD)) * 2^-1/2 with PD = 256 (one Q6_K superblock per layer block);
// block L computes layer 0's input norm xn = f16(rms(h) * w_attn0).
__global__ __launch_bounds__(256) void k_ple_prep(const float* __restrict__ proj, const uint8_t* __restrict__ table,
                                                  const float* __restrict__ w_pn, const uint32_t* __restrict__ params,
                                                  const uint32_t* __restrict__ prompt, int L, int vocab,
                                                  float proj_scale, float* __restrict__ ple,
                                                  const float* __restrict__ h, const float* __restrict__ w_attn0,
                                                  uint16_t* __restrict__ xn, int H, float eps) {
  __shared__ float red[4];
  const int b = blockIdx.x, t = threadIdx.x;
  if (b == L) {
    float hv[kMaxPer];
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < kMaxPer; ++k) {
      const int i = t + 256 * k;
      hv[k] = i < H ? h[i] : 0.f;
      ss = fmaf(hv[k], hv[k], ss);
    }
    const float inv = rms_inv(block_sum(ss, red), H, eps);
#pragma unroll
    for (int k = 0; k < kMaxPer; ++k) {
      const int i = t + 256 * k;
      if (i < H) xn[i] = f2h(hv[k] * inv * w_attn0[i]);
    }
    return;
  }
  const uint32_t pos = params[0];
  uint32_t tok = pos < params[3] ? prompt[pos] : params[1];
  if (tok >= (uint32_t)vocab) tok = 0;
  const float pv = proj[b * 256 + t] * proj_scale;
  const float inv = rms_inv(block_sum(pv * pv, red), 256, eps);
  const uint8_t* blk = table + ((int64_t)tok * L + b) * 210;
  const float idv = q6k_elem(blk, t) * 16.0f;  // sqrt(PD), PD = 256
  ple[b * 256 + t] = (pv * inv * w_pn[t] + idv) * 0.70710678118654752f;
}

// argmax fold of the lm-head partials + GPU-side greedy feedback: the token
// becomes the next step's input (params[1]), is appended to the token ring,
// and the position advances (src/engine-a4b.js:786-824 decodeChunk with the
// feedtok of kernels/feedtok.wgsl folded in).
__global__ __launch_bounds__(256) void k_feedback(const uint2* __restrict__ part, int nparts, uint32_t* amax,
                                                  uint32_t* params, uint32_t* tok_ring, int ring_cap) {
  __shared__ float sv[4];
  __shared__ uint32_t si[4];
  float v = -3.0e38f;
  uint32_t i = 0;
  for (int b = threadIdx.x; b < nparts; b += 256) {
    const uint2 p = part[b];
    const float pv = __uint_as_float(p.y);
    if (pv > v || (pv == v && p.x < i)) {
      v = pv;
      i = p.x;
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(v, off, 64);
    const uint32_t oi = __shfl_xor(i, off, 64);
    if (ov > v || (ov == v && oi < i)) {
      v = ov;
      i = oi;
    }
  }
  if ((threadIdx.x & 63) == 0) {
    sv[threadIdx.x >> 6] = v;
    si[threadIdx.x >> 6] = i;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 4; ++w)
      if (sv[w] > sv[0] || (sv[w] == sv[0] && si[w] < si[0])) {
        sv[0] = sv[w];
        si[0] = si[w];
      }
    amax[0] = si[0];
    amax[1] = __float_as_uint(sv[0]);
    const uint32_t r = params[2];
    if ((int)r < ring_cap) tok_ring[r] = si[0];
    params[1] = si[0];
    params[2] = r + 1;
    params[0] = params[0] + 1;
  }
}

}  // namespace

// ---- launchers --------------------------------------------------------------
int launch_attn(const AttnLaunch& a, hipStream_t st) {
  if (a.hd != HD || a.qh != GQA * a.kvh)
    return e4b_fail(E4B_EINVAL, "attention kernel supports head_dim 256 and 4 q heads per kv head (got %d, %d/%d)", a.hd,
                    a.qh, a.kvh);
  if (a.nch < 1) return e4b_fail(E4B_EINVAL, "attention: nch %d", a.nch);
  AttnArgs A;
  A.qkv = a.qkv;
  A.qw = a.qw;
  A.kw = a.kw;
  A.inv_freq = a.inv_freq;
  A.kc = a.kc;
  A.vc = a.vc;
  A.params = a.params;
  A.part_o = a.part_o;
  A.part_ml = a.part_ml;
  A.qh = a.qh;
  A.kvh = a.kvh;
  A.angles = a.angles;
  A.slots = a.slots;
  A.window = a.window;
  A.nch = a.nch;
  A.eps = a.eps;
  hipLaunchKernelGGL(k_attn, dim3(a.kvh, a.nch), dim3(256), 0, st, A);
  hipLaunchKernelGGL(k_attn_combine, dim3(a.qh), dim3(256), 0, st, a.part_o, a.part_ml, a.nch, a.out);
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}

int attn_max_positions(int nch) { return nch * kMaxChunk; }

int launch_post_attn(float* h, const float* o, const float* w_pa, const float* w_ffn, uint16_t* xf, int H, float eps,
                     hipStream_t st) {
  hipLaunchKernelGGL(k_post_attn, dim3(1), dim3(256), 0, st, h, o, w_pa, w_ffn, xf, H, eps);
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}
int launch_post_ffn(float* h, const float* dn, int ks, const float* w_pf, uint16_t* xg, int H, float eps,
                    hipStream_t st) {
  hipLaunchKernelGGL(k_post_ffn, dim3(1), dim3(256), 0, st, h, dn, ks, w_pf, xg, H, eps);
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}
int launch_tail(float* h, const float* p, const float* w_post, float scale, const float* w_next, uint16_t* xn,
                uint16_t* xo_hl, int H, float eps, hipStream_t st) {
  hipLaunchKernelGGL(k_tail, dim3(1), dim3(256), 0, st, h, p, w_post, scale, w_next, xn, xo_hl, H, eps);
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}
int launch_embed(const Q6Mat& E, const uint32_t* params, const uint32_t* prompt, float mult, float* h, uint16_t* h_hl,
                 uint32_t* status, hipStream_t st) {
  hipLaunchKernelGGL(k_embed, dim3((E.nseg + 255) / 256), dim3(256), 0, st, E, params, prompt, mult, h, h_hl, status);
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}
int launch_ple_prep(const float* proj, const uint8_t* table, const float* w_pn, const uint32_t* params,
                    const uint32_t* prompt, int L, int vocab, float proj_scale, float* ple, const float* h,
                    const float* w_attn0, uint16_t* xn, int H, float eps, hipStream_t st) {
  hipLaunchKernelGGL(k_ple_prep, dim3(L + 1), dim3(256), 0, st, proj, table, w_pn, params, prompt, L, vocab, proj_scale,
                     ple, h, w_attn0, xn, H, eps);
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}
int launch_feedback(const uint2* part, int nparts, uint32_t* amax, uint32_t* params, uint32_t* tok_ring, int ring_cap,
                    hipStream_t st) {
  hipLaunchKernelGGL(k_feedback, dim3(1), dim3(256), 0, st, part, nparts, amax, params, tok_ring, ring_cap);
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}
