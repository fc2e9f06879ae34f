// k_step.hip -- the small decode-step kernels around the GEMVs and the
// attention: token embedding, per-layer-embedding (PLE) input prep, the final
// residual + norm before the lm-head, and the argmax fold with GPU-side
// greedy feedback.
//
// Position-dependent kernels read the current position from params[0] on the
// device, so one captured hipGraph serves every token.
#include "../../include/e4b.h"
#include "kernels.h"
#include "step.h"
#include "util.h"
#include "trace.h"

namespace {

constexpr int kMaxPer = 16;  // elements per thread in the one-block kernels (H <= 4096)

// Last residual of the step and the final norm: p = the sum of `np` partial
// PLE projections (or the down projection when there is no PLE);
// h = (h + rms(p) * w_post) * scale; xo = rms(h) * w_out stored as an
// f16 hi/lo pair for the lm-head (hi + lo within max(2^-22 |xo|, 2^-25) of xo) (kernels/a4btail.wgsl:26-71 with the
// reference's f32 final norm, src/engine-a4b.js:688).
template <int NP, int PER>
__global__ __launch_bounds__(256) void k_tail(float* __restrict__ h, const float* __restrict__ p,
                                              const float* __restrict__ w_post, float scale,
                                              const float* __restrict__ w_out, uint16_t* __restrict__ xo_hl, int H,
                                              float eps) {
  E4B_TRACE_SCOPE(trace_tag(TR_TAIL, 0));
  __shared__ float red[4];
  float hv[PER];
  float pv[PER];
  float wp[PER], wo[PER];
  // every input is requested before the first reduction waits
  float pp[PER][NP];
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int i = min((int)threadIdx.x + 256 * k, H - 1);
#pragma unroll
    for (int s = 0; s < NP; ++s) pp[k][s] = p[(int64_t)s * H + i];
    hv[k] = h[i];
    wp[k] = w_post[i];
    wo[k] = w_out[i];
  }
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const bool in = (int)threadIdx.x + 256 * k < H;
    float v = pp[k][0];
#pragma unroll
    for (int s = 1; s < NP; ++s) v += pp[k][s];
    pv[k] = in ? v : 0.f;
    ss = fmaf(pv[k], pv[k], ss);
  }
  const float inv = rms_inv(block_sum(ss, red), H, eps);
  float s2 = 0.f;
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const bool in = (int)threadIdx.x + 256 * k < H;
    hv[k] = in ? (hv[k] + pv[k] * inv * wp[k]) * scale : 0.f;
    s2 = fmaf(hv[k], hv[k], s2);
  }
  const float inv2 = rms_inv(block_sum(s2, red), H, eps);
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int i = threadIdx.x + 256 * k;
    if (i < H) {
      h[i] = hv[k];
      const float y = hv[k] * inv2 * wo[k];
      const _Float16 hi = (_Float16)y;
      xo_hl[i] = __builtin_bit_cast(uint16_t, hi);
      xo_hl[H + i] = __builtin_bit_cast(uint16_t, (_Float16)(y - (float)hi));
    }
  }
}

// token embedding: h = E[token] * sqrt(H) from the packed Q6_K lm-head planes
// (kernels/q6k.wgsl:37-73 with the TOKSRC feedback folded in), plus the
// f16 hi/lo pair of h for the PLE model projection.  The token is prompt[pos]
// while pos < params[3], else params[1] (GPU-fed greedy decode).  Block 0 also
// evaluates the step's RoPE table (cos, sin)(pos * inv_freq[p]) for local and
// global layers, the same expression the attention kernel would evaluate.
__global__ __launch_bounds__(256) void k_embed(Q6Mat E, const uint32_t* __restrict__ params,
                                               const uint32_t* __restrict__ prompt, float mult,
                                               float* __restrict__ h, uint16_t* __restrict__ h_hl,
                                               uint32_t* __restrict__ status, const float* __restrict__ inv_local,
                                               const float* __restrict__ inv_global, int half,
                                               float2* __restrict__ rope) {
  E4B_TRACE_SCOPE(trace_tag(TR_EMBED, 0));
  const uint32_t pos = params[0];
  if (blockIdx.x == 0)
    for (int t = threadIdx.x; t < 2 * half; t += 256) {
      const float f = t < half ? inv_local[t] : inv_global[t - half];
      float sn, cs;
      sincosf((float)pos * f, &sn, &cs);
      rope[t] = make_float2(cs, sn);
    }
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
  E4B_TRACE_SCOPE(trace_tag(TR_PLE_PREP, 0));
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
  // the projection value and norm weight load while the token chain
  // (position -> token -> table row) resolves; the reduction waits last
  const float pv = proj[b * 256 + t] * proj_scale;
  const float wn = w_pn[t];
  const uint32_t pos = params[0];
  uint32_t tok = pos < params[3] ? prompt[pos] : params[1];
  if (tok >= (uint32_t)vocab) tok = 0;
  const uint8_t* blk = table + ((int64_t)tok * L + b) * 210;
  const float idv = q6k_elem(blk, t) * 16.0f;  // sqrt(PD), PD = 256
  const float inv = rms_inv(block_sum(pv * pv, red), 256, eps);
  ple[b * 256 + t] = (pv * inv * wn + idv) * 0.70710678118654752f;
}

// argmax fold of the lm-head partials + GPU-side greedy feedback: the token
// becomes the next step's input (params[1]), is appended to the token ring,
// and the position advances (src/engine-a4b.js:786-824 decodeChunk with the
// feedtok of kernels/feedtok.wgsl folded in).  Ties -> lowest index, NaN never
// wins (kernels/argmax2.wgsl:8-48).
__global__ __launch_bounds__(256) void k_feedback(const uint2* __restrict__ part, int nparts, uint32_t* amax,
                                                  uint32_t* params, uint32_t* tok_ring, int ring_cap) {
  E4B_TRACE_SCOPE(trace_tag(TR_FEEDBACK, 0));
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
  lds_sync();
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
    params[4] = params[4] + 1;  // full-layer entries: the next token's slot
  }
}

}  // namespace

// ---- launchers --------------------------------------------------------------
template <int NP>
static void launch_tail_np(float* h, const float* p, const float* w_post, float scale, const float* w_out,
                           uint16_t* xo_hl, int H, float eps, hipStream_t st) {
  // elements per thread: the smallest power of two covering H over 256 threads
  if (H <= 256)
    hipLaunchKernelGGL((k_tail<NP, 1>), dim3(1), dim3(256), 0, st, h, p, w_post, scale, w_out, xo_hl, H, eps);
  else if (H <= 512)
    hipLaunchKernelGGL((k_tail<NP, 2>), dim3(1), dim3(256), 0, st, h, p, w_post, scale, w_out, xo_hl, H, eps);
  else if (H <= 1024)
    hipLaunchKernelGGL((k_tail<NP, 4>), dim3(1), dim3(256), 0, st, h, p, w_post, scale, w_out, xo_hl, H, eps);
  else if (H <= 2048)
    hipLaunchKernelGGL((k_tail<NP, 8>), dim3(1), dim3(256), 0, st, h, p, w_post, scale, w_out, xo_hl, H, eps);
  else
    hipLaunchKernelGGL((k_tail<NP, kMaxPer>), dim3(1), dim3(256), 0, st, h, p, w_post, scale, w_out, xo_hl, H, eps);
}

int launch_tail(float* h, const float* p, int np, const float* w_post, float scale, const float* w_out,
                uint16_t* xo_hl, int H, float eps, hipStream_t st) {
  if (np != 1 && np != kMaxPartials) return e4b_fail(E4B_EINVAL, "tail: %d partial vectors (1 or %d)", np, kMaxPartials);
  if (H < 1 || H > 256 * kMaxPer) return e4b_fail(E4B_EINVAL, "tail: hidden %d outside 1..%d", H, 256 * kMaxPer);
  if (np == 1)
    launch_tail_np<1>(h, p, w_post, scale, w_out, xo_hl, H, eps, st);
  else
    launch_tail_np<kMaxPartials>(h, p, w_post, scale, w_out, xo_hl, H, eps, st);
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}
int launch_embed(const Q6Mat& E, const uint32_t* params, const uint32_t* prompt, float mult, float* h, uint16_t* h_hl,
                 uint32_t* status, const float* inv_local, const float* inv_global, int half, float2* rope,
                 hipStream_t st) {
  hipLaunchKernelGGL(k_embed, dim3((E.nseg + 255) / 256), dim3(256), 0, st, E, params, prompt, mult, h, h_hl, status,
                     inv_local, inv_global, half, rope);
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
