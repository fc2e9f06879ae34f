// k_a4b.hip -- step kernels of the A4B recipe (src/engine-a4b.js:424-463)
// that the E4B kernels do not cover:
//   k_rownorm       residual + RMSNorm of one vector, any hidden size up to
//                   4096 (kernels/rmsacc3.wgsl:36-53, kernels/rmsnorm.wgsl
//                   :13-51; one workgroup)
//   k_headprep_gen  q/k weighted head-RMS + NeoX RoPE over the first
//                   `angles` pairs, scale-less v RMS with V read from the raw
//                   K slice on KEQV layers, K/V row write at the token's slot
//                   (kernels/headprep.wgsl:19-87), head dim 256 or 512, any
//                   number of KV heads
//   k_attn_chunk    split-K partials of one (q head, chunk of 64 positions):
//                   scale-1.0 scores, the chunk's max and exponential sum, the
//                   unnormalised P.V (kernels/attsplit.wgsl:16-76 over the
//                   ring of attnf32.wgsl:21-105 or the counted slots of
//                   attnos.wgsl:22-98)
//   k_attn_merge    log-sum-exp merge of a head's live chunks to f16
//                   (kernels/attcomb.wgsl:10-36)
#include "../../include/e4b.h"
#include "a4b.h"
#include "kernels.h"
#include "util.h"

namespace {

constexpr int kRowMax = 16;  // elements per thread of k_rownorm: H <= 16 * 256

// thread t owns the elements i = t + 256 k
__global__ __launch_bounds__(256) void k_rownorm(const float* __restrict__ h_in, float* __restrict__ h_out,
                                                 const float* __restrict__ a, const float* __restrict__ w1, float scale,
                                                 const float* __restrict__ w2, uint16_t* __restrict__ x,
                                                 uint16_t* __restrict__ xlo, int H, float eps) {
  __shared__ float red[4];
  const int t = threadIdx.x;
  float hv[kRowMax], av[kRowMax];
#pragma unroll
  for (int k = 0; k < kRowMax; ++k) {
    const int i = t + 256 * k;
    hv[k] = i < H ? h_in[i] : 0.f;
    av[k] = (a && i < H) ? a[i] : 0.f;
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

// one wave per head row b: q heads [0, qh), k heads [qh, qh + kvh), v heads
// [qh + kvh, qh + 2 kvh).  Lane l holds the PER = HD / 64 contiguous dims
// [PER l, PER l + PER): the RoPE partner of dim p < HD / 2 (p + HD / 2) sits
// in lane l + 32.
template <int HD>
__global__ __launch_bounds__(64) void k_headprep_gen(HeadPrepGen A) {
  constexpr int PER = HD / 64;
  const int b = blockIdx.x, lane = threadIdx.x;
  const int QH = A.qh, KVH = A.kvh;
  const int kind = b < QH ? 0 : b < QH + KVH ? 1 : 2;  // q, k, v
  const int g = kind == 0 ? b : kind == 1 ? b - QH : b - QH - KVH;
  const int src = kind == 0 ? b : kind == 1 ? QH + g : (A.keqv ? QH + g : QH + KVH + g);
  const float* xr = A.qkv + (int64_t)src * HD + PER * lane;
  float x[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) x[i] = xr[i];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < PER; ++i) ss = fmaf(x[i], x[i], ss);
  const float inv = rms_inv(wave_sum(ss), HD, A.eps);
  const float* w = kind == 0 ? A.qw : A.kw;
#pragma unroll
  for (int i = 0; i < PER; ++i) x[i] = x[i] * inv * (kind < 2 ? w[PER * lane + i] : 1.f);
  const uint32_t pos = A.params[0];
  if (kind < 2) {
    const float fpos = (float)pos;
    const bool hi = lane >= 32;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      float lo_v = x[i], hi_v = x[i];
      swapx32(lo_v, hi_v);  // lanes < 32: hi_v = partner (dim p + HD/2); lanes >= 32: lo_v = partner (dim p)
      const float partner = hi ? lo_v : hi_v;
      const int p = PER * (lane & 31) + i;
      if (p < A.angles) {
        float sn, c;
        sincosf(fpos * A.inv_freq[p], &sn, &c);
        x[i] = hi ? (partner * sn + x[i] * c) : (x[i] * c - partner * sn);
      }
    }
  }
  if (kind == 0) {
    float* q = A.q + (int64_t)b * HD + PER * lane;
#pragma unroll
    for (int i = 0; i < PER; ++i) q[i] = x[i];
    return;
  }
  const uint32_t slot = A.window > 0 ? pos % (uint32_t)A.slots : A.params[A.kv_idx];
  uint16_t* dst = (kind == 1 ? A.kc : A.vc) + ((int64_t)g * A.slots + slot) * HD + PER * lane;
#pragma unroll
  for (int i = 0; i < PER; ++i) dst[i] = f2h(x[i]);
}

// live positions of the layer at this step: (lo, n) with the token's index
// `cur` in the cache's own numbering (the position on a ring, the counted
// slot on a full layer)
struct Live {
  int cur, lo, n;
};
DEV Live live_of(const AttnGen& A) {
  const int pos = (int)A.params[0];
  Live L;
  L.cur = A.window > 0 ? pos : (int)A.params[A.kv_idx];
  L.lo = (A.window > 0 && L.cur + 1 > A.window) ? L.cur + 1 - A.window : 0;
  L.n = L.cur + 1 - L.lo;
  return L;
}

// block (head h, chunk c); wave w scores positions j = w + 4 i of the chunk,
// one position per pass, each lane PER = HD / 64 dims of the key
template <int HD>
__global__ __launch_bounds__(256) void k_attn_chunk(AttnGen A) {
  constexpr int CS = kAttnGenChunk, PER = HD / 64, PW = CS / 4;
  __shared__ float qs[HD];
  __shared__ float es[CS];
  __shared__ float red[4];
  const int h = blockIdx.x, c = blockIdx.y, t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const Live L = live_of(A);
  const int nch = (L.n + CS - 1) / CS;
  if (c >= nch) return;
  const int c_lo = L.lo + c * CS;
  const int m = min(CS, L.n - c * CS);
  const int g = h / (A.qh / A.kvh);
  const uint16_t* kc = A.kc + (int64_t)g * A.slots * HD;
  const uint16_t* vc = A.vc + (int64_t)g * A.slots * HD;
  const int s_lo = A.window > 0 ? c_lo % A.slots : c_lo;
  auto slot_at = [&](int j) -> int64_t {
    const int s = s_lo + j;
    return (A.window > 0 && s >= A.slots) ? s - A.slots : s;
  };
  // the wave's key rows, requested before the query is staged
  uint32_t kr[PW][PER / 2];
#pragma unroll
  for (int i = 0; i < PW; ++i) {
    const int j = min(wave + 4 * i, m - 1);
    const uint32_t* row = reinterpret_cast<const uint32_t*>(kc + slot_at(j) * HD + PER * lane);
#pragma unroll
    for (int e = 0; e < PER / 2; ++e) kr[i][e] = row[e];
  }
  for (int d = t; d < HD; d += 256) qs[d] = A.q[(int64_t)h * HD + d];
  lds_sync();
  float qv[PER];
#pragma unroll
  for (int e = 0; e < PER; ++e) qv[e] = qs[PER * lane + e];
#pragma unroll
  for (int i = 0; i < PW; ++i) {
    float dot = 0.f;
#pragma unroll
    for (int e = 0; e < PER / 2; ++e) {
      dot = fmaf(qv[2 * e], h2f((uint16_t)(kr[i][e] & 0xffffu)), dot);
      dot = fmaf(qv[2 * e + 1], h2f((uint16_t)(kr[i][e] >> 16)), dot);
    }
    dot = wave_sum(dot);
    const int j = wave + 4 * i;
    if (lane == 0 && j < m) es[j] = dot;
  }
  lds_sync();
  const float s = t < m ? es[t] : -3.0e38f;
  const float M = block_max(s, red);
  const float e = t < m ? __expf(s - M) : 0.f;
  const float lsum = block_sum(e, red);
  if (t < CS) es[t] = e;
  lds_sync();
  for (int d = t; d < HD; d += 256) {
    float acc = 0.f;
    for (int j = 0; j < m; ++j) acc = fmaf(es[j], h2f(vc[slot_at(j) * HD + d]), acc);
    A.part_o[((int64_t)h * A.gch + c) * HD + d] = acc;
  }
  if (t == 0) {
    A.part_ml[((int64_t)h * A.gch + c) * 2] = M;
    A.part_ml[((int64_t)h * A.gch + c) * 2 + 1] = lsum;
  }
}

// one block per head: out = sum_c e^(m_c - M) part_o[c] / sum_c e^(m_c - M) l_c
template <int HD>
__global__ __launch_bounds__(256) void k_attn_merge(AttnGen A) {
  constexpr int CS = kAttnGenChunk;
  __shared__ float red[4];
  const int h = blockIdx.x, t = threadIdx.x;
  const Live L = live_of(A);
  const int nch = (L.n + CS - 1) / CS;
  const float* ml = A.part_ml + (int64_t)h * A.gch * 2;
  float mloc = -3.0e38f;
  for (int c = t; c < nch; c += 256) mloc = fmaxf(mloc, ml[2 * c]);
  const float M = block_max(mloc, red);
  float den = 0.f;
  for (int c = t; c < nch; c += 256) den += __expf(ml[2 * c] - M) * ml[2 * c + 1];
  den = block_sum(den, red);
  for (int d = t; d < HD; d += 256) {
    float acc = 0.f;
    for (int c = 0; c < nch; ++c) acc = fmaf(__expf(ml[2 * c] - M), A.part_o[((int64_t)h * A.gch + c) * HD + d], acc);
    A.out[(int64_t)h * HD + d] = f2h(acc / den);
  }
}

}  // namespace

int launch_rownorm(const float* h_in, float* h_out, const float* a, const float* w1, float scale, const float* w2,
                   uint16_t* x, uint16_t* xlo, int H, float eps, hipStream_t st) {
  if (H <= 0 || H > 256 * kRowMax) return e4b_fail(E4B_EINVAL, "row norm: hidden %d outside 1..%d", H, 256 * kRowMax);
  if (a && !w1) return e4b_fail(E4B_EINVAL, "row norm: residual without its norm weight");
  hipLaunchKernelGGL(k_rownorm, dim3(1), dim3(256), 0, st, h_in, h_out, a, w1, scale, w2, x, xlo, H, eps);
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}

int launch_headprep_gen(const HeadPrepGen& a, hipStream_t st) {
  if ((a.hd != 256 && a.hd != 512) || a.kvh <= 0 || a.qh % a.kvh || a.angles < 0 || a.angles > a.hd / 2 ||
      a.slots <= 0 || (a.window > 0 && a.slots < a.window))
    return e4b_fail(E4B_EINVAL, "head prep: head_dim %d, %d/%d heads, %d pairs, %d slots", a.hd, a.qh, a.kvh,
                    a.angles, a.slots);
  const dim3 grid(a.qh + 2 * a.kvh);
  if (a.hd == 256)
    hipLaunchKernelGGL(k_headprep_gen<256>, grid, dim3(64), 0, st, a);
  else
    hipLaunchKernelGGL(k_headprep_gen<512>, grid, dim3(64), 0, st, a);
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}

int launch_attn_gen(const AttnGen& a, hipStream_t st) {
  if ((a.hd != 256 && a.hd != 512) || a.kvh <= 0 || a.qh % a.kvh || a.slots <= 0 || a.gch <= 0 ||
      (a.window > 0 && a.slots < a.window) || (int64_t)a.gch * kAttnGenChunk < (a.window > 0 ? a.window : a.slots))
    return e4b_fail(E4B_EINVAL, "attention: head_dim %d, %d/%d heads, %d slots, %d chunks", a.hd, a.qh, a.kvh,
                    a.slots, a.gch);
  const dim3 grid(a.qh, a.gch);
  if (a.hd == 256) {
    hipLaunchKernelGGL(k_attn_chunk<256>, grid, dim3(256), 0, st, a);
    hipLaunchKernelGGL(k_attn_merge<256>, dim3(a.qh), dim3(256), 0, st, a);
  } else {
    hipLaunchKernelGGL(k_attn_chunk<512>, grid, dim3(256), 0, st, a);
    hipLaunchKernelGGL(k_attn_merge<512>, dim3(a.qh), dim3(256), 0, st, a);
  }
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}
