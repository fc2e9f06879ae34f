// k_gemv.hip -- Q6_K dequant-GEMV (lm-head + softcap + argmax), Q6_K row
// dequant, argmax and the f32 -> hi/lo f16 split for gfx950 (wave64).  The
// q4_0 GEMV lives in q40_kernel.h.
//
// f32 activations are carried as an f16 pair hi = f16(x), lo = f16(x - hi)
// whose sum is within max(2^-22 |x|, 2^-25) of x (22 of f32's 24 significant
// bits; lo is subnormal below |x| = 2^-3); v_dot2_f32_f16 over both halves
// then accumulates the products in f32.
#include "../../include/e4b.h"
#include "kernels.h"
#include "util.h"
#include "trace.h"

namespace {

constexpr float kTwo24 = 16777216.0f;
constexpr int kQ6Rows = 8;  // lm-head rows per wave tile

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

__global__ __launch_bounds__(256) void k_split_f32(const float* __restrict__ x, int64_t n, uint16_t* __restrict__ hi,
                                                   uint16_t* __restrict__ lo) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) {
    const float v = x[i];
    const _Float16 h = (_Float16)v;
    hi[i] = __builtin_bit_cast(uint16_t, h);
    lo[i] = __builtin_bit_cast(uint16_t, (_Float16)(v - (float)h));
  }
}

// ---- argmax helpers (kernels/argmax2.wgsl semantics: lowest index among the
// maxima, NaN never taken, empty -> (0, -3e38)) --------------------------------
DEV void amax_take(float& bv, uint32_t& bi, float v, uint32_t i) {
  if (v > bv || (v == bv && i < bi)) {
    bv = v;
    bi = i;
  }
}

DEV void amax_wave(float& bv, uint32_t& bi) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(bv, off, 64);
    const uint32_t oi = __shfl_xor(bi, off, 64);
    amax_take(bv, bi, ov, oi);
  }
}

// Block-level argmax partial: reduce the block and store (index, value) to
// part[blockIdx.x] with a plain store.  The fold over blocks runs in
// k_amax_final on the same stream (the kernel boundary makes the partials
// visible); a per-block atomic counter costs ~12-25 ns per block on this part
// because same-address atomics serialise.
DEV void amax_block(float bv, uint32_t bi, uint2* part) {
  __shared__ float sv[4];
  __shared__ uint32_t si[4];
  amax_wave(bv, bi);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    sv[wave] = bv;
    si[wave] = bi;
  }
  lds_sync();
  if (threadIdx.x == 0) {
    float v = sv[0];
    uint32_t i = si[0];
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w) amax_take(v, i, sv[w], si[w]);
    part[blockIdx.x] = make_uint2(i, __float_as_uint(v));
  }
}

__global__ __launch_bounds__(256) void k_amax_final(const uint2* __restrict__ part, int nparts, uint32_t* amax) {
  __shared__ float sv[4];
  __shared__ uint32_t si[4];
  float v = -3.0e38f;
  uint32_t i = 0;
  for (int b = threadIdx.x; b < nparts; b += 256) {
    const uint2 p = part[b];
    amax_take(v, i, __uint_as_float(p.y), p.x);
  }
  amax_wave(v, i);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    sv[wave] = v;
    si[wave] = i;
  }
  lds_sync();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 4; ++w) amax_take(sv[0], si[0], sv[w], si[w]);
    amax[0] = si[0];
    amax[1] = __float_as_uint(sv[0]);
  }
}

// Q6_K GEMV + softcap + argmax.  Lane <-> 32-element segment (s = lane +
// 64k); a wave owns R rows per tile and strides over tiles; after the
// transposed reduction lane l holds row l/(64/R), so the softcap and the
// argmax update run once per R rows.  The workgroup reads x (hi and lo) from
// memory once, into LDS: with one read per wave the x traffic of the grid
// would be 4x its size again.
template <int BPL, int R>
__global__ __launch_bounds__(256) void k_q6k_gemv_argmax(Q6Mat W, const uint32_t* __restrict__ xh,
                                                         const uint32_t* __restrict__ xl, float softcap,
                                                         float* __restrict__ logits, uint2* part,
                                                         int64_t ntiles) {
  E4B_TRACE_SCOPE(trace_tag(TR_LMHEAD, 0));
  constexpr int SPAN = 64 / R;
  constexpr int XW = BPL * 64 * 16;  // 32-bit words of x (hi or lo) the block can hold
  __shared__ __align__(16) uint32_t xs[2][XW];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nseg = W.nseg, nsb = nseg / 8;
  {
    const int nw = nseg * 16;  // words of x
    for (int i = 4 * (int)threadIdx.x; i < nw; i += 4 * 256) {
      *reinterpret_cast<uint4*>(&xs[0][i]) = *reinterpret_cast<const uint4*>(xh + i);
      *reinterpret_cast<uint4*>(&xs[1][i]) = *reinterpret_cast<const uint4*>(xl + i);
    }
    lds_sync();
  }
  uint32_t xph[BPL][16], xpl[BPL][16];
  float gs[BPL][2];
#pragma unroll
  for (int k = 0; k < BPL; ++k) {
    const int s = lane + 64 * k;
    gs[k][0] = gs[k][1] = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) xph[k][i] = xpl[k][i] = 0u;  // lanes past the row end contribute 0
    if (s < nseg) {
      load_x16(xs[0], s, xph[k]);
      load_x16(xs[1], s, xpl[k]);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        gs[k][0] = fdot2u(xph[k][i], 0x3C003C00u, gs[k][0]);
        gs[k][0] = fdot2u(xpl[k][i], 0x3C003C00u, gs[k][0]);
        gs[k][1] = fdot2u(xph[k][8 + i], 0x3C003C00u, gs[k][1]);
        gs[k][1] = fdot2u(xpl[k][8 + i], 0x3C003C00u, gs[k][1]);
      }
      gs[k][0] *= -32.f;
      gs[k][1] *= -32.f;
    }
  }
  float bv = -3.0e38f;
  uint32_t bi = 0;
  for (int64_t tile = (int64_t)blockIdx.x * 4 + wave; tile < ntiles; tile += (int64_t)gridDim.x * 4) {
    const int64_t row0 = tile * R;
    const uint4* qa = W.qa + row0 * nseg;
    const uint2* qb = W.qb + row0 * nseg;
    const uint16_t* sc16 = reinterpret_cast<const uint16_t*>(W.sc);  // int8 scale pairs, one per segment
    uint4 a[R][BPL];
    uint2 b[R][BPL];
    // 16-bit scale pairs and f16 d loaded as aligned 32-bit pairs (see
    // ld_scale_pair): no early wait on the rows' other loads
    uint32_t s2[R][BPL], dh[R][BPL];
    uint32_t sodd = 0, dodd = 0;
    const int rlast = (int)min((int64_t)R - 1, W.rows - 1 - row0);  // clamp the tail tile
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
      for (int k = 0; k < BPL; ++k) {
        const int s = min(lane + 64 * k, nseg - 1);  // x is zero past the row end
        const uint32_t o = (uint32_t)(min(r, rlast) * nseg + s);
        const int64_t es = row0 * nseg + o;
        const int64_t ed = (row0 + min(r, rlast)) * nsb + (s >> 3);
        a[r][k] = ld_nt_u4(qa + o);
        b[r][k] = ld_nt_u2(qb + o);
        s2[r][k] = ld_scale_pair(sc16, es);
        dh[r][k] = ld_scale_pair(W.d, ed);
        sodd |= (uint32_t)(es & 1) << (r * BPL + k);
        dodd |= (uint32_t)(ed & 1) << (r * BPL + k);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      acc[r] = 0.f;
#pragma unroll
      for (int k = 0; k < BPL; ++k) {
        uint32_t p[8];
        q6_pairs(a[r][k].x, a[r][k].y, b[r][k].x, p);
        float a0 = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          a0 = fdot2u(p[i], xph[k][i], a0);
          a0 = fdot2u(p[i], xpl[k][i], a0);
        }
        q6_pairs(a[r][k].z, a[r][k].w, b[r][k].y, p);
        float a1 = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          a1 = fdot2u(p[i], xph[k][8 + i], a1);
          a1 = fdot2u(p[i], xpl[k][8 + i], a1);
        }
        const uint32_t sp = s2[r][k] >> (((sodd >> (r * BPL + k)) & 1) * 16);
        const float s0 = (float)(int8_t)(sp & 0xff), s1 = (float)(int8_t)((sp >> 8) & 0xff);
        const float t = s0 * fmaf(a0, kTwo24, gs[k][0]) + s1 * fmaf(a1, kTwo24, gs[k][1]);
        acc[r] = fmaf(scale_of(dh[r][k], (dodd >> (r * BPL + k)) & 1), t, acc[r]);
      }
    }
    float v = reduce_rows<64, R>(acc);
    const int64_t row = row0 + lane / SPAN;
    if (softcap != 0.f) v = softcap * tanhf(v / softcap);
    if (row < W.rows) {
      if (logits && (lane % SPAN) == 0) logits[row] = v;
      amax_take(bv, bi, v, (uint32_t)row);
    }
  }
  amax_block(bv, bi, part);
}

// one Q6_K row * mult -> f32 (kernels/q6k.wgsl:37-73); thread per segment
__global__ __launch_bounds__(256) void k_q6k_row(Q6Mat W, int64_t row, const uint32_t* __restrict__ row_dev,
                                                 float mult, float* __restrict__ out) {
  const int s = blockIdx.x * 256 + threadIdx.x;
  if (s >= W.nseg) return;
  const int64_t r = row_dev ? (int64_t)row_dev[0] : row;
  if (r < 0 || r >= W.rows) return;
  const uint4 a = W.qa[r * W.nseg + s];
  const uint2 b = W.qb[r * W.nseg + s];
  const float d = h2f(W.d[r * (W.nseg / 8) + (s >> 3)]);
  const int8_t* sc = W.sc + r * (W.nseg * 2) + 2 * s;
  uint32_t p[8];
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    q6_pairs(g ? a.z : a.x, g ? a.w : a.y, g ? b.y : b.x, p);
    const float ds = d * (float)sc[g];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      out[32 * s + 16 * g + 2 * i] = ds * (float)((int)(p[i] & 0x3f) - 32) * mult;
      out[32 * s + 16 * g + 2 * i + 1] = ds * (float)((int)((p[i] >> 16) & 0x3f) - 32) * mult;
    }
  }
}

__global__ __launch_bounds__(256) void k_argmax(const float* __restrict__ x, int64_t n, uint2* part) {
  float bv = -3.0e38f;
  uint32_t bi = 0;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    amax_take(bv, bi, x[i], (uint32_t)i);
  amax_block(bv, bi, part);
}

}  // namespace

int launch_split_f32(const float* x, int64_t n, uint16_t* hi, uint16_t* lo, hipStream_t st) {
  hipLaunchKernelGGL(k_split_f32, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, n, hi, lo);
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}

// rows per wave tile: kQ6Rows with one segment per lane (<= 2048 columns);
// a quarter as many with two (each row then takes 8 loads per lane: the 63 a
// wave can keep in flight are not exceeded, and the 2816-column A4B lm-head
// measured 177 us with 8 rows, 127 with 4, 124 with 2)
static int q6k_rows(int nseg) { return nseg <= 64 ? kQ6Rows : kQ6Rows / 4; }

int q6k_gemv_grid(int64_t rows, int nseg) {
  const int R = q6k_rows(nseg);
  const int64_t ntiles = (rows + R - 1) / R;
  const int64_t wgs = (ntiles + 3) / 4;
  return (int)(wgs < 2048 ? wgs : 2048);
}

int launch_q6k_gemv_argmax(const Q6Mat& W, const uint32_t* xh, const uint32_t* xl, float softcap, float* logits,
                           uint32_t* amax, uint2* part, hipStream_t st) {
  const int R = q6k_rows(W.nseg);
  const int64_t ntiles = (W.rows + R - 1) / R;
  const int64_t wgs = q6k_gemv_grid(W.rows, W.nseg);
  if (W.nseg <= 64)
    hipLaunchKernelGGL((k_q6k_gemv_argmax<1, kQ6Rows>), dim3((unsigned)wgs), dim3(256), 0, st, W, xh, xl, softcap,
                       logits, part, ntiles);
  else if (W.nseg <= 128)
    hipLaunchKernelGGL((k_q6k_gemv_argmax<2, kQ6Rows / 4>), dim3((unsigned)wgs), dim3(256), 0, st, W, xh, xl, softcap,
                       logits, part, ntiles);
  else
    return e4b_fail(E4B_EINVAL, "Q6_K GEMV: %d columns exceeds the 4096-column maximum", W.nseg * 32);
  if (amax) hipLaunchKernelGGL(k_amax_final, dim3(1), dim3(256), 0, st, part, (int)wgs, amax);
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}

int launch_q6k_row(const Q6Mat& W, int64_t row, const uint32_t* row_dev, float mult, float* out, hipStream_t st) {
  hipLaunchKernelGGL(k_q6k_row, dim3((unsigned)((W.nseg + 255) / 256)), dim3(256), 0, st, W, row, row_dev, mult, out);
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}

int launch_argmax(const float* x, int64_t n, uint32_t* amax, uint2* part, hipStream_t st) {
  const int64_t want = (n + 255) / 256;
  const unsigned grid = (unsigned)(want < 1024 ? (want > 0 ? want : 1) : 1024);
  hipLaunchKernelGGL(k_argmax, dim3(grid), dim3(256), 0, st, x, n, part);
  hipLaunchKernelGGL(k_amax_final, dim3(1), dim3(256), 0, st, part, (int)grid, amax);
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}
