// common.h -- shared host/device definitions for libe4b (gfx950 / MI355X).
//
// Packed weight layouts (built on the host by pack.cpp, read by the kernels):
//
// q4_0 matrix [rows][cols], nb = cols/32 blocks per row:
//   nibble plane  rows*nb uint4 (16 B per block)      at offset 0
//   scale plane   rows*nb f16 (the block's d)          at offset align256(rows*nb*16)
//   Inside a block the 32 nibbles are re-ordered so that dword k (k = 0..3)
//   holds elements 8k..8k+7 with element 8k+2i in bits [8*i' ...] such that
//       (w >> s_i) & 0x000F000F  ==  (n[8k+2i], n[8k+2i+1])  as two u16 halves,
//   s_0 = 0, s_1 = 8, s_2 = 4, s_3 = 12.  A half holding n (0..15) is the f16
//   subnormal n * 2^-24, so v_dot2_f32_f16 against the natural f16 pair
//   (x[2j], x[2j+1]) yields 2^-24 * (n0 x0 + n1 x1) exactly; the -8 offset is
//   folded as d * (2^24 * acc - 8 * sum(x_block)).
//
// Q6_K matrix [rows][cols], cols % 256 == 0; a 32-element "segment" s covers
// scale groups 2s and 2s+1 (a ggml Q6_K scale group is 16 contiguous elements):
//   qa plane  rows*nseg uint4  = (g0.w0, g0.w1, g1.w0, g1.w1)
//   qb plane  rows*nseg uint2  = (g0.w2, g1.w2)
//   sc plane  rows*ngrp int8   (ggml per-group scale, group order)
//   d  plane  rows*nsb  f16    (ggml superblock d)
//   Group words hold the 6-bit values q0..q15 of one group as u16-half pairs:
//     w0: (q0,q1)@[0:5|16:21] (q2,q3)@[6:11|22:27] low nibbles of (q4,q5)@[12:15|28:31]
//     w1: (q6,q7)            (q8,q9)              low nibbles of (q10,q11)
//     w2: (q12,q13)          (q14,q15)            hi bits q4@[12:13] q5@[28:29]
//                                                  hi bits q10@[14:15] q11@[30:31]
#pragma once
#include <stdint.h>
#include <stddef.h>

#define E4B_ALIGN256(x) ((((size_t)(x)) + 255u) & ~(size_t)255u)

static inline size_t q40_nib_bytes(int64_t rows, int64_t cols) {
  return (size_t)rows * (size_t)(cols / 32) * 16u;
}
static inline size_t q40_packed_bytes(int64_t rows, int64_t cols) {
  return E4B_ALIGN256(q40_nib_bytes(rows, cols)) + E4B_ALIGN256((size_t)rows * (size_t)(cols / 32) * 2u);
}

struct Q6Planes {
  size_t qa, qb, sc, d, total;
};
static inline Q6Planes q6k_planes(int64_t rows, int64_t cols) {
  Q6Planes p;
  size_t nseg = (size_t)(cols / 32), ngrp = (size_t)(cols / 16), nsb = (size_t)(cols / 256);
  p.qa = 0;
  p.qb = E4B_ALIGN256((size_t)rows * nseg * 16u);
  p.sc = p.qb + E4B_ALIGN256((size_t)rows * nseg * 8u);
  p.d = p.sc + E4B_ALIGN256((size_t)rows * ngrp);
  p.total = p.d + E4B_ALIGN256((size_t)rows * nsb * 2u);
  return p;
}

#ifdef __HIPCC__
#include <hip/hip_runtime.h>

typedef _Float16 e4b_h2 __attribute__((ext_vector_type(2)));

#define DEV __device__ __forceinline__

// acc + a.lo*b.lo + a.hi*b.hi with f16 inputs, f32 accumulate (v_dot2_f32_f16)
DEV float fdot2u(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(e4b_h2, a), __builtin_bit_cast(e4b_h2, b), c, false);
}

DEV float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
DEV uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

// sum of the 32 f16 values of one q4_0 x block (16 packed pairs)
DEV float xsum16(const uint32_t* xp) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) s = fdot2u(xp[i], 0x3C003C00u, s);
  return s;
}

// Two-accumulator form of q40_dot: the pairs at bits 0-3 of each half go to
// a0 (value n * 2^-24), the pairs at bits 4-7 are used in place (value
// 16 n * 2^-24) and go to a1, so a word costs 4 masks and 1 shift instead of
// 4 masks and 3 shifts.  2^-24 sum n_i x_i = a0 + a1 / 16.
DEV void q40_dot2(uint4 w, const uint32_t* xp, float& a0, float& a1) {
  const uint32_t M = 0x000F000Fu, M4 = 0x00F000F0u;
  const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t v = ws[k], v8 = ws[k] >> 8;
    a0 = fdot2u(v & M, xp[4 * k + 0], a0);
    a1 = fdot2u(v & M4, xp[4 * k + 2], a1);
    a0 = fdot2u(v8 & M, xp[4 * k + 1], a0);
    a1 = fdot2u(v8 & M4, xp[4 * k + 3], a1);
  }
}

// 2^-24 * sum n_i x_i over one repacked q4_0 block
DEV float q40_dot(uint4 w, const uint32_t* xp, float acc) {
  const uint32_t M = 0x000F000Fu;
  const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t v = ws[k];
    acc = fdot2u(v & M, xp[4 * k + 0], acc);
    acc = fdot2u((v >> 8) & M, xp[4 * k + 1], acc);
    acc = fdot2u((v >> 4) & M, xp[4 * k + 2], acc);
    acc = fdot2u((v >> 12) & M, xp[4 * k + 3], acc);
  }
  return acc;
}

// the 8 (q_2i, q_2i+1) subnormal-f16 pairs of one packed Q6_K group
DEV void q6_pairs(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t* p) {
  const uint32_t M6 = 0x003F003Fu, M4 = 0x000F000Fu, MH = 0x00300030u;
  p[0] = w0 & M6;
  p[1] = (w0 >> 6) & M6;
  p[2] = ((w0 >> 12) & M4) | ((w2 >> 8) & MH);
  p[3] = w1 & M6;
  p[4] = (w1 >> 6) & M6;
  p[5] = ((w1 >> 12) & M4) | ((w2 >> 10) & MH);
  p[6] = w2 & M6;
  p[7] = (w2 >> 6) & M6;
}

template <typename T>
DEV T wave_shfl_xor(T v, int m) {
  return __shfl_xor(v, m, 64);
}

DEV float group_sum(float v, int lpr) {
  for (int off = lpr >> 1; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// ---- cross-lane exchange (wave64) -------------------------------------------
// swapx32(a, b): lanes [32,64) of a <-> lanes [0,32) of b (v_permlane32_swap);
// swapx16(a, b): odd 16-lane rows of a <-> even rows of b (v_permlane16_swap).
// After either, a + b on every lane is "my own value of the half I keep plus
// my partner's value of the same half", i.e. one transposed-butterfly step.
DEV void swapx32(float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}
DEV void swapx16(float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}
// value of lane (l ^ m) for m in {1, 2, 4, 8}
template <int M>
DEV float lane_xor(float v) {
  static_assert(M == 1 || M == 2 || M == 4 || M == 8, "lane_xor: 1, 2, 4 or 8");
  const int iv = __float_as_int(v);
  if constexpr (M == 1) return __int_as_float(__builtin_amdgcn_mov_dpp(iv, 0xB1, 0xF, 0xF, true));
  if constexpr (M == 2) return __int_as_float(__builtin_amdgcn_mov_dpp(iv, 0x4E, 0xF, 0xF, true));
  if constexpr (M == 4) return __int_as_float(__builtin_amdgcn_ds_swizzle(iv, 0x101F));
  if constexpr (M == 8) return __int_as_float(__builtin_amdgcn_ds_swizzle(iv, 0x201F));
  return v;
}

// One transposed step with lane-distance M on the pair (lo, hi): lanes whose
// bit M is clear keep the `lo` row, the others keep `hi`; the result is the
// kept row's partial summed over the lane pair.
template <int M>
DEV float tstep(float lo, float hi) {
  if constexpr (M == 32) {
    swapx32(lo, hi);
    return lo + hi;
  } else if constexpr (M == 16) {
    swapx16(lo, hi);
    return lo + hi;
  } else {
    const float plo = lane_xor<M>(lo), phi = lane_xor<M>(hi);
    const bool up = (threadIdx.x & M) != 0;
    return up ? hi + phi : lo + plo;
  }
}
template <int M>
DEV float xsum_step(float s) {
  if constexpr (M == 32) {
    float t = s;
    swapx32(s, t);
    return s + t;
  } else if constexpr (M == 16) {
    float t = s;
    swapx16(s, t);
    return s + t;
  } else {
    return s + lane_xor<M>(s);
  }
}

template <int LPR, int R, int N>
struct RowReduce {
  // N partials remain, next step distance M = LPR * N / (2 R)
  static DEV float run(float* v) {
    constexpr int M = LPR * N / (2 * R);
#pragma unroll
    for (int i = 0; i < N / 2; ++i) v[i] = tstep<M>(v[i], v[N / 2 + i]);
    return RowReduce<LPR, R, N / 2>::run(v);
  }
};
template <int LPR, int R>
struct RowReduce<LPR, R, 1> {
  template <int M>
  static DEV float tail(float s) {
    if constexpr (M == 0) {
      return s;
    } else {
      return tail<M / 2>(xsum_step<M>(s));
    }
  }
  static DEV float run(float* v) { return tail<LPR / (2 * R)>(v[0]); }
};

// Transposed butterfly inside LPR-lane groups: lane l of a group holds
// partials v[0..R) of R rows; on return it holds the group total of row
// l / (LPR/R).  R-1 exchanges + log2(LPR/R) reduction steps instead of
// R*log2(LPR) shuffles.  R <= LPR, powers of two.
template <int LPR, int R>
DEV float reduce_rows(float (&v)[R]) {
  static_assert(R <= LPR && (R & (R - 1)) == 0 && (LPR & (LPR - 1)) == 0, "powers of two, R <= LPR");
  return RowReduce<LPR, R, R>::run(v);
}

// ---- block-level helpers (256 threads = 4 waves) --------------------------------
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
// Workgroup barrier that orders LDS only.  __syncthreads() also waits for
// every outstanding global load of the wave (a workgroup-scope fence over all
// address spaces), which would stall a kernel on its whole in-flight weight
// stream; barriers that only publish LDS data use this one.
DEV void lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// sum over a 256-thread block; every thread gets the total.  `red` = 4 floats of LDS.
DEV float block_sum(float v, float* red) {
  v = wave_sum(v);
  lds_sync();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  lds_sync();
  return (red[0] + red[1]) + (red[2] + red[3]);
}
DEV float block_max(float v, float* red) {
  v = wave_max(v);
  lds_sync();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  lds_sync();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}
// RMSNorm scale (mean(x^2) + eps)^-1/2 from a sum of squares
DEV float rms_inv(float ss, int n, float eps) { return 1.0f / sqrtf(ss / (float)n + eps); }
// gelu_pytorch_tanh with the tanh argument clamped to +-20 (kernels/q40gu.wgsl:114)
DEV float gelu_tanh(float g) {
  float t = 0.7978845608028654f * (g + 0.044715f * g * g * g);
  t = fminf(fmaxf(t, -20.f), 20.f);
  return 0.5f * g * (1.f + tanhf(t));
}

// non-temporal 16 B load for streamed weights (read once per token)
typedef uint32_t e4b_u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t e4b_u32x2 __attribute__((ext_vector_type(2)));
DEV uint4 ld_nt_u4(const uint4* p) {
  const e4b_u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const e4b_u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
DEV uint2 ld_nt_u2(const uint2* p) {
  const e4b_u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const e4b_u32x2*>(p));
  return make_uint2(v.x, v.y);
}
DEV uint16_t ld_nt_u16(const uint16_t* p) { return __builtin_nontemporal_load(p); }
DEV uint32_t ld_nt_u32(const uint32_t* p) { return __builtin_nontemporal_load(p); }

// f16 block scale e (= row * nb + block) of a q4_0 scale plane, loaded as the
// aligned 32-bit pair that holds it (the plane is padded to 256 bytes, so the
// pair is always inside it).  A 16-bit load would let the compiler pack two
// scales into one register right after the loads, which forces a wait on
// every load issued before them; the half is selected when it is used.
DEV uint32_t ld_scale_pair(const uint16_t* sc, int64_t e) {
  return ld_nt_u32(reinterpret_cast<const uint32_t*>(sc) + (e >> 1));
}
DEV float scale_of(uint32_t pair, uint32_t odd) { return h2f((uint16_t)(pair >> (odd * 16))); }

// The same loads at a 32-bit offset from a uniform base: the compiler keeps
// the base in scalar registers and spends one VGPR per address instead of
// two, which keeps the whole tile's loads in flight without register reuse
// (callers check that the plane is below 4 GiB).
DEV uint4 ld_nt_u4_off(const uint4* base, uint32_t block) {
  return ld_nt_u4(reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(base) + block * 16u));
}
DEV uint32_t ld_scale_pair_off(const uint16_t* sc, uint32_t e) {
  return ld_nt_u32(reinterpret_cast<const uint32_t*>(reinterpret_cast<const char*>(sc) + (e >> 1) * 4u));
}

#endif  // __HIPCC__
