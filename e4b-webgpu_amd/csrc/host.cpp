// host.cpp -- host-side parts of libe4b: weight repacking (ggml blocks to the
// device layouts described in common.h) and the seeded synthetic generators.
// Plain C++17 + OpenMP; no device code.
#include <math.h>
#include <string.h>

#include <algorithm>
#include <vector>

#include "../../include/e4b.h"
#include "common.h"
#include "util.h"

// ---------------------------------------------------------------------------
// q4_0 repack.  Replaces repackQ40 (src/engine-a4b.js:29-39): the nibble and
// scale planes are split as there, and in addition the 32 nibbles of a block
// are re-ordered for the v_dot2 pairing described in common.h.
// ---------------------------------------------------------------------------
static const int kQ40Shift[8] = {0, 16, 8, 24, 4, 20, 12, 28};

static inline uint32_t ggml_q40_nibble(const uint8_t* qs, int e) {
  return e < 16 ? (qs[e] & 15u) : (qs[e - 16] >> 4);
}

extern "C" size_t e4b_q40_packed_bytes(int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0 || cols % 32) return 0;
  return q40_packed_bytes(rows, cols);
}

extern "C" int e4b_q40_pack(const void* ggml, int64_t rows, int64_t cols, void* packed) {
  if (!ggml || !packed || rows <= 0 || cols <= 0 || cols % 32)
    return e4b_fail(E4B_EINVAL, "e4b_q40_pack: bad arguments (rows=%lld cols=%lld)", (long long)rows,
                    (long long)cols);
  const int64_t nblk = rows * (cols / 32);
  const uint8_t* src = (const uint8_t*)ggml;
  uint32_t* nib = (uint32_t*)packed;
  uint16_t* sc = (uint16_t*)((uint8_t*)packed + E4B_ALIGN256(q40_nib_bytes(rows, cols)));
#pragma omp parallel for schedule(static)
  for (int64_t b = 0; b < nblk; ++b) {
    const uint8_t* p = src + b * 18;
    sc[b] = (uint16_t)(p[0] | (p[1] << 8));
    const uint8_t* qs = p + 2;
    for (int k = 0; k < 4; ++k) {
      uint32_t w = 0;
      for (int t = 0; t < 8; ++t) w |= ggml_q40_nibble(qs, 8 * k + t) << kQ40Shift[t];
      nib[b * 4 + k] = w;
    }
  }
  return E4B_OK;
}

// ---------------------------------------------------------------------------
// Q6_K repack.  Replaces repackQ6K (src/engine-a4b.js:43-73).  Element order
// and the (q - 32) * sc * d value follow ggml's Q6_K superblock as the
// reference decodes it (kernels/q6k.wgsl:44-71).
// ---------------------------------------------------------------------------
static inline int ggml_q6_val(const uint8_t* blk, int e) {
  const int half = e >> 7, r = e & 127, quad = r >> 5, l = r & 31;
  const uint8_t* ql = blk + 64 * half;
  const uint8_t* qh = blk + 128 + 32 * half;
  int lo = (quad & 1) ? ql[l + 32] : ql[l];
  lo = (quad >= 2) ? (lo >> 4) : (lo & 15);
  const int hi = (qh[l] >> (2 * quad)) & 3;
  return lo | (hi << 4);
}

extern "C" size_t e4b_q6k_packed_bytes(int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0 || cols % 256) return 0;
  return q6k_planes(rows, cols).total;
}

extern "C" int e4b_q6k_pack(const void* ggml, int64_t rows, int64_t cols, void* packed) {
  if (!ggml || !packed || rows <= 0 || cols <= 0 || cols % 256)
    return e4b_fail(E4B_EINVAL, "e4b_q6k_pack: bad arguments (rows=%lld cols=%lld)", (long long)rows,
                    (long long)cols);
  const Q6Planes P = q6k_planes(rows, cols);
  const int64_t nsb = cols / 256, nseg = cols / 32, ngrp = cols / 16;
  uint8_t* base = (uint8_t*)packed;
  uint32_t* qa = (uint32_t*)(base + P.qa);
  uint32_t* qb = (uint32_t*)(base + P.qb);
  int8_t* sc = (int8_t*)(base + P.sc);
  uint16_t* dd = (uint16_t*)(base + P.d);
  const uint8_t* src = (const uint8_t*)ggml;
#pragma omp parallel for schedule(static)
  for (int64_t o = 0; o < rows; ++o) {
    for (int64_t b = 0; b < nsb; ++b) {
      const uint8_t* blk = src + (o * nsb + b) * 210;
      dd[o * nsb + b] = (uint16_t)(blk[208] | (blk[209] << 8));
      for (int j = 0; j < 16; ++j) {
        const int64_t G = b * 16 + j;  // row-level group index
        sc[o * ngrp + G] = (int8_t)blk[192 + j];
        int q[16];
        for (int i = 0; i < 16; ++i) q[i] = ggml_q6_val(blk, 16 * j + i);
        const uint32_t w0 = (uint32_t)q[0] | (uint32_t)q[2] << 6 | (uint32_t)(q[4] & 15) << 12 |
                            (uint32_t)q[1] << 16 | (uint32_t)q[3] << 22 | (uint32_t)(q[5] & 15) << 28;
        const uint32_t w1 = (uint32_t)q[6] | (uint32_t)q[8] << 6 | (uint32_t)(q[10] & 15) << 12 |
                            (uint32_t)q[7] << 16 | (uint32_t)q[9] << 22 | (uint32_t)(q[11] & 15) << 28;
        const uint32_t w2 = (uint32_t)q[12] | (uint32_t)q[14] << 6 | (uint32_t)(q[4] >> 4) << 12 |
                            (uint32_t)(q[10] >> 4) << 14 | (uint32_t)q[13] << 16 | (uint32_t)q[15] << 22 |
                            (uint32_t)(q[5] >> 4) << 28 | (uint32_t)(q[11] >> 4) << 30;
        const int64_t s = G >> 1, g = G & 1;
        qa[(o * nseg + s) * 4 + 2 * g + 0] = w0;
        qa[(o * nseg + s) * 4 + 2 * g + 1] = w1;
        qb[(o * nseg + s) * 2 + g] = w2;
      }
    }
  }
  return E4B_OK;
}

// ---------------------------------------------------------------------------
// Seeded synthetic data: element i of stream `seed` is the (i+1)-th output of
// splitmix64 started at `seed`, i.e. mix64(seed + (i+1) * golden), so any
// element is computable independently (and identically from C, Python or JS).
// ---------------------------------------------------------------------------
static inline uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
  return z ^ (z >> 31);
}
extern "C" uint64_t e4b_synth_u64(uint64_t seed, uint64_t index) {
  return mix64(seed + (index + 1) * 0x9e3779b97f4a7c15ULL);
}
static inline uint64_t substream(uint64_t seed, uint64_t tag) { return mix64(seed ^ (tag * 0x9e3779b97f4a7c15ULL)); }

// Box-Muller (cosine branch) on u64 pairs (2i, 2i+1)
static inline double synth_normal(uint64_t seed, uint64_t i) {
  const double u1 = ((double)(e4b_synth_u64(seed, 2 * i) >> 11) + 0.5) * (1.0 / 9007199254740992.0);
  const double u2 = (double)(e4b_synth_u64(seed, 2 * i + 1) >> 11) * (1.0 / 9007199254740992.0);
  return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

static inline uint16_t f32_to_f16_rne(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
  if (ax < 0x38800000u) {
    float a;
    memcpy(&a, &ax, 4);
    const double q = (double)a * 16777216.0, fl = floor(q), r = q - fl;
    uint32_t m = (uint32_t)fl;
    if (r > 0.5 || (r == 0.5 && (m & 1u))) m++;
    return (uint16_t)(sign | m);
  }
  uint32_t h = (((ax >> 23) - 112u) << 10) | ((ax >> 13) & 0x3ffu);
  const uint32_t rest = ax & 0x1fffu;
  if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h++;
  return (uint16_t)(sign | h);
}

extern "C" int e4b_synth_normal_f32(uint64_t seed, int64_t n, float mean, float stdv, float* out) {
  if (n < 0 || (n && !out)) return e4b_fail(E4B_EINVAL, "e4b_synth_normal_f32: bad arguments");
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) out[i] = (float)((double)mean + (double)stdv * synth_normal(seed, (uint64_t)i));
  return E4B_OK;
}

extern "C" int e4b_synth_uniform_u32(uint64_t seed, int64_t n, uint32_t lo, uint32_t hi, uint32_t* out) {
  if (n < 0 || (n && !out) || hi <= lo) return e4b_fail(E4B_EINVAL, "e4b_synth_uniform_u32: bad arguments");
  const uint64_t span = (uint64_t)hi - lo;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i)
    out[i] = lo + (uint32_t)(((e4b_synth_u64(seed, (uint64_t)i) >> 32) * span) >> 32);
  return E4B_OK;
}

extern "C" int e4b_synth_q40(uint64_t seed, int64_t rows, int64_t cols, float sigma, void* out) {
  if (!out || rows <= 0 || cols <= 0 || cols % 32) return e4b_fail(E4B_EINVAL, "e4b_synth_q40: bad arguments");
  const uint64_t sA = substream(seed, 1), sB = substream(seed, 2);
  const int64_t nblk = rows * (cols / 32);
  uint8_t* dst = (uint8_t*)out;
#pragma omp parallel for schedule(static)
  for (int64_t b = 0; b < nblk; ++b) {
    uint8_t* p = dst + b * 18;
    const uint16_t d = f32_to_f16_rne((float)(fabs((double)sigma * synth_normal(sA, (uint64_t)b)) / 8.0));
    p[0] = (uint8_t)(d & 0xff);
    p[1] = (uint8_t)(d >> 8);
    const uint64_t r0 = e4b_synth_u64(sB, 2 * (uint64_t)b), r1 = e4b_synth_u64(sB, 2 * (uint64_t)b + 1);
    for (int j = 0; j < 8; ++j) {
      p[2 + j] = (uint8_t)(r0 >> (8 * j));
      p[10 + j] = (uint8_t)(r1 >> (8 * j));
    }
  }
  return E4B_OK;
}

extern "C" int e4b_synth_q6k(uint64_t seed, int64_t rows, int64_t cols, float sigma, void* out) {
  if (!out || rows <= 0 || cols <= 0 || cols % 256) return e4b_fail(E4B_EINVAL, "e4b_synth_q6k: bad arguments");
  const uint64_t sA = substream(seed, 1), sB = substream(seed, 2), sC = substream(seed, 3);
  const int64_t nblk = rows * (cols / 256);
  uint8_t* dst = (uint8_t*)out;
#pragma omp parallel for schedule(static)
  for (int64_t b = 0; b < nblk; ++b) {
    uint8_t* p = dst + b * 210;
    for (int u = 0; u < 24; ++u) {  // ql[128] + qh[64]: any bits are valid 6-bit quants
      const uint64_t r = e4b_synth_u64(sB, 24 * (uint64_t)b + u);
      for (int j = 0; j < 8; ++j) p[8 * u + j] = (uint8_t)(r >> (8 * j));
    }
    for (int u = 0; u < 2; ++u) {  // 16 int8 scales ~ U{-32..31}
      const uint64_t r = e4b_synth_u64(sC, 2 * (uint64_t)b + u);
      for (int j = 0; j < 8; ++j) p[192 + 8 * u + j] = (uint8_t)(int8_t)((int)((r >> (8 * j)) & 63) - 32);
    }
    const uint16_t d = f32_to_f16_rne((float)fabs((double)sigma * synth_normal(sA, (uint64_t)b)));
    p[208] = (uint8_t)(d & 0xff);
    p[209] = (uint8_t)(d >> 8);
  }
  return E4B_OK;
}

// ---------------------------------------------------------------------------
// RoPE table (the inverse-frequency uniform of kernels/headprep.wgsl)
// ---------------------------------------------------------------------------
void rope_inv_freq(float theta, int head_dim, int angles, float* out) {
  for (int p = 0; p < angles; ++p) out[p] = (float)pow((double)theta, -2.0 * (double)p / (double)head_dim);
}

// ---------------------------------------------------------------------------
// compactAll's selection (src/engine-a4b.js:590-603) for one full layer:
// mass[t] = sum over heads of score[h][t] in f64, head order; the candidates
// [0, n - prot) by decreasing mass, equal masses in slot order (the stable
// Array.prototype.sort of an ascending list); the first budget - prot of them
// plus the prot = min(protect, n) newest slots, ascending.
// ---------------------------------------------------------------------------
extern "C" int64_t e4b_kv_select(const float* score, int q_heads, int64_t stride, int64_t n, int budget, int protect,
                                 uint32_t* keep_out) {
  if (!score || !keep_out || q_heads < 1 || n < 0 || stride < n || budget < 0 || protect < 0)
    return e4b_fail(E4B_EINVAL, "e4b_kv_select: bad arguments");
  std::vector<double> mass((size_t)std::max<int64_t>(n, 1), 0.0);
  for (int h = 0; h < q_heads; ++h)
    for (int64_t t = 0; t < n; ++t) mass[(size_t)t] += (double)score[(size_t)h * (size_t)stride + (size_t)t];
  const int64_t prot = std::min<int64_t>(protect, n), nc = n - prot;
  const int64_t want = std::max<int64_t>(0, std::min<int64_t>(budget - prot, nc));
  std::vector<uint32_t> cand((size_t)nc);
  for (int64_t t = 0; t < nc; ++t) cand[(size_t)t] = (uint32_t)t;
  std::stable_sort(cand.begin(), cand.end(), [&](uint32_t a, uint32_t b) { return mass[a] > mass[b]; });
  std::vector<uint32_t> keep(cand.begin(), cand.begin() + want);
  for (int64_t t = nc; t < n; ++t) keep.push_back((uint32_t)t);
  std::sort(keep.begin(), keep.end());
  std::copy(keep.begin(), keep.end(), keep_out);
  return (int64_t)keep.size();
}
