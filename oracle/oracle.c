/*
 * oracle.c -- CPU restatement of the reference's batch-1 decode step.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h).  Plain C99 + OpenMP; no GPU code,
 * no dependency on the product library.  Each function cites the reference
 * file:line whose semantics it restates.  Sums are carried in double and
 * rounded where the reference stores f32/f16.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* IEEE binary16 <-> binary32 (textbook; round-to-nearest-even)             */
/* ------------------------------------------------------------------------ */
float orc_h2f(uint16_t h) {
  uint32_t s = (uint32_t)(h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  uint32_t bits;
  if (e == 0) {
    if (m == 0) {
      bits = s;
    } else { /* subnormal: value = m * 2^-24 */
      float v = (float)m * 5.9604644775390625e-08f;
      memcpy(&bits, &v, 4);
      bits |= s;
    }
  } else if (e == 31) {
    bits = s | 0x7f800000u | (m << 13);
  } else {
    bits = s | ((e + 112u) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

uint16_t orc_f2h(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) /* inf / nan */
    return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
  if (ax >= 0x477ff000u) /* >= 65520 rounds to inf */
    return (uint16_t)(sign | 0x7c00u);
  if (ax < 0x38800000u) { /* below the smallest normal half: subnormal or 0 */
    /* value / 2^-24, rounded to nearest even integer */
    float a;
    memcpy(&a, &ax, 4);
    double q = (double)a * 16777216.0;
    double fl = floor(q);
    double r = q - fl;
    uint32_t m = (uint32_t)fl;
    if (r > 0.5 || (r == 0.5 && (m & 1u))) m++;
    return (uint16_t)(sign | m); /* m == 1024 becomes the smallest normal */
  }
  uint32_t e = ((ax >> 23) - 112u) << 10;
  uint32_t m = (ax >> 13) & 0x3ffu;
  uint32_t rest = ax & 0x1fffu;
  uint32_t h = e | m;
  if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h++;
  return (uint16_t)(sign | h);
}

void orc_h2f_n(const uint16_t* h, int64_t n, float* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = orc_h2f(h[i]);
}
void orc_f2h_n(const float* f, int64_t n, uint16_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = orc_f2h(f[i]);
}

static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* ------------------------------------------------------------------------ */
/* q4_0: 18 B = f16 d, qs[16]; element j = (qs[j] & 15) - 8, element j+16 =  */
/* (qs[j] >> 4) - 8, value * d.  Follows kernels/q40mv.wgsl:22-29 (lo plane */
/* = elements 0..15, hi plane = 16..31) and scripts/ternarize_a4b.py:80-88. */
/* ------------------------------------------------------------------------ */
void orc_q40_dequant(const uint8_t* blocks, int64_t nblocks, float* out) {
  for (int64_t b = 0; b < nblocks; ++b) {
    const uint8_t* p = blocks + b * 18;
    double d = orc_h2f(rd16(p));
    for (int j = 0; j < 16; ++j) {
      out[b * 32 + j] = (float)(d * (double)((p[2 + j] & 15) - 8));
      out[b * 32 + j + 16] = (float)(d * (double)((p[2 + j] >> 4) - 8));
    }
  }
}

/* y[o] = sum_b d(o,b) * sum_i (q-8) x[32b+i]  (kernels/q40mv.wgsl:56-89) */
static double q40_row_dot(const uint8_t* row, int64_t nb, const float* x) {
  double acc = 0.0;
  for (int64_t b = 0; b < nb; ++b) {
    const uint8_t* p = row + b * 18;
    const float* xb = x + b * 32;
    double s = 0.0;
    for (int j = 0; j < 16; ++j) {
      s += (double)((p[2 + j] & 15) - 8) * (double)xb[j];
      s += (double)((p[2 + j] >> 4) - 8) * (double)xb[j + 16];
    }
    acc += (double)orc_h2f(rd16(p)) * s;
  }
  return acc;
}

void orc_q40_gemv(const uint8_t* w, int64_t rows, int64_t cols, const float* x, float* y) {
  const int64_t nb = cols / 32;
#pragma omp parallel for schedule(static)
  for (int64_t o = 0; o < rows; ++o) y[o] = (float)q40_row_dot(w + o * nb * 18, nb, x);
}

/* EXPERT=1 indirection: weight base = topk[z] * OUT * rowB (q40mv.wgsl:70-74) */
void orc_q40_gemv_expert(const uint8_t* w, int expert, int64_t rows, int64_t cols,
                         const float* x, float* y) {
  orc_q40_gemv(w + (int64_t)expert * rows * (cols / 32) * 18, rows, cols, x, y);
}

/* ------------------------------------------------------------------------ */
/* Q6_K: 210 B = ql[128], qh[64], int8 scales[16], f16 d.  Element order is */
/* ggml dequantize_row_q6_K as restated by kernels/q6k.wgsl:44-71 (MODE 0). */
/* ------------------------------------------------------------------------ */
static inline int q6_val(const uint8_t* blk, int e) {
  /* element e (0..255) of one superblock -> 6-bit value 0..63 */
  int half = e >> 7, r = e & 127, quad = r >> 5, l = r & 31;
  const uint8_t* ql = blk + 64 * half;
  const uint8_t* qh = blk + 128 + 32 * half;
  int lo = (quad & 1) ? ql[l + 32] : ql[l];
  lo = (quad >= 2) ? (lo >> 4) : (lo & 15);
  int hi = (qh[l] >> (2 * quad)) & 3;
  return lo | (hi << 4);
}
static inline int q6_scale_index(int e) {
  /* sc_h[is + 2*quad], is = l/16, sc_h = scales + 8*half */
  int half = e >> 7, r = e & 127, quad = r >> 5, l = r & 31;
  return 8 * half + (l >> 4) + 2 * quad;
}

void orc_q6k_dequant(const uint8_t* blocks, int64_t nblocks, float mult, float* out) {
  for (int64_t b = 0; b < nblocks; ++b) {
    const uint8_t* blk = blocks + b * 210;
    double d = orc_h2f(rd16(blk + 208));
    const int8_t* sc = (const int8_t*)(blk + 192);
    for (int e = 0; e < 256; ++e)
      out[b * 256 + e] =
          (float)(d * (double)sc[q6_scale_index(e)] * (double)(q6_val(blk, e) - 32) * (double)mult);
  }
}

void orc_q6k_dequant_row(const uint8_t* w, int64_t cols, int64_t row, float mult, float* out) {
  const int64_t nsb = cols / 256;
  orc_q6k_dequant(w + row * nsb * 210, nsb, mult, out);
}

/* MODE 1 lm-head (kernels/q6k.wgsl:75-130): the 255*bacc - 32*gsum refold is */
/* algebraically sum d*s_j*(q-32)*x, computed here directly; then           */
/* SOFTCAP*tanh(y/SOFTCAP) when SOFTCAP != 0.                               */
void orc_q6k_gemv(const uint8_t* w, int64_t rows, int64_t cols, const float* x, float softcap,
                  float* y) {
  const int64_t nsb = cols / 256;
#pragma omp parallel for schedule(static)
  for (int64_t o = 0; o < rows; ++o) {
    double acc = 0.0;
    for (int64_t b = 0; b < nsb; ++b) {
      const uint8_t* blk = w + (o * nsb + b) * 210;
      const int8_t* sc = (const int8_t*)(blk + 192);
      const float* xb = x + b * 256;
      double g[16] = {0};
      for (int e = 0; e < 256; ++e) g[q6_scale_index(e)] += (double)(q6_val(blk, e) - 32) * (double)xb[e];
      double s = 0.0;
      for (int j = 0; j < 16; ++j) s += (double)sc[j] * g[j];
      acc += (double)orc_h2f(rd16(blk + 208)) * s;
    }
    float v = (float)acc;
    if (softcap != 0.0f) v = (float)((double)softcap * tanh((double)v / (double)softcap));
    y[o] = v;
  }
}

/* argmax2 (kernels/argmax2.wgsl:8-48): start (bv=-3e38, bi=0), take v when */
/* v > bv or (v == bv and i < bi): lowest index among maxima; NaN never wins. */
void orc_argmax(const float* x, int64_t n, uint32_t out[2]) {
  float bv = -3.0e38f;
  uint32_t bi = 0;
  for (int64_t i = 0; i < n; ++i) {
    float v = x[i];
    if (v > bv || (v == bv && (uint32_t)i < bi)) {
      bv = v;
      bi = (uint32_t)i;
    }
  }
  out[0] = bi;
  memcpy(&out[1], &bv, 4);
}

/* ------------------------------------------------------------------------ */
/* RMSNorm y = x * (mean x^2 + eps)^-1/2 * w  (kernels/rmsnorm.wgsl:13-51;   */
/* Gemma weight used directly, NOTES/arch-spec.md:97-118).  w may be NULL.  */
/* ------------------------------------------------------------------------ */
static double rms_inv(const float* x, int64_t n, float eps) {
  double s = 0.0;
  for (int64_t i = 0; i < n; ++i) s += (double)x[i] * (double)x[i];
  return 1.0 / sqrt(s / (double)n + (double)eps);
}
void orc_rmsnorm(const float* x, const float* w, int64_t n, float eps, float* y) {
  double inv = rms_inv(x, n, eps);
  for (int64_t i = 0; i < n; ++i) y[i] = (float)((double)x[i] * inv * (w ? (double)w[i] : 1.0));
}

/* gelu_pytorch_tanh with the reference's +-20 clamp (kernels/q40gu.wgsl:114) */
static double gelu_d(double g) {
  double t = 0.7978845608028654 * (g + 0.044715 * g * g * g);
  if (t > 20.0) t = 20.0;
  if (t < -20.0) t = -20.0;
  return 0.5 * g * (1.0 + tanh(t));
}
float orc_gelu_tanh(float g) { return (float)gelu_d(g); }

/* ------------------------------------------------------------------------ */
/* Router + top-K (kernels/routertop.wgsl:19-71, same epilogue as           */
/* kernels/top8.wgsl:9-29): f32 scores s = x.W_e; f32 p = exp(s - max)     */
/* (:53-56, the subtraction in f32, exp rounded once to f32); K rounds of  */
/* a strict '>' scan of p from bv = -1, so p values that round equal --    */
/* scores apart by less than the f32 spacing, or both underflowed to 0 --  */
/* go to the lowest index (:58-64); the winner is set to -2; w_k = p_k /   */
/* sum p, renormalised by the sum of the K picks, times pes[idx_k] (:66-68)*/
/* ------------------------------------------------------------------------ */
/* p[e] = f32 exp(f32(s_e - max s)) (kernels/routertop.wgsl:53-56); returns sum p */
static double router_probs(const float* sf, int E, double* p) {
  float mx = -3.0e38f;
  for (int e = 0; e < E; ++e)
    if (sf[e] > mx) mx = sf[e];
  double sum = 0.0;
  for (int e = 0; e < E; ++e) {
    const float d = sf[e] - mx; /* f32 difference */
    p[e] = (double)(float)exp((double)d);
    sum += p[e];
  }
  return sum;
}

void orc_router_topk(const float* x, const float* W, const float* pes, int H, int E, int K,
                     uint32_t* idx, float* wts, float* scores) {
  float* sf = (float*)malloc(sizeof(float) * (size_t)E);
  double* p = (double*)malloc(sizeof(double) * (size_t)E);
  for (int e = 0; e < E; ++e) {
    double s = 0.0;
    for (int j = 0; j < H; ++j) s += (double)x[j] * (double)W[(int64_t)e * H + j];
    sf[e] = (float)s; /* the reference stores f32 scores */
    if (scores) scores[e] = sf[e];
  }
  const double sum = router_probs(sf, E, p);
  double wk[64], wsum = 0.0;
  for (int k = 0; k < K; ++k) {
    int bi = 0;
    double bv = -1.0;
    for (int e = 0; e < E; ++e)
      if (p[e] > bv) {
        bv = p[e];
        bi = e;
      }
    idx[k] = (uint32_t)bi;
    wk[k] = bv / sum;
    wsum += wk[k];
    p[bi] = -2.0;
  }
  for (int k = 0; k < K; ++k) wts[k] = (float)(wk[k] / wsum * (double)pes[idx[k]]);
  free(p);
  free(sf);
}

/* ------------------------------------------------------------------------ */
/* RoPE inverse frequencies THETA^(-2p/HD) for p < angles, rounded once to  */
/* f32; the angle is th = f32(pos) * inv[p] in f32, as headprep.wgsl:54-64 */
/* forms fp * pow(THETA, -2p/HD).                                          */
/* ------------------------------------------------------------------------ */
void orc_rope_inv_freq(float theta, int head_dim, int angles, float* inv) {
  for (int p = 0; p < angles; ++p) inv[p] = (float)pow((double)theta, -2.0 * (double)p / (double)head_dim);
}

/* headprep (kernels/headprep.wgsl:19-87): per head weighted RMS; q/k rotate  */
/* pairs (p, p+HD/2) for p < angles; k and v (scale-less RMS) stored as f16. */
static void prep_head(const float* x, int hd, int angles, const float* inv_freq, const float* w,
                      float eps, uint32_t pos, double* out) {
  double inv = rms_inv(x, hd, eps);
  int half = hd / 2;
  float fp = (float)pos;
  for (int p = 0; p < half; ++p) {
    double x0 = (double)x[p] * inv * (double)w[p];
    double x1 = (double)x[p + half] * inv * (double)w[p + half];
    if (p < angles) {
      float th = fp * inv_freq[p];
      double c = cos((double)th), s = sin((double)th);
      out[p] = x0 * c - x1 * s;
      out[p + half] = x0 * s + x1 * c;
    } else {
      out[p] = x0;
      out[p + half] = x1;
    }
  }
}

void orc_headprep(const float* qkv, int qh, int kvh, int hd, int angles, const float* inv_freq,
                  const float* qw, const float* kw, float eps, uint32_t pos, float* q_out,
                  uint16_t* k_out, uint16_t* v_out) {
  double tmp[1024];
  for (int h = 0; h < qh; ++h) {
    prep_head(qkv + h * hd, hd, angles, inv_freq, qw, eps, pos, tmp);
    for (int d = 0; d < hd; ++d) q_out[h * hd + d] = (float)tmp[d];
  }
  for (int h = 0; h < kvh; ++h) {
    prep_head(qkv + (qh + h) * hd, hd, angles, inv_freq, kw, eps, pos, tmp);
    for (int d = 0; d < hd; ++d) k_out[h * hd + d] = orc_f2h((float)tmp[d]);
    const float* v = qkv + (qh + kvh + h) * hd;
    double inv = rms_inv(v, hd, eps);
    for (int d = 0; d < hd; ++d) v_out[h * hd + d] = orc_f2h((float)((double)v[d] * inv));
  }
}

/* ------------------------------------------------------------------------ */
/* KV ring slot recovery RecPs(t, m) = m - ((m + RING - t) % RING)           */
/* (specs/KVRing.tla:45, kernels/attnf32.wgsl:50-52).                       */
/* ------------------------------------------------------------------------ */
int64_t orc_kvring_recover(int64_t t, int64_t mw, int64_t ring) {
  return mw - ((mw + ring - t) % ring);
}

/* Softmax attention of one q head over a list of (slot) rows; scale 1.0    */
/* (NOTES/arch-spec.md:383-392).  Dead rows are skipped: their contribution */
/* is exactly 0 (the reference multiplies 0*v, kernels/attnf32.wgsl:89-90). */
/* probs (may be NULL) receives each row's normalised weight e^(s-m)/den,   */
/* the quantity attnos.wgsl's SCORE pass adds to the slot's mass (:78-92).  */
static void attn_rows_p(const float* q, const uint16_t* kc, const uint16_t* vc, int kvh, int h_kv,
                        int hd, const int64_t* slots, int64_t n, uint16_t* out, double* probs) {
  double* s = (double*)malloc(sizeof(double) * (size_t)(n > 0 ? n : 1));
  double m = -3.0e38;
  for (int64_t i = 0; i < n; ++i) {
    const uint16_t* k = kc + (slots[i] * kvh + h_kv) * hd;
    double a = 0.0;
    for (int d = 0; d < hd; ++d) a += (double)q[d] * (double)orc_h2f(k[d]);
    s[i] = a;
    if (a > m) m = a;
  }
  double den = 0.0;
  double acc[1024];
  for (int d = 0; d < hd; ++d) acc[d] = 0.0;
  for (int64_t i = 0; i < n; ++i) {
    double e = exp(s[i] - m);
    den += e;
    const uint16_t* v = vc + (slots[i] * kvh + h_kv) * hd;
    for (int d = 0; d < hd; ++d) acc[d] += e * (double)orc_h2f(v[d]);
  }
  for (int d = 0; d < hd; ++d) out[d] = orc_f2h((float)(acc[d] / den));
  if (probs)
    for (int64_t i = 0; i < n; ++i) probs[i] = exp(s[i] - m) / den;
  free(s);
}
static void attn_rows(const float* q, const uint16_t* kc, const uint16_t* vc, int kvh, int h_kv,
                      int hd, const int64_t* slots, int64_t n, uint16_t* out) {
  attn_rows_p(q, kc, vc, kvh, h_kv, hd, slots, n, out, NULL);
}

/* attnf32 CACHEMODE 1 decode (kernels/attnf32.wgsl:21-105): qp = maxW = pos, */
/* len = min(pos+1, RING); slot t dead iff ps > qp or ps + W <= qp.           */
void orc_attn_ring(const float* q, const uint16_t* kc, const uint16_t* vc, int qh, int kvh,
                   int hd, int ring, int window, uint32_t pos, uint16_t* out) {
  int64_t qp = pos, mw = pos;
  int64_t len = mw + 1 < ring ? mw + 1 : ring;
  int64_t* slots = (int64_t*)malloc(sizeof(int64_t) * (size_t)len);
  int64_t n = 0;
  for (int64_t t = 0; t < len; ++t) {
    int64_t ps = orc_kvring_recover(t, mw, ring);
    int dead = ps > qp || ps + window <= qp;
    if (!dead) slots[n++] = t;
  }
  for (int h = 0; h < qh; ++h)
    attn_rows(q + h * hd, kc, vc, kvh, h / (qh / kvh), hd, slots, n, out + h * hd);
  free(slots);
}

/* attnos full-layer decode (kernels/attnos.wgsl:22-98): positions 0..len-1. */
void orc_attn_linear(const float* q, const uint16_t* kc, const uint16_t* vc, int qh, int kvh,
                     int hd, uint32_t len, uint16_t* out) {
  int64_t* slots = (int64_t*)malloc(sizeof(int64_t) * (size_t)(len ? len : 1));
  for (uint32_t t = 0; t < len; ++t) slots[t] = t;
  for (int h = 0; h < qh; ++h)
    attn_rows(q + h * hd, kc, vc, kvh, h / (qh / kvh), hd, slots, len, out + h * hd);
  free(slots);
}

/* Split-K phase A (kernels/attsplit.wgsl:16-76): chunk c covers positions  */
/* [start + c*cs, min(start+(c+1)*cs, len)); start = len - window when the  */
/* window is active.  Empty chunk -> (m, e) = (-3e38, 0).  part_o is the     */
/* unnormalised sum e^{s-m_c} v; part_me = (m_c, sum e^{s-m_c}).            */
void orc_attn_split(const float* q, const uint16_t* kc, const uint16_t* vc, int qh, int kvh,
                    int hd, uint32_t len, int window, int chunks, int cs, float* part_o,
                    float* part_me) {
  int64_t start = (window != 0 && (int64_t)len > window) ? (int64_t)len - window : 0;
  for (int h = 0; h < qh; ++h) {
    int hk = h / (qh / kvh);
    for (int c = 0; c < chunks; ++c) {
      int64_t pi = (int64_t)h * chunks + c;
      int64_t lo = start + (int64_t)c * cs;
      float* po = part_o + pi * hd;
      for (int d = 0; d < hd; ++d) po[d] = 0.0f;
      if (lo >= (int64_t)len) {
        part_me[2 * pi] = -3.0e38f;
        part_me[2 * pi + 1] = 0.0f;
        continue;
      }
      int64_t hi = lo + cs < (int64_t)len ? lo + cs : (int64_t)len;
      double m = -3.0e38;
      double* s = (double*)malloc(sizeof(double) * (size_t)(hi - lo));
      for (int64_t t = lo; t < hi; ++t) {
        const uint16_t* k = kc + (t * kvh + hk) * hd;
        double a = 0.0;
        for (int d = 0; d < hd; ++d) a += (double)q[h * hd + d] * (double)orc_h2f(k[d]);
        s[t - lo] = a;
        if (a > m) m = a;
      }
      double e = 0.0, acc[1024];
      for (int d = 0; d < hd; ++d) acc[d] = 0.0;
      for (int64_t t = lo; t < hi; ++t) {
        double p = exp(s[t - lo] - m);
        e += p;
        const uint16_t* v = vc + (t * kvh + hk) * hd;
        for (int d = 0; d < hd; ++d) acc[d] += p * (double)orc_h2f(v[d]);
      }
      free(s);
      for (int d = 0; d < hd; ++d) po[d] = (float)acc[d];
      part_me[2 * pi] = (float)m;
      part_me[2 * pi + 1] = (float)e;
    }
  }
}

/* Split-K phase B (kernels/attcomb.wgsl:10-36): M = max m_c over the n live */
/* chunks, o = sum_{e_c>0} partO_c e^{m_c-M} / sum e_c e^{m_c-M}; the        */
/* reference then SRQ-packs for the E4B o-proj, this build stores f16.      */
void orc_attn_combine(const float* part_o, const float* part_me, int qh, int hd, int n_chunks,
                      int chunks, uint16_t* out) {
  for (int h = 0; h < qh; ++h) {
    double M = -3.0e38;
    for (int c = 0; c < n_chunks; ++c) {
      double m = part_me[2 * ((int64_t)h * chunks + c)];
      if (m > M) M = m;
    }
    double den = 0.0;
    for (int c = 0; c < n_chunks; ++c) {
      const float* me = part_me + 2 * ((int64_t)h * chunks + c);
      den += (double)me[1] * exp((double)me[0] - M);
    }
    for (int d = 0; d < hd; ++d) {
      double a = 0.0;
      for (int c = 0; c < n_chunks; ++c) {
        const float* me = part_me + 2 * ((int64_t)h * chunks + c);
        if (me[1] > 0.0f) a += (double)part_o[((int64_t)h * chunks + c) * hd + d] * exp((double)me[0] - M);
      }
      out[h * hd + d] = orc_f2h((float)(a / den));
    }
  }
}

/* ------------------------------------------------------------------------ */
/* KVRing.tla (specs/KVRing.tla:29-85) as a direct state walk: the spec's   */
/* Next relation is deterministic, so TLC's reachable set is one behaviour. */
/* Returns 0 = both invariants hold, 1 = SoundRec violated, 2 = Complete.  */
/* ------------------------------------------------------------------------ */
static int served(int64_t qp, int64_t m, int64_t W, int64_t RING) {
  int64_t lo = qp + 1 >= W ? qp + 1 - W : 0;
  for (int64_t p = lo; p <= qp; ++p)
    if (orc_kvring_recover(p % RING, m, RING) != p) return 0;
  return 1;
}
static int sound_rec(int64_t mw, int64_t RING) {
  for (int64_t t = 0; t < RING; ++t) {
    if (t > mw) continue;
    int64_t r = orc_kvring_recover(t, mw, RING);
    int64_t best = -1;
    for (int64_t p = t; p <= mw; p += RING) best = p; /* max of S */
    if (r != best) return 0;
  }
  return 1;
}
int orc_kvring_check(int W, int C, int RING, int NCHUNKS, int GEN) {
  int64_t total = (int64_t)NCHUNKS * C;
  int64_t mw = C - 1, base = 0;
  int phase = 0; /* 0 pre, 1 gen, 2 done */
  for (;;) {
    if (!sound_rec(mw, RING)) return 1;
    if (phase == 0) {
      for (int64_t qp = base; qp <= base + C - 1; ++qp)
        if (!served(qp, mw, W, RING)) return 2;
    } else if (phase == 1) {
      if (!served(mw, mw, W, RING)) return 2;
    }
    if (phase == 2) break;
    if (phase == 0) {
      if (base + C < total) {
        mw = base + 2 * (int64_t)C - 1;
        base = base + C;
      } else if (GEN > 0) {
        mw = mw + 1;
        phase = 1;
      } else {
        phase = 2;
      }
    } else {
      if (mw < total + GEN - 1)
        mw = mw + 1;
      else
        phase = 2;
    }
  }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* MoE FFN half-layer, A4B engine order (src/engine-a4b.js:438-462):         */
/* rmsacc3's three scaled outputs (kernels/rmsacc3.wgsl:44-53, without the   */
/* attention residual), routertop, q40gu EXPERT=2 (kernels/q40gu.wgsl:62-119) */
/* for the dense branch and the K expert slots, dense q40mv down,            */
/* q40moedown (kernels/q40moedown.wgsl:42-75) and a4btail                    */
/* (kernels/a4btail.wgsl:26-71, NEXT=0).                                     */
/* ------------------------------------------------------------------------ */
static void geglu_rows(const uint8_t* gu, int64_t ff, int64_t in, const float* x, float* out_f16_as_f32) {
  float* g = (float*)malloc(sizeof(float) * (size_t)ff * 2);
  orc_q40_gemv(gu, 2 * ff, in, x, g);
  for (int64_t i = 0; i < ff; ++i)
    out_f16_as_f32[i] = orc_h2f(orc_f2h((float)(gelu_d(g[i]) * (double)g[ff + i])));
  free(g);
}

/* the selection's decision margin: (K-th largest score - (K+1)-th) / max |score| */
static double route_margin_of(const float* sc, int E, int K) {
  double mx = 0.0;
  for (int e = 0; e < E; ++e) mx = fmax(mx, fabs((double)sc[e]));
  if (K >= E || mx == 0.0) return 0.0;
  /* K-th and (K+1)-th largest by repeated scans (E <= 256) */
  double prev = INFINITY, kth = 0.0, next = 0.0;
  int taken = 0;
  while (taken <= K) {
    double best = -INFINITY;
    int cnt = 0;
    for (int e = 0; e < E; ++e)
      if ((double)sc[e] < prev && (double)sc[e] > best) best = (double)sc[e];
    if (best == -INFINITY) return 0.0; /* NaN scores: no margin */
    for (int e = 0; e < E; ++e)
      if ((double)sc[e] == best) ++cnt;
    for (int c = 0; c < cnt && taken <= K; ++c, ++taken) {
      if (taken == K - 1) kth = best;
      if (taken == K) next = best;
    }
    prev = best;
  }
  return (kth - next) / mx;
}

void orc_moe_ffn(const orc_moe* m, const float* h, uint32_t* topk_idx, float* topk_w,
                 float* dense_out, float* moe_out, float* h_out) {
  orc_moe_ffn_m(m, h, topk_idx, topk_w, dense_out, moe_out, h_out, NULL);
}

void orc_moe_ffn_m(const orc_moe* m, const float* h, uint32_t* topk_idx, float* topk_w,
                   float* dense_out, float* moe_out, float* h_out, double* margin) {
  orc_moe_ffn_f(m, h, NULL, NULL, topk_idx, topk_w, dense_out, moe_out, h_out, margin);
}

/* force_idx != NULL: the expert slots use those K experts instead of the     */
/* oracle's own top-K (a test hands over the GPU's picks at a routing near-   */
/* tie), weighted as routertop weights its picks: softmax probability over   */
/* all E scores, renormalised over the K, times pes (kernels/routertop.wgsl:  */
/* 19-71); own_idx (may be NULL) receives the oracle's own top-K.           */
void orc_moe_ffn_f(const orc_moe* m, const float* h, const uint32_t* force_idx, uint32_t* own_idx,
                   uint32_t* topk_idx, float* topk_w, float* dense_out, float* moe_out, float* h_out,
                   double* margin) {
  const int H = m->hidden, E = m->n_experts, K = m->top_k, FF = m->expert_ffn, FF2 = m->dense_ffn;
  float *xd = malloc(sizeof(float) * H), *xr = malloc(sizeof(float) * H), *xm = malloc(sizeof(float) * H);
  double inv = rms_inv(h, H, m->eps);
  double rs = 1.0 / sqrt((double)H); /* ffn_gate_inp.scale * H^-1/2, src/engine-a4b.js:174-179 */
  for (int i = 0; i < H; ++i) {
    double v = (double)h[i] * inv;
    xd[i] = orc_h2f(orc_f2h((float)(v * (double)m->ffn_norm[i])));
    xr[i] = (float)(v * (double)((float)((double)m->router_scale[i] * rs)));
    xm[i] = orc_h2f(orc_f2h((float)(v * (double)m->pre_ffw2[i])));
  }
  float* sc = malloc(sizeof(float) * E);
  orc_router_topk(xr, m->router_w, m->pes, H, E, K, topk_idx, topk_w, sc);
  if (margin) *margin = route_margin_of(sc, E, K);
  if (own_idx) memcpy(own_idx, topk_idx, sizeof(uint32_t) * (size_t)K);
  if (force_idx) {
    double* p = malloc(sizeof(double) * (size_t)E);
    const double sum = router_probs(sc, E, p);
    double wsum = 0.0, wk[64];
    for (int k = 0; k < K; ++k) {
      topk_idx[k] = force_idx[k];
      wk[k] = p[force_idx[k]] / sum;
      wsum += wk[k];
    }
    for (int k = 0; k < K; ++k) topk_w[k] = (float)(wk[k] / wsum * (double)m->pes[topk_idx[k]]);
    free(p);
  }
  free(sc);

  /* dense branch: gate rows [0,FF2), up rows [FF2,2FF2) */
  float* gd = malloc(sizeof(float) * FF2);
  {
    uint8_t* cat = malloc((size_t)2 * FF2 * (H / 32) * 18);
    size_t half = (size_t)FF2 * (H / 32) * 18;
    memcpy(cat, m->dense_gate, half);
    memcpy(cat + half, m->dense_up, half);
    geglu_rows(cat, FF2, H, xd, gd);
    free(cat);
  }
  orc_q40_gemv(m->dense_down, H, FF2, gd, dense_out);

  /* expert slots: sum_k w_k * W_down[e_k] . geglu_k */
  float* ge = malloc(sizeof(float) * FF);
  float* yk = malloc(sizeof(float) * H);
  double* acc = calloc((size_t)H, sizeof(double));
  const int64_t gu_stride = (int64_t)2 * FF * (H / 32) * 18;
  for (int k = 0; k < K; ++k) {
    int e = (int)topk_idx[k];
    geglu_rows(m->exp_gate_up + e * gu_stride, FF, H, xm, ge);
    orc_q40_gemv_expert(m->exp_down, e, H, FF, ge, yk);
    for (int i = 0; i < H; ++i) acc[i] += (double)topk_w[k] * (double)yk[i];
  }
  for (int i = 0; i < H; ++i) moe_out[i] = (float)acc[i];

  /* a4btail: comb = rms(t1) w1 + rms(m) w2; h = (h + rms(comb) wp) * MUL */
  double i1 = rms_inv(dense_out, H, m->eps), i2 = rms_inv(moe_out, H, m->eps);
  float* comb = malloc(sizeof(float) * H);
  for (int i = 0; i < H; ++i)
    comb[i] = (float)((double)dense_out[i] * i1 * (double)m->post_ffw1[i] +
                      (double)moe_out[i] * i2 * (double)m->post_ffw2[i]);
  double i3 = rms_inv(comb, H, m->eps);
  for (int i = 0; i < H; ++i)
    h_out[i] = (float)(((double)h[i] + (double)comb[i] * i3 * (double)m->post_ffw[i]) * (double)m->layer_scale);
  free(xd); free(xr); free(xm); free(gd); free(ge); free(yk); free(acc); free(comb);
}

/* ------------------------------------------------------------------------ */
/* Full E4B-shaped decode step.  Layer order follows the A4B engine's        */
/* encodeLayer (src/engine-a4b.js:424-463) for the attention/FFN halves and  */
/* the E4B engine's PLE dataflow (src/engine.js:282-323, kernels/pleprep.wgsl */
/* :15-46, kernels/plegatemv.wgsl:20-60) with the SRQ int8 steps dropped;    */
/* the lm-head is the tied Q6_K embedding with softcap, then argmax          */
/* (src/engine-a4b.js:683-693).                                             */
/* ------------------------------------------------------------------------ */
/* Full (global) layers are "counted" (src/engine-a4b.js:217, :695-699,    */
/* CACHEMODE 2): the new row goes to slot kv_count and attention reads      */
/* slots [0, kv_count]; kv_count restarts at 0 when pos == 0 and equals     */
/* pos until a compaction.  With scoring on, every step adds each live      */
/* slot's normalised attention weight to score[l][h][slot] in f32 (attnos    */
/* SCORE = 1, kernels/attnos.wgsl:78-92).                                   */
struct orc_state {
  int layers, hidden;
  uint16_t** kc;
  uint16_t** vc;
  float* ple; /* [layers][ple_dim] per-layer inputs of the current token */
  int64_t kv_count;
  int scoring;
  float** score; /* global layers: [q_heads][max_seq] */
  /* this step's own K/V rows per layer [layers][kv_heads][head_dim] (f16  */
  /* bits); with keep_rows the step leaves the cache slot of the current  */
  /* token as it was handed over (orc_state_set_kv) and attends to that   */
  /* row, so a test can start a step from another implementation's rows  */
  int keep_rows;
  uint16_t* krow;
  uint16_t* vrow;
  int64_t row_stride; /* krow/vrow entries per layer: the largest kv_heads * head_dim */
  /* A4B recipe: the smallest top-8 decision margin of the last step's      */
  /* layers ((8th - 9th router score) / max |score|; orc_moe_ffn_m)        */
  double route_margin;
  /* per layer of the last step: the residual stream after the layer        */
  /* ([layers][hidden]); A4B: the oracle's own top-8 ([layers][8]), its     */
  /* decision margin, and the experts a test forces on that layer (force[l] */
  /* set: used instead of the own picks)                                    */
  float* lh;
  uint32_t* ltopk;
  double* lmargin;
  uint32_t* lforce;
  uint8_t* forced;
};

static int64_t slots_of(const orc_model* m, int l) {
  return m->layer_global[l] ? m->max_seq : m->ring;
}
/* per-layer attention shape: the A4B recipe's full layers use head_dim_full, */
/* rope_angles_full and V = K (src/engine-a4b.js:152-156, 330-334)            */
static int lay_hd(const orc_model* m, int l) {
  return (m->recipe == 1 && m->layer_global[l] && m->head_dim_full > 0) ? m->head_dim_full : m->head_dim;
}
static int lay_kvh(const orc_model* m, int l) {
  return (m->recipe == 1 && m->layer_kv_heads) ? m->layer_kv_heads[l] : m->kv_heads;
}
static int lay_angles(const orc_model* m, int l) {
  return (m->recipe == 1 && m->layer_global[l]) ? m->rope_angles_full : m->rope_angles;
}
static int lay_keqv(const orc_model* m, int l) { return m->recipe == 1 && m->layer_global[l]; }
static int64_t row_max(const orc_model* m) {
  int64_t r = 0;
  for (int l = 0; l < m->layers; ++l)
    if ((int64_t)lay_kvh(m, l) * lay_hd(m, l) > r) r = (int64_t)lay_kvh(m, l) * lay_hd(m, l);
  return r;
}

orc_state* orc_state_new(const orc_model* m) {
  orc_state* s = calloc(1, sizeof(orc_state));
  s->layers = m->layers;
  s->hidden = m->hidden;
  s->kc = calloc((size_t)m->layers, sizeof(uint16_t*));
  s->vc = calloc((size_t)m->layers, sizeof(uint16_t*));
  for (int l = 0; l < m->layers; ++l) {
    size_t n = (size_t)slots_of(m, l) * lay_kvh(m, l) * lay_hd(m, l);
    s->kc[l] = calloc(n, sizeof(uint16_t));
    s->vc[l] = calloc(n, sizeof(uint16_t));
  }
  s->ple = calloc((size_t)m->layers * (m->ple_dim > 0 ? m->ple_dim : 1), sizeof(float));
  s->krow = calloc((size_t)m->layers * row_max(m), sizeof(uint16_t));
  s->vrow = calloc((size_t)m->layers * row_max(m), sizeof(uint16_t));
  s->row_stride = row_max(m);
  s->lh = calloc((size_t)m->layers * m->hidden, sizeof(float));
  s->ltopk = calloc((size_t)m->layers * 8, sizeof(uint32_t));
  s->lmargin = calloc((size_t)m->layers, sizeof(double));
  s->lforce = calloc((size_t)m->layers * 8, sizeof(uint32_t));
  s->forced = calloc((size_t)m->layers, 1);
  s->score = calloc((size_t)m->layers, sizeof(float*));
  for (int l = 0; l < m->layers; ++l)
    if (m->layer_global[l]) s->score[l] = calloc((size_t)m->q_heads * m->max_seq, sizeof(float));
  return s;
}
void orc_state_free(orc_state* s) {
  if (!s) return;
  for (int l = 0; l < s->layers; ++l) {
    free(s->kc[l]);
    free(s->vc[l]);
  }
  free(s->kc);
  free(s->vc);
  free(s->ple);
  free(s->krow);
  free(s->vrow);
  for (int l = 0; l < s->layers; ++l) free(s->score[l]);
  free(s->score);
  free(s->lh);
  free(s->ltopk);
  free(s->lmargin);
  free(s->lforce);
  free(s->forced);
  free(s);
}
void orc_state_set_scoring(orc_state* s, int on) { s->scoring = on; }
void orc_state_set_keep_rows(orc_state* s, int on) { s->keep_rows = on; }
const uint16_t* orc_state_krow(const orc_state* s, int layer) { return s->krow + (size_t)layer * s->row_stride; }
const uint16_t* orc_state_vrow(const orc_state* s, int layer) { return s->vrow + (size_t)layer * s->row_stride; }
int64_t orc_state_kv_count(const orc_state* s) { return s->kv_count; }
double orc_state_route_margin(const orc_state* s) { return s->route_margin; }
const float* orc_state_layer_hidden(const orc_state* s, int layer) { return s->lh + (size_t)layer * s->hidden; }
const uint32_t* orc_state_layer_topk(const orc_state* s, int layer) { return s->ltopk + (size_t)layer * 8; }
double orc_state_layer_margin(const orc_state* s, int layer) { return s->lmargin[layer]; }
void orc_state_force_topk(orc_state* s, int layer, const uint32_t* idx) {
  s->forced[layer] = idx != NULL;
  if (idx) memcpy(s->lforce + (size_t)layer * 8, idx, sizeof(uint32_t) * 8);
}
const float* orc_state_score(const orc_state* s, int layer) { return s->score[layer]; }

/* compactAll's selection (src/engine-a4b.js:587-617) for one full layer:    */
/* mass[t] = sum over heads of score[h][t] (f64, head order); the candidates */
/* [0, n - prot) sorted by mass, largest first, ties in index order (the     */
/* stable Array.prototype.sort over an ascending list); keep the first       */
/* budget - prot of them and the prot = min(protect, n) newest slots, in     */
/* slot order.  Returns the number kept (<= n).                             */
int64_t orc_kv_keep(const float* score, int qh, int64_t scap, int64_t n, int budget, int protect,
                    uint32_t* keep) {
  double* mass = calloc((size_t)(n > 0 ? n : 1), sizeof(double));
  for (int h = 0; h < qh; ++h)
    for (int64_t t = 0; t < n; ++t) mass[t] += (double)score[h * scap + t];
  const int64_t prot = protect < n ? protect : n;
  const int64_t nc = n - prot;
  int64_t want = budget - prot;
  if (want < 0) want = 0;
  if (want > nc) want = nc;
  /* selection of the `want` largest by repeated scans: the first candidate  */
  /* (lowest index) among equal masses wins, as the stable sort orders them */
  char* taken = calloc((size_t)(nc > 0 ? nc : 1), 1);
  int64_t cnt = 0;
  for (int64_t k = 0; k < want; ++k) {
    int64_t best = -1;
    for (int64_t t = 0; t < nc; ++t)
      if (!taken[t] && (best < 0 || mass[t] > mass[best])) best = t;
    taken[best] = 1;
  }
  for (int64_t t = 0; t < nc; ++t)
    if (taken[t]) keep[cnt++] = (uint32_t)t;
  for (int64_t t = nc; t < n; ++t) keep[cnt++] = (uint32_t)t;
  free(taken);
  free(mass);
  return cnt;
}

/* kvgather (kernels/kvgather.wgsl) of one full layer: slot i <- slot        */
/* keep[i] for K and V, then its scores zeroed (src/engine-a4b.js:604-614).  */
void orc_kv_gather_layer(const orc_model* m, orc_state* s, int layer, const uint32_t* keep, int64_t cnt) {
  const int64_t row = (int64_t)lay_kvh(m, layer) * lay_hd(m, layer);
  uint16_t* tmp = malloc(sizeof(uint16_t) * (size_t)((cnt > 0 ? cnt : 1) * row));
  uint16_t* caches[2] = {s->kc[layer], s->vc[layer]};
  for (int c = 0; c < 2; ++c) {
    for (int64_t i = 0; i < cnt; ++i) memcpy(tmp + i * row, caches[c] + (int64_t)keep[i] * row, sizeof(uint16_t) * row);
    memcpy(caches[c], tmp, sizeof(uint16_t) * (size_t)(cnt * row));
  }
  memset(s->score[layer], 0, sizeof(float) * (size_t)m->q_heads * m->max_seq);
  free(tmp);
}
void orc_state_set_kv_count(orc_state* s, int64_t n) { s->kv_count = n; }

/* compactAll (src/engine-a4b.js:587-617) on every full layer: the keep list */
/* of orc_kv_keep, the gather, zeroed scores; kv_count = the number kept.    */
int64_t orc_kv_compact(const orc_model* m, orc_state* s, int budget, int protect) {
  const int64_t n = s->kv_count;
  uint32_t* keep = malloc(sizeof(uint32_t) * (size_t)(n > 0 ? n : 1));
  int64_t cnt = n;
  for (int l = 0; l < m->layers; ++l) {
    if (!m->layer_global[l]) continue;
    cnt = orc_kv_keep(s->score[l], m->q_heads, m->max_seq, n, budget, protect, keep);
    orc_kv_gather_layer(m, s, l, keep, cnt);
  }
  s->kv_count = cnt;
  free(keep);
  return cnt;
}
/* Overwrite one layer's K and V caches ([slots][kvh][hd] f16 bits): tests */
/* hand the oracle another implementation's caches so that one step can be  */
/* compared from identical state.                                           */
void orc_state_set_kv(const orc_model* m, orc_state* s, int layer, const uint16_t* k, const uint16_t* v) {
  const size_t n = (size_t)slots_of(m, layer) * lay_kvh(m, layer) * lay_hd(m, layer);
  memcpy(s->kc[layer], k, n * sizeof(uint16_t));
  memcpy(s->vc[layer], v, n * sizeof(uint16_t));
}
const uint16_t* orc_state_kcache(const orc_state* s, int layer) { return s->kc[layer]; }
const uint16_t* orc_state_vcache(const orc_state* s, int layer) { return s->vc[layer]; }

int64_t orc_kv_slot(const orc_model* m, int is_global, uint32_t pos) {
  return is_global ? (int64_t)pos : (int64_t)(pos % (uint32_t)m->ring);
}

static void round_f16(float* x, int64_t n) {
  for (int64_t i = 0; i < n; ++i) x[i] = orc_h2f(orc_f2h(x[i]));
}

/* One layer of the A4B recipe (src/engine-a4b.js:424-463): attn_norm -> q|k|v */
/* GEMVs on the f16 input (full layers have no V projection: V is the raw K  */
/* slice, KEQV, kernels/headprep.wgsl:23) -> headprep with the layer's head   */
/* dim and rotated pairs (src/engine-a4b.js:330-334) -> ring or counted       */
/* attention -> o -> h1 = h + rms(o) post_attention_norm (rmsacc3,             */
/* kernels/rmsacc3.wgsl:36-53) -> the MoE FFN half on h1 (orc_moe_ffn:        */
/* rmsacc3's branch inputs, routertop, q40gu, q40moedown, a4btail).          */
static void a4b_layer(const orc_model* m, orc_state* st, int l, float* h, uint32_t pos, int64_t kv) {
  const orc_layer* ly = &m->L[l];
  const int H = m->hidden, QH = m->q_heads, glob = m->layer_global[l];
  const int HD = lay_hd(m, l), KVH = lay_kvh(m, l), ANG = lay_angles(m, l), keqv = lay_keqv(m, l);
  float* x = malloc(sizeof(float) * H);
  float* qkv = malloc(sizeof(float) * (size_t)(QH + 2 * KVH) * HD);
  float* qp = malloc(sizeof(float) * (size_t)QH * HD);
  uint16_t* ao = malloc(sizeof(uint16_t) * (size_t)QH * HD);
  float* a = malloc(sizeof(float) * (size_t)QH * HD);
  float* o = malloc(sizeof(float) * H);
  float* inv = malloc(sizeof(float) * (size_t)(HD / 2));
  orc_rope_inv_freq(glob ? m->theta_global : m->theta_local, HD, ANG, inv);
  orc_rmsnorm(h, ly->attn_norm, H, m->eps, x);
  round_f16(x, H);
  orc_q40_gemv(ly->wq, QH * HD, H, x, qkv);
  orc_q40_gemv(ly->wk, KVH * HD, H, x, qkv + QH * HD);
  if (keqv)
    memcpy(qkv + (size_t)(QH + KVH) * HD, qkv + (size_t)QH * HD, sizeof(float) * (size_t)KVH * HD);
  else
    orc_q40_gemv(ly->wv, KVH * HD, H, x, qkv + (size_t)(QH + KVH) * HD);
  const int64_t slot = glob ? kv : orc_kv_slot(m, glob, pos);
  uint16_t* krow = st->krow + (size_t)l * st->row_stride;
  uint16_t* vrow = st->vrow + (size_t)l * st->row_stride;
  orc_headprep(qkv, QH, KVH, HD, ANG, inv, ly->q_norm, ly->k_norm, m->eps, pos, qp, krow, vrow);
  if (!st->keep_rows) {
    memcpy(st->kc[l] + slot * KVH * HD, krow, sizeof(uint16_t) * (size_t)KVH * HD);
    memcpy(st->vc[l] + slot * KVH * HD, vrow, sizeof(uint16_t) * (size_t)KVH * HD);
  }
  if (glob) {
    /* slots [0, kv]; with scoring, each slot's weight joins its mass (attnos */
    /* SCORE, kernels/attnos.wgsl:78-92), as on the E4B recipe's full layers   */
    const int64_t len = kv + 1;
    int64_t* sl = malloc(sizeof(int64_t) * (size_t)len);
    double* pr = malloc(sizeof(double) * (size_t)len);
    for (int64_t t = 0; t < len; ++t) sl[t] = t;
    for (int hh = 0; hh < QH; ++hh) {
      attn_rows_p(qp + (size_t)hh * HD, st->kc[l], st->vc[l], KVH, hh / (QH / KVH), HD, sl, len,
                  ao + (size_t)hh * HD, st->scoring ? pr : NULL);
      if (st->scoring)
        for (int64_t t = 0; t < len; ++t)
          st->score[l][hh * m->max_seq + t] = st->score[l][hh * m->max_seq + t] + (float)pr[t];
    }
    free(sl);
    free(pr);
  } else {
    orc_attn_ring(qp, st->kc[l], st->vc[l], QH, KVH, HD, m->ring, m->window, pos, ao);
  }
  orc_h2f_n(ao, (int64_t)QH * HD, a);
  orc_q40_gemv(ly->wo, H, QH * HD, a, o);
  double io = rms_inv(o, H, m->eps);
  for (int i = 0; i < H; ++i) h[i] = (float)((double)h[i] + (double)o[i] * io * (double)ly->post_attn_norm[i]);
  float* dn = malloc(sizeof(float) * H);
  float* mo = malloc(sizeof(float) * H);
  float* ho = malloc(sizeof(float) * H);
  uint32_t idx[64];
  float w[64];
  double mg = INFINITY;
  orc_moe_ffn_f(&ly->moe, h, st->forced[l] ? st->lforce + (size_t)l * 8 : NULL, st->ltopk + (size_t)l * 8, idx, w,
                dn, mo, ho, &mg);
  st->lmargin[l] = mg;
  if (mg < st->route_margin) st->route_margin = mg;
  memcpy(h, ho, sizeof(float) * H);
  free(x); free(qkv); free(qp); free(ao); free(a); free(o); free(inv); free(dn); free(mo); free(ho);
}

uint32_t orc_step(const orc_model* m, orc_state* st, uint32_t token, uint32_t pos, float* logits,
                  float* hidden_out) {
  const int H = m->hidden, QH = m->q_heads, KVH = m->kv_heads, HD = m->head_dim;
  const int FF = m->ffn, PD = m->ple_dim, L = m->layers;
  const int QKV = (QH + 2 * KVH) * HD;
  float* h = malloc(sizeof(float) * H);
  float* x = malloc(sizeof(float) * (FF > QKV ? FF : QKV) * 2);
  float* qkv = malloc(sizeof(float) * QKV);
  float* qp = malloc(sizeof(float) * QH * HD);
  uint16_t* ao = malloc(sizeof(uint16_t) * QH * HD);
  float* a = malloc(sizeof(float) * QH * HD);
  float* o = malloc(sizeof(float) * H);
  float* gu = malloc(sizeof(float) * 2 * FF);
  float* gg = malloc(sizeof(float) * FF);
  float* inv_l = malloc(sizeof(float) * HD);
  float* inv_g = malloc(sizeof(float) * HD);
  orc_rope_inv_freq(m->theta_local, HD, m->rope_angles, inv_l);
  orc_rope_inv_freq(m->theta_global, HD, m->rope_angles, inv_g);
  if (pos == 0) st->kv_count = 0;
  const int64_t kv = st->kv_count; /* full-layer slot of this token */
  st->route_margin = INFINITY;

  /* embedding row * sqrt(H) (kernels/q6k.wgsl:37-73, MULT = sqrt(hidden)) */
  orc_q6k_dequant_row(m->tok_embd, H, token, (float)sqrt((double)H), h);

  if (PD > 0) {
    /* PLE inputs: proj = W_pm h * H^-1/2; per block b:                      */
    /* (rms(proj_b) * w_pn + row_b(token) * sqrt(PD)) * 2^-1/2             */
    const int NP = L * PD;
    float* proj = malloc(sizeof(float) * NP);
    float* idv = malloc(sizeof(float) * NP);
    orc_q40_gemv(m->ple_proj, NP, H, h, proj);
    double sc = 1.0 / sqrt((double)H);
    for (int i = 0; i < NP; ++i) proj[i] = (float)((double)proj[i] * sc);
    orc_q6k_dequant_row(m->ple_tab, NP, token, (float)sqrt((double)PD), idv);
    for (int b = 0; b < L; ++b) {
      double inv = rms_inv(proj + b * PD, PD, m->eps);
      for (int i = 0; i < PD; ++i)
        st->ple[b * PD + i] = (float)(((double)proj[b * PD + i] * inv * (double)m->ple_proj_norm[i] +
                                       (double)idv[b * PD + i]) * 0.70710678118654752);
    }
    free(proj);
    free(idv);
  }

  for (int l = 0; l < L; ++l) {
    if (m->recipe == 1) {
      a4b_layer(m, st, l, h, pos, kv);
      memcpy(st->lh + (size_t)l * H, h, sizeof(float) * H);
      continue;
    }
    const orc_layer* ly = &m->L[l];
    const int glob = m->layer_global[l];
    /* attention block */
    orc_rmsnorm(h, ly->attn_norm, H, m->eps, x);
    round_f16(x, H);
    orc_q40_gemv(ly->wq, QH * HD, H, x, qkv);
    orc_q40_gemv(ly->wk, KVH * HD, H, x, qkv + QH * HD);
    orc_q40_gemv(ly->wv, KVH * HD, H, x, qkv + (QH + KVH) * HD);
    int64_t slot = glob ? kv : orc_kv_slot(m, glob, pos);
    uint16_t* krow = st->krow + (size_t)l * st->row_stride;
    uint16_t* vrow = st->vrow + (size_t)l * st->row_stride;
    orc_headprep(qkv, QH, KVH, HD, m->rope_angles, glob ? inv_g : inv_l, ly->q_norm, ly->k_norm,
                 m->eps, pos, qp, krow, vrow);
    if (!st->keep_rows) {
      memcpy(st->kc[l] + slot * KVH * HD, krow, sizeof(uint16_t) * (size_t)KVH * HD);
      memcpy(st->vc[l] + slot * KVH * HD, vrow, sizeof(uint16_t) * (size_t)KVH * HD);
    }
    if (glob) {
      /* slots [0, kv]; with scoring, each slot's weight joins its mass */
      const int64_t len = kv + 1;
      int64_t* sl = malloc(sizeof(int64_t) * (size_t)len);
      double* pr = malloc(sizeof(double) * (size_t)len);
      for (int64_t t = 0; t < len; ++t) sl[t] = t;
      for (int hh = 0; hh < QH; ++hh) {
        attn_rows_p(qp + hh * HD, st->kc[l], st->vc[l], KVH, hh / (QH / KVH), HD, sl, len, ao + hh * HD,
                    st->scoring ? pr : NULL);
        if (st->scoring)
          for (int64_t t = 0; t < len; ++t)
            st->score[l][hh * m->max_seq + t] = st->score[l][hh * m->max_seq + t] + (float)pr[t];
      }
      free(sl);
      free(pr);
    } else {
      orc_attn_ring(qp, st->kc[l], st->vc[l], QH, KVH, HD, m->ring, m->window, pos, ao);
    }
    orc_h2f_n(ao, QH * HD, a);
    orc_q40_gemv(ly->wo, H, QH * HD, a, o);
    /* h1 = h + rms(o) w_pa; x = f16(rms(h1) w_ffn) (kernels/rmsacc3.wgsl:36-53) */
    {
      double io = rms_inv(o, H, m->eps);
      for (int i = 0; i < H; ++i) h[i] = (float)((double)h[i] + (double)o[i] * io * (double)ly->post_attn_norm[i]);
    }
    orc_rmsnorm(h, ly->ffn_norm, H, m->eps, x);
    round_f16(x, H);
    /* gate/up + GeGLU -> f16 (kernels/q40gu.wgsl:62-119) */
    orc_q40_gemv(ly->wgate, FF, H, x, gu);
    orc_q40_gemv(ly->wup, FF, H, x, gu + FF);
    for (int i = 0; i < FF; ++i) gg[i] = orc_h2f(orc_f2h((float)(gelu_d(gu[i]) * (double)gu[FF + i])));
    orc_q40_gemv(ly->wdown, H, FF, gg, o);
    {
      double io = rms_inv(o, H, m->eps);
      for (int i = 0; i < H; ++i) h[i] = (float)((double)h[i] + (double)o[i] * io * (double)ly->post_ffw_norm[i]);
    }
    if (PD > 0) {
      /* PLE block: g = f16(gelu(W_gate f16(h)) * ple_l); p = W_proj g;       */
      /* h = (h + rms(p) w_post) * layer_scale                                */
      for (int i = 0; i < H; ++i) x[i] = orc_h2f(orc_f2h(h[i]));
      float* pg = gu;
      orc_q40_gemv(ly->inp_gate, PD, H, x, pg);
      for (int i = 0; i < PD; ++i)
        gg[i] = orc_h2f(orc_f2h((float)(gelu_d(pg[i]) * (double)st->ple[l * PD + i])));
      orc_q40_gemv(ly->proj, H, PD, gg, o);
      double io = rms_inv(o, H, m->eps);
      for (int i = 0; i < H; ++i)
        h[i] = (float)(((double)h[i] + (double)o[i] * io * (double)ly->post_norm[i]) * (double)ly->layer_scale);
    } else {
      for (int i = 0; i < H; ++i) h[i] = (float)((double)h[i] * (double)ly->layer_scale);
    }
    memcpy(st->lh + (size_t)l * H, h, sizeof(float) * H);
  }
  if (hidden_out) memcpy(hidden_out, h, sizeof(float) * H);

  /* final norm (f32) -> Q6_K lm-head + softcap -> argmax */
  orc_rmsnorm(h, m->out_norm, H, m->eps, x);
  float* lg = logits ? logits : malloc(sizeof(float) * (size_t)m->vocab);
  orc_q6k_gemv(m->tok_embd, m->vocab, H, x, m->softcap, lg);
  uint32_t am[2];
  orc_argmax(lg, m->vocab, am);
  if (!logits) free(lg);
  free(h); free(x); free(qkv); free(qp); free(ao); free(a); free(o); free(gu); free(gg);
  free(inv_l); free(inv_g);
  st->kv_count = kv + 1;
  return am[0];
}
