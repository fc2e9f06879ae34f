// a4b.h -- launchers of the A4B-recipe step kernels (k_a4b.hip): the parts
// of the reference's live engine (src/engine-a4b.js:424-463) that the E4B
// kernels do not cover -- hidden sizes that are not a power-of-two multiple
// of 256, KV heads per layer, head dim 512 with a quarter of the pairs
// rotated, and V taken from the raw K projection on full layers.
#pragma once
#include <hip/hip_runtime.h>

#include "kernels.h"

// h_out = (h_in + rms(a) * w1) * scale (a null: h_in * scale; h_out null: not
// stored, h_in and h_out may alias); x (null: none) = f16(rms(h_out) * w2)
// (w2 null: f16(h_out)); xlo (null: none) = f16(y - f16(y)), the low half of
// the hi/lo pair of the same value.  H <= 4096.  One workgroup per row: M
// rows at stride H in h_in, h_out, a, x and xlo (the weights are shared).
// na > 1 (<= 4): a is the sum of na split-K slices at stride a_slice, added in
// slice order.
int launch_rownorm(const float* h_in, float* h_out, const float* a, const float* w1, float scale, const float* w2,
                   uint16_t* x, uint16_t* xlo, int H, float eps, hipStream_t st, int M = 1, int na = 1,
                   int64_t a_slice = 0);

struct AttnGen {
  const float* qkv;        // raw q [qh][hd] | k [kvh][hd] | v [kvh][hd] (no v rows when keqv)
  const float* qw;         // [hd] q head-norm weight
  const float* kw;         // [hd] k head-norm weight
  const float* inv_freq;   // [hd / 2] THETA^(-2p/hd), f32
  const float2* rope;      // [>= angles] (cos, sin)(pos inv_freq[p]) of this step, or null: evaluated here
  const uint32_t* params;  // [0] position, [kv_idx] the full layers' slot
  uint16_t* kc;            // [kvh][slots][hd]
  uint16_t* vc;
  float* part_o;           // [qh][gch][hd] unnormalised chunk outputs
  float* part_ml;          // [qh][gch][2] (chunk max, chunk sum)
  uint16_t* out;           // [qh][hd] f16 attention output (the merge)
  float* raw;              // full layers, may be null: raw scores [qh][slots] of the live slots
  int qh, kvh, hd, angles, slots, window, kv_idx, gch;
  bool keqv;               // V = the raw K slice (kernels/headprep.wgsl:23)
  bool no_merge;           // the consumer merges the partials (the o projection's prologue): no merge launch
  float eps;
};
constexpr int kAttnGenChunk = 64;  // positions per split-K chunk
constexpr int kAttnGenMaxChunks = 256;  // chunks per head the merge holds (max_seq <= 16384)
// head prep with the K/V row write, split-K partials over the live chunks,
// then their log-sum-exp merge (two launches); head dim 256 or 512, 1, 2, 4
// or 8 q heads per KV head
int launch_attn_gen(const AttnGen& a, hipStream_t st);

// ---- batched prefill of the A4B recipe (src/engine-a4b.js:465-549) ----------
struct HeadRowsGen {
  const float* qkv;        // [M][ld]: raw q | k (| v) rows of each token
  int64_t ld;
  const float* qw;
  const float* kw;
  const float* inv_freq;
  uint16_t* kc;            // [kvh][slots][hd]
  uint16_t* vc;
  float* q;                // [M][qh][hd] prepped queries
  int qh, kvh, hd, angles, slots, window;
  bool keqv;
  uint32_t p0;             // position (= full-layer slot) of token 0
  float eps;
  int ks = 1;              // qkv = the sum of ks split-K slices at stride slice
  int64_t slice = 0;
};
// head prep of M tokens: queries out, the K/V rows of positions p0 .. p0 + M - 1 into the caches
int launch_headprep_rows_gen(const HeadRowsGen& a, int M, hipStream_t st);

struct AttnRowsGen {
  const float* q;          // [M][qh][hd]
  const uint16_t* kc;      // [kvh][slots][hd], every position <= p0 + M - 1 written
  const uint16_t* vc;
  uint16_t* out;           // [M][qh hd] f16
  int qh, kvh, hd, slots, window;
  uint32_t p0;
};
// causal attention of M tokens (token m at position p0 + m over its live
// window), one workgroup per (KV group, token)
int launch_attn_rows_gen(const AttnRowsGen& a, int M, hipStream_t st);

// compaction gather of one layer: dst[g][i] = src[g][keep[i]] for K and V,
// rows of hd f16 (any head dim up to 1024)
int launch_kv_gather_gen(const uint32_t* keep, int n, const uint16_t* kc, const uint16_t* vc, int kvh, int slots,
                         int hd, uint16_t* dk, uint16_t* dv, int dslots, hipStream_t st);
