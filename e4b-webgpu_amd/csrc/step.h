// step.h -- launchers of the decode-step kernels in k_attn.hip / k_step.hip.
#pragma once
#include <hip/hip_runtime.h>

#include "kernels.h"

struct AttnLaunch {
  const float* qkv;        // raw q | k | v (f32) of the current token
  const float* qw;         // q head-norm weight [hd]
  const float* kw;         // k head-norm weight [hd]
  const float* inv_freq;   // RoPE inverse frequencies [angles]
  const float2* rope;      // (cos, sin) of pos * inv_freq[p] for this step, or null
  uint16_t* kc;            // [kvh][slots][hd] f16 key cache
  uint16_t* vc;            // [kvh][slots][hd] f16 value cache
  const uint32_t* params;  // params[0] = position of the current token (device), or
  uint32_t pos;            //   this position when params is null
  int kv_idx = 0;          // full layers: params[kv_idx] = the token's slot (0: the position)
  float* raw = nullptr;    // full layers, may be null: raw scores [qh][slots] for the mass
  float* part_o;           // [qh][attn_chunks(span, chunk)][hd] split-K partial outputs
  float* part_ml;          // [qh][attn_chunks(span, chunk)][2]  (chunk max, chunk sum)
  uint16_t* out;           // [qh][hd] f16 attention output
  int qh, kvh, hd, angles;
  int slots;               // ring slots (sliding) or capacity (global)
  int window;              // sliding window; 0 = global layer (linear cache)
  int chunk;               // positions per split-K chunk: 32 or 64
  int vslices = 4;         // V-dim slices per chunk (blocks per chunk): 4 (4 waves each) or 2 (8 waves each)
  bool combine;            // also launch the combine (false: the o projection's prologue merges)
  float eps;
};

int launch_attn(const AttnLaunch& a, hipStream_t st);
// score[h][t] += normalised attention weight of live slot t (after launch_attn
// with raw set); slots = the layer's capacity (score and raw row stride)
int launch_attn_score(const float* part_ml, const float* raw, const uint32_t* params, int kv_idx, int qh, int slots,
                      int chunk, float* score, hipStream_t st);
// dst[g][i] = src[g][keep[i]] (K and V) for i < n; dst rows per head: dslots
int launch_kv_gather(const uint32_t* keep, int n, const uint16_t* kc, const uint16_t* vc, int kvh, int slots,
                     uint16_t* dk, uint16_t* dv, int dslots, hipStream_t st);
constexpr int kAttnMaxChunks = 512;
// split-K chunks a layer of `max_positions` live positions needs
int attn_chunks(int max_positions, int chunk);
// the PLE branch of one layer (k_ple.hip)
struct PleLaunch {
  Q40Mat gate;              // [PD][H]
  const uint4* proj_nib;    // projection [H][PD] stored block-transposed: [PD/32][H] nibble blocks
  const uint16_t* proj_sc;  // [PD/32][H] block scales
  const float* ple;         // [PD] this layer's per-layer input
  float* part;              // [PD/32][H] partial projections (summed by the consumer)
  int H, PD;
};
int launch_ple(const PleLaunch& a, const ProArgs& pa, hipStream_t st);
// p = sum of np partial vectors (stride H)
int launch_tail(float* h, const float* p, int np, const float* w_post, float scale, const float* w_out,
                uint16_t* xo_hl, int H, float eps, hipStream_t st);
// also fills rope[2 * half] = (cos, sin)(pos * inv_{local,global}[p]) for the
// attention kernels of this step
int launch_embed(const Q6Mat& E, const uint32_t* params, const uint32_t* prompt, float mult, float* h, uint16_t* h_hl,
                 uint32_t* status, const float* inv_local, const float* inv_global, int half, float2* rope,
                 hipStream_t st);
int launch_ple_prep(const float* proj, const uint8_t* table, const float* w_pn, const uint32_t* params,
                    const uint32_t* prompt, int L, int vocab, float proj_scale, float* ple, const float* h,
                    const float* w_attn0, uint16_t* xn, int H, float eps, hipStream_t st);
int launch_feedback(const uint2* part, int nparts, uint32_t* amax, uint32_t* params, uint32_t* tok_ring, int ring_cap,
                    hipStream_t st);

// ---- batched prefill (k_prefill.hip) -----------------------------------------
// h[m] = E[ids[m]] * mult; xhl = [hi][M][H] then [lo][M][H] f16 split of h
int launch_embed_rows(const Q6Mat& E, const uint32_t* ids, int M, float mult, float* h, uint16_t* xhl, hipStream_t st);
// proj: two partial slices [M][L*256] at distance `slice`
int launch_ple_prep_rows(const float* proj, int64_t slice, const uint8_t* table, const float* w_pn,
                         const uint32_t* ids, int M, int L, float proj_scale, float* ple, float eps, hipStream_t st);
// per token: h = (h + rms(sum of na slices of a) * w1) * scale (a may be
// null); x = f16(rms(h) * w2) (w2 null: f16(h)); xlo (may be null) = the low
// half of the f16 hi/lo pair of the same value (hi + lo within
// max(2^-22 |y|, 2^-25) of y)
int launch_resnorm_rows(int M, float* h, const float* a, int na, int64_t slice, const float* w1, float scale,
                        const float* w2, uint16_t* x, uint16_t* xlo, int H, float eps, hipStream_t st);
// y[m][i] = f16(gelu(sum of ks slices of part[m][i]) * mul[m mul_ld + i]), i < n
int launch_gelu_mul_rows(const float* part, int ks, int64_t slice, int M, int64_t n, const float* mul, int64_t mul_ld,
                         uint16_t* y, hipStream_t st);
// qkv: ks partial slices [M][(qh + 2 kvh) 256]; q out [M][qh][256] f32; K/V
// rows of positions p0 .. p0 + M - 1 written to the caches (ring: slot p % slots)
int launch_headprep_rows(const float* qkv, int ks, int64_t slice, const float* qw, const float* kw,
                         const float* inv_freq, int angles, uint16_t* kc, uint16_t* vc, int slots, bool ring,
                         uint32_t p0, int M, float* q, int qh, int kvh, float eps, hipStream_t st);
struct PrefillAttnArgs {
  const float* q;     // [M][qh][hd] prepped queries of positions p0 .. p0 + M - 1
  const uint16_t* kc; // [kvh][slots][hd]
  const uint16_t* vc;
  uint16_t* out;      // [M][qh * hd] f16
  int M, qh, kvh, slots;
  int hd = 256;       // 256 (1, 2 or 4 q heads per KV head) or 512 (8)
  int window;         // 0 = global layer
  uint32_t p0;
  // split-key partials (attn_prefill_part_bytes(M, kvh, qh / kvh, hd) bytes); null: every
  // query tile walks its keys in one workgroup
  float* part = nullptr;
  size_t part_bytes = 0;
  int kspl = 0, ns = 1;  // keys per split and splits per query tile (set by the launcher)
};
// the partial buffer a chunk of M queries needs at most
size_t attn_prefill_part_bytes(int M, int kvh, int gqa, int hd = 256);
int launch_attn_prefill(PrefillAttnArgs a, hipStream_t st);
