// moe.h -- arguments and launchers of the MoE FFN half-layer (k_moe.hip).
#pragma once
#include <hip/hip_runtime.h>

#include "kernels.h"

constexpr int kMoeTopK = 8;

struct MoeArgs {
  // inputs
  const float* h;             // [H] hidden state entering the FFN half
  const float* ffn_norm;      // [H] dense-branch input norm
  const float* router_scale;  // [H] ffn_gate_inp.scale (raw)
  float router_mult;          // H^-1/2, applied to router_scale (src/engine-a4b.js:174-179)
  const float* pre_ffw2;      // [H] expert-branch input norm
  const float* router_w;      // [E][H] f32
  const float* pes;           // [E] per-expert output scale
  Q40Mat dense_gu;            // [2 FF2][H]: gate rows, then up rows
  Q40Mat exp_gu;              // [E * 2 FF][H]: expert e = rows [2 FF e, 2 FF (e+1)), gate then up
  Q40Mat dense_down;          // [H][FF2]
  Q40Mat exp_down;            // [E * H][FF]
  const float* post_ffw1;     // [H]
  const float* post_ffw2;     // [H]
  const float* post_ffw;      // [H]
  float layer_scale, eps;
  int H, E, FF, FF2;
  // intermediates (device scratch) and outputs
  float* scores;              // [E]
  uint16_t* xd;               // [H] f16 dense input
  uint16_t* xm;               // [H] f16 expert input
  uint32_t* topk_idx;         // [8]
  float* topk_w;              // [8]
  uint16_t* g_dense;          // [FF2] f16
  uint16_t* g_slots;          // [8][FF] f16
  float* dense_out;           // [H]
  float* moe_out;             // [H]
  float* h_out;               // [H]; null: no tail launch (a consumer's prologue finishes the layer)
  // optional attention residual folded into the router (decode step only):
  // h1 = h + rms(attn_o) post_attn is the FFN half's input, written to h1
  // (a buffer other than h) by router block 0 and read by the tail
  const float* attn_o;        // [attn_o_slices][H] o projection output (column-slice partials), or null
  int attn_o_slices;          // 1, 2 or 4 (0 = 1): attn_o = their sum, added in slice order
  const float* post_attn;     // [H]
  float* h1;                  // [H]
};

// router scores (+ the f16 branch inputs)
int launch_moe_router(const MoeArgs& a, hipStream_t st);
// router + top-8 only: writes topk_idx / topk_w
int launch_moe_topk(const MoeArgs& a, hipStream_t st);
// the whole half-layer: router, gate/up, down, tail
int launch_moe_ffn(const MoeArgs& a, hipStream_t st);
// the same router / top-8 / tail kernels over M token rows (row y of h, xd,
// xm, dense_out, moe_out, h_out at y * H, of scores at y * E, of topk at y * 8)
int launch_moe_router_rows(const MoeArgs& a, int M, hipStream_t st);
int launch_moe_topk_rows(const MoeArgs& a, int M, hipStream_t st);
int launch_moe_tail_rows(const MoeArgs& a, int M, hipStream_t st);

// ---- batched prefill of the half-layer (k_moe_prefill.hip) -----------------
struct MoePrefillBufs {
  float* scores;       // [M][E]
  uint16_t *xd, *xm;   // [M][H] f16 branch inputs
  uint32_t* topk_idx;  // [M][8]
  float* topk_w;       // [M][8]
  uint32_t* list;      // [M*8] draws (m*8 + k) sorted by expert
  uint32_t* pos;       // [M*8] sorted position of each draw
  int4* tiles;         // [max_tiles] (expert, first sorted row, rows)
  int* ntiles;
  int max_tiles;
  uint16_t* g_sorted;  // [M*8][FF] f16 expert GeGLU outputs, sorted
  float* d_sorted;     // [M*8][H] expert down outputs, sorted
  uint16_t* g_dense;   // [M][FF2]
  float* gd_part;      // [kMoePfDenseKs][M][2 FF2] dense gate|up split-K partials
                       // (then the dense down's, [kMoePfDenseKs][M][H]; sized for both)
  float* dense_out;    // [M][H]
  float* moe_out;      // [M][H]
};
// K slices of the dense gate|up GEMM over the prompt rows (its 2 x 2112 rows
// give too few workgroups for one slice); k_geglu_rows sums them
constexpr int kMoePfDenseKs = 2;
// bytes of scratch for M tokens; with base != null also fills b from it
size_t moe_prefill_scratch(const MoeArgs& a, int M, MoePrefillBufs* b, uint8_t* base);
// h_out[m] (a.h_out, rows of H) for the M token rows of a.h
int launch_moe_prefill(const MoeArgs& a, int M, const MoePrefillBufs& b, hipStream_t st);
