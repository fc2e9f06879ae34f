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
  float* h_out;               // [H]
};

// router scores (+ the f16 branch inputs)
int launch_moe_router(const MoeArgs& a, hipStream_t st);
// router + top-8 only: writes topk_idx / topk_w
int launch_moe_topk(const MoeArgs& a, hipStream_t st);
// the whole half-layer: router, gate/up, down, tail
int launch_moe_ffn(const MoeArgs& a, hipStream_t st);
