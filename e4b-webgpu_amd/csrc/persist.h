// persist.h -- host/device interface of the persistent layer-loop kernel
// (k_persist.hip): one cooperative launch runs every layer of a decode step.
#pragma once
#include <stdint.h>

#include "kernels.h"

constexpr int kPersistThreads = 512;  // threads per block (8 waves)
constexpr int kPersistPhases = 8;     // hand-offs per layer (tags per layer)

// one layer's weights and caches, as the device reads them
struct PersistLayer {
  Q40Mat qkv, o, gu, down, pg, pp;     // pp: PLE projection [H][PD], row-major
  const float *attn_norm, *q_norm, *k_norm, *post_attn, *ffn_norm, *post_ffw, *post_norm;
  float scale;
  int global;                          // 1 = full layer (counted slots), 0 = sliding ring
  uint16_t *kc, *vc;                   // [kvh][slots][256] f16
  int slots;
  // this layer's tagged hand-off words (u64), one of two sets alternating by
  // layer parity: p [H], qkv [(QH + 2 KVH) 256], attention partials
  // [QH][nch_max][256 + 2], attention out [QH 256 / 2], o [H], GeGLU
  // [FF / 2], down [H], PLE gate [PD / 2].  Loaded per layer, the addresses
  // are not loop invariants the compiler could hoist (and spill) out of
  // the layer loop.
  unsigned long long *ll_p, *ll_qkv, *ll_pm, *ll_att, *ll_o, *ll_gg, *ll_dn, *ll_g;
};

struct PersistArgs {
  const PersistLayer* L;               // [layers], device memory
  int layers, H, FF, QH, KVH, PD, window, nch_max;
  float eps;
  const uint32_t* params;              // [0] position, [4] full-layer slot, [8] tag epoch
  uint32_t* epoch;                     // params + 8: advanced by block 0 at the end
  const float* h_in;                   // the token's embedding row (f32 [H])
  const float* ple;                    // per-layer inputs [layers][PD]
  const float2* rope;                  // (cos, sin) [2][128]: sliding, full layers
  int* abort;                          // raised by a block whose wait gave up
  float* h_out;                        // hidden state after the last layer
  uint16_t* xo_hl;                     // f16 hi[H] then lo[H] of rms(h) w_out (lm-head input)
  const float* out_norm;
  // optional phase trace (e4b_profile_step): thread 0 of every block stores
  // wall_clock64() at [block][layer][phase][0 start, 1 input ready, 2 done]
  unsigned long long* trace;
};
constexpr int kPersistTraceSlots = kPersistPhases * 3;

// launch on `st` (cooperative, one block per CU); chunk 32 or 64 positions
int launch_persist(const PersistArgs& a, int blocks, int chunk, hipStream_t st);
// blocks the launch uses on the current device (H / 8, one per CU; 0 when
// that many cannot be co-resident, -hipError_t when the query failed), and
// whether a configuration is supported
int persist_blocks(int H, int FF, int chunk);
bool persist_supported(int H, int FF, int QH, int KVH, int PD);
// why the last persist_blocks call returned 0
const char* persist_why();
