// k_moe_prefill.hip -- the MoE FFN half-layer over M prompt tokens (the
// batched prefill of the A4B engine, src/engine-a4b.js:478-549 routerTopB /
// expGroup / guGsg32 / downGsg32 / waccB, kernels/expgroup.wgsl:15-50,
// kernels/q40gugrp.wgsl:47-103), with the per-token arithmetic of the decode
// half-layer (k_moe.hip):
//
//   router + top-8      the decode kernels over token rows (bit-identical picks)
//   k_moe_group         counting sort of the M*8 (token, slot) draws by expert
//                       into contiguous runs, cut into tiles of <= 32 rows
//   grouped GEMMs       expert gate/up + GeGLU and expert down on the matrix
//                       cores (k_gemm.hip grouped mode): each tile reads its
//                       expert's rows once for up to 32 draws
//   dense branch        gate|up GEMM in K slices, k_geglu_rows, down GEMM in
//                       K slices over all M tokens
//   k_moe_combine_rows  moe[m] = sum_k w_k down_sorted[pos(m, k)], in k order,
//                       and the dense down's K slices summed
//   tail                the decode tail over token rows
#include "../../include/e4b.h"
#include "kernels.h"
#include "moe.h"
#include "util.h"

namespace {

constexpr int K = kMoeTopK;
constexpr int kTileRows = 32;

// one workgroup: histogram of the draws' experts in LDS, exclusive scan,
// placement (list[slot] = draw, pos[draw] = slot) and the tile table.  The
// order of draws inside an expert's run depends on LDS atomics; every output
// row is computed from its own input row only, so results do not.
__global__ __launch_bounds__(1024) void k_moe_group(const uint32_t* __restrict__ topk_idx, int npairs, int E,
                                                    uint32_t* __restrict__ list, uint32_t* __restrict__ pos,
                                                    int4* __restrict__ tiles, int* __restrict__ ntiles) {
  __shared__ int cnt[256], off[256], fill[256], toff[256];
  const int t = threadIdx.x;
  if (t < 256) {
    cnt[t] = 0;
    fill[t] = 0;
  }
  __syncthreads();
  for (int p = t; p < npairs; p += 1024) atomicAdd(&cnt[min((int)topk_idx[p], E - 1)], 1);
  __syncthreads();
  if (t == 0) {
    int o = 0, tt = 0;
    for (int e = 0; e < E; ++e) {
      off[e] = o;
      toff[e] = tt;
      o += cnt[e];
      tt += (cnt[e] + kTileRows - 1) / kTileRows;
    }
    *ntiles = tt;
  }
  __syncthreads();
  for (int p = t; p < npairs; p += 1024) {
    const int e = min((int)topk_idx[p], E - 1);
    const int s = off[e] + atomicAdd(&fill[e], 1);
    list[s] = (uint32_t)p;
    pos[p] = (uint32_t)s;
  }
  for (int e = t; e < E; e += 1024)
    for (int j = 0; j * kTileRows < cnt[e]; ++j)
      tiles[toff[e] + j] = make_int4(e, off[e] + j * kTileRows, min(kTileRows, cnt[e] - j * kTileRows), 0);
}

// out[m][j] = f16(gelu(gate) * up) of the dense branch, gate and up each the
// sum of the ks split-K slices of the gate|up GEMM (rows j and FF + j), in
// slice order; the arithmetic of the GEMM's GeGLU epilogue after that sum
__global__ __launch_bounds__(256) void k_geglu_rows(const float* __restrict__ part, int ks, int64_t slice, int FF,
                                                    uint16_t* __restrict__ out) {
  const int m = blockIdx.y, j = blockIdx.x * 256 + threadIdx.x;
  if (j >= FF) return;
  const float* p = part + (int64_t)m * 2 * FF + j;
  float g = p[0], u = p[FF];
  for (int s = 1; s < ks; ++s) {
    g += p[s * slice];
    u += p[s * slice + FF];
  }
  out[(int64_t)m * FF + j] = f2h(gelu_tanh(g) * u);
}

// moe[m][i] = sum_k w[m][k] * down[pos[m K + k]][i], in slot order
// (and dense[m] = the sum of the dense down GEMM's dks K slices of row m, in
// slice order)
__global__ __launch_bounds__(256) void k_moe_combine_rows(const float* __restrict__ down,
                                                          const uint32_t* __restrict__ pos,
                                                          const float* __restrict__ topk_w, int H,
                                                          float* __restrict__ moe, const float* __restrict__ dpart,
                                                          int dks, int64_t dslice, float* __restrict__ dense) {
  const int m = blockIdx.y;
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= H) return;
  const int64_t o = (int64_t)m * H + i;
  float ds = dpart[o];
  for (int s = 1; s < dks; ++s) ds += dpart[s * dslice + o];
  float acc = 0.f;
#pragma unroll
  for (int k = 0; k < K; ++k) acc = fmaf(topk_w[m * K + k], down[(int64_t)pos[m * K + k] * H + i], acc);
  moe[o] = acc;
  dense[o] = ds;
}

}  // namespace

size_t moe_prefill_scratch(const MoeArgs& a, int M, MoePrefillBufs* b, uint8_t* base) {
  const int H = a.H, E = a.E, FF = a.FF, FF2 = a.FF2;
  const size_t P = (size_t)M * K;
  const int max_tiles = E + (int)((P + kTileRows - 1) / kTileRows);
  size_t cur = 0;
  auto take = [&](size_t bytes) {
    uint8_t* p = base ? base + cur : nullptr;
    cur += E4B_ALIGN256(bytes);
    return p;
  };
  uint8_t* p_scores = take((size_t)M * E * 4);
  uint8_t* p_xd = take((size_t)M * H * 2);
  uint8_t* p_xm = take((size_t)M * H * 2);
  uint8_t* p_idx = take(P * 4);
  uint8_t* p_w = take(P * 4);
  uint8_t* p_list = take(P * 4);
  uint8_t* p_pos = take(P * 4);
  uint8_t* p_tiles = take((size_t)max_tiles * 16);
  uint8_t* p_nt = take(16);
  uint8_t* p_g = take(P * FF * 2);
  uint8_t* p_d = take(P * H * 4);
  uint8_t* p_gd = take((size_t)M * FF2 * 2);
  uint8_t* p_gdp = take((size_t)kMoePfDenseKs * M * (2 * FF2 > H ? 2 * FF2 : H) * 4);
  uint8_t* p_dense = take((size_t)M * H * 4);
  uint8_t* p_moe = take((size_t)M * H * 4);
  if (b) {
    b->scores = (float*)p_scores;
    b->xd = (uint16_t*)p_xd;
    b->xm = (uint16_t*)p_xm;
    b->topk_idx = (uint32_t*)p_idx;
    b->topk_w = (float*)p_w;
    b->list = (uint32_t*)p_list;
    b->pos = (uint32_t*)p_pos;
    b->tiles = (int4*)p_tiles;
    b->ntiles = (int*)p_nt;
    b->max_tiles = max_tiles;
    b->g_sorted = (uint16_t*)p_g;
    b->d_sorted = (float*)p_d;
    b->g_dense = (uint16_t*)p_gd;
    b->gd_part = (float*)p_gdp;
    b->dense_out = (float*)p_dense;
    b->moe_out = (float*)p_moe;
  }
  return cur;
}

int launch_moe_prefill(const MoeArgs& base, int M, const MoePrefillBufs& b, hipStream_t st) {
  const int H = base.H, E = base.E, FF = base.FF, FF2 = base.FF2;
  if (M < 1 || (int64_t)M * K > 8192)
    return e4b_fail(E4B_EINVAL, "MoE prefill: %d tokens (1..1024 per call)", M);
  if (E < K || E > 256 || H % 256 || FF % 32 || FF2 % 32)
    return e4b_fail(E4B_EINVAL, "MoE prefill: bad shape (H=%d E=%d FF=%d FF2=%d)", H, E, FF, FF2);
  MoeArgs a = base;
  a.scores = b.scores;
  a.xd = b.xd;
  a.xm = b.xm;
  a.topk_idx = b.topk_idx;
  a.topk_w = b.topk_w;
  a.dense_out = b.dense_out;
  a.moe_out = b.moe_out;
  int rc;
  if ((rc = launch_moe_router_rows(a, M, st)) || (rc = launch_moe_topk_rows(a, M, st))) return rc;
  hipLaunchKernelGGL(k_moe_group, dim3(1), dim3(1024), 0, st, b.topk_idx, M * K, E, b.list, b.pos, b.tiles, b.ntiles);
  E4B_HIP(hipGetLastError());
  // expert gate/up + GeGLU over the sorted draws, then expert down
  GemmArgs g{};
  g.W = a.exp_gu;
  g.X = b.xm;
  g.M = M * K;
  g.ldx = H;
  g.epi = GEMM_GLU;
  g.Yh = b.g_sorted;
  g.ff = FF;
  g.ks = 1;
  g.tiles = b.tiles;
  g.ntiles = b.ntiles;
  g.max_tiles = b.max_tiles;
  g.group_rows = 2 * (int64_t)FF;
  g.gather = b.list;
  g.gather_div = K;
  if ((rc = launch_q40_gemm(g, st))) return rc;
  g.W = a.exp_down;
  g.X = b.g_sorted;
  g.ldx = FF;
  g.epi = GEMM_F32;
  g.Y = b.d_sorted;
  g.Yh = nullptr;
  g.ff = 0;
  g.group_rows = H;
  g.gather = nullptr;
  g.gather_div = 1;
  if ((rc = launch_q40_gemm(g, st))) return rc;
  // dense branch over all tokens: gate|up in K slices, then the GeGLU rows
  GemmArgs d{};
  d.W = a.dense_gu;
  d.X = b.xd;
  d.M = M;
  d.ldx = H;
  d.epi = GEMM_F32;
  d.Y = b.gd_part;
  d.ks = q40_gemm_kslices(a.dense_gu.nb, kMoePfDenseKs);
  if ((rc = launch_q40_gemm(d, st))) return rc;
  hipLaunchKernelGGL(k_geglu_rows, dim3((FF2 + 255) / 256, M), dim3(256), 0, st, b.gd_part, d.ks,
                     (int64_t)M * 2 * FF2, FF2, b.g_dense);
  E4B_HIP(hipGetLastError());
  d.W = a.dense_down;
  d.X = b.g_dense;
  d.ldx = FF2;
  d.epi = GEMM_F32;
  d.Y = b.gd_part;  // the down's K slices reuse the gate|up partials' space
  d.ks = q40_gemm_kslices(a.dense_down.nb, kMoePfDenseKs);
  if ((rc = launch_q40_gemm(d, st))) return rc;
  hipLaunchKernelGGL(k_moe_combine_rows, dim3((H + 255) / 256, M), dim3(256), 0, st, b.d_sorted, b.pos, b.topk_w, H,
                     b.moe_out, b.gd_part, d.ks, (int64_t)M * H, b.dense_out);
  E4B_HIP(hipGetLastError());
  return launch_moe_tail_rows(a, M, st);
}
