// kernels.h -- device-side views of packed weights and launch helpers shared
// by the kernel translation units and the engine.
#pragma once
#include <hip/hip_runtime.h>

#include "common.h"

struct Q40Mat {
  const uint4* nib;      // [rows][nb] re-ordered nibble blocks
  const uint16_t* sc;    // [rows][nb] f16 block scales
  int64_t rows;
  int nb;                // blocks per row = cols / 32
};

static inline Q40Mat q40_view(const void* packed, int64_t rows, int64_t cols) {
  Q40Mat m;
  m.nib = (const uint4*)packed;
  m.sc = (const uint16_t*)((const uint8_t*)packed + E4B_ALIGN256(q40_nib_bytes(rows, cols)));
  m.rows = rows;
  m.nb = (int)(cols / 32);
  return m;
}

struct Q6Mat {
  const uint4* qa;       // [rows][nseg]
  const uint2* qb;       // [rows][nseg]
  const int8_t* sc;      // [rows][ngrp]
  const uint16_t* d;     // [rows][nsb]
  int64_t rows;
  int nseg;              // cols / 32
};

static inline Q6Mat q6_view(const void* packed, int64_t rows, int64_t cols) {
  const Q6Planes P = q6k_planes(rows, cols);
  const uint8_t* b = (const uint8_t*)packed;
  Q6Mat m;
  m.qa = (const uint4*)(b + P.qa);
  m.qb = (const uint2*)(b + P.qb);
  m.sc = (const int8_t*)(b + P.sc);
  m.d = (const uint16_t*)(b + P.d);
  m.rows = rows;
  m.nseg = (int)(cols / 32);
  return m;
}

// Per-device library workspace (argmax and attention partials, x staging).
// Grow-only: a call that needs more than the current capacity allocates a
// larger buffer (never while `st` is being captured into a graph: that is an
// error) and keeps the old one until the process ends, so work already
// queued or captured with the old address stays valid.
struct Workspace {
  uint8_t* buf;          // general scratch
  size_t cap;
};
int e4b_workspace(size_t bytes, Workspace* ws, hipStream_t st);

// q4_0 GEMV epilogues
enum GemvEpi {
  EPI_F32 = 0,       // y[ks * rows + row] = dot                       (partials when KS > 1)
  EPI_GEGLU = 1,     // rows [0,FF) gate, [FF,2FF) up: yh[i] = f16(gelu(g_i) * u_i)
  EPI_GELU_MUL = 2,  // yh[row] = f16(gelu(dot) * mul[row])
};
struct GemvOut {
  float* y;          // EPI_F32 output (KS slices of `rows` each)
  uint16_t* yh;      // f16 output of EPI_GEGLU / EPI_GELU_MUL
  const float* mul;  // EPI_GELU_MUL multiplier
  int64_t ff;        // EPI_GEGLU: rows per half
};

// Optional fused input prologue of a q4_0 GEMV (q40_kernel.h), one of:
//  * residual + norm: h = (hin + rms(a) * w1) * scale (a may be null: h =
//    hin * scale), x = w2 ? f16(rms(h) * w2) : f16(h); block (0,0) stores h
//    to hout; a is the sum of `na` partial vectors a[s*H + i] (s < na <= 8).
//    H = cols must be 256, 512, 1024 or 2048.
//  * attention combine (part_o != null): x = the log-sum-exp merge of the
//    split-K partials of the live chunks of the current position, f16, for
//    an o projection of 2048 columns (8 heads of 256).
constexpr int kMaxPartials = 8;
constexpr int kProAttnH = 2048;  // columns of an o projection with the attention prologue (8 heads of 256)
constexpr int kProAttnMaxChunks = 64;  // split-K chunks per head the attention prologue merges (one lane each)
struct ProArgs {
  const float* hin;
  float* hout;       // may be null
  float* hsnap;      // may be null: block (0,0) also stores h here (the per-layer readout)
  const float* a;    // may be null
  const float* w1;
  const float* w2;   // may be null
  float scale;
  int H;
  float eps;
  int na;            // partial vectors summed into a (0 -> 1)
  // attention combine
  const float* part_o;     // [heads][gch][256]
  const float* part_ml;    // [heads][gch][2]
  const uint32_t* params;  // params[0] = position
  int kv_idx;              // full layers: params[kv_idx] = the token's slot (0: the position)
  int window;              // 0 = global layer
  int chunk_shift;         // log2 of the positions per chunk
  int gch;                 // chunks allocated per head
  int head_dim;            // 256 or 512 (0: 256); with ks column slices of 4 heads each
  // A4B layer boundary (tail != 0; any H <= 3072 divisible by 4): the
  // previous layer's MoE tail, then this layer's input norm:
  //   h = (hin + rms(rms(a) w1 + rms(a2) w1b) wp) * scale; x = f16(rms(h) w2)
  // a == null (the first layer): h = hin * scale
  int tail;
  const float* a2;
  const float* w1b;
  const float* wp;
};
bool q40_prologue_supported(int H);

// launchers (q4_0 in k_q40.hip, the rest in k_gemv.hip); all asynchronous on `st`
// ks > 1 splits the columns into ks equal slices (cols/32 divisible by ks)
// and writes ks partial vectors (EPI_F32 only).  pro != null replaces the
// f16 input xh by the fused prologue (cols must equal pro->H).
// batched q4_0 GEMM on the matrix cores (k_gemm.hip): Y f32 [M][rows], or
// with Yh the GeGLU over [gate; up] rows to f16 [M][ff]
int launch_q40_gemm(const Q40Mat& W, const uint16_t* X, int M, float* Y, uint16_t* Yh, int64_t ff, hipStream_t st);
enum GemmEpi {
  GEMM_F32 = 0,       // Y[(z M + m) rows + n]: split-K slice z of ks (ks = 1: the product)
  GEMM_GLU = 1,       // rows [0,ff) gate, [ff,2ff) up: Yh[m ff + i] = f16(gelu(g) * u)
  GEMM_GELU_MUL = 2,  // Yh[m rows + n] = f16(gelu(y) * mul[m mul_ld + n])
};
struct GemmArgs {
  Q40Mat W;
  const uint16_t* X;  // f16 [M][ldx], 16-byte aligned rows
  int M, ldx;
  int epi;
  float* Y;
  uint16_t* Yh;
  int64_t ff;
  const float* mul;
  int64_t mul_ld;
  int ks;             // split-K slices (GEMM_F32)
  // grouped mode (the expert-indexed MoE prefill; tiles != null): blockIdx.y
  // picks tiles[y] = (group g, first row r0, rows n <= 32) of the M sorted
  // rows, y < *ntiles; the weights are rows [g group_rows, (g+1) group_rows)
  // of W (GLU: group_rows = 2 ff, gate then up); X row r is gather[r] /
  // gather_div (gather null: row r); outputs are rows r0 .. r0 + n - 1 of an
  // [M][group_rows] (GLU: [M][ff]) matrix
  const int4* tiles;
  const int* ntiles;
  int max_tiles;
  int64_t group_rows;
  const uint32_t* gather;
  int gather_div;
};
int launch_q40_gemm(const GemmArgs& a, hipStream_t st);
// the largest split-K slice count <= want that cuts nb blocks into whole
// slices (what GemmArgs::ks must be)
int q40_gemm_kslices(int nb, int want);
int launch_q40(const Q40Mat& W, const uint32_t* xh, const uint32_t* xl, int epi, const GemvOut& o, int ks,
               hipStream_t st, const ProArgs* pro = nullptr);
int launch_q40_gemv(const Q40Mat& W, const uint32_t* xh, const uint32_t* xl, float* y, hipStream_t st);
int launch_split_f32(const float* x, int64_t n, uint16_t* hi, uint16_t* lo, hipStream_t st);
// part: one (index, value) partial per block (<= 2048); amax may be NULL to
// leave the fold to the caller (k_amax_final semantics)
int q6k_gemv_grid(int64_t rows, int nseg);  // number of argmax partials the lm-head writes (nseg = cols / 32)
int launch_q6k_gemv_argmax(const Q6Mat& W, const uint32_t* xh, const uint32_t* xl, float softcap,
                           float* logits, uint32_t* amax, uint2* part, hipStream_t st);
int launch_q6k_row(const Q6Mat& W, int64_t row, const uint32_t* row_dev, float mult, float* out, hipStream_t st);
int launch_argmax(const float* x, int64_t n, uint32_t* amax, uint2* part, hipStream_t st);
