// k_gemm.hip -- q4_0 weight x f16 activation GEMM on the gfx950 matrix cores,
// the batched-prefill counterpart of the decode GEMV (src/engine-a4b.js:465-585
// runs its prefill as multi-column GEMVs, kernels/q40mm.wgsl /
// kernels/q40sg.wgsl; here it is an MFMA GEMM).
//
//   Y[m][n] = sum_k X[m][k] W[n][k],  W q4_0 [N][K] (repacked planes),
//   X f16 [M][K] row-major, Y f32 [M][N] (or, with the GeGLU epilogue over
//   W = [gate; up], f16 [M][FF] = gelu(gate) * up).
//
// v_mfma_f32_32x32x16_f16 with A = a 32-token x 16-k slice of X and B = the
// 16-k x 32-row slice of W^T: lane l holds A[l % 32][8 (l / 32) + t] (t < 8),
// B[8 (l / 32) + t][l % 32] and D[8 (r / 4) + 4 (l / 32) + r % 4][l % 32]
// (r < 16), so every lane owns one weight row n = l % 32 of the tile.  B
// comes straight from the repacked nibble words: word 2s + l / 32 of a block
// holds the 8 elements step s needs, turned into the exact f16 values n - 8
// (the pattern 0x6400 | n is the f16 1024 + n; subtracting 1032 leaves
// n - 8).  Each q4_0 block (two K steps) is accumulated from zero and then
// scaled by the row's block scale, as the decode GEMV does, so the products
// are exact and only the f32 summation order differs.
//
// Workgroup: 4 waves x 32 rows (x2 for GeGLU: gate and up tiles), T token
// tiles of 32 per wave; the X slice of KB blocks for the workgroup's 32 T
// tokens is staged in LDS and shared by the 4 waves.
#include "../../include/e4b.h"
#include "kernels.h"
#include "util.h"

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16v __attribute__((ext_vector_type(16)));

constexpr int KB = 2;  // q4_0 blocks per LDS stage (64 k)

// 8 exact f16 values (n - 8) of one repacked nibble word, in element order
DEV h8 nib_word_f16(uint32_t w) {
  const uint32_t M = 0x000F000Fu, MAG = 0x64006400u;
  uint32_t p[4] = {(w & M) | MAG, ((w >> 8) & M) | MAG, ((w >> 4) & M) | MAG, ((w >> 12) & M) | MAG};
  h8 r;
  const _Float16 off = (_Float16)1032.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const auto v = __builtin_bit_cast(_Float16 __attribute__((ext_vector_type(2))), p[i]);
    r[2 * i] = v[0] - off;
    r[2 * i + 1] = v[1] - off;
  }
  return r;
}

template <int T, bool GLU>
__global__ __launch_bounds__(256) void k_q40_gemm(Q40Mat W, const uint16_t* __restrict__ X, int M, int K,
                                                   float* __restrict__ Y, uint16_t* __restrict__ Yh, int64_t ff) {
  constexpr int NT = GLU ? 2 : 1;          // weight tiles per wave (gate, up)
  constexpr int TOK = 32 * T;              // tokens per workgroup
  __shared__ __align__(16) uint4 xs[TOK][KB * 4];  // KB blocks x 64 B per token
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l32 = lane & 31, hi = lane >> 5;
  const int nb = K / 32;
  const int64_t rows = W.rows;
  const int64_t units = GLU ? ff : rows;   // output columns
  const int64_t n0 = ((int64_t)blockIdx.x * 4 + wave) * 32;  // first output column of this wave
  const int tok0 = blockIdx.y * TOK;
  // this lane's weight rows (clamped: tiles past the end compute duplicates, never stored)
  int64_t wrow[NT];
  wrow[0] = min(n0 + l32, units - 1);
  if constexpr (GLU) wrow[1] = ff + wrow[0];
  f16v acc[NT][T];
#pragma unroll
  for (int u = 0; u < NT; ++u)
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[u][t][r] = 0.f;

  for (int kb0 = 0; kb0 < nb; kb0 += KB) {
    // stage X[tok0 .. tok0+TOK)[32 kb0 .. 32 (kb0+KB)) (zeros past M or K)
    for (int i = threadIdx.x; i < TOK * KB * 4; i += 256) {
      const int m = i / (KB * 4), q = i % (KB * 4);
      const int kq = kb0 * 32 + q * 8;  // first k of this 16-byte piece
      uint4 v = make_uint4(0u, 0u, 0u, 0u);
      if (tok0 + m < M && kq < K) v = *reinterpret_cast<const uint4*>(X + (int64_t)(tok0 + m) * K + kq);
      xs[m][q] = v;
    }
    // this lane's weight words and scales for the stage
    uint32_t wv[NT][KB][2];
    float dsc[NT][KB];
#pragma unroll
    for (int u = 0; u < NT; ++u)
#pragma unroll
      for (int b = 0; b < KB; ++b) {
        const int kb = min(kb0 + b, nb - 1);
        const uint32_t e = (uint32_t)wrow[u] * (uint32_t)nb + (uint32_t)kb;
        const uint4 w4 = ld_nt_u4_off(W.nib, e);
        wv[u][b][0] = hi ? w4.y : w4.x;  // step 0: word (l / 32)
        wv[u][b][1] = hi ? w4.w : w4.z;  // step 1: word 2 + (l / 32)
        dsc[u][b] = kb0 + b < nb ? scale_of(ld_scale_pair_off(W.sc, e), e & 1) : 0.f;
      }
    lds_sync();
#pragma unroll
    for (int b = 0; b < KB; ++b) {
      h8 bw[NT][2];
#pragma unroll
      for (int u = 0; u < NT; ++u) {
        bw[u][0] = nib_word_f16(wv[u][b][0]);
        bw[u][1] = nib_word_f16(wv[u][b][1]);
      }
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const uint4 a0 = xs[32 * t + l32][4 * b + hi];
        const uint4 a1 = xs[32 * t + l32][4 * b + 2 + hi];
        const h8 av0 = __builtin_bit_cast(h8, a0), av1 = __builtin_bit_cast(h8, a1);
#pragma unroll
        for (int u = 0; u < NT; ++u) {
          f16v d = {};
          d = __builtin_amdgcn_mfma_f32_32x32x16_f16(av0, bw[u][0], d, 0, 0, 0);
          d = __builtin_amdgcn_mfma_f32_32x32x16_f16(av1, bw[u][1], d, 0, 0, 0);
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[u][t][r] = fmaf(dsc[u][b], d[r], acc[u][t][r]);
        }
      }
    }
    lds_sync();
  }
  // store: lane owns column n0 + l32, tokens 32 t + 8 (r / 4) + 4 hi + r % 4
  const int64_t n = n0 + l32;
  if (n >= units) return;
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = tok0 + 32 * t + 8 * (r / 4) + 4 * hi + (r % 4);
      if (m < M) {
        if constexpr (GLU)
          Yh[(int64_t)m * ff + n] = f2h(gelu_tanh(acc[0][t][r]) * acc[1][t][r]);
        else
          Y[(int64_t)m * rows + n] = acc[0][t][r];
      }
    }
}

}  // namespace

int launch_q40_gemm(const Q40Mat& W, const uint16_t* X, int M, float* Y, uint16_t* Yh, int64_t ff, hipStream_t st) {
  const int K = W.nb * 32;
  if (M < 1 || K < 32) return e4b_fail(E4B_EINVAL, "q4_0 GEMM: empty operand (M=%d K=%d)", M, K);
  if ((uint64_t)W.rows * (uint64_t)W.nb * 16u > 0xffffffffull)
    return e4b_fail(E4B_EINVAL, "q4_0 GEMM: a %lld x %d-block matrix exceeds the 4 GiB plane limit",
                    (long long)W.rows, W.nb);
  const bool glu = Yh != nullptr;
  if (glu && (ff < 1 || 2 * ff != W.rows)) return e4b_fail(E4B_EINVAL, "q4_0 GEMM: GeGLU needs 2*ff rows");
  if (!glu && !Y) return e4b_fail(E4B_EINVAL, "q4_0 GEMM: null output");
  constexpr int T = 4;
  const int64_t units = glu ? ff : W.rows;
  const dim3 grid((unsigned)((units + 127) / 128), (unsigned)((M + 32 * T - 1) / (32 * T)));
  if (glu)
    hipLaunchKernelGGL((k_q40_gemm<T, true>), grid, dim3(256), 0, st, W, X, M, K, Y, Yh, ff);
  else
    hipLaunchKernelGGL((k_q40_gemm<T, false>), grid, dim3(256), 0, st, W, X, M, K, Y, Yh, ff);
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}
