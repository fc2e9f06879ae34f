// k_gemm.hip -- q4_0 weight x f16 activation GEMM on the gfx950 matrix cores,
// the batched-prefill counterpart of the decode GEMV (src/engine-a4b.js:465-585
// runs its prefill as multi-column GEMVs, kernels/q40mm.wgsl /
// kernels/q40sg.wgsl; here it is an MFMA GEMM).
//
//   Y[m][n] = sum_k X[m][k] W[n][k],  W q4_0 [N][K] (repacked planes),
//   X f16 [M][K] row-major (row stride ldx), Y f32 [M][N]; epilogues: split-K
//   partial slices (Y + z M N, summed by the consumer), the GeGLU over
//   W = [gate; up] to f16 [M][FF] = gelu(gate) * up, or f16 gelu(y) * mul.
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
// Workgroup: 4 waves x 32 output columns (GeGLU: a gate and an up tile), T
// token tiles of 32 per wave.  Per stage of KBL blocks (128 k) the weight
// tile (128 rows; GeGLU 256), its block scales and the activations of the
// workgroup's 32 T tokens are staged in LDS with row-contiguous cooperative
// loads and shared by the 4 waves; the next stage is requested into
// registers before the current stage's MFMAs.  blockIdx.z selects a split-K
// slice.  Row tiles are blockIdx.x, so the workgroups that share a weight
// tile (same x, different token tiles) sit a multiple of 8 apart in dispatch
// order when the row-tile count is a multiple of 8: the same XCD and its L2.
#include "../../include/e4b.h"
#include "kernels.h"
#include "util.h"

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16v __attribute__((ext_vector_type(16)));
// staged 16-byte pieces as a native vector: an array of HIP's uint4 struct
// kept across the K loop is not split into registers (it stays in scratch,
// and the next stage's loads are waited for before the current MFMAs;
// measured 1.55x slower on the expert-grouped GEMMs)
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
// the prefetch registers of a stage: native vectors, except in the widest
// GeGLU tile (4 token tiles x 2 x 32 rows per wave), whose accumulators and
// operands already take 256 VGPRs.  There the uint4 struct array is what the
// compiler moves to LDS (16 KB per workgroup), which keeps 2 waves per SIMD
// (the native vectors in registers leave 1 wave: the E4B prefill measured
// 16 % slower)
template <int T, int EPI>
using StageVec = std::conditional_t<T == 4 && EPI == GEMM_GLU, uint4, u32x4>;
DEV u32x4 as_vec(u32x4 v) { return v; }
DEV u32x4 as_vec(const uint4& v) { return u32x4{v.x, v.y, v.z, v.w}; }

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

// The weight tile is loaded cooperatively, KBL contiguous blocks (64 bytes)
// per row and thread group -- a wave that loaded its own B fragments would
// touch 32 rows with 16 bytes each per instruction, which measured 1.5-2.3x
// slower -- and each stage's loads overlap the previous stage's math.
constexpr int KBL = 4;            // q4_0 blocks per stage (128 k); split-K slices are multiples of it

// KB blocks per stage (KBL, or 8 for the grouped expert GEMMs: their weight
// rows are read once per 32-row tile, and 8 blocks make each row's stage
// one whole 128-byte line)
template <int T, int EPI, bool GRP, int KB = KBL>
__global__ __launch_bounds__(256) void k_q40_gemm_lds(GemmArgs a, int K, int nbs) {
  constexpr int KBL = KB;
  constexpr int WSL = KBL + 1;      // 16-byte pieces per staged weight row (+1 pad: conflict-free 16-byte reads)
  constexpr int SSL = KBL + 2;      // f16 scales per staged row (+2 pad)
  constexpr int XSL = KBL * 4 + 1;  // 16-byte pieces per staged token row (+1 pad)
  static_assert(KBL == 4 || KBL == 8, "4 or 8 blocks per stage");
  constexpr int NT = EPI == GEMM_GLU ? 2 : 1;
  constexpr int TOK = 32 * T;
  constexpr int RW = 128 * NT;                 // staged weight rows
  constexpr int WP = RW * KBL / 256;           // nibble pieces per thread and stage
  constexpr int SP = RW * KBL / 256;           // scales per thread and stage
  constexpr int XP = TOK * KBL * 4 / 256;      // activation pieces per thread and stage
  static_assert(WP >= 1 && SP >= 1 && XP >= 1, "whole pieces per thread");
  __shared__ __align__(16) StageVec<T, EPI> wl[RW][WSL];
  __shared__ uint16_t sl[RW][SSL];
  __shared__ __align__(16) StageVec<T, EPI> xs[TOK][XSL];
  const Q40Mat& W = a.W;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l32 = lane & 31, hi = lane >> 5;
  const int nb = K / 32;
  const int M = a.M;
  const int64_t units = EPI == GEMM_GLU ? a.ff : (GRP ? a.group_rows : W.rows);
  int tok0, nrows;
  int64_t wbase = 0;
  if constexpr (GRP) {
    if ((int)blockIdx.y >= *a.ntiles) return;  // the grid is sized for the most tiles
    const int4 tl = a.tiles[blockIdx.y];
    wbase = (int64_t)tl.x * a.group_rows;
    tok0 = tl.y;
    nrows = tl.z;
  } else {
    tok0 = blockIdx.y * TOK;
    nrows = M - tok0;
  }
  const int64_t c0 = (int64_t)blockIdx.x * 128;  // first output column of the workgroup
  const int kz = blockIdx.z;
  const int kbeg = kz * nbs, kend = min(nb, kbeg + nbs);
  // global weight row of staged row r (clamped: rows past the end are loaded
  // from a valid row and never stored)
  auto grow = [&](int r) -> int64_t {
    if constexpr (EPI == GEMM_GLU)
      return wbase + (r >= 128 ? a.ff : 0) + min(c0 + (r & 127), units - 1);
    else
      return wbase + min(c0 + r, units - 1);
  };
  // activation row and validity of this thread's XP pieces: fixed for the
  // whole K loop (grouped mode: the gathered row index, one load and one
  // division per piece here instead of a dependent load chain per stage)
  int64_t xrow_of[XP];
  bool mrow_in[XP];
#pragma unroll
  for (int j = 0; j < XP; ++j) {
    const int m = (threadIdx.x + 256 * j) / (KBL * 4);
    mrow_in[j] = m < nrows;
    int64_t xrow = tok0 + m;
    if constexpr (GRP) xrow = a.gather ? (int64_t)(a.gather[mrow_in[j] ? xrow : tok0] / (uint32_t)a.gather_div) : xrow;
    xrow_of[j] = xrow;
  }
  StageVec<T, EPI> wr[WP];
  uint16_t sr[SP];
  StageVec<T, EPI> xr[XP];
  auto issue = [&](int kb0) {
#pragma unroll
    for (int j = 0; j < WP; ++j) {
      const int p = threadIdx.x + 256 * j;
      const int r = p / KBL, b = p % KBL;
      const uint32_t e = (uint32_t)grow(r) * (uint32_t)nb + (uint32_t)min(kb0 + b, nb - 1);
      wr[j] = *reinterpret_cast<const StageVec<T, EPI>*>(reinterpret_cast<const char*>(W.nib) + e * 16u);
    }
#pragma unroll
    for (int j = 0; j < SP; ++j) {
      const int q = threadIdx.x + 256 * j;
      const int r = q / KBL, b = q % KBL;
      // blocks past the row end repeat the last block's scale (they meet zero activations)
      const uint32_t e = (uint32_t)grow(r) * (uint32_t)nb + (uint32_t)min(kb0 + b, nb - 1);
      sr[j] = W.sc[e];
    }
#pragma unroll
    for (int j = 0; j < XP; ++j) {
      const int q = (threadIdx.x + 256 * j) % (KBL * 4);
      const int kq = kb0 * 32 + q * 8;
      const bool in = mrow_in[j] && kq < kend * 32;
      const StageVec<T, EPI> v = *reinterpret_cast<const StageVec<T, EPI>*>(a.X + (in ? xrow_of[j] * a.ldx + kq : 0));
      xr[j] = in ? v : StageVec<T, EPI>{};
    }
  };
  auto store = [&]() {
#pragma unroll
    for (int j = 0; j < WP; ++j) {
      const int p = threadIdx.x + 256 * j;
      wl[p / KBL][p % KBL] = wr[j];
    }
#pragma unroll
    for (int j = 0; j < SP; ++j) {
      const int q = threadIdx.x + 256 * j;
      sl[q / KBL][q % KBL] = sr[j];
    }
#pragma unroll
    for (int j = 0; j < XP; ++j) {
      const int i = threadIdx.x + 256 * j;
      xs[i / (KBL * 4)][i % (KBL * 4)] = xr[j];
    }
  };

  f16v acc[NT][T];
#pragma unroll
  for (int u = 0; u < NT; ++u)
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[u][t][r] = 0.f;
  // this wave's staged rows: tile u = rows 128 u + 32 wave + l32
  int lrow[NT];
#pragma unroll
  for (int u = 0; u < NT; ++u) lrow[u] = 128 * u + 32 * wave + l32;

  issue(kbeg);
  store();
  lds_sync();
  for (int kb0 = kbeg; kb0 < kend; kb0 += KBL) {
    // the next stage (the last iteration repeats its own, unused): the loop
    // body stays one basic block
    issue(kb0 + KBL < kend ? kb0 + KBL : kb0);
#pragma unroll
    for (int b = 0; b < KBL; ++b) {
      h8 bw[NT][2];
      float dsc[NT];
#pragma unroll
      for (int u = 0; u < NT; ++u) {
        const u32x4 w4 = as_vec(wl[lrow[u]][b]);
        bw[u][0] = nib_word_f16(hi ? w4.y : w4.x);
        bw[u][1] = nib_word_f16(hi ? w4.w : w4.z);
        dsc[u] = h2f(sl[lrow[u]][b]);
      }
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const u32x4 a0 = as_vec(xs[32 * t + l32][4 * b + hi]);
        const u32x4 a1 = as_vec(xs[32 * t + l32][4 * b + 2 + hi]);
        const h8 av0 = __builtin_bit_cast(h8, a0), av1 = __builtin_bit_cast(h8, a1);
#pragma unroll
        for (int u = 0; u < NT; ++u) {
          f16v d = {};
          d = __builtin_amdgcn_mfma_f32_32x32x16_f16(av0, bw[u][0], d, 0, 0, 0);
          d = __builtin_amdgcn_mfma_f32_32x32x16_f16(av1, bw[u][1], d, 0, 0, 0);
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[u][t][r] = fmaf(dsc[u], d[r], acc[u][t][r]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    lds_sync();
    store();
    lds_sync();
  }
  // store: lane owns column c0 + 32 wave + l32, tokens 32 t + 8 (r / 4) + 4 hi + r % 4
  const int64_t n = c0 + 32 * wave + l32;
  if (n >= units) return;
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int ml = 32 * t + 8 * (r / 4) + 4 * hi + (r % 4);
      const int m = tok0 + ml;
      if (ml < nrows) {
        if constexpr (EPI == GEMM_GLU)
          a.Yh[(int64_t)m * a.ff + n] = f2h(gelu_tanh(acc[0][t][r]) * acc[1][t][r]);
        else if constexpr (EPI == GEMM_GELU_MUL)
          a.Yh[(int64_t)m * units + n] = f2h(gelu_tanh(acc[0][t][r]) * a.mul[(int64_t)m * a.mul_ld + n]);
        else
          a.Y[((int64_t)kz * M + m) * units + n] = acc[0][t][r];
      }
    }
}

template <int EPI>
void launch_t(int T, const GemmArgs& a, dim3 grid, int K, int nbs, hipStream_t st) {
  if (a.tiles) {
    hipLaunchKernelGGL((k_q40_gemm_lds<1, EPI, true, 8>), grid, dim3(256), 0, st, a, K, nbs);
    return;
  }
  if (T == 4)
    hipLaunchKernelGGL((k_q40_gemm_lds<4, EPI, false>), grid, dim3(256), 0, st, a, K, nbs);
  else if (T == 2)
    hipLaunchKernelGGL((k_q40_gemm_lds<2, EPI, false>), grid, dim3(256), 0, st, a, K, nbs);
  else
    hipLaunchKernelGGL((k_q40_gemm_lds<1, EPI, false>), grid, dim3(256), 0, st, a, K, nbs);
}

}  // namespace

int q40_gemm_kslices(int nb, int want) {
  for (int ks = want < 1 ? 1 : want; ks > 1; --ks) {
    const int nbs = ((nb + ks - 1) / ks + KBL - 1) / KBL * KBL;
    if ((nb + nbs - 1) / nbs == ks) return ks;
  }
  return 1;
}

int launch_q40_gemm(const GemmArgs& a, hipStream_t st) {
  const Q40Mat& W = a.W;
  const int K = W.nb * 32;
  if (a.M < 1 || K < 32) return e4b_fail(E4B_EINVAL, "q4_0 GEMM: empty operand (M=%d K=%d)", a.M, K);
  if ((uint64_t)W.rows * (uint64_t)W.nb * 16u > 0xffffffffull)
    return e4b_fail(E4B_EINVAL, "q4_0 GEMM: a %lld x %d-block matrix exceeds the 4 GiB plane limit",
                    (long long)W.rows, W.nb);
  if (a.ldx < K || a.ldx % 8) return e4b_fail(E4B_EINVAL, "q4_0 GEMM: x row stride %d (>= %d, multiple of 8)", a.ldx, K);
  const int ks = a.ks > 0 ? a.ks : 1;
  if (ks > 1 && a.epi != GEMM_F32) return e4b_fail(E4B_EINVAL, "q4_0 GEMM: split-K needs the f32 epilogue");
  if (ks > W.nb) return e4b_fail(E4B_EINVAL, "q4_0 GEMM: %d K slices for %d blocks", ks, W.nb);
  const bool grp = a.tiles != nullptr;
  if (grp && (!a.ntiles || a.max_tiles < 1 || a.group_rows < 1 || W.rows % a.group_rows || ks != 1 ||
              (a.gather && a.gather_div < 1)))
    return e4b_fail(E4B_EINVAL, "q4_0 GEMM: bad grouped-mode arguments");
  int64_t units = grp ? a.group_rows : W.rows;
  switch (a.epi) {
    case GEMM_F32:
      if (!a.Y) return e4b_fail(E4B_EINVAL, "q4_0 GEMM: null output");
      break;
    case GEMM_GLU:
      if (!a.Yh || a.ff < 1 || 2 * a.ff != (grp ? a.group_rows : W.rows))
        return e4b_fail(E4B_EINVAL, "q4_0 GEMM: GeGLU needs 2*ff rows");
      units = a.ff;
      break;
    case GEMM_GELU_MUL:
      if (!a.Yh || !a.mul) return e4b_fail(E4B_EINVAL, "q4_0 GEMM: GELU-multiply needs yh and mul");
      break;
    default: return e4b_fail(E4B_EINVAL, "q4_0 GEMM: epilogue %d", a.epi);
  }
  // blocks per split-K slice, a multiple of the LDS stage; the consumer sums
  // exactly `ks` slices, so every slice must hold blocks
  const int nbs = ((W.nb + ks - 1) / ks + KBL - 1) / KBL * KBL;
  const int kslices = (W.nb + nbs - 1) / nbs;
  if (kslices != ks)
    return e4b_fail(E4B_EINVAL, "q4_0 GEMM: %d blocks do not split into %d slices (use q40_gemm_kslices)", W.nb, ks);
  // the widest token tile (4 x 32 tokens per wave: the weight-word
  // conversion is shared by 4 MFMA pairs) that still gives >= 512 workgroups
  // (two per CU: a stage's load latency is hidden by the other workgroup's
  // MFMAs; measured best for the E4B prefill shapes at 512 tokens)
  const int64_t rt = (units + 127) / 128;
  int T = 4;
  while (T > 1 && rt * ((a.M + 32 * T - 1) / (32 * T)) * kslices < 512) T >>= 1;
  if (grp) T = 1;  // tiles of <= 32 rows
  const unsigned gy = grp ? (unsigned)a.max_tiles : (unsigned)((a.M + 32 * T - 1) / (32 * T));
  const dim3 grid((unsigned)rt, gy, (unsigned)kslices);
  if (a.epi == GEMM_GLU)
    launch_t<GEMM_GLU>(T, a, grid, K, nbs, st);
  else if (a.epi == GEMM_GELU_MUL)
    launch_t<GEMM_GELU_MUL>(T, a, grid, K, nbs, st);
  else
    launch_t<GEMM_F32>(T, a, grid, K, nbs, st);
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}

int launch_q40_gemm(const Q40Mat& W, const uint16_t* X, int M, float* Y, uint16_t* Yh, int64_t ff, hipStream_t st) {
  GemmArgs a{};
  a.W = W;
  a.X = X;
  a.M = M;
  a.ldx = W.nb * 32;
  a.epi = Yh ? GEMM_GLU : GEMM_F32;
  a.Y = Y;
  a.Yh = Yh;
  a.ff = ff;
  a.ks = 1;
  return launch_q40_gemm(a, st);
}
