// k_q40.hip -- q4_0 GEMV entry point: validates the request, picks the lane
// split / rows per group / column split, and hands over to the translation
// unit that instantiates the matching kernel variant (k_q40_*.hip).
#include "../../include/e4b.h"
#include "q40_kernel.h"
#include "util.h"

bool q40_prologue_supported(int H) { return H == 256 || H == 512 || H == 1024 || H == 2048; }

int launch_q40(const Q40Mat& W, const uint32_t* xh, const uint32_t* xl, int epi, const GemvOut& o, int ks,
               hipStream_t st, const ProArgs* pro) {
  if (epi != EPI_F32 && epi != EPI_GEGLU && epi != EPI_GELU_MUL)
    return e4b_fail(E4B_EINVAL, "q4_0 GEMV: unknown epilogue %d", epi);
  if (ks < 1 || W.nb % ks) return e4b_fail(E4B_EINVAL, "q4_0 GEMV: %d blocks per row not divisible by ks=%d", W.nb, ks);
  if (ks > 1 && epi != EPI_F32) return e4b_fail(E4B_EINVAL, "q4_0 GEMV: column split needs the f32 epilogue");
  if (xl && epi != EPI_F32) return e4b_fail(E4B_EINVAL, "q4_0 GEMV: hi/lo input needs the f32 epilogue");
  if (epi == EPI_GEGLU && (o.ff < 1 || 2 * o.ff != W.rows))
    return e4b_fail(E4B_EINVAL, "q4_0 GEMV: GeGLU needs 2*ff rows (rows=%lld ff=%lld)", (long long)W.rows,
                    (long long)o.ff);
  if ((uint64_t)W.rows * (uint64_t)W.nb * 16u > 0xffffffffull)
    return e4b_fail(E4B_EINVAL, "q4_0 GEMV: a %lld x %d-block matrix exceeds the 4 GiB plane limit", (long long)W.rows,
                    W.nb);
  const int nbk = W.nb / ks;
  if (nbk < 1) return e4b_fail(E4B_EINVAL, "q4_0 GEMV: empty row");
  if (W.nb > 0xffff)  // the kernels take nb and nbk packed in 16 bits each (Q40_LEAD_PARAMS)
    return e4b_fail(E4B_EINVAL, "q4_0 GEMV: %d blocks per row exceeds 65535", W.nb);
  if (pro && pro->part_o) {
    // one slice of 8 heads of 256 (ks = 1) or ks slices of 4 heads of 256 or 512
    const int hd = pro->head_dim ? pro->head_dim : 256;
    const bool shape = ks == 1 ? (hd == 256 && W.nb * 32 == kProAttnH) : ((hd == 256 || hd == 512) && nbk * 32 == 4 * hd);
    if (xl || !shape || epi != EPI_F32 || !pro->part_ml || !pro->params || pro->chunk_shift < 0 ||
        pro->chunk_shift > 10 || pro->gch < 1 || pro->gch > q40k::kProAttnMaxCh)
      return e4b_fail(E4B_EINVAL, "q4_0 GEMV: the attention prologue needs 8 heads of 256 columns or slices of 4 "
                      "heads of 256 or 512 (got %d columns, %d slices, head dim %d)", W.nb * 32, ks, hd);
  } else if (pro && pro->tail) {
    if (xl || ks != 1 || epi != EPI_F32 || pro->H != W.nb * 32 || pro->H % 4 || pro->H > q40k::kProTailMaxH ||
        !pro->hin || !pro->w2 || (pro->a && (!pro->a2 || !pro->w1 || !pro->w1b || !pro->wp)))
      return e4b_fail(E4B_EINVAL, "q4_0 GEMV: the layer-boundary prologue needs an f32 GEMV of H <= %d columns "
                      "(multiple of 4; got %d) and all its vectors", q40k::kProTailMaxH, W.nb * 32);
  } else if (pro && (xl || ks != 1 || pro->H != W.nb * 32 || !q40_prologue_supported(pro->H) || !pro->hin ||
                     (pro->a && !pro->w1) ||
                     (pro->na > 1 && !((pro->na == kMaxPartials && epi == EPI_F32) || (pro->na == 2 && epi == EPI_GEGLU))))) {
    return e4b_fail(E4B_EINVAL, "q4_0 GEMV: prologue needs f16 input of a full 256/512/1024/2048 row (H=%d, cols=%d)",
                    pro ? pro->H : 0, W.nb * 32);
  }
  q40k::Launch L;
  L.W = W;
  L.xh = xh;
  L.xl = xl;
  L.o = o;
  L.units = (epi == EPI_GEGLU) ? 2 * o.ff : W.rows;
  L.ks = ks;
  L.nbk = nbk;
  L.pa = pro ? *pro : ProArgs{};
  L.st = st;
  q40k::Cfg c = q40k::pick(nbk, L.units, epi, pro != nullptr, ks, pro && pro->part_o);
  if (pro && pro->tail) {
    // lanes: one block each up to 64-block rows, else 32 lanes x 2-3 blocks
    // (H <= 3072); every workgroup repeats the prologue's seven vector
    // reads, so tiles grow (up to 4 rows per lane group) while >= 256
    // workgroups remain
    c.kw = 1;
    c.nwv = 4;
    c.lpr = nbk <= 8 ? 8 : nbk <= 16 ? 16 : nbk <= 32 ? 32 : nbk <= 64 ? 64 : 32;
    c.bpl = nbk <= 64 ? 1 : (nbk + 31) / 32;
    c.r = 1;
    const int64_t per_wg = 4 * (64 / c.lpr);
#ifndef E4B_TUNE_TAIL_MINWGS
#define E4B_TUNE_TAIL_MINWGS 256
#endif
#ifdef E4B_TUNE_TAIL_R8
    constexpr int rmax = 8;
#else
    constexpr int rmax = 4;
#endif
    while (c.r < rmax && (L.units + per_wg * 2 * c.r - 1) / (per_wg * 2 * c.r) >= E4B_TUNE_TAIL_MINWGS) c.r *= 2;
  }
  if (c.bpl > 8 || c.lpr * c.bpl * c.kw < nbk)
    return e4b_fail(E4B_EINVAL, "q4_0 GEMV: %d blocks per slice exceeds the 2048-block (65536-column) maximum", nbk);
  bool ok;
  if (pro)
    ok = q40k::dispatch_pro(c, L, epi);
  else if (c.kw == 4)
    ok = q40k::dispatch_kw4(c, L, epi);
  else if (epi != EPI_F32)
    ok = q40k::dispatch_glu(c, L, epi);
  else
    ok = xl ? q40k::dispatch_f32_hl(c, L) : q40k::dispatch_f32(c, L);
  if (!ok) return e4b_fail(E4B_EINVAL, "q4_0 GEMV: no kernel for epi=%d lpr=%d bpl=%d r=%d kw=%d", epi, c.lpr, c.bpl, c.r, c.kw);
  E4B_HIP(hipGetLastError());
  return E4B_OK;
}

int launch_q40_gemv(const Q40Mat& W, const uint32_t* xh, const uint32_t* xl, float* y, hipStream_t st) {
  GemvOut o = {y, nullptr, nullptr, 0};
  return launch_q40(W, xh, xl, EPI_F32, o, 1, st, nullptr);
}
