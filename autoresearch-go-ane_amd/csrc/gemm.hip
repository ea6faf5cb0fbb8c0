// GEMM dispatch: tile and split-K choice, the split-K reduction and
// gemm_run().  The kernels and their launchers are in gemm_impl.h; the
// launchers of each epilogue are instantiated in one of the gemm_*.hip files.
#include "gemm_impl.h"

namespace ane {
using namespace gemm_detail;

namespace gemm_detail {
// the launchers, instantiated in the gemm_part<n>.hip files
#define ANE_GEMM_LAUNCH(AT, BT, E) \
  extern template hipError_t launch<AT, BT, E>(const GemmArgs&, const EpiParams&, hipStream_t, int, int, int, int);
#define ANE_GEMM_G1 ANE_GEMM_LAUNCH
#define ANE_GEMM_G2 ANE_GEMM_LAUNCH
#define ANE_GEMM_G3 ANE_GEMM_LAUNCH
#define ANE_GEMM_G4 ANE_GEMM_LAUNCH
#define ANE_GEMM_G5 ANE_GEMM_LAUNCH
#include "gemm_launchers.inc"
}  // namespace gemm_detail

void gemm_pick_tile(int M, int N, int K, int epi, int* pbm, int* pbn) {
  // Preference order with a minimum block count each: a tile is taken only
  // if it yields enough blocks to keep the 256 CUs (and 2-3 resident blocks
  // per CU for the smaller tiles) busy.  Thresholds come from a sweep of
  // the stories110M shapes on MI355X (M = 8192 and 4096 tokens, random
  // operands): 256x256 with 8 waves wins from 256 blocks (W1|W3 at M = 8192:
  // 925 vs 817 TFLOP/s for 128x128, at M = 4096: 953 vs 809; classifier 885
  // vs 801), 128x128 from 512 blocks (the SwiGLU-backward GEMM at M = 4096:
  // 18.0 vs 21.4 us for 128x64), 128x64 at N = 768 with K <= 2048, 64x64
  // for narrow outputs with long K.  A nonzero
  // *pbm / *pbn on entry is a constraint the chosen tile keeps (callers
  // size buffers by it).
  static const int cand[][3] = {{256, 256, 256}, {128, 128, 512}, {128, 64, 600}, {64, 128, 600},
                                {256, 128, 600},  {128, 256, 600},  {256, 64, 600}, {64, 64, 0}};
  constexpr int NCAND = 8;
  const int want_bm = *pbm, want_bn = *pbn;
  // Wide outputs that are a multiple of 192 but not of 1024 (the fused
  // Wq|Wk|Wv output, 2304 = 12 x 192): 128x192 blocks split N into whole
  // waves; measured 33.6 us vs 38.5 for 128x128 at M = 8192, 19.9 vs 21.3
  // for 128x64 at 4096
  epi = epi_base(epi);  // the deferred-norm variants tile as their plain forms
  if ((epi == EPI_STORE_H || epi == EPI_STORE_F || epi == EPI_RESID) && N % 192 == 0 && N >= 1536 && N % 1024 != 0 &&
      M % 128 == 0 && (long)(M / 128) * (N / 192) >= 384 && (!want_bm || want_bm == 128) &&
      (!want_bn || want_bn == 192)) {
    *pbm = 128;
    *pbn = 192;
    return;
  }
  int fbm = 0, fbn = 0;
  for (int c = 0; c < NCAND; c++) {
    const int bm = cand[c][0], bn = cand[c][1];
    if ((want_bm && bm != want_bm) || (want_bn && bn != want_bn)) continue;
    if (M % bm || N % bn) continue;
    if (epi == EPI_SWIGLU && bn < 128) continue;
    const long blocks = (long)(M / bm) * (N / bn);
    if (!fbm) { fbm = bm; fbn = bn; }  // first that fits, if none is big enough
    if (blocks >= cand[c][2]) {
      *pbm = bm;
      *pbn = bn;
      return;
    }
  }
  // nothing reaches its threshold: the smallest-tile choice that fits
  for (int c = NCAND - 1; c >= 0; c--) {
    const int bm = cand[c][0], bn = cand[c][1];
    if ((want_bm && bm != want_bm) || (want_bn && bn != want_bn)) continue;
    if (M % bm || N % bn || (epi == EPI_SWIGLU && bn < 128)) continue;
    fbm = bm;
    fbn = bn;
    break;
  }
  *pbm = fbm;
  *pbn = fbn;
  (void)K;
}

void gemm_pick_split(int M, int N, int K, int epi, size_t ws_cap, int* pbm, int* pbn, int* psplits) {
  // Rules from a sweep of the training shapes on MI355X (B16 x 256, so
  // K = tokens = 4096 for the weight gradients):
  //  (a) very long K (dy = dlogits Embed, K = vocab): 256x256 tiles, split
  //      so that the last round of blocks over the 256 CUs is the fullest
  //      (fewest splits on a tie): 48 tiles at B16 take 5 splits, 240
  //      blocks (204 us vs 229 for 4 splits, 192 blocks; 233 for 10);
  //  (b) long K and room for >= 256 blocks of 256x256: one pass of the big
  //      tile (classifier weight gradient: 953 vs 832 for 128x128);
  //  (c) long K with fewer than 512 blocks of the default tile (dW of
  //      Wq|Wk|Wv, Wo, W2): the largest tile and fewest splits reaching 384
  //      blocks with >= 512 k per split (Wo: 18.5 us vs 32.3; W2 28.0 vs
  //      34.6; QKV 29.3 vs 36.5).
  // Otherwise the plain heuristic, one pass.
  int bm = 0, bn = 0;
  gemm_pick_tile(M, N, K, epi, &bm, &bn);
  *pbm = bm;
  *pbn = bn;
  *psplits = 1;
  if (bm == 0 || (epi != EPI_STORE_F && epi != EPI_STORE_H && epi != EPI_STORE_W13)) return;
  auto fits = [&](int sp) { return K % (sp * BK) == 0 && (size_t)sp * M * N <= ws_cap; };
  const bool big = M % 256 == 0 && N % 256 == 0;
  const long t256 = big ? (long)(M / 256) * (N / 256) : 0;
  if (big && K >= 16384) {
    int best = 0;
    double best_fill = 0.0;
    for (int sp : {1, 2, 3, 4, 5, 6, 8, 10}) {
      if (!fits(sp)) continue;
      const long b = t256 * sp;
      const double fill = (double)b / (double)(((b + 255) / 256) * 256);
      if (fill > best_fill + 1e-9) {
        best_fill = fill;
        best = sp;
      }
    }
    if (best) {
      *pbm = 256; *pbn = 256; *psplits = best;
      return;
    }
  }
  if (big && K >= 2048 && t256 >= 256) {
    *pbm = 256; *pbn = 256;
    return;
  }
  if (K < 2048 || (long)(M / bm) * (N / bn) >= 512) return;
  static const int cand[][2] = {{128, 128}, {64, 128}, {128, 64}, {64, 64}};
  for (const auto& c : cand) {
    if (M % c[0] || N % c[1]) continue;
    const long t = (long)(M / c[0]) * (N / c[1]);
    for (int sp = 2; sp <= 16; sp++) {
      if (K / sp < 512) break;
      if (!fits(sp)) continue;
      if (t * sp >= 384) {
        *pbm = c[0]; *pbn = c[1]; *psplits = sp;
        return;
      }
    }
  }
}

template <int EPI>
static hipError_t splitk_reduce(const GemmArgs& g, const EpiParams& e, hipStream_t s) {
  const size_t MN = (size_t)g.M * g.N;
  const dim3 grid((unsigned)((MN / 4 + 255) / 256));
  const bool vec = EPI != EPI_STORE_H && (e.ldc % 4) == 0 && ((uintptr_t)e.C % 16) == 0 &&
                   (EPI != EPI_STORE_W13 || ((uintptr_t)e.C3 % 16) == 0);
  if (vec)
    hipLaunchKernelGGL((splitk_reduce_kernel<EPI, true>), grid, dim3(256), 0, s, g.ws, g.splits, g.M, g.N, e);
  else
    hipLaunchKernelGGL((splitk_reduce_kernel<EPI, false>), grid, dim3(256), 0, s, g.ws, g.splits, g.M, g.N, e);
  return hipGetLastError();
}

hipError_t gemm_run(const GemmArgs& g, int epi, const EpiParams& e, hipStream_t s, int bm, int bn, int nw,
                    int ns) {
  if (g.M <= 0 || g.N <= 0 || g.K <= 0 || (g.K % BK) != 0 || g.splits < 1 || g.splits > kMaxSplits)
    return hipErrorInvalidValue;
  if (g.pf_bytes && (!g.pf || ((uintptr_t)g.pf % 16) != 0)) return hipErrorInvalidValue;
  if (epi == EPI_RESID_NORM &&
      (!e.R || !e.C2 || !e.gain || !e.ssq_part || e.ssq_ld < g.M || g.splits != 1 || g.grp || g.a_t || g.b_t))
    return hipErrorInvalidValue;
  if (epi_rr(epi) && (!e.rr_part || e.rr_nparts < 1 || e.rr_nparts > kRrMaxParts || e.rr_dim <= 0 ||
                      e.rr_ld < (epi == EPI_CE_RR ? g.N : g.M) || g.splits != 1 || g.grp || g.a_t || g.b_t))
    return hipErrorInvalidValue;
  if (g.splits > 1) {
    // layouts 0 (K-major), 1 (B M-major) and 3 (both M-major)
    if ((g.a_t && !g.b_t) || g.grp || !g.ws || (g.K % (g.splits * BK)) != 0 || (ns != 0 && ns != 2) ||
        (epi != EPI_STORE_F && epi != EPI_STORE_H && epi != EPI_STORE_W13) || (g.N % 4) != 0)
      return hipErrorInvalidValue;
    if (bm == 0 || bn == 0) gemm_pick_tile(g.M, g.N, g.K, epi, &bm, &bn);
    if (bm == 0 || bn == 0 || (g.M % bm) || (g.N % bn)) return hipErrorInvalidValue;
    if (nw == 0) nw = (bm == 256 && bn == 256) ? 8 : 4;
    if (nw != 4 && !(nw == 8 && bm == 256 && bn == 256)) return hipErrorInvalidValue;
    EpiParams pw;  // fp32 partials, ws[s][M][N]
    pw.C = g.ws;
    pw.ldc = g.N;
    hipError_t r = g.a_t   ? launch<true, true, EPI_STORE_F>(g, pw, s, bm, bn, nw, 2)
                   : g.b_t ? launch<false, true, EPI_STORE_F>(g, pw, s, bm, bn, nw, 2)
                           : launch<false, false, EPI_STORE_F>(g, pw, s, bm, bn, nw, 2);
    if (r != hipSuccess) return r;
    if (epi == EPI_STORE_F) return splitk_reduce<EPI_STORE_F>(g, e, s);
    if (epi == EPI_STORE_H) return splitk_reduce<EPI_STORE_H>(g, e, s);
    return splitk_reduce<EPI_STORE_W13>(g, e, s);
  }
  if (bm == 0 || bn == 0) gemm_pick_tile(g.M, g.N, g.K, epi, &bm, &bn);
  if (bm == 0 || bn == 0 || (g.M % bm) || (g.N % bn)) return hipErrorInvalidValue;
  // 256x256 tiles run with 8 waves unless 4 are asked for (measured faster
  // on every shape and layout: two waves per SIMD hide each other's barrier
  // and LDS waits; the 4-wave tile's classifier reductions also spill)
  if (nw == 0) nw = (bm == 256 && bn == 256) ? 8 : 4;
  if (nw != 4 && !(nw == 8 && bm == 256 && bn == 256)) return hipErrorInvalidValue;
  if (ns == 0) ns = 2;
  // the self-prefetch is a hint: kPfBlocks blocks of 64 nw threads cover at
  // most kPfLoads 16-byte loads each per thread; a longer region is cut
  GemmArgs gp = g;
  gp.pf_bytes = std::min(g.pf_bytes, (size_t)kPfBlocks * kPfLoads * 64 * nw * 16);
  const GemmArgs& g2 = gp;
  // three LDS stages: both operands K-major, 4 waves, tiles whose 3 stages fit the 160 KB LDS
  if (ns != 2 && !(ns == 3 && nw == 4 && !g.a_t && !g.b_t && (bm + bn) <= 384 && !(bm == 256 && bn == 64) &&
                   !(bm == 128 && bn == 256)))
    return hipErrorInvalidValue;
  const int lay = (g.a_t ? 2 : 0) | (g.b_t ? 1 : 0);
  if (g.grp && (lay != 0 || ns != 2)) return hipErrorInvalidValue;
#define CASE(L, AT, BT, E) \
  if (lay == L && epi == E) return launch<AT, BT, E>(g2, e, s, bm, bn, nw, ns);
  // forward (activation x weight^T)
  CASE(0, false, false, EPI_STORE_H)
  CASE(0, false, false, EPI_STORE_F)
  CASE(0, false, false, EPI_LOGITS)
  CASE(0, false, false, EPI_RESID)
  CASE(0, false, false, EPI_SWIGLU)
  CASE(0, false, false, EPI_RELU2)
  CASE(0, false, false, EPI_SMEAR)
  CASE(0, false, false, EPI_CE)
  CASE(0, false, false, EPI_DLOGITS)
  CASE(0, false, false, EPI_STORE_RS)
  CASE(0, false, false, EPI_RESID_NORM)
  CASE(0, false, false, EPI_STORE_H_RR)
  CASE(0, false, false, EPI_SWIGLU_RR)
  CASE(0, false, false, EPI_CE_RR)
  // backward with transposed weight shadows / operands (all K-major)
  CASE(0, false, false, EPI_SWIGLU_BWD)
  CASE(0, false, false, EPI_RELU2_BWD)
  CASE(0, false, false, EPI_STORE_W13)
  // backward dX = dY * W  (B transposed)
  CASE(1, false, true, EPI_STORE_H)
  CASE(1, false, true, EPI_STORE_F)
  CASE(1, false, true, EPI_SWIGLU_BWD)
  CASE(1, false, true, EPI_RELU2_BWD)
  // backward dW = dY^T * X (both transposed)
  CASE(3, true, true, EPI_STORE_F)
  CASE(3, true, true, EPI_STORE_W13)
#undef CASE
  return hipErrorInvalidValue;
}

}  // namespace ane
