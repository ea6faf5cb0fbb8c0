// MFMA GEMM for gfx950: C[m, n] = sum_k A(m, k) * B(n, k), fp16 in, fp32 acc.
//
// Operand storage (ld = leading dimension, in elements):
//   A(m, k) = a_t ? A[k * lda + m] : A[m * lda + k]
//   B(n, k) = b_t ? B[k * ldb + n] : B[n * ldb + k]
// The non-transposed form is the natural one for "activation x weight^T"
// with token-major activations [T, in] and row-major weights [out, in]
// (the reference's linearCF, ane/common.go:91-105).  Transposed operands
// (dX = dY * W and dW = dY^T * X of the backward) are transposed while
// being staged into LDS, so every MFMA reads K-contiguous fragments.
//
// M, N must be multiples of the chosen block tile (64/128/256) and K a
// multiple of 64; gemm_run() checks this on the host and refuses
// anything else with hipErrorInvalidValue.
#pragma once
#include "hip_common.h"

namespace ane {

enum Epi : int {
  EPI_STORE_H = 0,   // C (fp16) = scale * acc
  EPI_STORE_F = 1,   // C (fp32) = scale * acc  (+= when accumulate)
  EPI_LOGITS = 2,    // C (fp32) = softcap ? cap * tanh(acc / cap) : acc
  EPI_RESID = 3,     // C (fp32) = alpha * R + acc + beta * X0; C2 (fp32, optional) = same
  EPI_SWIGLU = 4,    // C (fp16) = silu(h1) * h3 over 32-column interleaved W1|W3; C2 (fp16) = h1|h3
  EPI_RELU2 = 5,     // C (fp16) = max(acc, 0)^2; C2 (fp16, optional) = acc
  EPI_SMEAR = 6,     // C (fp32) = X0 + [t % seq != 0] * alpha * sigmoid(acc) * X0[t-1]; C2 (fp32) = sigmoid(acc)
  EPI_CE = 7,        // rows = vocab, cols = tokens: per-column partial (max, sumexp) + target logit
  EPI_DLOGITS = 8,   // rows = vocab, cols = tokens: C (fp16) = dlogit (see kernel)
  EPI_STORE_W13 = 9, // C (fp32) rows of an interleaved W1|W3 gradient scattered to two outputs
  EPI_SWIGLU_BWD = 10, // acc = dgate [T, H]; C2 (fp16) = h1|h3 interleaved -> C (fp16) = dh1|dh3 interleaved
  EPI_RELU2_BWD = 11,  // acc = dgate [T, H]; C2 (fp16) = h1 -> C (fp16) = dgate * 2 * max(h1, 0)
  EPI_STORE_RS = 12,   // C (fp32) = acc * rowscale[row]
  // Deferred RMSNorm (llama2 eval forward): the residual GEMM leaves its
  // consumers fp16(x * gain) and per-row partial sums of x^2; the consumer
  // GEMMs scale their (linear) outputs by rr = 1 / rms(x) per token.
  EPI_RESID_NORM = 13, // C (fp32) = R + acc; C2 (fp16, ld ldc2) = C * gain[col];
                       // ssq_part[(n0 / BN) * ssq_ld + row] = sum over the block's BN columns of C^2
  EPI_STORE_H_RR = 14, // EPI_STORE_H of acc * rr[row]
  EPI_SWIGLU_RR = 15,  // EPI_SWIGLU of acc * rr[row]
  EPI_CE_RR = 16,      // EPI_CE of acc * rr[col] (columns = tokens)
};
// Partial sums of squares a consumer combines (rr_nparts <= kRrMaxParts).
constexpr int kRrMaxParts = 16;
// split-K: most K slices of one GEMM (the reduce keeps one load per slice in flight)
constexpr int kMaxSplits = 16;
__host__ __device__ constexpr bool epi_rr(int epi) {
  return epi == EPI_STORE_H_RR || epi == EPI_SWIGLU_RR || epi == EPI_CE_RR;
}
// The epilogue an rr variant shares with its plain form.
__host__ __device__ constexpr int epi_base(int epi) {
  return epi == EPI_STORE_H_RR ? EPI_STORE_H
         : epi == EPI_SWIGLU_RR ? EPI_SWIGLU
         : epi == EPI_CE_RR     ? EPI_CE
         : epi == EPI_RESID_NORM ? EPI_RESID
                                 : epi;
}

struct GemmArgs {
  const half_t* A;
  const half_t* B;
  int lda, ldb;
  int M, N, K;
  bool a_t, b_t;
  // Grouped GEMM (layout 0 only): M is the row capacity; grp[0] = number of
  // valid BM-row tiles, then per tile (first row, group); the B operand of
  // group g starts at B + g * b_group_stride.  Tiles past grp[0] exit.
  const int* grp = nullptr;
  size_t b_group_stride = 0;
  // Split-K (layout 0, epilogues STORE_F / STORE_H / STORE_W13): split s of
  // `splits` reduces k in [s K/splits, (s+1) K/splits) into the fp32
  // workspace ws[s][M][N]; a second kernel sums the splits in a fixed order
  // and applies the epilogue, so results do not depend on block timing.
  int splits = 1;
  float* ws = nullptr;
  // Self-prefetch: the launch's first kPfBlocks blocks each stream one slice
  // of [pf, pf + pf_bytes) (16-byte aligned, at most kPfBlocks * kPfLoads *
  // 256 * 16 bytes) through the caches with their prologue loads, so that a
  // cold weight operand is requested whole at the start instead of one
  // k-tile per k-step.  K-major kernel only.
  const void* pf = nullptr;
  size_t pf_bytes = 0;
};
// Blocks that share a self-prefetch, and 16-byte loads per thread at most.
constexpr int kPfBlocks = 256;
constexpr int kPfLoads = 8;

struct EpiParams {
  void* C = nullptr;
  int ldc = 0;
  void* C2 = nullptr;
  int ldc2 = 0;
  const float* R = nullptr;   // residual input (EPI_RESID), ld = ldc
  const float* X0 = nullptr;  // x0 (EPI_RESID / EPI_SMEAR), ld = ldc
  float alpha = 1.f, beta = 0.f, scale = 1.f;
  const float* alpha_ptr = nullptr;   // when set, alpha = *alpha_ptr (device scalar)
  const float* beta_ptr = nullptr;    // when set, beta = *beta_ptr
  int accumulate = 0;
  int seq = 0;
  // classifier epilogues
  const uint16_t* targets = nullptr;  // [N] target id per token column
  float2* partial = nullptr;          // [M / BM][N] (max, sumexp) per block row
  float* tgt_logit = nullptr;         // [N]
  const float* lse = nullptr;         // [N] log-sum-exp (EPI_DLOGITS)
  const float* colscale = nullptr;    // [N] dlogit scale per token (EPI_DLOGITS)
  int softcap = 0;
  float cap = 15.f;
  int vocab = 0;                      // rows >= vocab are padding (ignored)
  float* C3 = nullptr;                // second fp32 output (EPI_STORE_W13: W3 grad)
  const float* rowscale = nullptr;    // [M] (EPI_STORE_RS)
  // deferred RMSNorm
  const float* gain = nullptr;        // [N] (EPI_RESID_NORM)
  float* ssq_part = nullptr;          // [N / BN][ssq_ld] out (EPI_RESID_NORM)
  int ssq_ld = 0;
  const float* rr_part = nullptr;     // [rr_nparts][rr_ld] in (rr variants): rr = 1 / sqrt(sum / rr_dim + 1e-5)
  int rr_ld = 0, rr_nparts = 0, rr_dim = 0;
};

// Launches one GEMM on `stream`.  bm/bn force a block tile (0 = heuristic);
// nw = waves per block: 4 (default) or 8 (256x256 tiles only).
// ns = LDS pipeline stages: 2 (default) or 3 (K-major operands, 4 waves,
// tiles 256x128, 128x128, 64x128, 128x64, 64x64).
hipError_t gemm_run(const GemmArgs& g, int epi, const EpiParams& e, hipStream_t stream,
                    int bm = 0, int bn = 0, int nw = 0, int ns = 0);

// Tile and split count for a K-major GEMM whose output is too small to
// fill the chip with one block per tile (the backward's dW = dY^T X with
// K = tokens, dX with K = 2048..32000); *splits = 1 when no split pays.
// ws_cap = workspace floats available (splits * M * N must fit).
void gemm_pick_split(int M, int N, int K, int epi, size_t ws_cap, int* bm, int* bn, int* splits);

// Tile the heuristic picks; nonzero *bm / *bn on entry are kept as
// constraints (set both to 0 for a free choice).  0 = no tile fits.
void gemm_pick_tile(int M, int N, int K, int epi, int* bm, int* bn);

}  // namespace ane
