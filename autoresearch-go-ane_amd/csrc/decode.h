// Kernels of the greedy KV-cache decoder (grouped-query attention).
//
// The reference has no decode path (it evaluates whole windows,
// ane/engine.go:954-1038); these kernels serve the decode benchmark's
// Llama2-style model built from the same primitives: gain RMSNorm
// (ane/stories/cpu.go:97-111), RoPE (ane/train_util.go:183-224), causal
// softmax attention (ane/common.go:61-89), SwiGLU, tied classifier
// (ane/stories/cpu.go:303-327), greedy argmax.
//
// Decode-step rows: every decode-time activation buffer holds 64 token rows
// (one per sequence, rows >= the active batch are ignored), so the
// projections are 64-row "skinny" GEMMs that stream the fp16 weights once.
#pragma once
#include "hip_common.h"

namespace ane {

constexpr int kDecRows = 64;    // token rows of a decode step (max sequences)
constexpr int kDecChunk = 256;  // keys per decode-attention split

// partial[s][64][N] = X[64, s-th K range] . W[N, same range]^T  (EPI 0)
// EPI 1 (splits == 1): per 32-column group and row, (max, first index of
// the max) over columns < nvalid -> amax[N/32][64]; logits (optional)
// receives the fp32 row [64][N].
struct SkinnyArgs {
  const half_t* X;  // [64, K], ld = ldx
  int ldx;
  const half_t* W;  // [N, K], ld = ldw
  int ldw;
  int N, K, splits;  // N % 32 == 0, K % (64 * splits) == 0
  float* partial;
  float2* amax;
  float* logits;
  int nvalid;
};
hipError_t skinny_gemm(const SkinnyArgs& a, int epi, hipStream_t s);
// smallest split count that gives >= 256 waves with K ranges of whole 64s
int skinny_splits(int N, int K);

// tok_out[b] = argmax over groups (first index on ties) for b < nb;
// hist (optional) [..][nb]: row *step receives the same tokens.
hipError_t argmax_reduce(uint16_t* tok_out, uint16_t* hist, const int* step, const float2* amax, int ngroups,
                         int nb, hipStream_t s);

// ctr = {position of the current step's token, step index}: advance both /
// set both (kernels, so the counters never depend on host memory lifetimes)
hipError_t dec_advance(int* ctr, hipStream_t s);
hipError_t dec_set_ctr(int* ctr, int pos, int step, hipStream_t s);

// x[b] = embed[tok_b] (zero row if tok_b >= V); xn[b] = fp16(rmsnorm(x[b]) * g)
hipError_t dec_embed_norm(float* x, half_t* xn, const float* embed, const uint16_t* tok, const float* g, int nb,
                          int D, int V, hipStream_t s);

// x[b] += sum_s partial[s][b]; xn[b] = fp16(rmsnorm(x[b]) * g)   (partial may be null: norm only)
hipError_t dec_resid_norm(float* x, half_t* xn, const float* partial, int splits, const float* g, int nb, int D,
                          hipStream_t s);

// gate[b][j] = silu(h1) * h3 with h1, h3 the split sums of the W1|W3 rows
// interleaved in 32-row blocks (col (j/32)*64 + j%32 and +32)
hipError_t dec_swiglu(half_t* gate, const float* partial, int splits, int nb, int H, hipStream_t s);

// Split sums of the fused q|k|v projection at position *ctr: q (RoPE) ->
// q_out [64][NH*64]; k (RoPE), v -> cache [.. b][kvh][pos][64] of the layer.
struct DecQkvArgs {
  const float* partial;
  int splits;
  const int* ctr;
  const float* rope_cos;  // [max_ctx][32]
  const float* rope_sin;
  half_t* q;
  half_t* kc;  // layer base, [Bcap][NKV][max_ctx][64]
  half_t* vc;
  int nb, NH, NKV, max_ctx;
};
hipError_t dec_qkv_finish(const DecQkvArgs& a, hipStream_t s);

// Attention of one query token per sequence over keys 0..pos (pos = *ctr)
// in chunks of kDecChunk keys: partials o (unnormalized), m, l per
// (b, head, chunk); then the merge into att [64][NH*64] fp16.
struct DecAttnArgs {
  const half_t* q;   // [64][NH*64]
  const half_t* kc;  // layer base
  const half_t* vc;
  const int* ctr;
  float* part;       // [nb][NH][nsplit][66]
  half_t* att;       // [64][NH*64]
  int nb, NH, NKV, max_ctx, nsplit;
  float scale;
};
hipError_t dec_attention(const DecAttnArgs& a, hipStream_t s);

// ---- prefill ---------------------------------------------------------------
// qkv [T][N1] (T = nseq * S tokens of sequences seq0..): RoPE q in place;
// k (RoPE), v -> cache positions 0..S-1 of each sequence.
hipError_t prefill_kv_write(half_t* qkv, half_t* kc, half_t* vc, const float* rope_cos, const float* rope_sin,
                            int seq0, int nseq, int S, int NH, int NKV, int max_ctx, hipStream_t s);

// Causal attention of the prefix: queries from qkv (after RoPE), keys and
// values from the cache; out [T][NH*64] fp16.  S % 32 == 0.
struct PrefillAttnArgs {
  const half_t* qkv;
  int ldq;
  const half_t* kc;
  const half_t* vc;
  half_t* out;
  int seq0, nseq, S, NH, NKV, max_ctx;
  float scale;
};
hipError_t prefill_attention(const PrefillAttnArgs& a, hipStream_t s);

// rows[i] = src[(i * S + S - 1)] for i < nseq (fp32 rows of D): the last
// prefix position of each sequence -> decode rows seq0 + i
hipError_t gather_last_rows(float* dst, const float* src, int nseq, int S, int D, hipStream_t s);

}  // namespace ane
