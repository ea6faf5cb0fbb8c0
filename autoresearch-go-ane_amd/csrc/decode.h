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
constexpr int kDecWideChunk = 1152;   // keys per split of the 1024-thread form (9 passes of 128)
constexpr int kDecWideMinBlocks = 192;  // batch x kv heads from which that form is chosen

// MFMA-fragment-major layout of the decode-step operands.  A 32x32x16 MFMA
// operand lane l takes row l%32 and eight k-values; with the k-slot map
// k = 64*w + 32*(l/32) + 8*s + j (window w, step s = 0..3, j = 0..7) one
// operand fragment is 64 lanes x 16 B, stored here as 1 KB contiguous so a
// wave loads it with one fully coalesced instruction (8 whole cache lines)
// instead of touching 32 rows.
//   activations [64 rows][K]: fragment (w, s, tile = row/32)
//   weights     [N rows][K]:  fragment (row group g = row/32, w, s)
__device__ __host__ __forceinline__ size_t act_frag_off(int t, int k) {
  const int w = k >> 6, kk = k & 63;
  const int lane = (t & 31) + 32 * (kk >> 5), s = (kk >> 3) & 3;
  return ((((size_t)(w * 4 + s) * 2 + (t >> 5)) * 64 + lane) << 3) + (kk & 7);
}
// row-major fp16 W [N][K] -> fragment-major (N % 32 == 0, K % 64 == 0)
hipError_t weight_to_frag(half_t* dst, const half_t* src, int N, int K, hipStream_t s);

// Classifier of the decode rows: Y = X[64, K] . W[N, K]^T (fragment-major
// operands), K split over the waves of one block per 32 vocabulary rows
// and added in a fixed order; epilogue: per 32-column group (max, first
// index) over n < nvalid -> amax[N/32][64], optionally logits [64][N] fp32.
struct SkinnyArgs {
  const half_t* X;  // [64, K] activation fragments (act_frag_off)
  const half_t* W;  // [N, K] weight fragments (weight_to_frag)
  int N, K, nb;     // N % 32 == 0, K % 64 == 0 (classifier: K <= 1024), 1 <= nb <= 64
  float2* amax;
  float* logits;
  int nvalid;
  const float* rr = nullptr;  // [64] per-token scale of the logits written (argmax is unaffected: rr > 0)
};
hipError_t classifier_argmax(const SkinnyArgs& a, hipStream_t s);

// Split-K form of the decode-step GEMMs (Y = X[64, K] . W[N, K]^T, same
// fragment-major operands): skinny_partials writes ks = skinny_splits(N, K)
// fp32 partials part[ks][64][N] from (N/32) x ks one-wave blocks; a finish
// kernel per token row sums them in split order and applies the epilogue
// (the QKV partials are finished inside dec_attention):
//   resid_norm: x[t] += Y[t]; xn[t] = fp16(rmsnorm(x[t]) * g)  (N = D <= 1024)
//   swiglu:     gate[t][j] = silu(h1) * h3 over W1|W3 interleaved by 32 rows (fragment layout)
int skinny_splits(int N, int K);
hipError_t skinny_partials(const half_t* X, const half_t* W, float* part, size_t part_cap, int N, int K,
                           hipStream_t s);
hipError_t skinny_finish_resid_norm(const float* part, int N, int K, float* x, half_t* xn, const float* g, int nb,
                                    hipStream_t s);
hipError_t skinny_finish_swiglu(const float* part, int N, int K, half_t* gate, int nb, hipStream_t s);

// tok_out[b] = argmax over groups (first index on ties) for b < nb;
// hist (optional) [..][nb]: row *step receives the same tokens.
hipError_t argmax_reduce(uint16_t* tok_out, uint16_t* hist, const int* step, const float2* amax, int ngroups,
                         int nb, hipStream_t s);

// ctr = {position of the current step's token, step index of this call,
// steps since open}: advance all three / set the first two (kernels, so the
// counters never depend on host memory lifetimes).  The third never resets:
// it numbers the uses of the tail kernel's counters and flags.
hipError_t dec_advance(int* ctr, hipStream_t s);
hipError_t dec_set_ctr(int* ctr, int pos, int step, hipStream_t s);

// x[b] = embed[tok_b] (zero row if tok_b >= V); xn[b] = fp16(rmsnorm(x[b]) * g)
// (xn, att and gate of the decode rows are in the activation fragment layout)
hipError_t dec_embed_norm(float* x, half_t* xn, const float* embed, const uint16_t* tok, const float* g, int nb,
                          int D, int V, hipStream_t s);

// xn[b] = fp16(rmsnorm(x[b]) * g) for b < nb
hipError_t dec_norm(const float* x, half_t* xn, const float* g, int nb, int D, hipStream_t s);

// Attention of one query token per sequence over keys 0..pos (pos = *ctr)
// in chunks of kDecChunk keys: partials o (unnormalized), m, l per
// (b, head, chunk); then the merge into att [64][NH*64] fp16.
// The step's q, k, v come straight from the QKV GEMM's split-K partials
// (skinny_partials, N = (NH + 2 NKV) * 64): every block sums the q columns
// of its heads and applies RoPE at ctr[0]; the block whose key split holds
// that position also forms the new k (RoPE) and v rows, writes them to the
// cache and uses them in place of the row it read.
struct DecAttnArgs {
  const float* qkv_part;  // [qkv_ks][64][(NH + 2 NKV) * 64]
  int qkv_ks;
  const float* rope_cos;
  const float* rope_sin;
  half_t* kc;        // layer base [Bcap][NKV][max_ctx][64]
  half_t* vc;
  const int* ctr;
  float* part;       // [nb][NH][nsplit][66]
  half_t* att;       // [64][NH*64]
  int nb, NH, NKV, max_ctx, nsplit;  // nsplit: partial slots per head (max_ctx / kDecChunk)
  float scale;
  int form = 0;  // 0: by batch size, 1: 1024-thread blocks, 2: 256-thread splits
  const float* rr = nullptr;  // [64] 1 / rms of each row's input when the partials are of fp16(x * gain)
};
hipError_t dec_attention(const DecAttnArgs& a, hipStream_t s);

// ---- the per-layer GEMM chain in one launch (decode_tail.hip) ---------------
// Wo + residual, W1|W3 + SwiGLU, W2 + residual, the next layer's QKV
// projection and its 1 / rms: one 16-wave block per 32-column group (per
// W1|W3 pair) over the whole K, blocks ordered by phase; a block waits on the
// done counter of the phase it reads (no grid barrier).  Requires every block
// resident at once: dec_tail_blocks_per_cu() x CUs >= the block count.
// The data-polling form of the chain exchanges its activations through one
// of two buffer sets (by the parity of the use), in which every dword starts
// as kTailStale: a consumer polls the data itself until no dword is stale,
// and each launch resets the other set for the next use.
constexpr uint32_t kTailStale = 0xFFFFFFFFu;
struct TailSet {
  half_t* xg_ffn;   // [64][D] fragments: fp16(x * g_ffn) after Wo
  half_t* gate;     // [64][H] fragments
  half_t* xg_next;  // [64][D] fragments: fp16(x * g_next) after W2 (for the next QKV)
  float* x_mid;     // [64][D] the residual after Wo
  float* ssq_wo;    // [D/32][64] per column group sum of squares after Wo
  float* ssq_w2;    // [D/32][64] and after W2
  float* p_q;       // [64][N1] the next layer's q | k | v (read by attention blocks of the same launch)
  float* rr;        // [64] 1 / rms after W2 (likewise)
};
__host__ __device__ inline size_t tail_set_bytes(int D, int H, int N1) {
  return (size_t)64 * (2 * D + H) * 2 + (size_t)64 * D * 4 + (size_t)2 * (D / 32) * 64 * 4 + (size_t)64 * N1 * 4 +
         64 * 4;
}
__host__ __device__ inline TailSet tail_set(void* base, int D, int H, int N1) {
  char* p = static_cast<char*>(base);
  TailSet t;
  t.xg_ffn = reinterpret_cast<half_t*>(p); p += (size_t)64 * D * 2;
  t.gate = reinterpret_cast<half_t*>(p); p += (size_t)64 * H * 2;
  t.xg_next = reinterpret_cast<half_t*>(p); p += (size_t)64 * D * 2;
  t.x_mid = reinterpret_cast<float*>(p); p += (size_t)64 * D * 4;
  t.ssq_wo = reinterpret_cast<float*>(p); p += (size_t)(D / 32) * 64 * 4;
  t.ssq_w2 = reinterpret_cast<float*>(p); p += (size_t)(D / 32) * 64 * 4;
  t.p_q = reinterpret_cast<float*>(p); p += (size_t)64 * N1 * 4;
  t.rr = reinterpret_cast<float*>(p);
  return t;
}
struct TailArgs {
  const half_t* att;        // [64][D] activation fragments: the attention output
  float* x;                 // [64][D] residual stream (fp32, row-major)
  const half_t* wo;         // fragment-major [D][D]
  const half_t* w13;        // fragment-major [2H][D], W1 / W3 interleaved by 32 rows
  const half_t* w2;         // fragment-major [D][H]
  const half_t* wqkv_next;  // fragment-major [N1][D] of the next layer (unused when b_q == 0)
  const float* g_ffn;       // [D] gain of the FFN norm
  const float* g_next;      // [D] gain of the next norm (next layer's attention norm, or the final norm)
  half_t* xg_ffn;           // [64][D] fragments: fp16(x * g_ffn) after Wo
  half_t* gate;             // [64][H] fragments
  half_t* xg_next;          // [64][D] fragments: fp16(x * g_next) after W2
  float* rr_next;           // [64] 1 / rms of x after W2
  float* p_q;               // [64][N1] the next layer's q | k | v, before 1 / rms and RoPE
  float* ssq_wo;            // [D/32][64] per column group sum of squares of the residual
  float* ssq_w2;
  unsigned* sync;           // done counters (kDecTailSync words, zero at open)
  const int* gstep;         // steps since open (ctr[2])
  int* err;                 // set when a wait times out; later launches exit at once
  unsigned spin_limit;      // polls before a wait times out (kDecTailSpin; 0: every wait fails)
  int D, H, N1, layer, L;
  int b_wo, b_13, b_w2, b_q;  // blocks per phase: D/32, H/32, D/32, N1/32 (0 on the last layer)
  // data-polling form (poll != 0): the two buffer sets (tail_set_bytes each,
  // every dword kTailStale at open); xg_ffn, ssq_wo, ssq_w2 and sync above
  // are then unused, and xg_next receives the last layer's W2 output only
  int poll = 0;
  void* sets[2] = {nullptr, nullptr};
  // data-polling form only: b_att > 0 adds the next layer's decode attention
  // (wide form, one split) to the launch as b_att more blocks after the
  // chain's, one per (sequence, kv head): att_next's qkv_part, qkv_ks and rr
  // are then the launch's own (the buffer set), and p_q / rr_next above are
  // unused.  The attention blocks issue their K / V loads at once (the cache
  // does not depend on the chain) and poll q; every chain block is resident
  // before any of them (lower block indices), so no chain wait depends on
  // an attention block.
  int b_att = 0;
  DecAttnArgs att_next;
};
// Whether the attention of `a` can run inside the chain's launch (the wide
// form with one split, G <= kGMax).
bool dec_attention_fusable(const DecAttnArgs& a);
constexpr int kDecTailSync = 64;
constexpr unsigned kDecTailSpin = 1u << 20;  // polls of ~100 cycles: ~50 ms
hipError_t dec_tail(const TailArgs& a, hipStream_t s);
int dec_tail_blocks_per_cu();
// x [64][D] (or, with tok, x = embed[tok]) -> xg = fp16(x * g) fragments and
// rr = 1 / rms(x), for rows < nb
hipError_t dec_row_xg(float* x, half_t* xg, float* rr, const float* embed, const uint16_t* tok, const float* g,
                      int nb, int D, int V, hipStream_t s);

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
