/*
 * ane_kernels.h -- the gfx950 code objects a host that has no C++ library
 * loads itself: dlopen libamdhip64, hipModuleLoad the `.hsaco` files that
 * __graft_entry__.build() writes next to libane_hip.so, hipModuleGetFunction
 * by the names below, hipModuleLaunchKernel with each kernel's arguments as
 * one packed buffer (HIP_LAUNCH_PARAM_BUFFER_POINTER / _SIZE).  This is the
 * boundary the reference's Go host would use through purego (no CGo), in
 * place of the MIL programs it compiles for the Neural Engine:
 * ane/layer_darwin.go and ane/layer_dynamic_darwin.go (the per-layer
 * forward), ane/mil_stories.go (the classifier and cross-entropy head).
 *
 * The kernels are the ones libane_hip.so launches for the llama2 eval
 * forward + loss (the deferred-norm form); ane/hsaco.py drives all of them
 * through hipModuleLaunchKernel and is checked against ane_eval_loss bit for
 * bit.  Argument structs are plain C with the layout of the library's own
 * (checked by static_assert where the kernels are compiled, and by a test
 * against the offsets ane_kernel_abi() reports).
 *
 * Code objects (one per compilation unit):
 *   ane_gemm.hsaco       ane_k_gemm_*      (args: AneGemmArgs, AneEpiParams)
 *   ane_attention.hsaco  ane_k_attn_fwd, ane_k_attn_fwd15 (args: AneAttnArgs)
 *   ane_rowops.hsaco     ane_k_embed_xg, ane_k_prefetch, ane_k_ce_token,
 *                        ane_k_ce_reduce   (scalar / pointer args)
 */
#ifndef ANE_KERNELS_H
#define ANE_KERNELS_H

#include <stddef.h>
#include <stdint.h>

/* C[m, n] = sum_k A(m, k) B(n, k): A [M, lda] and B [N, ldb] fp16, K-major
 * (the a_t / b_t forms are not exported).  M, N multiples of the kernel's
 * tile, K of 64. */
typedef struct AneGemmArgs {
  const void *A;
  const void *B;
  int32_t lda, ldb;
  int32_t M, N, K;
  uint8_t a_t, b_t;              /* 0 for the exported kernels */
  const int32_t *grp;            /* NULL */
  size_t b_group_stride;         /* 0 */
  int32_t splits;                /* 1 */
  float *ws;                     /* NULL */
  const void *pf;                /* optional: region the first 256 blocks stream through the caches */
  size_t pf_bytes;               /* at most 256 blocks x 8 loads x 64 lanes x waves x 16 B */
} AneGemmArgs;

/* Epilogue parameters; fields a kernel does not name are ignored (zero). */
typedef struct AneEpiParams {
  void *C;
  int32_t ldc;
  void *C2;
  int32_t ldc2;
  const float *R;                /* residual input (RESID_NORM), ld = ldc */
  const float *X0;
  float alpha, beta, scale;      /* scale = 1 for the exported kernels */
  const float *alpha_ptr;
  const float *beta_ptr;
  int32_t accumulate;
  int32_t seq;
  const uint16_t *targets;       /* CE: [N] target id per token column */
  void *partial;                 /* CE: float2 [M / 256][N] (max, sum exp) per block row */
  float *tgt_logit;              /* CE: [N] */
  const float *lse;
  const float *colscale;
  int32_t softcap;
  float cap;
  int32_t vocab;
  float *C3;
  const float *rowscale;
  const float *gain;             /* RESID_NORM: [N] */
  float *ssq_part;               /* RESID_NORM: [N / 64][ssq_ld] per-row partial sums of squares */
  int32_t ssq_ld;
  const float *rr_part;          /* rr forms: [rr_nparts][rr_ld]; rr = 1 / sqrt(sum / rr_dim + 1e-5) */
  int32_t rr_ld, rr_nparts, rr_dim;
} AneEpiParams;

/* Causal attention, head dim 64 (see attention.h in the sources). */
typedef struct AneAttnArgs {
  const void *qkv;               /* [T, 3D] fp16: q | k | v per row (pre-RoPE) */
  void *out;                     /* [T, D] fp16 */
  float *lse;                    /* [T, NH] or NULL */
  const float *rope_cos;         /* [S, 32] */
  const float *rope_sin;         /* [S, 32] */
  int32_t nseq, S, NH;
  int32_t qknorm;                /* 0 (llama2) */
  float scale;                   /* 0.125 */
  const float *ve_x;             /* NULL */
  const float *ve_gate;
  const float *ve_embed;
  const uint16_t *tokens;
  int32_t vocab;
  void *qkvt;                    /* NULL */
  void *qkvt_lo;                 /* NULL */
  int32_t hilo;                  /* 0 */
  const void *pf;                /* optional: next GEMM's weights streamed through the caches */
  size_t pf_bytes;
  int32_t split_from;            /* 0: grid (1, NH, nseq); > 0: 1-D grid, see ane_k_attn_fwd */
} AneAttnArgs;

/*
 * Kernel table (block = threads per block; grid as stated):
 *
 *  ane_k_gemm_qkv_rr     128x192 tile, 256 threads, grid (M/128)(N/192):
 *                        fp16 C = (A B^T) * rr[row]                (Wq|Wk|Wv)
 *  ane_k_gemm_resid_norm 128x64 tile, 256 threads, grid (M/128)(N/64):
 *                        C (fp32) = R + A B^T; C2 (fp16, ldc2) = C * gain[col];
 *                        ssq_part[(n0/64) * ssq_ld + row] = sum over the block's
 *                        64 columns of C^2                        (Wo, W2)
 *  ane_k_gemm_swiglu_rr  256x256 tile, 512 threads, grid (M/256)(N/256):
 *                        fp16 C [M, N/2] = silu(h1) * h3 over 32-column
 *                        interleaved W1|W3 rows of (A B^T) * rr[row]  (W1|W3)
 *  ane_k_gemm_ce_rr      256x256 tile, 512 threads, grid (M/256)(N/256), rows =
 *                        vocabulary, columns = tokens: per block row and token
 *                        the (max, sum exp) of (A B^T) * rr[col], and the
 *                        target's logit                       (classifier + CE)
 *  ane_k_attn_fwd        512 threads; grid (1, NH, nseq) with split_from = 0
 *                        (S = 256), or 1-D 256 + 2 (nseq NH - 256) blocks with
 *                        split_from = 256 when 256 < nseq NH < 512 (the heads
 *                        past 256 as two half blocks)
 *  ane_k_attn_fwd15      768 threads, grid 256 (one block per CU), split_from =
 *                        0, S = 256, 256 < nseq NH <= 384: block c stages head c
 *                        and, for c < 2 (nseq NH - 256), half c % 2 of head
 *                        256 + c / 2 (the library's choice for those head counts)
 *  ane_k_embed_xg(x, xg, ssq, E, tok, gain, T, D, V, pf, pf_bytes)
 *                        256 threads, grid ceil(T / 4): x = E[tok] (0 when tok
 *                        >= V), xg = fp16(x * gain), ssq[t] = sum x^2
 *  ane_k_prefetch(p, bytes)   256 threads, any grid: streams [p, p + bytes)
 *  ane_k_ce_token(lse, tok_loss, partial, np, tgt_logit, tgt, V, T)
 *                        256 threads, grid ceil(T / 32): merges the np block-row
 *                        partials per token; tok_loss = -max(log p, log 1e-10)
 *  ane_k_ce_reduce(loss_seq, colscale, dscale, tok_loss, tgt, V, S)
 *                        256 threads, grid nseq: mean loss per sequence over
 *                        its valid targets (colscale may be NULL)
 */

#ifdef __cplusplus
extern "C" {
#endif

/* Size of the named argument struct ("AneGemmArgs", "AneEpiParams",
 * "AneAttnArgs") as the kernels see it, and up to `max` field offsets in
 * declaration order; returns the field count, or -1 for an unknown name.
 * No counterpart in the reference (a host binding checks its mirror of the
 * structs with it); needs no GPU. */
int ane_kernel_abi(const char *name, int64_t *size, int64_t *offsets, int max);

#ifdef __cplusplus
}
#endif

#endif /* ANE_KERNELS_H */
