// MFMA GEMM kernels for gfx950 and their launchers (internal to the GEMM;
// included by gemm.hip and by the gemm_*.hip files, which instantiate the
// launchers of disjoint sets of epilogues so that they compile in parallel).
//
// MFMA GEMM kernels (gfx950, v_mfma_f32_32x32x16_f16) with fused epilogues.
//
// Block = 4 waves in a 2x2 grid (or 8 in 2x4 for 256x256); block tile
// BM x BN, k-tile 64, each wave a sub-tile of 32x32 MFMA tiles.  Two k-loops:
//   gemm_ho_kernel  both operands K-major (forward, classifier, grouped MoE):
//                   HBM -> LDS by DMA, 2 stages, a hand-ordered instruction
//                   stream per 16-wide substep (see there);
//   gemm_kernel     transposed operands (the backward's dX / dW), staged
//                   through registers and a transposing LDS write, or the
//                   3-stage K-major variant.
// Both place the k-tile's one barrier before its last 16-wide substep;
// right after it the freed stage is refilled with a later k-tile, and LDS
// fragments are read one substep ahead of their MFMAs.
//
// MFMA 32x32 accumulator layout (CDNA3/CDNA4): lane l, register r holds
// row 8*(r/4) + 4*(l/32) + (r%4), column l%32.  Operand fragments: lane l
// supplies row l%32 of A (column l%32 of B) and 8 k-values; A and B use the
// same k-slot assignment, so the kernel's choice k = 16*s + 8*(l/32) + j
// only permutes the reduction order.
#pragma once
#include "gemm.h"

namespace ane {
namespace gemm_detail {

constexpr int BK = 64;

// ---- K-major operand: rows of 64 contiguous k -------------------------------
template <int R>
__device__ __forceinline__ void load_kmajor(half8 (&v)[R / 32], const half_t* base, int ld, int row0,
                                            int k0, int tid) {
#pragma unroll
  for (int i = 0; i < R / 32; i++) {
    int c = tid + 256 * i;
    int row = c >> 3, ch = c & 7;
    v[i] = ld_h8(base + (size_t)(row0 + row) * ld + k0 + ch * 8);
  }
}
template <int R>
__device__ __forceinline__ void store_kmajor(half_t* tile, const half8 (&v)[R / 32], int tid) {
#pragma unroll
  for (int i = 0; i < R / 32; i++) {
    int c = tid + 256 * i;
    int row = c >> 3, ch = c & 7;
    st_h8(tile + row * BK + swz(row, ch) * 8, v[i]);
  }
}

// ---- transposed operand: element (r, k) at k * ld + r ------------------------
// R/8 row-chunks x 8 k-chunks = R blocks of 8x8; thread tid < R owns one.
template <int R>
__device__ __forceinline__ void load_tmajor(half8 (&v)[8], const half_t* base, int ld, int row0, int k0,
                                            int tid) {
  if (tid < R) {
    int rc = tid % (R / 8), kc = tid / (R / 8);
#pragma unroll
    for (int j = 0; j < 8; j++) v[j] = ld_h8(base + (size_t)(k0 + kc * 8 + j) * ld + row0 + rc * 8);
  }
}
template <int R>
__device__ __forceinline__ void store_tmajor(half_t* tile, const half8 (&v)[8], int tid) {
  if (tid < R) {
    int rc = tid % (R / 8), kc = tid / (R / 8);
#pragma unroll
    for (int i = 0; i < 8; i++) {
      half8 w;
#pragma unroll
      for (int j = 0; j < 8; j++) w[j] = v[j][i];
      int row = rc * 8 + i;
      st_h8(tile + row * BK + swz(row, kc) * 8, w);
    }
  }
}

// ---- K-major operand, direct HBM -> LDS (global_load_lds_dwordx4) ----------
// One wave instruction fills 1 KB of LDS = 8 swizzled rows; lane l lands at
// slot l (row l/8, physical chunk l%8), so it fetches the logical chunk that
// the swizzle maps to that slot (the XOR swizzle is its own inverse).
//
// The load is issued from inline asm rather than __builtin_amdgcn_global_load_lds:
// the compiler's wait-count model treats a pending LDS DMA as an
// out-of-order LGKM event and then waits for lgkmcnt(0) before every use
// of an LDS fragment -- including the reads just issued for the next
// k-substep -- which exposes the full LDS latency on every substep.  The
// kernel waits for these loads itself (vmcnt, before the barrier that
// publishes the tile).
// M0 is named as clobbered (these kernels keep nothing else in it; clang
// warns that it is a reserved register).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// lds_addr: the destination's LDS byte address, wave-uniform
__device__ __forceinline__ void dma16_at(const half_t* gp, unsigned lds_addr) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds_addr), "v"(gp)
               : "memory", "m0");
}
__device__ __forceinline__ void dma16(const half_t* gp, half_t* lds_dst) {
  dma16_at(gp, __builtin_amdgcn_readfirstlane((unsigned)(size_t)(lds_ptr_t)lds_dst));
}
#pragma clang diagnostic pop
template <int R, int NW>
__device__ __forceinline__ void load_direct(half_t* tile, const half_t* base, int ld, int row0, int k0, int tid) {
  static_assert(R % (8 * NW) == 0, "each wave fills whole 8-row groups");
  const int lane = tid & 63, wave = tid >> 6;
#pragma unroll
  for (int it = 0; it < R / (8 * NW); it++) {
    const int gi = wave + NW * it;
    const int r = gi * 8 + (lane >> 3);
    const int lc = swz(r, lane & 7);
    dma16(base + (size_t)(row0 + r) * ld + k0 + lc * 8, tile + gi * 8 * BK);
  }
}

// Stage<R, transposed, waves>: issue() starts the HBM reads of one k-tile,
// commit() makes them LDS-resident (register path) -- the direct path has
// nothing to commit; its completion is awaited by wait_tile() before the
// barrier.
template <int R, bool T, int NW>
struct Stage;
template <int R, int NW>
struct Stage<R, false, NW> {
  __device__ __forceinline__ void issue(const half_t* b, int ld, int r0, int k0, half_t* tile, int tid) {
    load_direct<R, NW>(tile, b, ld, r0, k0, tid);
  }
  __device__ __forceinline__ void commit(half_t*, int) const {}
};
template <int R, int NW>
struct Stage<R, true, NW> {
  half8 v[8];
  __device__ __forceinline__ void issue(const half_t* b, int ld, int r0, int k0, half_t*, int tid) {
    load_tmajor<R>(v, b, ld, r0, k0, tid);
  }
  __device__ __forceinline__ void commit(half_t* tile, int tid) const { store_tmajor<R>(tile, v, tid); }
};

__device__ __forceinline__ void wait_tile() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// s_waitcnt vmcnt(N) with the other counters left alone (gfx9 encoding:
// vmcnt in bits [3:0] and [15:14], expcnt [6:4], lgkmcnt [11:8]).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Workgroup barrier without the release fence of __syncthreads(): for LDS
// written by global_load_lds that fence makes the compiler drain vmcnt to 0,
// which would also wait for the loads meant to stay in flight.  The caller
// has waited for the loads it needs; LDS reads/writes are drained here.
__device__ __forceinline__ void barrier_keep_loads() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__device__ __forceinline__ float softcap_f(float v, float cap) { return cap * tanhf(v / cap); }

// logistic function with the hardware reciprocal (1 ulp) instead of an IEEE
// division sequence; its results feed fp16 stores or fp32 gates
__device__ __forceinline__ float sigmoid_f(float x) { return __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }

// Block -> output tile: spread consecutive tiles of one XCD over a
// contiguous range (hardware deals block i to XCD i % 8), then walk groups
// of 8 M-tiles so neighbouring blocks share A rows and B columns in L2.
__device__ __forceinline__ void block_tile(int nbm, int nbn, int bid, int& bm, int& bn) {
  const int nb = nbm * nbn;
  if ((nb & 7) == 0) bid = (bid & 7) * (nb >> 3) + (bid >> 3);
  constexpr int GROUP = 8;
  const int group_size = GROUP * nbn;
  const int first_m = (bid / group_size) * GROUP;
  const int gm = min(nbm - first_m, GROUP);
  bm = first_m + (bid % group_size) % gm;
  bn = (bid % group_size) / gm;
}

// Fused epilogue of one wave's TM x TN grid of 32x32 accumulator tiles.
// The wave owns rows m0 + wm*WTM + [0, WTM) and columns n0 + wn*WTN + [0, WTN)
// of C; bm is the block's row-tile index (classifier partials); lds is
// free scratch once the main loop is done (classifier reduction).
// rr_s (rr variants): LDS, 1 / rms of the block's rows (EPI_CE_RR: columns),
// indexed from m0 (n0).  tg_pre (cross-entropy, optional): the target id of
// each of the lane's TN columns, loaded ahead.
template <int BN, int WTM, int WTN, int TM, int TN, int EPI>
__device__ __forceinline__ void epilogue(floatx16 (&acc)[TM][TN], const GemmArgs& g, const EpiParams& e, int m0,
                                         int n0, int bm, int wm, int wn, int lane, half_t* lds,
                                         const float* rr_s = nullptr, const int* tg_pre = nullptr) {
  const int rbase = m0 + wm * WTM + 4 * (lane >> 5);
  const int cbase = n0 + wn * WTN + (lane & 31);
#define ROW(i, r) (rbase + (i) * 32 + 8 * ((r) >> 2) + ((r) & 3))
#define COL(j) (cbase + (j) * 32)
#define LROW(i, r) (wm * WTM + 4 * (lane >> 5) + (i) * 32 + 8 * ((r) >> 2) + ((r) & 3))

  // rr of this lane's 16 rows of row tile i (rows 8 q + 4 (lane / 32) + 0..3
  // are consecutive: four 16-byte LDS reads, all issued before any use)
  auto rr_rows = [&](int i, float (&v)[16]) {
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const float4 f = *reinterpret_cast<const float4*>(rr_s + LROW(i, 4 * q));
      v[4 * q] = f.x; v[4 * q + 1] = f.y; v[4 * q + 2] = f.z; v[4 * q + 3] = f.w;
    }
  };
  if constexpr (EPI == EPI_STORE_H || EPI == EPI_STORE_H_RR) {
    half_t* C = (half_t*)e.C;
#pragma unroll
    for (int i = 0; i < TM; i++) {
      float sc[16];
#pragma unroll
      for (int r = 0; r < 16; r++) sc[r] = e.scale;
      if constexpr (EPI == EPI_STORE_H_RR) {
        rr_rows(i, sc);
#pragma unroll
        for (int r = 0; r < 16; r++) sc[r] *= e.scale;
      }
#pragma unroll
      for (int j = 0; j < TN; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) C[(size_t)ROW(i, r) * e.ldc + COL(j)] = (half_t)(acc[i][j][r] * sc[r]);
    }
  } else if constexpr (EPI == EPI_STORE_F) {
    // Loads of a tile's 16 old values are issued before any of its stores:
    // C may alias nothing else, but the compiler cannot know that, and a
    // load-use-store chain per element would serialise on memory latency.
    float* C = (float*)e.C;
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
      for (int j = 0; j < TN; j++) {
        const size_t base = (size_t)(rbase + i * 32) * e.ldc + COL(j);
        float old[16];
#pragma unroll
        for (int r = 0; r < 16; r++)
          old[r] = e.accumulate ? C[base + (size_t)(8 * (r >> 2) + (r & 3)) * e.ldc] : 0.f;
#pragma unroll
        for (int r = 0; r < 16; r++) C[base + (size_t)(8 * (r >> 2) + (r & 3)) * e.ldc] = old[r] + acc[i][j][r] * e.scale;
      }
  } else if constexpr (EPI == EPI_STORE_RS) {
    float* C = (float*)e.C;
#pragma unroll
    for (int i = 0; i < TM; i++) {
      float rs[16];
#pragma unroll
      for (int r = 0; r < 16; r++) rs[r] = e.rowscale[ROW(i, r)];
#pragma unroll
      for (int j = 0; j < TN; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) C[(size_t)ROW(i, r) * e.ldc + COL(j)] = acc[i][j][r] * rs[r];
    }
  } else if constexpr (EPI == EPI_STORE_W13) {
    // rows are 32-row blocks alternating W1 / W3 (block b even -> W1 row
    // (b/2)*32 + r%32, odd -> W3); C = W1 grad, C3 = W3 grad, both [H, ldc]
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
      for (int j = 0; j < TN; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
          int f = ROW(i, r);
          int b = f >> 5;
          float* dst = (b & 1) ? e.C3 : (float*)e.C;
          size_t idx = (size_t)((b >> 1) * 32 + (f & 31)) * e.ldc + COL(j);
          float v = acc[i][j][r] * e.scale;
          dst[idx] = e.accumulate ? dst[idx] + v : v;
        }
  } else if constexpr (EPI == EPI_LOGITS) {
    float* C = (float*)e.C;
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
      for (int j = 0; j < TN; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
          float v = acc[i][j][r];
          if (e.softcap) v = softcap_f(v, e.cap);
          C[(size_t)ROW(i, r) * e.ldc + COL(j)] = v;
        }
  } else if constexpr (EPI == EPI_RESID) {
    float* C = (float*)e.C;
    float* C2 = (float*)e.C2;
    const float alpha = e.alpha_ptr ? *e.alpha_ptr : e.alpha;
    const float beta = e.beta_ptr ? *e.beta_ptr : e.beta;
    const bool has_x0 = e.X0 != nullptr;
    // R usually IS C (in-place residual); all 16 reads of a tile precede its
    // writes, and each element is read and written by the same lane only.
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
      for (int j = 0; j < TN; j++) {
        const size_t base = (size_t)(rbase + i * 32) * e.ldc + COL(j);
        float rv[16], xv[16];
#pragma unroll
        for (int r = 0; r < 16; r++) rv[r] = e.R[base + (size_t)(8 * (r >> 2) + (r & 3)) * e.ldc];
#pragma unroll
        for (int r = 0; r < 16; r++) xv[r] = has_x0 ? e.X0[base + (size_t)(8 * (r >> 2) + (r & 3)) * e.ldc] : 0.f;
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const size_t idx = base + (size_t)(8 * (r >> 2) + (r & 3)) * e.ldc;
          const float v = alpha * rv[r] + acc[i][j][r] + beta * xv[r];
          C[idx] = v;
          if (C2) C2[idx] = v;
        }
      }
  } else if constexpr (EPI == EPI_SWIGLU || EPI == EPI_SWIGLU_RR) {
    static_assert(TN % 2 == 0, "SwiGLU epilogue pairs 32-column tiles");
    half_t* C = (half_t*)e.C;
    half_t* C2 = (half_t*)e.C2;
#pragma unroll
    for (int i = 0; i < TM; i++) {
      float rrv[16];
      if constexpr (EPI == EPI_SWIGLU_RR) rr_rows(i, rrv);
#pragma unroll
      for (int j = 0; j < TN; j += 2) {
        const int b = (COL(j) - (lane & 31)) >> 5;  // even 32-column block of W1
        const int hcol = (b >> 1) * 32 + (lane & 31);
#pragma unroll
        for (int r = 0; r < 16; r++) {
          float h1 = acc[i][j][r], h3 = acc[i][j + 1][r];
          if constexpr (EPI == EPI_SWIGLU_RR) {
            h1 *= rrv[r];
            h3 *= rrv[r];
          }
          float sg = sigmoid_f(h1);
          size_t row = (size_t)ROW(i, r);
          C[row * e.ldc + hcol] = (half_t)(h1 * sg * h3);
          if (C2) {
            C2[row * e.ldc2 + COL(j)] = (half_t)h1;
            C2[row * e.ldc2 + COL(j + 1)] = (half_t)h3;
          }
        }
      }
    }
  } else if constexpr (EPI == EPI_RELU2) {
    half_t* C = (half_t*)e.C;
    half_t* C2 = (half_t*)e.C2;
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
      for (int j = 0; j < TN; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
          float h = acc[i][j][r];
          size_t row = (size_t)ROW(i, r);
          float rl = h > 0.f ? h : 0.f;
          C[row * e.ldc + COL(j)] = (half_t)(rl * rl);
          if (C2) C2[row * e.ldc2 + COL(j)] = (half_t)h;
        }
  } else if constexpr (EPI == EPI_SWIGLU_BWD) {
    // columns are hidden units h; W1|W3 rows are interleaved by 32, so the
    // pre-activations of h sit at (h/32)*64 + h%32 (h1) and +32 (h3).
    // SwiGLU derivative as the llama2 variant's CPU restatement computes it.
    half_t* C = (half_t*)e.C;
    const half_t* H13 = (const half_t*)e.C2;
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
      for (int j = 0; j < TN; j++) {
        const int h = COL(j);
        const int c1 = (h >> 5) * 64 + (h & 31);
        float h1v[16], h3v[16];
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const size_t row = (size_t)ROW(i, r) * e.ldc2;
          h1v[r] = (float)H13[row + c1];
          h3v[r] = (float)H13[row + c1 + 32];
        }
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const float dg = acc[i][j][r];
          const float sg = sigmoid_f(h1v[r]);
          const size_t row = (size_t)ROW(i, r) * e.ldc;
          C[row + c1] = (half_t)(dg * h3v[r] * (sg + h1v[r] * sg * (1.f - sg)));
          C[row + c1 + 32] = (half_t)(dg * h1v[r] * sg);
        }
      }
  } else if constexpr (EPI == EPI_RELU2_BWD) {
    // reluSquaredBackwardSimple (ane/accel_stub.go:21-29): dh = dgate * 2 * relu(h)
    half_t* C = (half_t*)e.C;
    const half_t* H1 = (const half_t*)e.C2;
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
      for (int j = 0; j < TN; j++) {
        float hv[16];
#pragma unroll
        for (int r = 0; r < 16; r++) hv[r] = (float)H1[(size_t)ROW(i, r) * e.ldc2 + COL(j)];
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const float rl = hv[r] > 0.f ? hv[r] : 0.f;
          C[(size_t)ROW(i, r) * e.ldc + COL(j)] = (half_t)(acc[i][j][r] * 2.f * rl);
        }
      }
  } else if constexpr (EPI == EPI_SMEAR) {
    float* C = (float*)e.C;
    float* C2 = (float*)e.C2;
    const float alpha = e.alpha_ptr ? *e.alpha_ptr : e.alpha;
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
      for (int j = 0; j < TN; j++) {
        float cur[16], prev[16];
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int t = ROW(i, r);
          const size_t idx = (size_t)t * e.ldc + COL(j);
          cur[r] = e.X0[idx];
          prev[r] = (t % e.seq != 0) ? e.X0[idx - e.ldc] : 0.f;
        }
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const size_t idx = (size_t)ROW(i, r) * e.ldc + COL(j);
          const float ga = sigmoid_f(acc[i][j][r]);
          C[idx] = cur[r] + alpha * ga * prev[r];
          if (C2) C2[idx] = ga;
        }
      }
  } else if constexpr (EPI == EPI_RESID_NORM) {
    // llama2 residual (alpha 1, no x0) + the deferred norm's inputs: this
    // block's per-row sum of squares over its BN columns goes through LDS
    // (lane partials, then the WN waves of a row range) in a fixed order.
    float* C = (float*)e.C;
    half_t* C2 = (half_t*)e.C2;
    constexpr int WN = BN / WTN;
    constexpr int RS = WN * 32 + 1;  // padded LDS row of the lane partials
    float rs[TM][16];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
      for (int r = 0; r < 16; r++) rs[i][r] = 0.f;
#pragma unroll
    for (int j = 0; j < TN; j++) {
      const float gc = e.gain[COL(j)];
#pragma unroll
      for (int i = 0; i < TM; i++) {
        const size_t base = (size_t)(rbase + i * 32) * e.ldc + COL(j);
        float rv[16];
#pragma unroll
        for (int r = 0; r < 16; r++) rv[r] = e.R[base + (size_t)(8 * (r >> 2) + (r & 3)) * e.ldc];
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const float v = rv[r] + acc[i][j][r];
          C[base + (size_t)(8 * (r >> 2) + (r & 3)) * e.ldc] = v;
          C2[(size_t)ROW(i, r) * e.ldc2 + COL(j)] = (half_t)(v * gc);
          rs[i][r] += v * v;
        }
      }
    }
    __syncthreads();  // every wave is past its last read of the LDS stages
    float* red = reinterpret_cast<float*>(lds);  // [2 WTM][RS]
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
      for (int r = 0; r < 16; r++) red[LROW(i, r) * RS + wn * 32 + (lane & 31)] = rs[i][r];
    __syncthreads();
    for (int row = threadIdx.x; row < 2 * WTM; row += blockDim.x) {
      float sum = 0.f;
      for (int c = 0; c < WN * 32; c++) sum += red[row * RS + c];
      e.ssq_part[(size_t)(n0 / BN) * e.ssq_ld + m0 + row] = sum;
    }
  } else if constexpr (EPI == EPI_CE || EPI == EPI_CE_RR) {
    // rows = vocab ids (M == vocab), columns = tokens.  Each wave reduces
    // its BM/2 rows of every column to (max, sum exp(v - max)); lanes l and
    // l^32 hold the two row halves of one column; the two waves sharing a
    // column range merge through LDS into one partial per block row.
    float2* red = reinterpret_cast<float2*>(lds);  // [2][BN], main loop done
#pragma unroll
    for (int j = 0; j < TN; j++) {
      const int nl = wn * WTN + j * 32 + (lane & 31);
      const int n = n0 + nl;
      // the target's row relative to this lane's first row: a match is one
      // compare against a constant per register
      const int tsel = (tg_pre ? tg_pre[j] : (int)e.targets[n]) - ROW(0, 0);
      const bool hit = tsel >= 0 && tsel < 32 * TM && (tsel & 4) == 0;
      const float rr_col = EPI == EPI_CE_RR ? rr_s[nl] : 1.f;
      float mx = -INFINITY, tv = 0.f;
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
          float v = acc[i][j][r];
          if constexpr (EPI == EPI_CE_RR) v *= rr_col;
          if (e.softcap) v = softcap_f(v, e.cap);
          acc[i][j][r] = v;
          mx = fmaxf(mx, v);
          tv = (32 * i + 8 * (r >> 2) + (r & 3)) == tsel ? v : tv;
        }
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      // sum exp(v - max) as exp2(v log2e - max log2e): one FMA per value
      constexpr float kLog2e = 1.4426950408889634f;
      const float mxl = mx * kLog2e;
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) s += __builtin_amdgcn_exp2f(__builtin_fmaf(acc[i][j][r], kLog2e, -mxl));
      s += __shfl_xor(s, 32, 64);
      if (hit) e.tgt_logit[n] = tv;  // exactly one lane of the grid holds (tg, n)
      if (lane < 32) red[wm * BN + nl] = make_float2(mx, s);
    }
    __syncthreads();
    if (wm == 0) {
#pragma unroll
      for (int j = 0; j < TN; j++) {
        const int nl = wn * WTN + j * 32 + (lane & 31);
        if (lane < 32) {
          const float2 p0 = red[nl], p1 = red[BN + nl];
          const float M = fmaxf(p0.x, p1.x);
          e.partial[(size_t)bm * g.N + n0 + nl] =
              make_float2(M, p0.y * __expf(p0.x - M) + p1.y * __expf(p1.x - M));
        }
      }
    }
  } else if constexpr (EPI == EPI_DLOGITS) {
    // d = (softmax - onehot) * colscale[n], times (1 - tanh^2) under softcap.
    // C [M, ldc] and C2 (the same values transposed, [N, ldc2]) are each
    // optional; in C2, registers 4q .. 4q+3 hold 4 consecutive rows, stored
    // as one 8-byte chunk.
    half_t* C = (half_t*)e.C;
    half_t* C2 = (half_t*)e.C2;
    constexpr float kLog2e = 1.4426950408889634f;
#pragma unroll
    for (int j = 0; j < TN; j++) {
      const int n = COL(j);
      // target row and vocabulary end relative to this lane's first row:
      // per register one compare against a constant each
      const int tsel = e.targets[n] - ROW(0, 0), vend = e.vocab - ROW(0, 0);
      const float lsel = e.lse[n] * kLog2e, cs = e.colscale[n];
#pragma unroll
      for (int i = 0; i < TM; i++) {
        half_t hv[16];
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int mo = 32 * i + 8 * (r >> 2) + (r & 3);
          float v = acc[i][j][r], dsc = 1.f;
          if (e.softcap) {
            float th = tanhf(v / e.cap);
            v = e.cap * th;
            dsc = 1.f - th * th;
          }
          float d = __builtin_amdgcn_exp2f(__builtin_fmaf(v, kLog2e, -lsel)) - (mo == tsel ? 1.f : 0.f);
          d = mo < vend ? d * cs * dsc : 0.f;
          hv[r] = (half_t)d;
          if (C) C[(size_t)ROW(i, r) * e.ldc + n] = hv[r];
        }
        if (C2) {
#pragma unroll
          for (int q = 0; q < 4; q++) {
            half4 w;
            w[0] = hv[4 * q]; w[1] = hv[4 * q + 1]; w[2] = hv[4 * q + 2]; w[3] = hv[4 * q + 3];
            *reinterpret_cast<half4*>(C2 + (size_t)n * e.ldc2 + ROW(i, 4 * q)) = w;
          }
        }
      }
    }
  }
#undef ROW
#undef COL
#undef LROW
}

// NW = 4: waves 2 x 2, one wave per SIMD.  NW = 8: waves 2 x 4, two waves
// per SIMD, so one wave's barrier wait and LDS reads overlap the other's
// MFMAs (wave tile (BM/2) x (BN/4)).  NS = LDS stages: with NS = 3 the
// HBM->LDS loads run two k-tiles ahead of the MFMAs (K-major operands only).
template <int BM, int BN, bool AT, bool BT, int EPI, int NW, int NS>
__global__ __launch_bounds__(64 * NW) void gemm_kernel(GemmArgs g, EpiParams e) {
  constexpr int WN = NW / 2;                 // waves along N (2 along M)
  constexpr int WTM = BM / 2, WTN = BN / WN; // wave tile
  constexpr int TM = WTM / 32, TN = WTN / 32;
  static_assert(TN >= 1 && TM >= 1, "wave tile must hold 32x32 MFMA tiles");
  static_assert(NS == 2 || (NS == 3 && !AT && !BT), "3 stages need direct loads on both operands");
  constexpr int STAGE = (BM + BN) * BK;
  constexpr int LPT = (BM + BN) / (8 * NW);  // direct-load instructions per wave per k-tile
  __shared__ __attribute__((aligned(16))) half_t lds[NS * STAGE];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  int bm, bn;
  block_tile(g.M / BM, g.N / BN, blockIdx.x, bm, bn);
  int m0 = bm * BM;
  const int n0 = bn * BN;
  const half_t* Bp = g.B;
  if (g.grp) {  // grouped: row tile bm of the valid tiles, B of its group
    if (bm >= g.grp[0]) return;  // whole block, before any LDS traffic
    m0 = g.grp[1 + 2 * bm];
    Bp += (size_t)g.grp[2 + 2 * bm] * g.b_group_stride;
  }

  floatx16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

  Stage<BM, AT, NW> sa;
  Stage<BN, BT, NW> sb;
  const int nk = g.K / BK;
  // Prologue: tile 0 in LDS stage 0; tiles 1 .. NS-1 also fetched (direct
  // path: into their stages; register path: tile 1 waits in registers for
  // the first iteration's commit).
  sa.issue(g.A, g.lda, m0, 0, lds, tid);
  sb.issue(Bp, g.ldb, n0, 0, lds + BM * BK, tid);
  sa.commit(lds, tid);
  sb.commit(lds + BM * BK, tid);
#pragma unroll
  for (int p = 1; p < NS; p++) {
    if (p < nk) {
      sa.issue(g.A, g.lda, m0, p * BK, lds + p * STAGE, tid);
      sb.issue(Bp, g.ldb, n0, p * BK, lds + p * STAGE + BM * BK, tid);
    }
  }
  wait_tile();
  __syncthreads();

  const int frow = lane & 31, fch = lane >> 5;
  int arow[TM], brow[TN];
#pragma unroll
  for (int i = 0; i < TM; i++) arow[i] = wm * WTM + i * 32 + frow;
#pragma unroll
  for (int j = 0; j < TN; j++) brow[j] = wn * WTN + j * 32 + frow;

  // Fragments are double-buffered one 16-wide k-substep ahead of the MFMAs
  // that use them.  sched_barrier fences keep the compiler from sinking the
  // LDS reads next to their first use (which it otherwise does to save
  // registers, exposing the LDS latency every two MFMAs).
  half8 fa[2][TM], fb[2][TN];
  auto load_frags = [&](half8 (&a)[TM], half8 (&b)[TN], const half_t* st, int s) {
    const int ch = 2 * s + fch;
#pragma unroll
    for (int i = 0; i < TM; i++) a[i] = ld_h8(st + arow[i] * BK + swz(arow[i], ch) * 8);
#pragma unroll
    for (int j = 0; j < TN; j++) b[j] = ld_h8(st + BM * BK + brow[j] * BK + swz(brow[j], ch) * 8);
  };
  auto mfmas = [&](const half8 (&a)[TM], const half8 (&b)[TN]) {
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
      for (int j = 0; j < TN; j++)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], acc[i][j], 0, 0, 0);
  };
  load_frags(fa[0], fb[0], lds, 0);

  for (int kt = 0; kt < nk; kt++) {
    half_t* cur = lds + (kt % NS) * STAGE;
    half_t* nxt = lds + ((kt + 1) % NS) * STAGE;
#pragma unroll
    for (int s = 0; s + 1 < BK / 16; s++) {
      load_frags(fa[(s + 1) & 1], fb[(s + 1) & 1], cur, s + 1);
      __builtin_amdgcn_sched_barrier(0);
      mfmas(fa[s & 1], fb[s & 1]);
      __builtin_amdgcn_sched_barrier(0);
    }
    // The last substep's fragments are in registers: once every wave has
    // passed this barrier, stage kt is free.  So the barrier sits before the
    // last substep's MFMAs, which then hide the first LDS reads of tile
    // kt+1 and the issue of the HBM reads of tile kt+NS into stage kt --
    // those get four substeps of MFMA work to land.
    if (kt + 1 < nk) {
      sa.commit(nxt, tid);  // register path: tile kt+1, fetched one iteration ago
      sb.commit(nxt + BM * BK, tid);
      // tile kt+1 must have landed; with 3 stages tile kt+2 may stay in flight
      if constexpr (NS == 3) {
        if (kt + 2 < nk)
          wait_vm<LPT>();
        else
          wait_tile();
        barrier_keep_loads();
      } else {
        wait_tile();
        __syncthreads();
      }
      load_frags(fa[0], fb[0], nxt, 0);
      if (kt + NS < nk) {
        sa.issue(g.A, g.lda, m0, (kt + NS) * BK, cur, tid);
        sb.issue(Bp, g.ldb, n0, (kt + NS) * BK, cur + BM * BK, tid);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    mfmas(fa[1], fb[1]);
    __builtin_amdgcn_sched_barrier(0);
  }
  // the epilogue of the CE variant reuses LDS as scratch
  if constexpr (EPI == EPI_CE) __syncthreads();

  epilogue<BN, WTM, WTN, TM, TN, EPI>(acc, g, e, m0, n0, bm, wm, wn, lane, lds);
}

// ---- K-major operands: hand-ordered k-loop ---------------------------------
// Both operands K-major (the forward, the classifier and the grouped MoE
// GEMMs), HBM -> LDS by DMA, 2 LDS stages.  Waves 2 x NW/2; each 16-wide
// k-substep is TM x TN MFMAs, TM + TN LDS fragment reads (the next
// substep's) and, in two of the four substeps, the HBM -> LDS loads of a
// later k-tile.  The instruction order inside a substep is fixed by
// sched_barrier fences: the reads and loads are spread evenly between the
// MFMAs, so the MFMA stream never waits behind a burst of memory
// instructions -- with one wave per SIMD (the 4-wave 256x256 tile) nothing
// else would hide such a stall.  Per tile kt:
//   s0: reads of s1; B half of tile kt+1's loads into stage kt+1
//   s1: reads of s2
//   s2: reads of s3, all in the first half (they must land before the barrier)
//   wait for tile kt+1, barrier (stage kt is free from here)
//   s3: reads of s0 of tile kt+1; A half of tile kt+2's loads into stage kt
// so a tile's loads are issued 2-3 substeps before the barrier that needs
// them.  One straight-line body serves every tile (the register allocator
// keeps the accumulators in place only without diverging copies of the MFMA
// stream): the last tile's s3 still reads the other stage (in bounds,
// unused) and still passes the barrier.
//
// Loads use the scalar-base form of global_load_lds: load q of a wave
// fills rows 8 (w + NW q) .. +7 of the operand's tile (w = the wave), so the
// row part of the address is wave-uniform (an SGPR pair) and the per-lane
// part -- row lane/8 of the 8, the swizzled 16-byte chunk -- is a fixed
// 32-bit offset; the chunk's swizzle depends on q only through
// (w + NW q) mod 8, i.e. on q mod 8/NW.
__device__ __forceinline__ void dma16_s(const half_t* sbase, unsigned voff, unsigned lds_addr) {
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds_addr), "v"(voff),
               "s"(sbase)
               : "memory", "m0");
#pragma clang diagnostic pop
}

// Chunk swizzle of an M-major LDS tile (rows of CPR 16-byte chunks): the
// four 16-byte chunks a transposed read takes from one row move with the row
// (rows r and r + 4 share a position: a two-way bank conflict at most).
template <int CPR>
__device__ __forceinline__ int swt(int row) {
  return CPR >= 16 ? 4 * (row & 3) : 4 * (row & 1);
}
// The 32 x 16 operand (rows r0 + lane % 32, k = 16 s + 8 (lane / 32) + [0, 8))
// of an M-major tile [64 k][W] (W halves per row, swizzled by swt):
// lane 16 g + 4 e + q points at k-row 16 s + 8 (g / 2) + e (+ 4 for the
// second read), halves r0 + 16 (g % 2) + 4 q .. + 3.
template <int W>
__device__ __forceinline__ half8 tr_frag(const half_t* tile, int r0, int s, int lane) {
  constexpr int CPR = W / 8;
  const int g = lane >> 4, e = (lane >> 2) & 3, q = lane & 3;
  const int col = r0 + 16 * (g & 1) + 4 * q;
  const int row0 = 16 * s + 8 * (g >> 1) + e, row1 = row0 + 4;
  const short4v lo = ds_read_tr16(tile + row0 * W + (((col >> 3) ^ swt<CPR>(row0)) << 3) + (col & 7));
  const short4v hi = ds_read_tr16(tile + row1 * W + (((col >> 3) ^ swt<CPR>(row1)) << 3) + (col & 7));
  const short4v lohi[2] = {lo, hi};
  return __builtin_bit_cast(half8, lohi);
}

// PERSIST: a grid of fewer blocks than tiles, block b taking tiles b, b +
// gridDim.x, ... (K-major, one split, no groups): each next tile's first two
// k-tiles (and its rr partials) are requested before the current tile's
// epilogue runs, which then overlaps their latency instead of a block
// launch plus a prologue following it.  The epilogue's LDS scratch (the
// cross-entropy merge) and 1/rms rows are separate from the stages.
// The kernel body is a device function so that the code object's extern "C"
// entry points (module_gemm.hip) share it with the templated kernel.
template <int BM, int BN, int EPI, int NW, bool TRA = false, bool TRB = false, bool PERSIST = false>
__device__ __forceinline__ void gemm_ho_body(const GemmArgs& g, const EpiParams& e) {
  static_assert(!PERSIST || (!TRA && !TRB), "persistent form: K-major operands only");
  constexpr int WN = NW / 2;
  constexpr int WTM = BM / 2, WTN = BN / WN, TM = WTM / 32, TN = WTN / 32;
  constexpr int STAGE = (BM + BN) * BK;  // halves
  constexpr int LA = BM / (8 * NW), LB = BN / (8 * NW);  // loads per wave per k-tile
  constexpr int NMF = TM * TN, NRD = TM + TN;             // per substep
  constexpr int NV = 8 / NW;
  static_assert(TM >= 1 && TN >= 1 && LA >= 1 && LB >= 1, "tile too small for the wave grid");
  static_assert(!epi_rr(EPI) || (kRrMaxParts + 1) * (EPI == EPI_CE_RR ? BN : BM) * 4 <= 4 * STAGE,
                "rr staging exceeds the LDS stages");
  static_assert(EPI != EPI_RESID_NORM || BM * (WN * 32 + 1) * 4 <= 4 * STAGE, "row sums exceed the LDS stages");
  __shared__ __attribute__((aligned(16))) half_t lds[2 * STAGE];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  // split-K: blocks [s * tiles, (s+1) * tiles) reduce the s-th K range
  const int ntiles = (g.M / BM) * (g.N / BN);
  int bid = blockIdx.x, ks = 0;
  if (g.splits > 1) {
    ks = bid / ntiles;
    bid -= ks * ntiles;
  }
  int bm, bn;
  block_tile(g.M / BM, g.N / BN, bid, bm, bn);
  int m0 = bm * BM;
  int n0 = bn * BN;
  const half_t* Bp = g.B;
  if (g.grp) {  // grouped: row tile bm of the valid tiles, B of its group
    if (bm >= g.grp[0]) return;  // whole block, before any LDS traffic
    m0 = g.grp[1 + 2 * bm];
    Bp += (size_t)g.grp[2 + 2 * bm] * g.b_group_stride;
  }
  const int nk = g.K / BK / g.splits;
  const size_t koff = (size_t)ks * nk * BK;

  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  const unsigned lds0 = (unsigned)(size_t)(lds_ptr_t)lds;
  unsigned voa[NV], vob[NV];
#pragma unroll
  for (int v = 0; v < NV; v++) {
    const int lc = (lane & 7) ^ (((lane >> 3) ^ (wave + NW * v)) & 7);
    voa[v] = (unsigned)(((lane >> 3) * g.lda + lc * 8) * 2);
    vob[v] = (unsigned)(((lane >> 3) * g.ldb + lc * 8) * 2);
  }
  // M-major operands (TRA / TRB: stored [K][M], the tile kept [64 k][BM] in
  // LDS): one load instruction fills 1 KB = RPI whole k-rows; lane l lands
  // at row l / CPR, physical chunk l % CPR, so it fetches the logical chunk
  // swt maps there.  Row gi * RPI + r has the swizzle of r (RPI >= 4), or of
  // r and the parity of gi, which is the wave's (RPI == 2: gi = wave + NW q).
  auto tr_voff = [&](int W, int ld) {
    const int cpr = W / 8, r = lane / cpr, row = (512 / W) * wave + r;
    const int c = (lane % cpr) ^ (cpr >= 16 ? 4 * (row & 3) : 4 * (row & 1));
    return (unsigned)((r * ld + c * 8) * 2);
  };
  if constexpr (TRA) voa[0] = tr_voff(BM, g.lda);
  if constexpr (TRB) vob[0] = tr_voff(BN, g.ldb);
  const half_t* abase = TRA ? g.A + koff * g.lda + m0 : g.A + (size_t)m0 * g.lda + koff;
  const half_t* bbase = TRB ? Bp + koff * g.ldb + n0 : Bp + (size_t)n0 * g.ldb + koff;
  int tile = bid;  // PERSIST: the tile in hand
  auto dma_a = [&](int q, int kt, int st) {
    const int gi = wave_s + NW * q;
    if constexpr (TRA)
      dma16_s(abase + (size_t)(kt * BK + gi * (512 / BM)) * g.lda, voa[0], lds0 + 2u * (unsigned)(st * STAGE + gi * 512));
    else
      dma16_s(abase + (size_t)(gi * 8) * g.lda + kt * BK, voa[q % NV],
              lds0 + 2u * (unsigned)(st * STAGE + gi * 8 * BK));
  };
  auto dma_b = [&](int q, int kt, int st) {
    const int gi = wave_s + NW * q;
    if constexpr (TRB)
      dma16_s(bbase + (size_t)(kt * BK + gi * (512 / BN)) * g.ldb, vob[0],
              lds0 + 2u * (unsigned)(st * STAGE + BM * BK + gi * 512));
    else
      dma16_s(bbase + (size_t)(gi * 8) * g.ldb + kt * BK, vob[q % NV],
              lds0 + 2u * (unsigned)(st * STAGE + BM * BK + gi * 8 * BK));
  };

  // rr variants: the partial sums of squares of the block's rows (EPI_CE_RR:
  // token columns) are loaded into registers before the prologue (the
  // prologue's wait covers them) and combined in LDS after the main loop.
  constexpr bool RR = epi_rr(EPI);
  constexpr int NRR = EPI == EPI_CE_RR ? BN : BM;
  // RR_PRO (the 8-wave 256x256 tiles, one block per CU, whose LDS has room
  // for it): rr is formed in the prologue, thread t < NRR summing row t's
  // partials (loads in flight with the prologue's, added after its wait, in
  // part order) into its own LDS slot, which the prologue's barrier
  // publishes; the epilogue then needs no extra barrier (three extra
  // barriers and the partials staged through LDS after the main loop cost
  // the W1|W3 GEMM ~6 us of 55).  Otherwise the partials are loaded here and
  // combined after the main loop.
  constexpr bool RR_PRO = RR && NW == 8 && NRR <= 64 * NW;
  static_assert(!PERSIST || !RR || RR_PRO, "persistent form: rr formed in the prologue only");
  static_assert(!PERSIST || EPI != EPI_RESID_NORM, "persistent form: no epilogue that stages through the LDS stages");
  // PERSIST: two rr buffers (the tile in hand's, the next one's) and the
  // cross-entropy merge scratch of its own
  __shared__ float rs_pro[RR_PRO ? (PERSIST ? 2 : 1) * NRR : 1];
  constexpr bool CE_SCRATCH = PERSIST && (EPI == EPI_CE || EPI == EPI_CE_RR);
  __shared__ __attribute__((aligned(16))) float2 ce_red[CE_SCRATCH ? 2 * BN : 1];
  int rbuf = 0;
  // PERSIST: the rr partials come in by the same LDS DMA as the operands
  // (one 1 KB row segment per partial), so no registers hold them across
  // the epilogue that runs while they are in flight
  constexpr bool RR_STAGE = PERSIST && RR_PRO;
  static_assert(!RR_STAGE || NRR == 256, "rr staging: one 16-byte load per lane per partial");
  __shared__ __attribute__((aligned(16))) float rr_stage[RR_STAGE ? kRrMaxParts * NRR : 1];
  constexpr int RPER = RR && !RR_PRO ? (NRR * kRrMaxParts + 64 * NW - 1) / (64 * NW) : 1;
  float rrv[RPER];
  float rrl[RR_PRO && !RR_STAGE ? kRrMaxParts : 1];
  // PERSIST, cross-entropy: the target ids of the tile being set up (loaded
  // with its prologue) and of the tile in hand
  int tg_next[CE_SCRATCH ? TN : 1], tg_cur[CE_SCRATCH ? TN : 1];
  if constexpr (RR && !RR_PRO) {
    const int r0 = EPI == EPI_CE_RR ? n0 : m0;
#pragma unroll
    for (int k = 0; k < RPER; k++) {
      const int idx = tid + k * 64 * NW, p = idx / NRR;
      rrv[k] = p < e.rr_nparts ? e.rr_part[(size_t)p * e.rr_ld + r0 + idx % NRR] : 0.f;
    }
  }

  floatx16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

  const int frow = lane & 31, fch = lane >> 5;
  // fragment reads of one substep, in the order the MFMAs (i-major)
  // consume them: a0, b0 .. b(TN-1), then a1 .. a(TM-1)
  auto read_frag = [&](half8 (&a)[TM], half8 (&b)[TN], const half_t* st, int s, int q) {
    const int ch = 2 * s + fch;
    if (q == 0 || q > TN) {
      const int i = q == 0 ? 0 : q - TN;
      if constexpr (TRA) {
        a[i] = tr_frag<BM>(st, wm * WTM + i * 32, s, lane);
      } else {
        const int row = wm * WTM + i * 32 + frow;
        a[i] = ld_h8(st + row * BK + swz(row, ch) * 8);
      }
    } else {
      if constexpr (TRB) {
        b[q - 1] = tr_frag<BN>(st + BM * BK, wn * WTN + (q - 1) * 32, s, lane);
      } else {
        const int row = wn * WTN + (q - 1) * 32 + frow;
        b[q - 1] = ld_h8(st + BM * BK + row * BK + swz(row, ch) * 8);
      }
    }
  };
  // one substep: MFMA p of the TM x TN grid is followed by the reads r with
  // r * NMF / NRD == p (EARLY: r * NMF / (2 NRD) == p) and, when dma_on, the
  // loads d with d * NMF / ND == p (DMA 1: A half of tile dkt into stage
  // dst, 2: B half)
  auto substep = [&](auto early_c, auto dma_c, const half8 (&ca)[TM], const half8 (&cb)[TN], half8 (&na)[TM],
                     half8 (&nb)[TN], const half_t* rs, int rsub, bool dma_on, int dkt, int dst) {
    constexpr bool EARLY = decltype(early_c)::value;
    constexpr int DMA = decltype(dma_c)::value;
    constexpr int ND = DMA == 1 ? LA : (DMA == 2 ? LB : 0);
#pragma unroll
    for (int p = 0; p < NMF; p++) {
      const int i = p / TN, j = p % TN;
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ca[i], cb[j], acc[i][j], 0, 0, 0);
#pragma unroll
      for (int r = 0; r < NRD; r++)
        if ((EARLY ? r * NMF / (2 * NRD) : r * NMF / NRD) == p) read_frag(na, nb, rs, rsub, r);
      if (dma_on) {
#pragma unroll
        for (int d = 0; d < ND; d++)
          if (d * NMF / (ND > 0 ? ND : 1) == p) {
            if constexpr (DMA == 1) dma_a(d, dkt, dst);
            if constexpr (DMA == 2) dma_b(d, dkt, dst);
          }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  using F = std::false_type;
  using T = std::true_type;
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;

  // prologue: tiles 0 and 1 in flight, wait for both
  auto prologue_loads = [&]() {
#pragma unroll
    for (int q = 0; q < LA; q++) dma_a(q, 0, 0);
#pragma unroll
    for (int q = 0; q < LB; q++) dma_b(q, 0, 0);
    if (nk > 1) {
#pragma unroll
      for (int q = 0; q < LA; q++) dma_a(q, 1, 1);
#pragma unroll
      for (int q = 0; q < LB; q++) dma_b(q, 1, 1);
    }
    if constexpr (RR_STAGE) {
      const int r0 = EPI == EPI_CE_RR ? n0 : m0;
      const unsigned rr0 = (unsigned)(size_t)(lds_ptr_t)rr_stage;
#pragma unroll
      for (int q = 0; q < kRrMaxParts / NW; q++) {
        const int p = wave_s + NW * q;
        if (p < e.rr_nparts)
          dma16_at(reinterpret_cast<const half_t*>(e.rr_part + (size_t)p * e.rr_ld + r0 + lane * 4),
                   rr0 + (unsigned)(p * NRR * 4));
      }
    } else if constexpr (RR_PRO) {
      const int r0 = EPI == EPI_CE_RR ? n0 : m0;
      if (tid < NRR) {
#pragma unroll
        for (int p = 0; p < kRrMaxParts; p++)
          rrl[p] = p < e.rr_nparts ? e.rr_part[(size_t)p * e.rr_ld + r0 + tid] : 0.f;
      }
    }
    if constexpr (CE_SCRATCH) {
#pragma unroll
      for (int j = 0; j < TN; j++) tg_next[j] = e.targets[n0 + wn * WTN + j * 32 + (lane & 31)];
    }
  };
  prologue_loads();
  // self-prefetch: slice blockIdx.x of kPfBlocks, at most kPfLoads 16-byte
  // loads per thread (the host sizes pf_bytes), in flight with the
  // prologue's loads and waited for with them
  uint4 pfv[kPfLoads];
  bool pf_on = !TRA && !TRB && g.pf_bytes >= 16 && blockIdx.x < kPfBlocks;
  if (pf_on) {
    const uint4* q = reinterpret_cast<const uint4*>(g.pf);
    const size_t n16 = g.pf_bytes / 16, per = (n16 + kPfBlocks - 1) / kPfBlocks;
    const size_t i0 = blockIdx.x * per, i1 = min(n16, i0 + per);
#pragma unroll
    for (int u = 0; u < kPfLoads; u++) {
      const size_t i = i0 + (size_t)u * (64 * NW) + tid;
      pfv[u] = i < i1 ? q[i] : make_uint4(0, 0, 0, 0);  // lanes past the slice load nothing
    }
  }
  for (;;) {  // one pass, or (PERSIST) one per tile of the block
    wait_tile();
    if (pf_on) {
      uint32_t x = 0;
#pragma unroll
      for (int u = 0; u < kPfLoads; u++) x ^= pfv[u].x ^ pfv[u].y ^ pfv[u].z ^ pfv[u].w;
      asm volatile("" ::"v"(x));
      pf_on = false;
    }
    if constexpr (RR_STAGE) {
      barrier_keep_loads();  // every wave's partial rows are in
      if (tid < NRR) {
        float sum = 0.f;
#pragma unroll
        for (int p = 0; p < kRrMaxParts; p++)
          if (p < e.rr_nparts) sum += rr_stage[p * NRR + tid];
        rs_pro[rbuf * NRR + tid] = 1.0f / sqrtf(sum / (float)e.rr_dim + 1e-5f);
      }
    } else if constexpr (RR_PRO) {
      if (tid < NRR) {
        float sum = 0.f;
#pragma unroll
        for (int p = 0; p < kRrMaxParts; p++)
          if (p < e.rr_nparts) sum += rrl[p];
        rs_pro[rbuf * NRR + tid] = 1.0f / sqrtf(sum / (float)e.rr_dim + 1e-5f);
      }
    }
    if constexpr (CE_SCRATCH) {
#pragma unroll
      for (int j = 0; j < TN; j++) tg_cur[j] = tg_next[j];
    }
    __syncthreads();
    half8 fa[2][TM], fb[2][TN];
#pragma unroll
    for (int q = 0; q < NRD; q++) read_frag(fa[0], fb[0], lds, 0, q);
    __builtin_amdgcn_sched_barrier(0);

    for (int kt = 0; kt < nk; kt++) {
      const half_t* cur = lds + (kt & 1) * STAGE;
      const half_t* nxt = lds + ((kt + 1) & 1) * STAGE;
      substep(F{}, I2{}, fa[0], fb[0], fa[1], fb[1], cur, 1, kt >= 1 && kt + 1 < nk, kt + 1, (kt + 1) & 1);
      substep(F{}, I0{}, fa[1], fb[1], fa[0], fb[0], cur, 2, false, 0, 0);
      substep(T{}, I0{}, fa[0], fb[0], fa[1], fb[1], cur, 3, false, 0, 0);
      wait_tile();           // this wave's loads of tile kt+1
      barrier_keep_loads();  // everyone's, and every read of stage kt is done
      substep(F{}, I1{}, fa[1], fb[1], fa[0], fb[0], nxt, 0, kt + 2 < nk, kt + 2, kt & 1);
    }
    if constexpr (PERSIST) {
      // the next tile's first k-tiles (and rr partials, target ids) go out
      // before this tile's epilogue, once every wave is past its last read
      // of the stages
      const int bm_c = bm, m0_c = m0, n0_c = n0;
      const float* rr_c = RR_PRO ? rs_pro + rbuf * NRR : nullptr;
      const int next = tile + (int)gridDim.x;
      const bool more = next < ntiles;
      if (more) {
        __syncthreads();
        tile = next;
        block_tile(g.M / BM, g.N / BN, tile, bm, bn);
        m0 = bm * BM;
        n0 = bn * BN;
        abase = g.A + (size_t)m0 * g.lda;
        bbase = g.B + (size_t)n0 * g.ldb;
        prologue_loads();
      }
      epilogue<BN, WTM, WTN, TM, TN, EPI>(acc, g, e, m0_c, n0_c, bm_c, wm, wn, lane,
                                          CE_SCRATCH ? reinterpret_cast<half_t*>(ce_red) : lds, rr_c,
                                          CE_SCRATCH ? tg_cur : nullptr);
      if (!more) return;
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
          for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;
      rbuf ^= 1;
      continue;
    }
    // the epilogue of the CE variant reuses LDS as scratch
    if constexpr (EPI == EPI_CE || EPI == EPI_CE_RR) __syncthreads();
    const float* rr_s = RR_PRO ? rs_pro : nullptr;
    if constexpr (RR && !RR_PRO) {
      // LDS: partials [kRrMaxParts][NRR], then rr [NRR]; rr = 1 / rms over
      // rr_dim columns, the parts added in order
      if constexpr (EPI != EPI_CE_RR) __syncthreads();
      float* pl = reinterpret_cast<float*>(lds);
      float* rs = pl + kRrMaxParts * NRR;
#pragma unroll
      for (int k = 0; k < RPER; k++) {
        const int idx = tid + k * 64 * NW;
        if (idx < kRrMaxParts * NRR) pl[idx] = rrv[k];
      }
      __syncthreads();
      for (int row = tid; row < NRR; row += 64 * NW) {
        float sum = 0.f;
        for (int p = 0; p < e.rr_nparts; p++) sum += pl[p * NRR + row];
        rs[row] = 1.0f / sqrtf(sum / (float)e.rr_dim + 1e-5f);
      }
      __syncthreads();
      rr_s = rs;
    }
    if constexpr (EPI == EPI_STORE_F) {
      if (g.splits > 1) {  // this split's slice of the workspace (C = ws, ldc = N)
        EpiParams es = e;
        es.C = (float*)e.C + (size_t)ks * g.M * g.N;
        epilogue<BN, WTM, WTN, TM, TN, EPI>(acc, g, es, m0, n0, bm, wm, wn, lane, lds);
        return;
      }
    }
    epilogue<BN, WTM, WTN, TM, TN, EPI>(acc, g, e, m0, n0, bm, wm, wn, lane, lds, rr_s);
    return;
  }
}

template <int BM, int BN, int EPI, int NW, bool TRA = false, bool TRB = false, bool PERSIST = false>
__global__ __launch_bounds__(64 * NW) void gemm_ho_kernel(GemmArgs g, EpiParams e) {
  gemm_ho_body<BM, BN, EPI, NW, TRA, TRB, PERSIST>(g, e);
}

// Sum of the split-K workspace slices in split order, then the epilogue:
// STORE_F (C = [C +] scale * sum), STORE_H, STORE_W13 (interleaved W1|W3
// rows scattered to C / C3).  Four consecutive columns per thread.
template <int EPI, bool VEC>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* ws, int splits, int M, int N, EpiParams e) {
  const size_t MN = (size_t)M * N;
  const size_t i4 = ((size_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i4 >= MN) return;
  const int m = (int)(i4 / N), n = (int)(i4 % N);
  // every slice's load in flight at once (the workspace is not read again),
  // then the sum in split order
  float4 w[kMaxSplits];
#pragma unroll
  for (int s = 0; s < kMaxSplits; s++)
    if (s < splits) w[s] = ld_nt_f4(ws + (size_t)s * MN + i4);
  float4 v = w[0];
#pragma unroll
  for (int s = 1; s < kMaxSplits; s++)
    if (s < splits) {
      v.x += w[s].x; v.y += w[s].y; v.z += w[s].z; v.w += w[s].w;
    }
  float o[4] = {v.x * e.scale, v.y * e.scale, v.z * e.scale, v.w * e.scale};
  if constexpr (EPI == EPI_STORE_H) {
    half4 h;
#pragma unroll
    for (int u = 0; u < 4; u++) h[u] = (half_t)o[u];
    *reinterpret_cast<half4*>((half_t*)e.C + (size_t)m * e.ldc + n) = h;
    return;
  } else {
    float* dst = (float*)e.C;
    int row = m;
    if constexpr (EPI == EPI_STORE_W13) {
      const int b = m >> 5;
      dst = (b & 1) ? e.C3 : (float*)e.C;
      row = (b >> 1) * 32 + (m & 31);
    }
    float* p = dst + (size_t)row * e.ldc + n;
    if constexpr (VEC) {
      float4 r = make_float4(o[0], o[1], o[2], o[3]);
      if (e.accumulate) {
        const float4 old = *reinterpret_cast<const float4*>(p);
        r.x += old.x; r.y += old.y; r.z += old.z; r.w += old.w;
      }
      *reinterpret_cast<float4*>(p) = r;
    } else {
#pragma unroll
      for (int u = 0; u < 4; u++) p[u] = e.accumulate ? p[u] + o[u] : o[u];
    }
  }
}

template <bool AT, bool BT, int EPI, int BM, int BN, int NW = 4, int NS = 2>
hipError_t launch_tile(const GemmArgs& g, const EpiParams& e, hipStream_t s) {
  dim3 grid((g.M / BM) * (g.N / BN));
  hipLaunchKernelGGL((gemm_kernel<BM, BN, AT, BT, EPI, NW, NS>), grid, dim3(64 * NW), 0, s, g, e);
  return hipGetLastError();
}

#define LAUNCH_HO(BM_, BN_, NW_) \
  hipLaunchKernelGGL((gemm_ho_kernel<BM_, BN_, EPI, NW_>), grid, dim3(64 * NW_), 0, s, g, e)
#define LAUNCH_HOT(BM_, BN_, NW_) \
  hipLaunchKernelGGL((gemm_ho_kernel<BM_, BN_, EPI, NW_, AT, BT>), grid, dim3(64 * NW_), 0, s, g, e)

// Blocks of a persistent launch (opt-in, ANE_GEMM_PERSIST=1, read at each
// launch): the CU count, a multiple of the 8 XCDs the tile order assumes;
// 0 = one block per tile.  Measured on the B32 forward (W1|W3: 512 tiles,
// classifier: 4000) no faster than one block per tile (2.642 against 2.641
// ms per step), so not the default.
inline int persist_blocks() {
  static const int cus = [] {
    int dev = 0, cu = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev) !=
                                                  hipSuccess)
      return 0;
    return cu / 8 * 8;
  }();
  const char* f = getenv("ANE_GEMM_PERSIST");
  return f && atoi(f) != 0 ? cus : 0;
}

template <bool AT, bool BT, int EPI>
hipError_t launch(const GemmArgs& g, const EpiParams& e, hipStream_t s, int bm, int bn, int nw, int ns) {
  const int key = bm * 1000 + bn;
  // M-major operands of the weight gradients (dW = dY^T X with dY, X
  // token-major): the hand-ordered kernel with transposed LDS reads
  if constexpr ((AT || BT) && (EPI == EPI_STORE_F || EPI == EPI_STORE_W13)) {
    if (ns == 2 && !g.grp) {
      const dim3 grid((g.M / bm) * (g.N / bn) * g.splits);
      if (nw == 8) {
        LAUNCH_HOT(256, 256, 8);
        return hipGetLastError();
      }
      switch (key) {
        case 256256: LAUNCH_HOT(256, 256, 4); break;
        case 256128: LAUNCH_HOT(256, 128, 4); break;
        case 128256: LAUNCH_HOT(128, 256, 4); break;
        case 128128: LAUNCH_HOT(128, 128, 4); break;
        case 64128: LAUNCH_HOT(64, 128, 4); break;
        case 128064: LAUNCH_HOT(128, 64, 4); break;
        case 256064: LAUNCH_HOT(256, 64, 4); break;
        case 64064: LAUNCH_HOT(64, 64, 4); break;
        default: return hipErrorInvalidValue;
      }
      return hipGetLastError();
    }
  }
  // the deferred-norm epilogues exist for the hand-ordered K-major kernel only
  constexpr bool HO_ONLY = epi_rr(EPI) || EPI == EPI_RESID_NORM;
  if constexpr (!AT && !BT && EPI != EPI_RESID_NORM) {
    if (nw == 8 && ns == 2) {  // caller checked the tile
      const int ntiles = (g.M / 256) * (g.N / 256);
      if constexpr (EPI == EPI_CE || EPI == EPI_CE_RR || EPI == EPI_SWIGLU || EPI == EPI_SWIGLU_RR ||
                    EPI == EPI_STORE_H || EPI == EPI_STORE_H_RR) {
        // more tiles than CUs: one block per CU (the tile's LDS allows no
        // more), each walking its tiles (ANE_GEMM_PERSIST=1)
        const int ncu = persist_blocks();
        if (g.splits == 1 && !g.grp && ncu > 0 && ntiles > ncu) {
          hipLaunchKernelGGL((gemm_ho_kernel<256, 256, EPI, 8, false, false, true>), dim3(ncu), dim3(512), 0, s, g,
                             e);
          return hipGetLastError();
        }
      }
      const dim3 grid(ntiles * g.splits);
      LAUNCH_HO(256, 256, 8);
      return hipGetLastError();
    }
  }
  if constexpr (HO_ONLY) {
    if (nw == 8 || ns != 2) return hipErrorInvalidValue;
  } else {
    if (nw == 8) return launch_tile<AT, BT, EPI, 256, 256, 8>(g, e, s);  // caller checked the tile
  }
  if constexpr (!AT && !BT) {
    if (ns == 2) {  // hand-ordered kernel for every K-major tile
      const dim3 grid((g.M / bm) * (g.N / bn) * g.splits);
      switch (key) {
        case 256256: LAUNCH_HO(256, 256, 4); break;
        case 256128: LAUNCH_HO(256, 128, 4); break;
        case 128256: LAUNCH_HO(128, 256, 4); break;
        case 128128: LAUNCH_HO(128, 128, 4); break;
        case 64128: LAUNCH_HO(64, 128, 4); break;
        default:
          if constexpr (EPI != EPI_SWIGLU && EPI != EPI_SWIGLU_RR) {
            switch (key) {
              case 128064: LAUNCH_HO(128, 64, 4); break;
              case 256064: LAUNCH_HO(256, 64, 4); break;
              case 64064: LAUNCH_HO(64, 64, 4); break;
              // 192-wide tiles (three 32-column MFMA tiles per wave): N = 768
              // and 2304 split into whole waves of blocks
              case 128192:
                if constexpr (EPI == EPI_STORE_H || EPI == EPI_STORE_F || EPI == EPI_RESID || EPI == EPI_STORE_H_RR ||
                              EPI == EPI_RESID_NORM) {
                  LAUNCH_HO(128, 192, 4);
                  break;
                } else {
                  return hipErrorInvalidValue;
                }
              case 256192:
                if constexpr (EPI == EPI_STORE_H || EPI == EPI_STORE_F || EPI == EPI_RESID || EPI == EPI_STORE_H_RR ||
                              EPI == EPI_RESID_NORM) {
                  LAUNCH_HO(256, 192, 4);
                  break;
                } else {
                  return hipErrorInvalidValue;
                }
              default: return hipErrorInvalidValue;
            }
          } else {
            return hipErrorInvalidValue;
          }
      }
      return hipGetLastError();
    }
    if constexpr (!HO_ONLY) {
    if (ns == 3) {  // caller checked the tile
      switch (key) {
        case 256128: return launch_tile<AT, BT, EPI, 256, 128, 4, 3>(g, e, s);
        case 128128: return launch_tile<AT, BT, EPI, 128, 128, 4, 3>(g, e, s);
        case 64128: return launch_tile<AT, BT, EPI, 64, 128, 4, 3>(g, e, s);
        default: break;
      }
      if constexpr (EPI != EPI_SWIGLU) {
        switch (key) {
          case 128064: return launch_tile<AT, BT, EPI, 128, 64, 4, 3>(g, e, s);
          case 64064: return launch_tile<AT, BT, EPI, 64, 64, 4, 3>(g, e, s);
          default: break;
        }
      }
      return hipErrorInvalidValue;
    }
    }
  }
  if constexpr (HO_ONLY) {
    return hipErrorInvalidValue;
  } else {
  switch (key) {
    case 256256: return launch_tile<AT, BT, EPI, 256, 256>(g, e, s);
    case 256128: return launch_tile<AT, BT, EPI, 256, 128>(g, e, s);
    case 128256: return launch_tile<AT, BT, EPI, 128, 256>(g, e, s);
    case 128128: return launch_tile<AT, BT, EPI, 128, 128>(g, e, s);
    case 64128: return launch_tile<AT, BT, EPI, 64, 128>(g, e, s);
    default: break;
  }
  if constexpr (EPI != EPI_SWIGLU) {
    switch (key) {
      case 128064: return launch_tile<AT, BT, EPI, 128, 64>(g, e, s);
      case 256064: return launch_tile<AT, BT, EPI, 256, 64>(g, e, s);
      case 64064: return launch_tile<AT, BT, EPI, 64, 64>(g, e, s);
      default: break;
    }
  }
  return hipErrorInvalidValue;
  }
}

}  // namespace gemm_detail
}  // namespace ane
