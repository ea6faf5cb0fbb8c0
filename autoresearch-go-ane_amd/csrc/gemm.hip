// MFMA GEMM kernels (gfx950, v_mfma_f32_32x32x16_f16) with fused epilogues.
//
// Block = 256 threads = 4 waves in a 2x2 grid; block tile BM x BN, k-tile 64.
// Each wave owns a (BM/2) x (BN/2) sub-tile made of 32x32 MFMA tiles, so a
// 256x256 block keeps 256 fp32 accumulators per lane (AGPRs) and reads
// 8 fragments of 16 B from LDS per 16 MFMAs.  The k-loop double-buffers LDS:
// the next k-tile is fetched from HBM into registers while the current one
// is consumed, then written to the other LDS stage; one barrier per k-tile.
//
// MFMA 32x32 accumulator layout (CDNA3/CDNA4): lane l, register r holds
// row 8*(r/4) + 4*(l/32) + (r%4), column l%32.  Operand fragments: lane l
// supplies row l%32 of A (column l%32 of B) and 8 k-values; A and B use the
// same k-slot assignment, so the kernel's choice k = 16*s + 8*(l/32) + j
// only permutes the reduction order.
#include "gemm.h"

namespace ane {

namespace {

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
typedef __attribute__((address_space(3))) void* lds_ptr_t;
template <int R, int NW>
__device__ __forceinline__ void load_direct(half_t* tile, const half_t* base, int ld, int row0, int k0, int tid) {
  static_assert(R % (8 * NW) == 0, "each wave fills whole 8-row groups");
  const int lane = tid & 63, wave = tid >> 6;
#pragma unroll
  for (int it = 0; it < R / (8 * NW); it++) {
    const int gi = wave + NW * it;
    const int r = gi * 8 + (lane >> 3);
    const int lc = swz(r, lane & 7);
    const half_t* gp = base + (size_t)(row0 + r) * ld + k0 + lc * 8;
    __builtin_amdgcn_global_load_lds((const void*)gp, (lds_ptr_t)(tile + gi * 8 * BK), 16, 0, 0);
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

  // block -> tile: spread consecutive tiles of one XCD over a contiguous
  // range (hardware deals block i to XCD i % 8), then walk groups of 8
  // M-tiles so neighbouring blocks share A rows and B columns in L2.
  const int nbm = g.M / BM, nbn = g.N / BN, nb = nbm * nbn;
  int bid = blockIdx.x;
  if ((nb & 7) == 0) bid = (bid & 7) * (nb >> 3) + (bid >> 3);
  constexpr int GROUP = 8;
  const int group_size = GROUP * nbn;
  const int first_m = (bid / group_size) * GROUP;
  const int gm = min(nbm - first_m, GROUP);
  const int bm = first_m + (bid % group_size) % gm;
  const int bn = (bid % group_size) / gm;
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
#pragma unroll
  for (int p = 0; p < NS - 1; p++) {
    if (p < nk) {
      sa.issue(g.A, g.lda, m0, p * BK, lds + p * STAGE, tid);
      sb.issue(Bp, g.ldb, n0, p * BK, lds + p * STAGE + BM * BK, tid);
    }
  }
  sa.commit(lds, tid);
  sb.commit(lds + BM * BK, tid);
  if constexpr (NS == 3) {
    if (nk > 1)
      wait_vm<LPT>();  // tile 0 landed, tile 1 may still fly
    else
      wait_tile();
    barrier_keep_loads();
  } else {
    wait_tile();
    __syncthreads();
  }

  const int frow = lane & 31, fch = lane >> 5;
  int arow[TM], brow[TN];
#pragma unroll
  for (int i = 0; i < TM; i++) arow[i] = wm * WTM + i * 32 + frow;
#pragma unroll
  for (int j = 0; j < TN; j++) brow[j] = wn * WTN + j * 32 + frow;

  for (int kt = 0; kt < nk; kt++) {
    const half_t* cur = lds + (kt % NS) * STAGE;
    half_t* nxt = lds + ((kt + 1) % NS) * STAGE;             // register-path target (NS == 2)
    half_t* far = lds + ((kt + NS - 1) % NS) * STAGE;        // direct-load target
    if (kt + NS - 1 < nk) {
      sa.issue(g.A, g.lda, m0, (kt + NS - 1) * BK, far, tid);
      sb.issue(Bp, g.ldb, n0, (kt + NS - 1) * BK, far + BM * BK, tid);
    }
    // fragments double-buffered across the four 16-wide k-substeps
    half8 a[2][TM], b[2][TN];
#pragma unroll
    for (int i = 0; i < TM; i++) a[0][i] = ld_h8(cur + arow[i] * BK + swz(arow[i], fch) * 8);
#pragma unroll
    for (int j = 0; j < TN; j++) b[0][j] = ld_h8(cur + BM * BK + brow[j] * BK + swz(brow[j], fch) * 8);
#pragma unroll
    for (int s = 0; s < BK / 16; s++) {
      const int c = s & 1;
      if (s + 1 < BK / 16) {
        const int ch = (s + 1) * 2 + fch;
#pragma unroll
        for (int i = 0; i < TM; i++) a[c ^ 1][i] = ld_h8(cur + arow[i] * BK + swz(arow[i], ch) * 8);
#pragma unroll
        for (int j = 0; j < TN; j++) b[c ^ 1][j] = ld_h8(cur + BM * BK + brow[j] * BK + swz(brow[j], ch) * 8);
      }
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[c][i], b[c][j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) {
      sa.commit(nxt, tid);
      sb.commit(nxt + BM * BK, tid);
    }
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
  }

  // ---------------------------------------------------------------- epilogue
  const int rbase = m0 + wm * WTM + 4 * (lane >> 5);
  const int cbase = n0 + wn * WTN + (lane & 31);
#define ROW(i, r) (rbase + (i) * 32 + 8 * ((r) >> 2) + ((r) & 3))
#define COL(j) (cbase + (j) * 32)

  if constexpr (EPI == EPI_STORE_H) {
    half_t* C = (half_t*)e.C;
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
      for (int j = 0; j < TN; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) C[(size_t)ROW(i, r) * e.ldc + COL(j)] = (half_t)(acc[i][j][r] * e.scale);
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
  } else if constexpr (EPI == EPI_SWIGLU) {
    static_assert(TN % 2 == 0, "SwiGLU epilogue pairs 32-column tiles");
    half_t* C = (half_t*)e.C;
    half_t* C2 = (half_t*)e.C2;
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
      for (int j = 0; j < TN; j += 2) {
        const int b = (COL(j) - (lane & 31)) >> 5;  // even 32-column block of W1
        const int hcol = (b >> 1) * 32 + (lane & 31);
#pragma unroll
        for (int r = 0; r < 16; r++) {
          float h1 = acc[i][j][r], h3 = acc[i][j + 1][r];
          float sg = 1.0f / (1.0f + __expf(-h1));
          size_t row = (size_t)ROW(i, r);
          C[row * e.ldc + hcol] = (half_t)(h1 * sg * h3);
          if (C2) {
            C2[row * e.ldc2 + COL(j)] = (half_t)h1;
            C2[row * e.ldc2 + COL(j + 1)] = (half_t)h3;
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
          const float sg = 1.0f / (1.0f + __expf(-h1v[r]));
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
          const float ga = 1.0f / (1.0f + __expf(-acc[i][j][r]));
          C[idx] = cur[r] + alpha * ga * prev[r];
          if (C2) C2[idx] = ga;
        }
      }
  } else if constexpr (EPI == EPI_CE) {
    // rows = vocab ids (M == vocab), columns = tokens.  Each wave reduces
    // its BM/2 rows of every column to (max, sum exp(v - max)); lanes l and
    // l^32 hold the two row halves of one column; the two waves sharing a
    // column range merge through LDS into one partial per block row.
    float2* red = reinterpret_cast<float2*>(lds);  // [2][BN], main loop done
#pragma unroll
    for (int j = 0; j < TN; j++) {
      const int nl = wn * WTN + j * 32 + (lane & 31);
      const int n = n0 + nl;
      const int tg = e.targets[n];
      float mx = -INFINITY, tv = 0.f;
      bool hit = false;
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
          float v = acc[i][j][r];
          if (e.softcap) v = softcap_f(v, e.cap);
          acc[i][j][r] = v;
          mx = fmaxf(mx, v);
          const bool h = ROW(i, r) == tg;
          tv = h ? v : tv;
          hit = hit || h;
        }
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) s += __expf(acc[i][j][r] - mx);
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
    // d = (softmax - onehot) * colscale[n], times (1 - tanh^2) under softcap
    half_t* C = (half_t*)e.C;
#pragma unroll
    for (int j = 0; j < TN; j++) {
      const int n = COL(j);
      const int tg = e.targets[n];
      const float lse = e.lse[n], cs = e.colscale[n];
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int m = ROW(i, r);
          float v = acc[i][j][r], dsc = 1.f;
          if (e.softcap) {
            float th = tanhf(v / e.cap);
            v = e.cap * th;
            dsc = 1.f - th * th;
          }
          float d = __expf(v - lse) - (m == tg ? 1.f : 0.f);
          d = (m < e.vocab) ? d * cs * dsc : 0.f;
          C[(size_t)m * e.ldc + n] = (half_t)d;
        }
    }
  }
#undef ROW
#undef COL
}

template <bool AT, bool BT, int EPI, int BM, int BN, int NW = 4, int NS = 2>
hipError_t launch_tile(const GemmArgs& g, const EpiParams& e, hipStream_t s) {
  dim3 grid((g.M / BM) * (g.N / BN));
  hipLaunchKernelGGL((gemm_kernel<BM, BN, AT, BT, EPI, NW, NS>), grid, dim3(64 * NW), 0, s, g, e);
  return hipGetLastError();
}

template <bool AT, bool BT, int EPI>
hipError_t launch(const GemmArgs& g, const EpiParams& e, hipStream_t s, int bm, int bn, int nw, int ns) {
  const int key = bm * 1000 + bn;
  if (nw == 8) return launch_tile<AT, BT, EPI, 256, 256, 8>(g, e, s);  // caller checked the tile
  if constexpr (!AT && !BT) {
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

}  // namespace

void gemm_pick_tile(int M, int N, int K, int epi, int* pbm, int* pbn) {
  // Preference order with a minimum block count each: a tile is taken only
  // if it yields enough blocks to keep the 256 CUs (and 2-3 resident blocks
  // per CU for the smaller tiles) busy.  Thresholds come from a sweep of
  // the stories110M shapes on MI355X (M = 8192 tokens, random operands):
  // 256x256 with 8 waves wins from 512 blocks (W1|W3: 925 vs 817 TFLOP/s
  // for 128x128; classifier 885 vs 801), 128x128 at N >= 2048, 128x64 at
  // N = 768 with K <= 2048, 64x64 for narrow outputs with long K.  A nonzero
  // *pbm / *pbn on entry is a constraint the chosen tile keeps (callers
  // size buffers by it).
  static const int cand[][3] = {{256, 256, 512}, {128, 128, 1024}, {128, 64, 600}, {64, 128, 600},
                                {256, 128, 600},  {128, 256, 600},  {256, 64, 600}, {64, 64, 0}};
  constexpr int NCAND = 8;
  const int want_bm = *pbm, want_bn = *pbn;
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

hipError_t gemm_run(const GemmArgs& g, int epi, const EpiParams& e, hipStream_t s, int bm, int bn, int nw,
                    int ns) {
  if (g.M <= 0 || g.N <= 0 || g.K <= 0 || (g.K % BK) != 0) return hipErrorInvalidValue;
  if (bm == 0 || bn == 0) gemm_pick_tile(g.M, g.N, g.K, epi, &bm, &bn);
  if (bm == 0 || bn == 0 || (g.M % bm) || (g.N % bn)) return hipErrorInvalidValue;
  // 256x256 tiles run with 8 waves unless 4 are asked for (measured faster on every shape)
  if (nw == 0) nw = (bm == 256 && bn == 256) ? 8 : 4;
  if (nw != 4 && !(nw == 8 && bm == 256 && bn == 256)) return hipErrorInvalidValue;
  if (ns == 0) ns = 2;
  // three LDS stages: both operands K-major, 4 waves, tiles whose 3 stages fit the 160 KB LDS
  if (ns != 2 && !(ns == 3 && nw == 4 && !g.a_t && !g.b_t && (bm + bn) <= 384 && !(bm == 256 && bn == 64) &&
                   !(bm == 128 && bn == 256)))
    return hipErrorInvalidValue;
  const int lay = (g.a_t ? 2 : 0) | (g.b_t ? 1 : 0);
  if (g.grp && (lay != 0 || ns != 2)) return hipErrorInvalidValue;
#define CASE(L, AT, BT, E) \
  if (lay == L && epi == E) return launch<AT, BT, E>(g, e, s, bm, bn, nw, ns);
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
