// Device helpers shared by the decode kernels (decode_kernels.hip) and the
// fused per-layer chain (decode_tail.hip): device-coherent accesses, the
// data-polling form's stale pattern, the step's q / k / v finish, and the
// wide decode-attention body, which runs in its own kernel or inside the
// chain's launch.
#pragma once
#include "decode.h"

namespace ane {
namespace {

constexpr float kL2E = 1.4426950408889634f;
constexpr int kGMax = 4;

// ---- device-coherent accesses of shared data (uniform base + per-lane byte offset)
constexpr int kSc1 = 16;  // cache policy bit sc1: device scope
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, 0x7fffffff, 0x00020000);
}
__device__ __forceinline__ float ld_c1(const float* base, uint32_t elem) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rsrc(base), elem * 4u, 0, kSc1));
}
// A stored dword never equals kTailStale (the data-polling form's "not yet
// written"): the one NaN pattern that would is replaced by another quiet NaN.
__device__ __forceinline__ uint32_t not_stale(uint32_t v, uint32_t nan) { return v == kTailStale ? nan : v; }
__device__ __forceinline__ bool fresh(float v) { return __float_as_uint(v) != kTailStale; }
__device__ __forceinline__ bool fresh8(half8 v) {
  const u32x4v u = __builtin_bit_cast(u32x4v, v);
  return (u[0] != kTailStale) & (u[1] != kTailStale) & (u[2] != kTailStale) & (u[3] != kTailStale);
}
__device__ __forceinline__ void st_c1(float* base, uint32_t elem, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(not_stale(__float_as_uint(v), 0x7FC00000u), rsrc(base), elem * 4u, 0, kSc1);
}
__device__ __forceinline__ half8 ld_ch8(const half_t* base, uint32_t elem) {
  const u32x4v a = __builtin_amdgcn_raw_buffer_load_b128(rsrc(base), elem * 2u, 0, kSc1);
  return __builtin_bit_cast(half8, a);
}
// this wave's stores have completed (s_waitcnt vmcnt(0)); the empty asm keeps
// the compiler from moving memory operations across
__device__ __forceinline__ void drain_stores() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0x0F70);
  asm volatile("" ::: "memory");
}

// Data-polling form: a wave re-issues its device-coherent input loads in
// rounds until none of them returns a stale dword.  give_up() after round r:
// true after `limit` rounds or when another block has failed (else a short
// sleep before the next round).  limit 0 fails before the first round.
__device__ __forceinline__ bool give_up(unsigned r, unsigned limit, const int* err) {
  if (r + 1 >= limit || __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) return true;
  __builtin_amdgcn_s_sleep(1);
  return false;
}

// Keys per split for ctx keys over nsplit splits: an even share rounded up
// to 32 (<= the kernel's chunk, as nsplit covers max_ctx in chunk-key
// pieces), so no split is left with a short tail while the others run full.
__device__ __forceinline__ int dec_chunk(int ctx, int nsplit) {
  return ((ctx + nsplit - 1) / nsplit + 31) & ~31;
}

// The step's projections from the QKV partials, one column pair per thread:
// q of the G heads (threads < 32 G) and, in the block whose split holds
// position pos, the new k (next 32) and v (next 32).  Summed in split order
// as the finish kernels do, RoPE on q and k.  issue() loads the partials and
// RoPE factors -- only in the waves holding projection columns, so fewer
// loads share the CU's memory pipeline with the K / V rows (the q loads
// still return late under a block's worth of K / V misses: the staging
// barrier waits for them).  finish() sums, rotates and writes q, the new
// k / v rows to LDS and the new rows to cache row `row` of the split.
template <int G, int QS>
struct QkvProj {
  float pe[QS], po[QS], cs = 0.f, sn = 0.f, rr = 1.f;
  int col = -1;
  bool rot = false;
  __device__ __forceinline__ void issue(const DecAttnArgs& a, int b, int kvh, int tid, int pos, bool own) {
    const int D = a.NH * 64, KVD = a.NKV * 64, N1 = D + 2 * KVD;
    if (tid < G * 32) col = kvh * G * 64 + 2 * tid;
    else if (own && tid < G * 32 + 32) col = D + kvh * 64 + 2 * (tid - G * 32);
    else if (own && tid < G * 32 + 64) col = D + KVD + kvh * 64 + 2 * (tid - G * 32 - 32);
    rot = col >= 0 && col < D + KVD;
    const int cc = col < 0 ? 0 : col;
    const float* pp = a.qkv_part + (size_t)b * N1 + cc;
    if (tid < G * 32 + 64) {
#pragma unroll
      for (int s = 0; s < QS; s++) {  // unconditional loads, split index clamped
        const size_t o = (size_t)min(s, a.qkv_ks - 1) * kDecRows * N1;
        pe[s] = pp[o];
        po[s] = pp[o + 1];
      }
      const int ri = (cc & 63) >> 1;
      cs = a.rope_cos[pos * 32 + ri];
      sn = a.rope_sin[pos * 32 + ri];
      if (a.rr) rr = a.rr[b];
    }
  }
  // The same loads device-coherent, for partials written inside the same
  // launch (the fused chain's QKV blocks, in the data-polling buffer set):
  // true when none of this thread's partials, nor its 1 / rms, is stale.
  __device__ __forceinline__ bool issue_c1(const DecAttnArgs& a, int b, int kvh, int tid, int pos, bool own) {
    const int D = a.NH * 64, KVD = a.NKV * 64, N1 = D + 2 * KVD;
    col = -1;
    if (tid < G * 32) col = kvh * G * 64 + 2 * tid;
    else if (own && tid < G * 32 + 32) col = D + kvh * 64 + 2 * (tid - G * 32);
    else if (own && tid < G * 32 + 64) col = D + KVD + kvh * 64 + 2 * (tid - G * 32 - 32);
    rot = col >= 0 && col < D + KVD;
    const int cc = col < 0 ? 0 : col;
    bool ok = true;
    if (tid < G * 32 + 64) {
      const uint32_t e = (uint32_t)(b * N1 + cc);
#pragma unroll
      for (int s = 0; s < QS; s++) {
        const uint32_t o = (uint32_t)min(s, a.qkv_ks - 1) * kDecRows * N1;
        pe[s] = ld_c1(a.qkv_part, e + o);
        po[s] = ld_c1(a.qkv_part, e + o + 1);
        ok &= fresh(pe[s]);
        ok &= fresh(po[s]);
      }
      const int ri = (cc & 63) >> 1;
      cs = a.rope_cos[pos * 32 + ri];
      sn = a.rope_sin[pos * 32 + ri];
      if (a.rr) {
        rr = ld_c1(a.rr, (uint32_t)b);
        ok &= fresh(rr);
      }
    }
    return ok;
  }
  __device__ __forceinline__ void finish(const DecAttnArgs& a, int tid, half_t (*qs)[64], half_t* knew, half_t* vnew,
                                         half_t* Kb, half_t* Vb, int row) const {
    if (col < 0) return;
    float e = 0.f, o = 0.f;
#pragma unroll
    for (int s = 0; s < QS; s++) {
      e += s < a.qkv_ks ? pe[s] : 0.f;
      o += s < a.qkv_ks ? po[s] : 0.f;
    }
    e *= rr;  // the partials are of fp16(x * gain): the norm's 1 / rms applied here
    o *= rr;
    if (rot) {
      const float e2 = e * cs - o * sn, o2 = o * cs + e * sn;
      e = e2;
      o = o2;
    }
    half2v w;
    w[0] = (half_t)e;
    w[1] = (half_t)o;
    if (tid < G * 32) {
      *reinterpret_cast<half2v*>(&qs[tid >> 5][2 * (tid & 31)]) = w;
    } else {
      const bool isk = tid < G * 32 + 32;
      const int d = 2 * ((tid - G * 32) & 31);
      *reinterpret_cast<half2v*>((isk ? knew : vnew) + d) = w;
      *reinterpret_cast<half2v*>((isk ? Kb : Vb) + (size_t)row * 64 + d) = w;  // cache row pos
    }
  }
};

// Wide form, one 1024-thread block per (sequence, kv head, split of up to
// kDecWideChunk keys).  Key tile t (16 keys) belongs to wave t % 16, which
// does all of that tile's work:
//   * scores S^T = K Q^T on v_mfma_f32_16x16x32_f16: A = 16 keys x 32 dims
//     straight from the cache rows (lane: key lane % 16, dims 8 (lane / 16)
//     + [0, 8)), B = the G query heads padded to 16 columns;
//   * the wave's own softmax over its keys (maximum and sum per head);
//   * O = P V on v_mfma_f32_16x16x16_f16.  The score accumulator already has
//     the A layout of P (head lane % 16, keys 4 (lane / 16) + [0, 4)), so the
//     probabilities stay in their lanes; each V tile goes through a per-wave
//     LDS tile, read back transposed (ds_read_b64_tr_b16) as the B operand.
// The waves' (maximum, sum, O) meet once in LDS at the end, rescaled to the
// block maximum.  No block-wide barrier separates the K loads from P V, so
// each wave works on its rows as they arrive.
// LDS of the wide form (one 1024-thread block): q of the G <= kGMax heads;
// per-wave V tiles [16 keys][64 dims], two used in turn (16-byte chunk c of
// row r at chunk slot c ^ (r & 7)); each wave's O (scaled to its own
// maximum), maximum and sum; the new k / v rows; per-wave failure flags.
struct WideLds {
  half_t qs[kGMax][64];
  __attribute__((aligned(16))) half_t vt[16][2][16 * 64];
  float wo[16][kGMax][64];
  float wm[16][kGMax], wl[16][kGMax];
  __attribute__((aligned(16))) half_t knew[64], vnew[64];
  int fail[16];
};
// Block (b, kvh, sp).  POLL: the QKV partials and the 1 / rms were written
// inside the same launch (the fused chain) and are re-read device-coherent
// until none is stale (at most spin_limit rounds; a timeout sets *err and
// the block exits).
// pf_k / pf_v (POLL only, may be null): after its own K / V loads, the
// block streams pf_rows cache rows of another (sequence, kv head) through
// the caches -- one that will start late, on the same XCD, and then finds
// them in L2 -- while it waits for q.
template <int G, bool DIRECT, bool POLL>
__device__ __forceinline__ void dec_attn_wide_body(const DecAttnArgs& a, int b, int kvh, int sp, WideLds& L,
                                                   unsigned spin_limit = 0, int* err = nullptr,
                                                   const half_t* pf_k = nullptr, const half_t* pf_v = nullptr,
                                                   int pf_rows = 0) {
  constexpr int NT = 1024, NW = NT / 64;
  constexpr int TW = (kDecWideChunk / 16 + NW - 1) / NW;  // key tiles per wave
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ctx = a.ctr[0] + 1;
  const int chunk = dec_chunk(ctx, a.nsplit);
  const int c0 = sp * chunk;
  if (c0 >= ctx) return;  // uniform over the block, before any barrier
  const int n = min(chunk, ctx - c0);
  auto& qs = L.qs;
  auto& vt = L.vt;
  auto& wo = L.wo;
  auto& wm = L.wm;
  auto& wl = L.wl;
  half_t* knew = L.knew;
  half_t* vnew = L.vnew;
  const float sl2 = a.scale * kL2E;
  const size_t cache0 = ((size_t)b * a.NKV + kvh) * a.max_ctx;
  half_t* Kb = a.kc + (cache0 + c0) * 64;
  half_t* Vb = a.vc + (cache0 + c0) * 64;
  const int pos = ctx - 1;
  const bool own = pos - c0 < n;
  const int kr = lane & 15, kq = lane >> 4;  // K fragment: key kr, dims 8 kq (+ 32)
  const int vr = lane >> 2, vc = lane & 3;   // V tile row: key vr, dims 16 vc + [0, 16)
  // K / V loads: unconditional (key index clamped; keys past n unused).
  half8 ka[TW][2], va[TW][2];
  auto load_kv = [&]() {
#pragma unroll
    for (int u = 0; u < TW; u++) {
      const half_t* row = Kb + (size_t)min((wave + NW * u) * 16 + kr, n - 1) * 64 + kq * 8;
      ka[u][0] = ld_h8(row);
      ka[u][1] = ld_h8(row + 32);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < TW; u++) {
      const half_t* row = Vb + (size_t)min((wave + NW * u) * 16 + vr, n - 1) * 64 + vc * 16;
      va[u][0] = ld_h8(row);
      va[u][1] = ld_h8(row + 8);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  QkvProj<G, 8> qp;
  if constexpr (POLL) {
    // inside the chain's launch: q is not there yet, the cache is -- every
    // K / V load first, then q polled (its loads wait behind them anyway)
    load_kv();
    if (pf_k) {  // 16 B per thread per load, 4 in flight; the values are only xor-folded
      const uint4* pk = reinterpret_cast<const uint4*>(pf_k);
      const uint4* pv = reinterpret_cast<const uint4*>(pf_v);
      const int n16 = pf_rows * 8;  // 16-byte chunks per tensor
      unsigned x = 0;
      for (int c = tid; c < n16; c += 2 * NT) {
        const int c1 = min(c + NT, n16 - 1);
        const uint4 v0 = pk[c], v1 = pk[c1], v2 = pv[c], v3 = pv[c1];
        x ^= v0.x ^ v0.y ^ v0.z ^ v0.w ^ v1.x ^ v1.y ^ v1.z ^ v1.w;
        x ^= v2.x ^ v2.y ^ v2.z ^ v2.w ^ v3.x ^ v3.y ^ v3.z ^ v3.w;
      }
      asm volatile("" ::"v"(x));
    }
    bool ok = false;
    for (unsigned r = 0; spin_limit != 0; r++) {
      asm volatile("" ::: "memory");
      if (__all(qp.issue_c1(a, b, kvh, tid, pos, own))) { ok = true; break; }
      if (give_up(r, spin_limit, err)) break;
    }
    if (lane == 0) {
      L.fail[wave] = ok ? 0 : 1;
      if (!ok) __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    int f = 0;
#pragma unroll
    for (int w = 0; w < NW; w++) f |= L.fail[w];
    if (f) return;  // uniform; a block whose q never arrived writes nothing (no cache row)
    qp.finish(a, tid, qs, knew, vnew, Kb, Vb, pos - c0);
    __syncthreads();
  } else {
    // q and the new k / v rows first, staged before any K / V load is
    // issued: a load issued beside the block's K / V misses returns only
    // after most of them (measured: the staging barrier then completes ~10 us
    // into a 17 us kernel, and the whole softmax and P V run after the last
    // row arrives)
    qp.issue(a, b, kvh, tid, pos, own);
    qp.finish(a, tid, qs, knew, vnew, Kb, Vb, pos - c0);
    __syncthreads();
    load_kv();
  }
  // Row pos is the last row of the split and every key index past n read it
  // too (clamped): those take the new k / v (the row read may be stale, or
  // the new one -- another thread stored it just before -- and a NaN in a
  // stale row must not reach the sums), by a select at each use.
  const int jrep = own ? pos - c0 : 1 << 30;
  half8 kn0 = {}, kn1 = {}, vn0 = {}, vn1 = {};
  if (own) {
    kn0 = ld_h8(knew + kq * 8);
    kn1 = ld_h8(knew + 32 + kq * 8);
    vn0 = ld_h8(vnew + vc * 16);
    vn1 = ld_h8(vnew + vc * 16 + 8);
  }
  half8 qb0, qb1;  // B operand: head kr (zero columns past G), dims as A
  {
    const int h = kr < G ? kr : 0;
    const half8 z = {};
    qb0 = kr < G ? ld_h8(&qs[h][kq * 8]) : z;
    qb1 = kr < G ? ld_h8(&qs[h][32 + kq * 8]) : z;
  }
  floatx4 st[TW];
  float m = -INFINITY;
#pragma unroll
  for (int u = 0; u < TW; u++) {
    const int kb = (wave + NW * u) * 16;
    const bool rep = kb + kr >= jrep;
    floatx4 c = {0.f, 0.f, 0.f, 0.f};
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(rep ? kn0 : ka[u][0], qb0, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(rep ? kn1 : ka[u][1], qb1, c, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int j = kb + 4 * kq + i;
      st[u][i] = j < n && kr < G ? c[i] * sl2 : -INFINITY;
      m = fmaxf(m, st[u][i]);
    }
  }
  // the wave's maximum per head (the lanes of head lane % 16); a wave with
  // no valid key, and the padding columns, have p = exp2(-inf) = 0
  m = fmaxf(m, __shfl_xor(m, 16, 64));
  m = fmaxf(m, xor32_f(m));
  const float mz = m == -INFINITY ? 0.f : m;
  // probabilities rounded to fp16 (the P V operand); the sum adds the same
  // rounded values
  half4 pa[TW];
  float l = 0.f;
#pragma unroll
  for (int u = 0; u < TW; u++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      pa[u][i] = (half_t)__builtin_amdgcn_exp2f(st[u][i] - mz);
      l += (float)pa[u][i];
    }
  l += __shfl_xor(l, 16, 64);
  l += xor32_f(l);
  // O[head][dim] += P[head][key] V[key][dim], 16 dims per MFMA: lane
  // 16 g + j takes V[4 g + e][16 db + j] (e = 0..3), which the transposed
  // read gives when lane l addresses row l / 4, halves 16 db + 4 (l % 4)
  floatx4 o[4];
#pragma unroll
  for (int db = 0; db < 4; db++) o[db] = floatx4{0.f, 0.f, 0.f, 0.f};
  const int rr = lane >> 2, rq = lane & 3;
#pragma unroll
  for (int u = 0; u < TW; u++) {
    half_t* t = vt[wave][u & 1];
    const bool rep = (wave + NW * u) * 16 + vr >= jrep;
    st_h8(t + vr * 64 + (((2 * vc) ^ (vr & 7)) << 3), rep ? vn0 : va[u][0]);
    st_h8(t + vr * 64 + (((2 * vc + 1) ^ (vr & 7)) << 3), rep ? vn1 : va[u][1]);
    // the wave's stores precede its reads (LDS runs one wave's operations
    // in order); the fence keeps the compiler from reordering them
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
#pragma unroll
    for (int db = 0; db < 4; db++) {
      const int cch = 2 * db + (rq >> 1);
      const short4v bv = ds_read_tr16(t + rr * 64 + ((cch ^ (rr & 7)) << 3) + 4 * (rq & 1));
      o[db] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa[u], __builtin_bit_cast(half4, bv), o[db], 0, 0, 0);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  }
  // the merge: O rows (heads) 4 (lane / 16) + i, column 16 db + lane % 16;
  // heads < G sit in lanes 0..15
  if (lane < 16) {
#pragma unroll
    for (int db = 0; db < 4; db++)
#pragma unroll
      for (int i = 0; i < G; i++) wo[wave][i][16 * db + lane] = o[db][i];
  }
  if (lane < G) {
    wm[wave][lane] = m;
    wl[wave][lane] = l;
  }
  __syncthreads();
  if (tid < G * 64) {
    const int h = tid >> 6, d = tid & 63;
    float mt = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; w++) mt = fmaxf(mt, wm[w][h]);  // finite: key 0 is valid
    float ot = 0.f, lt = 0.f;
#pragma unroll
    for (int w = 0; w < NW; w++) {
      const float f = __builtin_amdgcn_exp2f(wm[w][h] - mt);  // 0 for a wave without keys
      ot += f * wo[w][h][d];
      lt += f * wl[w][h];
    }
    if constexpr (DIRECT) {
      a.att[act_frag_off(b, (kvh * G + h) * 64 + d)] = (half_t)(ot / lt);
    } else {
      float* out = a.part + (((size_t)b * a.NH + kvh * G + h) * a.nsplit + sp) * 66;
      out[d] = ot;
      if (d == 0) { out[64] = mt; out[65] = lt; }
    }
  }
}

}  // namespace
}  // namespace ane
