// Shared device helpers for the gfx950 kernels of libane_hip.
//
// Conventions used by every kernel in this library:
//  * activations are token-major [T, C] (T = sequences * seq), so the
//    channel dimension is contiguous and feeds MFMA operands directly;
//  * GEMM operands are fp16 with fp32 accumulation; the residual stream,
//    norm statistics and softmax statistics stay fp32;
//  * waves are 64 lanes (CDNA4).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>

namespace ane {

typedef _Float16 half_t;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
// The value lane l ^ 32 holds, by v_permlane32_swap (a VALU exchange of
// the two 32-lane halves) instead of an LDS permute: with both operands x,
// the swap leaves the upper half's values in element 1 for lanes 0..31 and
// the lower half's in element 0 for lanes 32..63.
__device__ __forceinline__ float xor32_f(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(__lane_id() < 32 ? r[1] : r[0]);
}

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// 16-byte chunk swizzle for LDS tiles stored as rows of 64 halves (8 chunks
// of 16 B).  Rows r..r+7 read at one logical chunk land on 8 distinct
// chunk slots, and so do rows r, r+8, ..., r+56 (the transposed-staging
// write pattern), so both patterns are free of bank conflicts.
__device__ __forceinline__ int swz(int row, int chunk) {
  return chunk ^ ((row ^ (row >> 3)) & 7);
}

// Streaming 16-byte accesses (nontemporal: the data is not expected back in
// the caches soon).  Measured on the flush's update pass: 700 -> 625 us.
typedef float f32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 ld_nt_f4(const float* p) {
  const f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
  return make_float4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ void st_nt_f4(float* p, const float4& x) {
  const f32x4 v = {x.x, x.y, x.z, x.w};
  __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(p));
}

__device__ __forceinline__ half8 ld_h8(const half_t* p) {
  return *reinterpret_cast<const half8*>(p);
}
__device__ __forceinline__ void st_h8(half_t* p, half8 v) {
  *reinterpret_cast<half8*>(p) = v;
}

// LDS reads that transpose (gfx950 ds_read_b64_tr_b16): lane 16 g + j
// receives element j % 4 of the 4 halves that lane 16 g + 4 e + j / 4
// addresses, as its element e.  Such reads give an MFMA operand from a tile
// stored with the operand's row index contiguous ([k][row]).
typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef short short4v __attribute__((ext_vector_type(4)));
__device__ __forceinline__ short4v ds_read_tr16(const half_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4v*)(lds_ptr_t)p);
}

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + __expf(-x)); }

// Streams slice `part` of `nparts` equal slices of [p, p + bytes) through
// the cache hierarchy with ordinary loads and discards the data (an empty
// asm consumes it, so the loads stay).  Memory-bound kernels call it on the
// weights of the GEMM that runs next: by then those weights have been
// evicted from the memory-side cache by the rest of the step's traffic, and
// every block of the GEMM would otherwise wait on HBM latency for the same
// weight tiles at once.  p must be 16-byte aligned; NULL is a no-op.
__device__ __forceinline__ void prefetch_slice(const void* p, size_t bytes, size_t part, size_t nparts) {
  if (!p || bytes < 16) return;
  const uint4* q = reinterpret_cast<const uint4*>(p);
  const size_t n = bytes / 16;
  uint32_t x = 0;
  for (size_t i = part * blockDim.x + threadIdx.x; i < n; i += nparts * blockDim.x) {
    const uint4 v = q[i];
    x ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  asm volatile("" ::"v"(x));
}

// prefetch_slice in two halves for kernels with loads of their own: the
// first kPrefetchEarly 16-byte loads of the slice are issued by
// prefetch_begin (after the kernel has issued its own loads, so waiting
// for those does not wait for these) and consumed by prefetch_end, after
// the kernel's work; any rest of the slice is streamed by prefetch_end.
constexpr int kPrefetchEarly = 4;
struct Prefetch {
  uint4 v[kPrefetchEarly];
};
__device__ __forceinline__ Prefetch prefetch_begin(const void* p, size_t bytes, size_t part, size_t nparts) {
  Prefetch f;
  const size_t n = bytes / 16;
  if (!p || n == 0) {
#pragma unroll
    for (int u = 0; u < kPrefetchEarly; u++) f.v[u] = make_uint4(0, 0, 0, 0);
    return f;
  }
  const uint4* q = reinterpret_cast<const uint4*>(p);
  const size_t i0 = part * blockDim.x + threadIdx.x, stride = nparts * blockDim.x;
#pragma unroll
  for (int u = 0; u < kPrefetchEarly; u++) {  // unconditional: the index is clamped
    const size_t i = i0 + u * stride;
    f.v[u] = q[i < n ? i : n - 1];
  }
  return f;
}
__device__ __forceinline__ void prefetch_end(const Prefetch& f, const void* p, size_t bytes, size_t part,
                                             size_t nparts) {
  uint32_t x = 0;
#pragma unroll
  for (int u = 0; u < kPrefetchEarly; u++) x ^= f.v[u].x ^ f.v[u].y ^ f.v[u].z ^ f.v[u].w;
  const size_t n = bytes / 16;
  if (p && n > 0) {
    const uint4* q = reinterpret_cast<const uint4*>(p);
    const size_t stride = nparts * blockDim.x;
    for (size_t i = part * blockDim.x + threadIdx.x + kPrefetchEarly * stride; i < n; i += stride) {
      const uint4 v = q[i];
      x ^= v.x ^ v.y ^ v.z ^ v.w;
    }
  }
  asm volatile("" ::"v"(x));
}

// Sum over the 64 lanes: DPP within each 16-lane row (quad_perm [1,0,3,2],
// [2,3,0,1], row_half_mirror, row_mirror), then the rows by one lane
// permute and one half swap; every lane ends with the total.
template <int CTRL>
__device__ __forceinline__ float dpp_row_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += dpp_row_f<0xB1>(v);
  v += dpp_row_f<0x4E>(v);
  v += dpp_row_f<0x141>(v);
  v += dpp_row_f<0x140>(v);
  v += __shfl_xor(v, 16, 64);
  v += xor32_f(v);
  return v;
}

// Host: wait for everything queued on stream s by polling it, for calls
// that return results to their caller.  hipStreamSynchronize may block the
// thread until an interrupt wakes it, tens of microseconds after the GPU has
// finished; polling returns within a few.  ANE_SPIN_WAIT=0 blocks instead.
inline hipError_t stream_wait(hipStream_t s) {
  static const bool spin = [] {
    const char* f = getenv("ANE_SPIN_WAIT");
    return !f || atoi(f) != 0;
  }();
  if (!spin) return hipStreamSynchronize(s);
  hipError_t r;
  while ((r = hipStreamQuery(s)) == hipErrorNotReady) {
  }
  return r;
}

}  // namespace ane
