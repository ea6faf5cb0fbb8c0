// The reference's per-object accelerator seam: layerForward, layerBackward
// and offload (ane/engine_other.go:15-89 stubs them; the darwin files
// ane/layer_darwin.go, ane/backward_darwin.go, ane/offload_darwin.go and
// ane/layer_dynamic_darwin.go implement them on the Neural Engine).
//
// Each call takes the reference's channel-first fp32 slices [C, seq] from
// the host, turns them into the token-major fp16 operands this library's
// kernels read (one LDS-tiled transpose per slice), runs the same GEMM,
// attention and norm kernels as the whole-model entry points, and turns
// the results back.  The objects compute the accelerator programs'
// functions (ane/mil_stories.go), which differ from the CPU path: no
// QK-norm, residual lambdas or value embeddings, plain residuals.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <string>
#include <vector>

#include "../../include/ane_objects.h"
#include "attention.h"
#include "gemm.h"
#include "rowops.h"

using namespace ane;

namespace {

thread_local std::string g_seam_err;

int seam_fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_seam_err = buf;
  return code;
}

#define SEAMCHK(op, x)                                                                           \
  do {                                                                                           \
    hipError_t e_ = (x);                                                                         \
    if (e_ != hipSuccess) return seam_fail(ANE_ERR_HIP, "%s: %s", op, hipGetErrorString(e_)); \
  } while (0)

// ---- kernels ---------------------------------------------------------------

// out[c * ldo + r] = f(in[r * ldi + c]) over an R x C block of 64 x 64 tiles
// (R, C multiples of 64); f = identity, or relu(v)^2 (RELU2) as
// reluSquared32 (ane/common.go:146).  LDS rows padded to 65 floats keep
// both the row writes and the column reads free of bank conflicts.
template <typename TI, typename TO, bool RELU2>
__global__ __launch_bounds__(256) void xpose_kernel(TO* __restrict__ out, const TI* __restrict__ in, int ldi,
                                                    int ldo) {
  __shared__ float tile[64][65];
  const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
  const int lx = threadIdx.x & 63, ly = threadIdx.x >> 6;
#pragma unroll 4
  for (int i = ly; i < 64; i += 4) tile[i][lx] = (float)in[(size_t)(r0 + i) * ldi + c0 + lx];
  __syncthreads();
#pragma unroll 4
  for (int i = ly; i < 64; i += 4) {
    float v = tile[lx][i];
    if (RELU2) v = v <= 0.f ? 0.f : v * v;
    out[(size_t)(c0 + i) * ldo + r0 + lx] = (TO)v;
  }
}

template <typename TI, typename TO, bool RELU2 = false>
hipError_t xpose(TO* out, const TI* in, int R, int C, int ldi, int ldo, hipStream_t s) {
  if (R <= 0 || C <= 0 || R % 64 || C % 64) return hipErrorInvalidValue;
  hipLaunchKernelGGL((xpose_kernel<TI, TO, RELU2>), dim3(C / 64, R / 64), dim3(256), 0, s, out, in, ldi, ldo);
  return hipGetLastError();
}

// Column statistics of a channel-first [C, T] slice: 64 columns per block,
// 16 lanes of rows per column (1024 threads), rows read 256 contiguous
// bytes per wave.  kRmsRowLanes partial sums per column meet in LDS.
constexpr int kRmsRowLanes = 16;

// out = x / sqrt(mean_c x^2 + 1e-5) per column t: the parameterless RMSNorm
// rmsNormNoWeightCF (ane/common.go:157-174) in the channel-first layout.
__global__ __launch_bounds__(1024) void cf_rms_fwd_kernel(float* __restrict__ out, const float* __restrict__ x,
                                                          int C, int T) {
  __shared__ float red[kRmsRowLanes][64];
  const int lx = threadIdx.x & 63, g = threadIdx.x >> 6, t = blockIdx.x * 64 + lx;
  float ss = 0.f;
  for (int c = g; c < C; c += kRmsRowLanes) {
    const float v = x[(size_t)c * T + t];
    ss += v * v;
  }
  red[g][lx] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < kRmsRowLanes; i++) tot += red[i][lx];
  const float rr = 1.0f / sqrtf(tot / (float)C + 1e-5f);
  for (int c = g; c < C; c += kRmsRowLanes) out[(size_t)c * T + t] = x[(size_t)c * T + t] * rr;
}

// dx = dy * r - x * (sum_c dy x) * r^3 / C with r = 1 / sqrt(mean_c x^2 +
// 1e-5): rmsNormNoWeightBackwardCF (ane/common.go:176-197).
__global__ __launch_bounds__(1024) void cf_rms_bwd_kernel(float* __restrict__ dx, const float* __restrict__ dy,
                                                          const float* __restrict__ x, int C, int T) {
  __shared__ float red[2][kRmsRowLanes][64];
  const int lx = threadIdx.x & 63, g = threadIdx.x >> 6, t = blockIdx.x * 64 + lx;
  float ss = 0.f, dot = 0.f;
  for (int c = g; c < C; c += kRmsRowLanes) {
    const float v = x[(size_t)c * T + t];
    ss += v * v;
    dot += dy[(size_t)c * T + t] * v;
  }
  red[0][g][lx] = ss;
  red[1][g][lx] = dot;
  __syncthreads();
  float tss = 0.f, tdot = 0.f;
#pragma unroll
  for (int i = 0; i < kRmsRowLanes; i++) {
    tss += red[0][i][lx];
    tdot += red[1][i][lx];
  }
  const float r = 1.0f / sqrtf(tss / (float)C + 1e-5f);
  const float coef = tdot * r * r * r / (float)C;
  for (int c = g; c < C; c += kRmsRowLanes) {
    const size_t i = (size_t)c * T + t;
    dx[i] = dy[i] * r - coef * x[i];
  }
}

// Softmax over the vocabulary (rows) of each position (column) of a
// vocab-major [V, T] slice, in two passes over kSmRows-row chunks: each
// chunk leaves a (max, sum exp) per column, then every chunk merges all of
// them and writes its rows.  64 columns x 4 row lanes per block.
constexpr int kSmRows = 512;
__global__ __launch_bounds__(256) void vocab_softmax_stats_kernel(float2* __restrict__ part,
                                                                  const float* __restrict__ x, int V, int T) {
  __shared__ float2 red[4][64];
  const int lx = threadIdx.x & 63, g = threadIdx.x >> 6, t = blockIdx.x * 64 + lx;
  const int r0 = blockIdx.y * kSmRows, r1 = min(V, r0 + kSmRows);
  float m = -INFINITY, s = 0.f;
  for (int r = r0 + g; r < r1; r += 4) {
    const float v = x[(size_t)r * T + t];
    if (v > m) {
      s = s * expf(m - v) + 1.f;
      m = v;
    } else {
      s += expf(v - m);
    }
  }
  red[g][lx] = make_float2(m, s);
  __syncthreads();
  if (g == 0) {
    float M = red[0][lx].x;
    for (int i = 1; i < 4; i++) M = fmaxf(M, red[i][lx].x);
    float S = 0.f;
    for (int i = 0; i < 4; i++)
      if (red[i][lx].y > 0.f) S += red[i][lx].y * expf(red[i][lx].x - M);
    part[(size_t)blockIdx.y * T + t] = make_float2(M, S);
  }
}

// (out may be x: each element is read and then written by the same thread)
__global__ __launch_bounds__(256) void vocab_softmax_apply_kernel(float* out, const float* x,
                                                                  const float2* __restrict__ part, int nch, int V,
                                                                  int T) {
  const int lx = threadIdx.x & 63, g = threadIdx.x >> 6, t = blockIdx.x * 64 + lx;
  float M = -INFINITY;
  for (int c = 0; c < nch; c++) M = fmaxf(M, part[(size_t)c * T + t].x);
  float S = 0.f;
  for (int c = 0; c < nch; c++) {
    const float2 p = part[(size_t)c * T + t];
    if (p.y > 0.f) S += p.y * expf(p.x - M);
  }
  const float inv = 1.0f / S;
  const int r0 = blockIdx.y * kSmRows, r1 = min(V, r0 + kSmRows);
  for (int r = r0 + g; r < r1; r += 4) {
    const size_t i = (size_t)r * T + t;
    out[i] = expf(x[i] - M) * inv;
  }
}

// ---- shared object state ----------------------------------------------------

// Restores the calling thread's current device when a seam call returns
// (each object switches to the device it was opened on).
struct DeviceRestore {
  int prev = -1;
  DeviceRestore() {
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
  }
  ~DeviceRestore() {
    if (prev >= 0) (void)hipSetDevice(prev);
  }
};

struct SeamBase {
  int device = -1;
  hipStream_t st = nullptr;
  std::vector<void*> allocs;
  bool closed = false;

  template <typename T>
  hipError_t alloc(T** p, size_t n) {
    void* q = nullptr;
    hipError_t h = hipMalloc(&q, std::max<size_t>(n * sizeof(T), 256));
    if (h != hipSuccess) return h;
    allocs.push_back(q);
    *p = (T*)q;
    return hipSuccess;
  }
  void release() {
    if (device >= 0) (void)hipSetDevice(device);
    if (st) (void)hipStreamSynchronize(st);
    for (void* p : allocs) (void)hipFree(p);
    allocs.clear();
    if (st) (void)hipStreamDestroy(st);
    st = nullptr;
    closed = true;
  }
  // the device and stream every call of the object uses
  hipError_t enter() {
    if (device < 0) {
      hipError_t h = hipGetDevice(&device);
      if (h != hipSuccess) return h;
      return hipStreamCreateWithFlags(&st, hipStreamNonBlocking);
    }
    return hipSetDevice(device);
  }
  hipError_t up(void* dst, const void* src, size_t bytes) {
    return hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, st);
  }
  hipError_t down(void* dst, const void* src, size_t bytes) {
    return hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, st);
  }
};

int check_layer_shape(const char* op, int D, int H, int NH, int S, int max_seq) {
  if (NH <= 0 || D != 64 * NH || H <= 0 || H % 64 || S <= 0 || S % 64 || S > max_seq)
    return seam_fail(ANE_ERR_ARG,
                     "%s: invalid shape dim=%d hidden=%d heads=%d seq=%d (dim = 64*heads, hidden a multiple of "
                     "64, seq a multiple of 64 up to %d)",
                     op, D, H, NH, S, max_seq);
  return ANE_OK;
}

int check_weights(const char* op, const ane_layer_weights* w) {
  if (!w || !w->wq || !w->wk || !w->wv || !w->wo || !w->w1 || !w->w2)
    return seam_fail(ANE_ERR_ARG, "%s: missing layer weights", op);
  return ANE_OK;
}

// fp32 host matrix -> fp16 device copy, through a device staging buffer
hipError_t stage_f16(SeamBase* b, half_t* dst, const float* src, size_t n, float* staging) {
  hipError_t h = b->up(staging, src, n * sizeof(float));
  if (h != hipSuccess) return h;
  return f32_to_f16(dst, staging, n, b->st);
}

// Wq | Wk | Wv as one [3D, D] matrix, Wo [D, D], W1 [H, D], W2 [D, H]
struct LayerShadows {
  half_t *wqkv = nullptr, *wo = nullptr, *w1 = nullptr, *w2 = nullptr;
  float* staging = nullptr;  // max(H, 3 D) * D floats
};

hipError_t alloc_shadows(SeamBase* b, LayerShadows* s, int D, int H) {
  hipError_t h;
  if ((h = b->alloc(&s->wqkv, (size_t)3 * D * D)) != hipSuccess) return h;
  if ((h = b->alloc(&s->wo, (size_t)D * D)) != hipSuccess) return h;
  if ((h = b->alloc(&s->w1, (size_t)H * D)) != hipSuccess) return h;
  if ((h = b->alloc(&s->w2, (size_t)D * H)) != hipSuccess) return h;
  return b->alloc(&s->staging, (size_t)std::max(H, 3 * D) * D);
}

hipError_t stage_layer(SeamBase* b, LayerShadows* s, const ane_layer_weights* w, int D, int H) {
  const size_t DD = (size_t)D * D;
  hipError_t h;
  if ((h = stage_f16(b, s->wqkv, w->wq, DD, s->staging)) != hipSuccess) return h;
  if ((h = stage_f16(b, s->wqkv + DD, w->wk, DD, s->staging)) != hipSuccess) return h;
  if ((h = stage_f16(b, s->wqkv + 2 * DD, w->wv, DD, s->staging)) != hipSuccess) return h;
  if ((h = stage_f16(b, s->wo, w->wo, DD, s->staging)) != hipSuccess) return h;
  if ((h = stage_f16(b, s->w1, w->w1, (size_t)H * D, s->staging)) != hipSuccess) return h;
  if ((h = stage_f16(b, s->w2, w->w2, (size_t)D * H, s->staging)) != hipSuccess) return h;
  return stream_wait(b->st);  // the caller may free its host copies
}

// RoPE tables [S, 32] of the layer programs (theta 100000,
// ane/layer_dynamic_darwin.go:858-893), or the identity (cos 1, sin 0)
hipError_t upload_rope(SeamBase* b, float** cs_d, float** sn_d, int S, bool identity) {
  std::vector<float> cs((size_t)S * 32), sn((size_t)S * 32);
  for (int pos = 0; pos < S; pos++)
    for (int i = 0; i < 32; i++) {
      const double f = (double)pos / pow(100000.0, (double)(2 * i) / 64.0);
      cs[(size_t)pos * 32 + i] = identity ? 1.f : (float)cos(f);
      sn[(size_t)pos * 32 + i] = identity ? 0.f : (float)sin(f);
    }
  hipError_t h;
  if ((h = b->alloc(cs_d, cs.size())) != hipSuccess) return h;
  if ((h = b->alloc(sn_d, sn.size())) != hipSuccess) return h;
  if ((h = b->up(*cs_d, cs.data(), cs.size() * 4)) != hipSuccess) return h;
  if ((h = b->up(*sn_d, sn.data(), sn.size() * 4)) != hipSuccess) return h;
  return stream_wait(b->st);
}

GemmArgs gemm_args(const half_t* A, int lda, bool at, const half_t* B, int ldb, bool bt, int M, int N, int K) {
  GemmArgs g;
  g.A = A; g.B = B; g.lda = lda; g.ldb = ldb; g.M = M; g.N = N; g.K = K; g.a_t = at; g.b_t = bt;
  return g;
}

}  // namespace

// ---- layerForward ------------------------------------------------------------

struct ane_layer_fwd : SeamBase {
  int D = 0, H = 0, NH = 0, S = 0;
  LayerShadows w;
  float *rope_cos = nullptr, *rope_sin = nullptr;
  float *xcf = nullptr, *x = nullptr, *x2 = nullptr, *y = nullptr, *cf = nullptr, *cf2 = nullptr, *lse = nullptr;
  half_t *xn = nullptr, *qkv = nullptr, *qkvt = nullptr, *att = nullptr, *x2n = nullptr, *gate = nullptr,
         *h1 = nullptr;
};

namespace {

// The layer on token-major device buffers: attention block, then FFN block
// (genStoriesSDPAForwardDynamicTaps and genStoriesFFNForwardDynamicTaps,
// ane/mil_stories.go:75-163,301-340).
hipError_t layer_forward_device(ane_layer_fwd* f) {
  const int D = f->D, H = f->H, S = f->S;
  hipStream_t st = f->st;
  hipError_t h;
  if ((h = xpose<float, float>(f->x, f->xcf, D, S, S, D, st)) != hipSuccess) return h;
  if ((h = rmsnorm_f16(f->xn, f->x, nullptr, nullptr, nullptr, S, D, st)) != hipSuccess) return h;
  {
    EpiParams p;
    p.C = f->qkv; p.ldc = 3 * D;
    if ((h = gemm_run(gemm_args(f->xn, D, false, f->w.wqkv, D, false, S, 3 * D, D), EPI_STORE_H, p, st)) !=
        hipSuccess)
      return h;
  }
  {
    AttnArgs a;
    memset(&a, 0, sizeof a);
    a.qkv = f->qkv; a.out = f->att; a.lse = f->lse; a.qkvt = f->qkvt;
    a.rope_cos = f->rope_cos; a.rope_sin = f->rope_sin;
    a.nseq = 1; a.S = S; a.NH = f->NH; a.qknorm = 0; a.scale = 0.125f;
    if ((h = attention_fwd(a, st)) != hipSuccess) return h;
  }
  {
    EpiParams p;  // x2 = x + Wo att
    p.C = f->x2; p.ldc = D; p.R = f->x;
    if ((h = gemm_run(gemm_args(f->att, D, false, f->w.wo, D, false, S, D, D), EPI_RESID, p, st)) != hipSuccess)
      return h;
  }
  if ((h = rmsnorm_f16(f->x2n, f->x2, nullptr, nullptr, nullptr, S, D, st)) != hipSuccess) return h;
  {
    EpiParams p;  // gate = relu(h1)^2, h1 = W1 rms(x2)
    p.C = f->gate; p.ldc = H; p.C2 = f->h1; p.ldc2 = H;
    if ((h = gemm_run(gemm_args(f->x2n, D, false, f->w.w1, D, false, S, H, D), EPI_RELU2, p, st)) != hipSuccess)
      return h;
  }
  EpiParams p;  // out = x2 + W2 gate
  p.C = f->y; p.ldc = D; p.R = f->x2;
  return gemm_run(gemm_args(f->gate, H, false, f->w.w2, H, false, S, D, H), EPI_RESID, p, st);
}

int layer_forward_call(ane_layer_fwd* f, float* out, const float* x, ane_layer_cache* cache) {
  const char* op = "run layer forward";
  if (!f) return seam_fail(ANE_ERR_ARG, "%s: layer is nil", op);
  if (f->closed) return seam_fail(ANE_ERR_CLOSED, "%s: layer is closed", op);
  if (!out || !x) return seam_fail(ANE_ERR_ARG, "%s: null buffer", op);
  const int D = f->D, H = f->H, S = f->S;
  const size_t DS = (size_t)D * S, HS = (size_t)H * S;
  hipStream_t st = f->st;
  SEAMCHK(op, f->enter());
  SEAMCHK(op, f->up(f->xcf, x, DS * 4));
  SEAMCHK(op, layer_forward_device(f));
  SEAMCHK(op, (xpose<float, float>(f->cf, f->y, S, D, D, S, st)));
  SEAMCHK(op, f->down(out, f->cf, DS * 4));
  if (cache) {
    // each tap goes through one of two channel-first staging buffers; the
    // stream orders every staging write after the copy-out of its last use
    auto tap = [&](float* dst, size_t n, float* from) -> hipError_t {
      return dst ? f->down(dst, from, n * 4) : hipSuccess;
    };
    if (cache->x_norm) {
      hipLaunchKernelGGL(cf_rms_fwd_kernel, dim3(S / 64), dim3(64 * kRmsRowLanes), 0, st, f->cf2, f->xcf, D, S);
      SEAMCHK(op, hipGetLastError());
      SEAMCHK(op, tap(cache->x_norm, DS, f->cf2));
    }
    const half_t* parts[3] = {f->qkvt, f->qkvt + D, f->qkvt + 2 * D};
    float* dsts[3] = {cache->q, cache->k, cache->v};
    for (int i = 0; i < 3; i++)
      if (dsts[i]) {
        SEAMCHK(op, (xpose<half_t, float>(f->cf, parts[i], S, D, 3 * D, S, st)));
        SEAMCHK(op, tap(dsts[i], DS, f->cf));
      }
    if (cache->att_out) {
      SEAMCHK(op, (xpose<half_t, float>(f->cf2, f->att, S, D, D, S, st)));
      SEAMCHK(op, tap(cache->att_out, DS, f->cf2));
    }
    if (cache->x2 || cache->x2_norm) {
      SEAMCHK(op, (xpose<float, float>(f->cf, f->x2, S, D, D, S, st)));
      SEAMCHK(op, tap(cache->x2, DS, f->cf));
      if (cache->x2_norm) {
        hipLaunchKernelGGL(cf_rms_fwd_kernel, dim3(S / 64), dim3(64 * kRmsRowLanes), 0, st, f->cf2, f->cf, D, S);
        SEAMCHK(op, hipGetLastError());
        SEAMCHK(op, tap(cache->x2_norm, DS, f->cf2));
      }
    }
    if (cache->h1) {
      SEAMCHK(op, (xpose<half_t, float>(f->cf, f->h1, S, H, H, S, st)));
      SEAMCHK(op, tap(cache->h1, HS, f->cf));
    }
    if (cache->gate) {  // relu(h1)^2 of the h1 the tap holds (the reference squares it on the host)
      SEAMCHK(op, (xpose<half_t, float, true>(f->cf2, f->h1, S, H, H, S, st)));
      SEAMCHK(op, tap(cache->gate, HS, f->cf2));
    }
  }
  SEAMCHK(op, stream_wait(st));
  if (cache) {
    cache->att_taps_ready = 1;
    cache->ffn_taps_ready = 1;
  }
  return ANE_OK;
}

}  // namespace

extern "C" const char* ane_seam_last_error(void) { return g_seam_err.c_str(); }

extern "C" int ane_layer_forward_open(int32_t dim, int32_t hidden, int32_t heads, int32_t seq,
                                      const ane_layer_weights* w, ane_layer_fwd** out) {
  const char* op = "compile layer forward";
  if (!out) return seam_fail(ANE_ERR_ARG, "%s: null handle", op);
  *out = nullptr;
  int rc = check_layer_shape(op, dim, hidden, heads, seq, 512);
  if (rc) return rc;
  if ((rc = check_weights(op, w))) return rc;
  ane_layer_fwd* f = new ane_layer_fwd;
  f->D = dim; f->H = hidden; f->NH = heads; f->S = seq;
  const size_t DS = (size_t)dim * seq, HS = (size_t)hidden * seq;
  hipError_t h = f->enter();
  if (h == hipSuccess) h = alloc_shadows(f, &f->w, dim, hidden);
  if (h == hipSuccess) h = upload_rope(f, &f->rope_cos, &f->rope_sin, seq, false);
  if (h == hipSuccess) h = f->alloc(&f->xcf, DS);
  if (h == hipSuccess) h = f->alloc(&f->x, DS);
  if (h == hipSuccess) h = f->alloc(&f->x2, DS);
  if (h == hipSuccess) h = f->alloc(&f->y, DS);
  if (h == hipSuccess) h = f->alloc(&f->cf, std::max(DS, HS));
  if (h == hipSuccess) h = f->alloc(&f->cf2, std::max(DS, HS));
  if (h == hipSuccess) h = f->alloc(&f->lse, (size_t)seq * heads);
  if (h == hipSuccess) h = f->alloc(&f->xn, DS);
  if (h == hipSuccess) h = f->alloc(&f->qkv, 3 * DS);
  if (h == hipSuccess) h = f->alloc(&f->qkvt, 3 * DS);
  if (h == hipSuccess) h = f->alloc(&f->att, DS);
  if (h == hipSuccess) h = f->alloc(&f->x2n, DS);
  if (h == hipSuccess) h = f->alloc(&f->gate, HS);
  if (h == hipSuccess) h = f->alloc(&f->h1, HS);
  if (h == hipSuccess) h = stage_layer(f, &f->w, w, dim, hidden);
  if (h != hipSuccess) {
    f->release();
    delete f;
    return seam_fail(h == hipErrorOutOfMemory ? ANE_ERR_NOMEM : ANE_ERR_HIP, "%s: %s", op, hipGetErrorString(h));
  }
  *out = f;
  return ANE_OK;
}

extern "C" int ane_layer_forward_run(ane_layer_fwd* lf, float* out, const float* x) {
  DeviceRestore restore;
  return layer_forward_call(lf, out, x, nullptr);
}

extern "C" int ane_layer_forward_run_taps(ane_layer_fwd* lf, float* out, const float* x, ane_layer_cache* cache) {
  DeviceRestore restore;
  return layer_forward_call(lf, out, x, cache);
}

extern "C" int ane_layer_forward_refresh(ane_layer_fwd* lf, const ane_layer_weights* w) {
  DeviceRestore restore;
  const char* op = "refresh layer forward";
  if (!lf) return seam_fail(ANE_ERR_ARG, "%s: layer is nil", op);
  if (lf->closed) return seam_fail(ANE_ERR_CLOSED, "%s: layer is closed", op);
  int rc = check_weights(op, w);
  if (rc) return rc;
  SEAMCHK(op, lf->enter());
  SEAMCHK(op, stage_layer(lf, &lf->w, w, lf->D, lf->H));
  return ANE_OK;
}

extern "C" void ane_layer_forward_close(ane_layer_fwd* lf) {
  DeviceRestore restore;
  if (lf && !lf->closed) lf->release();
}

extern "C" void ane_layer_forward_destroy(ane_layer_fwd* lf) {
  if (!lf) return;
  ane_layer_forward_close(lf);
  delete lf;
}

// ---- layerBackward -------------------------------------------------------------

struct ane_layer_bwd : SeamBase {
  int D = 0, H = 0, NH = 0, S = 0;
  LayerShadows w;
  float *rope_one = nullptr, *rope_zero = nullptr;  // identity rotation: q, k arrive as used
  float *cf = nullptr, *dxn = nullptr, *lse = nullptr, *delta = nullptr;
  half_t *qkvt = nullptr, *dx2 = nullptr, *da = nullptr, *o = nullptr, *dqkv = nullptr, *dffn = nullptr,
         *h1 = nullptr, *dh1 = nullptr;
};

namespace {

int backward_enter(const char* op, ane_layer_bwd* b) {
  if (!b) return seam_fail(ANE_ERR_ARG, "%s: layer is nil", op);
  if (b->closed) return seam_fail(ANE_ERR_CLOSED, "%s: layer is closed", op);
  SEAMCHK(op, b->enter());
  return ANE_OK;
}

// channel-first fp32 host slice [C, S] -> token-major fp16 device [S, ld] at column 0 of dst
hipError_t upload_cf(ane_layer_bwd* b, half_t* dst, int ld, const float* src, int C) {
  hipError_t h = b->up(b->cf, src, (size_t)C * b->S * 4);
  if (h != hipSuccess) return h;
  return xpose<float, half_t>(dst, b->cf, C, b->S, b->S, ld, b->st);
}

}  // namespace

extern "C" int ane_layer_backward_open(int32_t dim, int32_t hidden, int32_t heads, int32_t seq,
                                       const ane_layer_weights* w, ane_layer_bwd** out) {
  const char* op = "compile layer backward";
  if (!out) return seam_fail(ANE_ERR_ARG, "%s: null handle", op);
  *out = nullptr;
  int rc = check_layer_shape(op, dim, hidden, heads, seq, 256);
  if (rc) return rc;
  if ((rc = check_weights(op, w))) return rc;
  ane_layer_bwd* b = new ane_layer_bwd;
  b->D = dim; b->H = hidden; b->NH = heads; b->S = seq;
  const size_t DS = (size_t)dim * seq, HS = (size_t)hidden * seq;
  hipError_t h = b->enter();
  if (h == hipSuccess) h = alloc_shadows(b, &b->w, dim, hidden);
  if (h == hipSuccess) h = upload_rope(b, &b->rope_one, &b->rope_zero, seq, true);
  if (h == hipSuccess) h = b->alloc(&b->cf, std::max(DS, HS));
  if (h == hipSuccess) h = b->alloc(&b->dxn, DS);
  if (h == hipSuccess) h = b->alloc(&b->lse, (size_t)seq * heads);
  if (h == hipSuccess) h = b->alloc(&b->delta, (size_t)seq * heads);
  if (h == hipSuccess) h = b->alloc(&b->qkvt, 3 * DS);
  if (h == hipSuccess) h = b->alloc(&b->dx2, DS);
  if (h == hipSuccess) h = b->alloc(&b->da, DS);
  if (h == hipSuccess) h = b->alloc(&b->o, DS);
  if (h == hipSuccess) h = b->alloc(&b->dqkv, 3 * DS);
  if (h == hipSuccess) h = b->alloc(&b->dffn, DS);
  if (h == hipSuccess) h = b->alloc(&b->h1, HS);
  if (h == hipSuccess) h = b->alloc(&b->dh1, HS);
  if (h == hipSuccess) h = stage_layer(b, &b->w, w, dim, hidden);
  if (h != hipSuccess) {
    b->release();
    delete b;
    return seam_fail(h == hipErrorOutOfMemory ? ANE_ERR_NOMEM : ANE_ERR_HIP, "%s: %s", op, hipGetErrorString(h));
  }
  *out = b;
  return ANE_OK;
}

// The two stages of the attention backward program (sdpa1: da = Wo^T dx2,
// probabilities, dv = P^T da, dp = da V^T, ane/mil_stories.go:383-441;
// sdpa2: dq, dk from ds = P (dp - rowsum(P dp)) scaled as the forward's
// scores) and the dx program (ane/mil_stories.go:443-479), on the fused
// attention kernels: the forward pass recomputes O and the log-sum-exps the
// backward kernels read.
extern "C" int ane_layer_backward_run_attention(ane_layer_bwd* lb, float* dx_norm, float* dq, float* dk, float* dv,
                                                const float* q, const float* k, const float* v, const float* dx2) {
  DeviceRestore restore;
  const char* op = "run layer backward attention";
  int rc = backward_enter(op, lb);
  if (rc) return rc;
  if (!dx_norm || !dq || !dk || !dv || !q || !k || !v || !dx2) return seam_fail(ANE_ERR_ARG, "%s: null buffer", op);
  const int D = lb->D, S = lb->S;
  const size_t DS = (size_t)D * S;
  hipStream_t st = lb->st;
  SEAMCHK(op, upload_cf(lb, lb->qkvt, 3 * D, q, D));
  SEAMCHK(op, upload_cf(lb, lb->qkvt + D, 3 * D, k, D));
  SEAMCHK(op, upload_cf(lb, lb->qkvt + 2 * D, 3 * D, v, D));
  SEAMCHK(op, upload_cf(lb, lb->dx2, D, dx2, D));
  {
    EpiParams p;  // da = Wo^T dx2: [S, D] = dx2 [S, D] Wo [D, D]
    p.C = lb->da; p.ldc = D;
    SEAMCHK(op, gemm_run(gemm_args(lb->dx2, D, false, lb->w.wo, D, true, S, D, D), EPI_STORE_H, p, st));
  }
  {
    AttnArgs a;
    memset(&a, 0, sizeof a);
    a.qkv = lb->qkvt; a.out = lb->o; a.lse = lb->lse;
    a.rope_cos = lb->rope_one; a.rope_sin = lb->rope_zero;
    a.nseq = 1; a.S = S; a.NH = lb->NH; a.qknorm = 0; a.scale = 0.125f;
    SEAMCHK(op, attention_fwd(a, st));
  }
  {
    AttnBwdArgs b;
    memset(&b, 0, sizeof b);
    b.qkv = lb->qkvt; b.qkvt = lb->qkvt; b.o = lb->o; b.dout = lb->da; b.lse = lb->lse; b.delta = lb->delta;
    b.dqkv = lb->dqkv; b.rope_cos = lb->rope_one; b.rope_sin = lb->rope_zero;
    b.nseq = 1; b.S = S; b.NH = lb->NH; b.qknorm = 0; b.qk_coef2 = 1.f; b.rope_bwd = 0;
    b.scale_p = 0.125f; b.scale_ds = 0.125f;
    SEAMCHK(op, attention_bwd(b, st));
  }
  {
    EpiParams p;  // dx = Wq^T dq + Wk^T dk + Wv^T dv: [S, D] = dqkv [S, 3D] Wqkv [3D, D]
    p.C = lb->dxn; p.ldc = D;
    SEAMCHK(op,
            gemm_run(gemm_args(lb->dqkv, 3 * D, false, lb->w.wqkv, D, true, S, D, 3 * D), EPI_STORE_F, p, st));
  }
  float* outs[3] = {dq, dk, dv};
  for (int i = 0; i < 3; i++) {
    SEAMCHK(op, (xpose<half_t, float>(lb->cf, lb->dqkv + i * D, S, D, 3 * D, S, st)));
    SEAMCHK(op, lb->down(outs[i], lb->cf, DS * 4));
  }
  SEAMCHK(op, (xpose<float, float>(lb->cf, lb->dxn, S, D, D, S, st)));
  SEAMCHK(op, lb->down(dx_norm, lb->cf, DS * 4));
  SEAMCHK(op, stream_wait(st));
  return ANE_OK;
}

// The FFN backward programs: dsilu = W2^T dffn, then the tail dh1 = dsilu *
// 2 relu(h1), dx = W1^T dh1 (genStoriesFFNBackwardTailDynamic,
// ane/mil_stories.go:351-381).
extern "C" int ane_layer_backward_run_ffn(ane_layer_bwd* lb, float* dx_norm, float* dh1, const float* dffn,
                                          const float* h1) {
  DeviceRestore restore;
  const char* op = "run layer backward ffn";
  int rc = backward_enter(op, lb);
  if (rc) return rc;
  if (!dx_norm || !dh1 || !dffn || !h1) return seam_fail(ANE_ERR_ARG, "%s: null buffer", op);
  const int D = lb->D, H = lb->H, S = lb->S;
  hipStream_t st = lb->st;
  SEAMCHK(op, upload_cf(lb, lb->dffn, D, dffn, D));
  SEAMCHK(op, upload_cf(lb, lb->h1, H, h1, H));
  {
    EpiParams p;  // dh1 [S, H] = (dffn [S, D] W2 [D, H]) * 2 relu(h1)
    p.C = lb->dh1; p.ldc = H; p.C2 = lb->h1; p.ldc2 = H;
    SEAMCHK(op, gemm_run(gemm_args(lb->dffn, D, false, lb->w.w2, H, true, S, H, D), EPI_RELU2_BWD, p, st));
  }
  {
    EpiParams p;  // dx [S, D] = dh1 [S, H] W1 [H, D]
    p.C = lb->dxn; p.ldc = D;
    SEAMCHK(op, gemm_run(gemm_args(lb->dh1, H, false, lb->w.w1, D, true, S, D, H), EPI_STORE_F, p, st));
  }
  SEAMCHK(op, (xpose<half_t, float>(lb->cf, lb->dh1, S, H, H, S, st)));
  SEAMCHK(op, lb->down(dh1, lb->cf, (size_t)H * S * 4));
  SEAMCHK(op, (xpose<float, float>(lb->cf, lb->dxn, S, D, D, S, st)));
  SEAMCHK(op, lb->down(dx_norm, lb->cf, (size_t)D * S * 4));
  SEAMCHK(op, stream_wait(st));
  return ANE_OK;
}

extern "C" int ane_layer_backward_refresh(ane_layer_bwd* lb, const ane_layer_weights* w) {
  DeviceRestore restore;
  const char* op = "refresh layer backward";
  int rc = backward_enter(op, lb);
  if (rc) return rc;
  if ((rc = check_weights(op, w))) return rc;
  SEAMCHK(op, stage_layer(lb, &lb->w, w, lb->D, lb->H));
  return ANE_OK;
}

extern "C" void ane_layer_backward_close(ane_layer_bwd* lb) {
  DeviceRestore restore;
  if (lb && !lb->closed) lb->release();
}

extern "C" void ane_layer_backward_destroy(ane_layer_bwd* lb) {
  if (!lb) return;
  ane_layer_backward_close(lb);
  delete lb;
}

// ---- offload ---------------------------------------------------------------------

struct ane_offload : SeamBase {
  int V = 0, D = 0, S = 0;
  int pieces = 0;  // ANE_OFF_* present
  half_t *embed = nullptr, *xh = nullptr, *dlh = nullptr;
  float *staging = nullptr, *xcf = nullptr, *dycf = nullptr, *out = nullptr, *logits = nullptr, *ws = nullptr;
  float2* part = nullptr;
  int cls_bm = 0, cls_bn = 0, bwd_bm = 0, bwd_bn = 0, bwd_splits = 1;
};

namespace {

const char* piece_name(int piece) {
  switch (piece) {
    case ANE_OFF_RMS_FORWARD: return "rms forward";
    case ANE_OFF_CLASSIFIER_FORWARD: return "classifier forward";
    case ANE_OFF_SOFTMAX: return "softmax";
    case ANE_OFF_CLASSIFIER_BACKWARD: return "classifier backward";
    default: return "rms backward";
  }
}

int offload_enter(const char* op, ane_offload* o, int piece) {
  if (!o) return seam_fail(ANE_ERR_ARG, "%s: offload is nil", op);
  if (o->closed) return seam_fail(ANE_ERR_CLOSED, "%s: offload is closed", op);
  if (!(o->pieces & piece)) return seam_fail(ANE_ERR_STATE, "%s: %s kernel is unavailable", op, piece_name(piece));
  SEAMCHK(op, o->enter());
  return ANE_OK;
}

hipError_t stage_embed(ane_offload* o, const float* embed) {
  const size_t n = (size_t)o->V * o->D;
  hipError_t h = o->up(o->staging, embed, n * 4);
  if (h != hipSuccess) return h;
  if ((h = f32_to_f16(o->embed, o->staging, n, o->st)) != hipSuccess) return h;
  return stream_wait(o->st);
}

// logits [V, S] (device) = Embed x_norm, x_norm channel-first [D, S] from the host
hipError_t classifier_device(ane_offload* o, const float* x_norm) {
  const size_t DS = (size_t)o->D * o->S;
  hipError_t h = o->up(o->xcf, x_norm, DS * 4);
  if (h != hipSuccess) return h;
  if ((h = f32_to_f16(o->xh, o->xcf, DS, o->st)) != hipSuccess) return h;
  EpiParams p;  // C[v, t] = sum_d E[v, d] x_norm[d, t]: B read M-major from the channel-first slice
  p.C = o->logits; p.ldc = o->S;
  return gemm_run(gemm_args(o->embed, o->D, false, o->xh, o->S, true, o->V, o->S, o->D), EPI_STORE_F, p, o->st,
                  o->cls_bm, o->cls_bn);
}

hipError_t softmax_device(ane_offload* o) {
  const int nch = (o->V + kSmRows - 1) / kSmRows;
  const dim3 grid(o->S / 64, nch);
  hipLaunchKernelGGL(vocab_softmax_stats_kernel, grid, dim3(256), 0, o->st, o->part, o->logits, o->V, o->S);
  hipError_t h = hipGetLastError();
  if (h != hipSuccess) return h;
  hipLaunchKernelGGL(vocab_softmax_apply_kernel, grid, dim3(256), 0, o->st, o->logits, o->logits, o->part, nch,
                     o->V, o->S);
  return hipGetLastError();
}

}  // namespace

extern "C" int ane_offload_open(int32_t vocab, int32_t dim, int32_t seq, const float* embed,
                                int32_t cpu_classifier_head, ane_offload** out) {
  const char* op = "new offload";
  if (!out) return seam_fail(ANE_ERR_ARG, "%s: null handle", op);
  *out = nullptr;
  if (vocab <= 0 || vocab % 64 || dim <= 0 || dim % 64 || seq <= 0 || seq % 64)
    return seam_fail(ANE_ERR_ARG, "%s: invalid shape vocab=%d dim=%d seq=%d (multiples of 64)", op, vocab, dim, seq);
  const bool cls = !cpu_classifier_head;
  if (cls && !embed) return seam_fail(ANE_ERR_ARG, "%s: missing embedding", op);
  ane_offload* o = new ane_offload;
  o->V = vocab; o->D = dim; o->S = seq;
  o->pieces = ANE_OFF_RMS_FORWARD | ANE_OFF_RMS_BACKWARD;
  const size_t DS = (size_t)dim * seq, VS = (size_t)vocab * seq;
  hipError_t h = o->enter();
  if (h == hipSuccess) h = o->alloc(&o->xcf, DS);
  if (h == hipSuccess) h = o->alloc(&o->dycf, DS);
  if (h == hipSuccess) h = o->alloc(&o->out, DS);
  if (cls) {
    o->pieces |= ANE_OFF_CLASSIFIER_FORWARD | ANE_OFF_SOFTMAX | ANE_OFF_CLASSIFIER_BACKWARD;
    gemm_pick_tile(vocab, seq, dim, EPI_STORE_F, &o->cls_bm, &o->cls_bn);
    // dy = Embed^T dlogits: a [D, S] output over K = vocab, split so the
    // 64 x 64 tiles give a few hundred blocks
    o->bwd_bm = 64;
    o->bwd_bn = 64;
    const int kt = vocab / 64;
    for (int sp = 1; sp <= kMaxSplits; sp++)
      if (kt % sp == 0 && (long)(dim / 64) * (seq / 64) * sp <= 512) o->bwd_splits = sp;
    if (!o->cls_bm || !o->cls_bn) {
      delete o;
      return seam_fail(ANE_ERR_ARG, "%s: no classifier tile fits vocab=%d seq=%d", op, vocab, seq);
    }
    if (h == hipSuccess) h = o->alloc(&o->embed, (size_t)vocab * dim);
    if (h == hipSuccess) h = o->alloc(&o->staging, std::max((size_t)vocab * dim, VS));
    if (h == hipSuccess) h = o->alloc(&o->xh, DS);
    if (h == hipSuccess) h = o->alloc(&o->dlh, VS);
    if (h == hipSuccess) h = o->alloc(&o->logits, VS);
    if (h == hipSuccess) h = o->alloc(&o->part, (size_t)((vocab + kSmRows - 1) / kSmRows) * seq);
    if (h == hipSuccess && o->bwd_splits > 1) h = o->alloc(&o->ws, (size_t)o->bwd_splits * DS);
    if (h == hipSuccess) h = stage_embed(o, embed);
  }
  if (h != hipSuccess) {
    o->release();
    delete o;
    return seam_fail(h == hipErrorOutOfMemory ? ANE_ERR_NOMEM : ANE_ERR_HIP, "%s: %s", op, hipGetErrorString(h));
  }
  *out = o;
  return ANE_OK;
}

extern "C" int ane_offload_has(const ane_offload* o, int32_t piece) {
  return o && !o->closed && (o->pieces & piece) == piece && piece != 0 ? 1 : 0;
}

extern "C" void ane_offload_disable(ane_offload* o, int32_t piece) {
  if (o) o->pieces &= ~piece;
}

extern "C" int ane_offload_run_rms_forward(ane_offload* o, float* out, const float* x) {
  DeviceRestore restore;
  const char* op = "run rms forward";
  int rc = offload_enter(op, o, ANE_OFF_RMS_FORWARD);
  if (rc) return rc;
  if (!out || !x) return seam_fail(ANE_ERR_ARG, "%s: null buffer", op);
  const size_t DS = (size_t)o->D * o->S;
  SEAMCHK(op, o->up(o->xcf, x, DS * 4));
  hipLaunchKernelGGL(cf_rms_fwd_kernel, dim3(o->S / 64), dim3(64 * kRmsRowLanes), 0, o->st, o->out, o->xcf, o->D,
                     o->S);
  SEAMCHK(op, hipGetLastError());
  SEAMCHK(op, o->down(out, o->out, DS * 4));
  SEAMCHK(op, stream_wait(o->st));
  return ANE_OK;
}

extern "C" int ane_offload_run_classifier_forward(ane_offload* o, float* logits, const float* x_norm) {
  DeviceRestore restore;
  const char* op = "run classifier forward";
  int rc = offload_enter(op, o, ANE_OFF_CLASSIFIER_FORWARD);
  if (rc) return rc;
  if (!logits || !x_norm) return seam_fail(ANE_ERR_ARG, "%s: null buffer", op);
  SEAMCHK(op, classifier_device(o, x_norm));
  SEAMCHK(op, o->down(logits, o->logits, (size_t)o->V * o->S * 4));
  SEAMCHK(op, stream_wait(o->st));
  return ANE_OK;
}

extern "C" int ane_offload_run_classifier_softmax(ane_offload* o, float* probs, const float* x_norm) {
  DeviceRestore restore;
  const char* op = "run classifier softmax";
  int rc = offload_enter(op, o, ANE_OFF_CLASSIFIER_FORWARD);
  if (rc) return rc;
  if (!(o->pieces & ANE_OFF_SOFTMAX)) return seam_fail(ANE_ERR_STATE, "%s: softmax kernel is unavailable", op);
  if (!probs || !x_norm) return seam_fail(ANE_ERR_ARG, "%s: null buffer", op);
  SEAMCHK(op, classifier_device(o, x_norm));
  SEAMCHK(op, softmax_device(o));
  SEAMCHK(op, o->down(probs, o->logits, (size_t)o->V * o->S * 4));
  SEAMCHK(op, stream_wait(o->st));
  return ANE_OK;
}

extern "C" int ane_offload_run_softmax(ane_offload* o, float* probs) {
  DeviceRestore restore;
  const char* op = "run softmax";
  int rc = offload_enter(op, o, ANE_OFF_SOFTMAX);
  if (rc) return rc;
  if (!probs) return seam_fail(ANE_ERR_ARG, "%s: null buffer", op);
  const size_t VS = (size_t)o->V * o->S;
  SEAMCHK(op, o->up(o->logits, probs, VS * 4));
  SEAMCHK(op, softmax_device(o));
  SEAMCHK(op, o->down(probs, o->logits, VS * 4));
  SEAMCHK(op, stream_wait(o->st));
  return ANE_OK;
}

extern "C" int ane_offload_run_classifier_backward(ane_offload* o, float* dy, const float* dlogits) {
  DeviceRestore restore;
  const char* op = "run classifier backward";
  int rc = offload_enter(op, o, ANE_OFF_CLASSIFIER_BACKWARD);
  if (rc) return rc;
  if (!dy || !dlogits) return seam_fail(ANE_ERR_ARG, "%s: null buffer", op);
  const size_t VS = (size_t)o->V * o->S;
  SEAMCHK(op, o->up(o->staging, dlogits, VS * 4));
  SEAMCHK(op, f32_to_f16(o->dlh, o->staging, VS, o->st));
  // dy[d, t] = sum_v E[v, d] dlogits[v, t]: both operands read M-major,
  // the output channel-first as the caller holds it
  GemmArgs g = gemm_args(o->embed, o->D, true, o->dlh, o->S, true, o->D, o->S, o->V);
  if (o->bwd_splits > 1) {
    g.splits = o->bwd_splits;
    g.ws = o->ws;
  }
  EpiParams p;
  p.C = o->dycf; p.ldc = o->S;
  SEAMCHK(op, gemm_run(g, EPI_STORE_F, p, o->st, o->bwd_bm, o->bwd_bn));
  SEAMCHK(op, o->down(dy, o->dycf, (size_t)o->D * o->S * 4));
  SEAMCHK(op, stream_wait(o->st));
  return ANE_OK;
}

extern "C" int ane_offload_run_rms_backward(ane_offload* o, float* dx, const float* dy, const float* x) {
  DeviceRestore restore;
  const char* op = "run rms backward";
  int rc = offload_enter(op, o, ANE_OFF_RMS_BACKWARD);
  if (rc) return rc;
  if (!dx || !dy || !x) return seam_fail(ANE_ERR_ARG, "%s: null buffer", op);
  const size_t DS = (size_t)o->D * o->S;
  SEAMCHK(op, o->up(o->xcf, x, DS * 4));
  SEAMCHK(op, o->up(o->dycf, dy, DS * 4));
  hipLaunchKernelGGL(cf_rms_bwd_kernel, dim3(o->S / 64), dim3(64 * kRmsRowLanes), 0, o->st, o->out, o->dycf,
                     o->xcf, o->D, o->S);
  SEAMCHK(op, hipGetLastError());
  SEAMCHK(op, o->down(dx, o->out, DS * 4));
  SEAMCHK(op, stream_wait(o->st));
  return ANE_OK;
}

extern "C" int ane_offload_refresh(ane_offload* o, const float* embed) {
  DeviceRestore restore;
  const char* op = "refresh offload weights";
  if (!o) return seam_fail(ANE_ERR_ARG, "%s: offload is nil", op);
  if (o->closed) return seam_fail(ANE_ERR_CLOSED, "%s: offload is closed", op);
  if (!o->embed) return ANE_OK;  // no classifier pieces: nothing staged
  if (!embed) return seam_fail(ANE_ERR_ARG, "%s: model weights are nil", op);
  SEAMCHK(op, o->enter());
  SEAMCHK(op, stage_embed(o, embed));
  return ANE_OK;
}

extern "C" void ane_offload_close(ane_offload* o) {
  DeviceRestore restore;
  if (o && !o->closed) {
    o->release();
    o->pieces = 0;
  }
}

extern "C" void ane_offload_destroy(ane_offload* o) {
  if (!o) return;
  ane_offload_close(o);
  delete o;
}
