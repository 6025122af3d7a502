// Op class (a): fused pointwise + reductions over contiguous runs.
//
// A "row" here is one of the reference's columns: a run of n contiguous
// floats (a reduction over dims = 1 of a column-major n x rows array).  One
// workgroup of 256 threads (four waves) takes a row.  The resident kernels
// hold the row's elements in registers (NV 16-byte loads per thread), so a
// softmax or LayerNorm and its gradient read x and g from HBM once and write
// dx once: the 3 x 4 bytes per element that bound them.  Longer rows stream:
// the fold sweeps the row, then a second sweep re-reads it to write.
//
// Folds follow the reference's fold algebra (src/Compiler/IR/folds.jl):
// softmax is the online exponential fold Relative{Exponential} over elements
// (x, g) -- state (max, sum exp, sum g*exp), combined by rebasing both sums
// to the larger maximum (folds.jl:186-222) -- and LayerNorm is the program's
// own two-pass mean / mean-square-deviation (test/fixtures/programs.jl:13-17).
#include <hip/hip_runtime.h>

#include <cmath>

#include "th_core.h"

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

struct RowArgs {
  const float* x;
  const float* g;
  float* out;      // dx (gradient kernels) or y (forward kernels)
  float* partial;  // per-row loss contribution (gradient kernels)
  int64_t rows;
  int64_t ld;
  int32_t n;
  float eps;
};

template <int VW>
struct Vec;
typedef float f32x4 __attribute__((ext_vector_type(4)));
template <>
struct Vec<4> {
  static __device__ __forceinline__ void load(const float* p, float* v) {
    f32x4 t = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
    v[0] = t[0], v[1] = t[1], v[2] = t[2], v[3] = t[3];
  }
  static __device__ __forceinline__ void store(float* p, const float* v) {
    f32x4 t = {v[0], v[1], v[2], v[3]};
    __builtin_nontemporal_store(t, reinterpret_cast<f32x4*>(p));
  }
};
template <>
struct Vec<1> {
  static __device__ __forceinline__ void load(const float* p, float* v) {
    v[0] = __builtin_nontemporal_load(p);
  }
  static __device__ __forceinline__ void store(float* p, const float* v) {
    __builtin_nontemporal_store(v[0], p);
  }
};

// ---- the online exponential fold's state -----------------------------------

struct Exp3 {
  float m, s, t;
};

__device__ __forceinline__ Exp3 exp_combine(Exp3 a, Exp3 b) {
  float m = fmaxf(a.m, b.m);
  float sh = thd::lse_shift(m);
  float fa = __expf(a.m - sh), fb = __expf(b.m - sh);
  return Exp3{m, a.s * fa + b.s * fb, a.t * fa + b.t * fb};
}

__device__ __forceinline__ Exp3 wave_combine(Exp3 v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    Exp3 w{__shfl_xor(v.m, o, 64), __shfl_xor(v.s, o, 64), __shfl_xor(v.t, o, 64)};
    v = exp_combine(v, w);
  }
  return v;
}

// Every thread gets the block's combined state.  The waves' states combine
// in wave order, so the result does not depend on timing.
__device__ __forceinline__ Exp3 block_combine(Exp3 v, float* lds) {
  v = wave_combine(v);
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  __syncthreads();  // lds may still be read from a previous use
  if (lane == 0) {
    lds[wave * 3 + 0] = v.m;
    lds[wave * 3 + 1] = v.s;
    lds[wave * 3 + 2] = v.t;
  }
  __syncthreads();
  Exp3 r{lds[0], lds[1], lds[2]};
#pragma unroll
  for (int w = 1; w < kWaves; ++w) r = exp_combine(r, Exp3{lds[w * 3], lds[w * 3 + 1], lds[w * 3 + 2]});
  return r;
}

template <int K>
__device__ __forceinline__ void block_sums(float (&v)[K], float* lds) {
#pragma unroll
  for (int k = 0; k < K; ++k) v[k] = thd::wave_sum(v[k]);
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  __syncthreads();
  if (lane == 0)
#pragma unroll
    for (int k = 0; k < K; ++k) lds[wave * K + k] = v[k];
  __syncthreads();
#pragma unroll
  for (int k = 0; k < K; ++k) {
    float s = lds[k];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) s += lds[w * K + k];
    v[k] = s;
  }
}

// ---- resident kernels: NV loads of VW floats per thread ----------------------

// Softmax over the row and its gradient against g; the row's share of the loss.
template <int VW, int NV>
__global__ __launch_bounds__(kThreads) void softmax_grad_resident(RowArgs a) {
  __shared__ float lds[kWaves * 3];
  const int64_t row = blockIdx.x;
  const float* xr = a.x + row * a.ld;
  const float* gr = a.g + row * a.ld;
  float* dr = a.out + row * a.ld;
  float x[NV][VW], g[NV][VW];
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int q = (i * kThreads + threadIdx.x) * VW;
    if (q < a.n) {
      Vec<VW>::load(xr + q, x[i]);
      Vec<VW>::load(gr + q, g[i]);
    } else {
#pragma unroll
      for (int j = 0; j < VW; ++j) x[i][j] = -INFINITY, g[i][j] = 0.0f;
    }
#pragma unroll
    for (int j = 0; j < VW; ++j) m = fmaxf(m, x[i][j]);
  }
  const float sh = thd::lse_shift(m);
  float s = 0.0f, t = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i)
#pragma unroll
    for (int j = 0; j < VW; ++j) {
      float e = __expf(x[i][j] - sh);
      s += e;
      t = fmaf(g[i][j], e, t);
    }
  Exp3 st = block_combine(Exp3{m, s, t}, lds);
  const float inv = 1.0f / st.s;
  const float dot = st.t * inv;  // sum(y .* g) over the row
  const float shift = thd::lse_shift(st.m);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int q = (i * kThreads + threadIdx.x) * VW;
    if (q < a.n) {
      float d[VW];
#pragma unroll
      for (int j = 0; j < VW; ++j) {
        float y = __expf(x[i][j] - shift) * inv;
        d[j] = y * (g[i][j] - dot);
      }
      Vec<VW>::store(dr + q, d);
    }
  }
  if (threadIdx.x == 0) a.partial[row] = dot;
}

template <int VW, int NV>
__global__ __launch_bounds__(kThreads) void layernorm_grad_resident(RowArgs a) {
  __shared__ float lds[kWaves * 2];
  const int64_t row = blockIdx.x;
  const float* xr = a.x + row * a.ld;
  const float* gr = a.g + row * a.ld;
  float* dr = a.out + row * a.ld;
  float x[NV][VW], g[NV][VW];
  float sums[2] = {0.0f, 0.0f};
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int q = (i * kThreads + threadIdx.x) * VW;
    if (q < a.n) {
      Vec<VW>::load(xr + q, x[i]);
      Vec<VW>::load(gr + q, g[i]);
    } else {
#pragma unroll
      for (int j = 0; j < VW; ++j) x[i][j] = 0.0f, g[i][j] = 0.0f;
    }
#pragma unroll
    for (int j = 0; j < VW; ++j) sums[0] += x[i][j], sums[1] += g[i][j];
  }
  block_sums(sums, lds);
  const float rn = 1.0f / (float)a.n;
  const float mean = sums[0] * rn, gmean = sums[1] * rn;
  float dev[2] = {0.0f, 0.0f};  // sum (x - m)^2, sum g (x - m)
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int q = (i * kThreads + threadIdx.x) * VW;
    const bool live = q < a.n;
#pragma unroll
    for (int j = 0; j < VW; ++j) {
      float d = live ? x[i][j] - mean : 0.0f;
      x[i][j] = d;
      dev[0] = fmaf(d, d, dev[0]);
      dev[1] = fmaf(g[i][j], d, dev[1]);
    }
  }
  block_sums(dev, lds);
  const float r = 1.0f / sqrtf(dev[0] * rn + a.eps);
  const float gy = dev[1] * r;  // sum(g .* y) over the row
  const float gy_mean = gy * rn;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int q = (i * kThreads + threadIdx.x) * VW;
    if (q < a.n) {
      float d[VW];
#pragma unroll
      for (int j = 0; j < VW; ++j) {
        float y = x[i][j] * r;
        d[j] = r * (g[i][j] - gmean - y * gy_mean);
      }
      Vec<VW>::store(dr + q, d);
    }
  }
  if (threadIdx.x == 0) a.partial[row] = gy;
}

template <int VW, int NV>
__global__ __launch_bounds__(kThreads) void softmax_fwd_resident(RowArgs a) {
  __shared__ float lds[kWaves * 3];
  const int64_t row = blockIdx.x;
  const float* xr = a.x + row * a.ld;
  float* yr = a.out + row * a.ld;
  float x[NV][VW];
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int q = (i * kThreads + threadIdx.x) * VW;
    if (q < a.n) {
      Vec<VW>::load(xr + q, x[i]);
    } else {
#pragma unroll
      for (int j = 0; j < VW; ++j) x[i][j] = -INFINITY;
    }
#pragma unroll
    for (int j = 0; j < VW; ++j) m = fmaxf(m, x[i][j]);
  }
  const float sh = thd::lse_shift(m);
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i)
#pragma unroll
    for (int j = 0; j < VW; ++j) s += __expf(x[i][j] - sh);
  Exp3 st = block_combine(Exp3{m, s, 0.0f}, lds);
  const float inv = 1.0f / st.s;
  const float shift = thd::lse_shift(st.m);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int q = (i * kThreads + threadIdx.x) * VW;
    if (q < a.n) {
      float y[VW];
#pragma unroll
      for (int j = 0; j < VW; ++j) y[j] = __expf(x[i][j] - shift) * inv;
      Vec<VW>::store(yr + q, y);
    }
  }
}

template <int VW, int NV>
__global__ __launch_bounds__(kThreads) void layernorm_fwd_resident(RowArgs a) {
  __shared__ float lds[kWaves];
  const int64_t row = blockIdx.x;
  const float* xr = a.x + row * a.ld;
  float* yr = a.out + row * a.ld;
  float x[NV][VW];
  float sum[1] = {0.0f};
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int q = (i * kThreads + threadIdx.x) * VW;
    if (q < a.n) {
      Vec<VW>::load(xr + q, x[i]);
    } else {
#pragma unroll
      for (int j = 0; j < VW; ++j) x[i][j] = 0.0f;
    }
#pragma unroll
    for (int j = 0; j < VW; ++j) sum[0] += x[i][j];
  }
  block_sums(sum, lds);
  const float rn = 1.0f / (float)a.n;
  const float mean = sum[0] * rn;
  float dev[1] = {0.0f};
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int q = (i * kThreads + threadIdx.x) * VW;
    const bool live = q < a.n;
#pragma unroll
    for (int j = 0; j < VW; ++j) {
      float d = live ? x[i][j] - mean : 0.0f;
      x[i][j] = d;
      dev[0] = fmaf(d, d, dev[0]);
    }
  }
  block_sums(dev, lds);
  const float r = 1.0f / sqrtf(dev[0] * rn + a.eps);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int q = (i * kThreads + threadIdx.x) * VW;
    if (q < a.n) {
      float y[VW];
#pragma unroll
      for (int j = 0; j < VW; ++j) y[j] = x[i][j] * r;
      Vec<VW>::store(yr + q, y);
    }
  }
}

// ---- streamed kernels: rows longer than the registers hold ------------------
// The fold sweeps the row once; a second sweep re-reads it (from L2 where it
// stayed) to write.

template <int VW>
__global__ __launch_bounds__(kThreads) void softmax_grad_streamed(RowArgs a) {
  __shared__ float lds[kWaves * 3];
  const int64_t row = blockIdx.x;
  const float* xr = a.x + row * a.ld;
  const float* gr = a.g + row * a.ld;
  float* dr = a.out + row * a.ld;
  Exp3 st{-INFINITY, 0.0f, 0.0f};
  for (int q = threadIdx.x * VW; q < a.n; q += kThreads * VW) {
    float x[VW], g[VW];
    Vec<VW>::load(xr + q, x);
    Vec<VW>::load(gr + q, g);
#pragma unroll
    for (int j = 0; j < VW; ++j) st = exp_combine(st, Exp3{x[j], 1.0f, g[j]});
  }
  st = block_combine(st, lds);
  const float inv = 1.0f / st.s;
  const float dot = st.t * inv;
  const float shift = thd::lse_shift(st.m);
  for (int q = threadIdx.x * VW; q < a.n; q += kThreads * VW) {
    float x[VW], g[VW], d[VW];
    Vec<VW>::load(xr + q, x);
    Vec<VW>::load(gr + q, g);
#pragma unroll
    for (int j = 0; j < VW; ++j) d[j] = __expf(x[j] - shift) * inv * (g[j] - dot);
    Vec<VW>::store(dr + q, d);
  }
  if (threadIdx.x == 0) a.partial[row] = dot;
}

template <int VW>
__global__ __launch_bounds__(kThreads) void layernorm_grad_streamed(RowArgs a) {
  __shared__ float lds[kWaves * 2];
  const int64_t row = blockIdx.x;
  const float* xr = a.x + row * a.ld;
  const float* gr = a.g + row * a.ld;
  float* dr = a.out + row * a.ld;
  float sums[2] = {0.0f, 0.0f};
  for (int q = threadIdx.x * VW; q < a.n; q += kThreads * VW) {
    float x[VW], g[VW];
    Vec<VW>::load(xr + q, x);
    Vec<VW>::load(gr + q, g);
#pragma unroll
    for (int j = 0; j < VW; ++j) sums[0] += x[j], sums[1] += g[j];
  }
  block_sums(sums, lds);
  const float rn = 1.0f / (float)a.n;
  const float mean = sums[0] * rn, gmean = sums[1] * rn;
  float dev[2] = {0.0f, 0.0f};
  for (int q = threadIdx.x * VW; q < a.n; q += kThreads * VW) {
    float x[VW], g[VW];
    Vec<VW>::load(xr + q, x);
    Vec<VW>::load(gr + q, g);
#pragma unroll
    for (int j = 0; j < VW; ++j) {
      float d = x[j] - mean;
      dev[0] = fmaf(d, d, dev[0]);
      dev[1] = fmaf(g[j], d, dev[1]);
    }
  }
  block_sums(dev, lds);
  const float r = 1.0f / sqrtf(dev[0] * rn + a.eps);
  const float gy = dev[1] * r;
  const float gy_mean = gy * rn;
  for (int q = threadIdx.x * VW; q < a.n; q += kThreads * VW) {
    float x[VW], g[VW], d[VW];
    Vec<VW>::load(xr + q, x);
    Vec<VW>::load(gr + q, g);
#pragma unroll
    for (int j = 0; j < VW; ++j) d[j] = r * (g[j] - gmean - (x[j] - mean) * r * gy_mean);
    Vec<VW>::store(dr + q, d);
  }
  if (threadIdx.x == 0) a.partial[row] = gy;
}

// ---- a full sum: one workgroup, in double, in a fixed order ----------------

struct SumArgs {
  const float* x;
  float* out;
  int64_t count;
};

// Each thread sums a contiguous share (16-byte loads where aligned), the
// waves reduce by shuffles, and wave 0 folds the 16 wave sums in order.
__global__ __launch_bounds__(1024) void sum_all(SumArgs a) {
  __shared__ double lds[16];
  const int64_t per = (a.count + 1023) / 1024;
  const int64_t lo = min<int64_t>(a.count, per * threadIdx.x);
  const int64_t hi = min<int64_t>(a.count, lo + per);
  double s = 0.0;
  int64_t i = lo;
  if ((reinterpret_cast<uintptr_t>(a.x + i) & 15) == 0)
    for (; i + 4 <= hi; i += 4) {
      f32x4 v = *reinterpret_cast<const f32x4*>(a.x + i);
      s += (double)v[0] + (double)v[1] + (double)v[2] + (double)v[3];
    }
  for (; i < hi; ++i) s += (double)a.x[i];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
  if (threadIdx.x % 64 == 0) lds[threadIdx.x / 64] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    double t = 0.0;
    for (int w = 0; w < 16; ++w) t += lds[w];
    a.out[0] = (float)t;
  }
}

// ---- dispatch --------------------------------------------------------------

enum Op { kSoftmaxGrad, kLayerNormGrad, kSoftmaxFwd, kLayerNormFwd };

template <int VW, int NV>
const void* resident(Op op) {
  switch (op) {
    case kSoftmaxGrad: return (const void*)softmax_grad_resident<VW, NV>;
    case kLayerNormGrad: return (const void*)layernorm_grad_resident<VW, NV>;
    case kSoftmaxFwd: return (const void*)softmax_fwd_resident<VW, NV>;
    case kLayerNormFwd: return (const void*)layernorm_fwd_resident<VW, NV>;
  }
  return nullptr;
}

// The kernel for a row of n at stride ld: 16-byte loads where the rows allow
// them, resident while a thread's share is at most 16 loads.
const void* pick(Op op, int32_t n, int64_t ld, bool aligned, const char** name) {
  const bool v4 = aligned && n % 4 == 0 && ld % 4 == 0;
  const int vw = v4 ? 4 : 1;
  const int64_t per = ((int64_t)n + (int64_t)kThreads * vw - 1) / ((int64_t)kThreads * vw);
  const bool fwd = op == kSoftmaxFwd || op == kLayerNormFwd;
  if (per <= 16) {
    *name = v4 ? "rows_resident_v4" : "rows_resident_v1";
    if (v4) {
      if (per <= 1) return resident<4, 1>(op);
      if (per <= 2) return resident<4, 2>(op);
      if (per <= 4) return resident<4, 4>(op);
      if (per <= 8) return resident<4, 8>(op);
      return resident<4, 16>(op);
    }
    if (per <= 1) return resident<1, 1>(op);
    if (per <= 4) return resident<1, 4>(op);
    if (per <= 16) return resident<1, 16>(op);
  }
  if (fwd) return nullptr;  // forward rows longer than 16 K elements: not built
  *name = v4 ? "rows_streamed_v4" : "rows_streamed_v1";
  if (op == kSoftmaxGrad) return v4 ? (const void*)softmax_grad_streamed<4> : (const void*)softmax_grad_streamed<1>;
  return v4 ? (const void*)layernorm_grad_streamed<4> : (const void*)layernorm_grad_streamed<1>;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

int build_rows(Op op, const char* title, int64_t rows, int32_t n, int64_t ld, float eps,
               const float* x, const float* g, float* out, float* loss, th_launch** host_out) {
  if (int r = th::require_ready()) return r;
  *host_out = nullptr;
  const bool grad = op == kSoftmaxGrad || op == kLayerNormGrad;
  TH_REQUIRE(rows >= 1 && rows <= 0x7fffffff, std::string(title) + ": rows must be in 1..2^31-1");
  TH_REQUIRE(n >= 1, std::string(title) + ": n must be positive");
  TH_REQUIRE(ld >= n, std::string(title) + ": ld must be at least n");
  TH_REQUIRE(x && out && (!grad || (g && loss)), std::string(title) + ": null pointer");
  // Repointed storage must keep the alignment the build chose.
  const bool aligned = aligned16(x) && aligned16(out) && (!grad || aligned16(g));
  const char* kname = "";
  const void* fn = pick(op, n, ld, aligned, &kname);
  if (!fn)
    return th::fail(TH_E_UNSUPPORTED, std::string(title) + ": rows longer than 16384 are not built");
  th::Builder b(title, grad ? 4 : 2);
  RowArgs a{x, g, out, nullptr, rows, ld, n, eps};
  // Workspace: the rows' loss partials.
  const uint64_t at_partial = grad ? b.workspace((uint64_t)rows * sizeof(float)) : 0;
  int k = b.kernel(fn, kname, dim3((unsigned)rows), dim3(kThreads), 0, a);
  b.ref(0, k, TH_OFFSET(RowArgs, x));
  const uint32_t need = (n % 4 == 0 && ld % 4 == 0 && aligned) ? 16 : 4;
  b.align(0, need);
  b.align(grad ? 2 : 1, need);
  if (grad) b.align(1, need);
  if (grad) {
    b.ref(1, k, TH_OFFSET(RowArgs, g));
    b.ref(2, k, TH_OFFSET(RowArgs, out));
    SumArgs s{a.partial, loss, rows};
    int k2 = b.kernel((const void*)sum_all, "sum_all", dim3(1), dim3(1024), 0, s);
    b.ref(3, k2, TH_OFFSET(SumArgs, out));
    b.ws_ref(k, TH_OFFSET(RowArgs, partial), at_partial);
    b.ws_ref(k2, TH_OFFSET(SumArgs, x), at_partial);
    b.work(3.0 * 4.0 * (double)rows * n, (op == kSoftmaxGrad ? 8.0 : 10.0) * (double)rows * n,
           rows);
  } else {
    b.ref(1, k, TH_OFFSET(RowArgs, out));
    b.work(2.0 * 4.0 * (double)rows * n, 5.0 * (double)rows * n, rows);
  }
  *host_out = b.release();
  return TH_OK;
}

}  // namespace

// ---- the softmax gradient that allocates nothing --------------------------
//
// th_softmax_grad_noalloc keeps its per-row loss partials in this array, one
// copy per GPU, held until the process ends.  Host code reaches it only
// through the address hipGetSymbolAddress gives on each device (the array's
// name in host code is a stand-in, not a device address).
constexpr int64_t kScratchRows = int64_t(1) << 20;  // 4 MiB of fp32 partials
constexpr int kScratchDevices = 64;
static __device__ __align__(256) float scratch[kScratchRows];
static float* g_scratch[kScratchDevices];

namespace th {

int rows_scratch_setup(int device) {
  TH_REQUIRE(device >= 0 && device < kScratchDevices, "rows_scratch_setup: device out of range");
  if (g_scratch[device]) return TH_OK;
  void* ptr = nullptr;
  TH_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
  g_scratch[device] = static_cast<float*>(ptr);
  return TH_OK;
}

}  // namespace th

extern "C" {

int th_softmax_grad_noalloc(int64_t rows, int32_t n, int64_t ld, const float* x, const float* g,
                            float* dx, float* loss) {
  if (int r = th::require_ready()) return r;
  const char* title = "th_softmax_grad_noalloc";
  TH_REQUIRE(rows >= 1 && rows <= kScratchRows,
             std::string(title) + ": rows must be in 1.." + std::to_string(kScratchRows) +
                 " (the partials' static scratch holds that many)");
  TH_REQUIRE(n >= 1, std::string(title) + ": n must be positive");
  TH_REQUIRE(ld >= n, std::string(title) + ": ld must be at least n");
  TH_REQUIRE(x && g && dx && loss, std::string(title) + ": null pointer");
  float* partial = g_scratch[th::ctx().device];
  if (!partial) return th::fail(TH_E_STATE, std::string(title) + ": scratch address not set up by th_init");
  const bool aligned = aligned16(x) && aligned16(g) && aligned16(dx);
  const char* kname = "";
  const void* fn = pick(kSoftmaxGrad, n, ld, aligned, &kname);
  // Every row's partial is written before sum_all reads it: nothing to clear.
  th::Kernel k;
  k.fn = fn;
  k.name = kname;
  k.grid = dim3((unsigned)rows);
  k.block = dim3(kThreads);
  RowArgs a{x, g, dx, partial, rows, ld, n, 0.0f};
  std::memcpy(k.args, &a, sizeof a);
  k.args_size = sizeof a;
  if (int r = th::launch_kernel(k, th::ctx().stream)) return r;
  th::Kernel k2;
  k2.fn = (const void*)sum_all;
  k2.name = "sum_all";
  k2.grid = dim3(1);
  k2.block = dim3(1024);
  SumArgs sa{partial, loss, rows};
  std::memcpy(k2.args, &sa, sizeof sa);
  k2.args_size = sizeof sa;
  return th::launch_kernel(k2, th::ctx().stream);
}

int th_build_softmax_grad(int64_t rows, int32_t n, int64_t ld, const float* x, const float* g,
                          float* dx, float* loss, th_launch** out) {
  return build_rows(kSoftmaxGrad, "softmax_grad", rows, n, ld, 0.0f, x, g, dx, loss, out);
}

int th_build_layernorm_grad(int64_t rows, int32_t n, int64_t ld, float eps, const float* x,
                            const float* g, float* dx, float* loss, th_launch** out) {
  return build_rows(kLayerNormGrad, "layernorm_grad", rows, n, ld, eps, x, g, dx, loss, out);
}

int th_build_softmax_fwd(int64_t rows, int32_t n, int64_t ld, const float* x, float* y,
                         th_launch** out) {
  return build_rows(kSoftmaxFwd, "softmax_fwd", rows, n, ld, 0.0f, x, nullptr, y, nullptr, out);
}

int th_build_layernorm_fwd(int64_t rows, int32_t n, int64_t ld, float eps, const float* x,
                           float* y, th_launch** out) {
  return build_rows(kLayerNormFwd, "layernorm_fwd", rows, n, ld, eps, x, nullptr, y, nullptr,
                    out);
}

int th_build_sum(int64_t count, const float* x, float* out, th_launch** host_out) {
  if (int r = th::require_ready()) return r;
  *host_out = nullptr;
  TH_REQUIRE(count >= 0, "th_build_sum: negative count");
  TH_REQUIRE(x && out, "th_build_sum: null pointer");
  th::Builder b("sum", 2);
  SumArgs s{x, out, count};
  int k = b.kernel((const void*)sum_all, "sum_all", dim3(1), dim3(1024), 0, s);
  b.ref(0, k, TH_OFFSET(SumArgs, x));
  b.ref(1, k, TH_OFFSET(SumArgs, out));
  b.work(4.0 * (double)count, (double)count, 1);
  *host_out = b.release();
  return TH_OK;
}

}  // extern "C"
