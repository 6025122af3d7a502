// The small program of config 1, whole in one workgroup:
//   loss(w, b, x) = sum(abs2, tanh.(w' * x .+ b))
// and its gradient as withgradient forms it.  Every value fits the LDS
// (w 32 x 64, x 32 x 16 floats), so the product, the pointwise map, the loss's
// fold and the three gradient products run as one launch: the step is bound
// by launch latency, and one kernel is the least of it.
//
// Gradient (the reverse pass of the program, scalar_partials of tanh and
// abs2, src/Compiler/program/differentiate.jl:106-155):
//   z = w' x .+ b, y = tanh.(z), loss = sum(y .^ 2)
//   dz = 2 y (1 - y^2)
//   dw = x dz',  dx = w dz,  db = sum(dz; dims = 2)
// Every fold is sequential within its item, left to right, as the CPU floor
// runs it (src/Compiler/codegen/scalar.jl:200-256); the loss's is a tree.
#include <hip/hip_runtime.h>

#include <cmath>

#include "th_core.h"

namespace {

constexpr int kThreads = 1024;
constexpr int kMaxLds = 16384;  // floats (64 KiB)

struct TanhArgs {
  const float* w;
  const float* b;
  const float* x;
  float* loss;
  float* dw;
  float* db;
  float* dx;
  int32_t d, h, c;
};

// LDS rows are padded to a multiple of 4 floats plus 4, so that the lanes of
// a wave reading neighbouring columns with 16-byte loads hit distinct banks.
__device__ __forceinline__ int padded(int d) { return ((d + 3) / 4) * 4 + 4; }

__global__ __launch_bounds__(kThreads) void tanh_layer_grad(TanhArgs a) {
  extern __shared__ float lds[];
  const int d = a.d, h = a.h, c = a.c;
  const int pd = padded(d);
  float* w = lds;            // h columns of d, stride pd
  float* x = w + pd * h;     // c columns of d, stride pd
  float* dz = x + pd * c;    // h x c
  float* red = dz + h * c;   // kThreads / 64 partial sums
  const int tid = threadIdx.x;
  for (int i = tid; i < d * h; i += kThreads) w[(i / d) * pd + i % d] = a.w[i];
  for (int i = tid; i < d * c; i += kThreads) x[(i / d) * pd + i % d] = a.x[i];
  for (int i = tid; i < (pd - d) * (h + c); i += kThreads) {
    const int col = i / (pd - d), k = d + i % (pd - d);
    (col < h ? w + col * pd : x + (col - h) * pd)[k] = 0.0f;  // zero padding
  }
  __syncthreads();
  float sq = 0.0f;
  for (int item = tid; item < h * c; item += kThreads) {
    const int j = item % h, col = item / h;
    const float4* wj = reinterpret_cast<const float4*>(w + j * pd);
    const float4* xc = reinterpret_cast<const float4*>(x + col * pd);
    float z = 0.0f;
    for (int q = 0; q < pd / 4; ++q) {
      const float4 u = wj[q], v = xc[q];
      z = fmaf(u.x, v.x, z);
      z = fmaf(u.y, v.y, z);
      z = fmaf(u.z, v.z, z);
      z = fmaf(u.w, v.w, z);
    }
    z += a.b[j];
    const float y = tanhf(z);
    sq = fmaf(y, y, sq);
    dz[item] = 2.0f * y * (1.0f - y * y);
  }
  // The loss: a tree over the workgroup, waves in order.
  sq = thd::wave_sum(sq);
  if (tid % 64 == 0) red[tid / 64] = sq;
  __syncthreads();
  if (tid == 0) {
    float s = 0.0f;
    for (int k = 0; k < kThreads / 64; ++k) s += red[k];
    a.loss[0] = s;
  }
  // dw = x dz' (d x h), dx = w dz (d x c), db = sum over columns (h).
  for (int item = tid; item < d * h; item += kThreads) {
    const int i = item % d, j = item / d;
    float s = 0.0f;
    for (int col = 0; col < c; ++col) s = fmaf(x[col * pd + i], dz[j + h * col], s);
    a.dw[item] = s;
  }
  for (int item = tid; item < d * c; item += kThreads) {
    const int i = item % d, col = item / d;
    float s = 0.0f;
    for (int j = 0; j < h; ++j) s = fmaf(w[j * pd + i], dz[j + h * col], s);
    a.dx[item] = s;
  }
  for (int j = tid; j < h; j += kThreads) {
    float s = 0.0f;
    for (int col = 0; col < c; ++col) s += dz[j + h * col];
    a.db[j] = s;
  }
}

}  // namespace

extern "C" int th_build_tanh_layer_grad(int32_t d, int32_t h, int32_t c, const float* w,
                                        const float* b, const float* x, float* loss, float* dw,
                                        float* db, float* dx, th_launch** out) {
  if (int r = th::require_ready()) return r;
  *out = nullptr;
  TH_REQUIRE(d >= 1 && h >= 1 && c >= 1, "th_build_tanh_layer_grad: sizes must be positive");
  const int64_t pd = ((d + 3) / 4) * 4 + 4;
  const int64_t floats = pd * h + pd * c + (int64_t)h * c + kThreads / 64;
  TH_REQUIRE(floats <= kMaxLds,
             "th_build_tanh_layer_grad: (d+4)*(h+c) + h*c floats must fit one workgroup's 64 KiB");
  TH_REQUIRE(w && b && x && loss && dw && db && dx, "th_build_tanh_layer_grad: null pointer");
  th::Builder bld("tanh_layer_grad", 7);
  TanhArgs a{w, b, x, loss, dw, db, dx, d, h, c};
  int k = bld.kernel((const void*)tanh_layer_grad, "tanh_layer_grad", dim3(1), dim3(kThreads),
                     (uint32_t)(floats * sizeof(float)), a);
  bld.ref(0, k, TH_OFFSET(TanhArgs, w));
  bld.ref(1, k, TH_OFFSET(TanhArgs, b));
  bld.ref(2, k, TH_OFFSET(TanhArgs, x));
  bld.ref(3, k, TH_OFFSET(TanhArgs, loss));
  bld.ref(4, k, TH_OFFSET(TanhArgs, dw));
  bld.ref(5, k, TH_OFFSET(TanhArgs, db));
  bld.ref(6, k, TH_OFFSET(TanhArgs, dx));
  const double dd = d, hh = h, cc = c;
  bld.work(4.0 * (dd * hh + hh + dd * cc + 1 + dd * hh + hh + dd * cc),
           2.0 * dd * hh * cc * 3 + 8.0 * hh * cc, 1);
  *out = bld.release();
  return TH_OK;
}
