/*
 * TEST INFRASTRUCTURE ONLY -- the CPU restatement of the reference's floor.
 *
 * Tempest's CPU path runs every kernel of a plan as a generated loop over its
 * items on one thread (floor_launch(::CPUTarget), src/Compiler/runtime/
 * target.jl:308-327), each fold sequential left to right in its accumulator
 * type: Float32 for Float32 data and for half data (IR/folds.jl:40,306-309;
 * codegen/scalar.jl:200-256).  This file restates that order for the
 * programs of the hot path, single-threaded by construction.  It is the
 * checker and the CPU baseline; nothing in the product links it.
 *
 * Julia is absent here, so the plan each program takes (which folds are
 * stored, which recomputed) is restated from the program's text, not read
 * from the reference's planner; each function says the plan it follows.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* The shift an exponential sum takes against its maximum
 * (lse_shift, src/Compiler/IR/folds.jl:194). */
static float lse_shift(float m) { return isfinite(m) ? m : 0.0f; }

/*
 * sum(softmax_columns(x) .* g) and its gradient, x and g n x rows
 * (test/fixtures/programs.jl:8,74).  Plan: per column, the log-sum-exp as the
 * online exponential fold (Relative{Exponential} observed as LOGSUMEXP,
 * folds.jl:186-222, 263), element by element; then y = exp(x - lse) and the
 * column's sum(y .* g) in order; then dx = y .* (g - that sum).  The loss
 * folds the columns' sums in column order.
 */
void floor_softmax_grad(int64_t rows, int32_t n, int64_t ld, const float* x, const float* g,
                        float* dx, float* loss) {
  float total = 0.0f;
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * ld;
    const float* gr = g + r * ld;
    float* dr = dx + r * ld;
    float m = -INFINITY, s = 0.0f;
    for (int32_t j = 0; j < n; ++j) {
      float mn = fmaxf(m, xr[j]);
      float sh = lse_shift(mn);
      s = s * expf(m - sh) + expf(xr[j] - sh);
      m = mn;
    }
    const float lse = m + logf(s);
    float dot = 0.0f;
    for (int32_t j = 0; j < n; ++j) dot += expf(xr[j] - lse) * gr[j];
    for (int32_t j = 0; j < n; ++j) dr[j] = expf(xr[j] - lse) * (gr[j] - dot);
    total += dot;
  }
  *loss = total;
}

/*
 * sum(layernorm(x) .* g) and its gradient, weight 1 and bias 0, as
 * test/fixtures/programs.jl:13-17 spells it: m = sum(x)/n, then
 * v = sum(abs2, x .- m)/n, y = (x .- m) ./ sqrt.(v .+ eps); the gradient
 * r .* (g .- mean(g) .- y .* mean(g .* y)), r = 1/sqrt(v + eps).
 */
void floor_layernorm_grad(int64_t rows, int32_t n, int64_t ld, float eps, const float* x,
                          const float* g, float* dx, float* loss) {
  float total = 0.0f;
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * ld;
    const float* gr = g + r * ld;
    float* dr = dx + r * ld;
    float sx = 0.0f, sg = 0.0f;
    for (int32_t j = 0; j < n; ++j) sx += xr[j];
    const float m = sx / (float)n;
    float v = 0.0f;
    for (int32_t j = 0; j < n; ++j) v += (xr[j] - m) * (xr[j] - m);
    v = v / (float)n;
    const float rs = 1.0f / sqrtf(v + eps);
    float gy = 0.0f;
    for (int32_t j = 0; j < n; ++j) {
      gy += gr[j] * ((xr[j] - m) * rs);
      sg += gr[j];
    }
    const float gmean = sg / (float)n, gymean = gy / (float)n;
    for (int32_t j = 0; j < n; ++j) dr[j] = rs * (gr[j] - gmean - ((xr[j] - m) * rs) * gymean);
    total += gy;
  }
  *loss = total;
}

/* Forward softmax over each column (test/fixtures/programs.jl:8). */
void floor_softmax_fwd(int64_t rows, int32_t n, int64_t ld, const float* x, float* y) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * ld;
    float m = -INFINITY, s = 0.0f;
    for (int32_t j = 0; j < n; ++j) {
      float mn = fmaxf(m, xr[j]);
      float sh = lse_shift(mn);
      s = s * expf(m - sh) + expf(xr[j] - sh);
      m = mn;
    }
    const float lse = m + logf(s);
    for (int32_t j = 0; j < n; ++j) y[r * ld + j] = expf(xr[j] - lse);
  }
}

/* Forward LayerNorm, weight 1, bias 0 (test/fixtures/programs.jl:13-17). */
void floor_layernorm_fwd(int64_t rows, int32_t n, int64_t ld, float eps, const float* x,
                         float* y) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * ld;
    float sx = 0.0f;
    for (int32_t j = 0; j < n; ++j) sx += xr[j];
    const float m = sx / (float)n;
    float v = 0.0f;
    for (int32_t j = 0; j < n; ++j) v += (xr[j] - m) * (xr[j] - m);
    const float rs = 1.0f / sqrtf(v / (float)n + eps);
    for (int32_t j = 0; j < n; ++j) y[r * ld + j] = (xr[j] - m) * rs;
  }
}

/*
 * Config 1: loss(w, b, x) = sum(abs2, tanh.(w' * x .+ b)) and its gradient;
 * w d x h, b h, x d x c, column-major.  Plan: z = w'x .+ b item by item (a
 * fold over d in order), y = tanh(z), the loss a left fold over the h x c
 * items in column-major order, dz = 2y(1 - y^2), then the three products,
 * each a fold in order (scalar_partials of tanh and abs2,
 * src/Compiler/program/differentiate.jl:106-155).
 */
void floor_tanh_layer_grad(int32_t d, int32_t h, int32_t c, const float* w, const float* b,
                           const float* x, float* loss, float* dw, float* db, float* dx,
                           float* dz /* h x c scratch */) {
  float l = 0.0f;
  for (int32_t col = 0; col < c; ++col)
    for (int32_t j = 0; j < h; ++j) {
      float z = 0.0f;
      for (int32_t i = 0; i < d; ++i) z += w[i + d * j] * x[i + d * col];
      z += b[j];
      float y = tanhf(z);
      l += y * y;
      dz[j + h * col] = 2.0f * y * (1.0f - y * y);
    }
  *loss = l;
  for (int32_t j = 0; j < h; ++j)
    for (int32_t i = 0; i < d; ++i) {
      float s = 0.0f;
      for (int32_t col = 0; col < c; ++col) s += x[i + d * col] * dz[j + h * col];
      dw[i + d * j] = s;
    }
  for (int32_t col = 0; col < c; ++col)
    for (int32_t i = 0; i < d; ++i) {
      float s = 0.0f;
      for (int32_t j = 0; j < h; ++j) s += w[i + d * j] * dz[j + h * col];
      dx[i + d * col] = s;
    }
  for (int32_t j = 0; j < h; ++j) {
    float s = 0.0f;
    for (int32_t col = 0; col < c; ++col) s += dz[j + h * col];
    db[j] = s;
  }
}
