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

/* bfloat16 bits widened to float. */
static float bf(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, sizeof f);
  return f;
}

/*
 * Config 3's products as the floor runs them on one core: C(i, j) = the fold
 * over l of A(i, l) B(l, j), an item per element of C in column-major order,
 * each fold sequential in fp32 over bf16 factors widened (codegen/scalar.jl:
 * 200-256; half factors accumulate in fp32, IR/folds.jl:306-309).  A(i, l) is
 * a[i a_m + l a_k], B(l, j) is b[l b_k + j b_n]; only the columns j0 .. j1 - 1
 * of C are computed (a slice whose work is (j1 - j0) / n of the product's).
 */
void floor_matmul_bf16(int32_t m, int32_t k, const uint16_t* a, int64_t a_m, int64_t a_k, const uint16_t* b,
                       int64_t b_k, int64_t b_n, float* c, int64_t c_ld, int32_t j0, int32_t j1) {
  for (int32_t j = j0; j < j1; ++j)
    for (int32_t i = 0; i < m; ++i) {
      float s = 0.0f;
      for (int32_t l = 0; l < k; ++l) s += bf(a[i * a_m + l * a_k]) * bf(b[l * b_k + j * b_n]);
      c[i + (int64_t)(j - j0) * c_ld] = s;
    }
}

/*
 * Config 4 on one core for one (batch, head) and a sample of its queries
 * (q0, q0 + step, ...): the program's forward (scores over the keys a query
 * sees, causal; its maximum, exponentials and sum; o = P V) and backward
 * (delta = dO . o, dP = dO V', dS = P (dP - delta), dq = scale dS K,
 * dk += scale dS' q, dv += P' dO) for each sampled query, every fold
 * sequential in fp32 (test/fixtures/operations.jl:21-70).  q, k, v, dout:
 * bf16 rows of d at `stride` elements per position.  dq: one row per sampled
 * query; dk, dv: seq x d fp32, accumulated.  `p` is seq floats of scratch.
 * Work: 12 d flops per (query, key) pair it sweeps.
 */
void floor_attention_sample(int32_t seq, int32_t d, float scale, const uint16_t* q, const uint16_t* k,
                            const uint16_t* v, const uint16_t* dout, int64_t stride, int32_t q0, int32_t step,
                            float* dq, float* dk, float* dv, float* p) {
  int32_t row = 0;
  for (int32_t i = q0; i < seq; i += step, ++row) {
    const uint16_t* qi = q + (int64_t)i * stride;
    const uint16_t* gi = dout + (int64_t)i * stride;
    float mx = -INFINITY;
    for (int32_t j = 0; j <= i; ++j) {
      float s = 0.0f;
      for (int32_t e = 0; e < d; ++e) s += bf(qi[e]) * bf(k[(int64_t)j * stride + e]);
      p[j] = s * scale;
      mx = p[j] > mx ? p[j] : mx;
    }
    float l = 0.0f;
    for (int32_t j = 0; j <= i; ++j) {
      p[j] = expf(p[j] - lse_shift(mx));
      l += p[j];
    }
    float delta = 0.0f;
    float* dqi = dq + (int64_t)row * d;
    for (int32_t e = 0; e < d; ++e) {
      float o = 0.0f;
      for (int32_t j = 0; j <= i; ++j) o += p[j] * bf(v[(int64_t)j * stride + e]);
      delta += bf(gi[e]) * (o / l);
      dqi[e] = 0.0f;
    }
    for (int32_t j = 0; j <= i; ++j) {
      const float pj = p[j] / l;
      float dp = 0.0f;
      for (int32_t e = 0; e < d; ++e) dp += bf(gi[e]) * bf(v[(int64_t)j * stride + e]);
      const float ds = pj * (dp - delta);
      for (int32_t e = 0; e < d; ++e) {
        dqi[e] += scale * ds * bf(k[(int64_t)j * stride + e]);
        dk[(int64_t)j * d + e] += scale * ds * bf(qi[e]);
        dv[(int64_t)j * d + e] += pj * bf(gi[e]);
      }
    }
  }
}
