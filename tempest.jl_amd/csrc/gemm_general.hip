// Op class (b), general shapes: C = A B (+ D) over a batch, for what the bf16
// tile kernel does not take: fp32 or fp16 factors, any m, n, k (the
// reference's product fixtures are 9 x 7 * 7 x 10, matrix-vector, 5 x 4 ...,
// test/fixtures/programs.jl:79-96), operands without a unit stride, and
// results in fp32, bf16 or fp16.  cuBLASProducts takes Float32, Float16 and
// BFloat16 factors with a same-type or fp32 result (ext/cuBLASExt.jl:23-36).
//
// Factors are widened to fp32 on their way into LDS and multiplied on the
// matrix cores in fp32 (v_mfma_f32_16x16x4_f32: exact products, fp32 sums),
// so the result is the reference interpreter's contraction (half factors
// widened, one rounding at the end, src/Compiler/program/interpret.jl:58-63)
// up to the order of the additions.  A workgroup of four waves takes a
// 64 x 64 tile of C, each wave 32 x 32 as 2 x 2 blocks of 16 x 16; K moves 16
// at a time through LDS, the next slice loaded into registers while the
// current one is multiplied.  Bounds are checked on every load and store.
#include <hip/hip_runtime.h>

#include "th_core.h"

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

struct GenGemmArgs {
  const void* a;
  const void* b;
  void* c;
  const void* d;  // C = D + A B where non-null, laid out as C at d_ld / d_batch
  int64_t a_m, a_k, a_batch;
  int64_t b_k, b_n, b_batch;
  int64_t c_ld, c_batch;
  int64_t d_ld, d_batch;
  int32_t m, n, k;
  int32_t factor;  // TH_F32, TH_BF16 or TH_F16
  int32_t result;  // TH_F32, TH_BF16 or TH_F16
};

constexpr int kT = 64;   // C tile
constexpr int kKs = 16;  // K per step
constexpr int kPad = kT + 4;

__device__ __forceinline__ float widen(const void* p, int64_t i, int type) {
  if (type == TH_F32) return static_cast<const float*>(p)[i];
  const uint16_t h = static_cast<const uint16_t*>(p)[i];
  if (type == TH_BF16) return __uint_as_float((uint32_t)h << 16);
  return (float)__builtin_bit_cast(_Float16, h);
}

__device__ __forceinline__ void narrow(void* p, int64_t i, int type, float x) {
  if (type == TH_F32) {
    static_cast<float*>(p)[i] = x;
  } else if (type == TH_BF16) {
    static_cast<uint16_t*>(p)[i] = __builtin_bit_cast(uint16_t, (__bf16)x);
  } else {
    static_cast<uint16_t*>(p)[i] = __builtin_bit_cast(uint16_t, (_Float16)x);
  }
}

// The 64 x 16 slice of A (rows m0.., columns k0..) or 16 x 64 of B into four
// registers a thread: along the operand's unit stride where it has one.
struct Slice {
  float v[4];
};

__device__ __forceinline__ void load_a(const GenGemmArgs& p, const void* a, int m0, int k0, Slice& s) {
  const int t = threadIdx.x;
  const bool m_unit = p.a_m == 1;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int mm = m_unit ? t % kT : t / kKs + 16 * i;
    const int kk = m_unit ? t / kT + 4 * i : t % kKs;
    const int m = m0 + mm, k = k0 + kk;
    s.v[i] = (m < p.m && k < p.k) ? widen(a, (int64_t)m * p.a_m + (int64_t)k * p.a_k, p.factor) : 0.0f;
  }
}

__device__ __forceinline__ void store_a(const GenGemmArgs& p, float* As, const Slice& s) {
  const int t = threadIdx.x;
  const bool m_unit = p.a_m == 1;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int mm = m_unit ? t % kT : t / kKs + 16 * i;
    const int kk = m_unit ? t / kT + 4 * i : t % kKs;
    As[kk * kPad + mm] = s.v[i];
  }
}

__device__ __forceinline__ void load_b(const GenGemmArgs& p, const void* b, int n0, int k0, Slice& s) {
  const int t = threadIdx.x;
  const bool n_unit = p.b_n == 1 && p.b_k != 1;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int nn = n_unit ? t % kT : t / kKs + 16 * i;
    const int kk = n_unit ? t / kT + 4 * i : t % kKs;
    const int n = n0 + nn, k = k0 + kk;
    s.v[i] = (n < p.n && k < p.k) ? widen(b, (int64_t)k * p.b_k + (int64_t)n * p.b_n, p.factor) : 0.0f;
  }
}

__device__ __forceinline__ void store_b(const GenGemmArgs& p, float* Bs, const Slice& s) {
  const int t = threadIdx.x;
  const bool n_unit = p.b_n == 1 && p.b_k != 1;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int nn = n_unit ? t % kT : t / kKs + 16 * i;
    const int kk = n_unit ? t / kT + 4 * i : t % kKs;
    Bs[kk * kPad + nn] = s.v[i];
  }
}

__global__ __launch_bounds__(256) void gemm_general(GenGemmArgs p) {
  __shared__ float As[2][kKs * kPad];  // [k][m]
  __shared__ float Bs[2][kKs * kPad];  // [k][n]
  const int z = blockIdx.z;
  const int m0 = blockIdx.x * kT, n0 = blockIdx.y * kT;
  const char* a = static_cast<const char*>(p.a) + z * p.a_batch * (p.factor == TH_F32 ? 4 : 2);
  const char* b = static_cast<const char*>(p.b) + z * p.b_batch * (p.factor == TH_F32 ? 4 : 2);
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int wm = (wave / 2) * 32, wn = (wave % 2) * 32;
  f32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  Slice sa, sb;
  load_a(p, a, m0, 0, sa);
  load_b(p, b, n0, 0, sb);
  store_a(p, As[0], sa);
  store_b(p, Bs[0], sb);
  __syncthreads();
  const int steps = (p.k + kKs - 1) / kKs;
  for (int st = 0; st < steps; ++st) {
    const int cur = st & 1;
    if (st + 1 < steps) {
      load_a(p, a, m0, (st + 1) * kKs, sa);
      load_b(p, b, n0, (st + 1) * kKs, sb);
    }
    // v_mfma_f32_16x16x4_f32: lane l gives A(row l % 16, k l / 16) and
    // B(k l / 16, column l % 16); it holds C(rows 4 (l / 16) + 0..3, column l % 16).
#pragma unroll
    for (int kk = 0; kk < kKs; kk += 4) {
      const int kr = kk + lane / 16;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const float av = As[cur][kr * kPad + wm + 16 * i + lane % 16];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const float bv = Bs[cur][kr * kPad + wn + 16 * j + lane % 16];
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc[i][j], 0, 0, 0);
        }
      }
    }
    if (st + 1 < steps) {
      store_a(p, As[cur ^ 1], sa);
      store_b(p, Bs[cur ^ 1], sb);
    }
    __syncthreads();
  }
  const int rt = p.result == TH_F32 ? 4 : 2;
  char* c = static_cast<char*>(p.c) + z * p.c_batch * rt;
  const char* d = p.d ? static_cast<const char*>(p.d) + z * p.d_batch * rt : nullptr;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = n0 + wn + 16 * j + lane % 16;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + wm + 16 * i + 4 * (lane / 16) + r;
        if (m < p.m && n < p.n) {
          float v = acc[i][j][r];
          if (d) v += widen(d, (int64_t)m + (int64_t)n * p.d_ld, p.result);
          narrow(c, (int64_t)m + (int64_t)n * p.c_ld, p.result, v);
        }
      }
    }
}

int esize(int t) { return t == TH_F32 ? 4 : 2; }

}  // namespace

namespace th {

int build_gemm_general(const th_gemm_desc* d, th_launch** out) {
  const int batch = d->batch > 0 ? d->batch : 1;
  TH_REQUIRE(d->epilogue == TH_EPI_STORE && !d->bias,
             "th_build_gemm: fused epilogues and biases need bf16 factors in the tile kernel's shapes");
  const int factor = (d->flags & TH_GEMM_F32_FACTORS) ? TH_F32 : (d->flags & TH_GEMM_F16_FACTORS) ? TH_F16 : TH_BF16;
  TH_REQUIRE(d->c_dtype == TH_F32 || d->c_dtype == TH_BF16 || d->c_dtype == TH_F16,
             "th_build_gemm: the result is fp32, bf16 or fp16");
  TH_REQUIRE(d->c_dtype == factor || d->c_dtype == TH_F32,
             "th_build_gemm: the result is the factors' type or fp32 (widened)");
  TH_REQUIRE(d->m <= 65535 * kT && d->n <= 65535 * kT && batch <= 65535, "th_build_gemm: grid too large");
  const bool acc = (d->flags & TH_GEMM_ACCUMULATE) != 0;
  TH_REQUIRE(!acc || d->d, "th_build_gemm: accumulating needs d");
  GenGemmArgs a{};
  a.a = d->a, a.b = d->b, a.c = d->c, a.d = acc ? d->d : nullptr;
  a.a_m = d->a_m, a.a_k = d->a_k, a.a_batch = d->a_batch;
  a.b_k = d->b_k, a.b_n = d->b_n, a.b_batch = d->b_batch;
  a.c_ld = d->c_ld, a.c_batch = d->c_batch;
  a.d_ld = d->d_ld ? d->d_ld : d->c_ld, a.d_batch = d->d_ld ? d->d_batch : d->c_batch;
  a.m = d->m, a.n = d->n, a.k = d->k;
  a.factor = factor, a.result = d->c_dtype;
  th::Builder b("gemm_general", 9);
  const dim3 grid((d->m + kT - 1) / kT, (d->n + kT - 1) / kT, batch);
  int k = b.kernel((const void*)gemm_general, "gemm_general_f32mfma", grid, dim3(256), 0, a);
  b.ref(0, k, TH_OFFSET(GenGemmArgs, a));
  b.ref(1, k, TH_OFFSET(GenGemmArgs, b));
  b.ref(2, k, TH_OFFSET(GenGemmArgs, c));
  b.ref(8, k, TH_OFFSET(GenGemmArgs, d));
  const double mm = d->m, nn = d->n, kk = d->k, bb = batch;
  const double bytes = bb * (esize(factor) * (mm * kk + kk * nn) + esize(d->c_dtype) * mm * nn * (acc ? 2 : 1));
  b.work(bytes, 2.0 * bb * mm * nn * kk, (int64_t)grid.x * grid.y * grid.z);
  *out = b.release();
  return TH_OK;
}

}  // namespace th
