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

#include <algorithm>

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

// ---- fp32 factors: 128 x 128 tiles, K split over parts ----------------------------
// A workgroup of four waves takes a 128 x 128 tile of C, each wave 64 x 64 as
// 2 x 2 blocks of v_mfma_f32_32x32x2_f32 (exact products, fp32 sums).  K
// moves 16 at a time through LDS ([k][m] and [k][n] rows of 160 floats: the
// two k rows a wave reads at once fall on different banks), the next slice
// held in registers while the current one is multiplied.  Interior slices of
// operands with a unit stride load 16 bytes a thread; edges and other
// strides load element by element, bounds-checked.  K may be split over
// parts (grid.y), each writing its fp32 sums to the launch's workspace, and a
// second kernel adds the parts (in part order) and D.

constexpr int kFT = 128;        // C tile
constexpr int kFK = 16;         // K per step
constexpr int kFRow = kFT + 32;  // LDS row (floats)

struct F32GemmArgs {
  const float* a;
  const float* b;
  float* c;        // the result, or the parts' workspace ([batch][part][m x n], ld m)
  const float* d;  // added to the product where non-null (not with parts)
  int64_t a_m, a_k, a_batch;
  int64_t b_k, b_n, b_batch;
  int64_t c_ld, c_batch, c_part;  // c_part: elements between parts (0 without parts)
  int64_t d_ld, d_batch;
  int32_t m, n, k;
  int32_t ksplit;  // K per part, a multiple of kFK
  int32_t va, vb;  // 1: A (B) has a unit stride and 16-byte aligned rows along it
};

typedef float f32x16g __attribute__((ext_vector_type(16)));

// A's 128 x 16 slice at (m0, k0) into LDS As[k][m]: eight values a thread.
__device__ __forceinline__ void f32_load_a(const F32GemmArgs& p, const float* a, int m0, int k0, int kend,
                                           f32x4 (&r)[2]) {
  const int t = threadIdx.x;
  const bool full = m0 + kFT <= p.m && k0 + kFK <= kend;
  if (p.va && full) {
    if (p.a_m == 1) {  // along m: rows k0 + t / 32 and + 8
#pragma unroll
      for (int i = 0; i < 2; ++i)
        r[i] = *reinterpret_cast<const f32x4*>(a + (m0 + 4 * (t % 32)) + (int64_t)(k0 + t / 32 + 8 * i) * p.a_k);
    } else {  // along k: rows m0 + t / 4 and + 64
#pragma unroll
      for (int i = 0; i < 2; ++i)
        r[i] = *reinterpret_cast<const f32x4*>(a + (int64_t)(m0 + t / 4 + 64 * i) * p.a_m + k0 + 4 * (t % 4));
    }
    return;
  }
  const bool along_m = p.a_m <= p.a_k;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      int mm, kk;
      if (along_m) mm = 4 * (t % 32) + e, kk = t / 32 + 8 * i;
      else mm = t / 4 + 64 * i, kk = 4 * (t % 4) + e;
      const int m = m0 + mm, k = k0 + kk;
      r[i][e] = (m < p.m && k < kend) ? a[(int64_t)m * p.a_m + (int64_t)k * p.a_k] : 0.0f;
    }
}

__device__ __forceinline__ void f32_store_a(const F32GemmArgs& p, float* As, const f32x4 (&r)[2]) {
  const int t = threadIdx.x;
  // The layout f32_load_a used, on either of its paths: four m a thread when
  // m has the smaller stride (the vector path's a_m == 1), four k otherwise.
  const bool m_rows = p.a_m <= p.a_k;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    if (m_rows) {
      *reinterpret_cast<f32x4*>(As + (t / 32 + 8 * i) * kFRow + 4 * (t % 32)) = r[i];
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) As[(4 * (t % 4) + e) * kFRow + t / 4 + 64 * i] = r[i][e];
    }
  }
}

// B's 16 x 128 slice at (k0, n0) into LDS Bs[k][n].
__device__ __forceinline__ void f32_load_b(const F32GemmArgs& p, const float* b, int n0, int k0, int kend,
                                           f32x4 (&r)[2]) {
  const int t = threadIdx.x;
  const bool full = n0 + kFT <= p.n && k0 + kFK <= kend;
  if (p.vb && full) {
    if (p.b_n == 1) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
        r[i] = *reinterpret_cast<const f32x4*>(b + (n0 + 4 * (t % 32)) + (int64_t)(k0 + t / 32 + 8 * i) * p.b_k);
    } else {
#pragma unroll
      for (int i = 0; i < 2; ++i)
        r[i] = *reinterpret_cast<const f32x4*>(b + (int64_t)(n0 + t / 4 + 64 * i) * p.b_n + k0 + 4 * (t % 4));
    }
    return;
  }
  const bool along_n = p.b_n <= p.b_k;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      int nn, kk;
      if (along_n) nn = 4 * (t % 32) + e, kk = t / 32 + 8 * i;
      else nn = t / 4 + 64 * i, kk = 4 * (t % 4) + e;
      const int n = n0 + nn, k = k0 + kk;
      r[i][e] = (n < p.n && k < kend) ? b[(int64_t)k * p.b_k + (int64_t)n * p.b_n] : 0.0f;
    }
}

__device__ __forceinline__ void f32_store_b(const F32GemmArgs& p, float* Bs, const f32x4 (&r)[2]) {
  const int t = threadIdx.x;
  const bool n_rows = p.b_n <= p.b_k;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    if (n_rows) {
      *reinterpret_cast<f32x4*>(Bs + (t / 32 + 8 * i) * kFRow + 4 * (t % 32)) = r[i];
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) Bs[(4 * (t % 4) + e) * kFRow + t / 4 + 64 * i] = r[i][e];
    }
  }
}

__global__ __launch_bounds__(256, 2) void gemm_f32(F32GemmArgs p) {
  __shared__ __attribute__((aligned(16))) float As[2][kFK * kFRow];
  __shared__ __attribute__((aligned(16))) float Bs[2][kFK * kFRow];
  const int tiles_m = (p.m + kFT - 1) / kFT;
  const int m0 = (blockIdx.x % tiles_m) * kFT, n0 = (blockIdx.x / tiles_m) * kFT;
  const int part = blockIdx.y, z = blockIdx.z;
  const int kbeg = part * p.ksplit, kend = min(p.k, kbeg + p.ksplit);
  const float* a = p.a + z * p.a_batch;
  const float* b = p.b + z * p.b_batch;
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int wm = (wave / 2) * 64, wn = (wave % 2) * 64;
  f32x16g acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x16g{};
  f32x4 ra[2], rb[2];
  f32_load_a(p, a, m0, kbeg, kend, ra);
  f32_load_b(p, b, n0, kbeg, kend, rb);
  f32_store_a(p, As[0], ra);
  f32_store_b(p, Bs[0], rb);
  __syncthreads();
  const int steps = (kend - kbeg + kFK - 1) / kFK;
  for (int st = 0; st < steps; ++st) {
    const int cur = st & 1;
    const int kn = kbeg + (st + 1) * kFK;
    if (st + 1 < steps) {
      f32_load_a(p, a, m0, kn, kend, ra);
      f32_load_b(p, b, n0, kn, kend, rb);
    }
    // v_mfma_f32_32x32x2_f32: lane l gives A(row l % 32, k l / 32) and
    // B(k l / 32, column l % 32).
    const float* A = As[cur];
    const float* B = Bs[cur];
#pragma unroll
    for (int kk = 0; kk < kFK; kk += 2) {
      const int kr = kk + lane / 32;
      float av[2], bv[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) av[i] = A[kr * kFRow + wm + 32 * i + lane % 32];
#pragma unroll
      for (int j = 0; j < 2; ++j) bv[j] = B[kr * kFRow + wn + 32 * j + lane % 32];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i], bv[j], acc[i][j], 0, 0, 0);
    }
    if (st + 1 < steps) {
      f32_store_a(p, As[cur ^ 1], ra);
      f32_store_b(p, Bs[cur ^ 1], rb);
    }
    __syncthreads();
  }
  // Lane l holds C(rows 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32) of each block.
  float* c = p.c + z * p.c_batch + part * p.c_part;
  const float* d = p.d ? p.d + z * p.d_batch : nullptr;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = n0 + wn + 32 * j + lane % 32;
      if (n >= p.n) continue;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int mb = m0 + wm + 32 * i + 8 * q + 4 * (lane / 32);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int m = mb + e;
          if (m < p.m) {
            float v = acc[i][j][4 * q + e];
            if (d) v += d[(int64_t)m + (int64_t)n * p.d_ld];
            c[(int64_t)m + (int64_t)n * p.c_ld] = v;
          }
        }
      }
    }
}

// ---- fp32 factors, small products: 32 x 32 blocks ---------------------------------
// A product whose 128 x 128 tiles would leave most of the device idle, with
// K short enough not to need parts: a workgroup of four waves per 32 x 32
// block of C, wave w taking a quarter of K (in pairs) with
// v_mfma_f32_32x32x2_f32 on operands loaded from memory straight into
// registers, eight products' worth at a time (the operands of such a
// product sit in L2).  The three other waves' partial blocks go through LDS
// and wave 0 adds them in wave order, so the result does not depend on
// timing, then D, and stores.  Every load and store is bounds-checked.

constexpr int kSB = 32;  // C block
constexpr int kSU = 8;   // products per batch of loads

__global__ __launch_bounds__(256) void gemm_f32_small(F32GemmArgs p) {
  __shared__ float part[3][16 * 64];  // waves 1..3's blocks, [register][lane]
  const int tiles_m = (p.m + kSB - 1) / kSB;
  const int m0 = (blockIdx.x % tiles_m) * kSB, n0 = (blockIdx.x / tiles_m) * kSB;
  const int z = blockIdx.z;
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int pairs = (p.k + 1) / 2, per = (pairs + 3) / 4;
  const int kb = 2 * min(pairs, wave * per), ke = min(p.k, 2 * min(pairs, (wave + 1) * per));
  const int mi = m0 + lane % 32, nj = n0 + lane % 32, kh = lane / 32;
  const bool m_in = mi < p.m, n_in = nj < p.n;
  const float* ap = p.a + z * p.a_batch + (int64_t)(m_in ? mi : 0) * p.a_m;
  const float* bp = p.b + z * p.b_batch + (int64_t)(n_in ? nj : 0) * p.b_n;
  f32x16g acc = {};
  // Lane l gives A(row l % 32, k l / 32) and B(k l / 32, column l % 32); the
  // next batch's loads are issued before this batch's products.
  float ra[2][kSU], rb[2][kSU];
  auto load = [&](int k0, float (&xa)[kSU], float (&xb)[kSU]) {
#pragma unroll
    for (int u = 0; u < kSU; ++u) {
      const int k = k0 + 2 * u + kh;
      const bool k_in = k < ke;
      xa[u] = (m_in && k_in) ? ap[(int64_t)k * p.a_k] : 0.0f;
      xb[u] = (n_in && k_in) ? bp[(int64_t)k * p.b_k] : 0.0f;
    }
  };
  auto multiply = [&](const float (&xa)[kSU], const float (&xb)[kSU]) {
#pragma unroll
    for (int u = 0; u < kSU; ++u) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(xa[u], xb[u], acc, 0, 0, 0);
  };
  constexpr int kStep = 2 * kSU;
  if (kb < ke) load(kb, ra[0], rb[0]);
  for (int k0 = kb; k0 < ke; k0 += 2 * kStep) {
    if (k0 + kStep < ke) load(k0 + kStep, ra[1], rb[1]);
    multiply(ra[0], rb[0]);
    if (k0 + kStep >= ke) break;
    if (k0 + 2 * kStep < ke) load(k0 + 2 * kStep, ra[0], rb[0]);
    multiply(ra[1], rb[1]);
  }
  if (wave > 0) {
#pragma unroll
    for (int r = 0; r < 16; ++r) part[wave - 1][r * 64 + lane] = acc[r];
  }
  __syncthreads();
  if (wave > 0) return;
#pragma unroll
  for (int w = 0; w < 3; ++w)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] += part[w][r * 64 + lane];
  // Lane l holds C(rows 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32).
  if (!n_in) return;
  float* c = p.c + z * p.c_batch;
  const float* d = p.d ? p.d + z * p.d_batch : nullptr;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int m = m0 + 8 * (r / 4) + 4 * kh + r % 4;
    if (m < p.m) {
      float v = acc[r];
      if (d) v += d[(int64_t)m + (int64_t)nj * p.d_ld];
      c[(int64_t)m + (int64_t)nj * p.c_ld] = v;
    }
  }
}

// C_z = D_z + the parts' sums in part order (fp32).
struct F32SumArgs {
  const float* ws;  // [batch][parts][m x n], ld m
  float* c;
  const float* d;
  int64_t c_ld, c_batch, d_ld, d_batch;
  int32_t m, n, parts;
};

__global__ __launch_bounds__(256) void gemm_f32_sum_parts(F32SumArgs a) {
  const int64_t mn = (int64_t)a.m * a.n;
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= mn) return;
  const int64_t z = blockIdx.y;
  const int64_t i = e % a.m, j = e / a.m;
  float v = thd::sum_in_order(a.ws + z * a.parts * mn + e, mn, a.parts);
  if (a.d) v += a.d[z * a.d_batch + i + j * a.d_ld];
  a.c[z * a.c_batch + i + j * a.c_ld] = v;
}

int esize(int t) { return t == TH_F32 ? 4 : 2; }

}  // namespace

namespace th {

static int build_gemm_f32(const th_gemm_desc* d, th_launch** out);

int build_gemm_general(const th_gemm_desc* d, th_launch** out) {
  if ((d->flags & TH_GEMM_F32_FACTORS) && d->c_dtype == TH_F32 && d->epilogue == TH_EPI_STORE && !d->bias)
    return build_gemm_f32(d, out);
  TH_REQUIRE(d->splits <= 1, "th_build_gemm: the general kernel splits K for fp32 factors only");
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

// The parts of K an fp32 product takes when the caller leaves them: enough
// for about 256 workgroups where the tiles alone give fewer than 128, each
// part at least 32 deep (two steps: 256 x 256 x 8192 takes 64 parts, 256 x
// 512 x 384 twelve).
static int f32_splits(const th_gemm_desc* d) {
  const int64_t tiles = (int64_t)((d->m + kFT - 1) / kFT) * ((d->n + kFT - 1) / kFT) * std::max(1, d->batch);
  if (tiles >= 128 || d->k < 64) return 1;
  return (int)std::max<int64_t>(1, std::min<int64_t>((256 + tiles - 1) / tiles, d->k / 32));
}

static bool f32_vector(const void* base, int64_t unit_other, int64_t other, int64_t batch_stride, int n_batch) {
  return reinterpret_cast<uintptr_t>(base) % 16 == 0 && other % 4 == 0 && (n_batch <= 1 || batch_stride % 4 == 0) &&
         unit_other == 1;
}

static int build_gemm_f32_small(const th_gemm_desc* d, th_launch** out);

// Whether an fp32 product takes the 32 x 32 kernel: the parts left to the
// library, its 128 x 128 tiles fewer than 64 (a quarter of the device), K
// at most 2048 (a wave's quarter of it at most 512 deep).
static bool f32_small(const th_gemm_desc* d) {
  const int64_t tiles = (int64_t)((d->m + kFT - 1) / kFT) * ((d->n + kFT - 1) / kFT) * std::max(1, d->batch);
  return d->splits == 0 && tiles < 64 && d->k <= 2048;
}

static int build_gemm_f32(const th_gemm_desc* d, th_launch** out) {
  if (f32_small(d)) return build_gemm_f32_small(d, out);
  const int batch = d->batch > 0 ? d->batch : 1;
  const int64_t tiles = (int64_t)((d->m + kFT - 1) / kFT) * ((d->n + kFT - 1) / kFT);
  TH_REQUIRE(tiles <= 0x7fffffff && batch <= 65535, "th_build_gemm: grid too large");
  const bool acc = (d->flags & TH_GEMM_ACCUMULATE) != 0;
  int splits = d->splits > 0 ? d->splits : f32_splits(d);
  int ksplit = d->k;
  if (splits > 1) {
    ksplit = ((d->k + splits - 1) / splits + kFK - 1) / kFK * kFK;
    splits = (d->k + ksplit - 1) / ksplit;
  }
  TH_REQUIRE(splits <= 65535, "th_build_gemm: too many parts of K");
  const bool staged = splits > 1;
  F32GemmArgs a{};
  a.a = static_cast<const float*>(d->a), a.b = static_cast<const float*>(d->b);
  a.a_m = d->a_m, a.a_k = d->a_k, a.a_batch = d->a_batch;
  a.b_k = d->b_k, a.b_n = d->b_n, a.b_batch = d->b_batch;
  a.m = d->m, a.n = d->n, a.k = d->k, a.ksplit = ksplit;
  a.va = (d->a_m == 1 && f32_vector(d->a, 1, d->a_k, d->a_batch, batch)) ||
         (d->a_k == 1 && d->a_m != 1 && f32_vector(d->a, 1, d->a_m, d->a_batch, batch));
  a.vb = (d->b_n == 1 && f32_vector(d->b, 1, d->b_k, d->b_batch, batch)) ||
         (d->b_k == 1 && d->b_n != 1 && f32_vector(d->b, 1, d->b_n, d->b_batch, batch));
  th::Builder b("gemm_f32", 9);
  uint64_t at_parts = 0;
  const int64_t mn = (int64_t)d->m * d->n;
  if (staged) {
    at_parts = b.workspace((uint64_t)batch * splits * mn * sizeof(float));
    a.c = nullptr, a.c_ld = d->m, a.c_batch = (int64_t)splits * mn, a.c_part = mn, a.d = nullptr;
  } else {
    a.c = static_cast<float*>(d->c), a.c_ld = d->c_ld, a.c_batch = d->c_batch, a.c_part = 0;
    a.d = acc ? static_cast<const float*>(d->d) : nullptr;
    a.d_ld = d->d_ld ? d->d_ld : d->c_ld, a.d_batch = d->d_ld ? d->d_batch : d->c_batch;
  }
  int k = b.kernel((const void*)gemm_f32, "gemm_f32_128x128", dim3((unsigned)tiles, splits, batch), dim3(256), 0, a);
  b.ref(0, k, TH_OFFSET(F32GemmArgs, a));
  b.ref(1, k, TH_OFFSET(F32GemmArgs, b));
  if (staged) {
    b.ws_ref(k, TH_OFFSET(F32GemmArgs, c), at_parts);
    F32SumArgs r{nullptr, static_cast<float*>(d->c), acc ? static_cast<const float*>(d->d) : nullptr, d->c_ld,
                 d->c_batch, d->d_ld ? d->d_ld : d->c_ld, d->d_ld ? d->d_batch : d->c_batch, d->m, d->n, splits};
    int kr = b.kernel((const void*)gemm_f32_sum_parts, "gemm_f32_sum_parts", dim3((unsigned)((mn + 255) / 256), batch),
                      dim3(256), 0, r);
    b.ws_ref(kr, TH_OFFSET(F32SumArgs, ws), at_parts);
    b.ref(2, kr, TH_OFFSET(F32SumArgs, c));
    b.ref(8, kr, TH_OFFSET(F32SumArgs, d));
  } else {
    b.ref(2, k, TH_OFFSET(F32GemmArgs, c));
    b.ref(8, k, TH_OFFSET(F32GemmArgs, d));
  }
  // The vector loads assume the operands stay 16-byte aligned.
  if (a.va) b.align(0, 16);
  if (a.vb) b.align(1, 16);
  const double mm = d->m, nn = d->n, kk = d->k, bb = batch;
  b.work(bb * (4.0 * (mm * kk + kk * nn) + 4.0 * mm * nn * (acc ? 2 : 1)), 2.0 * bb * mm * nn * kk,
         tiles * splits * batch);
  *out = b.release();
  return TH_OK;
}

static int build_gemm_f32_small(const th_gemm_desc* d, th_launch** out) {
  const int batch = d->batch > 0 ? d->batch : 1;
  const int64_t blocks = (int64_t)((d->m + kSB - 1) / kSB) * ((d->n + kSB - 1) / kSB);
  TH_REQUIRE(blocks <= 0x7fffffff && batch <= 65535, "th_build_gemm: grid too large");
  const bool acc = (d->flags & TH_GEMM_ACCUMULATE) != 0;
  TH_REQUIRE(!acc || d->d, "th_build_gemm: accumulating needs d");
  F32GemmArgs a{};
  a.a = static_cast<const float*>(d->a), a.b = static_cast<const float*>(d->b);
  a.a_m = d->a_m, a.a_k = d->a_k, a.a_batch = d->a_batch;
  a.b_k = d->b_k, a.b_n = d->b_n, a.b_batch = d->b_batch;
  a.m = d->m, a.n = d->n, a.k = d->k, a.ksplit = d->k;
  a.c = static_cast<float*>(d->c), a.c_ld = d->c_ld, a.c_batch = d->c_batch, a.c_part = 0;
  a.d = acc ? static_cast<const float*>(d->d) : nullptr;
  a.d_ld = d->d_ld ? d->d_ld : d->c_ld, a.d_batch = d->d_ld ? d->d_batch : d->c_batch;
  th::Builder b("gemm_f32", 9);
  int k = b.kernel((const void*)gemm_f32_small, "gemm_f32_32x32", dim3((unsigned)blocks, 1, batch), dim3(256), 0, a);
  b.ref(0, k, TH_OFFSET(F32GemmArgs, a));
  b.ref(1, k, TH_OFFSET(F32GemmArgs, b));
  b.ref(2, k, TH_OFFSET(F32GemmArgs, c));
  b.ref(8, k, TH_OFFSET(F32GemmArgs, d));
  const double mm = d->m, nn = d->n, kk = d->k, bb = batch;
  b.work(bb * (4.0 * (mm * kk + kk * nn) + 4.0 * mm * nn * (acc ? 2 : 1)), 2.0 * bb * mm * nn * kk, blocks * batch);
  *out = b.release();
  return TH_OK;
}

}  // namespace th
