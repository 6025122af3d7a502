// Config 5: chunked gated DeltaNet, forward and gradient (rows a16: the
// reference's scan and recurrence kernels, ext/cuTileExt/build.jl:715-839,
// codegen/scalar.jl:354-440, runtime/stepped.jl, for the program of
// examples/deltanet.jl:58-86).
//
// Per position t of a (batch, head) sequence, S (dk x dv) follows
//   S = exp(a_t) (I - beta_t k_t k_t') S + beta_t k_t v_t',  o_t = S' q_t.
// In chunks of 64 positions (ca = cumsum(a) within the chunk,
// Gamma_ij = exp(ca_i - ca_j)):
//   A = strict lower (beta_i Gamma_ij k_i.k_j),  T = (I + A)^-1,
//   W = T diag(beta e^ca) K,  U~ = T diag(beta) V,
//   P = lower (Gamma_ij q_i.k_j),  Qg = diag(e^ca) Q,  Kd = diag(e^(ca_63 - ca)) K,  g = e^ca_63;
// across chunks:  U = U~ - W S,  O = Qg S + P U,  S <- g S + Kd' U.
//
// Kernels (fp32 arithmetic, every product on the bf16 matrix cores with each
// fp32 operand split into two bf16 halves; inputs bf16 q, k, v and fp32 a, beta):
//   dn_chunk_prep   one workgroup per chunk: ca, A, T (forward substitution,
//                   one lane per column), W, U~.
//   dn_state_scan   one eight-wave workgroup per (sequence, 32 columns of S):
//                   the sequential recurrence, each column block independent;
//                   stores each chunk's starting state and U.
//   dn_output       one workgroup per chunk: P, O.
//   dn_state_grad   one eight-wave workgroup per (sequence, 32 columns): the state
//                   gradient swept back over chunks; stores dU and dS_{n+1}.
//   dn_grad_a/b     one workgroup per chunk: the chunk's products' gradients,
//                   the inverse's (dA = -T' dT T'), the decays', a's.
#include <hip/hip_runtime.h>

#include <cmath>

#include "th_core.h"

namespace {

constexpr int kC = 64;    // chunk
constexpr int kD = 128;   // dk = dv
constexpr int kCols = 32; // columns of S per scan workgroup

struct DnArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const float* a;
  const float* beta;
  uint16_t* o;
  const uint16_t* dout;
  uint16_t* dq;
  uint16_t* dk;
  uint16_t* dv;
  float* da;
  float* dbeta;
  // workspace, per chunk c = (b * heads + h) * chunks + n
  float* ca;    // [c][64]
  float* T;     // [c][64][64]
  float* W;     // [c][64][128]
  float* Ut;    // [c][64][128]
  float* S;     // [c][128][128] state at the chunk's start
  float* U;     // [c][64][128]
  float* P;     // [c][64][64]
  float* dU;    // [c][64][128]
  float* dSn;   // [c][128][128] gradient w.r.t. the chunk's end state
  float* dQg;   // [c][64][128]
  float* dW;    // [c][64][128]
  float* dKd;   // [c][64][128]
  float* dP;    // [c][64][64]
  float* dg;    // [c][kDgParts]: <S, dSn> by (column slice, wave) of the state gradient
  int64_t s_h, s_t, s_b;  // strides (elements) of q, k, v, o, dout, dq, dk, dv along head, position, batch
  int64_t g_h, g_t, g_b;  // strides of a, beta, da, dbeta
  int32_t batch, heads, seq, chunks;
};

__device__ __forceinline__ float bf(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }
__device__ __forceinline__ uint16_t to_bf(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

struct Chunk {
  int b, h, n;
  int64_t c;       // chunk number
  int64_t row0;    // element offset of position n*64, head h, batch b
  int64_t grow0;   // the same for the gate arrays
};

__device__ __forceinline__ Chunk chunk_of(const DnArgs& p, int64_t c) {
  Chunk k;
  k.c = c;
  k.n = (int)(c % p.chunks);
  const int64_t bh = c / p.chunks;
  k.h = (int)(bh % p.heads);
  k.b = (int)(bh / p.heads);
  k.row0 = k.b * p.s_b + k.h * p.s_h + (int64_t)k.n * kC * p.s_t;
  k.grow0 = k.b * p.g_b + k.h * p.g_h + (int64_t)k.n * kC * p.g_t;
  return k;
}

// ca = inclusive cumulative sum of a over the chunk (wave 0), into LDS.
__device__ __forceinline__ void cumulative_gates(float* ca, const DnArgs& p, const Chunk& ck) {
  if (threadIdx.x < 64) {
    float x = p.a[ck.grow0 + (int64_t)threadIdx.x * p.g_t];
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const float y = __shfl_up(x, o, 64);
      if ((int)threadIdx.x >= o) x += y;
    }
    ca[threadIdx.x] = x;
  }
}

// ---- fp32 products on the bf16 matrix cores -----------------------------------------
// Each fp32 operand x is split as hi = bf16(x), lo = bf16(x - hi); a b is
// summed in fp32 as hi hi + hi lo + lo hi on v_mfma_f32_16x16x32_bf16 (the
// lo lo term and lo's rounding leave about 2^-16 of each product; operands
// that are bf16 values, Q K V, have no lo).  The three bf16 products of 32 k
// take 48 matrix-core cycles, the eight fp32 ones (v_mfma_f32_16x16x4_f32)
// for the same k would take 256.
// Operands sit in LDS as fp32 rows of kLd floats: a row's 16-byte quads land
// on distinct bank quads for 16 consecutive rows (kLd / 4 odd), and a column
// read by 16 consecutive rows x 4 row groups hits 64 distinct banks
// (kLd = 4 mod 16).
//
// Lane l = 16 g + r of a 16 x 16 block over 32 consecutive k takes the eight
// k = kb + 8 g + (0..7): two quads per operand when k runs along its rows,
// split to bf16, each pairing A(i0 + r, k) with B(k, j0 + r); the products'
// k slot g then holds the same k in both operands.  The block
// C(i0 + 4 g + v, j0 + r) sits in register v of lane l.

typedef float f32x4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
constexpr int kLd = 132;   // LDS row of 128 fp32
constexpr int kLdC = 68;   // LDS row of 64 fp32
constexpr int kLdS = 36;   // LDS row of 32 fp32

__device__ __forceinline__ f32x4v quad(const float* row) { return *reinterpret_cast<const f32x4v*>(row); }

// The four k of lane g's quad along a column: X(k, c) at x[k * ld + c].
__device__ __forceinline__ f32x4v column_quad(const float* x, int ld, int k0, int c) {
  return f32x4v{x[k0 * ld + c], x[(k0 + 1) * ld + c], x[(k0 + 2) * ld + c], x[(k0 + 3) * ld + c]};
}

typedef __bf16 bf16x8v __attribute__((ext_vector_type(8)));
typedef float f32x2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));

// Two fp32 as a pair of bf16 (nearest even), a in the low half.
__device__ __forceinline__ uint32_t pk2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2v{a, b}, bf16x2v));
}

// A product operand's eight k (two quads of one row) as bf16 halves: hi the
// nearest bf16, lo the nearest bf16 to the remainder x - hi (exact in fp32),
// so hi + lo holds x to about 2^-16 of it.  kExact: x is a bf16 value, lo is 0.
struct Split8 {
  bf16x8v hi, lo;
};
template <bool kExact>
__device__ __forceinline__ Split8 split8(f32x4v q0, f32x4v q1) {
  const float x[8] = {q0[0], q0[1], q0[2], q0[3], q1[0], q1[1], q1[2], q1[3]};
  u32x4v h, l = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int e = 0; e < 4; ++e) h[e] = pk2(x[2 * e], x[2 * e + 1]);
  if constexpr (!kExact) {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      l[e] = pk2(x[2 * e] - __uint_as_float(h[e] << 16), x[2 * e + 1] - __uint_as_float(h[e] & 0xffff0000u));
  }
  return Split8{__builtin_bit_cast(bf16x8v, h), __builtin_bit_cast(bf16x8v, l)};
}

// c += a b over 32 k on the bf16 matrix cores (v_mfma_f32_16x16x32_bf16,
// fp32 sums): hi hi + hi lo + lo hi, the lo lo term (about 2^-16 of the
// product) dropped, and the terms of an operand exact in bf16 skipped.
template <bool kExactA, bool kExactB>
__device__ __forceinline__ f32x4v mma_split(const Split8& a, const Split8& b, f32x4v c) {
  if constexpr (!kExactB) c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.hi, b.lo, c, 0, 0, 0);
  if constexpr (!kExactA) c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.lo, b.hi, c, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.hi, b.hi, c, 0, 0, 0);
}

// acc[bi][bj] += X(i0 + 16 bi .., k) Y(j0 + 16 bj .., k) over k in [0, K):
// both operands with k along their rows (row-major in LDS, stride kLd);
// kExactX: X's fp32 values are bf16 values (no lo part).
template <int BI, int BJ, bool kExactX = false>
__device__ __forceinline__ void mm_nt(f32x4v (&acc)[BI][BJ], const float* X, int i0, const float* Y, int j0, int K) {
  const int r = threadIdx.x % 16, g = (threadIdx.x % 64) / 16;
  for (int kb = 0; kb < K; kb += 32) {
    Split8 a[BI], b[BJ];
#pragma unroll
    for (int bi = 0; bi < BI; ++bi) {
      const float* row = X + (i0 + 16 * bi + r) * kLd + kb + 8 * g;
      a[bi] = split8<kExactX>(quad(row), quad(row + 4));
    }
#pragma unroll
    for (int bj = 0; bj < BJ; ++bj) {
      const float* row = Y + (j0 + 16 * bj + r) * kLd + kb + 8 * g;
      b[bj] = split8<false>(quad(row), quad(row + 4));
    }
#pragma unroll
    for (int bi = 0; bi < BI; ++bi)
#pragma unroll
      for (int bj = 0; bj < BJ; ++bj) acc[bi][bj] = mma_split<kExactX, false>(a[bi], b[bj], acc[bi][bj]);
  }
}

// acc[bi][bj] += X(i0 + 16 bi .., k) Y(k, j0 + 16 bj ..) over k in [0, K), each
// operand read along its rows (X(i, k) = X[i * ldx + k], Y(k, j) = Y[j * ldy + k])
// or, when XT / YT, along its columns (X(i, k) = X[k * ldx + i], Y(k, j) =
// Y[k * ldy + j]).  Strides satisfy ld / 4 odd and ld = 4 mod 16.
template <bool XT, bool YT, int BI, int BJ>
__device__ __forceinline__ void mm_gen(f32x4v (&acc)[BI][BJ], const float* X, int ldx, int i0, const float* Y, int ldy,
                                       int j0, int K) {
  const int r = threadIdx.x % 16, g = (threadIdx.x % 64) / 16;
  auto xq = [&](int k0, int i) { return XT ? column_quad(X, ldx, k0, i) : quad(X + i * ldx + k0); };
  auto yq = [&](int k0, int j) { return YT ? column_quad(Y, ldy, k0, j) : quad(Y + j * ldy + k0); };
  for (int kb = 0; kb < K; kb += 32) {
    const int k0 = kb + 8 * g;
    Split8 a[BI], b[BJ];
#pragma unroll
    for (int bi = 0; bi < BI; ++bi) a[bi] = split8<false>(xq(k0, i0 + 16 * bi + r), xq(k0 + 4, i0 + 16 * bi + r));
#pragma unroll
    for (int bj = 0; bj < BJ; ++bj) b[bj] = split8<false>(yq(k0, j0 + 16 * bj + r), yq(k0 + 4, j0 + 16 * bj + r));
#pragma unroll
    for (int bi = 0; bi < BI; ++bi)
#pragma unroll
      for (int bj = 0; bj < BJ; ++bj) acc[bi][bj] = mma_split<false, false>(a[bi], b[bj], acc[bi][bj]);
  }
}

template <int BI, int BJ>
__device__ __forceinline__ void clear(f32x4v (&acc)[BI][BJ]) {
#pragma unroll
  for (int bi = 0; bi < BI; ++bi)
#pragma unroll
    for (int bj = 0; bj < BJ; ++bj) acc[bi][bj] = f32x4v{0.0f, 0.0f, 0.0f, 0.0f};
}

// rows x 128 fp32 from global (row stride 128) into LDS rows of kLd, 16-byte pieces.
// Each staging helper issues all of a thread's loads before its first LDS
// store, so their latencies overlap instead of adding up.
__device__ __forceinline__ void stage_f32(float* dst, const float* src) {
  constexpr int n = kC * 32 / 256;
  float4 x[n];
#pragma unroll
  for (int u = 0; u < n; ++u) {
    const int e = threadIdx.x + 256 * u;
    x[u] = *reinterpret_cast<const float4*>(src + (e / 32) * kD + 4 * (e % 32));
  }
#pragma unroll
  for (int u = 0; u < n; ++u) {
    const int e = threadIdx.x + 256 * u;
    *reinterpret_cast<float4*>(dst + (e / 32) * kLd + 4 * (e % 32)) = x[u];
  }
}

// 64 x 128 bf16 of a (d, heads, positions, batch) array into LDS as fp32 rows of kLd.
__device__ __forceinline__ void stage_bf16(float* dst, const uint16_t* src, int64_t s_t) {
  constexpr int n = kC * 16 / 256;
  uint4 x[n];
#pragma unroll
  for (int q = 0; q < n; ++q) {
    const int e = threadIdx.x + 256 * q;
    x[q] = *reinterpret_cast<const uint4*>(src + (e / 16) * s_t + 8 * (e % 16));
  }
#pragma unroll
  for (int q = 0; q < n; ++q) {
    const int e = threadIdx.x + 256 * q;
    const int r = e / 16, c8 = 8 * (e % 16);
    const uint4 w = x[q];
    const uint32_t u[4] = {w.x, w.y, w.z, w.w};
    float f[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) f[2 * j] = bf((uint16_t)u[j]), f[2 * j + 1] = bf((uint16_t)(u[j] >> 16));
    *reinterpret_cast<float4*>(dst + r * kLd + c8) = make_float4(f[0], f[1], f[2], f[3]);
    *reinterpret_cast<float4*>(dst + r * kLd + c8 + 4) = make_float4(f[4], f[5], f[6], f[7]);
  }
}

// Block (bi, bj) of acc to out (row stride ld), rows i0 + 16 bi + 4 g + v, columns j0 + 16 bj + r, times s.
template <int BI, int BJ>
__device__ __forceinline__ void store_blocks(float* out, int ld, const f32x4v (&acc)[BI][BJ], int i0, int j0, float s) {
  const int r = threadIdx.x % 16, g = (threadIdx.x % 64) / 16;
#pragma unroll
  for (int bi = 0; bi < BI; ++bi)
#pragma unroll
    for (int bj = 0; bj < BJ; ++bj)
#pragma unroll
      for (int v = 0; v < 4; ++v) out[(int64_t)(i0 + 16 * bi + 4 * g + v) * ld + j0 + 16 * bj + r] = s * acc[bi][bj][v];
}

// Operand readers for mm_by: quad(x, k) is this lane's (x, k .. k + 3).
struct RowF32 {  // (x, k) at p[x * ld + k]
  static constexpr bool kExact = false;
  const float* p;
  int ld;
  __device__ f32x4v quad(int x, int k) const { return *reinterpret_cast<const f32x4v*>(p + x * ld + k); }
};
struct ColF32 {  // (x, k) at p[k * ld + x]
  static constexpr bool kExact = false;
  const float* p;
  int ld;
  __device__ f32x4v quad(int x, int k) const { return column_quad(p, ld, k, x); }
};
struct RowF32Bf {  // (x, k) at p[x * ld + k], fp32 holding bf16 values
  static constexpr bool kExact = true;
  const float* p;
  int ld;
  __device__ f32x4v quad(int x, int k) const { return *reinterpret_cast<const f32x4v*>(p + x * ld + k); }
};
struct ColF32Bf {  // (x, k) at p[k * ld + x], fp32 holding bf16 values
  static constexpr bool kExact = true;
  const float* p;
  int ld;
  __device__ f32x4v quad(int x, int k) const { return column_quad(p, ld, k, x); }
};
struct RowBf16 {  // (x, k) at bf16 p[x * ld + k]
  static constexpr bool kExact = true;
  const uint16_t* p;
  int64_t ld;
  __device__ f32x4v quad(int x, int k) const {
    const uint2 w = *reinterpret_cast<const uint2*>(p + x * ld + k);
    return f32x4v{bf((uint16_t)w.x), bf((uint16_t)(w.x >> 16)), bf((uint16_t)w.y), bf((uint16_t)(w.y >> 16))};
  }
};
struct ColBf16 {  // (x, k) at bf16 p[k * ld + x]
  static constexpr bool kExact = true;
  const uint16_t* p;
  int ld;
  __device__ f32x4v quad(int x, int k) const {
    return f32x4v{bf(p[k * ld + x]), bf(p[(k + 1) * ld + x]), bf(p[(k + 2) * ld + x]), bf(p[(k + 3) * ld + x])};
  }
};

// acc[bi][bj] += X(i0 + 16 bi .., k) Y(k, j0 + 16 bj ..) over k in [0, K).
template <int BI, int BJ, class XR, class YR>
__device__ __forceinline__ void mm_by(f32x4v (&acc)[BI][BJ], const XR& X, int i0, const YR& Y, int j0, int K) {
  const int r = threadIdx.x % 16, g = (threadIdx.x % 64) / 16;
  for (int kb = 0; kb < K; kb += 32) {
    const int k0 = kb + 8 * g;
    Split8 b[BJ];
#pragma unroll
    for (int bj = 0; bj < BJ; ++bj)
      b[bj] = split8<YR::kExact>(Y.quad(j0 + 16 * bj + r, k0), Y.quad(j0 + 16 * bj + r, k0 + 4));
    // The rows of X one block at a time: only one of its split blocks live.
#pragma unroll
    for (int bi = 0; bi < BI; ++bi) {
      const Split8 a = split8<XR::kExact>(X.quad(i0 + 16 * bi + r, k0), X.quad(i0 + 16 * bi + r, k0 + 4));
#pragma unroll
      for (int bj = 0; bj < BJ; ++bj) acc[bi][bj] = mma_split<XR::kExact, YR::kExact>(a, b[bj], acc[bi][bj]);
    }
  }
}

// Sum over the 16 lanes of a row group (lanes 16 g .. 16 g + 15), a fixed tree.
__device__ __forceinline__ float row_group_sum(float x) {
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) x += __shfl_xor(x, o, 64);
  return x;
}

constexpr int kLdH = kD + 8;  // bf16 LDS row of Q, K

// ---- forward: the chunk's WY form -------------------------------------------------
// ca, A = strict lower (beta_i Gamma_ij k_i.k_j), T = (I + A)^-1 (forward
// substitution, one lane per column), W = T diag(beta e^ca) K and
// U~ = T diag(beta) V; the products on the matrix cores (split bf16), K and V in
// LDS as bf16.

// Two 64 x 128 bf16 arrays of rows at s_t into LDS rows of kLdH, every load
// issued before the first store.
__device__ __forceinline__ void stage_rows_bf16(uint16_t* dst1, const uint16_t* src1, uint16_t* dst2,
                                                const uint16_t* src2, int64_t s_t) {
  constexpr int n = kC * (kD / 8) / 256;
  uint4 x1[n], x2[n];
#pragma unroll
  for (int u = 0; u < n; ++u) {
    const int e = threadIdx.x + 256 * u, row = e / (kD / 8), c8 = (e % (kD / 8)) * 8;
    x1[u] = *reinterpret_cast<const uint4*>(src1 + row * s_t + c8);
    x2[u] = *reinterpret_cast<const uint4*>(src2 + row * s_t + c8);
  }
#pragma unroll
  for (int u = 0; u < n; ++u) {
    const int e = threadIdx.x + 256 * u, row = e / (kD / 8), c8 = (e % (kD / 8)) * 8;
    *reinterpret_cast<uint4*>(dst1 + row * kLdH + c8) = x1[u];
    *reinterpret_cast<uint4*>(dst2 + row * kLdH + c8) = x2[u];
  }
}

// Under 80 KB, so two workgroups share a CU (one's substitution beside the
// other's loads and products).
constexpr size_t kPrepLds = 2 * kC * kLdH * sizeof(uint16_t) + (2 * kC * kLdC + 2 * kC) * sizeof(float);

__global__ __launch_bounds__(256, 2) void dn_chunk_prep(DnArgs p) {
  extern __shared__ float lds[];
  uint16_t* Kh = reinterpret_cast<uint16_t*>(lds);       // [64][kLdH]
  uint16_t* Vh = Kh + kC * kLdH;                          // [64][kLdH]
  float* AT = reinterpret_cast<float*>(Vh + kC * kLdH);   // [64][kLdC]: A, then T, then T diag(beta)
  float* TX = AT + kC * kLdC;     // [64][kLdC]: T diag(beta e^ca)
  float* TY = AT;                 // each entry rewritten by the thread that read it
  float* ca = TX + kC * kLdC;     // [64]
  float* be = ca + kC;            // [64]
  const Chunk ck = chunk_of(p, blockIdx.x);
  const int t = threadIdx.x, w = t / 64;
  const int r = t % 16, g = (t % 64) / 16;
  stage_rows_bf16(Kh, p.k + ck.row0, Vh, p.v + ck.row0, p.s_t);
  cumulative_gates(ca, p, ck);
  if (t < 64) be[t] = p.beta[ck.grow0 + (int64_t)t * p.g_t];
  __syncthreads();
  if (t < 64) p.ca[ck.c * kC + t] = ca[t];
  // A (64 x 64): wave w takes row block w, blocks at or left of the diagonal.
  {
    const RowBf16 Kr{Kh, kLdH};
    for (int bj = 0; bj < 4; ++bj) {
      f32x4v acc[1][1];
      clear(acc);
      if (bj <= w) mm_by(acc, Kr, 16 * w, Kr, 16 * bj, kD);
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int i = 16 * w + 4 * g + v, j = 16 * bj + r;
        AT[i * kLdC + j] = i > j ? be[i] * expf(ca[i] - ca[j]) * acc[0][0][v] : 0.0f;
      }
    }
  }
  __syncthreads();
  // T = (I + A)^-1 by forward substitution: T_ij = -sum_{l<i} A_il T_lj for
  // i > j, T_jj = 1.  Column j = 16 w + (lane / 4) belongs to the four lanes
  // q = lane mod 4 of a quad of wave w: lane q sums the terms l = 4 m + q
  // and keeps T_lj for those l (c[m]), the quad adds its four partial sums
  // ((q0 + q1) + (q2 + q3) in every lane), so all four waves share the
  // 2080 fmas of the sweep.  A_il is 0 for l >= i, so the terms of rows not
  // yet solved (c[m] still 0) add nothing.
  {
    const int q = t % 4, j = 16 * w + (t % 64) / 4;
    float c[kC / 4];
#pragma unroll
    for (int m = 0; m < kC / 4; ++m) c[m] = 0.0f;
#pragma unroll
    for (int i = 0; i < kC; ++i) {
      float part = 0.0f;
#pragma unroll
      for (int m = 0; m < (i + 3) / 4; ++m) part = fmaf(AT[i * kLdC + 4 * m + q], c[m], part);
      part += __shfl_xor(part, 1, 64);
      part += __shfl_xor(part, 2, 64);
      const float ti = i == j ? 1.0f : (i < j ? 0.0f : -part);
      if (q == i % 4) c[i / 4] = ti;
    }
    __syncthreads();  // every wave's reads of A precede the writes of T
#pragma unroll
    for (int m = 0; m < kC / 4; ++m) AT[(4 * m + q) * kLdC + j] = c[m];
  }
  __syncthreads();
  {
    float* Tc = p.T + ck.c * kC * kC;
    for (int e = t; e < kC * kC; e += 256) {
      const int i = e / kC, l = e % kC;
      const float tv = AT[i * kLdC + l];
      Tc[e] = tv;
      TX[i * kLdC + l] = tv * be[l] * expf(ca[l]);
      TY[i * kLdC + l] = tv * be[l];
    }
  }
  __syncthreads();
  // W = TX K, U~ = TY V (64 x 128): wave w takes columns 32 w .. 32 w + 31.
  {
    f32x4v wk[4][2], uv[4][2];
    clear(wk);
    clear(uv);
    mm_by(wk, RowF32{TX, kLdC}, 0, ColBf16{Kh, kLdH}, 32 * w, kC);
    mm_by(uv, RowF32{TY, kLdC}, 0, ColBf16{Vh, kLdH}, 32 * w, kC);
    store_blocks(p.W + ck.c * kC * kD, kD, wk, 0, 32 * w, 1.0f);
    store_blocks(p.Ut + ck.c * kC * kD, kD, uv, 0, 32 * w, 1.0f);
  }
}

// ---- forward: the recurrence across chunks, 32 columns of S per workgroup ---------
// Per chunk: the starting state is stored, U = U~ - W S, S <- g S + Kd' U,
// the products on the matrix cores (split bf16).  While a chunk's products run,
// the next chunk's W, U~ columns, K and ca are loaded into registers.

// Eight waves, two on each SIMD: one workgroup per CU (its LDS), and a
// chunk's serial chain (stage, product, product, update) split eight ways.
constexpr int kScanThreads = 512;
// dg = <S, dSn> of a chunk in partial sums, one per wave of each column
// slice's state-gradient workgroup, folded in a fixed order by their reader.
constexpr int kDgParts = (kD / kCols) * (kScanThreads / 64);

struct ScanInputs {  // one chunk's inputs as this thread loads them
  f32x4v w[4];       // W: 4 x 16 bytes
  f32x4v u;          // U~ columns col0 .. col0 + 31: 16 bytes
  u32x4v k[2];       // K: 2 x 16 bytes (bf16)
  float ca;
};

__device__ __forceinline__ void scan_load(ScanInputs& in, const DnArgs& p, const Chunk& ck, int col0) {
  const int t = threadIdx.x;
  const float* Wc = p.W + ck.c * kC * kD;
  const float* Uc = p.Ut + ck.c * kC * kD;
#pragma unroll
  for (int e = 0; e < 4; ++e) in.w[e] = reinterpret_cast<const f32x4v*>(Wc)[t + kScanThreads * e];
  {
    const int r = t / 8, c = 4 * (t % 8);
    in.u = *reinterpret_cast<const f32x4v*>(Uc + r * kD + col0 + c);
  }
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int x = t + kScanThreads * e, r = x / 16, c = 8 * (x % 16);
    in.k[e] = *reinterpret_cast<const u32x4v*>(p.k + ck.row0 + (int64_t)r * p.s_t + c);
  }
  in.ca = t < kC ? p.ca[ck.c * kC + t] : 0.0f;
}

// The inputs to LDS; K as Kd = diag(e^(ca_63 - ca)) K (ca of the same chunk, already in LDS).
__device__ __forceinline__ void scan_store(const ScanInputs& in, float* W, float* Ut, float* Kd, const float* ca) {
  const int t = threadIdx.x;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int x = t + kScanThreads * e, r = x / 32, c = 4 * (x % 32);
    *reinterpret_cast<f32x4v*>(W + r * kLd + c) = in.w[e];
  }
  *reinterpret_cast<f32x4v*>(Ut + (t / 8) * kLdS + 4 * (t % 8)) = in.u;
  const float last = ca[kC - 1];
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int x = t + kScanThreads * e, r = x / 16, c = 8 * (x % 16);
    const float ed = expf(last - ca[r]);
    const u32x4v uk = in.k[e];
#pragma unroll
    for (int h = 0; h < 2; ++h)
      *reinterpret_cast<f32x4v*>(Kd + r * kLd + c + 4 * h) =
          f32x4v{ed * bf((uint16_t)uk[2 * h]), ed * bf((uint16_t)(uk[2 * h] >> 16)), ed * bf((uint16_t)uk[2 * h + 1]),
                 ed * bf((uint16_t)(uk[2 * h + 1] >> 16))};
  }
}

// Scan workgroup b -> (sequence, first column of its slice of S).  The chip
// hands workgroups to its 8 XCDs in turn (b mod 8), each XCD with its own L2;
// the slices of one sequence read the same chunk inputs (W, K, Q, P), so they
// go to one XCD, whose L2 then serves all but the first read: slice j of
// sequence s is workgroup 32 (s / 8) + 8 j + s mod 8 for the sequences in
// whole groups of eight, the rest in order after them.
struct ScanSlot {
  int64_t seq;
  int col0;
};
__device__ __forceinline__ ScanSlot scan_slot() {
  constexpr int kSlices = kD / kCols;
  const int b = blockIdx.x, nseq = gridDim.x / kSlices, whole = nseq / 8 * 8;
  if (b < whole * kSlices) {
    const int q = b / 8;
    return ScanSlot{(int64_t)(q / kSlices) * 8 + b % 8, (q % kSlices) * kCols};
  }
  const int x = b - whole * kSlices;
  return ScanSlot{(int64_t)whole + x / kSlices, (x % kSlices) * kCols};
}

constexpr size_t kScanLds = (2 * kC * kLd + kC * kLdS + kD * kLdS + kC * kLdS + kC) * sizeof(float);

__global__ __launch_bounds__(kScanThreads, 1) void dn_state_scan(DnArgs p) {
  extern __shared__ float lds[];
  float* W = lds;                 // [64][kLd]
  float* Kd = W + kC * kLd;       // [64][kLd]: diag(e^(ca_63 - ca)) K
  float* Ut = Kd + kC * kLd;      // [64][kLdS]: U~ columns col0 .. col0 + 31
  float* S = Ut + kC * kLdS;      // [128][kLdS]: the state's 32 columns
  float* U = S + kD * kLdS;       // [64][kLdS]
  float* ca = U + kC * kLdS;      // [64]
  const int t = threadIdx.x, w = t / 64;
  const int r = t % 16, g = (t % 64) / 16;
  const ScanSlot slot = scan_slot();
  const int64_t seq = slot.seq;
  const int col0 = slot.col0;
  for (int e = t; e < kD * kLdS; e += kScanThreads) S[e] = 0.0f;
  ScanInputs in;
  scan_load(in, p, chunk_of(p, seq * p.chunks), col0);
  if (t < kC) ca[t] = in.ca;
  __syncthreads();
  scan_store(in, W, Ut, Kd, ca);
  for (int n = 0; n < p.chunks; ++n) {
    const Chunk ck = chunk_of(p, seq * p.chunks + n);
    __syncthreads();
    if (n + 1 < p.chunks) scan_load(in, p, chunk_of(p, seq * p.chunks + n + 1), col0);
    const float gl = expf(ca[kC - 1]);
    // The chunk's starting state, stored for the output and the backward: read
    // now, written to memory at the chunk's end (and U with it), after the
    // next chunk's inputs are in LDS, whose wait for their loads would also
    // wait for every store issued before it.
    float* Sc = p.S + ck.c * kD * kD;
    f32x4v s_out[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int e = t + kScanThreads * u, row = e / 8, c = 4 * (e % 8);
      s_out[u] = *reinterpret_cast<const f32x4v*>(S + row * kLdS + c);
    }
    // U = U~ - W S (64 x 32): wave w takes the 16 x 16 block at rows
    // 16 (w mod 4), columns 16 (w / 4).
    {
      f32x4v ws[1][1];
      clear(ws);
      const int i0 = 16 * (w % 4), j0 = 16 * (w / 4);
      mm_gen<false, true>(ws, W, kLd, i0, S, kLdS, j0, kD);
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int i = i0 + 4 * g + v, j = j0 + r;
        U[i * kLdS + j] = Ut[i * kLdS + j] - ws[0][0][v];
      }
    }
    __syncthreads();
    // U for memory, 16 bytes a thread.
    const f32x4v u_out = *reinterpret_cast<const f32x4v*>(U + (t / 8) * kLdS + 4 * (t % 8));
    // S <- g S + Kd' U (128 x 32): wave w takes rows 16 w .. 16 w + 15.
    {
      f32x4v ku[1][2];
      clear(ku);
      mm_gen<true, true>(ku, Kd, kLd, 16 * w, U, kLdS, 0, kC);
      float nw[2][4];
#pragma unroll
      for (int bj = 0; bj < 2; ++bj)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int i = 16 * w + 4 * g + v, j = 16 * bj + r;
          nw[bj][v] = gl * S[i * kLdS + j] + ku[0][bj][v];
        }
      __syncthreads();  // every wave has read S, U and this chunk's inputs
#pragma unroll
      for (int bj = 0; bj < 2; ++bj)
#pragma unroll
        for (int v = 0; v < 4; ++v) S[(16 * w + 4 * g + v) * kLdS + 16 * bj + r] = nw[bj][v];
    }
    if (n + 1 < p.chunks) {
      if (t < kC) ca[t] = in.ca;
      __syncthreads();
      scan_store(in, W, Ut, Kd, ca);
    }
    // S and U of this chunk to memory.
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int e = t + kScanThreads * u, row = e / 8, c = 4 * (e % 8);
      *reinterpret_cast<f32x4v*>(Sc + row * kD + col0 + c) = s_out[u];
    }
    *reinterpret_cast<f32x4v*>(p.U + ck.c * kC * kD + (t / 8) * kD + col0 + 4 * (t % 8)) = u_out;
  }
}

// ---- forward: outputs ----------------------------------------------------------------
// P = lower(Gamma o Q K'), O = diag(e^ca) Q S + P U; the products on the
// matrix cores (split bf16), Q and K in LDS as bf16.

// S and U are read by columns straight from memory (each wave's 32 columns
// once), so only Q, K and P live in LDS and several workgroups share a CU.
constexpr size_t kOutLds = 2 * kC * kLdH * sizeof(uint16_t) + (kC * kLdC + kC) * sizeof(float);

__global__ __launch_bounds__(256, 2) void dn_output(DnArgs p) {
  extern __shared__ float lds[];
  uint16_t* Qh = reinterpret_cast<uint16_t*>(lds);       // [64][kLdH]
  uint16_t* Kh = Qh + kC * kLdH;                          // [64][kLdH]
  float* P = reinterpret_cast<float*>(Kh + kC * kLdH);    // [64][kLdC]
  float* ca = P + kC * kLdC;      // [64]
  const Chunk ck = chunk_of(p, blockIdx.x);
  const int t = threadIdx.x, w = t / 64;
  const int r = t % 16, g = (t % 64) / 16;
  const float* S = p.S + ck.c * kD * kD;  // [128][128]
  const float* U = p.U + ck.c * kC * kD;  // [64][128]
  stage_rows_bf16(Qh, p.q + ck.row0, Kh, p.k + ck.row0, p.s_t);
  if (t < 64) ca[t] = p.ca[ck.c * kC + t];
  __syncthreads();
  const RowBf16 Qr{Qh, kLdH};
  {
    float* Pc = p.P + ck.c * kC * kC;
    for (int bj = 0; bj < 4; ++bj) {
      f32x4v acc[1][1];
      clear(acc);
      if (bj <= w) mm_by(acc, Qr, 16 * w, RowBf16{Kh, kLdH}, 16 * bj, kD);
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int i = 16 * w + 4 * g + v, j = 16 * bj + r;
        const float x = i >= j ? expf(ca[i] - ca[j]) * acc[0][0][v] : 0.0f;
        P[i * kLdC + j] = x;
        Pc[i * kC + j] = x;
      }
    }
  }
  __syncthreads();
  // O (64 x 128): wave w takes columns 32 w .. 32 w + 31.
  {
    f32x4v qs[4][2], pu[4][2];
    clear(qs);
    clear(pu);
    mm_by(qs, Qr, 0, ColF32{S, kD}, 32 * w, kD);
    mm_by(pu, RowF32{P, kLdC}, 0, ColF32{U, kD}, 32 * w, kC);
#pragma unroll
    for (int bi = 0; bi < 4; ++bi)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int i = 16 * bi + 4 * g + v;
        const float e = expf(ca[i]);
        uint16_t* orow = p.o + ck.row0 + (int64_t)i * p.s_t + 32 * w + r;
#pragma unroll
        for (int bj = 0; bj < 2; ++bj) orow[16 * bj] = to_bf(e * qs[bi][bj][v] + pu[bi][bj][v]);
      }
  }
}

// ---- backward: the state gradient swept back over chunks -------------------------------
// One workgroup per (sequence, 32 columns of dS), chunks in reverse:
//   dSn_n = dS;  dU = P' dO + diag(e^(last - ca)) K dS;  dS <- Qg' dO + g dS - W' dU,
// the products on the matrix cores (split bf16).  While a chunk's products run,
// the previous chunk's inputs (P, the dO columns, Q, K, W, ca) are loaded
// into registers; they go to LDS once the chunk is done with its own.

constexpr size_t kSgLds =
    (kC * kLdC + kC * kLdS + 3 * kC * kLd + kD * kLdS + kC * kLdS + kC) * sizeof(float);

// One chunk's inputs as this thread loads them (plain vector types, so the
// whole set stays in registers).
struct SgInputs {
  f32x4v p[2];     // P: 2 x 16 bytes
  u32x2v d;        // dO columns col0 .. col0 + 31: 8 bytes (bf16)
  u32x4v q[2], k[2];  // Q, K: 2 x 16 bytes each (bf16)
  f32x4v w[4];
  float ca;
};

__device__ __forceinline__ void sg_load(SgInputs& in, const DnArgs& p, const Chunk& ck, int col0) {
  const int t = threadIdx.x;
  const float* Pc = p.P + ck.c * kC * kC;
  const float* Wc = p.W + ck.c * kC * kD;
#pragma unroll
  for (int e = 0; e < 2; ++e) in.p[e] = reinterpret_cast<const f32x4v*>(Pc)[t + kScanThreads * e];
  in.d = *reinterpret_cast<const u32x2v*>(p.dout + ck.row0 + (int64_t)(t / 8) * p.s_t + col0 + 4 * (t % 8));
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int x = t + kScanThreads * e, r = x / 16, c = 8 * (x % 16);
    in.q[e] = *reinterpret_cast<const u32x4v*>(p.q + ck.row0 + (int64_t)r * p.s_t + c);
    in.k[e] = *reinterpret_cast<const u32x4v*>(p.k + ck.row0 + (int64_t)r * p.s_t + c);
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) in.w[e] = reinterpret_cast<const f32x4v*>(Wc)[t + kScanThreads * e];
  in.ca = t < kC ? p.ca[ck.c * kC + t] : 0.0f;
}

// The inputs to LDS; Q as Qg = diag(e^ca) Q (ca of the same chunk, already in LDS).
__device__ __forceinline__ void sg_store(const SgInputs& in, float* P, float* dO, float* Qg, float* K, float* W,
                                         const float* ca) {
  const int t = threadIdx.x;
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int x = t + kScanThreads * e, r = x / 16, c = 4 * (x % 16);
    *reinterpret_cast<f32x4v*>(P + r * kLdC + c) = in.p[e];
  }
  *reinterpret_cast<f32x4v*>(dO + (t / 8) * kLdS + 4 * (t % 8)) =
      f32x4v{bf((uint16_t)in.d[0]), bf((uint16_t)(in.d[0] >> 16)), bf((uint16_t)in.d[1]), bf((uint16_t)(in.d[1] >> 16))};
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int x = t + kScanThreads * e, r = x / 16, c = 8 * (x % 16);
    const float eq = expf(ca[r]);
    const u32x4v uq = in.q[e], uk = in.k[e];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      *reinterpret_cast<f32x4v*>(Qg + r * kLd + c + 4 * h) =
          f32x4v{eq * bf((uint16_t)uq[2 * h]), eq * bf((uint16_t)(uq[2 * h] >> 16)), eq * bf((uint16_t)uq[2 * h + 1]),
                 eq * bf((uint16_t)(uq[2 * h + 1] >> 16))};
      *reinterpret_cast<f32x4v*>(K + r * kLd + c + 4 * h) =
          f32x4v{bf((uint16_t)uk[2 * h]), bf((uint16_t)(uk[2 * h] >> 16)), bf((uint16_t)uk[2 * h + 1]),
                 bf((uint16_t)(uk[2 * h + 1] >> 16))};
    }
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int x = t + kScanThreads * e, r = x / 32, c = 4 * (x % 32);
    *reinterpret_cast<f32x4v*>(W + r * kLd + c) = in.w[e];
  }
}

__global__ __launch_bounds__(kScanThreads, 1) void dn_state_grad(DnArgs p) {
  extern __shared__ float lds[];
  float* P = lds;                  // [64][kLdC]
  float* dO = P + kC * kLdC;       // [64][kLdS]: columns col0 .. col0 + 31 of dO
  float* Qg = dO + kC * kLdS;      // [64][kLd]: diag(e^ca) Q
  float* K = Qg + kC * kLd;        // [64][kLd]
  float* W = K + kC * kLd;         // [64][kLd]
  float* dS = W + kC * kLd;        // [128][kLdS]: the state gradient's 32 columns
  float* dU = dS + kD * kLdS;      // [64][kLdS]
  float* ca = dU + kC * kLdS;      // [64]
  const int t = threadIdx.x, w = t / 64;
  const int r = t % 16, g = (t % 64) / 16;
  const ScanSlot slot = scan_slot();
  const int64_t seq = slot.seq;
  const int col0 = slot.col0;
  for (int e = t; e < kD * kLdS; e += kScanThreads) dS[e] = 0.0f;
  SgInputs in;
  {
    const Chunk ck = chunk_of(p, seq * p.chunks + p.chunks - 1);
    sg_load(in, p, ck, col0);
    if (t < kC) ca[t] = in.ca;
    __syncthreads();
    sg_store(in, P, dO, Qg, K, W, ca);
  }
  for (int n = p.chunks - 1; n >= 0; --n) {
    const Chunk ck = chunk_of(p, seq * p.chunks + n);
    __syncthreads();
    // This chunk's starting state, where this thread's dS values below sit:
    // dg's partial sums take it at the chunk's end.
    f32x4v s_in[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int e = t + kScanThreads * u, row = e / 8, c = 4 * (e % 8);
      s_in[u] = *reinterpret_cast<const f32x4v*>(p.S + ck.c * kD * kD + row * kD + col0 + c);
    }
    if (n > 0) sg_load(in, p, chunk_of(p, seq * p.chunks + n - 1), col0);
    const float last = ca[kC - 1];
    // The gradient at the chunk's end state: read now, written to memory at
    // the chunk's end (and dU with it), after the previous chunk's inputs are
    // in LDS, whose wait for their loads would also wait for every store
    // issued before it.
    float* dSc = p.dSn + ck.c * kD * kD;
    f32x4v ds_out[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int e = t + kScanThreads * u, row = e / 8, c = 4 * (e % 8);
      ds_out[u] = *reinterpret_cast<const f32x4v*>(dS + row * kLdS + c);
    }
    // dU (64 x 32): wave w takes the 16 x 16 block at rows 16 (w mod 4),
    // columns 16 (w / 4).
    {
      f32x4v pd[1][1], kd[1][1];
      clear(pd);
      clear(kd);
      const int i0 = 16 * (w % 4), j0 = 16 * (w / 4);
      mm_by(pd, ColF32{P, kLdC}, i0, ColF32Bf{dO, kLdS}, j0, kC);  // dO: bf16 values
      mm_by(kd, RowF32Bf{K, kLd}, i0, ColF32{dS, kLdS}, j0, kD);  // K: bf16 values
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int i = i0 + 4 * g + v;
        dU[i * kLdS + j0 + r] = pd[0][0][v] + expf(last - ca[i]) * kd[0][0][v];
      }
    }
    __syncthreads();
    // dU for memory, 16 bytes a thread.
    const f32x4v du_out = *reinterpret_cast<const f32x4v*>(dU + (t / 8) * kLdS + 4 * (t % 8));
    // dS <- Qg' dO + g dS - W' dU (128 x 32): wave w takes rows 16 w .. 16 w + 15.
    {
      f32x4v qd[1][2], wu[1][2];
      clear(qd);
      clear(wu);
      mm_by(qd, ColF32{Qg, kLd}, 16 * w, ColF32Bf{dO, kLdS}, 0, kC);
      mm_gen<true, true>(wu, W, kLd, 16 * w, dU, kLdS, 0, kC);
      const float gl = expf(last);
      float nw[2][4];
#pragma unroll
      for (int bj = 0; bj < 2; ++bj)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int i = 16 * w + 4 * g + v, j = 16 * bj + r;
          nw[bj][v] = qd[0][bj][v] + gl * dS[i * kLdS + j] - wu[0][bj][v];
        }
      __syncthreads();  // every wave has read dS, dU and this chunk's inputs
#pragma unroll
      for (int bj = 0; bj < 2; ++bj)
#pragma unroll
        for (int v = 0; v < 4; ++v) dS[(16 * w + 4 * g + v) * kLdS + 16 * bj + r] = nw[bj][v];
    }
    if (n > 0) {
      if (t < kC) ca[t] = in.ca;
      __syncthreads();
      sg_store(in, P, dO, Qg, K, W, ca);
    }
    // dSn and dU of this chunk to memory.
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int e = t + kScanThreads * u, row = e / 8, c = 4 * (e % 8);
      *reinterpret_cast<f32x4v*>(dSc + row * kD + col0 + c) = ds_out[u];
    }
    *reinterpret_cast<f32x4v*>(p.dU + ck.c * kC * kD + (t / 8) * kD + col0 + 4 * (t % 8)) = du_out;
    // This wave's part of dg = <S, dSn>.
    float dot = 0.0f;
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e) dot = fmaf(s_in[u][e], ds_out[u][e], dot);
    dot = thd::wave_sum(dot);
    if (t % 64 == 0) p.dg[ck.c * kDgParts + (col0 / kCols) * (kScanThreads / 64) + w] = dot;
  }
}

// ---- backward: the chunk's products (part a) ---------------------------------------
// dQg = dO S', dW = -dU S', dKd = U dSn', dP = lower(dO U'),
// every product on the matrix cores (split bf16).  Two phases through LDS: dO, dU
// and S, then U and dSn (dO stays).  Wave w computes columns 32 w .. 32 w + 31
// of the 64 x 128 results and row block w of dP.

// S and dSn are read by rows straight from memory (each wave's 32 rows, for
// both products that use them at once), so only dO and one 64-row operand
// live in LDS and two workgroups share a CU.
constexpr size_t kGaLds = 2 * kC * kLd * sizeof(float);

// acc1 += X1 Y', acc2 += X2 Y' over k in [0, K): X1, X2 rows i0 .. of LDS
// (stride kLd), Y rows j0 + 16 bj .. of memory (stride kD), each Y quad read once;
// kExact1: X1's fp32 values are bf16 values.
template <int BI, int BJ, bool kExact1 = false>
__device__ __forceinline__ void mm_nt2(f32x4v (&acc1)[BI][BJ], const float* X1, f32x4v (&acc2)[BI][BJ], const float* X2,
                                       int i0, const float* Y, int j0, int K) {
  const int r = threadIdx.x % 16, g = (threadIdx.x % 64) / 16;
  for (int kb = 0; kb < K; kb += 32) {
    Split8 a1[BI], a2[BI], b[BJ];
#pragma unroll
    for (int bj = 0; bj < BJ; ++bj) {
      const float* row = Y + (j0 + 16 * bj + r) * kD + kb + 8 * g;
      b[bj] = split8<false>(quad(row), quad(row + 4));
    }
#pragma unroll
    for (int bi = 0; bi < BI; ++bi) {
      const float* r1 = X1 + (i0 + 16 * bi + r) * kLd + kb + 8 * g;
      const float* r2 = X2 + (i0 + 16 * bi + r) * kLd + kb + 8 * g;
      a1[bi] = split8<kExact1>(quad(r1), quad(r1 + 4));
      a2[bi] = split8<false>(quad(r2), quad(r2 + 4));
    }
#pragma unroll
    for (int bi = 0; bi < BI; ++bi)
#pragma unroll
      for (int bj = 0; bj < BJ; ++bj) {
        acc1[bi][bj] = mma_split<kExact1, false>(a1[bi], b[bj], acc1[bi][bj]);
        acc2[bi][bj] = mma_split<false, false>(a2[bi], b[bj], acc2[bi][bj]);
      }
  }
}

__global__ __launch_bounds__(256, 2) void dn_grad_a(DnArgs p) {
  extern __shared__ float lds[];
  float* dO = lds;              // [64][kLd]
  float* X = dO + kC * kLd;     // [64][kLd]: dU, then U
  const Chunk ck = chunk_of(p, blockIdx.x);
  const int t = threadIdx.x, w = t / 64;
  const float* Sc = p.S + ck.c * kD * kD;
  const float* dSc = p.dSn + ck.c * kD * kD;
  stage_bf16(dO, p.dout + ck.row0, p.s_t);
  stage_f32(X, p.dU + ck.c * kC * kD);
  __syncthreads();
  {
    f32x4v q[4][2], wq[4][2];
    clear(q);
    clear(wq);
    mm_nt2<4, 2, true>(q, dO, wq, X, 0, Sc, 32 * w, kD);  // dO: bf16 values
    store_blocks(p.dQg + ck.c * kC * kD, kD, q, 0, 32 * w, 1.0f);
    store_blocks(p.dW + ck.c * kC * kD, kD, wq, 0, 32 * w, -1.0f);
  }
  __syncthreads();
  stage_f32(X, p.U + ck.c * kC * kD);
  __syncthreads();
  {
    f32x4v kd[4][2];
    clear(kd);
    mm_by(kd, RowF32{X, kLd}, 0, RowF32{dSc, kD}, 32 * w, kD);
    store_blocks(p.dKd + ck.c * kC * kD, kD, kd, 0, 32 * w, 1.0f);
  }
  {
    // Row block w of dP: blocks (w, jb) for jb <= w, the diagonal masked, zeros above.
    const int r = t % 16, g = (t % 64) / 16;
    float* dPc = p.dP + ck.c * kC * kC;
    for (int jb = 0; jb < 4; ++jb) {
      f32x4v acc[1][1];
      clear(acc);
      if (jb <= w) mm_nt<1, 1, true>(acc, dO, 16 * w, X, 16 * jb, kD);  // dO: bf16 values
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int i = 16 * w + 4 * g + v, j = 16 * jb + r;
        dPc[i * kC + j] = i >= j ? acc[0][0][v] : 0.0f;
      }
    }
  }
}

// ---- backward: the chunk's WY form, decays and gates (part b) -----------------------
// Every product on the matrix cores, split bf16 (mm_by below); Q and K sit in LDS
// as bf16 (their exact values) and are widened as they are read, V is read
// from global where it is needed, and dW, dU~ take turns in one fp32 buffer.
// The row sums of the gate gradients are complete within a wave (each wave
// owns 16 rows of the 64 x 64 work, and 32 of the 128 columns of the
// 64 x 128 work, whose partials go to LDS by wave) and are folded in a fixed
// order, so the result does not depend on timing.

// dW, dU~ and T are read straight from memory by the products that use them,
// so LDS holds Q, K, M and N only and two workgroups share a CU; dQK = dP o
// Gamma (lower) takes N once N's own last use is past.
constexpr size_t kGbLds = 2 * kC * kLdH * sizeof(uint16_t) + 2 * kC * kLdC * sizeof(float) +
                          (2 * kC + 5 * 4 * kC + 2 * kC) * sizeof(float);

__global__ __launch_bounds__(256, 2) void dn_grad_b(DnArgs p) {
  extern __shared__ float lds[];
  uint16_t* Qh = reinterpret_cast<uint16_t*>(lds);       // [64][kLdH]
  uint16_t* Kh = Qh + kC * kLdH;                          // [64][kLdH]
  float* M = reinterpret_cast<float*>(Kh + kC * kLdH);   // [64][kLdC]: dT, then dA, then dG + dG'
  float* N = M + kC * kLdC;        // [64][kLdC]: T' dT, then dG, then dQK
  float* wrow = N + kC * kLdC;     // [64]: sum_j w_ij
  float* brow = wrow + kC;         // [64]: sum_j dA Gamma G
  float* wcol = brow + kC;         // [4][64]: sum_i w_ij by wave
  float* kx = wcol + 4 * kC;       // [4][64]: k . dX by wave (columns)
  float* vy = kx + 4 * kC;         // [4][64]
  float* qq = vy + 4 * kC;         // [4][64]
  float* kk = qq + 4 * kC;         // [4][64]
  float* ca = kk + 4 * kC;         // [64]
  float* be = ca + kC;             // [64]
  const Chunk ck = chunk_of(p, blockIdx.x);
  const int t = threadIdx.x, w = t / 64;
  const int r = t % 16, g = (t % 64) / 16;
  const uint16_t* qg = p.q + ck.row0;
  const uint16_t* kg = p.k + ck.row0;
  const uint16_t* vg = p.v + ck.row0;
  const float* Tc = p.T + ck.c * kC * kC;  // [64][64]
  const float* dW = p.dW + ck.c * kC * kD;
  const float* dUt = p.dU + ck.c * kC * kD;
  const int i0 = 16 * w;  // this wave's rows of the 64 x 64 work
  // The first products' operands from memory (this wave's rows of dW and
  // dU~, its lanes' V), requested before the staging so that their latency
  // overlaps it: lane (r, g) takes k = 32 kb + 8 g + (0..7).
  f32x4v dwq[8], duq[8];
  uint2 vq[4][8];
  {
    const float* dWr = dW + (i0 + r) * kD + 8 * g;
    const float* dUr = dUt + (i0 + r) * kD + 8 * g;
#pragma unroll
    for (int h = 0; h < 8; ++h) {
      dwq[h] = quad(dWr + 32 * (h / 2) + 4 * (h % 2));
      duq[h] = quad(dUr + 32 * (h / 2) + 4 * (h % 2));
    }
#pragma unroll
    for (int bj = 0; bj < 4; ++bj)
#pragma unroll
      for (int h = 0; h < 8; ++h)
        vq[bj][h] = *reinterpret_cast<const uint2*>(vg + (int64_t)(16 * bj + r) * p.s_t + 32 * (h / 2) + 8 * g + 4 * (h % 2));
  }
  stage_rows_bf16(Qh, qg, Kh, kg, p.s_t);
  const float* dQg = p.dQg + ck.c * kC * kD;
  const float* dKd = p.dKd + ck.c * kC * kD;
  const float* dP = p.dP + ck.c * kC * kC;
  const float dg_part = t < kDgParts ? p.dg[ck.c * kDgParts + t] : 0.0f;
  if (t < 64) {
    ca[t] = p.ca[ck.c * kC + t];
    be[t] = p.beta[ck.grow0 + (int64_t)t * p.g_t];
  }
  __syncthreads();
  const RowBf16 Kr{Kh, kLdH}, Qr{Qh, kLdH};
  const ColBf16 Kc{Kh, kLdH}, Qc{Qh, kLdH};
  const float last = ca[kC - 1];
  // dT = dW X' + dU~ Y',  X = diag(beta e^ca) K, Y = diag(beta) V.
  {
    f32x4v xk[1][4], yv[1][4];
    clear(xk);
    clear(yv);
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const Split8 aw = split8<false>(dwq[2 * kb], dwq[2 * kb + 1]);
      const Split8 au = split8<false>(duq[2 * kb], duq[2 * kb + 1]);
#pragma unroll
      for (int bj = 0; bj < 4; ++bj) {
        const int x = 16 * bj + r, k0 = 32 * kb + 8 * g;
        const Split8 bk = split8<true>(Kr.quad(x, k0), Kr.quad(x, k0 + 4));
        xk[0][bj] = mma_split<false, true>(aw, bk, xk[0][bj]);
        const uint2 v0 = vq[bj][2 * kb], v1 = vq[bj][2 * kb + 1];
        const Split8 bv{__builtin_bit_cast(bf16x8v, u32x4v{v0.x, v0.y, v1.x, v1.y}),
                        __builtin_bit_cast(bf16x8v, u32x4v{0u, 0u, 0u, 0u})};
        yv[0][bj] = mma_split<false, true>(au, bv, yv[0][bj]);
      }
    }
#pragma unroll
    for (int bj = 0; bj < 4; ++bj)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int i = i0 + 4 * g + v, l = 16 * bj + r;
        M[i * kLdC + l] = be[l] * (expf(ca[l]) * xk[0][bj][v] + yv[0][bj][v]);
      }
  }
  __syncthreads();
  // N = T' dT.
  {
    f32x4v acc[1][4];
    clear(acc);
    mm_by(acc, ColF32{Tc, kC}, i0, ColF32{M, kLdC}, 0, kC);
    store_blocks(N, kLdC, acc, i0, 0, 1.0f);
  }
  __syncthreads();
  // dA = -(N T') o strict lower (into M).
  {
    f32x4v acc[1][4];
    clear(acc);
    mm_by(acc, RowF32{N, kLdC}, i0, RowF32{Tc, kC}, 0, kC);
#pragma unroll
    for (int bj = 0; bj < 4; ++bj)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int i = i0 + 4 * g + v, j = 16 * bj + r;
        M[i * kLdC + j] = i > j ? -acc[0][bj][v] : 0.0f;
      }
  }
  // Every row of this wave's M was written by this wave; the other waves'
  // rows are not read before the next barrier.
  // With G = K K', QK = Q K', Gamma: dG = dA o beta_i o Gamma (into N);
  // dbeta_i gets sum_j dA Gamma G; w = (dA beta_i G + dP QK) o Gamma gives
  // dca_i += sum_j w_ij - sum_j w_ji.
  {
    // This lane's dP values, loaded under the products below.
    float dpv[4][4];
#pragma unroll
    for (int bj = 0; bj < 4; ++bj)
#pragma unroll
      for (int v = 0; v < 4; ++v) dpv[bj][v] = dP[(i0 + 4 * g + v) * kC + 16 * bj + r];
    f32x4v gk[1][4], qk[1][4];
    clear(gk);
    clear(qk);
#pragma unroll
    for (int bj = 0; bj < 4; ++bj) {
      if (bj <= w) {
        f32x4v a1[1][1], a2[1][1];
        clear(a1);
        clear(a2);
        mm_by(a1, Kr, i0, Kr, 16 * bj, kD);
        mm_by(a2, Qr, i0, Kr, 16 * bj, kD);
        gk[0][bj] = a1[0][0];
        qk[0][bj] = a2[0][0];
      }
    }
    float roww[4] = {0, 0, 0, 0}, rowb[4] = {0, 0, 0, 0};
    float colw[4] = {0, 0, 0, 0};  // column 16 bj + r, this wave's rows
#pragma unroll
    for (int bj = 0; bj < 4; ++bj)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int i = i0 + 4 * g + v, j = 16 * bj + r;
        const float gam = expf(ca[i] - ca[j]);
        const float dA = M[i * kLdC + j];
        const float gg = bj <= w ? gk[0][bj][v] : 0.0f, q = bj <= w ? qk[0][bj][v] : 0.0f;
        N[i * kLdC + j] = dA * be[i] * gam;
        rowb[v] += dA * gam * gg;
        const float wv = i >= j ? (dA * be[i] * gg + dpv[bj][v] * q) * gam : 0.0f;
        roww[v] += wv;
        colw[bj] += wv;
      }
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      roww[v] = row_group_sum(roww[v]);
      rowb[v] = row_group_sum(rowb[v]);
    }
    if (r == 0)
#pragma unroll
      for (int v = 0; v < 4; ++v) wrow[i0 + 4 * g + v] = roww[v], brow[i0 + 4 * g + v] = rowb[v];
    // Column sums over this wave's 16 rows: the four row groups g, in order.
#pragma unroll
    for (int bj = 0; bj < 4; ++bj) {
      float x = colw[bj];
      x += __shfl_xor(x, 16, 64);
      x += __shfl_xor(x, 32, 64);
      if (g == 0) wcol[w * kC + 16 * bj + r] = x;
    }
  }
  __syncthreads();
  // M <- dG + dG'.
  for (int e = t; e < kC * kC; e += 256) {
    const int i = e / kC, j = e % kC;
    M[i * kLdC + j] = N[i * kLdC + j] + N[j * kLdC + i];
  }
  __syncthreads();
  // dQK = dP o Gamma (lower), read by two of the products below along its rows
  // and its columns: formed once into N (free now), not at every read.
  {
    float x[kC * kC / 256];
#pragma unroll
    for (int u = 0; u < kC * kC / 256; ++u) x[u] = dP[t + 256 * u];
#pragma unroll
    for (int u = 0; u < kC * kC / 256; ++u) {
      const int e = t + 256 * u, i = e / kC, j = e % kC;
      N[i * kLdC + j] = i >= j ? x[u] * expf(ca[i] - ca[j]) : 0.0f;
    }
  }
  __syncthreads();
  // dQ = e^ca dQg + dQK K;  dV = beta T' dU~;  dK = dQK' Q + (dG + dG') K +
  // beta e^ca dX + e^(last - ca) dKd with dX = T' dW.  Wave w: columns
  // 32 w .. 32 w + 31, one output at a time (two accumulator sets live).
  {
    const int d0 = 32 * w;
    const RowF32 Rr{N, kLdC};  // dQK along its rows
    const ColF32 Rc{N, kLdC};  // and along its columns
    {
      float gqv[4][4][2];  // this lane's dQg, loaded under the product
#pragma unroll
      for (int bi = 0; bi < 4; ++bi)
#pragma unroll
        for (int v = 0; v < 4; ++v)
#pragma unroll
          for (int bj = 0; bj < 2; ++bj) gqv[bi][v][bj] = dQg[(16 * bi + 4 * g + v) * kD + d0 + 16 * bj + r];
      f32x4v dq[4][2];
      clear(dq);
      mm_by(dq, Rr, 0, Kc, d0, kC);
#pragma unroll
      for (int bi = 0; bi < 4; ++bi)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int i = 16 * bi + 4 * g + v;
          const float e = expf(ca[i]);
          float sq = 0.0f;
#pragma unroll
          for (int bj = 0; bj < 2; ++bj) {
            const int d = d0 + 16 * bj + r;
            const float gq = gqv[bi][v][bj], qv = bf(Qh[i * kLdH + d]);
            sq = fmaf(qv, gq, sq);
            p.dq[ck.row0 + (int64_t)i * p.s_t + d] = to_bf(e * gq + dq[bi][bj][v]);
          }
          sq = row_group_sum(sq);
          if (r == 0) qq[w * kC + i] = sq;
        }
    }
    {
      // This lane's V values, all read before the first dV store (same
      // element type: loaded in the loop, each read would wait for the
      // previous store).
      f32x4v dy[4][2];
      clear(dy);
      mm_by(dy, ColF32{Tc, kC}, 0, ColF32{dUt, kD}, d0, kC);
      // In two halves of row blocks: the V values of a half are all read
      // before its first dV store (same element type: loaded in the loop,
      // each read would wait for the previous store).
#pragma unroll
      for (int hb = 0; hb < 2; ++hb) {
        uint32_t vh[2][4];  // the two bf16 of columns d0 + r, d0 + 16 + r
#pragma unroll
        for (int b2 = 0; b2 < 2; ++b2)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const uint16_t* vr = vg + (int64_t)(16 * (2 * hb + b2) + 4 * g + v) * p.s_t + d0 + r;
            vh[b2][v] = (uint32_t)vr[0] | ((uint32_t)vr[16] << 16);
          }
#pragma unroll
        for (int b2 = 0; b2 < 2; ++b2)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int bi = 2 * hb + b2, i = 16 * bi + 4 * g + v;
            float sv = 0.0f;
#pragma unroll
            for (int bj = 0; bj < 2; ++bj) {
              const int d = d0 + 16 * bj + r;
              const float vv = bf((uint16_t)(vh[b2][v] >> (16 * bj))), yv = dy[bi][bj][v];
              sv = fmaf(vv, yv, sv);
              p.dv[ck.row0 + (int64_t)i * p.s_t + d] = to_bf(be[i] * yv);
            }
            sv = row_group_sum(sv);
            if (r == 0) vy[w * kC + i] = sv;
          }
      }
    }
    {
      // dX first; its terms of dK (beta e^ca dX + e^(last - ca) dKd) then
      // seed dK's accumulator, so one accumulator set is live at a time.
      float gkv[4][4][2];  // this lane's dKd, loaded under the product
#pragma unroll
      for (int bi = 0; bi < 4; ++bi)
#pragma unroll
        for (int v = 0; v < 4; ++v)
#pragma unroll
          for (int bj = 0; bj < 2; ++bj) gkv[bi][v][bj] = dKd[(16 * bi + 4 * g + v) * kD + d0 + 16 * bj + r];
      f32x4v acc[4][2];
      clear(acc);
      mm_by(acc, ColF32{Tc, kC}, 0, ColF32{dW, kD}, d0, kC);
#pragma unroll
      for (int bi = 0; bi < 4; ++bi)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int i = 16 * bi + 4 * g + v;
          const float e = expf(ca[i]), ed = expf(last - ca[i]);
          float sx = 0.0f, sk = 0.0f;
#pragma unroll
          for (int bj = 0; bj < 2; ++bj) {
            const int d = d0 + 16 * bj + r;
            const float gk = gkv[bi][v][bj], kv = bf(Kh[i * kLdH + d]);
            const float xv = acc[bi][bj][v];
            sx = fmaf(kv, xv, sx);
            sk = fmaf(kv, gk, sk);
            acc[bi][bj][v] = be[i] * e * xv + ed * gk;
          }
          sx = row_group_sum(sx);
          sk = row_group_sum(sk);
          if (r == 0) kx[w * kC + i] = sx, kk[w * kC + i] = sk;
        }
      mm_by(acc, Rc, 0, Qc, d0, kC);
      mm_by(acc, RowF32{M, kLdC}, 0, Kc, d0, kC);
#pragma unroll
      for (int bi = 0; bi < 4; ++bi)
#pragma unroll
        for (int v = 0; v < 4; ++v)
#pragma unroll
          for (int bj = 0; bj < 2; ++bj) {
            const int i = 16 * bi + 4 * g + v, d = d0 + 16 * bj + r;
            p.dk[ck.row0 + (int64_t)i * p.s_t + d] = to_bf(acc[bi][bj][v]);
          }
    }
  }
  __syncthreads();
  // Fold the partials in a fixed order (lane i: row i), then da = the
  // reverse cumulative sum of dca, dca_63 also taking sum kd + dg g.
  if (t < 64) {
    const int i = t;
    float sc = 0.0f, skx = 0.0f, svy = 0.0f, sqq = 0.0f, skk = 0.0f;
    for (int wv = 0; wv < 4; ++wv) {
      sc += wcol[wv * kC + i];
      skx += kx[wv * kC + i];
      svy += vy[wv * kC + i];
      sqq += qq[wv * kC + i];
      skk += kk[wv * kC + i];
    }
    const float sw = wrow[i], sb = brow[i];
    const float e = expf(ca[i]), ed = expf(last - ca[i]);
    const float kd = ed * skk;
    float dca = sw - sc + be[i] * e * skx + e * sqq - kd;
    float kd_all = kd;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) kd_all += __shfl_xor(kd_all, o, 64);
    // dg: its kDgParts partial sums, lane q holding part q, a fixed tree.
    float dg = i < kDgParts ? dg_part : 0.0f;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) dg += __shfl_xor(dg, o, 64);
    if (i == kC - 1) dca += kd_all + dg * expf(last);
    float x = dca;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const float y = __shfl_down(x, o, 64);
      if (i + o < 64) x += y;
    }
    p.da[ck.grow0 + (int64_t)i * p.g_t] = x;
    p.dbeta[ck.grow0 + (int64_t)i * p.g_t] = sb + e * skx + svy;
  }
}

bool aligned(const void* q, int bytes) { return (reinterpret_cast<uintptr_t>(q) % bytes) == 0; }

struct Workspace {
  size_t offs[14];
  size_t bytes;
};

Workspace workspace(int64_t chunks, bool backward) {
  const size_t sizes[14] = {(size_t)kC, (size_t)kC * kC, (size_t)kC * kD, (size_t)kC * kD, (size_t)kD * kD,
                            (size_t)kC * kD, (size_t)kC * kC, (size_t)kC * kD, (size_t)kD * kD, (size_t)kC * kD,
                            (size_t)kC * kD, (size_t)kC * kD, (size_t)kC * kC, (size_t)kDgParts};
  Workspace w{};
  size_t at = 0;
  for (int i = 0; i < 14; ++i) {
    w.offs[i] = at;
    if (i < 7 || backward) at += ((sizes[i] * chunks * sizeof(float)) + 255) & ~(size_t)255;
  }
  w.bytes = at;
  return w;
}

int check(const th_deltanet_desc* d, bool backward) {
  TH_REQUIRE(d != nullptr, "deltanet: null descriptor");
  TH_REQUIRE(d->dk == kD && d->dv == kD, "deltanet: dk and dv must be 128");
  TH_REQUIRE(d->chunk == kC, "deltanet: the chunk must be 64");
  TH_REQUIRE(d->seq > 0 && d->seq % kC == 0, "deltanet: the sequence length must be a positive multiple of 64");
  TH_REQUIRE(d->batch > 0 && d->heads > 0, "deltanet: batch and heads must be positive");
  TH_REQUIRE(d->q && d->k && d->v && d->a && d->beta && (d->o || backward), "deltanet: null q, k, v, a, beta or o");
  TH_REQUIRE(aligned(d->q, 16) && aligned(d->k, 16) && aligned(d->v, 16) && aligned(d->o, 16),
             "deltanet: q, k, v, o must be 16-byte aligned");
  TH_REQUIRE(d->strides[0] % 8 == 0 && d->strides[1] % 8 == 0 && d->strides[2] % 8 == 0,
             "deltanet: strides must be multiples of 8");
  if (backward) {
    TH_REQUIRE(d->dout && d->dq && d->dk_out && d->dv_out && d->da && d->dbeta, "deltanet backward: null gradient");
    TH_REQUIRE(aligned(d->dout, 16) && aligned(d->dq, 16) && aligned(d->dk_out, 16) && aligned(d->dv_out, 16),
               "deltanet backward: gradients must be 16-byte aligned");
  }
  return TH_OK;
}

int build(const th_deltanet_desc* d, bool backward, th_launch** out) {
  if (int r = th::require_ready()) return r;
  *out = nullptr;
  if (int r = check(d, backward)) return r;
  const int64_t chunks = (int64_t)d->batch * d->heads * (d->seq / kC);
  TH_REQUIRE(chunks <= 0x7fffffff, "deltanet: too many chunks");
  const Workspace w = workspace(chunks, backward);
  DnArgs a{};
  a.q = static_cast<const uint16_t*>(d->q);
  a.k = static_cast<const uint16_t*>(d->k);
  a.v = static_cast<const uint16_t*>(d->v);
  a.a = d->a;
  a.beta = d->beta;
  a.o = static_cast<uint16_t*>(d->o);
  a.dout = static_cast<const uint16_t*>(d->dout);
  a.dq = static_cast<uint16_t*>(d->dq);
  a.dk = static_cast<uint16_t*>(d->dk_out);
  a.dv = static_cast<uint16_t*>(d->dv_out);
  a.da = d->da;
  a.dbeta = d->dbeta;
  // The per-chunk intermediates (ca, T, W, Ut, S, U, P; for the backward dU,
  // dSn, dQg, dW, dKd, dP, dg) lie in the launch's workspace at w.offs.
  const size_t slot_args[14] = {TH_OFFSET(DnArgs, ca),  TH_OFFSET(DnArgs, T),   TH_OFFSET(DnArgs, W),
                                TH_OFFSET(DnArgs, Ut),  TH_OFFSET(DnArgs, S),   TH_OFFSET(DnArgs, U),
                                TH_OFFSET(DnArgs, P),   TH_OFFSET(DnArgs, dU),  TH_OFFSET(DnArgs, dSn),
                                TH_OFFSET(DnArgs, dQg), TH_OFFSET(DnArgs, dW),  TH_OFFSET(DnArgs, dKd),
                                TH_OFFSET(DnArgs, dP),  TH_OFFSET(DnArgs, dg)};
  a.s_h = d->strides[0];
  a.s_t = d->strides[1];
  a.s_b = d->strides[2];
  a.g_h = d->gate_strides[0];
  a.g_t = d->gate_strides[1];
  a.g_b = d->gate_strides[2];
  a.batch = d->batch;
  a.heads = d->heads;
  a.seq = d->seq;
  a.chunks = d->seq / kC;
  const void* fns[7] = {(const void*)dn_chunk_prep, (const void*)dn_state_scan, (const void*)dn_output,
                        (const void*)dn_state_grad, (const void*)dn_grad_a, (const void*)dn_grad_b, nullptr};
  const size_t ldss[6] = {kPrepLds, kScanLds, kOutLds, kSgLds, kGaLds, kGbLds};
  for (int i = 0; i < 6; ++i) TH_HIP(hipFuncSetAttribute(fns[i], hipFuncAttributeMaxDynamicSharedMemorySize, (int)ldss[i]));
  th::Builder b(backward ? "deltanet_fwd_bwd" : "deltanet_fwd", 12);
  const uint64_t at_ws = b.workspace(w.bytes);
  // A gradient with no o given keeps it in the workspace, at q's strides.
  const bool own_o = d->o == nullptr;
  const uint64_t o_bytes = 2 * ((uint64_t)(d->heads - 1) * d->strides[0] + (uint64_t)(d->seq - 1) * d->strides[1] +
                                (uint64_t)(d->batch - 1) * d->strides[2] + kD);
  const uint64_t at_o = own_o ? b.workspace(o_bytes) : 0;
  const unsigned nchunks = (unsigned)chunks;
  const unsigned scans = (unsigned)((int64_t)d->batch * d->heads * (kD / kCols));
  int ks[6];
  int nk = 0;
  ks[nk++] = b.kernel(fns[0], "dn_chunk_prep", dim3(nchunks), dim3(256), (uint32_t)kPrepLds, a);
  ks[nk++] = b.kernel(fns[1], "dn_state_scan", dim3(scans), dim3(kScanThreads), (uint32_t)kScanLds, a);
  ks[nk++] = b.kernel(fns[2], "dn_output", dim3(nchunks), dim3(256), (uint32_t)kOutLds, a);
  if (backward) {
    ks[nk++] = b.kernel(fns[3], "dn_state_grad", dim3(scans), dim3(kScanThreads), (uint32_t)kSgLds, a);
    ks[nk++] = b.kernel(fns[4], "dn_grad_a", dim3(nchunks), dim3(256), (uint32_t)kGaLds, a);
    ks[nk++] = b.kernel(fns[5], "dn_grad_b", dim3(nchunks), dim3(256), (uint32_t)kGbLds, a);
  }
  const size_t offs[12] = {TH_OFFSET(DnArgs, q),  TH_OFFSET(DnArgs, k),  TH_OFFSET(DnArgs, v),     TH_OFFSET(DnArgs, a),
                           TH_OFFSET(DnArgs, beta), TH_OFFSET(DnArgs, o), TH_OFFSET(DnArgs, dout), TH_OFFSET(DnArgs, dq),
                           TH_OFFSET(DnArgs, dk), TH_OFFSET(DnArgs, dv), TH_OFFSET(DnArgs, da),  TH_OFFSET(DnArgs, dbeta)};
  for (int v = 0; v < 12; ++v)
    if (!(own_o && v == 5))
      for (int i = 0; i < nk; ++i) b.ref(v, ks[i], offs[v]);
  if (own_o)
    for (int i = 0; i < nk; ++i) b.ws_ref(ks[i], offs[5], at_o);
  for (int j = 0; j < 14; ++j)
    if (j < 7 || backward)
      for (int i = 0; i < nk; ++i) b.ws_ref(ks[i], slot_args[j], at_ws + w.offs[j]);
  for (int v : {0, 1, 2, 5, 6, 7, 8, 9}) b.align(v, 16);
  // Algorithmic work: per chunk, forward ~ C^2 dk (A) + C^3/3 (T) + 2 C^2 d (W, U~) + C^2 dk (P)
  // + 2 C dk dv (W S, Qg S) + C^2 dv (P U) + C dk dv (Kd' U) multiply-adds; the backward ~2.3x.
  const double C = kC, D = kD;
  const double fwd = 2.0 * (C * C * D + C * C * C / 3 + 2 * C * C * D + C * C * D + 3 * C * D * D + C * C * D);
  const double bytes_fwd = 2.0 * (4 * C * D) + 8.0 * C;  // q, k, v read, o written (bf16); a, beta
  b.work(chunks * (backward ? fwd * 3.3 : fwd), chunks * (backward ? 2 * bytes_fwd + 2.0 * 4 * C * D : bytes_fwd),
         chunks);
  th_launch* l = b.release();
  l->work.bytes = chunks * (backward ? 2 * bytes_fwd + 2.0 * 4 * C * D : bytes_fwd);
  l->work.flops = chunks * (backward ? fwd * 3.3 : fwd);
  *out = l;
  return TH_OK;
}

}  // namespace

extern "C" int th_build_deltanet_fwd(const th_deltanet_desc* d, th_launch** out) { return build(d, false, out); }

extern "C" int th_build_deltanet(const th_deltanet_desc* d, th_launch** out) { return build(d, true, out); }
