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
// Kernels (fp32 arithmetic on fp32 FMA units; inputs bf16 q, k, v and fp32
// a, beta):
//   dn_chunk_prep   one workgroup per chunk: ca, A, T (forward substitution,
//                   one lane per column), W, U~.
//   dn_state_scan   one workgroup per (sequence, 32 columns of S): the
//                   sequential recurrence, each column block independent;
//                   stores each chunk's starting state and U.
//   dn_output       one workgroup per chunk: P, O.
//   dn_state_grad   one workgroup per (sequence, 32 columns): the state
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
constexpr int kPadD = kD + 4;
constexpr int kPadC = kC + 1;

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
  float* dg;    // [c]
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

// A 64 x 128 bf16 chunk of a (d, heads, positions, batch) array into LDS as fp32 [64][kPadD].
__device__ __forceinline__ void load_chunk(float* dst, const uint16_t* src, int64_t s_t) {
  for (int e = threadIdx.x; e < kC * (kD / 8); e += 256) {
    const int r = e / (kD / 8), c8 = (e % (kD / 8)) * 8;
    const uint4 w = *reinterpret_cast<const uint4*>(src + r * s_t + c8);
    const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      dst[r * kPadD + c8 + 2 * j] = bf((uint16_t)u[j]);
      dst[r * kPadD + c8 + 2 * j + 1] = bf((uint16_t)(u[j] >> 16));
    }
  }
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

// acc[TM][TN] += sum_k A(i0 + r, k) B(k, j0 + c).
template <int TM, int TN, class FA, class FB>
__device__ __forceinline__ void mm(float (&acc)[TM][TN], int i0, int j0, int K, FA A, FB B) {
  for (int k = 0; k < K; ++k) {
    float av[TM], bv[TN];
#pragma unroll
    for (int r = 0; r < TM; ++r) av[r] = A(i0 + r, k);
#pragma unroll
    for (int c = 0; c < TN; ++c) bv[c] = B(k, j0 + c);
#pragma unroll
    for (int r = 0; r < TM; ++r)
#pragma unroll
      for (int c = 0; c < TN; ++c) acc[r][c] = fmaf(av[r], bv[c], acc[r][c]);
  }
}

template <int TM, int TN>
__device__ __forceinline__ void zero(float (&acc)[TM][TN]) {
#pragma unroll
  for (int r = 0; r < TM; ++r)
#pragma unroll
    for (int c = 0; c < TN; ++c) acc[r][c] = 0.0f;
}


// ---- fp32 products on the matrix cores ----------------------------------------------
// v_mfma_f32_16x16x4_f32 multiplies fp32 exactly and accumulates in fp32, as
// the per-thread FMA tiles do (only the order of the additions differs).
// Operands sit in LDS as fp32 rows of kLd floats: a row's 16-byte quads land
// on distinct bank quads for 16 consecutive rows (kLd / 4 odd), and a column
// read by 16 consecutive rows x 4 row groups hits 64 distinct banks
// (kLd = 4 mod 16).
//
// Lane l = 16 g + r of a 16 x 16 block over 16 consecutive k takes the four
// k = 16 kb + 4 g + (0..3): one ds_read_b128 per operand when k runs along
// its rows, four products, each pairing A(i0 + r, k) with B(k, j0 + r); the
// products' k slot g then holds the same k in both operands.  The block
// C(i0 + 4 g + v, j0 + r) sits in register v of lane l.

typedef float f32x4v __attribute__((ext_vector_type(4)));
constexpr int kLd = 132;

__device__ __forceinline__ f32x4v quad(const float* row) { return *reinterpret_cast<const f32x4v*>(row); }

// The four k of lane g's quad along a column: X(k, c) at x[k * ld + c].
__device__ __forceinline__ f32x4v column_quad(const float* x, int ld, int k0, int c) {
  return f32x4v{x[k0 * ld + c], x[(k0 + 1) * ld + c], x[(k0 + 2) * ld + c], x[(k0 + 3) * ld + c]};
}

__device__ __forceinline__ f32x4v mma4(f32x4v a, f32x4v b, f32x4v c) {
#pragma unroll
  for (int s = 0; s < 4; ++s) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s], b[s], c, 0, 0, 0);
  return c;
}

// acc[bi][bj] += X(i0 + 16 bi .., k) Y(j0 + 16 bj .., k) over k in [0, K):
// both operands with k along their rows (row-major in LDS, stride kLd).
template <int BI, int BJ>
__device__ __forceinline__ void mm_nt(f32x4v (&acc)[BI][BJ], const float* X, int i0, const float* Y, int j0, int K) {
  const int r = threadIdx.x % 16, g = (threadIdx.x % 64) / 16;
  for (int kb = 0; kb < K; kb += 16) {
    f32x4v a[BI], b[BJ];
#pragma unroll
    for (int bi = 0; bi < BI; ++bi) a[bi] = quad(X + (i0 + 16 * bi + r) * kLd + kb + 4 * g);
#pragma unroll
    for (int bj = 0; bj < BJ; ++bj) b[bj] = quad(Y + (j0 + 16 * bj + r) * kLd + kb + 4 * g);
#pragma unroll
    for (int bi = 0; bi < BI; ++bi)
#pragma unroll
      for (int bj = 0; bj < BJ; ++bj) acc[bi][bj] = mma4(a[bi], b[bj], acc[bi][bj]);
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
  for (int kb = 0; kb < K; kb += 16) {
    const int k0 = kb + 4 * g;
    f32x4v a[BI], b[BJ];
#pragma unroll
    for (int bi = 0; bi < BI; ++bi)
      a[bi] = XT ? column_quad(X, ldx, k0, i0 + 16 * bi + r) : quad(X + (i0 + 16 * bi + r) * ldx + k0);
#pragma unroll
    for (int bj = 0; bj < BJ; ++bj)
      b[bj] = YT ? column_quad(Y, ldy, k0, j0 + 16 * bj + r) : quad(Y + (j0 + 16 * bj + r) * ldy + k0);
#pragma unroll
    for (int bi = 0; bi < BI; ++bi)
#pragma unroll
      for (int bj = 0; bj < BJ; ++bj) acc[bi][bj] = mma4(a[bi], b[bj], acc[bi][bj]);
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
__device__ __forceinline__ void stage_f32(float* dst, const float* src, int rows) {
  for (int e = threadIdx.x; e < rows * 32; e += 256) {
    const int r = e / 32, c = 4 * (e % 32);
    *reinterpret_cast<float4*>(dst + r * kLd + c) = *reinterpret_cast<const float4*>(src + r * kD + c);
  }
}

// 64 x 128 bf16 of a (d, heads, positions, batch) array into LDS as fp32 rows of kLd.
__device__ __forceinline__ void stage_bf16(float* dst, const uint16_t* src, int64_t s_t) {
  for (int e = threadIdx.x; e < kC * 16; e += 256) {
    const int r = e / 16, c8 = 8 * (e % 16);
    const uint4 w = *reinterpret_cast<const uint4*>(src + r * s_t + c8);
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

// ---- forward: the chunk's WY form -------------------------------------------------

constexpr size_t kPrepLds = (2 * kC * kPadD + kC * kPadC + 2 * kC) * sizeof(float);

__global__ __launch_bounds__(256) void dn_chunk_prep(DnArgs p) {
  extern __shared__ float lds[];
  float* K = lds;                  // [64][kPadD]
  float* V = K + kC * kPadD;       // [64][kPadD]
  float* AT = V + kC * kPadD;      // [64][kPadC]: A, then T
  float* ca = AT + kC * kPadC;     // [64]
  float* be = ca + kC;             // [64]
  const Chunk ck = chunk_of(p, blockIdx.x);
  const int t = threadIdx.x;
  load_chunk(K, p.k + ck.row0, p.s_t);
  load_chunk(V, p.v + ck.row0, p.s_t);
  cumulative_gates(ca, p, ck);
  if (t < 64) be[t] = p.beta[ck.grow0 + (int64_t)t * p.g_t];
  __syncthreads();
  if (t < 64) p.ca[ck.c * kC + t] = ca[t];
  // A = strict lower (beta_i Gamma_ij k_i.k_j): thread (4 x 4) micro-tile.
  {
    const int i0 = 4 * (t / 16), j0 = 4 * (t % 16);
    float acc[4][4];
    zero(acc);
    if (j0 < i0 + 4)
      mm(acc, i0, j0, kD, [&](int i, int k) { return K[i * kPadD + k]; },
         [&](int k, int j) { return K[j * kPadD + k]; });
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int i = i0 + r, j = j0 + c;
        AT[i * kPadC + j] = i > j ? be[i] * expf(ca[i] - ca[j]) * acc[r][c] : 0.0f;
      }
  }
  __syncthreads();
  // T = (I + A)^-1 by forward substitution, lane j owning column j:
  // T_ij = -sum_{l<i} A_il T_lj for i > j, T_jj = 1.
  if (t < 64) {
    const int j = t;
    float col[kC];
#pragma unroll
    for (int i = 0; i < kC; ++i) {
      float s = 0.0f;
#pragma unroll
      for (int l = 0; l < i; ++l) s = fmaf(AT[i * kPadC + l], col[l], s);
      col[i] = i == j ? 1.0f : (i < j ? 0.0f : -s);
    }
    // One wave: its LDS reads of A above complete before its writes of T below.
#pragma unroll
    for (int i = 0; i < kC; ++i) AT[i * kPadC + j] = col[i];
  }
  __syncthreads();
  // W = T diag(beta e^ca) K, U~ = T diag(beta) V: thread (4 rows x 8 columns).
  {
    const int i0 = 4 * (t / 16), j0 = 8 * (t % 16);
    float w[4][8], u[4][8];
    zero(w);
    zero(u);
    for (int l = 0; l < kC; ++l) {
      float tv[4], xk[8], yv[8];
      const float sx = be[l] * expf(ca[l]), sy = be[l];
#pragma unroll
      for (int r = 0; r < 4; ++r) tv[r] = AT[(i0 + r) * kPadC + l];
#pragma unroll
      for (int c = 0; c < 8; ++c) xk[c] = sx * K[l * kPadD + j0 + c], yv[c] = sy * V[l * kPadD + j0 + c];
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int c = 0; c < 8; ++c) w[r][c] = fmaf(tv[r], xk[c], w[r][c]), u[r][c] = fmaf(tv[r], yv[c], u[r][c]);
    }
    float* Wc = p.W + ck.c * kC * kD;
    float* Uc = p.Ut + ck.c * kC * kD;
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int c = 0; c < 8; c += 4) {
        *reinterpret_cast<float4*>(Wc + (i0 + r) * kD + j0 + c) = make_float4(w[r][c], w[r][c + 1], w[r][c + 2], w[r][c + 3]);
        *reinterpret_cast<float4*>(Uc + (i0 + r) * kD + j0 + c) = make_float4(u[r][c], u[r][c + 1], u[r][c + 2], u[r][c + 3]);
      }
  }
  float* Tc = p.T + ck.c * kC * kC;
  for (int e = t; e < kC * kC; e += 256) Tc[e] = AT[(e / kC) * kPadC + e % kC];
}

// ---- forward: the recurrence across chunks, 32 columns of S per workgroup ---------

constexpr int kPadS = kCols + 1;
constexpr size_t kScanLds = (kD * kPadS + kC * kPadD + kC * kPadD + kC * kPadS + kC * kPadS + kC) * sizeof(float);

__global__ __launch_bounds__(256) void dn_state_scan(DnArgs p) {
  extern __shared__ float lds[];
  float* S = lds;                   // [128][kPadS]
  float* W = S + kD * kPadS;        // [64][kPadD]
  float* K = W + kC * kPadD;        // [64][kPadD]
  float* Ut = K + kC * kPadD;       // [64][kPadS]
  float* U = Ut + kC * kPadS;       // [64][kPadS]
  float* ca = U + kC * kPadS;       // [64]
  const int t = threadIdx.x;
  const int64_t seq = blockIdx.x / (kD / kCols);
  const int col0 = (blockIdx.x % (kD / kCols)) * kCols;
  for (int e = t; e < kD * kPadS; e += 256) S[e] = 0.0f;
  for (int n = 0; n < p.chunks; ++n) {
    const Chunk ck = chunk_of(p, seq * p.chunks + n);
    __syncthreads();
    // The chunk's starting state, stored for the output and the backward.
    float* Sc = p.S + ck.c * kD * kD;
    for (int e = t; e < kD * kCols; e += 256) Sc[(e / kCols) * kD + col0 + e % kCols] = S[(e / kCols) * kPadS + e % kCols];
    const float* Wc = p.W + ck.c * kC * kD;
    for (int e = t; e < kC * kD / 4; e += 256) {
      const float4 w = reinterpret_cast<const float4*>(Wc)[e];
      const int r = (4 * e) / kD, c = (4 * e) % kD;
      W[r * kPadD + c] = w.x, W[r * kPadD + c + 1] = w.y, W[r * kPadD + c + 2] = w.z, W[r * kPadD + c + 3] = w.w;
    }
    const float* Uc = p.Ut + ck.c * kC * kD;
    for (int e = t; e < kC * kCols; e += 256) Ut[(e / kCols) * kPadS + e % kCols] = Uc[(e / kCols) * kD + col0 + e % kCols];
    load_chunk(K, p.k + ck.row0, p.s_t);
    if (t < 64) ca[t] = p.ca[ck.c * kC + t];
    __syncthreads();
    // U = U~ - W S: thread (2 rows x 4 columns) of 64 x 32.
    {
      const int i0 = 2 * (t / 8), j0 = 4 * (t % 8);
      float acc[2][4];
      zero(acc);
      mm(acc, i0, j0, kD, [&](int i, int k) { return W[i * kPadD + k]; }, [&](int k, int j) { return S[k * kPadS + j]; });
      float* Uo = p.U + ck.c * kC * kD;
#pragma unroll
      for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const float u = Ut[(i0 + r) * kPadS + j0 + c] - acc[r][c];
          U[(i0 + r) * kPadS + j0 + c] = u;
          Uo[(i0 + r) * kD + col0 + j0 + c] = u;
        }
    }
    __syncthreads();
    // S <- g S + Kd' U, Kd_l = e^(ca_63 - ca_l) k_l: thread (4 rows x 4 columns) of 128 x 32.
    {
      const int i0 = 4 * (t / 8), j0 = 4 * (t % 8);
      const float last = ca[kC - 1];
      float acc[4][4];
      zero(acc);
      mm(acc, i0, j0, kC, [&](int i, int l) { return expf(last - ca[l]) * K[l * kPadD + i]; },
         [&](int l, int j) { return U[l * kPadS + j]; });
      const float g = expf(last);
      __syncthreads();
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) S[(i0 + r) * kPadS + j0 + c] = g * S[(i0 + r) * kPadS + j0 + c] + acc[r][c];
    }
  }
}

// ---- forward: outputs ----------------------------------------------------------------

constexpr size_t kOutLds = (3 * kC * kPadD + kC * kPadC + kC) * sizeof(float);

__global__ __launch_bounds__(256) void dn_output(DnArgs p) {
  extern __shared__ float lds[];
  float* Q = lds;                // [64][kPadD]
  float* K = Q + kC * kPadD;     // [64][kPadD]
  float* U = K + kC * kPadD;     // [64][kPadD]
  float* P = U + kC * kPadD;     // [64][kPadC]
  float* ca = P + kC * kPadC;    // [64]
  const Chunk ck = chunk_of(p, blockIdx.x);
  const int t = threadIdx.x;
  load_chunk(Q, p.q + ck.row0, p.s_t);
  load_chunk(K, p.k + ck.row0, p.s_t);
  const float* Uc = p.U + ck.c * kC * kD;
  for (int e = t; e < kC * kD; e += 256) U[(e / kD) * kPadD + e % kD] = Uc[e];
  if (t < 64) ca[t] = p.ca[ck.c * kC + t];
  __syncthreads();
  {
    const int i0 = 4 * (t / 16), j0 = 4 * (t % 16);
    float acc[4][4];
    zero(acc);
    if (j0 < i0 + 4)
      mm(acc, i0, j0, kD, [&](int i, int k) { return Q[i * kPadD + k]; }, [&](int k, int j) { return K[j * kPadD + k]; });
    float* Pc = p.P + ck.c * kC * kC;
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int i = i0 + r, j = j0 + c;
        const float v = i >= j ? expf(ca[i] - ca[j]) * acc[r][c] : 0.0f;
        P[i * kPadC + j] = v;
        Pc[i * kC + j] = v;
      }
  }
  __syncthreads();
  // O = diag(e^ca) Q S + P U: thread (4 rows x 8 columns) of 64 x 128.
  {
    const int i0 = 4 * (t / 16), j0 = 8 * (t % 16);
    const float* Sc = p.S + ck.c * kD * kD;
    float qs[4][8], pu[4][8];
    zero(qs);
    zero(pu);
    mm(qs, i0, j0, kD, [&](int i, int k) { return Q[i * kPadD + k]; }, [&](int k, int j) { return Sc[k * kD + j]; });
    mm(pu, i0, j0, kC, [&](int i, int l) { return P[i * kPadC + l]; }, [&](int l, int j) { return U[l * kPadD + j]; });
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float e = expf(ca[i0 + r]);
      uint16_t* orow = p.o + ck.row0 + (int64_t)(i0 + r) * p.s_t + j0;
      uint32_t w[4];
#pragma unroll
      for (int c = 0; c < 8; c += 2)
        w[c / 2] = (uint32_t)to_bf(e * qs[r][c] + pu[r][c]) | ((uint32_t)to_bf(e * qs[r][c + 1] + pu[r][c + 1]) << 16);
      *reinterpret_cast<uint4*>(orow) = make_uint4(w[0], w[1], w[2], w[3]);
    }
  }
}

// ---- backward: the state gradient swept back over chunks -------------------------------
// One workgroup per (sequence, 32 columns of dS), chunks in reverse:
//   dSn_n = dS;  dU = P' dO + diag(e^(last - ca)) K dS;  dS <- Qg' dO + g dS - W' dU,
// the products on the matrix cores in fp32.  While a chunk's products run,
// the previous chunk's inputs (P, the dO columns, Q, K, W, ca) are loaded
// into registers; they go to LDS once the chunk is done with its own.

constexpr int kLdC = 68;   // LDS row of 64 fp32
constexpr int kLdS = 36;   // LDS row of 32 fp32
constexpr size_t kSgLds =
    (kC * kLdC + kC * kLdS + 3 * kC * kLd + kD * kLdS + kC * kLdS + kC) * sizeof(float);

typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));

// One chunk's inputs as this thread loads them (plain vector types, so the
// whole set stays in registers).
struct SgInputs {
  f32x4v p[4];     // P: 4 x 16 bytes
  u32x2v d[2];     // dO columns col0 .. col0 + 31: 2 x 8 bytes (bf16)
  u32x4v q[4], k[4];  // Q, K: 4 x 16 bytes each (bf16)
  f32x4v w[8];
  float ca;
};

__device__ __forceinline__ void sg_load(SgInputs& in, const DnArgs& p, const Chunk& ck, int col0) {
  const int t = threadIdx.x;
  const float* Pc = p.P + ck.c * kC * kC;
  const float* Wc = p.W + ck.c * kC * kD;
#pragma unroll
  for (int e = 0; e < 4; ++e) in.p[e] = reinterpret_cast<const f32x4v*>(Pc)[t + 256 * e];
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int x = t + 256 * e, r = x / 8, c = 4 * (x % 8);
    in.d[e] = *reinterpret_cast<const u32x2v*>(p.dout + ck.row0 + (int64_t)r * p.s_t + col0 + c);
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int x = t + 256 * e, r = x / 16, c = 8 * (x % 16);
    in.q[e] = *reinterpret_cast<const u32x4v*>(p.q + ck.row0 + (int64_t)r * p.s_t + c);
    in.k[e] = *reinterpret_cast<const u32x4v*>(p.k + ck.row0 + (int64_t)r * p.s_t + c);
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) in.w[e] = reinterpret_cast<const f32x4v*>(Wc)[t + 256 * e];
  in.ca = t < kC ? p.ca[ck.c * kC + t] : 0.0f;
}

// The inputs to LDS; Q as Qg = diag(e^ca) Q (ca of the same chunk, already in LDS).
__device__ __forceinline__ void sg_store(const SgInputs& in, float* P, float* dO, float* Qg, float* K, float* W,
                                         const float* ca) {
  const int t = threadIdx.x;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int x = t + 256 * e, r = x / 16, c = 4 * (x % 16);
    *reinterpret_cast<f32x4v*>(P + r * kLdC + c) = in.p[e];
  }
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int x = t + 256 * e, r = x / 8, c = 4 * (x % 8);
    *reinterpret_cast<f32x4v*>(dO + r * kLdS + c) =
        f32x4v{bf((uint16_t)in.d[e][0]), bf((uint16_t)(in.d[e][0] >> 16)), bf((uint16_t)in.d[e][1]),
               bf((uint16_t)(in.d[e][1] >> 16))};
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int x = t + 256 * e, r = x / 16, c = 8 * (x % 16);
    const float eq = expf(ca[r]);
    const u32x4v uq = in.q[e], uk = in.k[e];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      Qg[r * kLd + c + 2 * j] = eq * bf((uint16_t)uq[j]);
      Qg[r * kLd + c + 2 * j + 1] = eq * bf((uint16_t)(uq[j] >> 16));
      K[r * kLd + c + 2 * j] = bf((uint16_t)uk[j]);
      K[r * kLd + c + 2 * j + 1] = bf((uint16_t)(uk[j] >> 16));
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int x = t + 256 * e, r = x / 32, c = 4 * (x % 32);
    *reinterpret_cast<f32x4v*>(W + r * kLd + c) = in.w[e];
  }
}

__global__ __launch_bounds__(256, 1) void dn_state_grad(DnArgs p) {
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
  const int64_t seq = blockIdx.x / (kD / kCols);
  const int col0 = (blockIdx.x % (kD / kCols)) * kCols;
  for (int e = t; e < kD * kLdS; e += 256) dS[e] = 0.0f;
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
    if (n > 0) sg_load(in, p, chunk_of(p, seq * p.chunks + n - 1), col0);
    const float last = ca[kC - 1];
    // The gradient at the chunk's end state.
    float* dSc = p.dSn + ck.c * kD * kD;
    for (int e = t; e < kD * kCols / 4; e += 256) {
      const int row = e / 8, c = 4 * (e % 8);
      *reinterpret_cast<float4*>(dSc + row * kD + col0 + c) = *reinterpret_cast<const float4*>(dS + row * kLdS + c);
    }
    // dU (64 x 32): wave w takes rows 16 w .. 16 w + 15.
    {
      f32x4v pd[1][2], kd[1][2];
      clear(pd);
      clear(kd);
      mm_gen<true, true>(pd, P, kLdC, 16 * w, dO, kLdS, 0, kC);
      mm_gen<false, true>(kd, K, kLd, 16 * w, dS, kLdS, 0, kD);
      float* dUo = p.dU + ck.c * kC * kD;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int i = 16 * w + 4 * g + v;
        const float e = expf(last - ca[i]);
#pragma unroll
        for (int bj = 0; bj < 2; ++bj) {
          const float u = pd[0][bj][v] + e * kd[0][bj][v];
          dU[i * kLdS + 16 * bj + r] = u;
          dUo[i * kD + col0 + 16 * bj + r] = u;
        }
      }
    }
    __syncthreads();
    // dS <- Qg' dO + g dS - W' dU (128 x 32): wave w takes rows 32 w .. 32 w + 31.
    {
      f32x4v qd[2][2], wu[2][2];
      clear(qd);
      clear(wu);
      mm_gen<true, true>(qd, Qg, kLd, 32 * w, dO, kLdS, 0, kC);
      mm_gen<true, true>(wu, W, kLd, 32 * w, dU, kLdS, 0, kC);
      const float gl = expf(last);
      float nw[2][2][4];
#pragma unroll
      for (int bi = 0; bi < 2; ++bi)
#pragma unroll
        for (int bj = 0; bj < 2; ++bj)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int i = 32 * w + 16 * bi + 4 * g + v, j = 16 * bj + r;
            nw[bi][bj][v] = qd[bi][bj][v] + gl * dS[i * kLdS + j] - wu[bi][bj][v];
          }
      __syncthreads();  // every wave has read dS, dU and this chunk's inputs
#pragma unroll
      for (int bi = 0; bi < 2; ++bi)
#pragma unroll
        for (int bj = 0; bj < 2; ++bj)
#pragma unroll
          for (int v = 0; v < 4; ++v) dS[(32 * w + 16 * bi + 4 * g + v) * kLdS + 16 * bj + r] = nw[bi][bj][v];
    }
    if (n > 0) {
      if (t < kC) ca[t] = in.ca;
      __syncthreads();
      sg_store(in, P, dO, Qg, K, W, ca);
    }
  }
}

// ---- backward: the chunk's products (part a) ---------------------------------------
// dQg = dO S', dW = -dU S', dKd = U dSn', dP = lower(dO U'), dg = <S, dSn>,
// every product on the matrix cores in fp32.  Two phases through LDS: dO, dU
// and S, then U and dSn (dO stays).  Wave w computes columns 32 w .. 32 w + 31
// of the 64 x 128 results and row block w of dP.

constexpr size_t kGaLds = (2 * kC + kD) * kLd * sizeof(float) + 4 * sizeof(float);

__global__ __launch_bounds__(256, 1) void dn_grad_a(DnArgs p) {
  extern __shared__ float lds[];
  float* dO = lds;              // [64][kLd]
  float* X = dO + kC * kLd;     // [64][kLd]: dU, then U
  float* Y = X + kC * kLd;      // [128][kLd]: S, then dSn
  float* red = Y + kD * kLd;    // [4]
  const Chunk ck = chunk_of(p, blockIdx.x);
  const int t = threadIdx.x, w = t / 64;
  const float* Sc = p.S + ck.c * kD * kD;
  const float* dSc = p.dSn + ck.c * kD * kD;
  stage_bf16(dO, p.dout + ck.row0, p.s_t);
  stage_f32(X, p.dU + ck.c * kC * kD, kC);
  stage_f32(Y, Sc, kD);
  __syncthreads();
  {
    f32x4v q[4][2], wq[4][2];
    clear(q);
    clear(wq);
    mm_nt(q, dO, 0, Y, 32 * w, kD);
    mm_nt(wq, X, 0, Y, 32 * w, kD);
    store_blocks(p.dQg + ck.c * kC * kD, kD, q, 0, 32 * w, 1.0f);
    store_blocks(p.dW + ck.c * kC * kD, kD, wq, 0, 32 * w, -1.0f);
  }
  __syncthreads();
  stage_f32(X, p.U + ck.c * kC * kD, kC);
  stage_f32(Y, dSc, kD);
  __syncthreads();
  {
    f32x4v kd[4][2];
    clear(kd);
    mm_nt(kd, X, 0, Y, 32 * w, kD);
    store_blocks(p.dKd + ck.c * kC * kD, kD, kd, 0, 32 * w, 1.0f);
  }
  {
    // Row block w of dP: blocks (w, jb) for jb <= w, the diagonal masked, zeros above.
    const int r = t % 16, g = (t % 64) / 16;
    float* dPc = p.dP + ck.c * kC * kC;
    for (int jb = 0; jb < 4; ++jb) {
      f32x4v acc[1][1];
      clear(acc);
      if (jb <= w) mm_nt(acc, dO, 16 * w, X, 16 * jb, kD);
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int i = 16 * w + 4 * g + v, j = 16 * jb + r;
        dPc[i * kC + j] = i >= j ? acc[0][0][v] : 0.0f;
      }
    }
  }
  // dg = <S, dSn>: S from global, dSn from LDS, a fixed tree.
  float sum = 0.0f;
  for (int e = t; e < kD * kD / 4; e += 256) {
    const int r = e / 32, c = 4 * (e % 32);
    const float4 sv = *reinterpret_cast<const float4*>(Sc + r * kD + c);
    const f32x4v dv = quad(Y + r * kLd + c);
    sum = fmaf(sv.x, dv[0], sum);
    sum = fmaf(sv.y, dv[1], sum);
    sum = fmaf(sv.z, dv[2], sum);
    sum = fmaf(sv.w, dv[3], sum);
  }
  sum = thd::wave_sum(sum);
  if (t % 64 == 0) red[t / 64] = sum;
  __syncthreads();
  if (t == 0) p.dg[ck.c] = red[0] + red[1] + red[2] + red[3];
}

// ---- backward: the chunk's WY form, decays and gates (part b) -----------------------

// Q and K sit in LDS as bf16 (their exact values), V is read from global
// where it is needed; per-row partial sums of the gate gradients go to LDS
// by column group and are folded in a fixed order, so the result does not
// depend on timing.
constexpr int kPadH = kD + 8;   // bf16 row of Q, K
constexpr int kGroups = 16;     // column groups of the 4 x 4 and 4 x 8 micro-tiles
constexpr size_t kGbLds = 2 * kC * kPadH * sizeof(uint16_t) + (4 * kC * kPadC + 7 * kC * kGroups + 2 * kC) * sizeof(float);

__global__ __launch_bounds__(256) void dn_grad_b(DnArgs p) {
  extern __shared__ float lds[];
  uint16_t* Qh = reinterpret_cast<uint16_t*>(lds);   // [64][kPadH]
  uint16_t* Kh = Qh + kC * kPadH;                   // [64][kPadH]
  float* T = reinterpret_cast<float*>(Kh + kC * kPadH);  // [64][kPadC]
  float* M = T + kC * kPadC;      // [64][kPadC]: dT, then dA
  float* N = M + kC * kPadC;      // [64][kPadC]: T' dT, then dG
  float* R = N + kC * kPadC;      // [64][kPadC]: dQK = dP o Gamma
  float* wrow = R + kC * kPadC;   // [64][16]: partial sums of w over j, by column group
  float* wcol = wrow + kC * kGroups;  // [64][16]: partial sums of w over i, by row group
  float* brow = wcol + kC * kGroups;  // [64][16]: dA Gamma G over j
  float* kx = brow + kC * kGroups;    // [64][16]: k . dX by column group
  float* vy = kx + kC * kGroups;      // [64][16]: v . dY
  float* qq = vy + kC * kGroups;      // [64][16]: q . dQg
  float* kk = qq + kC * kGroups;      // [64][16]: k . dKd
  float* ca = kk + kC * kGroups;      // [64]
  float* be = ca + kC;                // [64]
  const Chunk ck = chunk_of(p, blockIdx.x);
  const int t = threadIdx.x;
  const uint16_t* qg = p.q + ck.row0;
  const uint16_t* kg = p.k + ck.row0;
  const uint16_t* vg = p.v + ck.row0;
  for (int e = t; e < kC * (kD / 8); e += 256) {
    const int r = e / (kD / 8), c8 = (e % (kD / 8)) * 8;
    *reinterpret_cast<uint4*>(Qh + r * kPadH + c8) = *reinterpret_cast<const uint4*>(qg + r * p.s_t + c8);
    *reinterpret_cast<uint4*>(Kh + r * kPadH + c8) = *reinterpret_cast<const uint4*>(kg + r * p.s_t + c8);
  }
  const float* Tc = p.T + ck.c * kC * kC;
  for (int e = t; e < kC * kC; e += 256) T[(e / kC) * kPadC + e % kC] = Tc[e];
  if (t < 64) {
    ca[t] = p.ca[ck.c * kC + t];
    be[t] = p.beta[ck.grow0 + (int64_t)t * p.g_t];
  }
  __syncthreads();
  auto Q = [&](int i, int d) { return bf(Qh[i * kPadH + d]); };
  auto K = [&](int i, int d) { return bf(Kh[i * kPadH + d]); };
  auto V = [&](int i, int d) { return bf(vg[(int64_t)i * p.s_t + d]); };
  const float* dW = p.dW + ck.c * kC * kD;
  const float* dUt = p.dU + ck.c * kC * kD;
  const float* dQg = p.dQg + ck.c * kC * kD;
  const float* dKd = p.dKd + ck.c * kC * kD;
  const float* dP = p.dP + ck.c * kC * kC;
  const float last = ca[kC - 1];
  // dT = dW X' + dU~ Y',  X = diag(beta e^ca) K, Y = diag(beta) V.
  {
    const int i0 = 4 * (t / 16), j0 = 4 * (t % 16);
    float acc[4][4], acc2[4][4];
    zero(acc);
    zero(acc2);
    mm(acc, i0, j0, kD, [&](int i, int k) { return dW[i * kD + k]; }, [&](int k, int l) { return K(l, k); });
    mm(acc2, i0, j0, kD, [&](int i, int k) { return dUt[i * kD + k]; }, [&](int k, int l) { return V(l, k); });
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int l = j0 + c;
        M[(i0 + r) * kPadC + l] = be[l] * (expf(ca[l]) * acc[r][c] + acc2[r][c]);
      }
  }
  __syncthreads();
  // N = T' dT.
  {
    const int i0 = 4 * (t / 16), j0 = 4 * (t % 16);
    float acc[4][4];
    zero(acc);
    mm(acc, i0, j0, kC, [&](int i, int l) { return T[l * kPadC + i]; }, [&](int l, int j) { return M[l * kPadC + j]; });
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int c = 0; c < 4; ++c) N[(i0 + r) * kPadC + j0 + c] = acc[r][c];
  }
  __syncthreads();
  // dA = -(N T') o strict lower (into M);  dQK = dP o Gamma, lower (into R).
  {
    const int i0 = 4 * (t / 16), j0 = 4 * (t % 16);
    float acc[4][4];
    zero(acc);
    mm(acc, i0, j0, kC, [&](int i, int l) { return N[i * kPadC + l]; }, [&](int l, int j) { return T[j * kPadC + l]; });
    __syncthreads();  // N is read above and rewritten below
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int i = i0 + r, j = j0 + c;
        M[i * kPadC + j] = i > j ? -acc[r][c] : 0.0f;
        R[i * kPadC + j] = i >= j ? dP[i * kC + j] * expf(ca[i] - ca[j]) : 0.0f;
      }
  }
  __syncthreads();
  // With G = K K', QK = Q K', Gamma: dG = dA o beta_i o Gamma (into N);
  // dbeta_i gets sum_j dA Gamma G; w = (dA beta_i G + dP QK) o Gamma gives
  // dca_i += sum_j w_ij - sum_j w_ji.
  {
    const int i0 = 4 * (t / 16), j0 = 4 * (t % 16);
    float g[4][4], qk[4][4];
    zero(g);
    zero(qk);
    if (j0 < i0 + 4) {
      mm(g, i0, j0, kD, [&](int i, int k) { return K(i, k); }, [&](int k, int j) { return K(j, k); });
      mm(qk, i0, j0, kD, [&](int i, int k) { return Q(i, k); }, [&](int k, int j) { return K(j, k); });
    }
    float colw[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = i0 + r;
      float rowb = 0.0f, roww = 0.0f;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int j = j0 + c;
        const float gam = expf(ca[i] - ca[j]);
        const float dA = M[i * kPadC + j];
        N[i * kPadC + j] = dA * be[i] * gam;
        rowb += dA * gam * g[r][c];
        const float w = i >= j ? (dA * be[i] * g[r][c] + dP[i * kC + j] * qk[r][c]) * gam : 0.0f;
        roww += w;
        colw[c] += w;
      }
      wrow[i * kGroups + t % 16] = roww;
      brow[i * kGroups + t % 16] = rowb;
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) wcol[(j0 + c) * kGroups + t / 16] = colw[c];
  }
  __syncthreads();
  // dQ = e^ca dQg + dQK K;  dK = dQK' Q + (dG + dG') K + beta e^ca dX + e^(last - ca) dKd;
  // dX = T' dW;  dV = beta T' dU~.
  {
    const int i0 = 4 * (t / 16), j0 = 8 * (t % 16);
    float dq[4][8], dk[4][8], dx[4][8], dy[4][8];
    zero(dq);
    zero(dk);
    zero(dx);
    zero(dy);
    mm(dq, i0, j0, kC, [&](int i, int l) { return R[i * kPadC + l]; }, [&](int l, int d) { return K(l, d); });
    mm(dk, i0, j0, kC, [&](int i, int l) { return R[l * kPadC + i]; }, [&](int l, int d) { return Q(l, d); });
    mm(dk, i0, j0, kC, [&](int i, int l) { return N[i * kPadC + l] + N[l * kPadC + i]; }, [&](int l, int d) { return K(l, d); });
    mm(dx, i0, j0, kC, [&](int i, int l) { return T[l * kPadC + i]; }, [&](int l, int d) { return dW[l * kD + d]; });
    mm(dy, i0, j0, kC, [&](int i, int l) { return T[l * kPadC + i]; }, [&](int l, int d) { return dUt[l * kD + d]; });
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = i0 + r;
      const float e = expf(ca[i]), ed = expf(last - ca[i]);
      float skx = 0.0f, svy = 0.0f, sqq = 0.0f, skk = 0.0f;
      uint32_t wq[4], wk[4], wv[4];
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const int d = j0 + c;
        const float gq = dQg[i * kD + d], gk = dKd[i * kD + d];
        const float vq = e * gq + dq[r][c];
        const float vk = dk[r][c] + be[i] * e * dx[r][c] + ed * gk;
        const float vv = be[i] * dy[r][c];
        skx = fmaf(K(i, d), dx[r][c], skx);
        svy = fmaf(V(i, d), dy[r][c], svy);
        sqq = fmaf(Q(i, d), gq, sqq);
        skk = fmaf(K(i, d), gk, skk);
        const uint32_t hq = to_bf(vq), hk = to_bf(vk), hv = to_bf(vv);
        if (c % 2 == 0) {
          wq[c / 2] = hq, wk[c / 2] = hk, wv[c / 2] = hv;
        } else {
          wq[c / 2] |= hq << 16, wk[c / 2] |= hk << 16, wv[c / 2] |= hv << 16;
        }
      }
      const int64_t at = ck.row0 + (int64_t)i * p.s_t + j0;
      *reinterpret_cast<uint4*>(p.dq + at) = make_uint4(wq[0], wq[1], wq[2], wq[3]);
      *reinterpret_cast<uint4*>(p.dk + at) = make_uint4(wk[0], wk[1], wk[2], wk[3]);
      *reinterpret_cast<uint4*>(p.dv + at) = make_uint4(wv[0], wv[1], wv[2], wv[3]);
      kx[i * kGroups + t % 16] = skx;
      vy[i * kGroups + t % 16] = svy;
      qq[i * kGroups + t % 16] = sqq;
      kk[i * kGroups + t % 16] = skk;
    }
  }
  __syncthreads();
  // Fold the partials in a fixed order (lane i: row i), then da = the
  // reverse cumulative sum of dca, dca_63 also taking sum kd + dg g.
  if (t < 64) {
    const int i = t;
    float sw = 0.0f, sc = 0.0f, sb = 0.0f, skx = 0.0f, svy = 0.0f, sqq = 0.0f, skk = 0.0f;
    for (int gi = 0; gi < kGroups; ++gi) {
      sw += wrow[i * kGroups + gi];
      sc += wcol[i * kGroups + gi];
      sb += brow[i * kGroups + gi];
      skx += kx[i * kGroups + gi];
      svy += vy[i * kGroups + gi];
      sqq += qq[i * kGroups + gi];
      skk += kk[i * kGroups + gi];
    }
    const float e = expf(ca[i]), ed = expf(last - ca[i]);
    const float kd = ed * skk;
    float dca = sw - sc + be[i] * e * skx + e * sqq - kd;
    float kd_all = kd;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) kd_all += __shfl_xor(kd_all, o, 64);
    if (i == kC - 1) dca += kd_all + p.dg[ck.c] * expf(last);
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
                            (size_t)kC * kD, (size_t)kC * kD, (size_t)kC * kC, 1};
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
  TH_REQUIRE(d->q && d->k && d->v && d->a && d->beta && d->o, "deltanet: null q, k, v, a, beta or o");
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
  void* ws = nullptr;
  if (int r = th::device_alloc(w.bytes, &ws)) return r;
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
  char* base = static_cast<char*>(ws);
  float** slots[14] = {&a.ca, &a.T, &a.W, &a.Ut, &a.S, &a.U, &a.P, &a.dU, &a.dSn, &a.dQg, &a.dW, &a.dKd, &a.dP, &a.dg};
  for (int i = 0; i < 14; ++i) *slots[i] = (i < 7 || backward) ? reinterpret_cast<float*>(base + w.offs[i]) : nullptr;
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
  b.own(ws);
  const unsigned nchunks = (unsigned)chunks;
  const unsigned scans = (unsigned)((int64_t)d->batch * d->heads * (kD / kCols));
  int ks[6];
  int nk = 0;
  ks[nk++] = b.kernel(fns[0], "dn_chunk_prep", dim3(nchunks), dim3(256), (uint32_t)kPrepLds, a);
  ks[nk++] = b.kernel(fns[1], "dn_state_scan", dim3(scans), dim3(256), (uint32_t)kScanLds, a);
  ks[nk++] = b.kernel(fns[2], "dn_output", dim3(nchunks), dim3(256), (uint32_t)kOutLds, a);
  if (backward) {
    ks[nk++] = b.kernel(fns[3], "dn_state_grad", dim3(scans), dim3(256), (uint32_t)kSgLds, a);
    ks[nk++] = b.kernel(fns[4], "dn_grad_a", dim3(nchunks), dim3(256), (uint32_t)kGaLds, a);
    ks[nk++] = b.kernel(fns[5], "dn_grad_b", dim3(nchunks), dim3(256), (uint32_t)kGbLds, a);
  }
  const size_t offs[12] = {TH_OFFSET(DnArgs, q),  TH_OFFSET(DnArgs, k),  TH_OFFSET(DnArgs, v),     TH_OFFSET(DnArgs, a),
                           TH_OFFSET(DnArgs, beta), TH_OFFSET(DnArgs, o), TH_OFFSET(DnArgs, dout), TH_OFFSET(DnArgs, dq),
                           TH_OFFSET(DnArgs, dk), TH_OFFSET(DnArgs, dv), TH_OFFSET(DnArgs, da),  TH_OFFSET(DnArgs, dbeta)};
  for (int v = 0; v < 12; ++v)
    for (int i = 0; i < nk; ++i) b.ref(v, ks[i], offs[v]);
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
