// Op class (c), general shapes: attention forward and backward for any head
// dimension up to 256, any sequence lengths (keys may be fewer or more than
// queries), fp32 or bf16 arrays, grouped heads, and the masks the device
// holds (a first key per query, a key count per sequence).  What the
// matrix-core kernels of attention.hip do not take runs here: the reference's
// cuDNN claim covers d <= 256 (ext/cuDNNExt.jl:95-100) and its tests use
// D = 4, 8, 16, 32 at odd lengths, packed documents and decode over a cache
// (test/fixtures/programs.jl:110-113, test/cuda/attention.jl:10-16,218-271).
//
// Everything computes in fp32 on the vector ALUs from fp32 copies of the
// tiles in LDS (rows padded by one float, so that the lanes reading one
// column of 16 rows hit 16 banks):
//   forward: a workgroup per (64 queries, head, batch) sweeps key tiles of
//   32 with the online softmax (the running maximum rebased by
//   exp(m_old - m_new), folds.jl:186-222), O = P V / l, lse = m + log(l);
//   backward (FA2's formulas, deterministic): delta = rowsum(dO .* O); a
//   workgroup per (32 keys, key/value head, batch) sweeps the query tiles of
//   each query head of its group for dK and dV; a workgroup per (queries,
//   head, batch) sweeps the key tiles for dQ.  P is recomputed from lse in both.
#include <hip/hip_runtime.h>

#include <cmath>

#include "th_core.h"

namespace {

struct GenArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  float* lse;
  const void* dout;
  void* dq;
  void* dk;
  void* dv;
  const int32_t* starts;   // (positions, batch), 1-based, or null
  const int32_t* lengths;  // (batch), or null
  float* delta;            // backward workspace: rowsum(dO .* O), [b][s][h]
  int64_t q_sh, q_ss, q_sb;
  int64_t k_sh, k_ss, k_sb;
  int32_t seq, kv_seq, heads, kv_heads, batch, d;
  int32_t causal;
  float scale;
};

template <bool F32>
struct Elem;
template <>
struct Elem<true> {
  __device__ static float load(const void* p, int64_t i) { return static_cast<const float*>(p)[i]; }
  __device__ static void store(void* p, int64_t i, float x) { static_cast<float*>(p)[i] = x; }
};
template <>
struct Elem<false> {
  __device__ static float load(const void* p, int64_t i) {
    return __uint_as_float((uint32_t) static_cast<const uint16_t*>(p)[i] << 16);
  }
  __device__ static void store(void* p, int64_t i, float x) {
    static_cast<uint16_t*>(p)[i] = __builtin_bit_cast(uint16_t, (__bf16)x);
  }
};

// The keys of sequence b: lengths[b] clamped to the keys' extent.
__device__ __forceinline__ int keys_of(const GenArgs& p, int b) {
  if (!p.lengths) return p.kv_seq;
  const int n = p.lengths[b];
  return n < 0 ? 0 : (n > p.kv_seq ? p.kv_seq : n);
}

// The first key query j of batch b sees (0-based).
__device__ __forceinline__ int first_of(const GenArgs& p, int j, int b) {
  return p.starts ? p.starts[(int64_t)j + (int64_t)p.seq * b] - 1 : 0;
}

// Rows of `n` positions starting at `row0` of a (d, position) operand into
// LDS as fp32 rows of `ld` floats; positions past `limit` read as zero.
template <bool F32>
__device__ __forceinline__ void stage(float* dst, int ld, const void* base, int64_t ss, int row0, int n, int limit,
                                      int d) {
  for (int i = threadIdx.x; i < n * d; i += blockDim.x) {
    const int r = i / d, c = i % d;
    const int pos = row0 + r;
    dst[r * ld + c] = pos < limit ? Elem<F32>::load(base, (int64_t)pos * ss + c) : 0.0f;
  }
}

// ---- forward ---------------------------------------------------------------------
// 256 threads: thread t owns query t / 4 of the tile; in the score phase its
// keys r, r + 4, ... (r = t % 4) of the key tile, in the product phase its
// features r, r + 4, ... of the query's output.

constexpr int kGQ = 64;  // queries per forward workgroup
constexpr int kGK = 32;  // keys per step

template <bool F32, int DP>
__global__ __launch_bounds__(256) void attn_gen_fwd(GenArgs p) {
  extern __shared__ float sm[];
  constexpr int LD = DP + 1;
  float* Qs = sm;                 // kGQ x LD
  float* Ks = Qs + kGQ * LD;      // kGK x LD
  float* Vs = Ks + kGK * LD;      // kGK x LD
  float* Ps = Vs + kGK * LD;      // kGQ x (kGK + 1)
  int* lo = reinterpret_cast<int*>(Ps + kGQ * (kGK + 1));
  const int q0 = blockIdx.x * kGQ, h = blockIdx.y, b = blockIdx.z;
  const int hk = h / (p.heads / p.kv_heads);
  const int t = threadIdx.x, qi = t / 4, r = t % 4;
  const int j = q0 + qi;  // this thread's query
  const int d = p.d;
  const int64_t qoff = (int64_t)b * p.q_sb + (int64_t)h * p.q_sh;
  const int64_t koff = (int64_t)b * p.k_sb + (int64_t)hk * p.k_sh;
  const int nk = keys_of(p, b);
  const int first = j < p.seq ? first_of(p, j, b) : 0;
  // The tile's keys: from the least first key of its queries to the last
  // visible to its last query.
  if (t == 0) lo[0] = 1 << 30;
  __syncthreads();
  if (r == 0 && j < p.seq) atomicMin(&lo[0], first);
  const int q_last = min(q0 + kGQ, p.seq) - 1;
  const int k_end = p.causal ? min(nk, q_last + 1) : nk;
  if constexpr (F32) {
    stage<F32>(Qs, LD, static_cast<const float*>(p.q) + qoff, p.q_ss, q0, kGQ, p.seq, d);
  } else {
    stage<F32>(Qs, LD, static_cast<const uint16_t*>(p.q) + qoff, p.q_ss, q0, kGQ, p.seq, d);
  }
  __syncthreads();
  const int k_begin = max(0, lo[0]) / kGK * kGK;
  constexpr int NO = DP / 4;
  float acc[NO];
#pragma unroll
  for (int i = 0; i < NO; ++i) acc[i] = 0.0f;
  float m = -INFINITY, l = 0.0f;
  const float sc = p.scale;
  for (int k0 = k_begin; k0 < k_end; k0 += kGK) {
    __syncthreads();  // the previous step's K, V and P are read
    if constexpr (F32) {
      stage<F32>(Ks, LD, static_cast<const float*>(p.k) + koff, p.k_ss, k0, kGK, nk, d);
      stage<F32>(Vs, LD, static_cast<const float*>(p.v) + koff, p.k_ss, k0, kGK, nk, d);
    } else {
      stage<F32>(Ks, LD, static_cast<const uint16_t*>(p.k) + koff, p.k_ss, k0, kGK, nk, d);
      stage<F32>(Vs, LD, static_cast<const uint16_t*>(p.v) + koff, p.k_ss, k0, kGK, nk, d);
    }
    __syncthreads();
    float s[kGK / 4];
#pragma unroll
    for (int e = 0; e < kGK / 4; ++e) s[e] = 0.0f;
    for (int c = 0; c < d; ++c) {
      const float x = Qs[qi * LD + c];
#pragma unroll
      for (int e = 0; e < kGK / 4; ++e) s[e] = fmaf(x, Ks[(r + 4 * e) * LD + c], s[e]);
    }
    float mt = -INFINITY;
#pragma unroll
    for (int e = 0; e < kGK / 4; ++e) {
      const int key = k0 + r + 4 * e;
      const bool seen = j < p.seq && key < nk && key >= first && (!p.causal || key <= j);
      s[e] = seen ? s[e] * sc : -INFINITY;
      mt = fmaxf(mt, s[e]);
    }
    mt = fmaxf(mt, __shfl_xor(mt, 1, 64));
    mt = fmaxf(mt, __shfl_xor(mt, 2, 64));
    const float mn = fmaxf(m, mt);
    // lse_shift: an all -inf maximum shifts by zero (folds.jl:194).
    const float shift = __builtin_isfinite(mn) ? mn : 0.0f;
    const float corr = expf(m - shift);
    float ls = 0.0f;
#pragma unroll
    for (int e = 0; e < kGK / 4; ++e) {
      const float w = expf(s[e] - shift);
      ls += w;
      Ps[qi * (kGK + 1) + r + 4 * e] = w;
    }
    ls += __shfl_xor(ls, 1, 64);
    ls += __shfl_xor(ls, 2, 64);
    l = l * corr + ls;
    m = mn;
#pragma unroll
    for (int i = 0; i < NO; ++i) acc[i] *= corr;
    __syncthreads();
    for (int e = 0; e < kGK; ++e) {
      const float w = Ps[qi * (kGK + 1) + e];
#pragma unroll
      for (int i = 0; i < NO; ++i) acc[i] = fmaf(w, Vs[e * LD + r + 4 * i], acc[i]);
    }
  }
  if (j >= p.seq) return;
  const float inv = 1.0f / l;
  const int64_t at = qoff + (int64_t)j * p.q_ss;
#pragma unroll
  for (int i = 0; i < NO; ++i) {
    const int c = r + 4 * i;
    if (c < d) Elem<F32>::store(p.o, at + c, acc[i] * inv);
  }
  if (p.lse && r == 0) {
    const float shift = __builtin_isfinite(m) ? m : 0.0f;
    p.lse[((int64_t)b * p.seq + j) * p.heads + h] = shift + logf(l);
  }
}

// ---- backward: delta = rowsum(dO .* O) ------------------------------------------

template <bool F32>
__global__ __launch_bounds__(256) void attn_gen_delta(GenArgs p) {
  const int64_t row = (int64_t)blockIdx.x * 4 + threadIdx.x / 64;  // [b][s][h]
  const int64_t total = (int64_t)p.batch * p.seq * p.heads;
  if (row >= total) return;
  const int h = (int)(row % p.heads);
  const int64_t s = (row / p.heads) % p.seq, b = row / ((int64_t)p.heads * p.seq);
  const int64_t at = b * p.q_sb + h * p.q_sh + s * p.q_ss;
  float v = 0.0f;
  for (int c = threadIdx.x % 64; c < p.d; c += 64) v += Elem<F32>::load(p.o, at + c) * Elem<F32>::load(p.dout, at + c);
  v = thd::wave_sum(v);
  if (threadIdx.x % 64 == 0) p.delta[row] = v;
}

// ---- backward: dK, dV for 32 keys ----------------------------------------------
// Thread t owns key t / 8 of the tile: in the score phase its queries
// r, r + 8, ... (r = t % 8) of the query tile, in the product phase its
// features r, r + 8, ... of dK and dV.

constexpr int kGBK = 32;  // keys per dK/dV workgroup

template <bool F32, int DP>
__global__ __launch_bounds__(256) void attn_gen_dkdv(GenArgs p) {
  extern __shared__ float sm[];
  constexpr int LD = DP + 1;
  constexpr int BQ = DP <= 128 ? 64 : 32;  // queries per step
  float* Ks = sm;                   // kGBK x LD
  float* Vs = Ks + kGBK * LD;       // kGBK x LD
  float* Qs = Vs + kGBK * LD;       // BQ x LD
  float* Gs = Qs + BQ * LD;         // BQ x LD (dO)
  float* Pt = Gs + BQ * LD;         // kGBK x (BQ + 1): P'
  float* St = Pt + kGBK * (BQ + 1); // kGBK x (BQ + 1): dS'
  float* Ls = St + kGBK * (BQ + 1); // BQ: lse
  float* Ds = Ls + BQ;              // BQ: delta
  const int k0 = blockIdx.x * kGBK, hk = blockIdx.y, b = blockIdx.z;
  const int group = p.heads / p.kv_heads;
  const int t = threadIdx.x, ki = t / 8, r = t % 8;
  const int key = k0 + ki;
  const int d = p.d;
  const int nk = keys_of(p, b);
  const int64_t koff = (int64_t)b * p.k_sb + (int64_t)hk * p.k_sh;
  constexpr int NO = DP / 8;
  float dk[NO], dv[NO];
#pragma unroll
  for (int i = 0; i < NO; ++i) dk[i] = dv[i] = 0.0f;
  if (k0 < nk) {
    if constexpr (F32) {
      stage<F32>(Ks, LD, static_cast<const float*>(p.k) + koff, p.k_ss, k0, kGBK, nk, d);
      stage<F32>(Vs, LD, static_cast<const float*>(p.v) + koff, p.k_ss, k0, kGBK, nk, d);
    } else {
      stage<F32>(Ks, LD, static_cast<const uint16_t*>(p.k) + koff, p.k_ss, k0, kGBK, nk, d);
      stage<F32>(Vs, LD, static_cast<const uint16_t*>(p.v) + koff, p.k_ss, k0, kGBK, nk, d);
    }
    const float sc = p.scale;
    const int q_begin = p.causal ? k0 / BQ * BQ : 0;
    for (int h = hk * group; h < (hk + 1) * group; ++h) {
      const int64_t qoff = (int64_t)b * p.q_sb + (int64_t)h * p.q_sh;
      for (int q0 = q_begin; q0 < p.seq; q0 += BQ) {
        __syncthreads();  // the previous step's tiles are read
        if constexpr (F32) {
          stage<F32>(Qs, LD, static_cast<const float*>(p.q) + qoff, p.q_ss, q0, BQ, p.seq, d);
          stage<F32>(Gs, LD, static_cast<const float*>(p.dout) + qoff, p.q_ss, q0, BQ, p.seq, d);
        } else {
          stage<F32>(Qs, LD, static_cast<const uint16_t*>(p.q) + qoff, p.q_ss, q0, BQ, p.seq, d);
          stage<F32>(Gs, LD, static_cast<const uint16_t*>(p.dout) + qoff, p.q_ss, q0, BQ, p.seq, d);
        }
        for (int i = t; i < BQ; i += 256) {
          const int j = q0 + i;
          const int64_t row = ((int64_t)b * p.seq + j) * p.heads + h;
          Ls[i] = j < p.seq ? p.lse[row] : 0.0f;
          Ds[i] = j < p.seq ? p.delta[row] : 0.0f;
        }
        __syncthreads();
        constexpr int NS = BQ / 8;
        float s[NS], g[NS];
#pragma unroll
        for (int e = 0; e < NS; ++e) s[e] = g[e] = 0.0f;
        for (int c = 0; c < d; ++c) {
          const float kx = Ks[ki * LD + c], vx = Vs[ki * LD + c];
#pragma unroll
          for (int e = 0; e < NS; ++e) {
            s[e] = fmaf(kx, Qs[(r + 8 * e) * LD + c], s[e]);
            g[e] = fmaf(vx, Gs[(r + 8 * e) * LD + c], g[e]);
          }
        }
#pragma unroll
        for (int e = 0; e < NS; ++e) {
          const int qi = r + 8 * e, j = q0 + qi;
          const bool seen = j < p.seq && key < nk && key >= first_of(p, j < p.seq ? j : 0, b) && (!p.causal || key <= j);
          const float w = seen ? expf(s[e] * sc - Ls[qi]) : 0.0f;
          Pt[ki * (BQ + 1) + qi] = w;
          St[ki * (BQ + 1) + qi] = w * (g[e] - Ds[qi]);
        }
        __syncthreads();
        for (int e = 0; e < BQ; ++e) {
          const float w = Pt[ki * (BQ + 1) + e], x = St[ki * (BQ + 1) + e];
#pragma unroll
          for (int i = 0; i < NO; ++i) {
            dv[i] = fmaf(w, Gs[e * LD + r + 8 * i], dv[i]);
            dk[i] = fmaf(x, Qs[e * LD + r + 8 * i], dk[i]);
          }
        }
      }
    }
  }
  if (key >= p.kv_seq) return;
  const int64_t at = koff + (int64_t)key * p.k_ss;
#pragma unroll
  for (int i = 0; i < NO; ++i) {
    const int c = r + 8 * i;
    if (c < d) {
      Elem<F32>::store(p.dk, at + c, dk[i] * p.scale);
      Elem<F32>::store(p.dv, at + c, dv[i]);
    }
  }
}

// ---- backward: dQ for a tile of queries -----------------------------------------
// BQ queries, 256 / BQ threads each: in the score phase a thread's keys are
// r, r + TPQ, ... of the key tile, in the product phase its features
// r, r + TPQ, ... of dQ.

template <bool F32, int DP>
__global__ __launch_bounds__(256) void attn_gen_dq(GenArgs p) {
  extern __shared__ float sm[];
  constexpr int LD = DP + 1;
  constexpr int BQ = DP <= 128 ? 64 : 32;
  constexpr int TPQ = 256 / BQ;
  float* Qs = sm;                  // BQ x LD
  float* Gs = Qs + BQ * LD;        // BQ x LD
  float* Ks = Gs + BQ * LD;        // kGK x LD
  float* Vs = Ks + kGK * LD;       // kGK x LD
  float* Ss = Vs + kGK * LD;       // BQ x (kGK + 1): dS
  int* lo = reinterpret_cast<int*>(Ss + BQ * (kGK + 1));
  const int q0 = blockIdx.x * BQ, h = blockIdx.y, b = blockIdx.z;
  const int hk = h / (p.heads / p.kv_heads);
  const int t = threadIdx.x, qi = t / TPQ, r = t % TPQ;
  const int j = q0 + qi;
  const int d = p.d;
  const int64_t qoff = (int64_t)b * p.q_sb + (int64_t)h * p.q_sh;
  const int64_t koff = (int64_t)b * p.k_sb + (int64_t)hk * p.k_sh;
  const int nk = keys_of(p, b);
  const int first = j < p.seq ? first_of(p, j, b) : 0;
  if (t == 0) lo[0] = 1 << 30;
  __syncthreads();
  if (r == 0 && j < p.seq) atomicMin(&lo[0], first);
  if constexpr (F32) {
    stage<F32>(Qs, LD, static_cast<const float*>(p.q) + qoff, p.q_ss, q0, BQ, p.seq, d);
    stage<F32>(Gs, LD, static_cast<const float*>(p.dout) + qoff, p.q_ss, q0, BQ, p.seq, d);
  } else {
    stage<F32>(Qs, LD, static_cast<const uint16_t*>(p.q) + qoff, p.q_ss, q0, BQ, p.seq, d);
    stage<F32>(Gs, LD, static_cast<const uint16_t*>(p.dout) + qoff, p.q_ss, q0, BQ, p.seq, d);
  }
  const int64_t row = ((int64_t)b * p.seq + (j < p.seq ? j : 0)) * p.heads + h;
  const float lse = p.lse[row], dl = p.delta[row];
  __syncthreads();
  const int q_last = min(q0 + BQ, p.seq) - 1;
  const int k_end = p.causal ? min(nk, q_last + 1) : nk;
  const int k_begin = max(0, lo[0]) / kGK * kGK;
  constexpr int NO = DP / TPQ;
  constexpr int NS = kGK / TPQ;
  float acc[NO];
#pragma unroll
  for (int i = 0; i < NO; ++i) acc[i] = 0.0f;
  const float sc = p.scale;
  for (int k0 = k_begin; k0 < k_end; k0 += kGK) {
    __syncthreads();
    if constexpr (F32) {
      stage<F32>(Ks, LD, static_cast<const float*>(p.k) + koff, p.k_ss, k0, kGK, nk, d);
      stage<F32>(Vs, LD, static_cast<const float*>(p.v) + koff, p.k_ss, k0, kGK, nk, d);
    } else {
      stage<F32>(Ks, LD, static_cast<const uint16_t*>(p.k) + koff, p.k_ss, k0, kGK, nk, d);
      stage<F32>(Vs, LD, static_cast<const uint16_t*>(p.v) + koff, p.k_ss, k0, kGK, nk, d);
    }
    __syncthreads();
    float s[NS], g[NS];
#pragma unroll
    for (int e = 0; e < NS; ++e) s[e] = g[e] = 0.0f;
    for (int c = 0; c < d; ++c) {
      const float qx = Qs[qi * LD + c], gx = Gs[qi * LD + c];
#pragma unroll
      for (int e = 0; e < NS; ++e) {
        s[e] = fmaf(qx, Ks[(r + TPQ * e) * LD + c], s[e]);
        g[e] = fmaf(gx, Vs[(r + TPQ * e) * LD + c], g[e]);
      }
    }
#pragma unroll
    for (int e = 0; e < NS; ++e) {
      const int key = k0 + r + TPQ * e;
      const bool seen = j < p.seq && key < nk && key >= first && (!p.causal || key <= j);
      const float w = seen ? expf(s[e] * sc - lse) : 0.0f;
      Ss[qi * (kGK + 1) + r + TPQ * e] = w * (g[e] - dl);
    }
    __syncthreads();
    for (int e = 0; e < kGK; ++e) {
      const float x = Ss[qi * (kGK + 1) + e];
#pragma unroll
      for (int i = 0; i < NO; ++i) acc[i] = fmaf(x, Ks[e * LD + r + TPQ * i], acc[i]);
    }
  }
  if (j >= p.seq) return;
  const int64_t at = qoff + (int64_t)j * p.q_ss;
#pragma unroll
  for (int i = 0; i < NO; ++i) {
    const int c = r + TPQ * i;
    if (c < d) Elem<F32>::store(p.dq, at + c, acc[i] * sc);
  }
}

// ---- dispatch ----------------------------------------------------------------------

int padded_dim(int d) {
  for (int dp : {16, 32, 64, 128, 256})
    if (d <= dp) return dp;
  return 0;
}

template <bool F32>
const void* fwd_kernel(int dp) {
  switch (dp) {
    case 16: return (const void*)attn_gen_fwd<F32, 16>;
    case 32: return (const void*)attn_gen_fwd<F32, 32>;
    case 64: return (const void*)attn_gen_fwd<F32, 64>;
    case 128: return (const void*)attn_gen_fwd<F32, 128>;
    default: return (const void*)attn_gen_fwd<F32, 256>;
  }
}

template <bool F32>
const void* dkdv_kernel(int dp) {
  switch (dp) {
    case 16: return (const void*)attn_gen_dkdv<F32, 16>;
    case 32: return (const void*)attn_gen_dkdv<F32, 32>;
    case 64: return (const void*)attn_gen_dkdv<F32, 64>;
    case 128: return (const void*)attn_gen_dkdv<F32, 128>;
    default: return (const void*)attn_gen_dkdv<F32, 256>;
  }
}

template <bool F32>
const void* dq_kernel(int dp) {
  switch (dp) {
    case 16: return (const void*)attn_gen_dq<F32, 16>;
    case 32: return (const void*)attn_gen_dq<F32, 32>;
    case 64: return (const void*)attn_gen_dq<F32, 64>;
    case 128: return (const void*)attn_gen_dq<F32, 128>;
    default: return (const void*)attn_gen_dq<F32, 256>;
  }
}

size_t fwd_lds(int dp) { return sizeof(float) * ((kGQ + 2 * kGK) * (dp + 1) + kGQ * (kGK + 1) + 1); }
int bq_of(int dp) { return dp <= 128 ? 64 : 32; }
size_t dkdv_lds(int dp) {
  const int bq = bq_of(dp);
  return sizeof(float) * ((2 * kGBK + 2 * bq) * (dp + 1) + 2 * kGBK * (bq + 1) + 2 * bq);
}
size_t dq_lds(int dp) {
  const int bq = bq_of(dp);
  return sizeof(float) * ((2 * bq + 2 * kGK) * (dp + 1) + bq * (kGK + 1) + 1);
}

int check(const th_attention_desc* d, bool backward) {
  TH_REQUIRE(d->head_dim >= 1 && d->head_dim <= 256, "attention: head_dim must be 1..256");
  TH_REQUIRE(d->seq >= 1 && d->kv_seq >= 0, "attention: the sequence lengths must be positive");
  TH_REQUIRE(d->heads > 0 && d->kv_heads > 0 && d->heads % d->kv_heads == 0,
             "attention: heads must be a positive multiple of kv_heads");
  TH_REQUIRE(d->batch > 0 && d->batch <= 65535 && d->heads <= 65535, "attention: grid too large");
  TH_REQUIRE(d->q && d->k && d->v && d->o, "attention: null q, k, v or o");
  for (int64_t s : {d->q_strides[0], d->q_strides[1], d->q_strides[2], d->k_strides[0], d->k_strides[1], d->k_strides[2]})
    TH_REQUIRE(s >= 0, "attention: strides must not be negative");
  if (backward) TH_REQUIRE(d->lse && d->dout && d->dq && d->dk && d->dv, "attention backward: null lse, dout, dq, dk or dv");
  return TH_OK;
}

GenArgs args_of(const th_attention_desc* d) {
  GenArgs a{};
  a.q = d->q, a.k = d->k, a.v = d->v, a.o = d->o, a.lse = d->lse;
  a.dout = d->dout, a.dq = d->dq, a.dk = d->dk, a.dv = d->dv;
  a.starts = d->starts, a.lengths = d->lengths;
  a.q_sh = d->q_strides[0], a.q_ss = d->q_strides[1], a.q_sb = d->q_strides[2];
  a.k_sh = d->k_strides[0], a.k_ss = d->k_strides[1], a.k_sb = d->k_strides[2];
  a.seq = d->seq, a.kv_seq = d->kv_seq > 0 ? d->kv_seq : d->seq;
  a.heads = d->heads, a.kv_heads = d->kv_heads, a.batch = d->batch, a.d = d->head_dim;
  a.causal = d->causal;
  a.scale = d->scale > 0 ? d->scale : 1.0f / sqrtf((float)d->head_dim);
  return a;
}

void refs(th::Builder& b, int k, const int* values, const size_t* offsets, int n) {
  for (int i = 0; i < n; ++i) b.ref(values[i], k, offsets[i]);
}

}  // namespace

namespace th {

int build_attention_general_fwd(const th_attention_desc* d, th_launch** out) {
  if (int r = check(d, false)) return r;
  const bool f32 = (d->flags & TH_ATTN_F32) != 0;
  const int dp = padded_dim(d->head_dim);
  const void* fn = f32 ? fwd_kernel<true>(dp) : fwd_kernel<false>(dp);
  const size_t lds = fwd_lds(dp);
  TH_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
  GenArgs a = args_of(d);
  th::Builder b("attention_fwd", 7);
  const unsigned nq = (unsigned)((d->seq + kGQ - 1) / kGQ);
  int k = b.kernel(fn, "attn_gen_fwd", dim3(nq, d->heads, d->batch), dim3(256), (uint32_t)lds, a);
  const int vals[7] = {0, 1, 2, 3, 4, 5, 6};
  const size_t offs[7] = {TH_OFFSET(GenArgs, q), TH_OFFSET(GenArgs, k),      TH_OFFSET(GenArgs, v),
                          TH_OFFSET(GenArgs, o), TH_OFFSET(GenArgs, lse),    TH_OFFSET(GenArgs, starts),
                          TH_OFFSET(GenArgs, lengths)};
  refs(b, k, vals, offs, 7);
  const double S = d->seq, K = a.kv_seq, BH = (double)d->batch * d->heads, e = f32 ? 4.0 : 2.0;
  const double flops = 4.0 * BH * S * K * d->head_dim * (d->causal ? 0.5 : 1.0);
  b.work(e * d->head_dim * (2.0 * BH * S + 2.0 * d->batch * d->kv_heads * K) + 4.0 * BH * S, flops,
         (int64_t)nq * d->heads * d->batch);
  *out = b.release();
  return TH_OK;
}

int build_attention_general_bwd(const th_attention_desc* d, th_launch** out) {
  if (int r = check(d, true)) return r;
  const bool f32 = (d->flags & TH_ATTN_F32) != 0;
  const int dp = padded_dim(d->head_dim);
  GenArgs a = args_of(d);
  th::Builder b("attention_bwd", 11);
  const int64_t rows = (int64_t)d->batch * d->seq * d->heads;
  const uint64_t at_delta = b.workspace((uint64_t)rows * sizeof(float));  // delta, [b][s][h]
  const void* f0 = f32 ? (const void*)attn_gen_delta<true> : (const void*)attn_gen_delta<false>;
  const void* f1 = f32 ? dkdv_kernel<true>(dp) : dkdv_kernel<false>(dp);
  const void* f2 = f32 ? dq_kernel<true>(dp) : dq_kernel<false>(dp);
  TH_HIP(hipFuncSetAttribute(f1, hipFuncAttributeMaxDynamicSharedMemorySize, (int)dkdv_lds(dp)));
  TH_HIP(hipFuncSetAttribute(f2, hipFuncAttributeMaxDynamicSharedMemorySize, (int)dq_lds(dp)));
  const int bq = bq_of(dp);
  int k0 = b.kernel(f0, "attn_gen_delta", dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, a);
  int k1 = b.kernel(f1, "attn_gen_dkdv", dim3((unsigned)((a.kv_seq + kGBK - 1) / kGBK), d->kv_heads, d->batch),
                    dim3(256), (uint32_t)dkdv_lds(dp), a);
  int k2 = b.kernel(f2, "attn_gen_dq", dim3((unsigned)((d->seq + bq - 1) / bq), d->heads, d->batch), dim3(256),
                    (uint32_t)dq_lds(dp), a);
  const size_t offs[11] = {TH_OFFSET(GenArgs, q),  TH_OFFSET(GenArgs, k),    TH_OFFSET(GenArgs, v),
                           TH_OFFSET(GenArgs, o),  TH_OFFSET(GenArgs, lse),  TH_OFFSET(GenArgs, dout),
                           TH_OFFSET(GenArgs, dq), TH_OFFSET(GenArgs, dk),   TH_OFFSET(GenArgs, dv),
                           TH_OFFSET(GenArgs, starts), TH_OFFSET(GenArgs, lengths)};
  for (int v = 0; v < 11; ++v)
    for (int kk : {k0, k1, k2}) b.ref(v, kk, offs[v]);
  for (int kk : {k0, k1, k2}) b.ws_ref(kk, TH_OFFSET(GenArgs, delta), at_delta);
  const double S = d->seq, K = a.kv_seq, BH = (double)d->batch * d->heads, e = f32 ? 4.0 : 2.0;
  const double flops = 2.5 * 4.0 * BH * S * K * d->head_dim * (d->causal ? 0.5 : 1.0);
  b.work(e * d->head_dim * (4.0 * BH * S + 4.0 * d->batch * d->kv_heads * K) + 8.0 * BH * S, flops,
         (int64_t)((a.kv_seq + kGBK - 1) / kGBK) * d->kv_heads * d->batch);
  *out = b.release();
  return TH_OK;
}

}  // namespace th
