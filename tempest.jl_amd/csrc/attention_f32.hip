// Op class (c) for fp32 arrays on the matrix cores: v_mfma_f32_32x32x2_f32
// (exact fp32 products, fp32 sums) at head dims 64 and 128, any lengths,
// grouped heads, causal or not.  fp32 attention with device-held masks, and
// other head dims, stay on attention_generic.hip.  The reference's cuTile
// sweep takes fp32 arrays (its TF32 mode rounds the factors to 10 bits,
// ext/cuTileExt/build.jl:326-532; TRIALS.md:2187); here the products are
// exact, as its default precision asks (src/Compiler/runtime/target.jl:42-44).
//
// The forms of the bf16 kernels of attention_mfma.hip, for one product of
// depth 2 instead of 16:
//   - products over d (S' = K Q', S = Q K', dP = dO V'): lane half h takes d
//     in [h D/2, (h + 1) D/2), step s the d h D/2 + s, so a lane's operand
//     of four steps is one 16-byte read of a tile row (rows of D + 4 floats:
//     16 lanes reading 16 rows start on 16 distinct bank quads), the other
//     operand (a position's row) in registers;
//   - products over positions (O' += V' P', dV' += dO' P, dK' += Q' dS,
//     dQ' += K' dS'): the score accumulator's register i is the B operand
//     of step i as it stands (lanes 0..31 holding position 8 (i / 4) + i % 4
//     of the block, lanes 32..63 the position 4 further), and the output's
//     row m of block b holds d = NB m + b (NB = D / 32 blocks), so that a
//     lane's A operands of the NB blocks are NB adjacent floats of one tile
//     row, one 8- or 16-byte read.
// Everything else as there: tiles of 64 positions staged through registers a
// step ahead (zeros past the sequence), one barrier a step, the online
// softmax in exp2 units (folds.jl:186-222), P in fp32, lse = m + log(l);
// the backward FA2's, deterministic: delta = rowsum(dO .* O); dK, dV per 128
// keys sweeping the query tiles of each query head of the group; dQ per 128
// queries sweeping the key tiles.  Keys past the keys' length and, causal,
// keys after the query weigh 0; queries past the sequence are computed on
// zeros and not stored.
#include <hip/hip_runtime.h>

#include <cmath>

#include "th_core.h"

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

struct FArgs {
  const float* q;
  const float* k;
  const float* v;
  float* o;
  float* lse;  // natural log, [b][s][h]
  const float* dout;
  float* delta;  // backward workspace: rowsum(dO .* O), [b][s][h]
  float* dq;
  float* dk;
  float* dv;
  int64_t q_sh, q_ss, q_sb;  // strides (elements) of q, o, dout, dq
  int64_t k_sh, k_ss, k_sb;  // strides of k, v, dk, dv
  int32_t seq, kv_seq, heads, kv_heads, batch, causal;
  float scale;
  // A sweep split into parts (small grids): nsplit parts of `span`
  // positions (a multiple of 64), partial results in `part`
  // ([part][b][position][head][d]) and the forward's (m, l) in `part_ml`.
  int32_t nsplit, span;
  float* part;
  float* part_ml;
};

__device__ __forceinline__ f32x16 mfma2(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// The value lane l ^ 32 holds.
__device__ __forceinline__ float other_half(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(threadIdx.x % 64 < 32 ? r[1] : r[0]);
}

template <int D>
constexpr int kLd = D + 4;  // LDS row of a tile (floats)
template <int D>
constexpr int kTileF = 64 * kLd<D>;

// A position's row as the B operand of a product over d: f[s] = row[h D/2 + s].
template <int D>
__device__ __forceinline__ void row_half(const float* row, bool live, float (&f)[D / 2]) {
  const int h = (threadIdx.x % 64) / 32;
#pragma unroll
  for (int u = 0; u < D / 8; ++u) {
    const f32x4 x = live ? *reinterpret_cast<const f32x4*>(row + h * (D / 2) + 4 * u) : f32x4{};
#pragma unroll
    for (int e = 0; e < 4; ++e) f[4 * u + e] = x[e];
  }
}

// acc += T[rows r0 + lane % 32] x f over d (D / 2 steps, four a read).
template <int D>
__device__ __forceinline__ void over_d(const float* t, int r0, const float (&f)[D / 2], f32x16& acc) {
  const int lane = threadIdx.x % 64;
  const float* row = t + (r0 + lane % 32) * kLd<D> + (lane / 32) * (D / 2);
#pragma unroll
  for (int u = 0; u < D / 8; ++u) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(row + 4 * u);
#pragma unroll
    for (int e = 0; e < 4; ++e) acc = mfma2(a[e], f[4 * u + e], acc);
  }
}

// The NB adjacent floats of tile row `r` this lane gives the NB output
// blocks of a product over positions: columns NB (lane % 32) + (0..NB-1).
template <int D>
struct Cols {
  float x[D / 32];
};
template <int D>
__device__ __forceinline__ Cols<D> cols_of(const float* t, int r) {
  constexpr int NB = D / 32;
  const float* at = t + r * kLd<D> + NB * (threadIdx.x % 32);
  Cols<D> c;
  if constexpr (NB == 2) {
    const f32x2 x = *reinterpret_cast<const f32x2*>(at);
    c.x[0] = x[0], c.x[1] = x[1];
  } else {
    const f32x4 x = *reinterpret_cast<const f32x4*>(at);
#pragma unroll
    for (int e = 0; e < NB; ++e) c.x[e] = x[e];
  }
  return c;
}

// out[db] += T'(d, positions of block pb) P over the block's 32 positions:
// step i pairs position 8 (i / 4) + i % 4 (lanes 0..31) with the one 4
// further (lanes 32..63), as register i of the score accumulator holds them.
template <int D>
__device__ __forceinline__ void over_positions(const float* t, int p0, const f32x16& pw, f32x16 (&out)[D / 32]) {
  const int lh = (threadIdx.x % 64) / 32;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const Cols<D> c = cols_of<D>(t, p0 + 8 * (i / 4) + 4 * lh + i % 4);
#pragma unroll
    for (int db = 0; db < D / 32; ++db) out[db] = mfma2(c.x[db], pw[i], out[db]);
  }
}

// Store an output block set: block db's register i holds d = NB (8 (i / 4) +
// 4 lh + i % 4) + db, for the lane's position; scaled by sc.
template <int D>
__device__ __forceinline__ void store_rows(float* row, const f32x16 (&x)[D / 32], float sc) {
  constexpr int NB = D / 32;
  const int lh = (threadIdx.x % 64) / 32;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    // d = NB (8 q + 4 lh) + (0 .. 4 NB - 1): register 4 q + e of block db at NB e + db.
    float* at = row + NB * (8 * q + 4 * lh);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if constexpr (NB == 2) {
        *reinterpret_cast<f32x2*>(at + 2 * e) = f32x2{x[0][4 * q + e] * sc, x[1][4 * q + e] * sc};
      } else {
        *reinterpret_cast<f32x4*>(at + 4 * e) =
            f32x4{x[0][4 * q + e] * sc, x[1][4 * q + e] * sc, x[2][4 * q + e] * sc, x[3][4 * q + e] * sc};
      }
    }
  }
}

// A 64-position tile staged through registers: thread t holds the 16-byte
// chunks t + 256 i; rows past `limit` read as zeros.
template <int D>
struct StageF {
  static constexpr int kChunks = D / 4;
  static constexpr int kPer = 64 * kChunks / 256;
  f32x4 r[kPer];
  __device__ void load(const float* base, int64_t ss, int row0, int limit) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int c = threadIdx.x + 256 * i, row = c / kChunks, col = c % kChunks;
      r[i] = row0 + row < limit ? *reinterpret_cast<const f32x4*>(base + (int64_t)(row0 + row) * ss + 4 * col)
                                : f32x4{};
    }
  }
  __device__ void store(float* t) const {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int c = threadIdx.x + 256 * i, row = c / kChunks, col = c % kChunks;
      *reinterpret_cast<f32x4*>(t + row * kLd<D> + 4 * col) = r[i];
    }
  }
};

// Causal sweeps do less work for earlier query blocks (and later key
// blocks): workgroup x takes blocks x and nb - 1 - x (one pass each), so
// every workgroup sweeps about the same number of tiles.
__device__ __forceinline__ int passes(bool causal, int x, int nb) { return causal && 2 * x + 1 != nb ? 2 : 1; }
__device__ __forceinline__ int block_of(int pass, int x, int nb) { return pass == 0 ? x : nb - 1 - x; }

// ---- forward ---------------------------------------------------------------------

// Keys [k_lo, k_hi) of query block qb: all (split < 0) or part `split`,
// which leaves its unnormalised O' and (m, l) for the combining kernel.
template <int D>
__device__ __forceinline__ void fwd_block(const FArgs& p, const int qb, const int b, const int split) {
  constexpr int NB = D / 32;
  extern __shared__ __attribute__((aligned(16))) float flds[];
  const int h = blockIdx.y;
  const int hk = h / (p.heads / p.kv_heads);
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64, lr = lane % 32, lh = lane / 32;
  const int q0 = qb * 128 + wave * 32, query = q0 + lr;
  const float* qbase = p.q + (int64_t)b * p.q_sb + (int64_t)h * p.q_sh;
  const float* kbase = p.k + (int64_t)b * p.k_sb + (int64_t)hk * p.k_sh;
  const float* vbase = p.v + (int64_t)b * p.k_sb + (int64_t)hk * p.k_sh;
  float qf[D / 2];
  row_half<D>(qbase + (int64_t)query * p.q_ss, query < p.seq, qf);
  f32x16 o[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) o[i] = f32x16{};
  float m = -INFINITY, l = 0.0f;
  const float c = p.scale * kLog2e;
  const int qlast = min(qb * 128 + 127, p.seq - 1);
  const int kend = p.causal ? min(p.kv_seq, qlast + 1) : p.kv_seq;
  const int k_lo = split < 0 ? 0 : split * p.span, k_hi = split < 0 ? kend : min(kend, k_lo + p.span);
  const int nsteps = k_hi > k_lo ? (k_hi - k_lo + 63) / 64 : 0;
  StageF<D> sk, sv;
  auto K = [&](int s) { return flds + 2 * s * kTileF<D>; };
  auto V = [&](int s) { return flds + (2 * s + 1) * kTileF<D>; };
  if (nsteps > 0) {
    sk.load(kbase, p.k_ss, k_lo, p.kv_seq);
    sv.load(vbase, p.k_ss, k_lo, p.kv_seq);
    sk.store(K(0));
    sv.store(V(0));
  }
  __syncthreads();
  for (int j = 0; j < nsteps; ++j) {
    const int cur = j & 1, k0 = k_lo + 64 * j;
    if (j + 1 < nsteps) {
      sk.load(kbase, p.k_ss, k0 + 64, p.kv_seq);
      sv.load(vbase, p.k_ss, k0 + 64, p.kv_seq);
    }
    // S' (64 keys x 32 queries): key 32 kb + 8 (i / 4) + 4 lh + i % 4 in register i.
    f32x16 s[2] = {f32x16{}, f32x16{}};
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) over_d<D>(K(cur), 32 * kb, qf, s[kb]);
    if (k0 + 64 > p.kv_seq || (p.causal && k0 + 64 > q0)) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int key = k0 + 32 * kb + 8 * (i / 4) + 4 * lh + i % 4;
          if (key >= p.kv_seq || (p.causal && key > query)) s[kb][i] = -INFINITY;
        }
    }
    float mb = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int i = 0; i < 16; ++i) mb = fmaxf(mb, s[kb][i]);
    mb = fmaxf(mb, other_half(mb)) * c;
    const float mn = fmaxf(m, mb);
    const float shift = isfinite(mn) ? mn : 0.0f;  // lse_shift (folds.jl:194)
    const float alpha = __builtin_amdgcn_exp2f(m - shift);
    l *= alpha;
#pragma unroll
    for (int i = 0; i < NB; ++i) o[i] *= alpha;
    m = mn;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float w = __builtin_amdgcn_exp2f(fmaf(s[kb][i], c, -shift));
        l += w;
        s[kb][i] = w;
      }
    // O' (D x 32 queries) += V' P'.
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) over_positions<D>(V(cur), 32 * kb, s[kb], o);
    if (j + 1 < nsteps) {
      // The other stage was last read in step j - 1, before the barrier that ended it.
      sk.store(K(cur ^ 1));
      sv.store(V(cur ^ 1));
    }
    __syncthreads();
  }
  l += other_half(l);
  if (query >= p.seq) return;
  if (split >= 0) {
    // This part's unnormalised O' and (m, l) (m = -inf, l = 0 where it saw no key).
    const int64_t row = (((int64_t)split * p.batch + b) * p.seq + query) * p.heads + h;
    store_rows<D>(p.part + row * D, o, 1.0f);
    if (lh == 0) reinterpret_cast<f32x2*>(p.part_ml)[row] = f32x2{m, l};
    return;
  }
  store_rows<D>(p.o + (int64_t)b * p.q_sb + (int64_t)h * p.q_sh + (int64_t)query * p.q_ss, o, 1.0f / l);
  if (lh == 0 && p.lse) p.lse[((int64_t)b * p.seq + query) * p.heads + h] = (m + log2f(l)) * kLn2;
}

template <int D>
__global__ __launch_bounds__(256, D <= 64 ? 2 : 1) void f32_attn_fwd(FArgs p) {
  // Split: one part of one block; else a block and, causal, its mirror (one call site).
  const bool split = p.nsplit > 1;
  const int nb = (p.seq + 127) / 128;
  const int npass = split ? 1 : passes(p.causal, blockIdx.x, nb);
  for (int pass = 0; pass < npass; ++pass) {
    if (pass > 0) __syncthreads();  // the first pass's last LDS reads are done
    fwd_block<D>(p, split ? blockIdx.x : block_of(pass, blockIdx.x, nb), split ? blockIdx.z / p.nsplit : blockIdx.z,
                 split ? blockIdx.z % p.nsplit : -1);
  }
}

// The parts of a split forward combined: per (b, query, head) row, M = max
// m_s, L = sum l_s 2^(m_s - M), O = sum O_s 2^(m_s - M) / L in part order;
// lse = (M + log2 L) ln 2.  A thread per four features of a row.
struct FCombineArgs {
  FArgs p;  // first: its members sit at FArgs' offsets
  int32_t d;
};

__global__ __launch_bounds__(256) void f32_attn_combine(FCombineArgs a) {
  const FArgs& p = a.p;
  const int quads = a.d / 4;
  const int64_t rows = (int64_t)p.batch * p.seq * p.heads;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= rows * quads) return;
  const int64_t row = t / quads;
  const int c = 4 * (int)(t % quads);
  const f32x2* ml = reinterpret_cast<const f32x2*>(p.part_ml);
  float mx = -INFINITY;
  for (int s = 0; s < p.nsplit; ++s) mx = fmaxf(mx, ml[s * rows + row][0]);
  const float shift = isfinite(mx) ? mx : 0.0f;
  float l = 0.0f;
  f32x4 acc = {};
  for (int s = 0; s < p.nsplit; ++s) {
    const f32x2 x = ml[s * rows + row];
    const float w = __builtin_amdgcn_exp2f(x[0] - shift);
    l += w * x[1];
    acc += w * *reinterpret_cast<const f32x4*>(p.part + (s * rows + row) * a.d + c);
  }
  const int h = (int)(row % p.heads);
  const int64_t pos = (row / p.heads) % p.seq, b = row / ((int64_t)p.heads * p.seq);
  *reinterpret_cast<f32x4*>(p.o + b * p.q_sb + h * p.q_sh + pos * p.q_ss + c) = acc * (1.0f / l);
  if (c == 0 && p.lse) p.lse[row] = (mx + log2f(l)) * kLn2;
}

// dQ, dK or dV from a split sweep's parts: out = scale * sum_s part_s in
// part order; rows [b][position][head] of `d` features.
struct FSumArgs {
  const float* part;
  float* out;
  int64_t sh, ss, sb;
  int32_t positions, heads, batch, d, nsplit;
  float scale;
};

__global__ __launch_bounds__(256) void f32_attn_sum(FSumArgs a) {
  const int quads = a.d / 4;
  const int64_t rows = (int64_t)a.batch * a.positions * a.heads;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= rows * quads) return;
  const int64_t row = t / quads;
  const int c = 4 * (int)(t % quads);
  // Part s of this quad at a.part + (s rows + row) d + c: a stride of rows d / 4 quads.
  f32x4 acc = thd::sum_in_order(reinterpret_cast<const f32x4*>(a.part + row * a.d + c), rows * a.d / 4, a.nsplit);
  const int h = (int)(row % a.heads);
  const int64_t pos = (row / a.heads) % a.positions, b = row / ((int64_t)a.heads * a.positions);
  *reinterpret_cast<f32x4*>(a.out + b * a.sb + h * a.sh + pos * a.ss + c) = acc * a.scale;
}

// ---- backward: delta = rowsum(dO .* O) ---------------------------------------------

struct FDeltaArgs {
  FArgs p;  // first: its members sit at FArgs' offsets
  int32_t d;
};

// D / 4 lanes per (batch, position, head) row, 16 bytes each (the path takes
// strides in multiples of 4 and 16-byte bases); each lane group takes
// kDeltaRowsF rows, 64 / (D / 4) apart, every load issued before the first
// product.  Rows are numbered with the head fastest, so a load instruction
// covers consecutive rows; row numbers fit 32 bits (the builder checks).
constexpr int kDeltaRowsF = 4;

template <int D>
__global__ __launch_bounds__(256) void f32_attn_delta(FDeltaArgs a) {
  constexpr int G = D / 4;   // lanes a row
  constexpr int R = 64 / G;  // rows a wave covers at once
  const FArgs& p = a.p;
  const uint32_t total = (uint32_t)p.batch * p.seq * p.heads;
  const int lane = threadIdx.x % 64, part = lane % G;
  const uint32_t row0 = (blockIdx.x * 4 + threadIdx.x / 64) * (R * kDeltaRowsF) + lane / G;
  auto at_of = [&](uint32_t row) {
    const uint32_t bs = row / (uint32_t)p.heads;
    const int64_t b = bs / (uint32_t)p.seq, s = bs % (uint32_t)p.seq, h = row - bs * (uint32_t)p.heads;
    return b * p.q_sb + h * p.q_sh + s * p.q_ss + 4 * part;
  };
  f32x4 ov[kDeltaRowsF], gv[kDeltaRowsF];
#pragma unroll
  for (int i = 0; i < kDeltaRowsF; ++i) {
    // Rows past the end re-read the last one; nothing is written for them.
    const int64_t at = at_of(min(row0 + R * i, total - 1));
    ov[i] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p.o + at));
    gv[i] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p.dout + at));
  }
  // Every load out before any of their data is used.
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < kDeltaRowsF; ++i) {
    float v = ov[i][0] * gv[i][0];
#pragma unroll
    for (int e = 1; e < 4; ++e) v += ov[i][e] * gv[i][e];
#pragma unroll
    for (int m = G / 2; m >= 1; m /= 2) v += __shfl_xor(v, m, G);
    const uint32_t row = row0 + R * i;
    if (row < total && part == 0) p.delta[row] = v;
  }
}

// ---- backward: dK, dV ----------------------------------------------------------------
// A workgroup takes 128 keys (32 a wave).  Per query tile of 64: S (64
// queries x 32 keys) with queries on the registers and keys on the lanes, so
// that P and dS feed the products over queries straight from the
// accumulators.

// Query tiles [qstart, qstop) for the keys of kblk: all (split < 0) or part
// `split`, which leaves its unscaled dK', dV'.
template <int D>
__device__ __forceinline__ void dkdv_block(const FArgs& p, const int kblk, const int b, const int split) {
  constexpr int NB = D / 32;
  extern __shared__ __attribute__((aligned(16))) float flds[];
  float* stats = flds + 4 * kTileF<D>;  // [stage][lse * log2e (64) | delta (64)]
  const int hk = blockIdx.y;
  const int group = p.heads / p.kv_heads;
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64, lh = lane / 32;
  const int kw0 = kblk * 128, key = kw0 + wave * 32 + lane % 32;
  const int64_t koff = (int64_t)b * p.k_sb + (int64_t)hk * p.k_sh;
  float kf[D / 2], vf[D / 2];
  row_half<D>(p.k + koff + (int64_t)key * p.k_ss, key < p.kv_seq, kf);
  row_half<D>(p.v + koff + (int64_t)key * p.k_ss, key < p.kv_seq, vf);
  f32x16 dk[NB], dv[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) dk[i] = f32x16{}, dv[i] = f32x16{};
  const float c = p.scale * kLog2e;
  auto Q = [&](int s) { return flds + 2 * s * kTileF<D>; };
  auto G = [&](int s) { return flds + (2 * s + 1) * kTileF<D>; };
  auto Ls = [&](int s) { return stats + 128 * s; };
  const int qfirst = p.causal ? kw0 / 64 * 64 : 0;
  const int qstart = split < 0 ? qfirst : qfirst + split * p.span;
  const int qstop = split < 0 ? p.seq : min(p.seq, qstart + p.span);
  const int nsteps = qstart < qstop ? (qstop - qstart + 63) / 64 : 0;
  StageF<D> sq, sg;
  float st = 0.0f;  // threads 0..127: a query's lse * log2e or delta
  auto load = [&](const float* qbase, const float* gbase, int h, int q0) {
    sq.load(qbase, p.q_ss, q0, p.seq);
    sg.load(gbase, p.q_ss, q0, p.seq);
    if (threadIdx.x < 128) {
      const int j = q0 + threadIdx.x % 64;
      const int64_t row = ((int64_t)b * p.seq + j) * p.heads + h;
      st = j < p.seq ? (threadIdx.x < 64 ? p.lse[row] * kLog2e : p.delta[row]) : 0.0f;
    }
  };
  auto store = [&](int s) {
    sq.store(Q(s));
    sg.store(G(s));
    if (threadIdx.x < 128) Ls(s)[threadIdx.x] = st;
  };
  for (int h = hk * group; h < (hk + 1) * group; ++h) {
    const float* qbase = p.q + (int64_t)b * p.q_sb + (int64_t)h * p.q_sh;
    const float* gbase = p.dout + (int64_t)b * p.q_sb + (int64_t)h * p.q_sh;
    if (nsteps > 0) {
      load(qbase, gbase, h, qstart);
      store(0);
    }
    __syncthreads();
    for (int j = 0; j < nsteps; ++j) {
      const int cur = j & 1, qq0 = qstart + 64 * j;
      if (j + 1 < nsteps) load(qbase, gbase, h, qq0 + 64);
      const float *Qt = Q(cur), *Gt = G(cur);
      const float* L = Ls(cur);
      // The tile's two halves of 32 queries in turn (half the score
      // accumulators live at once); the next tile goes to LDS after the first.
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        // S = Q K', dP = dO V' (32 queries x 32 keys): query 32 jj + 8 (i / 4) + 4 lh + i % 4 in register i.
        f32x16 s = {}, dp = {};
        over_d<D>(Qt, 32 * jj, kf, s);
        over_d<D>(Gt, 32 * jj, vf, dp);
        // P into s, dS into dp.
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int qi = 32 * jj + 8 * (i / 4) + 4 * lh + i % 4, query = qq0 + qi;
          const bool seen = query < p.seq && key < p.kv_seq && (!p.causal || key <= query);
          const float w = seen ? __builtin_amdgcn_exp2f(fmaf(s[i], c, -L[qi])) : 0.0f;
          s[i] = w;
          dp[i] = w * (dp[i] - L[64 + qi]);
        }
        // dV' (D x 32 keys) += dO' P;  dK' += Q' dS.
        over_positions<D>(Gt, 32 * jj, s, dv);
        over_positions<D>(Qt, 32 * jj, dp, dk);
        // The other stage was last read in step j - 1, before the barrier that ended it.
        if (jj == 0 && j + 1 < nsteps) store(cur ^ 1);
      }
      __syncthreads();
    }
  }
  if (key >= p.kv_seq) return;
  if (split >= 0) {
    const int64_t rows = (int64_t)p.batch * p.kv_seq * p.kv_heads;
    const int64_t row = (((int64_t)split * p.batch + b) * p.kv_seq + key) * p.kv_heads + hk;
    store_rows<D>(p.part + row * D, dk, 1.0f);
    store_rows<D>(p.part + ((int64_t)p.nsplit * rows + row) * D, dv, 1.0f);
    return;
  }
  const int64_t out = koff + (int64_t)key * p.k_ss;
  store_rows<D>(p.dk + out, dk, p.scale);
  store_rows<D>(p.dv + out, dv, 1.0f);
}

template <int D>
// One wave a SIMD: K and V of the wave's keys, dK' and dV' take D + D registers.
__global__ __launch_bounds__(256, 1) void f32_attn_dkdv(FArgs p) {
  const bool split = p.nsplit > 1;
  const int nb = (p.kv_seq + 127) / 128;
  const int npass = split ? 1 : passes(p.causal, blockIdx.x, nb);
  for (int pass = 0; pass < npass; ++pass) {
    if (pass > 0) __syncthreads();  // the first pass's last LDS reads are done
    dkdv_block<D>(p, split ? blockIdx.x : block_of(pass, blockIdx.x, nb), split ? blockIdx.z / p.nsplit : blockIdx.z,
                  split ? blockIdx.z % p.nsplit : -1);
  }
}

// ---- backward: dQ ----------------------------------------------------------------------
// A workgroup takes 128 queries (32 a wave) and sweeps key tiles of 64:
// S' = K Q', dP' = V dO' (keys on the registers, queries on the lanes),
// dS' = P' (dP' - delta), dQ' (D x 32 queries) += K' dS'.

// Keys [k_lo, k_hi) for query block qb: all (split < 0) or part `split`,
// which leaves its unscaled dQ'.
template <int D>
__device__ __forceinline__ void dq_block(const FArgs& p, const int qb, const int b, const int split) {
  constexpr int NB = D / 32;
  extern __shared__ __attribute__((aligned(16))) float flds[];
  const int h = blockIdx.y;
  const int hk = h / (p.heads / p.kv_heads);
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64, lh = lane / 32;
  const int q0 = qb * 128 + wave * 32, query = q0 + lane % 32;
  const int64_t qoff = (int64_t)b * p.q_sb + (int64_t)h * p.q_sh + (int64_t)query * p.q_ss;
  const bool live = query < p.seq;
  float qf[D / 2], gf[D / 2];
  row_half<D>(p.q + qoff, live, qf);
  row_half<D>(p.dout + qoff, live, gf);
  const int64_t srow = ((int64_t)b * p.seq + query) * p.heads + h;
  const float l2 = live ? p.lse[srow] * kLog2e : 0.0f;
  const float dl = live ? p.delta[srow] : 0.0f;
  const float c = p.scale * kLog2e;
  const float* kbase = p.k + (int64_t)b * p.k_sb + (int64_t)hk * p.k_sh;
  const float* vbase = p.v + (int64_t)b * p.k_sb + (int64_t)hk * p.k_sh;
  f32x16 dq[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) dq[i] = f32x16{};
  const int qlast = min(qb * 128 + 127, p.seq - 1);
  const int kend = p.causal ? min(p.kv_seq, qlast + 1) : p.kv_seq;
  const int k_lo = split < 0 ? 0 : split * p.span, k_hi = split < 0 ? kend : min(kend, k_lo + p.span);
  const int nsteps = k_hi > k_lo ? (k_hi - k_lo + 63) / 64 : 0;
  StageF<D> sk, sv;
  auto K = [&](int s) { return flds + 2 * s * kTileF<D>; };
  auto V = [&](int s) { return flds + (2 * s + 1) * kTileF<D>; };
  if (nsteps > 0) {
    sk.load(kbase, p.k_ss, k_lo, p.kv_seq);
    sv.load(vbase, p.k_ss, k_lo, p.kv_seq);
    sk.store(K(0));
    sv.store(V(0));
  }
  __syncthreads();
  for (int j = 0; j < nsteps; ++j) {
    const int cur = j & 1, k0 = k_lo + 64 * j;
    if (j + 1 < nsteps) {
      sk.load(kbase, p.k_ss, k0 + 64, p.kv_seq);
      sv.load(vbase, p.k_ss, k0 + 64, p.kv_seq);
    }
    // The tile's two halves of 32 keys in turn; the next tile goes to LDS after the first.
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      f32x16 sc = {}, dp = {};
      over_d<D>(K(cur), 32 * kb, qf, sc);
      over_d<D>(V(cur), 32 * kb, gf, dp);
      // dS' into sc.
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key = k0 + 32 * kb + 8 * (i / 4) + 4 * lh + i % 4;
        const bool seen = key < p.kv_seq && (!p.causal || key <= query);
        const float pw = seen ? __builtin_amdgcn_exp2f(fmaf(sc[i], c, -l2)) : 0.0f;
        sc[i] = pw * (dp[i] - dl);
      }
      over_positions<D>(K(cur), 32 * kb, sc, dq);
      if (kb == 0 && j + 1 < nsteps) {
        sk.store(K(cur ^ 1));
        sv.store(V(cur ^ 1));
      }
    }
    __syncthreads();
  }
  if (!live) return;
  if (split >= 0) {
    store_rows<D>(p.part + ((((int64_t)split * p.batch + b) * p.seq + query) * p.heads + h) * D, dq, 1.0f);
    return;
  }
  store_rows<D>(p.dq + qoff, dq, p.scale);
}

template <int D>
__global__ __launch_bounds__(256, D <= 64 ? 2 : 1) void f32_attn_dq(FArgs p) {
  const bool split = p.nsplit > 1;
  const int nb = (p.seq + 127) / 128;
  const int npass = split ? 1 : passes(p.causal, blockIdx.x, nb);
  for (int pass = 0; pass < npass; ++pass) {
    if (pass > 0) __syncthreads();  // the first pass's last LDS reads are done
    dq_block<D>(p, split ? blockIdx.x : block_of(pass, blockIdx.x, nb), split ? blockIdx.z / p.nsplit : blockIdx.z,
                split ? blockIdx.z % p.nsplit : -1);
  }
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

unsigned blocks_of(int n, int causal) {
  const unsigned nb = (unsigned)((n + 127) / 128);
  return causal ? (nb + 1) / 2 : nb;
}

FArgs fargs_of(const th_attention_desc* d) {
  FArgs a{};
  a.q = static_cast<const float*>(d->q);
  a.k = static_cast<const float*>(d->k);
  a.v = static_cast<const float*>(d->v);
  a.o = static_cast<float*>(d->o);
  a.lse = d->lse;
  a.dout = static_cast<const float*>(d->dout);
  a.dq = static_cast<float*>(d->dq);
  a.dk = static_cast<float*>(d->dk);
  a.dv = static_cast<float*>(d->dv);
  a.q_sh = d->q_strides[0], a.q_ss = d->q_strides[1], a.q_sb = d->q_strides[2];
  a.k_sh = d->k_strides[0], a.k_ss = d->k_strides[1], a.k_sb = d->k_strides[2];
  a.seq = d->seq;
  a.kv_seq = d->kv_seq > 0 ? d->kv_seq : d->seq;
  a.heads = d->heads, a.kv_heads = d->kv_heads, a.batch = d->batch, a.causal = d->causal;
  a.scale = d->scale > 0 ? d->scale : 1.0f / sqrtf((float)d->head_dim);
  return a;
}

double visible_pairs(const FArgs& a) {
  const double S = a.seq, K = a.kv_seq;
  if (!a.causal) return S * K;
  const double full = std::min(S, K);
  return full * (full + 1) / 2 + std::max(0.0, S - K) * K;
}

template <int D>
int fwd_launch(const th_attention_desc* d, th_launch** out) {
  const size_t lds = 4 * (size_t)kTileF<D> * sizeof(float);
  TH_HIP(hipFuncSetAttribute((const void*)f32_attn_fwd<D>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
  FArgs a = fargs_of(d);
  const int nqb = (d->seq + 127) / 128;
  const th::Split sp = th::split_of((int64_t)nqb * d->heads * d->batch, a.kv_seq);
  a.nsplit = sp.n, a.span = sp.span;
  TH_REQUIRE((int64_t)d->batch * sp.n <= 65535, "attention: grid too large");
  th::Builder b("attention_fwd_f32mfma", 7);
  const dim3 grid = sp.n > 1 ? dim3(nqb, d->heads, d->batch * sp.n) : dim3(blocks_of(d->seq, d->causal), d->heads, d->batch);
  int k = b.kernel((const void*)f32_attn_fwd<D>, D == 64 ? "f32_attn_fwd_d64" : "f32_attn_fwd_d128", grid, dim3(256),
                   (uint32_t)lds, a);
  b.ref(0, k, TH_OFFSET(FArgs, q));
  b.ref(1, k, TH_OFFSET(FArgs, k));
  b.ref(2, k, TH_OFFSET(FArgs, v));
  b.ref(3, k, TH_OFFSET(FArgs, o));
  b.ref(4, k, TH_OFFSET(FArgs, lse));
  if (sp.n > 1) {
    const int64_t rows = (int64_t)d->batch * d->seq * d->heads;
    const uint64_t at_o = b.workspace((uint64_t)sp.n * rows * D * sizeof(float));
    const uint64_t at_ml = b.workspace((uint64_t)sp.n * rows * 2 * sizeof(float));
    int kc = b.kernel((const void*)f32_attn_combine, "f32_attn_combine", dim3((unsigned)((rows * (D / 4) + 255) / 256)),
                      dim3(256), 0, FCombineArgs{a, D});
    for (int kk : {k, kc}) {
      b.ws_ref(kk, TH_OFFSET(FArgs, part), at_o);
      b.ws_ref(kk, TH_OFFSET(FArgs, part_ml), at_ml);
    }
    b.ref(3, kc, TH_OFFSET(FArgs, o));
    b.ref(4, kc, TH_OFFSET(FArgs, lse));
  }
  for (int v = 0; v < 4; ++v) b.align(v, 16);
  const double BH = (double)d->batch * d->heads, BHk = (double)d->batch * d->kv_heads;
  b.work(2.0 * BH * a.seq * D * 4 + 2.0 * BHk * a.kv_seq * D * 4 + 4.0 * BH * a.seq, 4.0 * BH * D * visible_pairs(a),
         (int64_t)grid.x * grid.y * grid.z);
  *out = b.release();
  return TH_OK;
}

template <int D>
int bwd_launch(const th_attention_desc* d, th_launch** out) {
  const size_t lds_kv = 4 * (size_t)kTileF<D> * sizeof(float);
  const size_t lds_dkdv = lds_kv + 2 * 128 * sizeof(float);
  TH_HIP(hipFuncSetAttribute((const void*)f32_attn_dkdv<D>, hipFuncAttributeMaxDynamicSharedMemorySize,
                             (int)lds_dkdv));
  TH_HIP(hipFuncSetAttribute((const void*)f32_attn_dq<D>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_kv));
  FArgs a = fargs_of(d);
  th::Builder b("attention_bwd_f32mfma", 11);
  const int64_t rows = (int64_t)d->batch * d->seq * d->heads;
  const int64_t rows_k = (int64_t)d->batch * a.kv_seq * d->kv_heads;
  const uint64_t at_delta = b.workspace((uint64_t)rows * sizeof(float));
  // Small grids split the dK/dV sweep over queries and the dQ sweep over keys.
  const int nkb = (a.kv_seq + 127) / 128, nqb = (d->seq + 127) / 128;
  const th::Split skv = th::split_of((int64_t)nkb * d->kv_heads * d->batch, d->seq);
  const th::Split sq = th::split_of((int64_t)nqb * d->heads * d->batch, a.kv_seq);
  TH_REQUIRE((int64_t)d->batch * std::max(skv.n, sq.n) <= 65535, "attention: grid too large");
  FArgs akv = a, aq = a;
  akv.nsplit = skv.n, akv.span = skv.span;
  aq.nsplit = sq.n, aq.span = sq.span;
  TH_REQUIRE(rows < 2147483648LL, "attention: batch x seq x heads must be under 2^31");
  constexpr int kDeltaBlockRows = 4 * (64 / (D / 4)) * kDeltaRowsF;  // rows a workgroup
  int k0 = b.kernel((const void*)f32_attn_delta<D>, "f32_attn_delta",
                    dim3((unsigned)((rows + kDeltaBlockRows - 1) / kDeltaBlockRows)), dim3(256), 0, FDeltaArgs{a, D});
  const dim3 gkv = skv.n > 1 ? dim3(nkb, d->kv_heads, d->batch * skv.n) : dim3(blocks_of(a.kv_seq, d->causal), d->kv_heads, d->batch);
  const dim3 gq = sq.n > 1 ? dim3(nqb, d->heads, d->batch * sq.n) : dim3(blocks_of(d->seq, d->causal), d->heads, d->batch);
  int k1 = b.kernel((const void*)f32_attn_dkdv<D>, D == 64 ? "f32_attn_dkdv_d64" : "f32_attn_dkdv_d128", gkv,
                    dim3(256), (uint32_t)lds_dkdv, akv);
  if (skv.n > 1) {
    const uint64_t at_kv = b.workspace((uint64_t)2 * skv.n * rows_k * D * sizeof(float));
    b.ws_ref(k1, TH_OFFSET(FArgs, part), at_kv);
    const unsigned g = (unsigned)((rows_k * (D / 4) + 255) / 256);
    // The outputs' pointers start as the descriptor's (repointing rewrites them with the others).
    FSumArgs sk{nullptr, static_cast<float*>(d->dk), d->k_strides[0], d->k_strides[1], d->k_strides[2], a.kv_seq,
                d->kv_heads, d->batch, D, skv.n, a.scale};
    FSumArgs sv = sk;
    sv.out = static_cast<float*>(d->dv), sv.scale = 1.0f;
    const int ks = b.kernel((const void*)f32_attn_sum, "f32_attn_sum_dk", dim3(g), dim3(256), 0, sk);
    const int kv = b.kernel((const void*)f32_attn_sum, "f32_attn_sum_dv", dim3(g), dim3(256), 0, sv);
    b.ws_ref(ks, TH_OFFSET(FSumArgs, part), at_kv);
    b.ws_ref(kv, TH_OFFSET(FSumArgs, part), at_kv + (uint64_t)skv.n * rows_k * D * sizeof(float));
    b.ref(7, ks, TH_OFFSET(FSumArgs, out));
    b.ref(8, kv, TH_OFFSET(FSumArgs, out));
  }
  int k2 = b.kernel((const void*)f32_attn_dq<D>, D == 64 ? "f32_attn_dq_d64" : "f32_attn_dq_d128", gq, dim3(256),
                    (uint32_t)lds_kv, aq);
  if (sq.n > 1) {
    const uint64_t at_q = b.workspace((uint64_t)sq.n * rows * D * sizeof(float));
    b.ws_ref(k2, TH_OFFSET(FArgs, part), at_q);
    FSumArgs s1{nullptr, static_cast<float*>(d->dq), d->q_strides[0], d->q_strides[1], d->q_strides[2], d->seq,
                d->heads, d->batch, D, sq.n, a.scale};
    const int kq = b.kernel((const void*)f32_attn_sum, "f32_attn_sum_dq", dim3((unsigned)((rows * (D / 4) + 255) / 256)),
                            dim3(256), 0, s1);
    b.ws_ref(kq, TH_OFFSET(FSumArgs, part), at_q);
    b.ref(6, kq, TH_OFFSET(FSumArgs, out));
  }
  const size_t offs[9] = {TH_OFFSET(FArgs, q),  TH_OFFSET(FArgs, k),  TH_OFFSET(FArgs, v),
                          TH_OFFSET(FArgs, o),  TH_OFFSET(FArgs, lse), TH_OFFSET(FArgs, dout),
                          TH_OFFSET(FArgs, dq), TH_OFFSET(FArgs, dk),  TH_OFFSET(FArgs, dv)};
  // The delta kernel's arguments are FArgs followed by d: the same offsets.
  for (int v = 0; v < 9; ++v)
    for (int kk : {k0, k1, k2}) b.ref(v, kk, offs[v]);
  for (int kk : {k0, k1, k2}) b.ws_ref(kk, TH_OFFSET(FArgs, delta), at_delta);
  for (int v : {0, 1, 2, 3, 5, 6, 7, 8}) b.align(v, 16);
  const double BH = (double)d->batch * d->heads, BHk = (double)d->batch * d->kv_heads;
  b.work(2.0 * BH * a.seq * D * 8 + 2.0 * BHk * a.kv_seq * D * 8 + 8.0 * BH * a.seq,
         2.5 * 4.0 * BH * D * visible_pairs(a), (int64_t)gkv.x * gkv.y * gkv.z);
  *out = b.release();
  return TH_OK;
}

}  // namespace

namespace th {

// fp32 arrays, head dim 64 or 128, positive lengths, no device-held masks,
// 16-byte aligned operands and rows (strides multiples of 4 floats).
bool f32_attention_takes(const th_attention_desc* d) {
  if (!d || !(d->flags & TH_ATTN_F32) || d->starts || d->lengths) return false;
  if (d->head_dim != 64 && d->head_dim != 128) return false;
  if (d->seq < 1 || d->kv_seq < 0 || d->batch < 1 || d->heads < 1 || d->kv_heads < 1 || d->heads % d->kv_heads)
    return false;
  for (int64_t s : {d->q_strides[0], d->q_strides[1], d->q_strides[2], d->k_strides[0], d->k_strides[1], d->k_strides[2]})
    if (s <= 0 || s % 4) return false;
  for (const void* ptr : {(const void*)d->q, (const void*)d->k, (const void*)d->v, (const void*)d->o,
                          (const void*)d->dout, (const void*)d->dq, (const void*)d->dk, (const void*)d->dv})
    if (!aligned16(ptr)) return false;
  const int64_t kv = d->kv_seq > 0 ? d->kv_seq : d->seq;
  return (d->seq + 127) / 128 <= 0x7fffffff && (kv + 127) / 128 <= 0x7fffffff && d->heads <= 65535 &&
         d->batch <= 65535;
}

int build_attention_f32_fwd(const th_attention_desc* d, th_launch** out) {
  TH_REQUIRE(d->q && d->k && d->v && d->o, "attention: null q, k, v or o");
  return d->head_dim == 64 ? fwd_launch<64>(d, out) : fwd_launch<128>(d, out);
}

int build_attention_f32_bwd(const th_attention_desc* d, th_launch** out) {
  TH_REQUIRE(d->q && d->k && d->v && d->o, "attention: null q, k, v or o");
  TH_REQUIRE(d->lse && d->dout && d->dq && d->dk && d->dv, "attention backward: null lse, dout, dq, dk or dv");
  return d->head_dim == 64 ? bwd_launch<64>(d, out) : bwd_launch<128>(d, out);
}

}  // namespace th
