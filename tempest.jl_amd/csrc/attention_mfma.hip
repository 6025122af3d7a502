// Op class (c) on the matrix cores at head dims 64, 128 and 256 and any
// lengths: what the tuned kernels of attention.hip (head dim 128, lengths in
// 128s) do not take, short of fp32 arrays and device-held masks, which stay
// on attention_generic.hip.  The reference's cuDNN claim takes half
// precision d <= 256 on tensor cores (ext/cuDNNExt.jl:90-100) and its cuTile
// sweep any tile (ext/cuTileExt/build.jl:326-493); d = 64 and d = 256 are
// the head dims models use beside 128.
//
// bf16 operands, v_mfma_f32_32x32x16_bf16, fp32 statistics; the forms of the
// tuned kernels, simpler: tiles of 64 positions x D in LDS as plain rows of
// D + 8 bf16 (16-byte reads along a row, ds_read_b64_tr_b16 down a column),
// staged through registers one step ahead (zeros past the sequence), one
// barrier a step.
//   forward: a workgroup of four waves per 128 queries, 32 a wave; S' = K Q'
//     (keys on registers, queries on lanes), online softmax in exp2 units,
//     O' += V' P' with P rounded to bf16 (folds.jl:186-222), lse = m + log(l);
//   backward (FA2's formulas, deterministic, no workspace beyond delta):
//     dK, dV: a workgroup per 128 keys (32 a wave, K and V rows in registers)
//     sweeping the query tiles of each query head of its group, S = Q K',
//     dP = dO V', P = exp(S - lse), dS = P (dP - delta), dV' += dO' P,
//     dK' += Q' dS; at d = 256 each workgroup keeps half of dK' and dV'
//     (grid twice as wide, the scores computed by both halves) so that its
//     accumulators fit one wave's registers;
//     dQ: a workgroup per 128 queries sweeping key tiles, S' and dP'
//     recomputed, dQ' += K' dS'.
// Masks: keys past the keys' length and, causal, keys after the query
// (key <= query, positions from 0) weigh 0; queries past the sequence are
// computed on zeros and not stored.
#include <hip/hip_runtime.h>

#include <cmath>

#include "th_core.h"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

struct MArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  float* lse;  // natural log, [b][s][h]
  const uint16_t* dout;
  float* delta;  // backward workspace: rowsum(dO .* O), [b][s][h]
  uint16_t* dq;
  uint16_t* dk;
  uint16_t* dv;
  int64_t q_sh, q_ss, q_sb;  // strides (elements) of q, o, dout, dq
  int64_t k_sh, k_ss, k_sb;  // strides of k, v, dk, dv
  int32_t seq, kv_seq, heads, kv_heads, batch, causal;
  float scale;
  // A sweep split into parts (small grids): nsplit parts of `span`
  // positions (a multiple of 64) each, fp32 partial results in `part`
  // ([part][b][position][head][d]) and, for the forward, (m, l) in
  // `part_ml`; nsplit <= 1: no split.
  int32_t nsplit, span;
  float* part;
  float* part_ml;
};

__device__ __forceinline__ float bf16_float(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
}
// The value lane l ^ 32 holds.
__device__ __forceinline__ float other_half(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(threadIdx.x % 64 < 32 ? r[1] : r[0]);
}
__device__ __forceinline__ f32x16 mfma(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// A operand from a tile (rows of D + 8 bf16), M along its rows: rows
// r0 + lane % 32, k = columns 16 ks + 8 (lane / 32) + (0..7).
template <int D>
__device__ __forceinline__ bf16x8 frag_rows(const uint16_t* t, int r0, int ks) {
  const int lane = threadIdx.x % 64;
  return *reinterpret_cast<const bf16x8*>(t + (r0 + lane % 32) * (D + 8) + 16 * ks + 8 * (lane / 32));
}

// A operand from a tile, M along its columns: m = column d0 + lane % 32, k
// = the 16 rows of step ks in the order the accumulator's registers give the
// B operand (k-slot 8 h + e <-> row 16 ks + 8 (e / 4) + 4 h + e % 4, h =
// lane / 32).  ds_read_b64_tr_b16 hands lane i of each 16 element i % 4 of
// the 8-byte pieces addressed by lanes 4 k + i / 4; lane j here addresses row
// base + j / 4, columns dgrp + 4 (j % 4) + (0..3), so lane i receives rows
// base + (0..3) of column dgrp + i; two reads cover the eight rows.
template <int D>
__device__ __forceinline__ bf16x8 frag_tr(const uint16_t* t, int d0, int ks) {
  const int lane = threadIdx.x % 64, j = lane % 16;
  const int col = d0 + 16 * ((lane / 16) % 2) + 4 * (j % 4);
  const int row = 16 * ks + 4 * (lane / 32) + j / 4;
  const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(t + row * (D + 8) + col));
  const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(t + (row + 8) * (D + 8) + col));
  const s16x8 w = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return __builtin_bit_cast(bf16x8, w);
}

// A row of a (position-major) operand as the B operand of a product over d:
// d = 16 ks + 8 (lane / 32) + (0..7); zeros for a position past the end.
template <int D>
__device__ __forceinline__ void row_operand(const uint16_t* row, bool live, bf16x8 (&f)[D / 16]) {
  const int lane = threadIdx.x % 64;
#pragma unroll
  for (int ks = 0; ks < D / 16; ++ks)
    f[ks] = live ? *reinterpret_cast<const bf16x8*>(row + 16 * ks + 8 * (lane / 32)) : bf16x8{};
}

// A 64-position tile of an operand staged through registers: thread t holds
// the 16-byte chunks t + 256 i; rows past `limit` read as zeros.
template <int D>
struct Stage {
  static constexpr int kChunks = D / 8;          // per row
  static constexpr int kPer = 64 * kChunks / 256;  // per thread
  u32x4 r[kPer];
  __device__ void load(const uint16_t* base, int64_t ss, int row0, int limit) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int c = threadIdx.x + 256 * i, row = c / kChunks, col = c % kChunks;
      r[i] = row0 + row < limit ? *reinterpret_cast<const u32x4*>(base + (int64_t)(row0 + row) * ss + 8 * col)
                                : u32x4{0, 0, 0, 0};
    }
  }
  __device__ void store(uint16_t* t) const {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int c = threadIdx.x + 256 * i, row = c / kChunks, col = c % kChunks;
      *reinterpret_cast<u32x4*>(t + row * (D + 8) + 8 * col) = r[i];
    }
  }
};

template <int D>
constexpr int kTile = 64 * (D + 8);  // bf16 elements of a tile in LDS

// Causal sweeps do less work for earlier query blocks (and later key
// blocks): workgroup x takes blocks x and nb - 1 - x, so every workgroup
// sweeps about the same number of tiles.
__device__ __forceinline__ int passes(bool causal, int x, int nb) { return causal && 2 * x + 1 != nb ? 2 : 1; }
__device__ __forceinline__ int block_of(int pass, int x, int nb) { return pass == 0 ? x : nb - 1 - x; }

// ---- forward ---------------------------------------------------------------------

// Keys [k_lo, k_hi) of query block qb: all of them (split < 0), or part
// `split` of the sweep, which leaves its unnormalised O' and (m, l) for the
// combining kernel.
template <int D>
__device__ __forceinline__ void fwd_block(const MArgs& p, const int qb, const int b, const int split) {
  constexpr int NS = D / 16, NB = D / 32;
  extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
  const int h = blockIdx.y;
  const int hk = h / (p.heads / p.kv_heads);
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64, lr = lane % 32, lh = lane / 32;
  const int q0 = qb * 128 + wave * 32, query = q0 + lr;
  const uint16_t* qbase = p.q + (int64_t)b * p.q_sb + (int64_t)h * p.q_sh;
  const uint16_t* kbase = p.k + (int64_t)b * p.k_sb + (int64_t)hk * p.k_sh;
  const uint16_t* vbase = p.v + (int64_t)b * p.k_sb + (int64_t)hk * p.k_sh;
  bf16x8 qf[NS];
  row_operand<D>(qbase + (int64_t)query * p.q_ss, query < p.seq, qf);
  f32x16 o[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) o[i] = f32x16{};
  float m = -INFINITY, l = 0.0f;
  const float c = p.scale * kLog2e;
  const int qlast = min(qb * 128 + 127, p.seq - 1);
  const int kend = p.causal ? min(p.kv_seq, qlast + 1) : p.kv_seq;
  const int k_lo = split < 0 ? 0 : split * p.span, k_hi = split < 0 ? kend : min(kend, k_lo + p.span);
  const int nsteps = k_hi > k_lo ? (k_hi - k_lo + 63) / 64 : 0;
  Stage<D> sk, sv;
  auto K = [&](int s) { return lds + 2 * s * kTile<D>; };
  auto V = [&](int s) { return lds + (2 * s + 1) * kTile<D>; };
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
    // S' (64 keys x 32 queries): keys 32 kb + 8 (i / 4) + 4 lh + i % 4 in register i.
    f32x16 s[2] = {f32x16{}, f32x16{}};
#pragma unroll
    for (int ks = 0; ks < NS; ++ks)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) s[kb] = mfma(frag_rows<D>(K(cur), 32 * kb, ks), qf[ks], s[kb]);
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
    bf16x8 pf[4];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int part = 0; part < 2; ++part) {
        u32x4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float w0 = __builtin_amdgcn_exp2f(fmaf(s[kb][8 * part + 2 * e], c, -shift));
          const float w1 = __builtin_amdgcn_exp2f(fmaf(s[kb][8 * part + 2 * e + 1], c, -shift));
          l += w0 + w1;
          w[e] = pack2(w0, w1);
        }
        pf[2 * kb + part] = (bf16x8)w;
      }
    // O' (D x 32 queries) += V' P', the weights rounded to bf16.
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int db = 0; db < NB; ++db) o[db] = mfma(frag_tr<D>(V(cur), 32 * db, ks), pf[ks], o[db]);
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
    float* po = p.part + row * D;
#pragma unroll
    for (int db = 0; db < NB; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *reinterpret_cast<f32x4*>(po + 32 * db + 8 * g + 4 * lh) =
            f32x4{o[db][4 * g], o[db][4 * g + 1], o[db][4 * g + 2], o[db][4 * g + 3]};
    if (lh == 0) reinterpret_cast<f32x2*>(p.part_ml)[row] = f32x2{m, l};
    return;
  }
  const float inv = 1.0f / l;
  uint16_t* obase = p.o + (int64_t)b * p.q_sb + (int64_t)h * p.q_sh + (int64_t)query * p.q_ss;
#pragma unroll
  for (int db = 0; db < NB; ++db)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d = 32 * db + 8 * g + 4 * lh;
      *reinterpret_cast<u32x2*>(obase + d) =
          u32x2{pack2(o[db][4 * g] * inv, o[db][4 * g + 1] * inv), pack2(o[db][4 * g + 2] * inv, o[db][4 * g + 3] * inv)};
    }
  if (lh == 0 && p.lse) p.lse[((int64_t)b * p.seq + query) * p.heads + h] = (m + log2f(l)) * kLn2;
}

template <int D>
__global__ __launch_bounds__(256, D <= 128 ? 2 : 1) void mfma_attn_fwd(MArgs p) {
  // Split: one part of one block; else a block and, causal, its mirror (one call site, inlined once).
  const bool split = p.nsplit > 1;
  const int nb = (p.seq + 127) / 128;
  const int npass = split ? 1 : passes(p.causal, blockIdx.x, nb);
  for (int pass = 0; pass < npass; ++pass) {
    if (pass > 0) __syncthreads();
    fwd_block<D>(p, split ? blockIdx.x : block_of(pass, blockIdx.x, nb), split ? blockIdx.z / p.nsplit : blockIdx.z,
                 split ? blockIdx.z % p.nsplit : -1);
  }
}

// The parts of a split forward combined: per (b, query, head) row, M = max
// m_s, L = sum l_s 2^(m_s - M), O = sum O_s 2^(m_s - M) / L in part order;
// lse = (M + log2 L) ln 2.  A thread per four features of a row.
struct CombineArgs {
  MArgs p;  // first: its members sit at MArgs' offsets
  int32_t d;
};

__global__ __launch_bounds__(256) void mfma_attn_combine(CombineArgs a) {
  const MArgs& p = a.p;
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
  const float inv = 1.0f / l;
  *reinterpret_cast<u32x2*>(p.o + b * p.q_sb + h * p.q_sh + pos * p.q_ss + c) =
      u32x2{pack2(acc[0] * inv, acc[1] * inv), pack2(acc[2] * inv, acc[3] * inv)};
  if (c == 0 && p.lse) p.lse[row] = (mx + log2f(l)) * kLn2;
}

// dQ, dK or dV from a split sweep's parts: out = scale * sum_s part_s in
// part order, rounded to bf16; rows [b][position][head] of `d` features.
struct SumArgs {
  const float* part;
  uint16_t* out;
  int64_t sh, ss, sb;
  int32_t positions, heads, batch, d, nsplit;
  float scale;
};

__global__ __launch_bounds__(256) void mfma_attn_sum(SumArgs a) {
  const int quads = a.d / 4;
  const int64_t rows = (int64_t)a.batch * a.positions * a.heads;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= rows * quads) return;
  const int64_t row = t / quads;
  const int c = 4 * (int)(t % quads);
  // Part s of this quad at a.part + (s rows + row) d + c: a stride of rows d / 4 quads.
  f32x4 acc = thd::sum_in_order(reinterpret_cast<const f32x4*>(a.part + row * a.d + c), rows * a.d / 4, a.nsplit);
  acc *= a.scale;
  const int h = (int)(row % a.heads);
  const int64_t pos = (row / a.heads) % a.positions, b = row / ((int64_t)a.heads * a.positions);
  *reinterpret_cast<u32x2*>(a.out + b * a.sb + h * a.sh + pos * a.ss + c) =
      u32x2{pack2(acc[0], acc[1]), pack2(acc[2], acc[3])};
}

// ---- backward: delta = rowsum(dO .* O) ---------------------------------------------

struct DeltaArgs {
  MArgs p;  // first: its members sit at MArgs' offsets
  int32_t d;
};

// D / 8 lanes per (batch, position, head) row, 16 bytes each (the builder
// checks the strides and bases for it); each lane group takes kDeltaRowsM
// rows, 64 / (D / 8) apart, every load issued before the first product.
// Rows are numbered with the head fastest, so a load instruction covers
// consecutive rows; row numbers fit 32 bits (the builder checks).
constexpr int kDeltaRowsM = 4;

template <int D>
__global__ __launch_bounds__(256) void mfma_attn_delta(DeltaArgs a) {
  constexpr int G = D / 8;        // lanes a row
  constexpr int R = 64 / G;       // rows a wave covers at once
  const MArgs& p = a.p;
  const uint32_t total = (uint32_t)p.batch * p.seq * p.heads;
  const int lane = threadIdx.x % 64, part = lane % G;
  const uint32_t row0 = (blockIdx.x * 4 + threadIdx.x / 64) * (R * kDeltaRowsM) + lane / G;
  auto at_of = [&](uint32_t row) {
    const uint32_t bs = row / (uint32_t)p.heads;
    const int64_t b = bs / (uint32_t)p.seq, s = bs % (uint32_t)p.seq, h = row - bs * (uint32_t)p.heads;
    return b * p.q_sb + h * p.q_sh + s * p.q_ss + 8 * part;
  };
  u32x4 ow[kDeltaRowsM], gw[kDeltaRowsM];
#pragma unroll
  for (int i = 0; i < kDeltaRowsM; ++i) {
    // Rows past the end re-read the last one; nothing is written for them.
    const int64_t at = at_of(min(row0 + R * i, total - 1));
    ow[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p.o + at));
    gw[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p.dout + at));
  }
  // Every load out before any of their data is used.
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < kDeltaRowsM; ++i) {
    float v = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      v += bf16_float((uint16_t)ow[i][e]) * bf16_float((uint16_t)gw[i][e]) +
           bf16_float((uint16_t)(ow[i][e] >> 16)) * bf16_float((uint16_t)(gw[i][e] >> 16));
#pragma unroll
    for (int m = G / 2; m >= 1; m /= 2) v += __shfl_xor(v, m, G);
    const uint32_t row = row0 + R * i;
    if (row < total && part == 0) p.delta[row] = v;
  }
}

// ---- backward: dK, dV ----------------------------------------------------------------
// A workgroup takes 128 keys (32 a wave) and DO of the D features of dK and
// dV (D, or half of 256).  Per query tile of 64: S (64 queries x 32 keys)
// with queries on the registers and keys on the lanes, so that P and dS feed
// the products over queries straight from the accumulators.

// Query tiles [qstart, qstop) for the keys of kblk: all of them (split <
// 0), or part `split` of the sweep, which leaves its unscaled fp32 dK', dV'.
template <int D, int DO>
__device__ __forceinline__ void dkdv_block(const MArgs& p, const int kblk, const int dh, const int b,
                                           const int split) {
  constexpr int NS = D / 16, NBO = DO / 32;
  extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
  float* stats = reinterpret_cast<float*>(lds + 4 * kTile<D>);  // [stage][lse * log2e (64) | delta (64)]
  const int hk = blockIdx.y;
  const int group = p.heads / p.kv_heads;
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64, lr = lane % 32, lh = lane / 32;
  const int kw0 = kblk * 128, key = kw0 + wave * 32 + lr;
  const int64_t koff = (int64_t)b * p.k_sb + (int64_t)hk * p.k_sh;
  bf16x8 kf[NS], vf[NS];
  row_operand<D>(p.k + koff + (int64_t)key * p.k_ss, key < p.kv_seq, kf);
  row_operand<D>(p.v + koff + (int64_t)key * p.k_ss, key < p.kv_seq, vf);
  f32x16 dk[NBO], dv[NBO];
#pragma unroll
  for (int i = 0; i < NBO; ++i) dk[i] = f32x16{}, dv[i] = f32x16{};
  const float c = p.scale * kLog2e;
  auto Q = [&](int s) { return lds + 2 * s * kTile<D>; };
  auto G = [&](int s) { return lds + (2 * s + 1) * kTile<D>; };
  auto Ls = [&](int s) { return stats + 128 * s; };
  const int qfirst = p.causal ? kw0 / 64 * 64 : 0;
  const int qstart = split < 0 ? qfirst : qfirst + split * p.span;
  const int qstop = split < 0 ? p.seq : min(p.seq, qstart + p.span);
  const int nsteps = qstart < qstop ? (qstop - qstart + 63) / 64 : 0;
  Stage<D> sq, sg;
  float st = 0.0f;  // threads 0..127: a query's lse * log2e or delta
  auto load = [&](const uint16_t* qbase, const uint16_t* gbase, int h, int q0) {
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
    const uint16_t* qbase = p.q + (int64_t)b * p.q_sb + (int64_t)h * p.q_sh;
    const uint16_t* gbase = p.dout + (int64_t)b * p.q_sb + (int64_t)h * p.q_sh;
    if (nsteps > 0) {
      load(qbase, gbase, h, qstart);
      store(0);
    }
    __syncthreads();
    for (int j = 0; j < nsteps; ++j) {
      const int cur = j & 1, qq0 = qstart + 64 * j;
      if (j + 1 < nsteps) load(qbase, gbase, h, qq0 + 64);
      const uint16_t *Qt = Q(cur), *Gt = G(cur);
      const float* L = Ls(cur);
      // S = Q K', dP = dO V' (64 queries x 32 keys): query 32 jj + 8 (i / 4) + 4 lh + i % 4 in register i.
      f32x16 s[2] = {f32x16{}, f32x16{}}, dp[2] = {f32x16{}, f32x16{}};
#pragma unroll
      for (int ks = 0; ks < NS; ++ks)
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
          s[jj] = mfma(frag_rows<D>(Qt, 32 * jj, ks), kf[ks], s[jj]);
          dp[jj] = mfma(frag_rows<D>(Gt, 32 * jj, ks), vf[ks], dp[jj]);
        }
      bf16x8 pf[4], sf[4];
#pragma unroll
      for (int jj = 0; jj < 2; ++jj)
#pragma unroll
        for (int part = 0; part < 2; ++part) {
          u32x4 wp, wd;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float w[2], x[2];
#pragma unroll
            for (int u = 0; u < 2; ++u) {
              const int i = 8 * part + 2 * e + u;
              const int qi = 32 * jj + 8 * (i / 4) + 4 * lh + i % 4, query = qq0 + qi;
              const bool seen = query < p.seq && key < p.kv_seq && (!p.causal || key <= query);
              w[u] = seen ? __builtin_amdgcn_exp2f(fmaf(s[jj][i], c, -L[qi])) : 0.0f;
              x[u] = w[u] * (dp[jj][i] - L[64 + qi]);
            }
            wp[e] = pack2(w[0], w[1]);
            wd[e] = pack2(x[0], x[1]);
          }
          pf[2 * jj + part] = (bf16x8)wp;
          sf[2 * jj + part] = (bf16x8)wd;
        }
      // dV' (DO features x 32 keys) += dO' P;  dK' += Q' dS.
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int db = 0; db < NBO; ++db) {
          dv[db] = mfma(frag_tr<D>(Gt, DO * dh + 32 * db, ks), pf[ks], dv[db]);
          dk[db] = mfma(frag_tr<D>(Qt, DO * dh + 32 * db, ks), sf[ks], dk[db]);
        }
      if (j + 1 < nsteps) store(cur ^ 1);
      __syncthreads();
    }
  }
  // At D = 128 the key as an opaque copy, so that the output addresses below
  // are computed here rather than kept from the sweep's start: measured 4 %
  // faster there; at D = 64 (4 registers spilled around the sweep otherwise)
  // and D = 256 the kept addresses measured faster.
  int ko = key;
  if constexpr (D == 128) asm volatile("" : "+v"(ko));
  if (ko >= p.kv_seq) return;
  if (split >= 0) {
    const int64_t rows = (int64_t)p.batch * p.kv_seq * p.kv_heads;
    const int64_t row = (((int64_t)split * p.batch + b) * p.kv_seq + ko) * p.kv_heads + hk;
    float* pk = p.part + row * D;
    float* pv = p.part + ((int64_t)p.nsplit * rows + row) * D;
#pragma unroll
    for (int db = 0; db < NBO; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = DO * dh + 32 * db + 8 * g + 4 * lh;
        *reinterpret_cast<f32x4*>(pk + d) = f32x4{dk[db][4 * g], dk[db][4 * g + 1], dk[db][4 * g + 2], dk[db][4 * g + 3]};
        *reinterpret_cast<f32x4*>(pv + d) = f32x4{dv[db][4 * g], dv[db][4 * g + 1], dv[db][4 * g + 2], dv[db][4 * g + 3]};
      }
    return;
  }
  const int64_t out = koff + (int64_t)ko * p.k_ss;
#pragma unroll
  for (int db = 0; db < NBO; ++db)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d = DO * dh + 32 * db + 8 * g + 4 * lh;
      const float sc = p.scale;
      *reinterpret_cast<u32x2*>(p.dk + out + d) =
          u32x2{pack2(dk[db][4 * g] * sc, dk[db][4 * g + 1] * sc), pack2(dk[db][4 * g + 2] * sc, dk[db][4 * g + 3] * sc)};
      *reinterpret_cast<u32x2*>(p.dv + out + d) =
          u32x2{pack2(dv[db][4 * g], dv[db][4 * g + 1]), pack2(dv[db][4 * g + 2], dv[db][4 * g + 3])};
    }
}

template <int D, int DO>
__global__ __launch_bounds__(256, D <= 64 ? 2 : 1) void mfma_attn_dkdv(MArgs p) {
  constexpr int halves = D / DO;
  const bool split = p.nsplit > 1;
  const int nb = (p.kv_seq + 127) / 128, x = blockIdx.x / halves;
  const int npass = split ? 1 : passes(p.causal, x, nb);
  for (int pass = 0; pass < npass; ++pass) {
    if (pass > 0) __syncthreads();
    dkdv_block<D, DO>(p, split ? x : block_of(pass, x, nb), blockIdx.x % halves, split ? blockIdx.z / p.nsplit : blockIdx.z,
                      split ? blockIdx.z % p.nsplit : -1);
  }
}

// ---- backward: dQ ----------------------------------------------------------------------
// A workgroup takes 128 queries (32 a wave) and sweeps key tiles of 64:
// S' = K Q', dP' = V dO' (keys on the registers, queries on the lanes),
// dS' = P' (dP' - delta), dQ' (D x 32 queries) += K' dS'.

// Keys [k_lo, k_hi) for query block qb: all of them (split < 0), or part
// `split` of the sweep, which leaves its unscaled fp32 dQ'.
template <int D>
__device__ __forceinline__ void dq_block(const MArgs& p, const int qb, const int b, const int split) {
  constexpr int NS = D / 16, NB = D / 32;
  extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
  const int h = blockIdx.y;
  const int hk = h / (p.heads / p.kv_heads);
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64, lr = lane % 32, lh = lane / 32;
  const int q0 = qb * 128 + wave * 32, query = q0 + lr;
  const int64_t qoff = (int64_t)b * p.q_sb + (int64_t)h * p.q_sh + (int64_t)query * p.q_ss;
  const bool live = query < p.seq;
  bf16x8 qf[NS], gf[NS];
  row_operand<D>(p.q + qoff, live, qf);
  row_operand<D>(p.dout + qoff, live, gf);
  const int64_t srow = ((int64_t)b * p.seq + query) * p.heads + h;
  const float l2 = live ? p.lse[srow] * kLog2e : 0.0f;
  const float dl = live ? p.delta[srow] : 0.0f;
  const float c = p.scale * kLog2e;
  const uint16_t* kbase = p.k + (int64_t)b * p.k_sb + (int64_t)hk * p.k_sh;
  const uint16_t* vbase = p.v + (int64_t)b * p.k_sb + (int64_t)hk * p.k_sh;
  f32x16 dq[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) dq[i] = f32x16{};
  const int qlast = min(qb * 128 + 127, p.seq - 1);
  const int kend = p.causal ? min(p.kv_seq, qlast + 1) : p.kv_seq;
  const int k_lo = split < 0 ? 0 : split * p.span, k_hi = split < 0 ? kend : min(kend, k_lo + p.span);
  const int nsteps = k_hi > k_lo ? (k_hi - k_lo + 63) / 64 : 0;
  Stage<D> sk, sv;
  auto K = [&](int s) { return lds + 2 * s * kTile<D>; };
  auto V = [&](int s) { return lds + (2 * s + 1) * kTile<D>; };
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
    f32x16 s[2] = {f32x16{}, f32x16{}}, dp[2] = {f32x16{}, f32x16{}};
#pragma unroll
    for (int ks = 0; ks < NS; ++ks)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        s[kb] = mfma(frag_rows<D>(K(cur), 32 * kb, ks), qf[ks], s[kb]);
        dp[kb] = mfma(frag_rows<D>(V(cur), 32 * kb, ks), gf[ks], dp[kb]);
      }
    bf16x8 sf[4];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int part = 0; part < 2; ++part) {
        u32x4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float x[2];
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const int i = 8 * part + 2 * e + u;
            const int key = k0 + 32 * kb + 8 * (i / 4) + 4 * lh + i % 4;
            const bool seen = key < p.kv_seq && (!p.causal || key <= query);
            const float pw = seen ? __builtin_amdgcn_exp2f(fmaf(s[kb][i], c, -l2)) : 0.0f;
            x[u] = pw * (dp[kb][i] - dl);
          }
          w[e] = pack2(x[0], x[1]);
        }
        sf[2 * kb + part] = (bf16x8)w;
      }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int db = 0; db < NB; ++db) dq[db] = mfma(frag_tr<D>(K(cur), 32 * db, ks), sf[ks], dq[db]);
    if (j + 1 < nsteps) {
      sk.store(K(cur ^ 1));
      sv.store(V(cur ^ 1));
    }
    __syncthreads();
  }
  if (!live) return;
  if (split >= 0) {
    const int64_t row = (((int64_t)split * p.batch + b) * p.seq + query) * p.heads + h;
    float* pq = p.part + row * D;
#pragma unroll
    for (int db = 0; db < NB; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *reinterpret_cast<f32x4*>(pq + 32 * db + 8 * g + 4 * lh) =
            f32x4{dq[db][4 * g], dq[db][4 * g + 1], dq[db][4 * g + 2], dq[db][4 * g + 3]};
    return;
  }
  uint16_t* out = p.dq + qoff;
#pragma unroll
  for (int db = 0; db < NB; ++db)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d = 32 * db + 8 * g + 4 * lh;
      const float sc = p.scale;
      *reinterpret_cast<u32x2*>(out + d) =
          u32x2{pack2(dq[db][4 * g] * sc, dq[db][4 * g + 1] * sc), pack2(dq[db][4 * g + 2] * sc, dq[db][4 * g + 3] * sc)};
    }
}

template <int D>
__global__ __launch_bounds__(256, D <= 64 ? 2 : 1) void mfma_attn_dq(MArgs p) {
  const bool split = p.nsplit > 1;
  const int nb = (p.seq + 127) / 128;
  const int npass = split ? 1 : passes(p.causal, blockIdx.x, nb);
  for (int pass = 0; pass < npass; ++pass) {
    if (pass > 0) __syncthreads();
    dq_block<D>(p, split ? blockIdx.x : block_of(pass, blockIdx.x, nb), split ? blockIdx.z / p.nsplit : blockIdx.z,
                split ? blockIdx.z % p.nsplit : -1);
  }
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

// Workgroups along a sequence of n positions in blocks of 128: causal ones
// take a block and its mirror.
unsigned blocks_of(int n, int causal) {
  const unsigned nb = (unsigned)((n + 127) / 128);
  return causal ? (nb + 1) / 2 : nb;
}

MArgs margs_of(const th_attention_desc* d) {
  MArgs a{};
  a.q = static_cast<const uint16_t*>(d->q);
  a.k = static_cast<const uint16_t*>(d->k);
  a.v = static_cast<const uint16_t*>(d->v);
  a.o = static_cast<uint16_t*>(d->o);
  a.lse = d->lse;
  a.dout = static_cast<const uint16_t*>(d->dout);
  a.dq = static_cast<uint16_t*>(d->dq);
  a.dk = static_cast<uint16_t*>(d->dk);
  a.dv = static_cast<uint16_t*>(d->dv);
  a.q_sh = d->q_strides[0], a.q_ss = d->q_strides[1], a.q_sb = d->q_strides[2];
  a.k_sh = d->k_strides[0], a.k_ss = d->k_strides[1], a.k_sb = d->k_strides[2];
  a.seq = d->seq;
  a.kv_seq = d->kv_seq > 0 ? d->kv_seq : d->seq;
  a.heads = d->heads, a.kv_heads = d->kv_heads, a.batch = d->batch, a.causal = d->causal;
  a.scale = d->scale > 0 ? d->scale : 1.0f / sqrtf((float)d->head_dim);
  return a;
}

// (query, key) pairs the mask leaves: the algorithmic work's count.
double visible_pairs(const MArgs& a) {
  const double S = a.seq, K = a.kv_seq;
  if (!a.causal) return S * K;
  // sum over queries q of min(q + 1, K)
  const double full = std::min(S, K);
  return full * (full + 1) / 2 + std::max(0.0, S - K) * K;
}

template <int D>
int fwd_launch(const th_attention_desc* d, th_launch** out) {
  const size_t lds = 4 * (size_t)kTile<D> * sizeof(uint16_t);
  TH_HIP(hipFuncSetAttribute((const void*)mfma_attn_fwd<D>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
  MArgs a = margs_of(d);
  const int nqb = (d->seq + 127) / 128;
  const th::Split sp = th::split_of((int64_t)nqb * d->heads * d->batch, a.kv_seq);
  a.nsplit = sp.n, a.span = sp.span;
  TH_REQUIRE((int64_t)d->batch * sp.n <= 65535, "attention: grid too large");
  th::Builder b("attention_fwd_mfma", 7);
  const dim3 grid = sp.n > 1 ? dim3(nqb, d->heads, d->batch * sp.n) : dim3(blocks_of(d->seq, d->causal), d->heads, d->batch);
  int k = b.kernel((const void*)mfma_attn_fwd<D>, D == 64 ? "mfma_attn_fwd_d64" : D == 128 ? "mfma_attn_fwd_d128"
                                                                                          : "mfma_attn_fwd_d256",
                   grid, dim3(256), (uint32_t)lds, a);
  b.ref(0, k, TH_OFFSET(MArgs, q));
  b.ref(1, k, TH_OFFSET(MArgs, k));
  b.ref(2, k, TH_OFFSET(MArgs, v));
  b.ref(3, k, TH_OFFSET(MArgs, o));
  b.ref(4, k, TH_OFFSET(MArgs, lse));
  if (sp.n > 1) {
    const int64_t rows = (int64_t)d->batch * d->seq * d->heads;
    const uint64_t at_o = b.workspace((uint64_t)sp.n * rows * D * sizeof(float));
    const uint64_t at_ml = b.workspace((uint64_t)sp.n * rows * 2 * sizeof(float));
    int kc = b.kernel((const void*)mfma_attn_combine, "mfma_attn_combine", dim3((unsigned)((rows * (D / 4) + 255) / 256)),
                      dim3(256), 0, CombineArgs{a, D});
    for (int kk : {k, kc}) {
      b.ws_ref(kk, TH_OFFSET(MArgs, part), at_o);
      b.ws_ref(kk, TH_OFFSET(MArgs, part_ml), at_ml);
    }
    b.ref(3, kc, TH_OFFSET(MArgs, o));
    b.ref(4, kc, TH_OFFSET(MArgs, lse));
  }
  for (int v = 0; v < 4; ++v) b.align(v, 16);
  const double BH = (double)d->batch * d->heads, BHk = (double)d->batch * d->kv_heads;
  b.work(2.0 * BH * a.seq * D * 2 + 2.0 * BHk * a.kv_seq * D * 2 + 4.0 * BH * a.seq, 4.0 * BH * D * visible_pairs(a),
         (int64_t)grid.x * grid.y * grid.z);
  *out = b.release();
  return TH_OK;
}

template <int D>
int bwd_launch(const th_attention_desc* d, th_launch** out) {
  constexpr int DO = D == 256 ? 128 : D;
  const size_t lds_kv = 4 * (size_t)kTile<D> * sizeof(uint16_t);
  const size_t lds_dkdv = lds_kv + 2 * 128 * sizeof(float);
  TH_HIP(hipFuncSetAttribute((const void*)mfma_attn_dkdv<D, DO>, hipFuncAttributeMaxDynamicSharedMemorySize,
                             (int)lds_dkdv));
  TH_HIP(hipFuncSetAttribute((const void*)mfma_attn_dq<D>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_kv));
  MArgs a = margs_of(d);
  th::Builder b("attention_bwd_mfma", 11);
  const int64_t rows = (int64_t)d->batch * d->seq * d->heads;
  const int64_t rows_k = (int64_t)d->batch * a.kv_seq * d->kv_heads;
  const uint64_t at_delta = b.workspace((uint64_t)rows * sizeof(float));
  // Small grids split the dK/dV sweep over queries and the dQ sweep over keys.
  const int nkb = (a.kv_seq + 127) / 128, nqb = (d->seq + 127) / 128;
  const th::Split skv = th::split_of((int64_t)nkb * (D / DO) * d->kv_heads * d->batch, d->seq);
  const th::Split sq = th::split_of((int64_t)nqb * d->heads * d->batch, a.kv_seq);
  TH_REQUIRE((int64_t)d->batch * std::max(skv.n, sq.n) <= 65535, "attention: grid too large");
  MArgs akv = a, aq = a;
  akv.nsplit = skv.n, akv.span = skv.span;
  aq.nsplit = sq.n, aq.span = sq.span;
  TH_REQUIRE(rows < 2147483648LL, "attention: batch x seq x heads must be under 2^31");
  constexpr int kDeltaBlockRows = 4 * (64 / (D / 8)) * kDeltaRowsM;  // rows a workgroup
  int k0 = b.kernel((const void*)mfma_attn_delta<D>, "mfma_attn_delta",
                    dim3((unsigned)((rows + kDeltaBlockRows - 1) / kDeltaBlockRows)), dim3(256), 0, DeltaArgs{a, D});
  const dim3 gkv = skv.n > 1 ? dim3(nkb * (D / DO), d->kv_heads, d->batch * skv.n)
                             : dim3(blocks_of(a.kv_seq, d->causal) * (D / DO), d->kv_heads, d->batch);
  const dim3 gq = sq.n > 1 ? dim3(nqb, d->heads, d->batch * sq.n) : dim3(blocks_of(d->seq, d->causal), d->heads, d->batch);
  int k1 = b.kernel((const void*)mfma_attn_dkdv<D, DO>, D == 64 ? "mfma_attn_dkdv_d64" : D == 128 ? "mfma_attn_dkdv_d128"
                                                                                               : "mfma_attn_dkdv_d256",
                    gkv, dim3(256), (uint32_t)lds_dkdv, akv);
  if (skv.n > 1) {
    const uint64_t at_kv = b.workspace((uint64_t)2 * skv.n * rows_k * D * sizeof(float));
    b.ws_ref(k1, TH_OFFSET(MArgs, part), at_kv);
    const unsigned g = (unsigned)((rows_k * (D / 4) + 255) / 256);
    // The outputs' pointers start as the descriptor's (repointing rewrites them with the others).
    SumArgs sk{nullptr, static_cast<uint16_t*>(d->dk), d->k_strides[0], d->k_strides[1], d->k_strides[2], a.kv_seq,
               d->kv_heads, d->batch, D, skv.n, a.scale};
    SumArgs sv = sk;
    sv.out = static_cast<uint16_t*>(d->dv), sv.scale = 1.0f;
    const int ks = b.kernel((const void*)mfma_attn_sum, "mfma_attn_sum_dk", dim3(g), dim3(256), 0, sk);
    const int kv = b.kernel((const void*)mfma_attn_sum, "mfma_attn_sum_dv", dim3(g), dim3(256), 0, sv);
    b.ws_ref(ks, TH_OFFSET(SumArgs, part), at_kv);
    b.ws_ref(kv, TH_OFFSET(SumArgs, part), at_kv + (uint64_t)skv.n * rows_k * D * sizeof(float));
    b.ref(7, ks, TH_OFFSET(SumArgs, out));
    b.ref(8, kv, TH_OFFSET(SumArgs, out));
  }
  int k2 = b.kernel((const void*)mfma_attn_dq<D>, D == 64 ? "mfma_attn_dq_d64" : D == 128 ? "mfma_attn_dq_d128"
                                                                                       : "mfma_attn_dq_d256",
                    gq, dim3(256), (uint32_t)lds_kv, aq);
  if (sq.n > 1) {
    const uint64_t at_q = b.workspace((uint64_t)sq.n * rows * D * sizeof(float));
    b.ws_ref(k2, TH_OFFSET(MArgs, part), at_q);
    SumArgs s1{nullptr, static_cast<uint16_t*>(d->dq), d->q_strides[0], d->q_strides[1], d->q_strides[2], d->seq,
               d->heads, d->batch, D, sq.n, a.scale};
    const int kq = b.kernel((const void*)mfma_attn_sum, "mfma_attn_sum_dq", dim3((unsigned)((rows * (D / 4) + 255) / 256)),
                            dim3(256), 0, s1);
    b.ws_ref(kq, TH_OFFSET(SumArgs, part), at_q);
    b.ref(6, kq, TH_OFFSET(SumArgs, out));
  }
  const size_t offs[9] = {TH_OFFSET(MArgs, q),  TH_OFFSET(MArgs, k),  TH_OFFSET(MArgs, v),
                          TH_OFFSET(MArgs, o),  TH_OFFSET(MArgs, lse), TH_OFFSET(MArgs, dout),
                          TH_OFFSET(MArgs, dq), TH_OFFSET(MArgs, dk),  TH_OFFSET(MArgs, dv)};
  // The delta kernel's arguments are MArgs followed by d: the same offsets.
  for (int v = 0; v < 9; ++v)
    for (int kk : {k0, k1, k2}) b.ref(v, kk, offs[v]);
  for (int kk : {k0, k1, k2}) b.ws_ref(kk, TH_OFFSET(MArgs, delta), at_delta);
  for (int v : {0, 1, 2, 3, 5, 6, 7, 8}) b.align(v, 16);
  const double BH = (double)d->batch * d->heads, BHk = (double)d->batch * d->kv_heads;
  b.work(2.0 * BH * a.seq * D * 4 + 2.0 * BHk * a.kv_seq * D * 4 + 8.0 * BH * a.seq,
         2.5 * 4.0 * BH * D * visible_pairs(a), (int64_t)gkv.x * gkv.y * gkv.z);
  *out = b.release();
  return TH_OK;
}

int check_mfma(const th_attention_desc* d, bool backward) {
  TH_REQUIRE(d->q && d->k && d->v && d->o, "attention: null q, k, v or o");
  TH_REQUIRE(aligned16(d->q) && aligned16(d->k) && aligned16(d->v) && aligned16(d->o),
             "attention: q, k, v, o must be 16-byte aligned");
  if (backward) {
    TH_REQUIRE(d->lse && d->dout && d->dq && d->dk && d->dv, "attention backward: null lse, dout, dq, dk or dv");
    TH_REQUIRE(aligned16(d->dout) && aligned16(d->dq) && aligned16(d->dk) && aligned16(d->dv),
               "attention backward: dout, dq, dk, dv must be 16-byte aligned");
  }
  return TH_OK;
}

}  // namespace

namespace th {

// bf16 arrays, head dim 64, 128 or 256, any positive lengths, no
// device-held masks, 16-byte rows, operands and strides.
bool mfma_attention_takes(const th_attention_desc* d) {
  if (!d || (d->flags & TH_ATTN_F32) || d->starts || d->lengths) return false;
  if (d->head_dim != 64 && d->head_dim != 128 && d->head_dim != 256) return false;
  if (d->seq < 1 || d->kv_seq < 0 || d->batch < 1 || d->heads < 1 || d->kv_heads < 1 || d->heads % d->kv_heads)
    return false;
  for (int64_t s : {d->q_strides[0], d->q_strides[1], d->q_strides[2], d->k_strides[0], d->k_strides[1], d->k_strides[2]})
    if (s <= 0 || s % 8) return false;
  const int64_t kv = d->kv_seq > 0 ? d->kv_seq : d->seq;
  return (d->seq + 127) / 128 <= 0x7fffffff && (kv + 127) / 128 * 2 <= 0x7fffffff && d->heads <= 65535 &&
         d->batch <= 65535;
}

int build_attention_mfma_fwd(const th_attention_desc* d, th_launch** out) {
  if (int r = check_mfma(d, false)) return r;
  switch (d->head_dim) {
    case 64: return fwd_launch<64>(d, out);
    case 128: return fwd_launch<128>(d, out);
    default: return fwd_launch<256>(d, out);
  }
}

int build_attention_mfma_bwd(const th_attention_desc* d, th_launch** out) {
  if (int r = check_mfma(d, true)) return r;
  switch (d->head_dim) {
    case 64: return bwd_launch<64>(d, out);
    case 128: return bwd_launch<128>(d, out);
    default: return bwd_launch<256>(d, out);
  }
}

}  // namespace th
