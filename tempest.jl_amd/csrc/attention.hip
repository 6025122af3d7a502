// Op class (c): causal flash attention, forward and backward, on CDNA4
// matrix cores (v_mfma_f32_32x32x16_bf16), bf16 operands, fp32 statistics.
//
// Arrays are the reference's (features, heads, positions, batch) column-major
// (test/fixtures/operations.jl:5-10): element (d, h, s, b) of a tensor with
// strides (1, sh, ss, sb).  Head dimension 128.  Query head h reads key/value
// head h / (heads / kv_heads) (grouped-query attention).
//
// Forward (replaces the cuTile online-softmax product sweep,
// ext/cuTileExt/build.jl:326-532, and cuDNN's SDPA, ext/cuDNNExt.jl:116-210):
// a workgroup of four waves takes 128 queries of one (head, batch); each wave
// 32 queries.  Scores are computed transposed, S' = K Q' (keys along the
// accumulator's registers, queries along its lanes), so that each query's
// running maximum and sum live in one lane.  Key blocks of 64 stream through
// LDS (double-buffered, the next block's loads in flight while the waves
// multiply): K row-major, V transposed into [d][key] with the keys of each
// 16 permuted so that a lane's eight keys of a product step are one 16-byte
// read, matching the registers the scores' accumulator gives it.  Weights are
// exp2((s - m) * log2e / sqrt(d)), rounded to bf16 before O' += V' P', and the
// accumulator rescaled when the maximum grows (folds.jl:186-222).  Causal key
// blocks past the diagonal are not visited; the diagonal block is masked.
// Query blocks run heaviest first (ext/cuTileExt/mask.jl:205).
//
// Backward (replaces ext/cuTileExt/transpose.jl): FA2's formulas, computed
// without atomics so the result does not depend on timing:
//   delta = rowsum(dO .* O);  P = exp(S - lse);  dP = dO V';
//   dS = P .* (dP - delta);  dV = P' dO;  dK = dS' Q / sqrt(d);  dQ = dS K / sqrt(d)
// one kernel sweeps query blocks for each key block (dK, dV), another sweeps
// key blocks for each query block (dQ).
#include <hip/hip_runtime.h>

#include <cmath>

#include "th_core.h"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kD = 128;        // head dimension
constexpr int kRowN = kD + 8;  // LDS row of a [row][d] tile: 128 bf16 + 8 padding (272 bytes)
constexpr int kRowT = 64 + 8;  // LDS row of a [d][row] tile of 64 rows: 64 bf16 + 8 padding
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

struct AttnArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  float* lse;            // natural-log log-sum-exp, [b][s][h]
  const uint16_t* dout;  // backward
  float* delta;          // backward: rowsum(dO .* O), [b][s][h]
  uint16_t* dq;
  uint16_t* dk;
  uint16_t* dv;
  int64_t q_sh, q_ss, q_sb;  // strides (elements) of q, o, dout, dq along head, position, batch
  int64_t k_sh, k_ss, k_sb;  // strides of k, v, dk, dv
  int32_t seq, heads, kv_heads, batch;
  int32_t causal;
  float scale;  // 1 / sqrt(d) unless given
};

// Round to bf16, nearest even (one v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint16_t bf16_bits(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
__device__ __forceinline__ float bf16_float(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  return (uint32_t)bf16_bits(a) | ((uint32_t)bf16_bits(b) << 16);
}

__device__ __forceinline__ f32x16 mfma(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// The eight bf16 of registers [8 part, 8 part + 8) of a 32 x 32 accumulator,
// as the B (or A) operand of a 16-deep product over the accumulator's rows
// 16 part .. 16 part + 15 (in the row order the permuted tiles use).
__device__ __forceinline__ bf16x8 rows_operand(const f32x16& acc, int part) {
  u32x4 w;
#pragma unroll
  for (int e = 0; e < 4; ++e) w[e] = pack2(acc[8 * part + 2 * e], acc[8 * part + 2 * e + 1]);
  return (bf16x8)w;
}

// ---- 64-row tiles: global -> registers -> LDS ------------------------------
// Thread t holds rows 4 (t / 16) + (0..3), columns 8 (t % 16) + (0..7).

__device__ __forceinline__ void load_tile(const uint16_t* base, int64_t rs, u32x4 (&r)[4]) {
  const int c = threadIdx.x % 16, g = threadIdx.x / 16;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = *reinterpret_cast<const u32x4*>(base + (int64_t)(4 * g + i) * rs + 8 * c);
}

// [row][d], rows of kRowN.
__device__ __forceinline__ void store_rows(uint16_t* lds, const u32x4 (&r)[4]) {
  const int c = threadIdx.x % 16, g = threadIdx.x / 16;
#pragma unroll
  for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4*>(lds + (4 * g + i) * kRowN + 8 * c) = r[i];
}

// The slot of row `row` (0..63) in a transposed tile's row: within each 16,
// rows 4h..4h+3 and 8+4h..8+4h+3 take slots 8h..8h+7.
__device__ __forceinline__ int slot_of(int row) {
  const int k16 = row % 16;
  return (row / 16) * 16 + 8 * ((k16 % 8) / 4) + (k16 < 8 ? 0 : 4) + row % 4;
}

// [d][slot(row)], rows of kRowT: each thread writes, for each of its 8
// columns, its 4 rows as 4 consecutive slots.
__device__ __forceinline__ void store_transposed(uint16_t* lds, const u32x4 (&r)[4]) {
  const int c = threadIdx.x % 16, g = threadIdx.x / 16;
  const int slot = slot_of(4 * g);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int sh = 16 * (j % 2);
    const uint32_t a0 = (r[0][j / 2] >> sh) & 0xffffu, a1 = (r[1][j / 2] >> sh) & 0xffffu;
    const uint32_t a2 = (r[2][j / 2] >> sh) & 0xffffu, a3 = (r[3][j / 2] >> sh) & 0xffffu;
    *reinterpret_cast<u32x2*>(lds + (8 * c + j) * kRowT + slot) = u32x2{a0 | (a1 << 16), a2 | (a3 << 16)};
  }
}

// A operand from a [row][d] tile: rows r0 + lane % 32, d 16 ks + 8 (lane / 32).
__device__ __forceinline__ bf16x8 frag_rows(const uint16_t* lds, int r0, int ks) {
  const int lane = threadIdx.x % 64;
  return *reinterpret_cast<const bf16x8*>(lds + (r0 + lane % 32) * kRowN + 16 * ks + 8 * (lane / 32));
}

// A operand from a [d][slot] tile: d d0 + lane % 32, the 16 rows of step ks.
__device__ __forceinline__ bf16x8 frag_cols(const uint16_t* lds, int d0, int ks) {
  const int lane = threadIdx.x % 64;
  return *reinterpret_cast<const bf16x8*>(lds + (d0 + lane % 32) * kRowT + 16 * ks + 8 * (lane / 32));
}

// B operand straight from global: row `row`, d 16 ks + 8 (lane / 32), for ks = 0..7.
__device__ __forceinline__ void row_operand(const uint16_t* base, bf16x8 (&f)[8]) {
  const int lane = threadIdx.x % 64;
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) f[ks] = *reinterpret_cast<const bf16x8*>(base + 16 * ks + 8 * (lane / 32));
}

// ---- forward -------------------------------------------------------------------

constexpr int kFwdQ = 128;  // queries per workgroup (32 per wave)
constexpr int kFwdK = 64;   // keys per step
constexpr size_t kFwdLds = 2 * (64 * kRowN + kD * kRowT) * sizeof(uint16_t);  // K and V', two stages

__global__ __launch_bounds__(256, 2) void attn_fwd(AttnArgs p) {
  extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
  const int fwd_stage = 64 * kRowN + kD * kRowT;  // bf16 per stage: K, then V'
  auto Ks = [&](int s) { return lds + s * fwd_stage; };
  auto Vt = [&](int s) { return lds + s * fwd_stage + 64 * kRowN; };
  const int nqb = p.seq / kFwdQ;
  const int qb = nqb - 1 - (int)blockIdx.x;  // heaviest first
  const int h = blockIdx.y, b = blockIdx.z;
  const int hk = h / (p.heads / p.kv_heads);
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int lr = lane % 32, lh = lane / 32;
  const int q0 = qb * kFwdQ + wave * 32;
  const int query = q0 + lr;

  const uint16_t* qbase = p.q + (int64_t)b * p.q_sb + (int64_t)h * p.q_sh;
  const uint16_t* kbase = p.k + (int64_t)b * p.k_sb + (int64_t)hk * p.k_sh;
  const uint16_t* vbase = p.v + (int64_t)b * p.k_sb + (int64_t)hk * p.k_sh;

  bf16x8 qf[8];
  row_operand(qbase + (int64_t)query * p.q_ss, qf);

  f32x16 o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = f32x16{};
  float m = -INFINITY, l = 0.0f;
  const float c = p.scale * kLog2e;

  const int nkb = p.causal ? ((qb + 1) * kFwdQ) / kFwdK : p.seq / kFwdK;
  u32x4 rk[4], rv[4];
  load_tile(kbase, p.k_ss, rk);
  load_tile(vbase, p.k_ss, rv);
  store_rows(Ks(0), rk);
  store_transposed(Vt(0), rv);
  __syncthreads();

  for (int kb = 0; kb < nkb; ++kb) {
    const int st = kb & 1;
    const bool more = kb + 1 < nkb;
    if (more) {
      load_tile(kbase + (int64_t)(kb + 1) * kFwdK * p.k_ss, p.k_ss, rk);
      load_tile(vbase + (int64_t)(kb + 1) * kFwdK * p.k_ss, p.k_ss, rv);
    }
    // S' (64 keys x 32 queries) = K Q'.
    f32x16 s[2] = {f32x16{}, f32x16{}};
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
#pragma unroll
      for (int j = 0; j < 2; ++j) s[j] = mfma(frag_rows(Ks(st), 32 * j, ks), qf[ks], s[j]);
    // Mask (diagonal blocks only), and the running maximum of this lane's
    // query in scaled units (the scale is positive, so max commutes with it).
    const int key0 = kb * kFwdK;
    if (p.causal && key0 + kFwdK > q0) {
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int key = key0 + 32 * j + 8 * (i / 4) + 4 * lh + i % 4;
          if (key > query) s[j][i] = -INFINITY;
        }
    }
    float mb = -INFINITY;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int i = 0; i < 16; ++i) mb = fmaxf(mb, s[j][i]);
    mb = fmaxf(mb, __shfl_xor(mb, 32, 64)) * c;
    const float mn = fmaxf(m, mb);
    const float shift = isfinite(mn) ? mn : 0.0f;
    float ls = 0.0f;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float w = __builtin_amdgcn_exp2f(fmaf(s[j][i], c, -shift));
        s[j][i] = w;
        ls += w;
      }
    // Rescale only when some query's maximum grew.
    if (__ballot(mn > m)) {
      const float alpha = __builtin_amdgcn_exp2f(m - shift);
      l *= alpha;
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] *= alpha;
    }
    l += ls;
    m = mn;
    // O' (128 d x 32 queries) += V' P', the weights rounded to bf16.
    bf16x8 pf[4] = {rows_operand(s[0], 0), rows_operand(s[0], 1), rows_operand(s[1], 0), rows_operand(s[1], 1)};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int db = 0; db < 4; ++db) o[db] = mfma(frag_cols(Vt(st), 32 * db, ks), pf[ks], o[db]);
    if (more) {
      store_rows(Ks(st ^ 1), rk);
      store_transposed(Vt(st ^ 1), rv);
    }
    __syncthreads();
  }

  // Both halves of the wave summed their keys' weights against the same maximum.
  l += __shfl_xor(l, 32, 64);
  const float inv = 1.0f / l;
  uint16_t* obase = p.o + (int64_t)b * p.q_sb + (int64_t)h * p.q_sh + (int64_t)query * p.q_ss;
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d = 32 * db + 8 * g + 4 * lh;
      *reinterpret_cast<u32x2*>(obase + d) =
          u32x2{pack2(o[db][4 * g] * inv, o[db][4 * g + 1] * inv), pack2(o[db][4 * g + 2] * inv, o[db][4 * g + 3] * inv)};
    }
  if (lh == 0 && p.lse) p.lse[((int64_t)b * p.seq + query) * p.heads + h] = (m + log2f(l)) * kLn2;
}

// ---- backward: delta = rowsum(dO .* O) -------------------------------------------

__global__ __launch_bounds__(256) void attn_bwd_delta(AttnArgs p) {
  // One wave per (query, head, batch) row of 128: 64 lanes x 2 elements.
  const int64_t row = (int64_t)blockIdx.x * 4 + threadIdx.x / 64;
  const int64_t total = (int64_t)p.batch * p.seq * p.heads;
  if (row >= total) return;
  const int lane = threadIdx.x % 64;
  const int h = (int)(row % p.heads);
  const int64_t s = (row / p.heads) % p.seq, b = row / ((int64_t)p.heads * p.seq);
  const int64_t at = b * p.q_sb + h * p.q_sh + s * p.q_ss + 2 * lane;
  const uint32_t ow = *reinterpret_cast<const uint32_t*>(p.o + at);
  const uint32_t gw = *reinterpret_cast<const uint32_t*>(p.dout + at);
  float v = bf16_float((uint16_t)ow) * bf16_float((uint16_t)gw) +
            bf16_float((uint16_t)(ow >> 16)) * bf16_float((uint16_t)(gw >> 16));
  v = thd::wave_sum(v);
  if (lane == 0) p.delta[(b * p.seq + s) * p.heads + h] = v;
}

// ---- backward: dK, dV for a block of 128 keys -------------------------------------
// Each wave owns 32 keys.  Per query block of 64: S (64 queries x 32 keys)
// = Q K' with queries along the registers and keys along the lanes, so the
// products over queries (dV = P' dO, dK = dS' Q) take P and dS straight from
// the accumulators as their B operands, against dO' and Q' tiles transposed
// into [d][slot(query)].

constexpr int kBwdK = 128;  // keys per workgroup
constexpr int kBwdQ = 64;   // queries per step
constexpr size_t kStageBwd = (size_t)(2 * 64 * kRowN + 2 * kD * kRowT) * sizeof(uint16_t) + 2 * 64 * sizeof(float);
constexpr size_t kDkdvLds = 2 * kStageBwd;

__global__ __launch_bounds__(256, 1) void attn_bwd_dkdv(AttnArgs p) {
  extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
  const size_t stage_elems = kStageBwd / sizeof(uint16_t);
  const int nkb = p.seq / kBwdK;
  const int kbk = (int)blockIdx.x;  // the first key blocks see the most queries: heaviest first
  (void)nkb;
  const int h = blockIdx.y, b = blockIdx.z;
  const int hk = h / (p.heads / p.kv_heads);
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int lr = lane % 32, lh = lane / 32;
  const int k0 = kbk * kBwdK + wave * 32;
  const int key = k0 + lr;

  const uint16_t* qbase = p.q + (int64_t)b * p.q_sb + (int64_t)h * p.q_sh;
  const uint16_t* gbase = p.dout + (int64_t)b * p.q_sb + (int64_t)h * p.q_sh;
  const float* lbase = p.lse + (int64_t)b * p.seq * p.heads + h;
  const float* dbase = p.delta + (int64_t)b * p.seq * p.heads + h;
  const int64_t koff = (int64_t)b * p.k_sb + (int64_t)hk * p.k_sh + (int64_t)key * p.k_ss;

  bf16x8 kf[8], vf[8];
  row_operand(p.k + koff, kf);
  row_operand(p.v + koff, vf);

  f32x16 dk[4], dv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) dk[i] = f32x16{}, dv[i] = f32x16{};
  const float c = p.scale * kLog2e;

  auto stage = [&](int s, uint16_t** Qs, uint16_t** Qt, uint16_t** Gs, uint16_t** Gt, float** L, float** Dl) {
    uint16_t* base = lds + s * stage_elems;
    *Qs = base;
    *Gs = base + 64 * kRowN;
    *Qt = base + 2 * 64 * kRowN;
    *Gt = base + 2 * 64 * kRowN + kD * kRowT;
    *L = reinterpret_cast<float*>(base + 2 * 64 * kRowN + 2 * kD * kRowT);
    *Dl = *L + 64;
  };
  const int qstart = p.causal ? (kbk * kBwdK) / kBwdQ : 0;
  const int nq = p.seq / kBwdQ;
  u32x4 rq[4], rg[4];
  float rl = 0.0f, rd = 0.0f;
  auto fetch = [&](int qb) {
    load_tile(qbase + (int64_t)qb * kBwdQ * p.q_ss, p.q_ss, rq);
    load_tile(gbase + (int64_t)qb * kBwdQ * p.q_ss, p.q_ss, rg);
    if (threadIdx.x < 64) {
      rl = lbase[(int64_t)(qb * kBwdQ + threadIdx.x) * p.heads];
      rd = dbase[(int64_t)(qb * kBwdQ + threadIdx.x) * p.heads];
    }
  };
  auto land = [&](int s) {
    uint16_t *Qs, *Qt, *Gs, *Gt;
    float *L, *Dl;
    stage(s, &Qs, &Qt, &Gs, &Gt, &L, &Dl);
    store_rows(Qs, rq);
    store_transposed(Qt, rq);
    store_rows(Gs, rg);
    store_transposed(Gt, rg);
    if (threadIdx.x < 64) L[threadIdx.x] = rl * kLog2e, Dl[threadIdx.x] = rd;
  };
  fetch(qstart);
  land(0);
  __syncthreads();
  for (int qb = qstart; qb < nq; ++qb) {
    const int st = (qb - qstart) & 1;
    const bool more = qb + 1 < nq;
    if (more) fetch(qb + 1);
    uint16_t *Qs, *Qt, *Gs, *Gt;
    float *L, *Dl;
    stage(st, &Qs, &Qt, &Gs, &Gt, &L, &Dl);
    // S = Q K', dP = dO V' (64 queries x 32 keys; queries on registers).
    f32x16 s[2] = {f32x16{}, f32x16{}}, dp[2] = {f32x16{}, f32x16{}};
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        s[j] = mfma(frag_rows(Qs, 32 * j, ks), kf[ks], s[j]);
        dp[j] = mfma(frag_rows(Gs, 32 * j, ks), vf[ks], dp[j]);
      }
    const int qq0 = qb * kBwdQ;
    const bool diagonal = p.causal && qq0 < k0 + 32;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int qi = 32 * j + 8 * (i / 4) + 4 * lh + i % 4;
        float pv = __builtin_amdgcn_exp2f(fmaf(s[j][i], c, -L[qi]));
        if (diagonal && key > qq0 + qi) pv = 0.0f;
        s[j][i] = pv;                          // P
        dp[j][i] = pv * (dp[j][i] - Dl[qi]);   // dS
      }
    // dV' (128 d x 32 keys) += dO' P;  dK' += Q' dS.
    bf16x8 pf[4] = {rows_operand(s[0], 0), rows_operand(s[0], 1), rows_operand(s[1], 0), rows_operand(s[1], 1)};
    bf16x8 sf[4] = {rows_operand(dp[0], 0), rows_operand(dp[0], 1), rows_operand(dp[1], 0), rows_operand(dp[1], 1)};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        dv[db] = mfma(frag_cols(Gt, 32 * db, ks), pf[ks], dv[db]);
        dk[db] = mfma(frag_cols(Qt, 32 * db, ks), sf[ks], dk[db]);
      }
    if (more) land(st ^ 1);
    __syncthreads();
  }
  // Lane holds dK'(d, key), dV'(d, key) for d = 32 db + 8 g + 4 lh + (0..3).
  const int64_t out = (int64_t)b * p.k_sb + (int64_t)hk * p.k_sh + (int64_t)key * p.k_ss;
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d = 32 * db + 8 * g + 4 * lh;
      const float sc = p.scale;
      *reinterpret_cast<u32x2*>(p.dk + out + d) =
          u32x2{pack2(dk[db][4 * g] * sc, dk[db][4 * g + 1] * sc), pack2(dk[db][4 * g + 2] * sc, dk[db][4 * g + 3] * sc)};
      *reinterpret_cast<u32x2*>(p.dv + out + d) =
          u32x2{pack2(dv[db][4 * g], dv[db][4 * g + 1]), pack2(dv[db][4 * g + 2], dv[db][4 * g + 3])};
    }
}

// ---- backward: dQ for a block of 128 queries -----------------------------------------
// Each wave owns 32 queries.  Per key block of 64: S' = K Q', dP' = V dO'
// (keys on registers, queries on lanes), dS' = P' .* (dP' - delta), and
// dQ' (128 d x 32 queries) += K' dS' with K' transposed into [d][slot(key)].

constexpr size_t kStageDq = (size_t)(2 * 64 * kRowN + kD * kRowT) * sizeof(uint16_t);
constexpr size_t kDqLds = 2 * kStageDq;

__global__ __launch_bounds__(256, 1) void attn_bwd_dq(AttnArgs p) {
  extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
  const size_t stage_elems = kStageDq / sizeof(uint16_t);
  const int nqb = p.seq / kFwdQ;
  const int qb = nqb - 1 - (int)blockIdx.x;  // heaviest first
  const int h = blockIdx.y, b = blockIdx.z;
  const int hk = h / (p.heads / p.kv_heads);
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int lr = lane % 32, lh = lane / 32;
  const int q0 = qb * kFwdQ + wave * 32;
  const int query = q0 + lr;

  const int64_t qoff = (int64_t)b * p.q_sb + (int64_t)h * p.q_sh + (int64_t)query * p.q_ss;
  bf16x8 qf[8], gf[8];
  row_operand(p.q + qoff, qf);
  row_operand(p.dout + qoff, gf);
  const int64_t srow = ((int64_t)b * p.seq + query) * p.heads + h;
  const float lq = p.lse[srow] * kLog2e;
  const float dq_delta = p.delta[srow];
  const float c = p.scale * kLog2e;

  const uint16_t* kbase = p.k + (int64_t)b * p.k_sb + (int64_t)hk * p.k_sh;
  const uint16_t* vbase = p.v + (int64_t)b * p.k_sb + (int64_t)hk * p.k_sh;
  f32x16 dq[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) dq[i] = f32x16{};

  const int nkb = p.causal ? ((qb + 1) * kFwdQ) / kFwdK : p.seq / kFwdK;
  u32x4 rk[4], rv[4];
  auto Ks = [&](int s) { return lds + s * stage_elems; };
  auto Vs = [&](int s) { return lds + s * stage_elems + 64 * kRowN; };
  auto Kt = [&](int s) { return lds + s * stage_elems + 2 * 64 * kRowN; };
  load_tile(kbase, p.k_ss, rk);
  load_tile(vbase, p.k_ss, rv);
  store_rows(Ks(0), rk);
  store_transposed(Kt(0), rk);
  store_rows(Vs(0), rv);
  __syncthreads();
  for (int kb = 0; kb < nkb; ++kb) {
    const int st = kb & 1;
    const bool more = kb + 1 < nkb;
    if (more) {
      load_tile(kbase + (int64_t)(kb + 1) * kFwdK * p.k_ss, p.k_ss, rk);
      load_tile(vbase + (int64_t)(kb + 1) * kFwdK * p.k_ss, p.k_ss, rv);
    }
    f32x16 s[2] = {f32x16{}, f32x16{}}, dp[2] = {f32x16{}, f32x16{}};
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        s[j] = mfma(frag_rows(Ks(st), 32 * j, ks), qf[ks], s[j]);
        dp[j] = mfma(frag_rows(Vs(st), 32 * j, ks), gf[ks], dp[j]);
      }
    const int key0 = kb * kFwdK;
    const bool diagonal = p.causal && key0 + kFwdK > q0;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key = key0 + 32 * j + 8 * (i / 4) + 4 * lh + i % 4;
        float pv = __builtin_amdgcn_exp2f(fmaf(s[j][i], c, -lq));
        if (diagonal && key > query) pv = 0.0f;
        dp[j][i] = pv * (dp[j][i] - dq_delta);  // dS'
      }
    bf16x8 sf[4] = {rows_operand(dp[0], 0), rows_operand(dp[0], 1), rows_operand(dp[1], 0), rows_operand(dp[1], 1)};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int db = 0; db < 4; ++db) dq[db] = mfma(frag_cols(Kt(st), 32 * db, ks), sf[ks], dq[db]);
    if (more) {
      store_rows(Ks(st ^ 1), rk);
      store_transposed(Kt(st ^ 1), rk);
      store_rows(Vs(st ^ 1), rv);
    }
    __syncthreads();
  }
  uint16_t* out = p.dq + qoff;
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d = 32 * db + 8 * g + 4 * lh;
      const float sc = p.scale;
      *reinterpret_cast<u32x2*>(out + d) =
          u32x2{pack2(dq[db][4 * g] * sc, dq[db][4 * g + 1] * sc), pack2(dq[db][4 * g + 2] * sc, dq[db][4 * g + 3] * sc)};
    }
}

bool aligned(const void* p, int bytes) { return (reinterpret_cast<uintptr_t>(p) % bytes) == 0; }

int check_desc(const th_attention_desc* d, bool backward) {
  TH_REQUIRE(d != nullptr, "attention: null descriptor");
  TH_REQUIRE(d->head_dim == kD, "attention: head_dim must be 128");
  TH_REQUIRE(d->seq > 0 && d->seq % 128 == 0, "attention: the sequence length must be a positive multiple of 128");
  TH_REQUIRE(d->heads > 0 && d->kv_heads > 0 && d->heads % d->kv_heads == 0,
             "attention: heads must be a positive multiple of kv_heads");
  TH_REQUIRE(d->batch > 0, "attention: batch must be positive");
  TH_REQUIRE(d->seq / 128 <= 65535 && d->heads <= 65535 && d->batch <= 65535, "attention: grid too large");
  TH_REQUIRE(d->q && d->k && d->v && d->o, "attention: null q, k, v or o");
  TH_REQUIRE(aligned(d->q, 16) && aligned(d->k, 16) && aligned(d->v, 16) && aligned(d->o, 16),
             "attention: q, k, v, o must be 16-byte aligned");
  for (int64_t s : {d->q_strides[0], d->q_strides[1], d->q_strides[2], d->k_strides[0], d->k_strides[1], d->k_strides[2]})
    TH_REQUIRE(s % 8 == 0 && s > 0, "attention: strides must be positive multiples of 8 (16-byte rows)");
  if (backward) {
    TH_REQUIRE(d->lse && d->dout && d->dq && d->dk && d->dv, "attention backward: null lse, dout, dq, dk or dv");
    TH_REQUIRE(aligned(d->dout, 16) && aligned(d->dq, 16) && aligned(d->dk, 16) && aligned(d->dv, 16),
               "attention backward: dout, dq, dk, dv must be 16-byte aligned");
    TH_REQUIRE(d->kv_heads == d->heads, "attention backward: grouped heads are not built (kv_heads must equal heads)");
  }
  return TH_OK;
}

AttnArgs args_of(const th_attention_desc* d) {
  AttnArgs a{};
  a.q = static_cast<const uint16_t*>(d->q);
  a.k = static_cast<const uint16_t*>(d->k);
  a.v = static_cast<const uint16_t*>(d->v);
  a.o = static_cast<uint16_t*>(d->o);
  a.lse = d->lse;
  a.dout = static_cast<const uint16_t*>(d->dout);
  a.dq = static_cast<uint16_t*>(d->dq);
  a.dk = static_cast<uint16_t*>(d->dk);
  a.dv = static_cast<uint16_t*>(d->dv);
  a.q_sh = d->q_strides[0];
  a.q_ss = d->q_strides[1];
  a.q_sb = d->q_strides[2];
  a.k_sh = d->k_strides[0];
  a.k_ss = d->k_strides[1];
  a.k_sb = d->k_strides[2];
  a.seq = d->seq;
  a.heads = d->heads;
  a.kv_heads = d->kv_heads;
  a.batch = d->batch;
  a.causal = d->causal;
  a.scale = d->scale > 0 ? d->scale : 1.0f / sqrtf((float)kD);
  return a;
}

}  // namespace

extern "C" int th_build_attention_fwd(const th_attention_desc* d, th_launch** out) {
  if (int r = th::require_ready()) return r;
  *out = nullptr;
  if (int r = check_desc(d, false)) return r;
  TH_HIP(hipFuncSetAttribute((const void*)attn_fwd, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kFwdLds));
  AttnArgs a = args_of(d);
  th::Builder b("attention_fwd", 5);
  int k = b.kernel((const void*)attn_fwd, "attn_fwd", dim3(d->seq / kFwdQ, d->heads, d->batch), dim3(256),
                   (uint32_t)kFwdLds, a);
  b.ref(0, k, TH_OFFSET(AttnArgs, q));
  b.ref(1, k, TH_OFFSET(AttnArgs, k));
  b.ref(2, k, TH_OFFSET(AttnArgs, v));
  b.ref(3, k, TH_OFFSET(AttnArgs, o));
  b.ref(4, k, TH_OFFSET(AttnArgs, lse));
  for (int v = 0; v < 4; ++v) b.align(v, 16);
  const double S = d->seq, BH = (double)d->batch * d->heads;
  const double flops = 4.0 * BH * S * S * kD * (d->causal ? 0.5 : 1.0);
  b.work(2.0 * BH * S * kD * 4 + 4.0 * BH * S, flops, (int64_t)(d->seq / kFwdQ) * d->heads * d->batch);
  *out = b.release();
  return TH_OK;
}

extern "C" int th_build_attention_bwd(const th_attention_desc* d, th_launch** out) {
  if (int r = th::require_ready()) return r;
  *out = nullptr;
  if (int r = check_desc(d, true)) return r;
  TH_HIP(hipFuncSetAttribute((const void*)attn_bwd_dkdv, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kDkdvLds));
  TH_HIP(hipFuncSetAttribute((const void*)attn_bwd_dq, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kDqLds));
  AttnArgs a = args_of(d);
  th::Builder b("attention_bwd", 9);
  void* delta = nullptr;
  const int64_t rows = (int64_t)d->batch * d->seq * d->heads;
  if (int r = th::device_alloc((size_t)rows * sizeof(float), &delta)) return r;
  b.own(delta);
  a.delta = static_cast<float*>(delta);
  int k0 = b.kernel((const void*)attn_bwd_delta, "attn_bwd_delta", dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, a);
  int k1 = b.kernel((const void*)attn_bwd_dkdv, "attn_bwd_dkdv", dim3(d->seq / kBwdK, d->heads, d->batch), dim3(256),
                    (uint32_t)kDkdvLds, a);
  int k2 = b.kernel((const void*)attn_bwd_dq, "attn_bwd_dq", dim3(d->seq / kFwdQ, d->heads, d->batch), dim3(256),
                    (uint32_t)kDqLds, a);
  const size_t offs[9] = {TH_OFFSET(AttnArgs, q),   TH_OFFSET(AttnArgs, k),  TH_OFFSET(AttnArgs, v),
                          TH_OFFSET(AttnArgs, o),   TH_OFFSET(AttnArgs, lse), TH_OFFSET(AttnArgs, dout),
                          TH_OFFSET(AttnArgs, dq),  TH_OFFSET(AttnArgs, dk), TH_OFFSET(AttnArgs, dv)};
  for (int v = 0; v < 9; ++v)
    for (int kk : {k0, k1, k2}) b.ref(v, kk, offs[v]);
  for (int v : {0, 1, 2, 3, 5, 6, 7, 8}) b.align(v, 16);
  const double S = d->seq, BH = (double)d->batch * d->heads;
  const double flops = 2.5 * 4.0 * BH * S * S * kD * (d->causal ? 0.5 : 1.0);
  b.work(2.0 * BH * S * kD * 8 + 8.0 * BH * S, flops, (int64_t)(d->seq / kBwdK) * d->heads * d->batch);
  *out = b.release();
  return TH_OK;
}
