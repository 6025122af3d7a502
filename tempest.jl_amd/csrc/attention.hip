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
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

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
// Two floats to a pair of bf16 (one v_cvt_pk_bf16_f32), a in the low half.
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
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
// Every load goes through a buffer resource at a uniform (scalar) base, with
// per-thread 32-bit byte offsets fixed for the whole kernel; a 64-row tile
// spans under 2 GiB (the builder checks the position stride).

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc_of(const uint16_t* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(base), (short)0, 0x7fffffff, 0x00020000);
}

// Row-major staging: thread t holds rows 4 (t / 16) + i (i = 0..3), columns
// 8 (t % 16) + (0..7), and writes them to [row][d] rows of kRowN: sixteen
// lanes fill one row's 256 bytes, so the stores never share a bank.
struct TileRows {
  int32_t off;     // this thread's byte offset of its first row
  int32_t stride;  // bytes between rows (uniform)
  __device__ explicit TileRows(int64_t rs) : stride((int32_t)(rs * 2)) {
    const int c = threadIdx.x % 16, g = threadIdx.x / 16;
    off = (int32_t)((4 * g * rs + 8 * c) * 2);
  }
  __device__ void load(const uint16_t* base, u32x4 (&r)[4]) const {
    const __amdgpu_buffer_rsrc_t rsrc = rsrc_of(base);
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = (u32x4)__builtin_amdgcn_raw_buffer_load_b128(rsrc, off, i * stride, 0);
  }
};

__device__ __forceinline__ void store_rows(uint16_t* lds, const u32x4 (&r)[4]) {
  const int c = threadIdx.x % 16, g = threadIdx.x / 16;
#pragma unroll
  for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4*>(lds + (4 * g + i) * kRowN + 8 * c) = r[i];
}

// Transposed staging into [d][slot] rows of kRowT.  Slots permute the rows
// so that a 32 x 32 accumulator's registers feed the next product directly:
// within each 16 rows, rows 4h..4h+3 and 8+4h..8+4h+3 take slots 8h..8h+7.
// Thread t owns slot chunk kb = t % 8 (slots 8 kb .. 8 kb + 7, i.e. rows
// row_of_slot(8 kb + e)) and the four d columns 4 ob .. 4 ob + 3, loaded as
// eight 8-byte pieces; it transposes them in registers and writes four
// 16-byte pieces, one per d row.  Lanes 0..7 fill one d row's 128 bytes and
// lanes 8..15 the row 8 further on (ob order 0, 2, 1, 3, 4, 6, 5, 7, ...),
// which starts 32 banks away with rows of 36 words, so no two lanes of a
// store share a bank.
__device__ __forceinline__ int row_of_slot(int slot) {
  const int chunk = slot / 8, e = slot % 8;
  return 16 * (chunk / 2) + 4 * (chunk % 2) + 8 * (e / 4) + e % 4;
}

__device__ __forceinline__ int cols_ob() {
  const int j = threadIdx.x / 8;
  return 2 * (j & 1) + ((j >> 1) & 1) + 4 * (j >> 2);
}

struct TileCols {
  int32_t off;     // byte offset of row_of_slot(8 kb), column 4 ob
  int32_t stride;  // bytes between rows (uniform)
  __device__ explicit TileCols(int64_t rs) : stride((int32_t)(rs * 2)) {
    const int kb = threadIdx.x % 8, ob = cols_ob();
    off = (int32_t)(((int64_t)row_of_slot(8 * kb) * rs + 4 * ob) * 2);
  }
  // Slot 8 kb + e is row row_of_slot(8 kb) + 8 (e / 4) + e % 4.
  __device__ void load(const uint16_t* base, u32x2 (&r)[8]) const {
    const __amdgpu_buffer_rsrc_t rsrc = rsrc_of(base);
#pragma unroll
    for (int e = 0; e < 8; ++e)
      r[e] = (u32x2)__builtin_amdgcn_raw_buffer_load_b64(rsrc, off, (8 * (e / 4) + e % 4) * stride, 0);
  }
};

__device__ __forceinline__ void store_cols(uint16_t* lds, const u32x2 (&r)[8]) {
  const int kb = threadIdx.x % 8, ob = cols_ob();
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    u32x4 w;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t lo = r[2 * e][c / 2], hi = r[2 * e + 1][c / 2];
      w[e] = (c % 2 == 0) ? ((lo & 0xffffu) | (hi << 16)) : ((lo >> 16) | (hi & 0xffff0000u));
    }
    *reinterpret_cast<u32x4*>(lds + (4 * ob + c) * kRowT + 8 * kb) = w;
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
// Per workgroup 128 queries (32 per wave), keys in steps of 64.  The loop is
// pipelined by one step: while the vector ALUs turn the scores of step j into
// weights, the matrix cores already compute the scores of step j + 1, so K
// runs one step ahead of V through LDS.  Iteration j reads K[(j + 1) & 1] and
// V'[j & 1], and refills K[j & 1] with step j + 2 and V'[(j + 1) & 1] with
// step j + 1 (indices past the last step are clamped; their scores are never
// used).  The running maximum is rebased lazily: the accumulators keep their
// shift until a query's maximum exceeds it by more than kLazy (log2 units),
// so no weight exceeds 2^kLazy and most steps skip the rescale.

constexpr int kFwdQ = 128;  // queries per workgroup (32 per wave)
constexpr int kFwdK = 64;   // keys per step
constexpr int kKTile = 64 * kRowN;  // bf16 of a K tile in LDS
constexpr int kVTile = kD * kRowT;  // bf16 of a V' tile in LDS
constexpr size_t kFwdLds = 2 * (kKTile + kVTile) * sizeof(uint16_t);
constexpr float kLazy = 8.0f;

__global__ __launch_bounds__(256, 2) void attn_fwd(AttnArgs p) {
  extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
  uint16_t* const Kl[2] = {lds, lds + kKTile};
  uint16_t* const Vl[2] = {lds + 2 * kKTile, lds + 2 * kKTile + kVTile};
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
  const int64_t step_elems = (int64_t)kFwdK * p.k_ss;
  const TileRows rows(p.k_ss);
  const TileCols cols(p.k_ss);

  bf16x8 qf[8];
  row_operand(qbase + (int64_t)query * p.q_ss, qf);

  f32x16 o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = f32x16{};
  float m = -INFINITY, l = 0.0f;
  const float c = p.scale * kLog2e;
  // An even number of steps (the sequence is a multiple of 128), at least 2.
  const int nkb = p.causal ? ((qb + 1) * kFwdQ) / kFwdK : p.seq / kFwdK;

  u32x4 rk[4];
  u32x2 rv[8];
  rows.load(kbase, rk);
  cols.load(vbase, rv);
  store_rows(Kl[0], rk);
  store_cols(Vl[0], rv);
  rows.load(kbase + step_elems, rk);
  store_rows(Kl[1], rk);
  __syncthreads();
  f32x16 sa[2] = {f32x16{}, f32x16{}}, sb[2];
#pragma unroll
  for (int ks = 0; ks < 8; ++ks)
#pragma unroll
    for (int j = 0; j < 2; ++j) sa[j] = mfma(frag_rows(Kl[0], 32 * j, ks), qf[ks], sa[j]);
  __syncthreads();

  // Step j: weights from s (its scores), scores of step j + 1 into sn.
  auto step = [&](const int j, f32x16 (&s)[2], f32x16 (&sn)[2]) {
    const int st = j & 1;
    rows.load(kbase + (int64_t)min(j + 2, nkb - 1) * step_elems, rk);
    cols.load(vbase + (int64_t)min(j + 1, nkb - 1) * step_elems, rv);
    const int key0 = j * kFwdK;
    if (p.causal && key0 + kFwdK > q0) {
#pragma unroll
      for (int jj = 0; jj < 2; ++jj)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int key = key0 + 32 * jj + 8 * (i / 4) + 4 * lh + i % 4;
          if (key > query) s[jj][i] = -INFINITY;
        }
    }
    sn[0] = f32x16{};
    sn[1] = f32x16{};
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) sn[jj] = mfma(frag_rows(Kl[st ^ 1], 32 * jj, ks), qf[ks], sn[jj]);
    // This lane's query maximum in scaled units (the scale is positive).
    float mb = -INFINITY;
#pragma unroll
    for (int jj = 0; jj < 2; ++jj)
#pragma unroll
      for (int i = 0; i < 16; ++i) mb = fmaxf(mb, s[jj][i]);
    mb = fmaxf(mb, __shfl_xor(mb, 32, 64)) * c;
    const bool grow = mb > m + kLazy;
    const float mn = grow ? mb : m;
    const float shift = isfinite(mn) ? mn : 0.0f;
    float ls = 0.0f;
    bf16x8 pf[4];
#pragma unroll
    for (int jj = 0; jj < 2; ++jj)
#pragma unroll
      for (int part = 0; part < 2; ++part) {
        u32x4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float w0 = __builtin_amdgcn_exp2f(fmaf(s[jj][8 * part + 2 * e], c, -shift));
          const float w1 = __builtin_amdgcn_exp2f(fmaf(s[jj][8 * part + 2 * e + 1], c, -shift));
          ls += w0 + w1;
          w[e] = pack2(w0, w1);
        }
        pf[2 * jj + part] = (bf16x8)w;
      }
    if (__ballot(grow)) {
      const float alpha = __builtin_amdgcn_exp2f(m - shift);
      l *= alpha;
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] *= alpha;
    }
    l += ls;
    m = mn;
    // O' (128 d x 32 queries) += V' P', the weights rounded to bf16.
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int db = 0; db < 4; ++db) o[db] = mfma(frag_cols(Vl[st], 32 * db, ks), pf[ks], o[db]);
    store_rows(Kl[st], rk);
    store_cols(Vl[st ^ 1], rv);
    __syncthreads();
  };
  for (int j = 0; j < nkb; j += 2) {
    step(j, sa, sb);
    step(j + 1, sb, sa);
  }

  // Both halves of the wave summed their keys' weights against the same shift.
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
  const TileRows rows(p.q_ss);
  const TileCols cols(p.q_ss);
  u32x4 rq[4], rg[4];
  u32x2 cq[8], cg[8];
  float rl = 0.0f, rd = 0.0f;
  auto fetch = [&](int qb) {
    const int64_t at = (int64_t)qb * kBwdQ * p.q_ss;
    rows.load(qbase + at, rq);
    rows.load(gbase + at, rg);
    cols.load(qbase + at, cq);
    cols.load(gbase + at, cg);
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
    store_cols(Qt, cq);
    store_rows(Gs, rg);
    store_cols(Gt, cg);
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
  const TileRows rows(p.k_ss);
  const TileCols cols(p.k_ss);
  u32x4 rk[4], rv[4];
  u32x2 ck[8];
  auto Ks = [&](int s) { return lds + s * stage_elems; };
  auto Vs = [&](int s) { return lds + s * stage_elems + 64 * kRowN; };
  auto Kt = [&](int s) { return lds + s * stage_elems + 2 * 64 * kRowN; };
  rows.load(kbase, rk);
  rows.load(vbase, rv);
  cols.load(kbase, ck);
  store_rows(Ks(0), rk);
  store_cols(Kt(0), ck);
  store_rows(Vs(0), rv);
  __syncthreads();
  for (int kb = 0; kb < nkb; ++kb) {
    const int st = kb & 1;
    const bool more = kb + 1 < nkb;
    if (more) {
      const int64_t at = (int64_t)(kb + 1) * kFwdK * p.k_ss;
      rows.load(kbase + at, rk);
      rows.load(vbase + at, rv);
      cols.load(kbase + at, ck);
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
      store_cols(Kt(st ^ 1), ck);
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
  TH_REQUIRE(d->k_strides[1] < (int64_t(1) << 24) && d->q_strides[1] < (int64_t(1) << 24),
             "attention: position strides must be below 2^24 elements (a 64-position tile spans under 2 GiB)");
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
