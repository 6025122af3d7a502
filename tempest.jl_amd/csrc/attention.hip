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

#include "lds_dma.h"
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
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

constexpr int kD = 128;                // head dimension
constexpr int kTileElems = 64 * kD;    // one 64-row tile in LDS (256-byte rows, no padding)
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
  // backward workspace: dS' as bf16 in the dQ product's operand order,
  // [b][h][query block of 64][key slice of 16][query half][lane][8] (two 1 KB
  // fragments per block and slice; lane l holds query 32 half + l % 32 and keys
  // 8 (e / 4) + 4 (l / 32) + e % 4 of the slice in element e), or null.
  uint16_t* ds;
  // backward workspace: per (b, h) and 64-query block qb, 128 floats: the 64
  // queries' -lse / scale, then their -delta ([b][h][qb][2][64]).
  float* stat;
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

// The value lane l ^ 32 holds (v_permlane32_swap: no LDS round trip).
__device__ __forceinline__ float other_half(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(threadIdx.x % 64 < 32 ? r[1] : r[0]);
}

__device__ __forceinline__ f32x16 mfma(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// c += a b with c held in AGPRs.  This file's products keep their
// accumulators in VGPRs (the vector ALUs read scores straight from them); an
// accumulator that only products touch until the end is better off in the
// AGPRs, leaving the VGPRs to operands and addresses.  Two wait states first,
// for a vector instruction that has just written a or b; the caller waits
// before vector instructions read c (agpr_settle).
__device__ __forceinline__ void mfma_agpr(bf16x8 a, bf16x8 b, f32x16& c) {
  asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
}

// 24 wait states before vector instructions read the accumulators: more than
// the ISA asks for after a 16-pass product writes its result.
__device__ __forceinline__ void agpr_settle(f32x16 (&x)[4], f32x16 (&y)[4]) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7"
               : "+a"(x[0]), "+a"(x[1]), "+a"(x[2]), "+a"(x[3]), "+a"(y[0]), "+a"(y[1]), "+a"(y[2]), "+a"(y[3]));
}

// The eight bf16 of registers [8 part, 8 part + 8) of a 32 x 32 accumulator
// as the B operand of a 16-deep product over the accumulator's rows
// 16 part .. 16 part + 15.  Lane l holds rows 8 (i / 4) + 4 (l / 32) + i % 4
// in register i, so its k-slot 8 (l / 32) + e is row 8 (e / 4) + 4 (l / 32)
// + e % 4 of the sixteen: the A operand must use the same row order.
__device__ __forceinline__ bf16x8 rows_operand(const f32x16& acc, int part) {
  u32x4 w;
#pragma unroll
  for (int e = 0; e < 4; ++e) w[e] = pack2(acc[8 * part + 2 * e], acc[8 * part + 2 * e + 1]);
  return (bf16x8)w;
}

// sched_barrier mask: vector, scalar and transcendental instructions may
// cross the fence; LDS accesses, global loads and products may not.
constexpr int kFence = 0x0406;
constexpr int kFenceFwd = kFence;

// ---- 64-row tiles in LDS ---------------------------------------------------------
// A tile holds 64 rows of 128 bf16 (256 bytes, one pass over the 64 banks).
// The sixteen 16-byte chunks of row r are stored XOR-permuted, chunk c at
// position c ^ swz(r) with swz(r) = 4 (r % 4) + (r / 4) % 4, which keeps the
// three access patterns below free of bank conflicts:
//  - 16 lanes storing one row (the positions are a permutation of 0..15);
//  - 16 lanes reading chunk c of 16 consecutive rows (swz is a bijection on r % 16);
//  - 32 lanes reading 8 bytes each from four consecutive rows (aligned to 4)
//    by four consecutive chunks (aligned to 4): the positions
//    4 ((c / 4) ^ (r % 4)) + ((c % 4) ^ ((r / 4) % 4)) are 16 distinct chunks.
__device__ __forceinline__ int tile_at(int row, int chunk) {
  return row * kD + 8 * (chunk ^ (4 * (row % 4) + (row / 4) % 4));
}

// Every global load goes through a buffer resource at a uniform (scalar)
// base; a 64-row tile spans under 2 GiB (the builder checks the strides).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc_of(const uint16_t* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(base), (short)0, 0x7fffffff, 0x00020000);
}

// Thread t holds rows 4 (t / 16) + i (i = 0..3), chunk t % 16 of a tile.
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
  for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4*>(lds + tile_at(4 * g + i, c)) = r[i];
}

// A operand from a tile, M along its rows: rows r0 + lane % 32, k = columns
// 16 ks + 8 (lane / 32) + (0..7).
__device__ __forceinline__ bf16x8 frag_rows(const uint16_t* lds, int r0, int ks) {
  const int lane = threadIdx.x % 64;
  return *reinterpret_cast<const bf16x8*>(lds + tile_at(r0 + lane % 32, 2 * ks + lane / 32));
}

// A operand from a tile, M along its columns: m = column d0 + lane % 32, k =
// the rows of 16-row step ks in the order rows_operand gives the B operand
// (k-slot 8 h + e <-> row 16 ks + 8 (e / 4) + 4 h + e % 4, h = lane / 32).
// ds_read_b64_tr_b16 hands lane i of each 16 element i % 4 of the 8-byte
// pieces addressed by lanes 4 k + i / 4 (k = 0..3).  Lane j here addresses
// row base + j / 4, columns dgrp + 4 (j % 4) + (0..3), so lane i receives
// rows base + (0..3) of column dgrp + i; two reads cover the eight rows.
__device__ __forceinline__ bf16x8 frag_tr(const uint16_t* lds, int d0, int ks) {
  const int lane = threadIdx.x % 64, j = lane % 16;
  const int col = d0 + 16 * ((lane / 16) % 2) + 4 * (j % 4);
  const int row = 16 * ks + 4 * (lane / 32) + j / 4;
  const int at0 = tile_at(row, col / 8) + col % 8, at1 = tile_at(row + 8, col / 8) + col % 8;
  const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(lds + at0));
  const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(lds + at1));
  typedef short s16x8 __attribute__((ext_vector_type(8)));
  const s16x8 w = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return __builtin_bit_cast(bf16x8, w);
}

// B operand straight from global: row `row`, d 16 ks + 8 (lane / 32), for ks = 0..7.
__device__ __forceinline__ void row_operand(const uint16_t* base, bf16x8 (&f)[8]) {
  const int lane = threadIdx.x % 64;
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) f[ks] = *reinterpret_cast<const bf16x8*>(base + 16 * ks + 8 * (lane / 32));
}

// ---- workgroup order ---------------------------------------------------------------
// Workgroups are dealt to the eight XCDs round-robin by linear index.  The
// logical block is remapped so that each XCD takes a contiguous range of
// (x fastest, then y, then z): the blocks of one (head, batch) run together
// on one XCD and stream the same tiles of the other operands through its L2.
struct Block {
  int x, y, z;
};
__device__ __forceinline__ Block xcd_block() {
  const int gx = gridDim.x, gy = gridDim.y;
  const int total = gx * gy * gridDim.z;
  int t = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
  if (total % 8 == 0) t = (t % 8) * (total / 8) + t / 8;
  return Block{t % gx, (t / gx) % gy, t / (gx * gy)};
}

// ---- forward -------------------------------------------------------------------
// Per workgroup 128 queries (32 per wave), keys in steps of 64.  The loop is
// pipelined by one step: while the vector ALUs turn the scores of step j into
// weights, the matrix cores already compute the scores of step j + 1, so K
// runs one step ahead of V through LDS.  Iteration j reads K[(j + 1) & 1] and
// V[j & 1], and refills K[j & 1] with step j + 2 and V[(j + 1) & 1] with
// step j + 1 (indices past the last step are clamped; their scores are never
// used).  The refills are direct global->LDS loads issued at the top of the
// iteration, into buffers the previous iteration finished with, and waited
// for at its end.  V is read transposed straight from its row-major tile.
// K and V fragments are read a few products ahead of their use (the two
// products of each 16-deep slice take 8 of the 256 registers; four slices
// are in flight).  The running maximum is rebased lazily: the accumulators
// keep their shift until a query's maximum exceeds it by more than kLazy
// (log2 units), so no weight exceeds 2^kLazy and most steps skip the rescale.

constexpr int kFwdQ = 128;  // queries per workgroup (32 per wave)
constexpr int kFwdK = 64;   // keys per step
constexpr size_t kFwdLds = 4 * kTileElems * sizeof(uint16_t);  // K[2], V[2]
constexpr float kLazy = 8.0f;

// The 64-row tile of rows [row0, row0 + 64) of a (position-major) operand,
// loaded straight into LDS in the permuted layout of tile_at: instruction i
// of wave w fills rows 16 w + 4 i .. + 3 (1 KB), lane l the 16 bytes of row
// 16 w + 4 i + l / 16 at position l % 16, i.e. chunk (l % 16) ^ swz(row).
struct TileDma {
  __amdgpu_buffer_rsrc_t rsrc;
  int32_t off[4];  // byte offsets of this lane's rows for row0 = 0
  int32_t row_bytes;
  __device__ TileDma(const uint16_t* base, int64_t rs) {
    rsrc = th_dev::buffer_of(base);
    row_bytes = (int32_t)(rs * 2);
    const int w = threadIdx.x / 64, l = threadIdx.x % 64;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 16 * w + 4 * i + l / 16;
      const int c = (l % 16) ^ (4 * (r % 4) + (r / 4) % 4);
      off[i] = (int32_t)(((int64_t)r * rs + 8 * c) * 2);
    }
  }
  __device__ __forceinline__ void load(int row0, const uint16_t* lds) const {
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const uint32_t dst = (uint32_t)(uintptr_t)lds + 1024 * 4 * w;
#pragma unroll
    for (int i = 0; i < 4; ++i) th_dev::dma16(rsrc, off[i], row0 * row_bytes, dst + 1024 * i);
  }
  // The same for tiles read once (non-temporal).
  __device__ __forceinline__ void load_stream(int row0, const uint16_t* lds) const {
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const uint32_t dst = (uint32_t)(uintptr_t)lds + 1024 * 4 * w;
#pragma unroll
    for (int i = 0; i < 4; ++i) th_dev::dma16_nt(rsrc, off[i], row0 * row_bytes, dst + 1024 * i);
  }
};

__global__ __launch_bounds__(256, 2) void attn_fwd(AttnArgs p) {
  extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
  uint16_t* const Kl[2] = {lds, lds + kTileElems};
  uint16_t* const Vl[2] = {lds + 2 * kTileElems, lds + 3 * kTileElems};
  const int nqb = p.seq / kFwdQ;
  // Causal: workgroup x takes query blocks x and nqb - 1 - x, so every
  // workgroup sweeps the same number of key blocks.
  const Block blk = xcd_block();
  const int npass = (p.causal && 2 * blk.x + 1 != nqb) ? 2 : 1;
  for (int pass = 0; pass < npass; ++pass) {
    const int qb = pass == 0 ? blk.x : nqb - 1 - blk.x;
    const int h = blk.y, b = blk.z;
    const int hk = h / (p.heads / p.kv_heads);
    const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const int lr = lane % 32, lh = lane / 32;
    const int q0 = qb * kFwdQ + wave * 32;
    const int query = q0 + lr;

    const uint16_t* qbase = p.q + (int64_t)b * p.q_sb + (int64_t)h * p.q_sh;
    const TileDma kt(p.k + (int64_t)b * p.k_sb + (int64_t)hk * p.k_sh, p.k_ss);
    const TileDma vt(p.v + (int64_t)b * p.k_sb + (int64_t)hk * p.k_sh, p.k_ss);

    bf16x8 qf[8];
    row_operand(qbase + (int64_t)query * p.q_ss, qf);

    f32x16 o[4];
  #pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = f32x16{};
    float m = -INFINITY, l = 0.0f;
    const float c = p.scale * kLog2e;
    // An even number of steps (the sequence is a multiple of 128), at least 2.
    const int nkb = p.causal ? ((qb + 1) * kFwdQ) / kFwdK : p.seq / kFwdK;

    // S' (64 keys x 32 queries) of the tile in K: two 32-key blocks, the
    // fragments of slice ks + 3 read while slice ks multiplies.
    auto scores = [&](const uint16_t* K, f32x16 (&s)[2]) {
      bf16x8 kf[4][2];
  #pragma unroll
      for (int ks = 0; ks < 3; ++ks) kf[ks][0] = frag_rows(K, 0, ks), kf[ks][1] = frag_rows(K, 32, ks);
      s[0] = f32x16{};
      s[1] = f32x16{};
  #pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
        if (ks + 3 < 8) kf[(ks + 3) % 4][0] = frag_rows(K, 0, ks + 3), kf[(ks + 3) % 4][1] = frag_rows(K, 32, ks + 3);
        s[0] = mfma(kf[ks % 4][0], qf[ks], s[0]);
        s[1] = mfma(kf[ks % 4][1], qf[ks], s[1]);
      }
    };

    kt.load(0, Kl[0]);
    vt.load(0, Vl[0]);
    kt.load(kFwdK, Kl[1]);
    th_dev::wait_and_meet<0>();
    f32x16 sa[2], sb[2];
    scores(Kl[0], sa);
    __syncthreads();

    // Step j: weights from s (its scores), scores of step j + 1 into sn.
    auto step = [&](const int j, f32x16 (&s)[2], f32x16 (&sn)[2]) {
      const int st = j & 1;
      kt.load(min(j + 2, nkb - 1) * kFwdK, Kl[st]);
      vt.load(min(j + 1, nkb - 1) * kFwdK, Vl[st ^ 1]);
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
      // The scores of step j + 1 on the matrix cores while the vector ALUs
      // turn step j's into weights (independent work, interleaved below).
      __builtin_amdgcn_sched_barrier(0);
      scores(Kl[st ^ 1], sn);
      // This lane's query maximum in scaled units (the scale is positive);
      // the other half of the wave holds the same query's other keys.
      float mb = -INFINITY;
  #pragma unroll
      for (int jj = 0; jj < 2; ++jj)
  #pragma unroll
        for (int i = 0; i < 16; ++i) mb = fmaxf(mb, s[jj][i]);
      mb = fmaxf(mb, other_half(mb)) * c;
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
      // The weights are complete here, before the rescale's branch (which
      // the compiler would otherwise hoist above them, splitting them from
      // the products they are interleaved with).
      asm volatile("" ::"v"(pf[0]), "v"(pf[1]), "v"(pf[2]), "v"(pf[3]), "v"(ls));
      // Order: the first three slices' K fragments, then each product
      // followed by its share of the weights' vector work (about six vector
      // and two transcendental instructions per product) and, for the first
      // ten products, the fragment read three slices ahead.
      __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);
  #pragma unroll
      for (int q = 0; q < 16; ++q) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (q < 10) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
        __builtin_amdgcn_sched_group_barrier(0x400, 2, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
      if (__ballot(grow)) {
        const float alpha = __builtin_amdgcn_exp2f(m - shift);
        l *= alpha;
  #pragma unroll
        for (int i = 0; i < 4; ++i) o[i] *= alpha;
      }
      l += ls;
      m = mn;
      // O' (128 d x 32 queries) += V' P', the weights rounded to bf16; the
      // V fragments of slice ks + 1 read while slice ks multiplies.
      const uint16_t* V = Vl[st];
      bf16x8 vf[2][4];
  #pragma unroll
      for (int db = 0; db < 4; ++db) vf[0][db] = frag_tr(V, 32 * db, 0);
  #pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        if (ks + 1 < 4)
  #pragma unroll
          for (int db = 0; db < 4; ++db) vf[(ks + 1) % 2][db] = frag_tr(V, 32 * db, ks + 1);
        __builtin_amdgcn_sched_barrier(kFenceFwd);
  #pragma unroll
        for (int db = 0; db < 4; ++db) o[db] = mfma(vf[ks % 2][db], pf[ks], o[db]);
        __builtin_amdgcn_sched_barrier(kFenceFwd);
      }
      th_dev::wait_and_meet<0>();
    };
    for (int j = 0; j < nkb; j += 2) {
      step(j, sa, sb);
      step(j + 1, sb, sa);
    }

    // Both halves of the wave summed their keys' weights against the same shift.
    l = l + other_half(l);
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
}

// ---- backward: delta = rowsum(dO .* O) -------------------------------------------

constexpr int kDeltaRows = 4;  // rows per sixteen lanes

__global__ __launch_bounds__(256) void attn_bwd_delta(AttnArgs p) {
  // Sixteen lanes per (query, head, batch) row of 128, 16 bytes each; the
  // sixteen lanes of group g take rows g + 16 i (i < kDeltaRows) of the
  // workgroup's 64, every load issued before the first product, so that a
  // wave has 8 KB in flight (with one row each it had 2 KB, and streamed at
  // 5 TB/s).  Rows are (batch, position, head) with the head fastest, so each
  // load instruction covers sixteen consecutive rows.  Row numbers fit 32
  // bits (the builder checks).
  const uint32_t total = (uint32_t)p.batch * p.seq * p.heads;
  const int part = threadIdx.x % 16;
  const uint32_t row0 = blockIdx.x * (16 * kDeltaRows) + threadIdx.x / 16;
  struct Pos {
    int64_t b, s;
    int h;
  };
  auto pos = [&](uint32_t row) {
    const uint32_t bs = row / (uint32_t)p.heads;
    return Pos{bs / (uint32_t)p.seq, bs % (uint32_t)p.seq, (int)(row - bs * (uint32_t)p.heads)};
  };
  u32x4 ow[kDeltaRows], gw[kDeltaRows];
  float lse[kDeltaRows];
#pragma unroll
  for (int i = 0; i < kDeltaRows; ++i) {
    // Rows past the end re-read the last one; nothing is written for them.
    const Pos q = pos(min(row0 + 16 * i, total - 1));
    const int64_t at = q.b * p.q_sb + q.h * p.q_sh + q.s * p.q_ss + 8 * part;
    ow[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p.o + at));
    gw[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p.dout + at));
    lse[i] = p.lse[(q.b * p.seq + q.s) * p.heads + q.h];
  }
  // Every load out before any of their data is used (the scheduler would
  // otherwise start on the first row and wait for it before the next loads).
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < kDeltaRows; ++i) {
    float v = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      v += bf16_float((uint16_t)ow[i][e]) * bf16_float((uint16_t)gw[i][e]) +
           bf16_float((uint16_t)(ow[i][e] >> 16)) * bf16_float((uint16_t)(gw[i][e] >> 16));
#pragma unroll
    for (int m = 8; m >= 1; m /= 2) v += __shfl_xor(v, m, 16);
    const uint32_t row = row0 + 16 * i;
    if (row < total && part == 0) {
      const Pos q = pos(row);
      p.delta[(q.b * p.seq + q.s) * p.heads + q.h] = v;
      const int64_t at = ((q.b * p.heads + q.h) * (p.seq / 64) + q.s / 64) * 128 + q.s % 64;
      p.stat[at] = lse[i] * (-1.0f / p.scale);
      p.stat[at + 64] = -v;
    }
  }
}

// ---- backward: shared pieces -----------------------------------------------------
// Both kernels run one wave per SIMD (each needs most of the register file),
// so each wave keeps its matrix core busy by itself.  A step's 64-row score
// tile is handled in two halves so that the vector work of one half runs
// while the matrix cores do the other half's products:
//   A0: scores of rows 0..31;   A1: scores of rows 32..63 || weights of rows 0..31;
//   C0: gradient products over rows 0..31 || weights of rows 32..63;
//   C1: gradient products over rows 32..63.
// LDS fragments are read a few slices ahead of the products that use them;
// sched_barrier fences that only vector, scalar and transcendental work may
// cross keep the compiler from sinking those reads back next to their
// products while letting the other half's arithmetic slide in between.
// The score accumulators start from the per-row constants they are later
// offset by (-lse / scale for S, -delta for dP), so the weights need no
// separate subtraction: P = exp2(c S~), dS = P dP~.


// 16 products over d = 128: s += x[rows 32 j ..] xf, t += y[rows 32 j ..] yf,
// the A fragments read three slices ahead.
__device__ __forceinline__ void scores_half(const uint16_t* x, const uint16_t* y, int j, const bf16x8 (&xf)[8],
                                            const bf16x8 (&yf)[8], f32x16& s, f32x16& t) {
  bf16x8 fx[4], fy[4];
#pragma unroll
  for (int ks = 0; ks < 3; ++ks) fx[ks] = frag_rows(x, 32 * j, ks), fy[ks] = frag_rows(y, 32 * j, ks);
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) {
    if (ks + 3 < 8) fx[(ks + 3) % 4] = frag_rows(x, 32 * j, ks + 3), fy[(ks + 3) % 4] = frag_rows(y, 32 * j, ks + 3);
    __builtin_amdgcn_sched_barrier(kFence);
    s = mfma(fx[ks % 4], xf[ks], s);
    t = mfma(fy[ks % 4], yf[ks], t);
    __builtin_amdgcn_sched_barrier(kFence);
  }
}

// The same with the A fragments read two slices ahead and the B operands
// (the wave's own keys of K and V) held in registers for the whole sweep.
__device__ __forceinline__ void scores_kv(const uint16_t* x, const uint16_t* y, int j, const bf16x8 (&kf)[8],
                                          const bf16x8 (&vf)[8], f32x16& s, f32x16& t) {
  bf16x8 f[3][2];
  auto read = [&](int ks, int r) { f[r][0] = frag_rows(x, 32 * j, ks), f[r][1] = frag_rows(y, 32 * j, ks); };
  read(0, 0);
  read(1, 1);
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) {
    if (ks + 2 < 8) read(ks + 2, (ks + 2) % 3);
    __builtin_amdgcn_sched_barrier(kFence);
    s = mfma(f[ks % 3][0], kf[ks], s);
    t = mfma(f[ks % 3][1], vf[ks], t);
    __builtin_amdgcn_sched_barrier(kFence);
  }
}

// ---- backward: dK, dV for a block of 128 keys -------------------------------------
// Each wave owns 32 keys.  Per query block of 64: S (64 queries x 32 keys)
// = Q K' with queries along the registers and keys along the lanes, so the
// products over queries (dV = P' dO, dK = dS' Q) take P and dS straight from
// the accumulators as their B operands, against dO' and Q' read transposed
// from the row-major tiles.

constexpr int kBwdK = 128;  // keys per workgroup
constexpr int kBwdQ = 64;   // queries per step
constexpr size_t kStageBwd = 2 * kTileElems * sizeof(uint16_t) + 2 * 64 * sizeof(float);
constexpr int kBwdStages = 3;  // query blocks in LDS: one read, two loading
constexpr size_t kDsScratch = kBwdStages * kStageBwd;  // then 4 waves x 32 rows of 64 bf16
constexpr size_t kDkdvLds = kDsScratch + 4 * 32 * 64 * sizeof(uint16_t);

// A wave's dS' transpose scratch: 32 key rows of 64 queries (128 bytes), the
// sixteen 8-byte chunks of row r stored at c ^ sw(r), sw(r) = 8 ((r / 2) % 2)
// + r / 4.  The rows' writes (32 lanes, one chunk of 32 rows) fill the 64
// banks once: rows of one parity share a half of the banks and sw is a
// bijection on them.  The transposed reads (32 lanes, rows 4 n .. 4 n + 3
// by eight aligned chunks) do too: rows 4 n and 4 n + 2 (and 4 n + 1, 4 n + 3)
// land in opposite aligned eights.
__device__ __forceinline__ int ds_at(int r, int c8) { return r * 64 + 4 * (c8 ^ (8 * ((r / 2) % 2) + r / 4)); }

// The gradient products of slices ks0, ks0 + 1 (rows 16 ks0 .. 16 ks0 + 31):
// dv += dO' P, dk += Q' dS, fragments read half a slice ahead.  kAgpr: dv and
// dk live in AGPRs (the stored-dS' sweep: 129 fewer register moves a step,
// -3 % on config 4's backward; the recompute sweep, whose registers are
// allocated differently, is left as it was).
template <bool kAgpr>
__device__ __forceinline__ void grads_half(const uint16_t* g, const uint16_t* q, int ks0, const bf16x8 (&pf)[4],
                                           const bf16x8 (&sf)[4], f32x16 (&dv)[4], f32x16 (&dk)[4]) {
  // Unit u = (slice ks0 + u / 2, d blocks 2 (u % 2), 2 (u % 2) + 1).
  bf16x8 fg[3][2], fq[3][2];
  auto read = [&](int u, int r) {
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int db = 2 * (u % 2) + e;
      fg[r][e] = frag_tr(g, 32 * db, ks0 + u / 2);
      fq[r][e] = frag_tr(q, 32 * db, ks0 + u / 2);
    }
  };
  read(0, 0);
  read(1, 1);
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    if (u + 2 < 4) read(u + 2, (u + 2) % 3);
    __builtin_amdgcn_sched_barrier(kFence);
    const int ks = ks0 + u / 2;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int db = 2 * (u % 2) + e;
      if constexpr (kAgpr) {
        mfma_agpr(fg[u % 3][e], pf[ks], dv[db]);
        mfma_agpr(fq[u % 3][e], sf[ks], dk[db]);
      } else {
        dv[db] = mfma(fg[u % 3][e], pf[ks], dv[db]);
        dk[db] = mfma(fq[u % 3][e], sf[ks], dk[db]);
      }
    }
    __builtin_amdgcn_sched_barrier(kFence);
  }
}

// P and dS of score rows 32 j .. 32 j + 31 into pf[2 j], pf[2 j + 1], sf[...].
__device__ __forceinline__ void weights_rows(const f32x16& s, const f32x16& dp, float c, bf16x8& p0, bf16x8& p1,
                                             bf16x8& s0, bf16x8& s1) {
  u32x4 wp[2], ws[2];
#pragma unroll
  for (int i = 0; i < 16; i += 2) {
    const float w0 = __builtin_amdgcn_exp2f(s[i] * c), w1 = __builtin_amdgcn_exp2f(s[i + 1] * c);
    wp[i / 8][(i % 8) / 2] = pack2(w0, w1);
    ws[i / 8][(i % 8) / 2] = pack2(w0 * dp[i], w1 * dp[i + 1]);
  }
  p0 = (bf16x8)wp[0], p1 = (bf16x8)wp[1], s0 = (bf16x8)ws[0], s1 = (bf16x8)ws[1];
}

// kStore: also write dS' (bf16, exactly the values the dK product uses) to
// the workspace, for the dQ kernel that reads it instead of recomputing.
template <bool kStore>
__global__ __launch_bounds__(256, 1) void attn_bwd_dkdv(AttnArgs p) {
  extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
  const size_t stage_elems = kStageBwd / sizeof(uint16_t);
  const int nkb = p.seq / kBwdK;
  // Causal: workgroup x takes key blocks x and nkb - 1 - x, so every
  // workgroup sweeps the same number of query blocks.
  const Block blk = xcd_block();
  const int npass = (p.causal && 2 * blk.x + 1 != nkb) ? 2 : 1;
  for (int pass = 0; pass < npass; ++pass) {
    const int kbk = pass == 0 ? blk.x : nkb - 1 - blk.x;
    // One workgroup per kv head: dK and dV sum over the query heads
    // hk * group .. hk * group + group - 1 that read it, swept in turn.
    const int hk = blk.y, b = blk.z;
    const int group = p.heads / p.kv_heads;
    const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const int lr = lane % 32, lh = lane / 32;
    const int k0 = kbk * kBwdK + wave * 32;
    const int key = k0 + lr;
    const int nq = p.seq / kBwdQ;
    // This wave's 32 keys of K and V as the B operands of the score products,
    // in registers for the whole sweep.
    bf16x8 kf[8], vf[8];
    {
      const int64_t at = (int64_t)b * p.k_sb + (int64_t)hk * p.k_sh + (int64_t)key * p.k_ss;
      row_operand(p.k + at, kf);
      row_operand(p.v + at, vf);
    }

    f32x16 dk[4], dv[4];
  #pragma unroll
    for (int i = 0; i < 4; ++i) dk[i] = f32x16{}, dv[i] = f32x16{};
    const float c = p.scale * kLog2e;

    for (int h = hk * group; h < (hk + 1) * group; ++h) {
      const uint16_t* qbase = p.q + (int64_t)b * p.q_sb + (int64_t)h * p.q_sh;
      const uint16_t* gbase = p.dout + (int64_t)b * p.q_sb + (int64_t)h * p.q_sh;
      // Stage layout: Q tile, dO tile, then [-lse / scale | -delta] of its 64 queries.
      auto Qs = [&](int s) { return lds + s * stage_elems; };
      auto Gs = [&](int s) { return lds + s * stage_elems + kTileElems; };
      auto Ls = [&](int s) { return reinterpret_cast<float*>(lds + s * stage_elems + 2 * kTileElems); };

      const int qstart = p.causal ? (kbk * kBwdK) / kBwdQ : 0;
      // A query block's Q and dO tiles and statistics go straight from global
      // memory into a stage, two blocks ahead: four 1 KB loads per wave for
      // each tile, and one 256-byte load of statistics per wave (waves w and
      // w + 2 fetch the same half, so every wave issues the same nine loads).
      const TileDma qt(qbase, p.q_ss), gt(gbase, p.q_ss);
      const __amdgpu_buffer_rsrc_t srsrc = th_dev::buffer_of(p.stat + ((int64_t)b * p.heads + h) * nq * 128);
      auto fetch = [&](int qb, int s) {
        qt.load(qb * kBwdQ, Qs(s));
        gt.load(qb * kBwdQ, Gs(s));
        const int half = __builtin_amdgcn_readfirstlane(wave) % 2;
        th_dev::dma4(srsrc, 4 * lane, qb * 512 + 256 * half, (uint32_t)(uintptr_t)Ls(s) + 256 * half);
      };
      // Accumulator start: register i of row block j holds query 32 j + 8 (i / 4) + 4 lh + i % 4.
      auto start = [&](const float* v, int j) {
        f32x16 a;
    #pragma unroll
        for (int m = 0; m < 4; ++m) {
          const f32x4 x = *reinterpret_cast<const f32x4*>(v + 32 * j + 8 * m + 4 * lh);
    #pragma unroll
          for (int e = 0; e < 4; ++e) a[4 * m + e] = x[e];
        }
        return a;
      };
      // dS' of a query block, transposed through this wave's LDS scratch (32
      // key rows) so that it leaves as whole 128-byte lines.  It is written
      // there at the end of its step and stored during the next one (or after
      // the sweep), beside that step's products.
      uint16_t* const scratch = lds + kDsScratch / sizeof(uint16_t) + wave * 32 * 64;
      // The four product fragments of the scratch's 32 keys x 64 queries, read
      // transposed (two ds_read_b64_tr_b16 each, as frag_tr): fragment 2 kk + f
      // is keys 16 kk .. + 15 by queries 32 f .. + 31, lane l holding query
      // 32 f + l % 32 and keys 16 kk + 8 (e / 4) + 4 (l / 32) + e % 4 in element e.
      u32x4 pend[4];
      auto scratch_read = [&]() {
        const int g = lane / 16, i = lane % 16;
  #pragma unroll
        for (int kk = 0; kk < 2; ++kk)
  #pragma unroll
          for (int f = 0; f < 2; ++f) {
            const int row = 16 * kk + 4 * (g / 2) + i / 4, c8 = 8 * f + 4 * (g % 2) + i % 4;
            const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(scratch + ds_at(row, c8)));
            const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(scratch + ds_at(row + 8, c8)));
            const u32x2 a = __builtin_bit_cast(u32x2, lo), c = __builtin_bit_cast(u32x2, hi);
            pend[2 * kk + f] = u32x4{a[0], a[1], c[0], c[1]};
          }
      };
      // dS' leaves in the dQ sweep's operand order: for each (batch, head), 64-query
      // block and 16-key slice, two 1 KB fragments (queries 0..31, 32..63 of the
      // block), lane l's 16 bytes at 16 l.  This wave's 32 keys and 64 queries
      // are the four fragments of slices k0 / 16, k0 / 16 + 1: 4 KB in one piece.
      auto store_pending = [&](int qq0) {
        uint16_t* frag0 = p.ds + (((int64_t)b * p.heads + h) * (p.seq / 64) + qq0 / 64) * ((int64_t)p.seq * 64) +
                          (int64_t)(k0 / 16) * 1024 + 8 * lane;
  #pragma unroll
        for (int i = 0; i < 4; ++i) __builtin_nontemporal_store(pend[i], reinterpret_cast<u32x4*>(frag0 + 512 * i));
      };
      // Blocks past the end are a harmless reload of the last one into an idle stage.
      fetch(qstart, 0);
      fetch(min(qstart + 1, nq - 1), 1);
      th_dev::wait_and_meet<9>();
      int st = 0;  // the stage of block qb
      for (int qb = qstart; qb < nq; ++qb) {
        const int s2 = st >= kBwdStages - 2 ? st + 2 - kBwdStages : st + 2;
        fetch(min(qb + 2, nq - 1), s2);
        if constexpr (kStore)
          if (qb > qstart) scratch_read();
        const uint16_t *Q = Qs(st), *G = Gs(st);
        const float* L = Ls(st);
        // S~ = Q K' - lse / scale, dP~ = dO V' - delta (64 queries x 32 keys).
        f32x16 s[2], dp[2];
        s[0] = start(L, 0), dp[0] = start(L + 64, 0);
        s[1] = start(L, 1), dp[1] = start(L + 64, 1);
        scores_kv(Q, G, 0, kf, vf, s[0], dp[0]);
        // The previous block's dS' leaves after this step's loads were issued,
        // so the wait for those loads at the end of the step can leave these
        // four stores in flight.
        if constexpr (kStore)
          if (qb > qstart) store_pending((qb - 1) * kBwdQ);
        // On the diagonal the masked scores become -inf: their P and dS are exactly 0.
        const int qq0 = qb * kBwdQ;
        const bool diagonal = p.causal && qq0 < k0 + 32;
        const int lim = key - qq0 - 4 * lh;  // masked: query offset 32 j + 8 (i / 4) + i % 4 < lim
        if (diagonal) {
    #pragma unroll
          for (int i = 0; i < 16; ++i)
            if (8 * (i / 4) + i % 4 < lim) s[0][i] = -INFINITY;
        }
        bf16x8 pf[4], sf[4];
        scores_kv(Q, G, 1, kf, vf, s[1], dp[1]);
        weights_rows(s[0], dp[0], c, pf[0], pf[1], sf[0], sf[1]);
        // Keep these weights here, beside the products above, rather than sunk
        // past the branch below into the next phase.
        asm volatile("" ::"v"(pf[0]), "v"(pf[1]), "v"(sf[0]), "v"(sf[1]));
        if (diagonal) {
    #pragma unroll
          for (int i = 0; i < 16; ++i)
            if (32 + 8 * (i / 4) + i % 4 < lim) s[1][i] = -INFINITY;
        }
        // dV' (128 d x 32 keys) += dO' P;  dK' += Q' dS.
        grads_half<kStore>(G, Q, 0, pf, sf, dv, dk);
        weights_rows(s[1], dp[1], c, pf[2], pf[3], sf[2], sf[3]);
        grads_half<kStore>(G, Q, 2, pf, sf, dv, dk);
        if constexpr (kStore) {
          // sf[ks] element e is query 16 ks + 8 (e / 4) + 4 lh + e % 4 of this lane's key.
  #pragma unroll
          for (int ks = 0; ks < 4; ++ks) {
            const u32x4 x = __builtin_bit_cast(u32x4, sf[ks]);
            *reinterpret_cast<u32x2*>(scratch + ds_at(lr, 4 * ks + lh)) = u32x2{x[0], x[1]};
            *reinterpret_cast<u32x2*>(scratch + ds_at(lr, 4 * ks + 2 + lh)) = u32x2{x[2], x[3]};
          }
        }
        // Wait for block qb + 1's stage.  After its nine loads this wave has
        // issued the previous step's four stores (past its first step), this
        // step's nine loads, and this step's four stores (past the first).
        if (!kStore || qb == qstart) th_dev::wait_and_meet<9>();
        else if (qb == qstart + 1) th_dev::wait_and_meet<13>();
        else th_dev::wait_and_meet<17>();
        st = st == kBwdStages - 1 ? 0 : st + 1;
      }
      // No load may land in this workgroup's LDS after the sweep.
      th_dev::wait_and_meet<0>();
      if constexpr (kStore) {
        scratch_read();
        store_pending((nq - 1) * kBwdQ);
      }
    }  // query heads of the group
    if constexpr (kStore) agpr_settle(dk, dv);
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
}

// ---- backward: dQ for a block of 128 queries -----------------------------------------
// Each wave owns 32 queries.  Per key block of 64: S' = K Q', dP' = V dO'
// (keys on registers, queries on lanes), dS' = P' .* (dP' - delta), and
// dQ' (128 d x 32 queries) += K' dS' with K' read transposed from K's tile.

constexpr size_t kDqLds = 4 * kTileElems * sizeof(uint16_t);  // (K, V) x 2 stages
constexpr double kDsBudget = 16.0 * (1 << 30);  // bytes of dS' workspace the backward may hold

// dq += K' dS' over slices ks0, ks0 + 1, fragments one slice ahead.
__device__ __forceinline__ void dq_half(const uint16_t* k, int ks0, const bf16x8 (&sf)[4], f32x16 (&dq)[4]) {
  bf16x8 f[2][4];
#pragma unroll
  for (int db = 0; db < 4; ++db) f[0][db] = frag_tr(k, 32 * db, ks0);
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    if (u == 0) {
#pragma unroll
      for (int db = 0; db < 4; ++db) f[1][db] = frag_tr(k, 32 * db, ks0 + 1);
    }
    __builtin_amdgcn_sched_barrier(kFence);
#pragma unroll
    for (int db = 0; db < 4; ++db) dq[db] = mfma(f[u][db], sf[ks0 + u], dq[db]);
    __builtin_amdgcn_sched_barrier(kFence);
  }
}

// dS' of key rows 32 j .. 32 j + 31 (one query per lane) into sf[2 j], sf[2 j + 1].
__device__ __forceinline__ void dq_weights(const f32x16& s, const f32x16& dp, float c, bf16x8& s0, bf16x8& s1) {
  u32x4 w[2];
#pragma unroll
  for (int i = 0; i < 16; i += 2) {
    const float p0 = __builtin_amdgcn_exp2f(s[i] * c), p1 = __builtin_amdgcn_exp2f(s[i + 1] * c);
    w[i / 8][(i % 8) / 2] = pack2(p0 * dp[i], p1 * dp[i + 1]);
  }
  s0 = (bf16x8)w[0], s1 = (bf16x8)w[1];
}

__global__ __launch_bounds__(256, 1) void attn_bwd_dq(AttnArgs p) {
  extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
  const int nqb = p.seq / kFwdQ;
  // Causal: workgroup x takes query blocks x and nqb - 1 - x (equal work).
  const Block blk = xcd_block();
  const int npass = (p.causal && 2 * blk.x + 1 != nqb) ? 2 : 1;
  for (int pass = 0; pass < npass; ++pass) {
    const int qb = pass == 0 ? blk.x : nqb - 1 - blk.x;
    const int h = blk.y, b = blk.z;
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
    // S~' = K Q' - lse / scale and dP~' = V dO' - delta start from these.
    const float ls0 = -p.lse[srow] / p.scale;
    const float dl0 = -p.delta[srow];
    const float c = p.scale * kLog2e;

    const uint16_t* kbase = p.k + (int64_t)b * p.k_sb + (int64_t)hk * p.k_sh;
    const uint16_t* vbase = p.v + (int64_t)b * p.k_sb + (int64_t)hk * p.k_sh;
    f32x16 dq[4];
  #pragma unroll
    for (int i = 0; i < 4; ++i) dq[i] = f32x16{};

    const int nkb = p.causal ? ((qb + 1) * kFwdQ) / kFwdK : p.seq / kFwdK;
    const int64_t step_elems = (int64_t)kFwdK * p.k_ss;
    const TileRows rows(p.k_ss);
    u32x4 rk[4], rv[4];
    auto Ks = [&](int s) { return lds + 2 * s * kTileElems; };
    auto Vs = [&](int s) { return lds + (2 * s + 1) * kTileElems; };
    rows.load(kbase, rk);
    rows.load(vbase, rv);
    store_rows(Ks(0), rk);
    store_rows(Vs(0), rv);
    __syncthreads();
    for (int kb = 0; kb < nkb; ++kb) {
      const int st = kb & 1;
      const int64_t at = (int64_t)min(kb + 1, nkb - 1) * step_elems;  // past the end: a harmless reload
      rows.load(kbase + at, rk);
      rows.load(vbase + at, rv);
      const uint16_t *K = Ks(st), *V = Vs(st);
      f32x16 s[2], dp[2];
  #pragma unroll
      for (int j = 0; j < 2; ++j)
  #pragma unroll
        for (int i = 0; i < 16; ++i) s[j][i] = ls0, dp[j][i] = dl0;
      scores_half(K, V, 0, qf, gf, s[0], dp[0]);
      const int key0 = kb * kFwdK;
      const bool diagonal = p.causal && key0 + kFwdK > q0;
      const int lim = query - key0 - 4 * lh;  // masked: key offset 32 j + 8 (i / 4) + i % 4 > lim
      if (diagonal) {
  #pragma unroll
        for (int i = 0; i < 16; ++i)
          if (8 * (i / 4) + i % 4 > lim) s[0][i] = -INFINITY;
      }
      bf16x8 sf[4];
      scores_half(K, V, 1, qf, gf, s[1], dp[1]);
      dq_weights(s[0], dp[0], c, sf[0], sf[1]);
      if (diagonal) {
  #pragma unroll
        for (int i = 0; i < 16; ++i)
          if (32 + 8 * (i / 4) + i % 4 > lim) s[1][i] = -INFINITY;
      }
      // dQ' (128 d x 32 queries) += K' dS'.
      dq_half(K, 0, sf, dq);
      dq_weights(s[1], dp[1], c, sf[2], sf[3]);
      dq_half(K, 2, sf, dq);
      store_rows(Ks(st ^ 1), rk);
      store_rows(Vs(st ^ 1), rv);
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
}

// ---- stores of 32 rows of 128 through LDS ----------------------------------------
// Four 32 x 32 accumulators acc[db] holding X'(d, row) (lane l: row l % 32,
// d = 32 db + 8 g + 4 (l / 32) + i for register 4 g + i), scaled and rounded
// to bf16, leave as whole 256-byte rows of X (row r at out + r * rs): written
// to a wave's 8 KB of LDS (stage_rows), row r's 16-byte chunk c at position
// c ^ (r % 16) (rows of one write are 16 distinct chunks, two rows apart by
// 16 share one; a row's read back is all 64 banks), then read back 16 lanes a
// row and stored 4 rows an instruction (flush_rows).  Scattered 8-byte stores
// of the same rows (two lanes a row, 32 rows an instruction) measured 15 us
// more for config 4's dQ.
// `lane` is threadIdx.x % 64, passed in so that a caller can make it opaque
// after its sweep (keeping this address arithmetic out of the sweep).
__device__ __forceinline__ void stage_rows(uint16_t* stage, const f32x16 (&acc)[4], float sc, int lane) {
  const int lr = lane % 32, lh = lane / 32;
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int c = 4 * db + g;
      *reinterpret_cast<u32x2*>(stage + lr * kD + 8 * (c ^ (lr % 16)) + 4 * lh) =
          u32x2{pack2(acc[db][4 * g] * sc, acc[db][4 * g + 1] * sc), pack2(acc[db][4 * g + 2] * sc, acc[db][4 * g + 3] * sc)};
    }
}

__device__ __forceinline__ void flush_rows(const uint16_t* stage, uint16_t* out, int64_t rs, int lane) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int r = 4 * i + lane / 16, c = lane % 16;
    const u32x4 v = *reinterpret_cast<const u32x4*>(stage + r * kD + 8 * (c ^ (r % 16)));
    *reinterpret_cast<u32x4*>(out + r * rs + 8 * c) = v;
  }
}

// ---- backward: dQ from dS' in operand order ---------------------------------------
// dQ' (128 d x 64 queries per wave, 256 queries per workgroup) += K' dS' over
// key steps of 64.  dS' comes straight from memory into registers: the dK/dV
// sweep stored it in this product's B-operand order (per 64-query block and
// 16-key slice, two 1 KB fragments, lane l's 16 bytes at 16 l), so each wave
// streams its own queries' dS' as whole contiguous kilobytes, read once
// (non-temporal), one step ahead.  Only K goes through LDS, where the four
// waves share it: a step's 64 K rows are loaded into registers two steps
// ahead and written to one of two LDS stages at the end of the step before
// their own, K' read transposed from there (frag_tr).  Per step a wave
// issues 32 products against 16 KB of LDS reads (64 B a clock a CU at the
// matrix cores' rate; the earlier sweep that staged dS' through LDS as well
// needed three times that).  Every load is an ordinary one that the compiler
// sees and waits for exactly; sweeps have an even number of steps (seq is a
// multiple of 128), so the loop runs two steps an iteration, the register
// sets trading roles, with no early exit.  Causal: waves multiply nothing
// past their own diagonal (fragments there were never written; their loads
// re-read the wave's last block) and workgroup x takes query blocks x and its
// mirror; waves whose queries lie past the sequence load K and compute nothing.

constexpr int kDqfQ = 256;  // queries per workgroup (64 per wave)
constexpr int kDqfK = 64;   // keys per step
constexpr size_t kDqfLds = 6 * kTileElems * sizeof(uint16_t);  // two 64-key stages of K, then 4 waves x 16 KB of kept dQ rows

__global__ __launch_bounds__(256, 1) void attn_bwd_dq_frag(AttnArgs p) {
  extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
  const int nqb = (p.seq + kDqfQ - 1) / kDqfQ;
  const Block blk = xcd_block();
  const int npass = (p.causal && 2 * blk.x + 1 != nqb) ? 2 : 1;
  for (int pass = 0; pass < npass; ++pass) {
    const int qb = pass == 0 ? blk.x : nqb - 1 - blk.x;
    const int h = blk.y, b = blk.z;
    const int hk = h / (p.heads / p.kv_heads);
    const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const int lr = lane % 32, lh = lane / 32;
    const int nq64 = p.seq / 64;
    const int q64 = qb * 4 + wave;  // this wave's 64-query block
    const bool live = q64 < nq64;
    // Steps the workgroup sweeps (even) and steps this wave multiplies.
    const int nsteps = p.causal ? min(p.seq, (qb + 1) * kDqfQ) / kDqfK : p.seq / kDqfK;
    const int wsteps = !live ? 0 : p.causal ? q64 + 1 : nsteps;
    const int last = max(wsteps, 1) - 1;  // dS' loads past a wave's last step re-read it
    const uint16_t* kbase = p.k + (int64_t)b * p.k_sb + (int64_t)hk * p.k_sh;
    const int64_t kstep = (int64_t)kDqfK * p.k_ss;
    const TileRows rows(p.k_ss);
    const uint16_t* dsw = p.ds + (((int64_t)b * p.heads + h) * nq64 + min(q64, nq64 - 1)) * ((int64_t)p.seq * 64) +
                          8 * lane;
    auto load_ds = [&](int kb, u32x4 (&r)[8]) {
      const uint16_t* at = dsw + (int64_t)min(kb, last) * (4 * 1024);
#pragma unroll
      for (int i = 0; i < 8; ++i) r[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(at + 512 * i));
    };
    auto load_k = [&](int kb, u32x4 (&r)[4]) { rows.load(kbase + (int64_t)min(kb, nsteps - 1) * kstep, r); };
    auto Ks = [&](int s) { return lds + s * kTileElems; };
    f32x16 dq0[4], dq1[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) dq0[i] = f32x16{}, dq1[i] = f32x16{};
    u32x4 dsa[8], dsb[8], ka[4], kb4[4];

    // Step kb: dS' of step kb + 1 and K rows of step kb + 2 are loaded, the
    // products of step kb run (its dS' in `cur`, its K in stage kb % 2), and
    // step kb + 1's K rows (loaded a step ago, in `kn`) go to stage (kb + 1) % 2.
    auto step = [&](int kb, u32x4 (&cur)[8], u32x4 (&nxt)[8], u32x4 (&kn)[4], u32x4 (&kl)[4]) {
      load_ds(kb + 1, nxt);
      load_k(kb + 2, kl);
      if (kb < wsteps) {
        const uint16_t* K = Ks(kb & 1);
        bf16x8 kf[2][4];
#pragma unroll
        for (int db = 0; db < 4; ++db) kf[0][db] = frag_tr(K, 32 * db, 0);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          if (ks + 1 < 4) {
#pragma unroll
            for (int db = 0; db < 4; ++db) kf[(ks + 1) % 2][db] = frag_tr(K, 32 * db, ks + 1);
          }
          const bf16x8 b0 = (bf16x8)cur[2 * ks], b1 = (bf16x8)cur[2 * ks + 1];
#pragma unroll
          for (int db = 0; db < 4; ++db) {
            mfma_agpr(kf[ks % 2][db], b0, dq0[db]);
            mfma_agpr(kf[ks % 2][db], b1, dq1[db]);
          }
        }
      }
      // Every wave has finished reading stage (kb + 1) % 2 (step kb - 1) before
      // the barrier that ended the previous step.
      store_rows(Ks((kb + 1) & 1), kn);
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    };

    load_k(0, ka);
    load_ds(0, dsa);
    load_k(1, kb4);
    store_rows(Ks(0), ka);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    for (int kb = 0; kb < nsteps; kb += 2) {
      step(kb, dsa, dsb, kb4, ka);
      step(kb + 1, dsb, dsa, ka, kb4);
    }
    agpr_settle(dq0, dq1);
    int el = lane;
    asm volatile("" : "+v"(el));  // the epilogue's addresses from here, not hoisted above the sweep
    // dQ leaves as whole rows, and only at the workgroup's end: stores share
    // the wave's in-order count of memory operations with loads, so a store
    // before the next pass's loads would hold up every wait in it until the
    // write is acknowledged (about 70 us over config 4's dQ).  A first pass
    // keeps its rows in this wave's 16 KB of LDS past the K stages; the last
    // stages each half (32 queries) in its 8 KB of the K stages, free after
    // the sweep's last barrier, and stores it and the kept rows.
    uint16_t* const keep = lds + 2 * kTileElems + wave * (64 * kD);
    if (live) {
      if (pass + 1 < npass) {
        stage_rows(keep, dq0, p.scale, el);
        stage_rows(keep + 32 * kD, dq1, p.scale, el);
      } else {
        uint16_t* const stage = lds + wave * (32 * kD);
        const int64_t row0 = (int64_t)b * p.q_sb + (int64_t)h * p.q_sh;
#pragma unroll
        for (int f = 0; f < 2; ++f) {
          stage_rows(stage, f == 0 ? dq0 : dq1, p.scale, el);
          flush_rows(stage, p.dq + row0 + (int64_t)(64 * q64 + 32 * f) * p.q_ss, p.q_ss, el);
        }
      }
    }
    if (pass == 1) {
      // The first pass's rows: query block blk.x.
      const int k64 = blk.x * 4 + wave;
      if (k64 < nq64) {
        const int64_t row0 = (int64_t)b * p.q_sb + (int64_t)h * p.q_sh;
#pragma unroll
        for (int f = 0; f < 2; ++f)
          flush_rows(keep + 32 * kD * f, p.dq + row0 + (int64_t)(64 * k64 + 32 * f) * p.q_ss, p.q_ss, el);
      }
    }
    // The next pass refills stage 0 only after every wave is done with it.
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  }
}

// Workgroups along the sequence: causal ones take a block and its mirror.
unsigned blocks_x(int nblocks, int causal) { return causal ? (unsigned)(nblocks + 1) / 2 : (unsigned)nblocks; }

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

// Whether the matrix-core kernels take the descriptor: bf16, head_dim 128,
// seq a multiple of 128, as many keys as queries, no device-held masks,
// 16-byte rows and operands, tiles and sequences their offsets can span.
bool matrix_cores_take(const th_attention_desc* d, bool backward) {
  const bool ok = (d->flags & TH_ATTN_F32) == 0 && (d->kv_seq == 0 || d->kv_seq == d->seq) && !d->starts &&
                  !d->lengths && d->head_dim == kD && d->seq > 0 && d->seq % 128 == 0;
  if (!ok) return false;
  const char* saved = th_last_error();
  const std::string keep = saved;
  const bool fits = check_desc(d, backward) == TH_OK &&
                    (double)d->seq * d->k_strides[1] * 2 < 2147483648.0 &&
                    (double)d->seq * d->q_strides[1] * 2 < 2147483648.0;
  th::set_error(keep);
  return fits;
}

extern "C" int th_build_attention_fwd(const th_attention_desc* d, th_launch** out) {
  if (int r = th::require_ready()) return r;
  *out = nullptr;
  TH_REQUIRE(d != nullptr, "attention: null descriptor");
  if (!matrix_cores_take(d, false))
    return th::mfma_attention_takes(d)  ? th::build_attention_mfma_fwd(d, out)
           : th::f32_attention_takes(d) ? th::build_attention_f32_fwd(d, out)
                                        : th::build_attention_general_fwd(d, out);
  if (int r = check_desc(d, false)) return r;
  // The forward's direct loads address a (batch, head) sequence of K and V
  // from one base with 32-bit byte offsets.
  TH_REQUIRE((double)d->seq * d->k_strides[1] * 2 < 2147483648.0,
             "attention: a sequence of K or V must span under 2 GiB (seq x position stride x 2 bytes)");
  TH_HIP(hipFuncSetAttribute((const void*)attn_fwd, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kFwdLds));
  AttnArgs a = args_of(d);
  th::Builder b("attention_fwd", 7);  // values 5, 6 (the masks) are read only by the general kernels
  int k = b.kernel((const void*)attn_fwd, "attn_fwd", dim3(blocks_x(d->seq / kFwdQ, d->causal), d->heads, d->batch),
                   dim3(256), (uint32_t)kFwdLds, a);
  b.ref(0, k, TH_OFFSET(AttnArgs, q));
  b.ref(1, k, TH_OFFSET(AttnArgs, k));
  b.ref(2, k, TH_OFFSET(AttnArgs, v));
  b.ref(3, k, TH_OFFSET(AttnArgs, o));
  b.ref(4, k, TH_OFFSET(AttnArgs, lse));
  for (int v = 0; v < 4; ++v) b.align(v, 16);
  const double S = d->seq, BH = (double)d->batch * d->heads;
  const double flops = 4.0 * BH * S * S * kD * (d->causal ? 0.5 : 1.0);
  b.work(2.0 * BH * S * kD * 4 + 4.0 * BH * S, flops, (int64_t)blocks_x(d->seq / kFwdQ, d->causal) * d->heads * d->batch);
  *out = b.release();
  return TH_OK;
}

extern "C" int th_build_attention_bwd(const th_attention_desc* d, th_launch** out) {
  if (int r = th::require_ready()) return r;
  *out = nullptr;
  TH_REQUIRE(d != nullptr, "attention: null descriptor");
  if (!matrix_cores_take(d, true))
    return th::mfma_attention_takes(d)  ? th::build_attention_mfma_bwd(d, out)
           : th::f32_attention_takes(d) ? th::build_attention_f32_bwd(d, out)
                                        : th::build_attention_general_bwd(d, out);
  if (int r = check_desc(d, true)) return r;
  AttnArgs a = args_of(d);
  th::Builder b("attention_bwd", 11);  // values 9, 10 (the masks) are read only by the general kernels
  // The dK/dV sweep loads Q and dO tiles directly into LDS with 32-bit byte
  // offsets from a (batch, head) base.
  TH_REQUIRE((double)d->seq * d->q_strides[1] * 2 < 2147483648.0,
             "attention: a sequence of Q or dO must span under 2 GiB (seq x position stride x 2 bytes)");
  const int64_t rows = (int64_t)d->batch * d->seq * d->heads;
  // Workspace: delta ([b][s][h]), then the per-block statistics (2 floats
  // per row); then dS', stored for the dQ sweep when it fits the budget
  // (4 GiB at B8 H16 S4096; beyond it dQ recomputes S and dP instead).
  const uint64_t at_delta = b.workspace((uint64_t)rows * 3 * sizeof(float));
  const double ds_bytes = 2.0 * d->batch * d->heads * (double)d->seq * d->seq;
  const bool store = ds_bytes <= kDsBudget && !(d->flags & TH_ATTN_RECOMPUTE_DQ);
  const uint64_t at_ds = store ? b.workspace((uint64_t)ds_bytes) : 0;
  const void* dkdv = store ? (const void*)attn_bwd_dkdv<true> : (const void*)attn_bwd_dkdv<false>;
  const void* dqk = store ? (const void*)attn_bwd_dq_frag : (const void*)attn_bwd_dq;
  const size_t dq_lds = store ? kDqfLds : kDqLds;
  TH_HIP(hipFuncSetAttribute(dkdv, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kDkdvLds));
  TH_HIP(hipFuncSetAttribute(dqk, hipFuncAttributeMaxDynamicSharedMemorySize, (int)dq_lds));
  TH_REQUIRE(rows < 2147483648LL, "attention: batch x seq x heads must be under 2^31");
  int k0 = b.kernel((const void*)attn_bwd_delta, "attn_bwd_delta", dim3((unsigned)((rows + 16 * kDeltaRows - 1) / (16 * kDeltaRows))),
                    dim3(256), 0, a);
  int k1 = b.kernel(dkdv, store ? "attn_bwd_dkdv_store" : "attn_bwd_dkdv",
                    dim3(blocks_x(d->seq / kBwdK, d->causal), d->kv_heads, d->batch), dim3(256), (uint32_t)kDkdvLds, a);
  const unsigned dq_blocks = store ? blocks_x((d->seq + kDqfQ - 1) / kDqfQ, d->causal) : blocks_x(d->seq / kFwdQ, d->causal);
  int k2 = b.kernel(dqk, store ? "attn_bwd_dq_frag" : "attn_bwd_dq", dim3(dq_blocks, d->heads, d->batch), dim3(256),
                    (uint32_t)dq_lds, a);
  const size_t offs[9] = {TH_OFFSET(AttnArgs, q),   TH_OFFSET(AttnArgs, k),  TH_OFFSET(AttnArgs, v),
                          TH_OFFSET(AttnArgs, o),   TH_OFFSET(AttnArgs, lse), TH_OFFSET(AttnArgs, dout),
                          TH_OFFSET(AttnArgs, dq),  TH_OFFSET(AttnArgs, dk), TH_OFFSET(AttnArgs, dv)};
  for (int v = 0; v < 9; ++v)
    for (int kk : {k0, k1, k2}) b.ref(v, kk, offs[v]);
  for (int kk : {k0, k1, k2}) {
    b.ws_ref(kk, TH_OFFSET(AttnArgs, delta), at_delta);
    b.ws_ref(kk, TH_OFFSET(AttnArgs, stat), at_delta + (uint64_t)rows * sizeof(float));
    if (store) b.ws_ref(kk, TH_OFFSET(AttnArgs, ds), at_ds);
  }
  for (int v : {0, 1, 2, 3, 5, 6, 7, 8}) b.align(v, 16);
  const double S = d->seq, BH = (double)d->batch * d->heads;
  const double flops = 2.5 * 4.0 * BH * S * S * kD * (d->causal ? 0.5 : 1.0);
  const double ds_traffic = store ? 2.0 * ds_bytes * (d->causal ? 0.5 : 1.0) : 0.0;
  b.work(2.0 * BH * S * kD * 8 + 8.0 * BH * S + ds_traffic, flops, (int64_t)blocks_x(d->seq / kBwdK, d->causal) * d->heads * d->batch);
  *out = b.release();
  return TH_OK;
}
