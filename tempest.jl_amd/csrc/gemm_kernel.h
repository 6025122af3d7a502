// Op class (b): bf16 products on CDNA4 matrix cores, fp32 accumulation, with
// the epilogues a planned group fuses after them.  The kernel template; each
// gemm_*.hip instantiates one epilogue (they compile in parallel).
//
// C (m x n, column-major) = A (m x k) * B (k x n), each operand given by its
// two strides, one of which is 1: "k-contiguous" or "mn-contiguous".  One
// workgroup of four waves computes a 256 x 256 tile of C; each wave a
// 128 x 128 quarter as 4 x 4 v_mfma_f32_32x32x16_bf16 blocks (256 fp32
// accumulators per lane, in AGPRs).
//
// Interior tiles (sizes multiples of the tile, k of 64) take the direct path:
// loads straight from global memory into LDS rings several K tiles deep, one
// barrier per 32 of K (sweep_direct below).  Edge tiles take the checked
// path: K advances 64 at a time through two LDS stages, the next tile's
// global loads in flight into registers while the waves multiply out of one
// stage.  Its LDS rows are k-contiguous, 64 bf16 plus 8 of padding (144
// bytes), so the 16-byte fragment reads of 16 lanes fall on 16 distinct bank
// quads.  An mn-contiguous operand is transposed on its way into LDS: each
// thread loads an 8 x 8 block (eight 16-byte rows along m or n, eight lanes
// along k side by side so their LDS writes spread over the banks) and writes
// it back as eight 16-byte rows along k.
//
// Workgroups are dealt to the eight XCDs round-robin; the tile order is
// remapped so each XCD takes a contiguous range of tiles, grouped 8 tile-rows
// high, and the tiles that share operands share an L2.
//
// Replaces the cuTile product sketch (ext/cuTileExt/contract.jl:32-206, MMA
// step emit.jl:894-948, swizzle build.jl:35-45) and cuBLAS's
// cublasGemmStridedBatchedEx (ext/cuBLASExt.jl:247-259).  Half factors are
// widened to fp32 products and the result rounded once, as the reference's
// interpreter evaluates a contraction (src/Compiler/program/interpret.jl:58-63).
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <type_traits>
#include <utility>

#include "lds_dma.h"

namespace thg {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kTile = 256;            // C tile, both sides
constexpr int kDepth = 64;            // K per stage
constexpr int kRow = 72;              // LDS row: 64 bf16 + 8 padding
constexpr int kStage = kTile * kRow;  // bf16 per operand stage
constexpr int kThreads = 256;
constexpr size_t kLds = 4 * kStage * sizeof(uint16_t);  // A and B, two stages: 147456 bytes

enum Layout { kK = 0, kMN = 1 };
enum Epilogue { kStore = 0, kStoreF32 = 1, kGelu = 2, kSquareLoss = 3, kGeluBackward = 4 };

struct GemmArgs {
  const uint16_t* a;
  const uint16_t* b;
  void* c;
  const uint16_t* bias;  // per-m, bf16 (kStore: optional)
  const uint16_t* aux;   // kGeluBackward: Z, column-major, ld aux_ld
  uint16_t* aux_out;     // kGelu: H, same layout as C
  float* partial;        // row sums per (tile n, wave column) x m; then loss partials
  int64_t a_o, a_k;      // A's strides along m and along k
  int64_t b_o, b_k;      // B's strides along n and along k
  int64_t ldc, aux_ld;
  int32_t m, n, k;
  int32_t tiles_m, tiles_n;
  // Batches (blockIdx.z) and parts of K (blockIdx.y): product z's operands
  // start a_batch, b_batch elements further, its result c_batch further; part
  // s sums k in [s ksplit, (s + 1) ksplit) into the result c_split further.
  int64_t a_batch, b_batch, c_batch, c_split;
  int32_t ksplit;
};

// Round to bf16, nearest even (one v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint16_t bf16_bits(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

__device__ __forceinline__ float bf16_float(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

__device__ __forceinline__ float half_of(uint32_t w, int r) { return bf16_float((uint16_t)(w >> (16 * r))); }

__device__ __forceinline__ u32x2 pack4(const uint16_t (&h)[4]) {
  return u32x2{(uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16)};
}

// GELU, tanh form (test/fixtures/programs.jl:19), and its derivative.  With
// u = c (x + a x^3) and s = 1 / (1 + e^(2u)):
//   1 + tanh u = 2 (1 - s),  1 - tanh^2 u = 4 s (1 - s),  so
//   gelu(x) = x (1 - s),  gelu'(x) = (1 - s) (1 + 2 c x s (1 + 3 a x^2)),
// and 1 - s = e^(2u) s, which has no cancellation for negative x.  e^(2u) is
// exp2(x (k1 + k2 x^2)) with log2(e) folded into the constants, the exponent
// capped at 126 so that e stays finite: there e s rounds to 1 and s is about
// 2^-126, so gelu(x) = x and gelu'(x) = 1 for large x; for large negative x
// e underflows to 0 and both are 0.  One exponential, one reciprocal and
// eight or nine other operations per element (the epilogues that apply them
// are bound by vector instructions).
struct GeluParts {
  float om;  // 1 - s
  float s;
};
__device__ __forceinline__ GeluParts gelu_parts(float x, float x2) {
  constexpr float k1 = 2.30220831f;   // 2 c log2(e), c = 0.7978846
  constexpr float k2 = 0.102943245f;  // 2 c a log2(e), a = 0.044715
  const float e = __builtin_amdgcn_exp2f(fminf(x * fmaf(k2, x2, k1), 126.0f));
  const float s = __builtin_amdgcn_rcpf(1.0f + e);
  return GeluParts{e * s, s};
}
__device__ __forceinline__ float gelu(float x) { return x * gelu_parts(x, x * x).om; }
__device__ __forceinline__ float gelu_grad(float x) {
  constexpr float k3 = 1.5957692f;    // 2 c
  constexpr float k4 = 0.214064459f;  // 6 c a
  const float x2 = x * x;
  const GeluParts g = gelu_parts(x, x2);
  return g.om * fmaf(g.s, x * fmaf(k4, x2, k3), 1.0f);
}

// ---- global -> registers -> LDS ----------------------------------------------

// k-contiguous operand: thread takes the 16-byte chunk tid % 8 of rows
// tid / 8 + 32 i (i = 0..7) of the tile's 256 rows.
template <bool CHECK>
__device__ __forceinline__ void load_k(const uint16_t* base, int64_t s_o, int o0, int k0, int O, int K,
                                       u32x4 (&r)[8]) {
  const int c = threadIdx.x % 8, row = threadIdx.x / 8;
  const int k = k0 + 8 * c;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int o = o0 + row + 32 * i;
    if (!CHECK || (o < O && k < K))
      r[i] = *reinterpret_cast<const u32x4*>(base + (int64_t)o * s_o + k);
    else
      r[i] = u32x4{0, 0, 0, 0};
  }
}

__device__ __forceinline__ void store_k(uint16_t* lds, const u32x4 (&r)[8]) {
  const int c = threadIdx.x % 8, row = threadIdx.x / 8;
#pragma unroll
  for (int i = 0; i < 8; ++i) *reinterpret_cast<u32x4*>(lds + (row + 32 * i) * kRow + 8 * c) = r[i];
}

// mn-contiguous operand: thread (kb = tid % 8, ob = tid / 8) takes the 8 x 8
// block of rows k0 + 8 kb + (0..7), columns o0 + 8 ob + (0..7).
template <bool CHECK>
__device__ __forceinline__ void load_mn(const uint16_t* base, int64_t s_k, int o0, int k0, int O, int K,
                                        u32x4 (&r)[8]) {
  const int kb = threadIdx.x % 8, ob = threadIdx.x / 8;
  const int o = o0 + 8 * ob;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int k = k0 + 8 * kb + i;
    if (!CHECK || (o < O && k < K))
      r[i] = *reinterpret_cast<const u32x4*>(base + o + (int64_t)k * s_k);
    else
      r[i] = u32x4{0, 0, 0, 0};
  }
}

// Transpose the 8 x 8 block in registers and write it as 8 rows along k.
__device__ __forceinline__ void store_mn(uint16_t* lds, const u32x4 (&r)[8]) {
  const int kb = threadIdx.x % 8, ob = threadIdx.x / 8;
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    u32x4 w;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t lo = r[2 * e][c / 2], hi = r[2 * e + 1][c / 2];
      w[e] = (c % 2 == 0) ? ((lo & 0xffffu) | (hi << 16)) : ((lo >> 16) | (hi & 0xffff0000u));
    }
    *reinterpret_cast<u32x4*>(lds + (8 * ob + c) * kRow + 8 * kb) = w;
  }
}

template <int L, bool CHECK>
__device__ __forceinline__ void load_tile(const uint16_t* base, int64_t s_o, int64_t s_k, int o0, int k0, int O,
                                          int K, u32x4 (&r)[8]) {
  if constexpr (L == kK)
    load_k<CHECK>(base, s_o, o0, k0, O, K, r);
  else
    load_mn<CHECK>(base, s_k, o0, k0, O, K, r);
}

template <int L>
__device__ __forceinline__ void store_tile(uint16_t* lds, const u32x4 (&r)[8]) {
  if constexpr (L == kK)
    store_k(lds, r);
  else
    store_mn(lds, r);
}

// Interior tiles load through a buffer resource: the operand's base in
// scalar registers, each of the thread's eight 16-byte loads a 32-bit byte
// offset fixed for the whole sweep, and the K tile's advance a scalar offset.
// Operands stay under 2 GiB on this path (the builder checks).
template <int L>
struct Sweep {
  __amdgpu_buffer_rsrc_t rsrc;
  uint32_t off[8];
  uint32_t step;

  __device__ __forceinline__ void init(const uint16_t* base, int64_t s_o, int64_t s_k, int o0) {
    rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(base), (short)0, 0x7fffffff, 0x00020000);
    if constexpr (L == kK) {
      const int c = threadIdx.x % 8, row = threadIdx.x / 8;
#pragma unroll
      for (int i = 0; i < 8; ++i) off[i] = (uint32_t)(((int64_t)(o0 + row + 32 * i) * s_o + 8 * c) * 2);
      step = kDepth * 2;
    } else {
      const int kb = threadIdx.x % 8, ob = threadIdx.x / 8;
#pragma unroll
      for (int i = 0; i < 8; ++i) off[i] = (uint32_t)(((int64_t)(o0 + 8 * ob) + (int64_t)(8 * kb + i) * s_k) * 2);
      step = (uint32_t)(kDepth * s_k * 2);
    }
  }

  __device__ __forceinline__ void load(int kt, u32x4 (&r)[8]) const {
    const int s = (int)(kt * step);
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = (u32x4)__builtin_amdgcn_raw_buffer_load_b128(rsrc, (int)off[i], s, 0);
  }
};

// The products of one K tile out of LDS stage `stage`: the fragments of the
// next 16-deep step are read while the 16 products of this one issue, and,
// when `land`, the registers of the next tile go to the other stage during
// the last two steps, each LDS access placed between products.
template <int LA, int LB>
__device__ __forceinline__ void multiply_tile(const uint16_t* As, const uint16_t* Bs, uint16_t* As_next,
                                              uint16_t* Bs_next, bool land, const u32x4 (&ra)[8],
                                              const u32x4 (&rb)[8], f32x16 (&acc)[4][4], int wm, int wn,
                                              int lr, int lh) {
  const uint16_t* Ac = As + (wm * 128 + lr) * kRow + 8 * lh;
  const uint16_t* Bc = Bs + (wn * 128 + lr) * kRow + 8 * lh;
  bf16x8 af[2][4], bf[2][4];
#pragma unroll
  for (int i = 0; i < 4; ++i) af[0][i] = *reinterpret_cast<const bf16x8*>(Ac + i * 32 * kRow);
#pragma unroll
  for (int j = 0; j < 4; ++j) bf[0][j] = *reinterpret_cast<const bf16x8*>(Bc + j * 32 * kRow);
#pragma unroll
  for (int kk = 0; kk < kDepth / 16; ++kk) {
    const int s = kk & 1;
    if (kk + 1 < kDepth / 16) {
#pragma unroll
      for (int i = 0; i < 4; ++i) af[s ^ 1][i] = *reinterpret_cast<const bf16x8*>(Ac + i * 32 * kRow + (kk + 1) * 16);
#pragma unroll
      for (int j = 0; j < 4; ++j) bf[s ^ 1][j] = *reinterpret_cast<const bf16x8*>(Bc + j * 32 * kRow + (kk + 1) * 16);
    }
    if (land && kk == 2) store_tile<LA>(As_next, ra);
    if (land && kk == 3) store_tile<LB>(Bs_next, rb);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[s][i], bf[s][j], acc[i][j], 0, 0, 0);
    if (kk < 2) {
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // two products
      }
    } else if (kk == 2) {
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // a product
        __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // one LDS write
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // a product
      }
    } else {
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // one LDS write
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // two products
      }
    }
  }
}

// ---- the direct path (interior tiles): global -> LDS with no registers -------
// buffer_load ... lds writes each lane's 16 bytes at M0 + 16 lane, so one
// wave instruction fills 1 KB of LDS.  The tiles have no padding; instead the
// 16-byte chunks of each row are XOR-permuted, which keeps both the direct
// writes and the fragment reads free of bank conflicts.
//
// K advances 32 at a time (a "tile" below is 32 deep), and each operand has
// its own 64 KiB ring in LDS, laid out for its layout:
//   mn-contiguous: four stages of one tile, [32 k][256 mn] with 512-byte
//     rows, chunk c of row r at c ^ 4 (r % 4), read transposed
//     (ds_read_b64_tr_b16): four consecutive rows x four consecutive chunks
//     land on 16 distinct bank quads.  Each load instruction covers two
//     whole rows.
//   k-contiguous: two slots of two tiles each, [256 rows][64 k] with
//     128-byte rows, chunk c of row r at c ^ ((r / 2) % 8) (16 consecutive
//     rows of one chunk: 16 distinct bank quads).  A slot rather than a
//     stage per tile keeps each load on whole 128-byte lines: a 64-byte row
//     per tile would fetch every line twice, a tile apart, and the CU's fill
//     rate from L2 would bound the sweep.
//
// Each tile's 32 products per wave run as two 16-deep steps with one barrier
// between them.  Step 0 reads the fragments of step 1; the barrier makes the
// next tile's data visible and frees the stage (or slot) read last; step 1
// reads the next tile's first fragments.  No wave ever waits on a fragment
// read at a tile boundary.  The loads of later tiles issue between the
// products (at most four per step and operand, one after every other or
// every fourth product):
//   mn-contiguous: step 0 of tile t, the second half of tile t + 3; step 1,
//     the first half of tile t + 4 (so a tile's loads lead its use by more
//     than two tiles);
//   k-contiguous: step 0 of an even tile 2u, the second half of pair u + 1;
//     step 1 of an odd tile 2u + 1, the first half of pair u + 2 (pair p
//     holds tiles 2p, 2p + 1; its loads lead by one to two tiles).
// Past the last tile the last one is loaded again, into a stage nothing reads
// any more (or the same bytes into its own), so the issue sequence and every
// wait count are the same for every tile; mid_wait counts, from this
// schedule, the loads a wave may leave in flight at each barrier.
// The direct loads are issued from inline assembly (lds_dma.h says why).

constexpr int kDepthD = 32;                                    // K per tile of the direct path
constexpr int kStageBytesMN = kTile * kDepthD * 2;             // one mn-contiguous stage: 16 KiB
constexpr int kSlotBytesK = 2 * kStageBytesMN;                 // one k-contiguous slot: 32 KiB
constexpr uint32_t kRingBytes = 4 * kStageBytesMN;             // one operand's ring: 64 KiB
constexpr int kEpiRow = 136;                                  // LDS row (bf16) of the epilogue's transpose: 128 m + 8
constexpr size_t kEpiWave = 128 * kEpiRow * sizeof(uint16_t);  // one wave's 128 x 128 tile
// Both rings (131072 bytes), or after the sweep the four waves' transposed
// tiles (139264 bytes).
constexpr size_t kLdsDirect = 4 * kEpiWave > 2 * kRingBytes ? 4 * kEpiWave : 2 * kRingBytes;

typedef __attribute__((address_space(3))) void lds_void;
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
typedef __attribute__((address_space(3))) bf16x8 lds_bf16x8;

using th_dev::static_for;
using th_dev::dma16;
using th_dev::wait_and_meet;

// The schedule.  Loads of one operand in step s of tile t:
template <int L>
constexpr int ring_loads(int t, int s) {
  if (L == kMN) return 2;
  return ((s == 0 && t % 2 == 0) || (s == 1 && t % 2 == 1)) ? 4 : 0;
}
// The product after which load j of a step issues: A after products 1 mod 4,
// B after 3 mod 4 (operand op: 0 = A, 1 = B).
template <int L>
constexpr int ring_slot(int op, int j) { return L == kMN ? 2 * op + 1 + 8 * j : 2 * op + 1 + 4 * j; }
// The tile (mn-contiguous) or pair (k-contiguous) the loads of step s of tile t fill.
template <int L>
constexpr int ring_target(int t, int s) {
  if (L == kMN) return s == 0 ? t + 3 : t + 4;
  return s == 0 ? t / 2 + 1 : (t + 1) / 2 + 1;
}
struct IssuePos { int t, s, q; };
constexpr bool issued_after(IssuePos a, IssuePos b) {
  return a.t != b.t ? a.t > b.t : a.s != b.s ? a.s > b.s : a.q > b.q;
}
// The last load of one operand that tile t + 1 needs.
template <int L>
constexpr IssuePos last_needed(int op, int t) {
  if (L == kMN) return IssuePos{t - 2, 0, ring_slot<L>(op, 1)};
  return IssuePos{t % 2 == 0 ? t - 2 : t - 1, 0, ring_slot<L>(op, 3)};
}
// Loads issued after the last one tile t + 1 needs, up to the barrier in the
// middle of tile t: what a wave may leave in flight there.  It depends on
// t's parity only (t >= 2; the prologue makes it hold for t = -1, 0, 1).
template <int LA, int LB>
constexpr int mid_wait(int t) {
  const IssuePos pa = last_needed<LA>(0, t), pb = last_needed<LB>(1, t);
  const IssuePos p = issued_after(pa, pb) ? pa : pb;
  int n = 0;
  for (int tau = t - 4; tau <= t; ++tau)
    for (int s = 0; s < 2 && !(tau == t && s == 1); ++s) {
      for (int j = 0; j < ring_loads<LA>(tau, s); ++j) n += issued_after(IssuePos{tau, s, ring_slot<LA>(0, j)}, p);
      for (int j = 0; j < ring_loads<LB>(tau, s); ++j) n += issued_after(IssuePos{tau, s, ring_slot<LB>(1, j)}, p);
    }
  return n;
}
static_assert(mid_wait<kK, kK>(10) == 16 && mid_wait<kK, kK>(11) == 0, "direct path schedule");
static_assert(mid_wait<kMN, kK>(10) == 16 && mid_wait<kMN, kK>(11) == 4, "direct path schedule");
static_assert(mid_wait<kK, kMN>(10) == 16 && mid_wait<kK, kMN>(11) == 4, "direct path schedule");
static_assert(mid_wait<kMN, kMN>(10) == 16 && mid_wait<kMN, kMN>(11) == 16, "direct path schedule");

// One operand's ring: its buffer resource, the byte offsets of the wave's
// load instructions for K tile (or pair) 0 (the K advance is the scalar
// offset), and the LDS byte addresses of this lane's fragment reads in stage
// (slot) 0.  `wo` is the wave's first row (m or n) of the tile, `ring` the
// ring's LDS byte address, `nk` the number of 32-deep tiles.
template <int L>
struct Ring;

template <>
struct Ring<kMN> {
  __amdgpu_buffer_rsrc_t rsrc;
  int32_t off[4];
  int32_t step;
  uint32_t rd[4];  // per 32-row block
  uint32_t ring;
  int last;

  // Instruction i of wave w fills bytes [1024 (4 w + i), + 1024) of a stage:
  // k rows 8 w + 2 i, + 1.
  __device__ __forceinline__ void init(const uint16_t* base, int64_t s_k, int o0, int wo, uint32_t ring_, int nk) {
    rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(base), (short)0, 0x7fffffff, 0x00020000);
    const int w = threadIdx.x / 64, l = threadIdx.x % 64;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int kr = 8 * w + 2 * i + l / 32, lc = (l % 32) ^ (4 * (kr % 4));
      off[i] = (int32_t)(((int64_t)kr * s_k + o0 + 8 * lc) * 2);
    }
    step = (int32_t)(kDepthD * s_k * 2);
    // ds_read_b64_tr_b16 hands lane i of each 16 element i % 4 of the
    // 8-byte pieces addressed by lanes 4 q + i / 4 (q = 0..3).  Lane j
    // addresses k row j / 4 (+ 8 (l / 32), + 16 kk, + 4 for the upper
    // half), columns ogrp + 4 (j % 4) + (0..3), so lane i receives k rows
    // base + (0..3) of column ogrp + i: k in natural order.
    const int j = l % 16, row = 8 * (l / 32) + j / 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int o = wo + 32 * i + 16 * ((l / 16) % 2) + 4 * (j % 4);
      rd[i] = ring_ + (uint32_t)((row * kTile + 8 * ((o / 8) ^ (4 * (row % 4))) + o % 8) * 2);
    }
    ring = ring_;
    last = nk - 1;
  }
  // Instruction i (0..3) of tile t, into stage t mod 4.
  __device__ __forceinline__ void load(int t, int i) const {
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    dma16(rsrc, off[i], min(t, last) * step, ring + (t & 3) * kStageBytesMN + 1024 * (4 * w + i));
  }
  // Load j of step S of tile t (PAR = t mod 2).
  template <int S, int PAR, int J>
  __device__ __forceinline__ void step_load(int t) const {
    if constexpr (S == 0)
      load(t + 3, 2 + J);
    else
      load(t + 4, J);
  }
  // Fragment I (rows wo + 32 I + lane % 32, k = 16 KK + 8 (lane / 32) + 0..7) of tile t.
  template <int I, int KK, int PAR>
  __device__ __forceinline__ bf16x8 frag(int t) const {
    const uint32_t a = rd[I] + (t & 3) * kStageBytesMN + KK * 16 * kTile * 2;
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(uintptr_t)a);
    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(uintptr_t)(a + 4 * kTile * 2));
    const s16x8 w = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    return __builtin_bit_cast(bf16x8, w);
  }
};

template <>
struct Ring<kK> {
  __amdgpu_buffer_rsrc_t rsrc;
  int32_t off[8];
  uint32_t rd[4];  // per 16-deep step of a pair
  uint32_t ring;
  int last;

  // Instruction i of wave w fills bytes [1024 (8 w + i), + 1024) of a slot:
  // rows 64 w + 8 i .. + 7.
  __device__ __forceinline__ void init(const uint16_t* base, int64_t s_o, int o0, int wo, uint32_t ring_, int nk) {
    rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(base), (short)0, 0x7fffffff, 0x00020000);
    const int w = threadIdx.x / 64, l = threadIdx.x % 64;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = 64 * w + 8 * i + l / 8, lc = (l % 8) ^ ((r / 2) % 8);
      off[i] = (int32_t)(((int64_t)(o0 + r) * s_o + 8 * lc) * 2);
    }
    // Fragment rows wo + l % 32 (+ 32 i: the same permutation), chunk 2 kk + l / 32.
    const int r = wo + l % 32;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
      rd[kk] = ring_ + (uint32_t)((r * 2 * kDepthD + 8 * ((2 * kk + l / 32) ^ ((r / 2) % 8))) * 2);
    ring = ring_;
    last = nk / 2 - 1;
  }
  // Instruction i (0..7) of pair p, into slot p mod 2.
  __device__ __forceinline__ void load(int p, int i) const {
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    dma16(rsrc, off[i], min(p, last) * (4 * kDepthD), ring + (p & 1) * kSlotBytesK + 1024 * (8 * w + i));
  }
  template <int S, int PAR, int J>
  __device__ __forceinline__ void step_load(int t) const {
    if constexpr (S == 0 && PAR == 0)
      load(t / 2 + 1, 4 + J);
    else if constexpr (S == 1 && PAR == 1)
      load((t + 1) / 2 + 1, J);
  }
  template <int I, int KK, int PAR>
  __device__ __forceinline__ bf16x8 frag(int t) const {
    return *reinterpret_cast<const lds_bf16x8*>(
        (uintptr_t)(rd[2 * PAR + KK] + ((t >> 1) & 1) * kSlotBytesK + I * 32 * 2 * kDepthD * 2));
  }
};

// The K sweep of an interior tile: acc += A(m0.., :) B(:, n0..); k a multiple of 64.
template <int LA, int LB>
__device__ __forceinline__ void sweep_direct(const GemmArgs& p, int m0, int n0, int wm, int wn,
                                             f32x16 (&acc)[4][4]) {
  extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
  const uint32_t ra = (uint32_t)(uintptr_t)lds, rb = ra + kRingBytes;
  const int nk = p.k / kDepthD;  // even
  Ring<LA> A;
  Ring<LB> B;
  if constexpr (LA == kK)
    A.init(p.a, p.a_o, m0, wm * 128, ra, nk);
  else
    A.init(p.a, p.a_k, m0, wm * 128, ra, nk);
  if constexpr (LB == kK)
    B.init(p.b, p.b_o, n0, wn * 128, rb, nk);
  else
    B.init(p.b, p.b_k, n0, wn * 128, rb, nk);
  // The loads of step S of tile tau that issue after product Q.
  auto loads_at = [&](int tau, auto S, auto PARI, auto Q) {
    constexpr int st = S, par = PARI, q = Q;
    static_for<4>([&](auto J) {
      if constexpr (J < ring_loads<LA>(par, st) && ring_slot<LA>(0, J) == q) A.template step_load<st, par, J>(tau);
      if constexpr (J < ring_loads<LB>(par, st) && ring_slot<LB>(1, J) == q) B.template step_load<st, par, J>(tau);
    });
  };
  // The prologue issues what the steps of tiles -4 .. -1 would have (loads
  // of tiles before 0 left out), in the same order, so that every wait count
  // of the sweep holds from its first barrier.
  auto virtual_step = [&](auto TAU, auto S) {
    constexpr int tau = TAU, st = S;
    using Par = std::integral_constant<int, ((tau % 2) + 2) % 2>;
    static_for<16>([&](auto Q) {
      static_for<4>([&](auto J) {
        if constexpr (J < ring_loads<LA>(Par::value, st) && ring_slot<LA>(0, J) == Q && ring_target<LA>(tau, st) >= 0)
          A.template step_load<st, Par::value, J>(tau);
        if constexpr (J < ring_loads<LB>(Par::value, st) && ring_slot<LB>(1, J) == Q && ring_target<LB>(tau, st) >= 0)
          B.template step_load<st, Par::value, J>(tau);
      });
    });
  };
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  static_for<4>([&](auto T) {
    using Tau = std::integral_constant<int, T - 4>;
    virtual_step(Tau{}, S0{});
    if constexpr (T == 3) wait_and_meet<mid_wait<LA, LB>(11)>();  // the middle of tile -1: tile 0 has landed
    virtual_step(Tau{}, S1{});
  });
  bf16x8 af[2][4], bf[2][4];
  static_for<4>([&](auto I) {
    af[0][I] = A.template frag<I, 0, 0>(0);
    bf[0][I] = B.template frag<I, 0, 0>(0);
  });
  for (int t0 = 0; t0 < nk; t0 += 2) {
    static_for<2>([&](auto PARI) {
      constexpr int par = PARI;
      const int t = t0 + par;
      // Step 0: products of (t, 0); fragments of (t, 1).
      __builtin_amdgcn_sched_barrier(0);
      static_for<16>([&](auto Q) {
        constexpr int q = Q;
        acc[q / 4][q % 4] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[0][q / 4], bf[0][q % 4], acc[q / 4][q % 4], 0, 0, 0);
        loads_at(t, S0{}, PARI, Q);
        if constexpr (q % 2 == 0) {
          constexpr int r = q / 2;  // a0 b0 a1 b1 ...
          if constexpr (r % 2 == 0)
            af[1][r / 2] = A.template frag<r / 2, 1, par>(t);
          else
            bf[1][r / 2] = B.template frag<r / 2, 1, par>(t);
        }
        __builtin_amdgcn_sched_barrier(0);
      });
      // Tile t + 1 has landed (every wave's share), and every wave is done
      // reading the stage (slot) the next loads fill.
      wait_and_meet<mid_wait<LA, LB>(10 + par)>();
      // Step 1: products of (t, 1); fragments of (t + 1, 0) (past the last
      // tile, bytes nothing uses).
      static_for<16>([&](auto Q) {
        constexpr int q = Q;
        acc[q / 4][q % 4] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[1][q / 4], bf[1][q % 4], acc[q / 4][q % 4], 0, 0, 0);
        loads_at(t, S1{}, PARI, Q);
        if constexpr (q % 2 == 0) {
          constexpr int r = q / 2;
          if constexpr (r % 2 == 0)
            af[0][r / 2] = A.template frag<r / 2, 0, 1 - par>(t + 1);
          else
            bf[0][r / 2] = B.template frag<r / 2, 0, 1 - par>(t + 1);
        }
        __builtin_amdgcn_sched_barrier(0);
      });
    });
  }
  // No load may land in LDS once the epilogue uses it.
  wait_and_meet<0>();
}

// ---- the interior tiles' epilogue: through LDS, whole lines out ------------------
// The accumulators give each lane four consecutive m of one column n, so
// storing straight from them writes 8 bytes into each of 32 columns per
// instruction and lines leave the L2 partly written (about twice the
// algorithmic bytes reach HBM for the fused epilogues).  Instead each wave
// rounds its 128 x 128 tile (plus the bias) to bf16 into its own LDS region,
// column-major with rows of kEpiRow, and reads it back eight m at a time:
// per instruction 16 lanes cover one column's 128 m (256 contiguous bytes),
// so every store writes whole lines.  The element-wise work of the fused
// epilogue (GELU, the square loss, the GELU backward) runs on the values read
// back, rounding where the values are stored, and the row sums fold this
// lane's eight m over its columns, then over the four column groups of lanes,
// in a fixed order.
__device__ __forceinline__ void tile_of(int block, int tiles_m, int tiles_n, int* tm, int* tn);

template <int EPI>
__device__ __forceinline__ void epilogue_lds(const GemmArgs& p, const f32x16 (&acc)[4][4]) {
  extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
  // The tile and wave coordinates are derived again here rather than kept
  // live across the sweep, where every register is taken.
  int tm, tn;
  tile_of(blockIdx.x, p.tiles_m, p.tiles_n, &tm, &tn);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
  const int wm = wave / 2, wn = wave % 2;
  uint16_t* tile = lds + wave * (kEpiWave / sizeof(uint16_t));
  int lane = threadIdx.x % 64;
  asm volatile("" : "+v"(lane));  // keep the epilogue's address arithmetic below the sweep
  const int lr = lane % 32, lh = lane / 32;
  const int mw = tm * kTile + wm * 128, nw = tn * kTile + wn * 128;
  // Phase 1: lane (lr, lh) holds m = 32 i + 8 g + 4 lh + (0..3), n = 32 j + lr.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float bias[4][4];
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int r = 0; r < 4; ++r) bias[g][r] = 0.0f;
    if (EPI == kGelu || EPI == kSquareLoss || (EPI == kStore && p.bias)) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const u32x2 bb = *reinterpret_cast<const u32x2*>(p.bias + mw + 32 * i + 8 * g + 4 * lh);
#pragma unroll
        for (int r = 0; r < 4; ++r) bias[g][r] = half_of(bb[r / 2], r % 2);
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        uint16_t h[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) h[r] = bf16_bits(acc[i][j][4 * g + r] + bias[g][r]);
        *reinterpret_cast<u32x2*>(tile + (32 * j + lr) * kEpiRow + 32 * i + 8 * g + 4 * lh) = pack4(h);
      }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  // Phase 2: lane takes m = 8 (lane % 16) + (0..7) of columns 4 t + lane / 16.
  constexpr bool kSums = EPI == kSquareLoss || EPI == kGeluBackward;
  const int mc = 8 * (lane % 16), cg = lane / 16;
  float rs[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) rs[e] = 0.0f;
  float loss = 0.0f;
  uint16_t* c = static_cast<uint16_t*>(p.c);
  // GELU backward: all of this lane's Z (32 x 16 bytes) is requested before
  // the first store.  Loaded inside the loop, each read would wait for the
  // previous iteration's store (the compiler cannot rule out that they
  // alias), one memory round trip per iteration.  The accumulators are dead
  // here, so the registers are free.
  u32x4 zv[EPI == kGeluBackward ? 32 : 1];
  if constexpr (EPI == kGeluBackward) {
#pragma unroll
    for (int t = 0; t < 32; ++t)
      zv[t] = *reinterpret_cast<const u32x4*>(p.aux + (int64_t)(mw + mc) + (int64_t)(nw + 4 * t + cg) * p.aux_ld);
  }
#pragma unroll
  for (int t = 0; t < 32; ++t) {
    const int nl = 4 * t + cg;
    const u32x4 v = *reinterpret_cast<const u32x4*>(tile + nl * kEpiRow + mc);
    const int64_t at = (int64_t)(mw + mc) + (int64_t)(nw + nl) * p.ldc;
    if constexpr (EPI == kStore) {
      *reinterpret_cast<u32x4*>(c + at) = v;
    } else if constexpr (EPI == kGelu) {
      u32x4 hv;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t lo = bf16_bits(gelu(half_of(v[e], 0))), hi = bf16_bits(gelu(half_of(v[e], 1)));
        hv[e] = lo | (hi << 16);
      }
      *reinterpret_cast<u32x4*>(c + at) = v;
      *reinterpret_cast<u32x4*>(p.aux_out + at) = hv;
    } else if constexpr (EPI == kSquareLoss) {
      u32x4 ov;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float y0 = half_of(v[e], 0), y1 = half_of(v[e], 1);
        const uint16_t o0 = bf16_bits(2.0f * y0), o1 = bf16_bits(2.0f * y1);
        loss = fmaf(y0, y0, loss);
        loss = fmaf(y1, y1, loss);
        rs[2 * e] += bf16_float(o0);
        rs[2 * e + 1] += bf16_float(o1);
        ov[e] = (uint32_t)o0 | ((uint32_t)o1 << 16);
      }
      *reinterpret_cast<u32x4*>(c + at) = ov;
    } else if constexpr (EPI == kGeluBackward) {
      const u32x4 z = zv[t];
      u32x4 ov;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint16_t o0 = bf16_bits(half_of(v[e], 0) * gelu_grad(half_of(z[e], 0)));
        const uint16_t o1 = bf16_bits(half_of(v[e], 1) * gelu_grad(half_of(z[e], 1)));
        rs[2 * e] += bf16_float(o0);
        rs[2 * e + 1] += bf16_float(o1);
        ov[e] = (uint32_t)o0 | ((uint32_t)o1 << 16);
      }
      *reinterpret_cast<u32x4*>(c + at) = ov;
    }
  }
  if constexpr (kSums) {
    // The four column groups of lanes (lane / 16) in order: 0 + 1, then + (2 + 3).
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      rs[e] += __shfl_xor(rs[e], 16, 64);
      rs[e] += __shfl_xor(rs[e], 32, 64);
    }
    if (cg == 0) {
      float* part = p.partial + (int64_t)(tn * 2 + wn) * p.m + mw + mc;
      *reinterpret_cast<f32x4*>(part) = f32x4{rs[0], rs[1], rs[2], rs[3]};
      *reinterpret_cast<f32x4*>(part + 4) = f32x4{rs[4], rs[5], rs[6], rs[7]};
    }
  }
  if constexpr (EPI == kSquareLoss) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) loss += __shfl_xor(loss, o, 64);
    if (lane == 0) p.partial[(int64_t)(2 * p.tiles_n) * p.m + blockIdx.x * 4 + wave] = loss;
  }
}

// ---- the tile order ----------------------------------------------------------

__device__ __forceinline__ void tile_of(int block, int tiles_m, int tiles_n, int* tm, int* tn) {
  const int total = tiles_m * tiles_n;
  int t = block;
  if (total % 8 == 0) t = (block % 8) * (total / 8) + block / 8;  // XCD-contiguous ranges
  const int group = 8;
  const int per_group = group * tiles_n;
  const int g = t / per_group;
  const int first = g * group;
  const int rows = min(tiles_m - first, group);
  const int in = t % per_group;
  *tm = first + in % rows;
  *tn = in / rows;
}

// ---- the kernel --------------------------------------------------------------

template <int LA, int LB, int EPI, bool CHECK>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(1, 1))) void gemm_bf16(
    GemmArgs p) {
  extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
  uint16_t* As = lds;
  uint16_t* Bs = lds + 2 * kStage;
  if (gridDim.y > 1 || gridDim.z > 1) {
    const int64_t z = blockIdx.z, k0 = (int64_t)blockIdx.y * p.ksplit;
    p.a += z * p.a_batch + k0 * p.a_k;
    p.b += z * p.b_batch + k0 * p.b_k;
    const int64_t at = z * p.c_batch + (int64_t)blockIdx.y * p.c_split;
    if constexpr (EPI == kStoreF32) p.c = static_cast<float*>(p.c) + at;
    else p.c = static_cast<uint16_t*>(p.c) + at;
    p.k = (int32_t)min((int64_t)p.ksplit, (int64_t)p.k - k0);
  }
  int tm, tn;
  tile_of(blockIdx.x, p.tiles_m, p.tiles_n, &tm, &tn);
  int m0 = tm * kTile, n0 = tn * kTile;
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int wm = wave / 2, wn = wave % 2;
  int lr = lane % 32, lh = lane / 32;

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};

  // Two register sets keep two K tiles in flight: while the waves multiply
  // tile kt out of one LDS stage, tile kt+1 (loaded during the step before)
  // lands in the other stage and tile kt+2's loads are issued.
  const int KT = (p.k + kDepth - 1) / kDepth;
  if constexpr (!CHECK) {
    sweep_direct<LA, LB>(p, m0, n0, wm, wn, acc);
  } else {
  Sweep<LA> sa;
  Sweep<LB> sb;
  if (!CHECK) {
    sa.init(p.a, p.a_o, p.a_k, m0);
    sb.init(p.b, p.b_o, p.b_k, n0);
  }
  u32x4 ra0[8], rb0[8], ra1[8], rb1[8];
#define TH_FETCH(kt, ra, rb)                                                    \
  do {                                                                          \
    if (CHECK) {                                                                \
      load_tile<LA, true>(p.a, p.a_o, p.a_k, m0, (kt) * kDepth, p.m, p.k, ra); \
      load_tile<LB, true>(p.b, p.b_o, p.b_k, n0, (kt) * kDepth, p.n, p.k, rb); \
    } else {                                                                    \
      sa.load(kt, ra);                                                          \
      sb.load(kt, rb);                                                          \
    }                                                                           \
  } while (0)

  TH_FETCH(0, ra0, rb0);
  store_tile<LA>(As, ra0);
  store_tile<LB>(Bs, rb0);
  if (KT > 1) TH_FETCH(1, ra1, rb1);
  __syncthreads();
  int kt = 0;
  for (; kt + 1 < KT; kt += 2) {
    // Stage 0 holds tile kt; set 1 brings tile kt+1, set 0 is free.
    if (kt + 2 < KT) TH_FETCH(kt + 2, ra0, rb0);
    multiply_tile<LA, LB>(As, Bs, As + kStage, Bs + kStage, true, ra1, rb1, acc, wm, wn, lr, lh);
    __syncthreads();
    // Stage 1 holds tile kt+1; set 0 brings tile kt+2, set 1 is free.
    if (kt + 3 < KT) TH_FETCH(kt + 3, ra1, rb1);
    multiply_tile<LA, LB>(As + kStage, Bs + kStage, As, Bs, kt + 2 < KT, ra0, rb0, acc, wm, wn, lr, lh);
    __syncthreads();
  }
  if (kt < KT) multiply_tile<LA, LB>(As, Bs, As + kStage, Bs + kStage, false, ra1, rb1, acc, wm, wn, lr, lh);
#undef TH_FETCH
  }

  if constexpr (!CHECK && EPI != kStoreF32) {
    epilogue_lds<EPI>(p, acc);
    return;
  }
  // ---- epilogue: lane holds C(m, n) for n = n_j + lane % 32 and
  // m = m_i + 8 g + 4 (lane / 32) + (0..3), register 4 g + (0..3).
  // The epilogue's indices are derived from opaque copies made here, so that
  // none of its address arithmetic is hoisted above the main loop, where
  // every register is taken.
  {
    int lane_e = lane, m0_e = m0, n0_e = n0;
    asm volatile("" : "+v"(lane_e));
    asm volatile("" : "+s"(m0_e), "+s"(n0_e));
    lr = lane_e % 32, lh = lane_e / 32;
    m0 = m0_e, n0 = n0_e;
  }
  constexpr bool kSums = EPI == kSquareLoss || EPI == kGeluBackward;
  float loss = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int mi = m0 + wm * 128 + i * 32 + 4 * lh;
    float rs[4][4];  // [g][r]: this lane's share of the row sums of block row i
    float bias[4][4];
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int r = 0; r < 4; ++r) rs[g][r] = 0.0f, bias[g][r] = 0.0f;
    if (EPI == kGelu || EPI == kSquareLoss || EPI == kStore) {
      if (EPI != kStore || p.bias) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int m = mi + 8 * g;
          if (!CHECK || m < p.m) {
            const u32x2 bb = *reinterpret_cast<const u32x2*>(p.bias + m);
#pragma unroll
            for (int r = 0; r < 4; ++r) bias[g][r] = half_of(bb[r / 2], r % 2);
          }
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + wn * 128 + j * 32 + lr;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int m = mi + 8 * g;
        const bool live = !CHECK || (m < p.m && n < p.n);
        const int64_t at = (int64_t)m + (int64_t)n * p.ldc;
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = acc[i][j][4 * g + r] + bias[g][r];
        if constexpr (EPI == kStoreF32) {
          if (live) *reinterpret_cast<f32x4*>(static_cast<float*>(p.c) + at) = f32x4{v[0], v[1], v[2], v[3]};
          continue;
        }
        uint16_t out[4];
        if constexpr (EPI == kGelu) {
          uint16_t h[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            out[r] = bf16_bits(v[r]);
            h[r] = bf16_bits(gelu(bf16_float(out[r])));
          }
          if (live) *reinterpret_cast<u32x2*>(p.aux_out + at) = pack4(h);
        } else if constexpr (EPI == kSquareLoss) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float y = bf16_float(bf16_bits(v[r]));
            out[r] = bf16_bits(2.0f * y);
            if (live) {
              loss = fmaf(y, y, loss);
              rs[g][r] += bf16_float(out[r]);
            }
          }
        } else if constexpr (EPI == kGeluBackward) {
          u32x2 zz = u32x2{0, 0};
          if (live) zz = *reinterpret_cast<const u32x2*>(p.aux + (int64_t)m + (int64_t)n * p.aux_ld);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float dh = bf16_float(bf16_bits(v[r]));
            out[r] = bf16_bits(dh * gelu_grad(half_of(zz[r / 2], r % 2)));
            if (live) rs[g][r] += bf16_float(out[r]);
          }
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r) out[r] = bf16_bits(v[r]);
        }
        if (live) *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(p.c) + at) = pack4(out);
      }
    }
    if constexpr (kSums) {
      // Row sums over the wave's 128 columns: the 32 lanes of a half share rows.
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float s = rs[g][r];
#pragma unroll
          for (int o = 1; o < 32; o <<= 1) s += __shfl_xor(s, o, 64);
          rs[g][r] = s;
        }
      if (lr == 0) {
        float* part = p.partial + (int64_t)(tn * 2 + wn) * p.m;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int m = mi + 8 * g;
          if (!CHECK || m < p.m) *reinterpret_cast<f32x4*>(part + m) = f32x4{rs[g][0], rs[g][1], rs[g][2], rs[g][3]};
        }
      }
    }
  }
  if constexpr (EPI == kSquareLoss) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) loss += __shfl_xor(loss, o, 64);
    if (lane == 0) p.partial[(int64_t)(2 * p.tiles_n) * p.m + blockIdx.x * 4 + wave] = loss;
  }
}

template <int LA, int LB, int EPI>
const void* kernel_for(bool check) {
  return check ? (const void*)gemm_bf16<LA, LB, EPI, true> : (const void*)gemm_bf16<LA, LB, EPI, false>;
}

template <int EPI>
const void* kernel_for(int la, int lb, bool check) {
  if (la == kK && lb == kK) return kernel_for<kK, kK, EPI>(check);
  if (la == kK && lb == kMN) return kernel_for<kK, kMN, EPI>(check);
  if (la == kMN && lb == kK) return kernel_for<kMN, kK, EPI>(check);
  return kernel_for<kMN, kMN, EPI>(check);
}

// One per epilogue, each defined in its own translation unit.
const void* gemm_store(int la, int lb, bool check);
const void* gemm_store_f32(int la, int lb, bool check);
const void* gemm_gelu(int la, int lb, bool check);
const void* gemm_square_loss(int la, int lb, bool check);
const void* gemm_gelu_backward(int la, int lb, bool check);

}  // namespace thg
