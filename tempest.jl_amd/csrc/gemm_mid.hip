// Op class (b), the product's middle tiles: C tiles of 128 x 128, 128 x 64,
// 64 x 128 and 64 x 64 on the half-precision matrix cores
// (v_mfma_f32_32x32x16_bf16 / _f16), the output tiles the reference's
// product sketch searches for half factors (ext/cuTileExt/contract.jl:36-39),
// for products whose 256 x 256 tiles would leave most of the device idle.
// Factors bf16 or fp16, each operand with a unit stride along k or along its
// rows, any m, n, k (bounds checked on every load and store), the other
// strides multiples of 8 and operands 16-byte aligned; K may be split over
// parts summed by the builder's second launch.
//
// A workgroup of four waves takes one tile, each wave a quarter as 32 x 32
// blocks; K advances 32 at a time through two LDS stages, the next step's
// 16-byte chunks loaded into registers while the current stage is
// multiplied.  A k-contiguous operand sits in LDS as rows of 32 k plus 8 of
// padding (80 bytes: the 16-byte fragment reads of 16 consecutive rows fall
// on 16 distinct bank quads) and is read a row per lane; an mn-contiguous one
// as rows of one k, R + 32 elements long (the 32 lanes of a transposed read
// cover 64 distinct banks), read with ds_read_b64_tr_b16 in natural k order.
#include <hip/hip_runtime.h>

#include "gemm_mid.h"
#include "th_core.h"

namespace thg {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

constexpr int kKd = 32;     // K per step
constexpr int kRowK = 40;   // k-contiguous operand: LDS row of 32 k + 8
constexpr int kPadMN = 32;  // mn-contiguous operand: LDS row of R + 32

// The n < 8 leading elements at p, the rest zero.
__device__ __forceinline__ u32x4 partial(const uint16_t* p, int n) {
  uint32_t e[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) e[i] = i < n ? p[i] : 0u;
  return u32x4{e[0] | (e[1] << 16), e[2] | (e[3] << 16), e[4] | (e[5] << 16), e[6] | (e[7] << 16)};
}

// One operand of R rows (m of A, n of B): element (row, k) at
// base[row * s + k] (KC) or base[row + k * s].
template <int R, bool KC>
struct Op {
  static constexpr int kChunks = R / 64;  // 16-byte chunks a thread moves per step
  static constexpr int kLine = KC ? kRowK : R + kPadMN;
  static constexpr int kElems = KC ? R * kRowK : kKd * (R + kPadMN);  // one stage

  // Chunk i of this thread: KC, row q / 4 at k 8 (q % 4); otherwise k q / (R / 8)
  // at rows 8 (q % (R / 8)) (lanes along the rows: whole lines).
  __device__ static void load(const uint16_t* base, int64_t s, int row0, int rows, int k0, int kend,
                              u32x4 (&r)[kChunks]) {
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
      const int q = (int)threadIdx.x + 256 * i;
      u32x4 v = {0u, 0u, 0u, 0u};
      if constexpr (KC) {
        const int row = row0 + q / 4, k = k0 + 8 * (q % 4);
        if (row < rows && k < kend) {
          const uint16_t* at = base + (int64_t)row * s + k;
          v = k + 8 <= kend ? *reinterpret_cast<const u32x4*>(at) : partial(at, kend - k);
        }
      } else {
        const int k = k0 + q / (R / 8), row = row0 + 8 * (q % (R / 8));
        if (k < kend && row < rows) {
          const uint16_t* at = base + row + (int64_t)k * s;
          v = row + 8 <= rows ? *reinterpret_cast<const u32x4*>(at) : partial(at, rows - row);
        }
      }
      r[i] = v;
    }
  }

  __device__ static void store(uint16_t* lds, const u32x4 (&r)[kChunks]) {
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
      const int q = (int)threadIdx.x + 256 * i;
      if constexpr (KC)
        *reinterpret_cast<u32x4*>(lds + (q / 4) * kRowK + 8 * (q % 4)) = r[i];
      else
        *reinterpret_cast<u32x4*>(lds + (q / (R / 8)) * kLine + 8 * (q % (R / 8))) = r[i];
    }
  }

  // The fragment of rows r0 + lane % 32, k = 16 ks + 8 (lane / 32) + (0..7).
  __device__ static s16x8 frag(const uint16_t* lds, int r0, int ks) {
    const int lane = threadIdx.x % 64;
    if constexpr (KC) {
      return *reinterpret_cast<const s16x8*>(lds + (r0 + lane % 32) * kRowK + 16 * ks + 8 * (lane / 32));
    } else {
      // ds_read_b64_tr_b16 hands lane i of each 16 element i % 4 of the
      // 8-byte pieces addressed by lanes 4 q + i / 4 (q = 0..3).  Lane j
      // addresses k row 16 ks + 8 (lane / 32) + j / 4 (+ 4 for the upper
      // half), rows r0 + 16 ((lane / 16) % 2) + 4 (j % 4) + (0..3), so lane i
      // receives k rows base + (0..3) of row r0 + 16 ((lane / 16) % 2) + i.
      const int j = lane % 16;
      const int k = 16 * ks + 8 * (lane / 32) + j / 4;
      const int row = r0 + 16 * ((lane / 16) % 2) + 4 * (j % 4);
      const uint16_t* at = lds + k * kLine + row;
      const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)at);
      const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(at + 4 * kLine));
      return s16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
  }
};

template <bool F16>
__device__ __forceinline__ f32x16 mfma(s16x8 a, s16x8 b, f32x16 c) {
  if constexpr (F16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                   0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                    0, 0, 0);
}

__device__ __forceinline__ float widen(const void* p, int64_t i, int type) {
  if (type == TH_F32) return static_cast<const float*>(p)[i];
  const uint16_t h = static_cast<const uint16_t*>(p)[i];
  if (type == TH_BF16) return __uint_as_float((uint32_t)h << 16);
  return (float)__builtin_bit_cast(_Float16, h);
}

__device__ __forceinline__ void narrow(void* p, int64_t i, int type, float x) {
  if (type == TH_F32)
    static_cast<float*>(p)[i] = x;
  else if (type == TH_BF16)
    static_cast<uint16_t*>(p)[i] = __builtin_bit_cast(uint16_t, (__bf16)x);
  else
    static_cast<uint16_t*>(p)[i] = __builtin_bit_cast(uint16_t, (_Float16)x);
}

template <int BM, int BN, bool F16, bool AKC, bool BKC>
__global__ __launch_bounds__(256, 2) void gemm_mid(MidArgs p) {
  extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
  using OA = Op<BM, AKC>;
  using OB = Op<BN, BKC>;
  constexpr int BI = BM / 64, BJ = BN / 64;  // 32 x 32 blocks a wave
  auto As = [&](int s) { return lds + s * OA::kElems; };
  auto Bs = [&](int s) { return lds + 2 * OA::kElems + s * OB::kElems; };
  const int tm = (int)(blockIdx.x % (unsigned)p.tiles_m), tn = (int)(blockIdx.x / (unsigned)p.tiles_m);
  const int64_t z = blockIdx.z, part = blockIdx.y;
  const int kbeg = (int)part * p.ksplit, kend = min(p.k, kbeg + p.ksplit);
  const uint16_t* a = p.a + z * p.a_batch;
  const uint16_t* b = p.b + z * p.b_batch;
  const int64_t sa = AKC ? p.a_m : p.a_k, sb = BKC ? p.b_n : p.b_k;
  const int m0 = tm * BM, n0 = tn * BN;
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int wm = wave / 2, wn = wave % 2;
  f32x16 acc[BI][BJ];
#pragma unroll
  for (int i = 0; i < BI; ++i)
#pragma unroll
    for (int j = 0; j < BJ; ++j) acc[i][j] = f32x16{};
  u32x4 ra[OA::kChunks], rb[OB::kChunks];
  const int steps = (kend - kbeg + kKd - 1) / kKd;
  OA::load(a, sa, m0, p.m, kbeg, kend, ra);
  OB::load(b, sb, n0, p.n, kbeg, kend, rb);
  OA::store(As(0), ra);
  OB::store(Bs(0), rb);
  __syncthreads();
  for (int st = 0; st < steps; ++st) {
    const int cur = st & 1;
    if (st + 1 < steps) {
      OA::load(a, sa, m0, p.m, kbeg + (st + 1) * kKd, kend, ra);
      OB::load(b, sb, n0, p.n, kbeg + (st + 1) * kKd, kend, rb);
    }
#pragma unroll
    for (int ks = 0; ks < kKd / 16; ++ks) {
      s16x8 fa[BI], fb[BJ];
#pragma unroll
      for (int i = 0; i < BI; ++i) fa[i] = OA::frag(As(cur), wm * (BM / 2) + 32 * i, ks);
#pragma unroll
      for (int j = 0; j < BJ; ++j) fb[j] = OB::frag(Bs(cur), wn * (BN / 2) + 32 * j, ks);
#pragma unroll
      for (int i = 0; i < BI; ++i)
#pragma unroll
        for (int j = 0; j < BJ; ++j) acc[i][j] = mfma<F16>(fa[i], fb[j], acc[i][j]);
    }
    if (st + 1 < steps) {
      OA::store(As(cur ^ 1), ra);
      OB::store(Bs(cur ^ 1), rb);
    }
    __syncthreads();
  }
  // Lane holds C(m, n) for n = the block's first column + lane % 32 and
  // m = its first row + 8 g + 4 (lane / 32) + (0..3), register 4 g + (0..3).
  const int rt = p.result;
  char* c = static_cast<char*>(p.c) + (z * p.c_batch + part * p.c_split) * (rt == TH_F32 ? 4 : 2);
  const char* d = p.d ? static_cast<const char*>(p.d) + z * p.d_batch * (rt == TH_F32 ? 4 : 2) : nullptr;
#pragma unroll
  for (int i = 0; i < BI; ++i)
#pragma unroll
    for (int j = 0; j < BJ; ++j) {
      const int n = n0 + wn * (BN / 2) + 32 * j + lane % 32;
      if (n >= p.n) continue;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int m = m0 + wm * (BM / 2) + 32 * i + 8 * (e / 4) + 4 * (lane / 32) + e % 4;
        if (m < p.m) {
          float v = acc[i][j][e];
          if (p.bias) v += __uint_as_float((uint32_t)p.bias[m] << 16);
          if (d) v += widen(d, (int64_t)m + (int64_t)n * p.d_ld, rt);
          narrow(c, (int64_t)m + (int64_t)n * p.c_ld, rt, v);
        }
      }
    }
}

template <int BM, int BN>
const void* for_tile(bool f16, bool a_kc, bool b_kc) {
#define TH_MID(F, A, B) (const void*)gemm_mid<BM, BN, F, A, B>
  if (f16) {
    if (a_kc) return b_kc ? TH_MID(true, true, true) : TH_MID(true, true, false);
    return b_kc ? TH_MID(true, false, true) : TH_MID(true, false, false);
  }
  if (a_kc) return b_kc ? TH_MID(false, true, true) : TH_MID(false, true, false);
  return b_kc ? TH_MID(false, false, true) : TH_MID(false, false, false);
#undef TH_MID
}

template <int BM, int BN>
int stage_bytes(bool a_kc, bool b_kc) {
  const int ea = a_kc ? BM * kRowK : kKd * (BM + kPadMN);
  const int eb = b_kc ? BN * kRowK : kKd * (BN + kPadMN);
  return 2 * (ea + eb) * (int)sizeof(uint16_t);
}

}  // namespace

const void* mid_kernel(int tile, bool f16, bool a_kc, bool b_kc, int* bm, int* bn, int* lds) {
  switch (tile) {
    case TH_TILE_128X128:
      *bm = 128, *bn = 128, *lds = stage_bytes<128, 128>(a_kc, b_kc);
      return for_tile<128, 128>(f16, a_kc, b_kc);
    case TH_TILE_128X64:
      *bm = 128, *bn = 64, *lds = stage_bytes<128, 64>(a_kc, b_kc);
      return for_tile<128, 64>(f16, a_kc, b_kc);
    case TH_TILE_64X128:
      *bm = 64, *bn = 128, *lds = stage_bytes<64, 128>(a_kc, b_kc);
      return for_tile<64, 128>(f16, a_kc, b_kc);
    case TH_TILE_64X64:
      *bm = 64, *bn = 64, *lds = stage_bytes<64, 64>(a_kc, b_kc);
      return for_tile<64, 64>(f16, a_kc, b_kc);
    default:
      return nullptr;
  }
}

}  // namespace thg
