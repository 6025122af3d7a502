// th_build_gemm: a product's launch on the kernel its tile names (the
// 256 x 256 kernel in gemm_kernel.h, the middle tiles in gemm_mid.hip, the
// general kernel in gemm_general.hip), the parts of K summed, and the folds
// the epilogues leave: bias gradients and the loss.  th_gemm_tune measures
// the choices.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <map>
#include <mutex>
#include <string>

#include "gemm_kernel.h"
#include "gemm_mid.h"
#include "th_core.h"

namespace thg {
namespace {

struct RowSumArgs {
  const float* partial;  // parts x m
  uint16_t* out;         // m, bf16
  int32_t m, parts;
};

// out[i] = sum over parts of partial[p, i], in part order.
__global__ __launch_bounds__(256) void sum_parts(RowSumArgs a) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= a.m) return;
  a.out[i] = bf16_bits(thd::sum_in_order(a.partial + i, a.m, a.parts));
}

struct LossArgs {
  const float* partial;
  float* loss;
  int32_t count;
};

__global__ __launch_bounds__(256) void sum_loss(LossArgs a) {
  __shared__ double lds[4];
  double s = 0.0;
  for (int i = threadIdx.x; i < a.count; i += 256) s += (double)a.partial[i];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
  if (threadIdx.x % 64 == 0) lds[threadIdx.x / 64] = s;
  __syncthreads();
  if (threadIdx.x == 0) a.loss[0] = (float)(lds[0] + lds[1] + lds[2] + lds[3]);
}

// The parts of K summed (in part order), plus the bias and what the product
// is added to, rounded once to the result's type (fp32, bf16 or fp16):
// C_z = D_z + sum_s W_zs + bias.
struct ReduceArgs {
  const float* ws;       // [batch][splits][m x n], column-major at ld m
  void* c;               // result, column-major at c_ld, product z at c_batch
  const uint16_t* bias;  // bf16, m, or null
  const void* d;         // or null: laid out as C at d_ld, d_batch
  int64_t c_ld, c_batch, d_ld, d_batch;
  int32_t m, n, splits, c_dtype;
};

__global__ __launch_bounds__(256) void sum_splits(ReduceArgs a) {
  const int64_t mn = (int64_t)a.m * a.n;
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= mn) return;
  const int64_t z = blockIdx.y;
  const int64_t i = e % a.m, j = e / a.m;
  float v = thd::sum_in_order(a.ws + z * a.splits * mn + e, mn, a.splits);
  if (a.bias) v += bf16_float(a.bias[i]);
  const int64_t at_d = z * a.d_batch + i + j * a.d_ld, at = z * a.c_batch + i + j * a.c_ld;
  if (a.c_dtype == TH_F32) {
    if (a.d) v += static_cast<const float*>(a.d)[at_d];
    static_cast<float*>(a.c)[at] = v;
  } else if (a.c_dtype == TH_F16) {
    if (a.d) v += (float)__builtin_bit_cast(_Float16, static_cast<const uint16_t*>(a.d)[at_d]);
    static_cast<uint16_t*>(a.c)[at] = __builtin_bit_cast(uint16_t, (_Float16)v);
  } else {
    if (a.d) v += bf16_float(static_cast<const uint16_t*>(a.d)[at_d]);
    static_cast<uint16_t*>(a.c)[at] = bf16_bits(v);
  }
}

bool aligned(const void* p, int bytes) { return (reinterpret_cast<uintptr_t>(p) % bytes) == 0; }

// An fp32 factor as three bf16 copies along K, for the bf16x3 products:
// x = hi + lo + (below lo), hi = bf16(x), lo = bf16(x - hi); A's copies are
// (hi, hi, lo) and B's (hi, lo, hi), so that the product of the two tripled
// operands is A_hi B_hi + A_hi B_lo + A_lo B_hi.  Each copy is k8 deep (k
// rounded up to 8, zeros past k); rows past `rows` (up to the destination's
// padded count) are zeros.
struct SplitArgs {
  const float* src;
  uint16_t* dst;
  int64_t s_r, s_k, s_batch;  // source strides along the rows (m or n), along k, between products
  int64_t d_r, d_k, d_batch;  // destination strides
  int64_t total;              // destination elements of one copy of one product: rows_pad x k8
  int32_t rows, rows_pad, k, k8;
  int32_t order;   // 0: (hi, hi, lo), 1: (hi, lo, hi)
  int32_t k_fast;  // 1: k is the destination's contiguous axis
};

__global__ __launch_bounds__(256) void split_bf16x3(SplitArgs a) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= a.total) return;
  const int64_t z = blockIdx.y;
  int64_t r, l;
  if (a.k_fast) r = e / a.k8, l = e % a.k8;
  else r = e % a.rows_pad, l = e / a.rows_pad;
  const float x = (r < a.rows && l < a.k) ? a.src[z * a.s_batch + r * a.s_r + l * a.s_k] : 0.0f;
  const uint16_t hi = bf16_bits(x);
  const uint16_t lo = bf16_bits(x - bf16_float(hi));
  uint16_t* d = a.dst + z * a.d_batch + r * a.d_r + l * a.d_k;
  const int64_t step = (int64_t)a.k8 * a.d_k;
  d[0] = hi;
  d[step] = a.order == 0 ? hi : lo;
  d[2 * step] = a.order == 0 ? lo : hi;
}

}  // namespace
}  // namespace thg

using namespace thg;

// Whether the bf16 tile kernel takes the descriptor: bf16 factors, a unit
// stride on each operand, sizes and strides multiples of 8, 16-byte operands.
bool tile_kernel_takes(const th_gemm_desc* d) {
  if (d->flags & (TH_GEMM_F32_FACTORS | TH_GEMM_F16_FACTORS)) return false;
  if (d->c_dtype != TH_BF16 && d->c_dtype != TH_F32) return false;
  if (d->m % 8 || d->n % 8 || d->k % 8) return false;
  const bool ua = d->a_k == 1 || d->a_m == 1, ub = d->b_k == 1 || d->b_n == 1;
  if (!ua || !ub) return false;
  const int64_t sa = d->a_k == 1 ? d->a_m : d->a_k, sb = d->b_k == 1 ? d->b_n : d->b_k;
  if (sa % 8 || sb % 8 || d->c_ld % 8 || d->c_ld < d->m) return false;
  if (d->batch > 1 && (d->a_batch % 8 || d->b_batch % 8 || d->c_batch % 8)) return false;
  return aligned(d->a, 16) && aligned(d->b, 16) && aligned(d->c, 16);
}

// Whether the middle tiles take the descriptor: half factors, a unit stride
// on each operand, the other strides multiples of 8, 16-byte operands, a
// plain product with a result of the factors' type or fp32.
static bool mid_takes(const th_gemm_desc* d) {
  if (d->flags & TH_GEMM_F32_FACTORS) return false;
  if (d->epilogue != TH_EPI_STORE) return false;
  const int factor = (d->flags & TH_GEMM_F16_FACTORS) ? TH_F16 : TH_BF16;
  if (d->c_dtype != factor && d->c_dtype != TH_F32) return false;
  if (!(d->a_k == 1 || d->a_m == 1) || !(d->b_k == 1 || d->b_n == 1)) return false;
  const int64_t sa = d->a_k == 1 ? d->a_m : d->a_k, sb = d->b_k == 1 ? d->b_n : d->b_k;
  if (sa % 8 || sb % 8 || d->c_ld < d->m) return false;
  if (d->batch > 1 && (d->a_batch % 8 || d->b_batch % 8)) return false;
  return aligned(d->a, 16) && aligned(d->b, 16);
}

static int mid_rows(int tile) { return tile == TH_TILE_64X128 || tile == TH_TILE_64X64 ? 64 : 128; }
static int mid_cols(int tile) { return tile == TH_TILE_128X64 || tile == TH_TILE_64X64 ? 64 : 128; }

static int64_t tiles_of(const th_gemm_desc* d, int bm, int bn) {
  return (int64_t)((d->m + bm - 1) / bm) * ((d->n + bn - 1) / bn) * std::max(1, d->batch);
}

// The parts of K a tile takes when the caller leaves them to the builder:
// enough for about 256 workgroups where the tiles alone give fewer than 128,
// each part at least `least` deep (1024 on the 256 x 256 kernel, 512 on the
// middle tiles).
static int auto_splits(const th_gemm_desc* d, int tile) {
  if (d->epilogue != TH_EPI_STORE) return 1;
  if (tile == TH_TILE_GENERAL) {
    // fp32 factors on 128 x 128 tiles split as the others; half factors do not.
    if (!(d->flags & TH_GEMM_F32_FACTORS) || d->c_dtype != TH_F32 || d->bias) return 1;
    const int64_t tiles = tiles_of(d, 128, 128);
    if (tiles >= 128 || d->k < 64) return 1;
    return (int)std::max<int64_t>(1, std::min<int64_t>((256 + tiles - 1) / tiles, d->k / 32));
  }
  const bool big = tile == TH_TILE_256;
  const int64_t tiles = big ? tiles_of(d, kTile, kTile) : tiles_of(d, mid_rows(tile), mid_cols(tile));
  const int least = big ? 1024 : 512;
  if (tiles >= 128 || d->k < 2 * least) return 1;
  return (int)std::max<int64_t>(1, std::min<int64_t>((256 + tiles - 1) / tiles, d->k / least));
}

// TH_TILE_AUTO: the 256 x 256 kernel where it takes the product and fills
// the device (split or not) or nothing else takes it, else the largest middle
// tile that gives 256 workgroups (the smallest if none does), else the
// general kernel.
static int choose_tile(const th_gemm_desc* d) {
  const bool mid = mid_takes(d);
  if (tile_kernel_takes(d) &&
      (!mid || tiles_of(d, kTile, kTile) * auto_splits(d, TH_TILE_256) >= 128))
    return TH_TILE_256;
  if (mid) {
    for (int t : {TH_TILE_128X128, TH_TILE_128X64, TH_TILE_64X128})
      if (tiles_of(d, mid_rows(t), mid_cols(t)) >= 256) return t;
    return TH_TILE_64X64;
  }
  return TH_TILE_GENERAL;
}

static int build_tile256(const th_gemm_desc* d, th_launch** out);
static int build_mid(const th_gemm_desc* d, int tile, th_launch** out);
static int build_bf16x3(const th_gemm_desc* d, th_launch** out);

extern "C" int th_build_gemm(const th_gemm_desc* d, th_launch** out) {
  if (int r = th::require_ready()) return r;
  *out = nullptr;
  TH_REQUIRE(d != nullptr, "th_build_gemm: null descriptor");
  TH_REQUIRE(d->m >= 1 && d->n >= 1 && d->k >= 1, "th_build_gemm: m, n, k must be positive");
  TH_REQUIRE(d->a && d->b && d->c, "th_build_gemm: null operand");
  TH_REQUIRE((d->flags & ~(TH_GEMM_F32_FACTORS | TH_GEMM_F16_FACTORS | TH_GEMM_ACCUMULATE | TH_GEMM_BF16X3)) == 0 &&
                 (d->flags & (TH_GEMM_F32_FACTORS | TH_GEMM_F16_FACTORS)) != (TH_GEMM_F32_FACTORS | TH_GEMM_F16_FACTORS),
             "th_build_gemm: unknown flags");
  const bool accumulate = (d->flags & TH_GEMM_ACCUMULATE) != 0;
  TH_REQUIRE(!accumulate || d->d, "th_build_gemm: accumulating needs d");
  const int epi = d->epilogue;
  TH_REQUIRE(epi >= TH_EPI_STORE && epi <= TH_EPI_GELU_BACKWARD, "th_build_gemm: unknown epilogue");
  TH_REQUIRE(epi == TH_EPI_STORE || ((d->batch <= 1) && !accumulate),
             "th_build_gemm: fused epilogues take one product and nothing to add");
  TH_REQUIRE(d->tile >= TH_TILE_AUTO && d->tile <= TH_TILE_GENERAL, "th_build_gemm: unknown tile");
  TH_REQUIRE(d->splits >= 0, "th_build_gemm: splits must be >= 0");
  if (d->flags & TH_GEMM_BF16X3) return build_bf16x3(d, out);
  const int tile = d->tile == TH_TILE_AUTO ? choose_tile(d) : d->tile;
  if (tile == TH_TILE_GENERAL) return th::build_gemm_general(d, out);
  if (tile == TH_TILE_256) {
    TH_REQUIRE(tile_kernel_takes(d),
               "th_build_gemm: the 256 x 256 kernel takes bf16 factors with a unit stride on each operand, m, n, k "
               "and the other strides multiples of 8 and 16-byte aligned operands");
    return build_tile256(d, out);
  }
  TH_REQUIRE(mid_takes(d),
             "th_build_gemm: the middle tiles take bf16 or fp16 factors with a unit stride on each operand, the other "
             "strides multiples of 8, 16-byte aligned operands, TH_EPI_STORE and a result of the factors' type or fp32");
  return build_mid(d, tile, out);
}

static int build_tile256(const th_gemm_desc* d, th_launch** out) {
  const int M = d->m, N = d->n, K = d->k;
  const int batch = d->batch > 0 ? d->batch : 1;
  const bool accumulate = (d->flags & TH_GEMM_ACCUMULATE) != 0;
  const int epi = d->epilogue;
  const int la = d->a_k == 1 ? kK : kMN;
  const int lb = d->b_k == 1 ? kK : kMN;
  TH_REQUIRE(d->c_dtype == TH_BF16 || (d->c_dtype == TH_F32 && epi == TH_EPI_STORE),
             "th_build_gemm: fused epilogues write bf16");
  TH_REQUIRE(!d->bias || aligned(d->bias, 8), "th_build_gemm: bias must be 8-byte aligned");
  TH_REQUIRE(!(d->c_dtype == TH_F32 && d->bias), "th_build_gemm: an fp32 result takes no bias");
  if (epi == TH_EPI_GELU)
    TH_REQUIRE(d->aux_out && d->bias && aligned(d->aux_out, 8), "th_build_gemm: GELU needs bias and aux_out");
  if (epi == TH_EPI_SQUARE_LOSS)
    TH_REQUIRE(d->bias && d->loss && d->row_sums, "th_build_gemm: the square loss needs bias, loss, row_sums");
  if (epi == TH_EPI_GELU_BACKWARD)
    TH_REQUIRE(d->aux && d->row_sums && d->aux_ld >= M && d->aux_ld % 4 == 0 && aligned(d->aux, 8),
               "th_build_gemm: the GELU backward needs aux (8-byte aligned, ld >= m, ld % 4 == 0) and row_sums");

  const int tiles_m = (M + kTile - 1) / kTile, tiles_n = (N + kTile - 1) / kTile;
  // K split over parts (each a multiple of 64 deep) where asked, or where the
  // tiles alone would leave most CUs idle.
  int splits = d->splits > 0 ? d->splits : auto_splits(d, TH_TILE_256);
  TH_REQUIRE(splits == 1 || epi == TH_EPI_STORE, "th_build_gemm: only a plain product splits K");
  int ksplit = K;
  if (splits > 1) {
    ksplit = ((K + splits - 1) / splits + kDepth - 1) / kDepth * kDepth;
    splits = (K + ksplit - 1) / ksplit;
  }
  TH_REQUIRE(splits <= 65535 && batch <= 65535, "th_build_gemm: grid too large");
  // Parts and what is added go through an fp32 workspace and a second launch.
  const bool staged = splits > 1 || accumulate;
  // Interior tiles read through 32-bit buffer offsets: operands past 2 GiB
  // take the bounds-checked kernel, which addresses with 64-bit pointers.
  const int64_t a_bytes = 2 * (la == kK ? (int64_t)(M - 1) * d->a_m + K : (int64_t)(K - 1) * d->a_k + M);
  const int64_t b_bytes = 2 * (lb == kK ? (int64_t)(N - 1) * d->b_n + K : (int64_t)(K - 1) * d->b_k + N);
  const bool check = (M % kTile) || (N % kTile) || (K % kDepth) || (ksplit % kDepth) || a_bytes > 0x7fffffff ||
                     b_bytes > 0x7fffffff;
  const void* fn = nullptr;
  const char* name = "";
  switch (epi) {
    case TH_EPI_STORE:
      fn = (staged || d->c_dtype == TH_F32) ? gemm_store_f32(la, lb, check) : gemm_store(la, lb, check);
      name = staged ? "gemm_bf16_parts_f32" : d->c_dtype == TH_F32 ? "gemm_bf16_store_f32" : "gemm_bf16_store";
      break;
    case TH_EPI_GELU: fn = gemm_gelu(la, lb, check), name = "gemm_bf16_gelu"; break;
    case TH_EPI_SQUARE_LOSS: fn = gemm_square_loss(la, lb, check), name = "gemm_bf16_square_loss"; break;
    default: fn = gemm_gelu_backward(la, lb, check), name = "gemm_bf16_gelu_backward"; break;
  }
  const size_t lds_bytes = check ? kLds : kLdsDirect;
  TH_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_bytes));

  th::Builder b("gemm_bf16", 9);
  GemmArgs g{};
  g.a = static_cast<const uint16_t*>(d->a);
  g.b = static_cast<const uint16_t*>(d->b);
  g.c = d->c;
  g.bias = staged ? nullptr : static_cast<const uint16_t*>(d->bias);
  g.aux = static_cast<const uint16_t*>(d->aux);
  g.aux_out = static_cast<uint16_t*>(d->aux_out);
  g.a_o = la == kK ? d->a_m : 1;
  g.a_k = la == kK ? 1 : d->a_k;
  g.b_o = lb == kK ? d->b_n : 1;
  g.b_k = lb == kK ? 1 : d->b_k;
  g.ldc = d->c_ld;
  g.aux_ld = d->aux_ld;
  g.m = M;
  g.n = N;
  g.k = K;
  g.tiles_m = tiles_m;
  g.tiles_n = tiles_n;
  g.a_batch = d->a_batch;
  g.b_batch = d->b_batch;
  g.c_batch = d->c_batch;
  g.c_split = 0;
  g.ksplit = ksplit;
  const int64_t mn = (int64_t)M * N;
  // Workspace: the fp32 sums of each part of K (staged products), then the
  // epilogue's per-tile row sums and loss partials.
  uint64_t at_parts = 0, at_sums = 0;
  if (staged) {
    at_parts = b.workspace((uint64_t)batch * splits * mn * sizeof(float));
    g.c = nullptr;
    g.ldc = M;
    g.c_batch = (int64_t)splits * mn;
    g.c_split = mn;
  }
  const bool sums = epi == TH_EPI_SQUARE_LOSS || epi == TH_EPI_GELU_BACKWARD;
  const int blocks = tiles_m * tiles_n;
  if (sums) at_sums = b.workspace(((uint64_t)2 * tiles_n * M + (uint64_t)4 * blocks) * sizeof(float));
  int k = b.kernel(fn, name, dim3(blocks, splits, batch), dim3(kThreads), (uint32_t)lds_bytes, g);
  if (staged) b.ws_ref(k, TH_OFFSET(GemmArgs, c), at_parts);
  if (sums) b.ws_ref(k, TH_OFFSET(GemmArgs, partial), at_sums);
  b.ref(0, k, TH_OFFSET(GemmArgs, a));
  b.ref(1, k, TH_OFFSET(GemmArgs, b));
  if (!staged) b.ref(2, k, TH_OFFSET(GemmArgs, c));
  if (!staged) b.ref(3, k, TH_OFFSET(GemmArgs, bias));
  b.ref(4, k, TH_OFFSET(GemmArgs, aux));
  b.ref(5, k, TH_OFFSET(GemmArgs, aux_out));
  for (int v : {0, 1, 2}) b.align(v, 16);
  for (int v : {3, 4, 5}) b.align(v, 8);
  if (staged) {
    ReduceArgs ra{nullptr, d->c, static_cast<const uint16_t*>(d->bias),
                  accumulate ? d->d : nullptr, d->c_ld, d->c_batch, d->d_ld ? d->d_ld : d->c_ld,
                  d->d_ld ? d->d_batch : d->c_batch, M, N, splits, d->c_dtype};
    int kr = b.kernel((const void*)sum_splits, "sum_splits", dim3((unsigned)((mn + 255) / 256), batch), dim3(256), 0,
                      ra);
    b.ref(2, kr, TH_OFFSET(ReduceArgs, c));
    b.ref(3, kr, TH_OFFSET(ReduceArgs, bias));
    b.ref(8, kr, TH_OFFSET(ReduceArgs, d));
    b.ws_ref(kr, TH_OFFSET(ReduceArgs, ws), at_parts);
  }
  if (sums) {
    RowSumArgs rs{nullptr, static_cast<uint16_t*>(d->row_sums), M, 2 * tiles_n};
    int k2 = b.kernel((const void*)sum_parts, "sum_parts", dim3((M + 255) / 256), dim3(256), 0, rs);
    b.ref(6, k2, TH_OFFSET(RowSumArgs, out));
    b.ws_ref(k2, TH_OFFSET(RowSumArgs, partial), at_sums);
  }
  if (epi == TH_EPI_SQUARE_LOSS) {
    LossArgs ls{nullptr, d->loss, 4 * blocks};
    int k3 = b.kernel((const void*)sum_loss, "sum_loss", dim3(1), dim3(256), 0, ls);
    b.ref(7, k3, TH_OFFSET(LossArgs, loss));
    b.ws_ref(k3, TH_OFFSET(LossArgs, partial), at_sums + (uint64_t)2 * tiles_n * M * sizeof(float));
  }
  const double mm = M, nn = N, kk = K, bb = batch;
  const double cbytes = d->c_dtype == TH_F32 ? 4 : 2;
  double bytes = bb * (2.0 * (mm * kk + kk * nn) + cbytes * mm * nn * (accumulate ? 2 : 1));
  if (epi == TH_EPI_GELU || epi == TH_EPI_GELU_BACKWARD) bytes += 2.0 * mm * nn;
  b.work(bytes, 2.0 * bb * mm * nn * kk, (int64_t)blocks * splits * batch);
  *out = b.release();
  return TH_OK;
}

// The middle tiles: one launch of the tile kernel, and for parts of K a
// second that sums them (with the bias and D) into the result.
static int build_mid(const th_gemm_desc* d, int tile, th_launch** out) {
  const int M = d->m, N = d->n, K = d->k;
  const int batch = d->batch > 0 ? d->batch : 1;
  const bool accumulate = (d->flags & TH_GEMM_ACCUMULATE) != 0;
  const bool f16 = (d->flags & TH_GEMM_F16_FACTORS) != 0;
  int bm = 0, bn = 0, lds = 0;
  const void* fn = mid_kernel(tile, f16, d->a_k == 1, d->b_k == 1, &bm, &bn, &lds);
  TH_REQUIRE(fn != nullptr, "th_build_gemm: unknown tile");
  const int64_t tiles_m = (M + bm - 1) / bm, tiles_n = (N + bn - 1) / bn;
  TH_REQUIRE(tiles_m * tiles_n <= 0x7fffffff, "th_build_gemm: grid too large");
  int splits = d->splits > 0 ? d->splits : auto_splits(d, tile);
  int ksplit = K;
  if (splits > 1) {
    ksplit = ((K + splits - 1) / splits + 31) / 32 * 32;
    splits = (K + ksplit - 1) / ksplit;
  }
  TH_REQUIRE(splits <= 65535 && batch <= 65535, "th_build_gemm: grid too large");
  const bool staged = splits > 1;
  const int64_t mn = (int64_t)M * N;
  th::Builder b("gemm_mid", 9);
  MidArgs g{};
  g.a = static_cast<const uint16_t*>(d->a);
  g.b = static_cast<const uint16_t*>(d->b);
  g.a_m = d->a_m, g.a_k = d->a_k, g.a_batch = d->a_batch;
  g.b_k = d->b_k, g.b_n = d->b_n, g.b_batch = d->b_batch;
  g.m = M, g.n = N, g.k = K, g.ksplit = ksplit, g.tiles_m = (int32_t)tiles_m;
  uint64_t at_parts = 0;
  if (staged) {
    // Each part's fp32 sums, [batch][part][m x n] column-major at ld m.
    at_parts = b.workspace((uint64_t)batch * splits * mn * sizeof(float));
    g.c = nullptr, g.c_ld = M, g.c_batch = (int64_t)splits * mn, g.c_split = mn, g.result = TH_F32;
  } else {
    g.c = d->c, g.c_ld = d->c_ld, g.c_batch = d->c_batch, g.c_split = 0, g.result = d->c_dtype;
    g.d = accumulate ? d->d : nullptr;
    g.d_ld = d->d_ld ? d->d_ld : d->c_ld;
    g.d_batch = d->d_ld ? d->d_batch : d->c_batch;
    g.bias = static_cast<const uint16_t*>(d->bias);
  }
  const char* name = staged ? "gemm_mid_parts_f32" : "gemm_mid";
  int k = b.kernel(fn, name, dim3((unsigned)(tiles_m * tiles_n), splits, batch), dim3(256), (uint32_t)lds, g);
  b.ref(0, k, TH_OFFSET(MidArgs, a));
  b.ref(1, k, TH_OFFSET(MidArgs, b));
  if (staged) {
    b.ws_ref(k, TH_OFFSET(MidArgs, c), at_parts);
  } else {
    b.ref(2, k, TH_OFFSET(MidArgs, c));
    b.ref(3, k, TH_OFFSET(MidArgs, bias));
    b.ref(8, k, TH_OFFSET(MidArgs, d));
  }
  b.align(0, 16);
  b.align(1, 16);
  if (staged) {
    ReduceArgs ra{nullptr, d->c, static_cast<const uint16_t*>(d->bias),
                  accumulate ? d->d : nullptr, d->c_ld, d->c_batch, d->d_ld ? d->d_ld : d->c_ld,
                  d->d_ld ? d->d_batch : d->c_batch, M, N, splits, d->c_dtype};
    int kr = b.kernel((const void*)sum_splits, "sum_splits", dim3((unsigned)((mn + 255) / 256), batch), dim3(256), 0,
                      ra);
    b.ref(2, kr, TH_OFFSET(ReduceArgs, c));
    b.ref(3, kr, TH_OFFSET(ReduceArgs, bias));
    b.ref(8, kr, TH_OFFSET(ReduceArgs, d));
    b.ws_ref(kr, TH_OFFSET(ReduceArgs, ws), at_parts);
  }
  const double mm = M, nn = N, kk = K, bb = batch;
  const double cbytes = d->c_dtype == TH_F32 ? 4 : 2;
  b.work(bb * (2.0 * (mm * kk + kk * nn) + cbytes * mm * nn * (accumulate ? 2 : 1)), 2.0 * bb * mm * nn * kk,
         tiles_m * tiles_n * splits * batch);
  *out = b.release();
  return TH_OK;
}

// fp32 factors as split bf16 on the bf16 tile kernels (TH_GEMM_BF16X3): each
// factor becomes three bf16 copies along K (split_bf16x3) in the launch's
// workspace, and one product over 3 k8 sums A_hi B_hi + A_hi B_lo + A_lo B_hi
// in fp32 — the MI355X counterpart of the reference's :tf32x3
// (src/Compiler/runtime/target.jl:42-44, ext/cuBLASExt.jl:61-65).  The
// launch is the two split kernels followed by the inner product's kernels;
// the inner product's operands point into the workspace.
static int build_bf16x3(const th_gemm_desc* d, th_launch** out) {
  TH_REQUIRE(d->flags & TH_GEMM_F32_FACTORS, "th_build_gemm: TH_GEMM_BF16X3 splits fp32 factors");
  TH_REQUIRE(d->epilogue == TH_EPI_STORE && !d->bias && d->c_dtype == TH_F32,
             "th_build_gemm: a bf16x3 product stores an fp32 result, with no epilogue or bias");
  TH_REQUIRE(d->tile == TH_TILE_AUTO || (d->tile >= TH_TILE_256 && d->tile <= TH_TILE_64X64),
             "th_build_gemm: a bf16x3 product runs on the bf16 tile kernels");
  const int batch = d->batch > 0 ? d->batch : 1;
  const int M = d->m, N = d->n, K = d->k;
  const int k8 = (K + 7) / 8 * 8, m8 = (M + 7) / 8 * 8, n8 = (N + 7) / 8 * 8;
  TH_REQUIRE((int64_t)3 * k8 <= 0x7fffffff, "th_build_gemm: K too large");
  // The tripled operands, dense, with the fp32 operand's unit-stride axis kept.
  th_gemm_desc in = *d;
  in.flags = d->flags & TH_GEMM_ACCUMULATE;
  in.k = 3 * k8;
  const bool a_kfast = d->a_k == 1 && d->a_m != 1;
  const bool b_kfast = d->b_k == 1 && d->b_n != 1;
  SplitArgs sa{}, sb{};
  sa.rows = M, sa.k = K, sa.k8 = k8, sa.order = 0, sa.k_fast = a_kfast;
  sa.s_r = d->a_m, sa.s_k = d->a_k, sa.s_batch = d->a_batch;
  if (a_kfast) sa.rows_pad = M, sa.d_r = 3 * k8, sa.d_k = 1, in.a_m = 3 * k8, in.a_k = 1;
  else sa.rows_pad = m8, sa.d_r = 1, sa.d_k = m8, in.a_m = 1, in.a_k = m8;
  sa.total = (int64_t)sa.rows_pad * k8;
  sa.d_batch = 3 * sa.total;
  sb.rows = N, sb.k = K, sb.k8 = k8, sb.order = 1, sb.k_fast = b_kfast;
  sb.s_r = d->b_n, sb.s_k = d->b_k, sb.s_batch = d->b_batch;
  if (b_kfast) sb.rows_pad = N, sb.d_r = 3 * k8, sb.d_k = 1, in.b_n = 3 * k8, in.b_k = 1;
  else sb.rows_pad = n8, sb.d_r = 1, sb.d_k = n8, in.b_n = 1, in.b_k = n8;
  sb.total = (int64_t)sb.rows_pad * k8;
  sb.d_batch = 3 * sb.total;
  in.a_batch = sa.d_batch, in.b_batch = sb.d_batch;
  // Stand-ins the inner build checks for alignment; the workspace replaces them.
  in.a = reinterpret_cast<const void*>(uintptr_t(256));
  in.b = reinterpret_cast<const void*>(uintptr_t(256));
  th_launch* inner = nullptr;
  if (int r = th_build_gemm(&in, &inner)) return r;
  const uint64_t a_bytes = (uint64_t)batch * sa.d_batch * 2, b_bytes = (uint64_t)batch * sb.d_batch * 2;
  th::Builder bl("gemm_bf16x3", 9);
  const uint64_t at_a = bl.workspace(a_bytes), at_b = bl.workspace(b_bytes);
  const uint64_t at_inner = bl.workspace(inner->ws_bytes);
  sa.src = static_cast<const float*>(d->a), sb.src = static_cast<const float*>(d->b);
  const int ka = bl.kernel((const void*)split_bf16x3, "split_bf16x3_a", dim3((unsigned)((sa.total + 255) / 256), batch),
                           dim3(256), 0, sa);
  const int kb = bl.kernel((const void*)split_bf16x3, "split_bf16x3_b", dim3((unsigned)((sb.total + 255) / 256), batch),
                           dim3(256), 0, sb);
  bl.ref(0, ka, TH_OFFSET(SplitArgs, src));
  bl.ref(1, kb, TH_OFFSET(SplitArgs, src));
  bl.ws_ref(ka, TH_OFFSET(SplitArgs, dst), at_a);
  bl.ws_ref(kb, TH_OFFSET(SplitArgs, dst), at_b);
  th_launch* l = bl.release();
  // The inner product's kernels after the splits: its operands a and b
  // become the tripled copies in the workspace, its other values ours.
  const int base = (int)l->kernels.size();
  for (const th::Kernel& k : inner->kernels) l->kernels.push_back(k);
  for (int v = 0; v < (int)inner->values.size() && v < (int)l->values.size(); ++v)
    for (const th::Ref& r : inner->values[v]) {
      if (v == 0) l->ws_refs.push_back(th::WsRef{base + r.kernel, r.offset, at_a});
      else if (v == 1) l->ws_refs.push_back(th::WsRef{base + r.kernel, r.offset, at_b});
      else l->values[v].push_back(th::Ref{base + r.kernel, r.offset});
    }
  for (const th::WsRef& w : inner->ws_refs) l->ws_refs.push_back(th::WsRef{base + w.kernel, w.offset, at_inner + w.at});
  for (int v = 2; v < (int)inner->align.size() && v < (int)l->align.size(); ++v) l->align[v] = inner->align[v];
  l->work.kernels = (int32_t)l->kernels.size();
  l->work.flops = 2.0 * batch * (double)M * N * K;
  l->work.bytes = batch * (4.0 * ((double)M * K + (double)K * N) + 4.0 * (double)M * N *
                          ((d->flags & TH_GEMM_ACCUMULATE) ? 2 : 1));
  l->work.blocks = inner->work.blocks;
  l->name = "gemm_bf16x3 (fp32 factors as hi + lo bf16, K tripled): " + inner->name;
  inner->kernels.clear();
  th_launch_destroy(inner);
  *out = l;
  return TH_OK;
}

// ---- measuring the choices -------------------------------------------------------

namespace {

struct Tuned {
  int32_t tile, splits;
  double seconds;
};

std::mutex g_tune_mutex;
std::map<std::string, Tuned> g_tuned;

std::string tune_key(const th_gemm_desc* d) {
  char buf[512];
  snprintf(buf, sizeof buf, "%d %d %d %d|%lld %lld %lld %lld %lld|%lld %lld %lld %lld %lld|%d %d %d %d %d|%d %d %d",
           d->m, d->n, d->k, std::max(1, d->batch), (long long)d->a_m, (long long)d->a_k, (long long)d->b_k,
           (long long)d->b_n, (long long)d->c_ld, (long long)d->a_batch, (long long)d->b_batch, (long long)d->c_batch,
           (long long)d->d_ld, (long long)d->d_batch, d->flags, d->c_dtype, d->epilogue, d->bias != nullptr,
           d->d != nullptr, (int)(reinterpret_cast<uintptr_t>(d->a) % 16 == 0),
           (int)(reinterpret_cast<uintptr_t>(d->b) % 16 == 0), (int)(reinterpret_cast<uintptr_t>(d->c) % 16 == 0));
  return buf;
}

// The splits a build with `splits` asked (0: the builder's choice) ends up
// with, as the builders round them.
int splits_used(const th_gemm_desc* d, int tile, int splits) {
  if (tile == TH_TILE_GENERAL) return 1;
  int s = splits > 0 ? splits : auto_splits(d, tile);
  if (s <= 1) return 1;
  const int step = tile == TH_TILE_256 ? kDepth : 32;
  const int ks = ((d->k + s - 1) / s + step - 1) / step * step;
  return (d->k + ks - 1) / ks;
}

int measure(const th_gemm_desc* base, int tile, int splits, double* seconds) {
  th_gemm_desc d = *base;
  d.tile = tile;
  d.splits = splits;
  th_launch* l = nullptr;
  if (int r = th_build_gemm(&d, &l)) return r;
  const int r = th_time_launch(l, 0, seconds);
  th_launch_destroy(l);
  return r;
}

}  // namespace

extern "C" int th_gemm_tune(const th_gemm_desc* desc, int32_t* tile_out, int32_t* splits_out, double* seconds_out) {
  if (int r = th::require_ready()) return r;
  TH_REQUIRE(desc != nullptr && tile_out && splits_out && seconds_out, "th_gemm_tune: null argument");
  TH_REQUIRE(!((desc->flags & TH_GEMM_ACCUMULATE) && desc->d == desc->c),
             "th_gemm_tune: D + A B in place would add the product again at every measurement");
  const std::string key = tune_key(desc);
  std::lock_guard<std::mutex> lock(g_tune_mutex);
  auto hit = g_tuned.find(key);
  if (hit == g_tuned.end()) {
    th_gemm_desc d = *desc;
    d.tile = TH_TILE_AUTO;
    d.splits = 0;
    std::vector<int> tiles;
    const bool x3 = (d.flags & TH_GEMM_BF16X3) != 0;
    if (x3) {
      // The bf16 tiles the tripled product may run on: those that build.
      for (int t : {TH_TILE_256, TH_TILE_128X128, TH_TILE_128X64, TH_TILE_64X128, TH_TILE_64X64}) tiles.push_back(t);
    } else {
      if (tile_kernel_takes(&d)) tiles.push_back(TH_TILE_256);
      if (mid_takes(&d))
        for (int t : {TH_TILE_128X128, TH_TILE_128X64, TH_TILE_64X128, TH_TILE_64X64}) tiles.push_back(t);
      if (d.epilogue == TH_EPI_STORE && !d.bias) tiles.push_back(TH_TILE_GENERAL);
    }
    TH_REQUIRE(!tiles.empty(), "th_gemm_tune: no kernel takes the product");
    // Stage one: every tile at the split the builder would choose.
    Tuned best{0, 0, 0.0};
    for (int t : tiles) {
      double s = 0;
      if (int r = measure(&d, t, 0, &s)) {
        if (x3) continue;  // a tile the tripled product does not fit
        return r;
      }
      if (best.tile == 0 || s < best.seconds) best = Tuned{t, splits_used(&d, t, 0), s};
    }
    TH_REQUIRE(best.tile != 0, "th_gemm_tune: no kernel takes the product");
    // Stage two: the other splits of the best (plain products on the tile
    // kernels, and fp32 ones on the general kernel), each part at least 256 deep.
    const bool general_splits = d.flags & TH_GEMM_F32_FACTORS && d.c_dtype == TH_F32 && !d.bias;
    if ((best.tile != TH_TILE_GENERAL || general_splits) && d.epilogue == TH_EPI_STORE) {
      for (int sp : {1, 2, 4, 8, 16}) {
        if (sp > 1 && d.k / sp < 256) break;
        const int used = splits_used(&d, best.tile, sp);
        if (used == best.splits) continue;
        double s = 0;
        if (int r = measure(&d, best.tile, sp, &s)) return r;
        if (s < best.seconds) best = Tuned{best.tile, used, s};
      }
    }
    hit = g_tuned.emplace(key, best).first;
  }
  *tile_out = hit->second.tile;
  *splits_out = hit->second.splits;
  *seconds_out = hit->second.seconds;
  return TH_OK;
}

extern "C" int th_build_gemm_grouped(const th_gemm_desc* descs, int count, th_launch** out) {
  if (int r = th::require_ready()) return r;
  *out = nullptr;
  TH_REQUIRE(descs != nullptr && count >= 1, "th_build_gemm_grouped: no products");
  std::vector<th_launch*> parts;
  auto drop = [&]() {
    for (th_launch* l : parts) th_launch_destroy(l);
  };
  for (int i = 0; i < count; ++i) {
    th_launch* l = nullptr;
    if (int r = th_build_gemm(&descs[i], &l)) {
      drop();
      return r;
    }
    parts.push_back(l);
  }
  // One launch: every product's kernels in order, its values after the
  // previous products', its workspaces owned by the whole.
  th_launch* g = new th_launch();
  g->name = "gemm_grouped";
  for (th_launch* l : parts) {
    const int k0 = (int)g->kernels.size();
    g->kernels.insert(g->kernels.end(), l->kernels.begin(), l->kernels.end());
    for (size_t v = 0; v < l->values.size(); ++v) {
      std::vector<th::Ref> refs = l->values[v];
      for (th::Ref& r : refs) r.kernel += k0;
      g->values.push_back(refs);
      g->align.push_back(l->align[v]);
    }
    g->owned.insert(g->owned.end(), l->owned.begin(), l->owned.end());
    l->owned.clear();
    // Its workspace follows the previous products' in the whole's.
    for (th::WsRef r : l->ws_refs) {
      r.kernel += k0;
      r.at += g->ws_bytes;
      g->ws_refs.push_back(r);
    }
    g->ws_bytes += l->ws_bytes;
    g->work.bytes += l->work.bytes;
    g->work.flops += l->work.flops;
    g->work.blocks += l->work.blocks;
  }
  g->work.kernels = (int32_t)g->kernels.size();
  g->work.values = (int32_t)g->values.size();
  drop();
  *out = g;
  return TH_OK;
}
