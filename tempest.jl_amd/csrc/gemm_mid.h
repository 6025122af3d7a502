// The product's middle tiles (gemm_mid.hip): the arguments and the kernel for
// a tile, layouts and factor type, shared with the builder (gemm.hip).
#pragma once

#include <cstdint>

namespace thg {

struct MidArgs {
  const uint16_t* a;
  const uint16_t* b;
  void* c;               // result, or (staged) the fp32 parts of K
  const void* d;         // C = D + A B where non-null (not staged), laid out at d_ld / d_batch
  const uint16_t* bias;  // bf16, per row of C, or null (not staged)
  int64_t a_m, a_k, a_batch;
  int64_t b_k, b_n, b_batch;
  int64_t c_ld, c_batch;
  int64_t c_split;  // part s of K writes s * c_split further (staged)
  int64_t d_ld, d_batch;
  int32_t m, n, k;
  int32_t ksplit;   // K per part
  int32_t tiles_m;
  int32_t result;   // TH_F32, TH_BF16 or TH_F16 (staged: TH_F32)
};

// The kernel for tile (TH_TILE_128X128 .. TH_TILE_64X64) over fp16 or bf16
// factors, A k-contiguous (a_k == 1) or m-contiguous, B k-contiguous (b_k ==
// 1) or n-contiguous; nullptr for any other tile.  Rows and columns of the
// tile (bm, bn) and its LDS bytes go to *bm, *bn, *lds.
const void* mid_kernel(int tile, bool f16, bool a_kc, bool b_kc, int* bm, int* bn, int* lds);

}  // namespace thg
