// Instantiates the bf16 product kernel with the kStoreF32 epilogue (gemm_kernel.h).
#include "gemm_kernel.h"

namespace thg {
const void* gemm_store_f32(int la, int lb, bool check) { return kernel_for<kStoreF32>(la, lb, check); }
}  // namespace thg
