// Instantiates the bf16 product kernel with the kGelu epilogue (gemm_kernel.h).
#include "gemm_kernel.h"

namespace thg {
const void* gemm_gelu(int la, int lb, bool check) { return kernel_for<kGelu>(la, lb, check); }
}  // namespace thg
