// Instantiates the bf16 product kernel with the kStore epilogue (gemm_kernel.h).
#include "gemm_kernel.h"

namespace thg {
const void* gemm_store(int la, int lb, bool check) { return kernel_for<kStore>(la, lb, check); }
}  // namespace thg
