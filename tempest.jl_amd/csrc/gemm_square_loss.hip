// Instantiates the bf16 product kernel with the kSquareLoss epilogue (gemm_kernel.h).
#include "gemm_kernel.h"

namespace thg {
const void* gemm_square_loss(int la, int lb, bool check) { return kernel_for<kSquareLoss>(la, lb, check); }
}  // namespace thg
