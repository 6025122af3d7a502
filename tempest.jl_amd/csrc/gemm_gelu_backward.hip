// Instantiates the bf16 product kernel with the kGeluBackward epilogue (gemm_kernel.h).
#include "gemm_kernel.h"

namespace thg {
const void* gemm_gelu_backward(int la, int lb, bool check) { return kernel_for<kGeluBackward>(la, lb, check); }
}  // namespace thg
