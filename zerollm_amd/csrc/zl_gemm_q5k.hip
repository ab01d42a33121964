// GEMM (10..64 tokens) instantiations for one weight format (kernel in zl_gemm.h).
#include "zl_gemm.h"

namespace zl {
template void launch_gemm_fmt<T_Q5_K>(const GemvArgs &a, int epi, hipStream_t st);
}  // namespace zl
