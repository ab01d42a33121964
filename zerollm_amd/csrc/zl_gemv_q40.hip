// Tile GEMV instantiations for one weight format (kernel in zl_gemv.h).
#include "zl_gemv.h"

namespace zl {
template void launch_gemv_fmt<T_Q4_0>(const GemvArgs &a, int epi, hipStream_t st);
}  // namespace zl
