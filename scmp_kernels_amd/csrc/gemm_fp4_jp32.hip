// FP4 SC GEMM kernels for stream tables of 32 intervals per inner dimension.
#include "gemm_fp4_kernel.h"

namespace scmp {
template int gemm_fp4_launch_jpf<32>(const GemmP &, int64_t, bool, hipStream_t);
}  // namespace scmp
