// FP4 SC GEMM kernels for stream tables of 16 intervals per inner dimension (four inner
// dimensions per MFMA k-step).
#include "gemm_fp4_kernel.h"

namespace scmp {
template int gemm_fp4_launch_jpf<16>(const GemmP &, int64_t, bool, hipStream_t);
}  // namespace scmp
