// vq2_gemv_f16.hip -- instantiations of the VQ GEMV kernel for f16 codebooks.
#include "vq2_gemv_kernel.hpp"

namespace vq2 {

hipError_t gemv_dispatch_f16(int s2, const GemvArgs& a, const GemvPlan& p, dim3 grid, size_t shm, hipStream_t st)
{
    return launch_s2<VQ2_DT_F16>(s2, a, p, grid, shm, st);
}

}  // namespace vq2
