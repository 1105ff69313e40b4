// vq2_gemv_f32.hip -- instantiations of the VQ GEMV kernel for f32 codebooks.
#include "vq2_gemv_kernel.hpp"

namespace vq2 {

hipError_t gemv_dispatch_f32(int s2, const GemvArgs& a, const GemvPlan& p, dim3 grid, size_t shm, hipStream_t st)
{
    return launch_s2<VQ2_DT_F32>(s2, a, p, grid, shm, st);
}

}  // namespace vq2
