// gemv_f32.hip -- instantiations of the K+1-row GEMV kernel (gemv_kernel.h)
// for W_F32 weights with A_F32 activations.
#include "gemv_kernel.h"

namespace opure_gemv {

int launch_f32(opure_dev* dev, uint32_t epi, uint32_t nm, bool staged, const KParams& kp, const Recipe& r, uint32_t grid,
        uint32_t lds)
{
    return launch_format<OPURE_W_F32, OPURE_A_F32>(dev, epi, nm, staged, kp, r, grid, lds);
}

int launch_valu_f32(opure_dev* dev, uint32_t epi, const KParams& kp)
{
    return launch_valu<OPURE_W_F32, OPURE_A_F32>(dev, epi, kp);
}

}  // namespace opure_gemv
