// gemv_i8.hip -- instantiations of the K+1-row GEMV kernel (gemv_kernel.h)
// and of the GEMV over more rows (gemm_wide.h)
// for W_I8PC weights with A_F16 activations.
#include "gemm_wide.h"

namespace opure_gemv {

int launch_i8(opure_dev* dev, uint32_t epi, uint32_t nm, bool staged, const KParams& kp, const Recipe& r, uint32_t grid,
        uint32_t lds)
{
    return launch_format<OPURE_W_I8PC, OPURE_A_F16>(dev, epi, nm, staged, kp, r, grid, lds);
}

int launch_valu_i8(opure_dev* dev, uint32_t epi, const KParams& kp)
{
    return launch_valu<OPURE_W_I8PC, OPURE_A_F16>(dev, epi, kp);
}

int launch_wide_i8(opure_dev* dev, uint32_t epi, const WParams& wp, uint32_t lds, const float* gain, void* xn)
{
    return launch_wide_format<OPURE_W_I8PC, OPURE_A_F16>(dev, epi, wp, lds, gain, xn);
}

}  // namespace opure_gemv
