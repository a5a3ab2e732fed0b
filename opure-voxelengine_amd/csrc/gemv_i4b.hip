// gemv_i4b.hip -- instantiations of the K+1-row GEMV kernel (gemv_kernel.h)
// for W_I4G128 weights with A_BF16 activations.
#include "gemv_kernel.h"

namespace opure_gemv {

int launch_i4_bf16(opure_dev* dev, uint32_t epi, bool norm, bool staged, const KParams& kp, const Recipe& r, uint32_t grid,
        uint32_t lds)
{
    return launch_format<OPURE_W_I4G128, OPURE_A_BF16>(dev, epi, norm, staged, kp, r, grid, lds);
}

}  // namespace opure_gemv
