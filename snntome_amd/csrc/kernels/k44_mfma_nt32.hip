// Translation unit of the MFMA tile kernel for 32-neuron tiles.
#include "k44_launch.hpp"

namespace k44dev {

hipError_t launch_mfma_tile_nt32(const MfmaGroup &a, uint32_t mt, uint32_t rows_per_stage,
                                 uint32_t items, hipStream_t stream, bool mis) {
    const dim3 grid(items, 1u, 1u), block(mt, 1u, 1u);
#define K44_MFMA_CASE(MT)                                                                       \
    case MT:                                                                                    \
        if (mis)                                                                                \
            hipLaunchKernelGGL((k44_mfma_tile_kernel<32, MT, 32, true>), grid, block, 0, stream, K44_GROUP_ARGS(a)); \
        else if (rows_per_stage == 64u)                                                         \
            hipLaunchKernelGGL((k44_mfma_tile_kernel<32, MT, 64>), grid, block, 0, stream, K44_GROUP_ARGS(a)); \
        else                                                                                    \
            hipLaunchKernelGGL((k44_mfma_tile_kernel<32, MT, 32>), grid, block, 0, stream, K44_GROUP_ARGS(a)); \
        break;
    switch (mt) {
        K44_MFMA_CASE(512u)
        K44_MFMA_CASE(256u)
        K44_MFMA_CASE(128u)
        K44_MFMA_CASE(64u)
    default:
        return hipErrorInvalidValue;
    }
#undef K44_MFMA_CASE
    return hipGetLastError();
}

}  // namespace k44dev
