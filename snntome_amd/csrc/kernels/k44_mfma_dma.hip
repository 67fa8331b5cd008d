// Translation unit of the LDS-DMA MFMA tile kernel (512 tokens per workgroup, NT 32 / 64).
#include "k44_launch.hpp"
#include "k44_mfma_dma.hpp"

namespace k44dev {

hipError_t launch_mfma_dma(const MfmaGroup &a, uint32_t nt, uint32_t items, hipStream_t stream) {
    const dim3 grid(items, 1u, 1u), block(512u, 1u, 1u);
    switch (nt) {
    case 32u:
        hipLaunchKernelGGL((k44_mfma_dma_kernel<32>), grid, block, 0, stream, a);
        break;
    case 64u:
        hipLaunchKernelGGL((k44_mfma_dma_kernel<64>), grid, block, 0, stream, a);
        break;
    default:
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace k44dev
