// Translation unit of the LDS-DMA MFMA tile kernel (512 tokens per workgroup, NT 32 / 64).
#include "k44_launch.hpp"
#include "k44_mfma_dma.hpp"

namespace k44dev {

hipError_t launch_mfma_dma(const MfmaGroup &a, uint32_t nt, uint32_t items, hipStream_t stream,
                           bool stream_loads) {
    const dim3 grid(items, 1u, 1u), block(512u, 1u, 1u);
#define K44_DMA(NT)                                                                    \
    if (stream_loads)                                                                  \
        hipLaunchKernelGGL((k44_mfma_dma_kernel<NT, true>), grid, block, 0, stream, a); \
    else                                                                               \
        hipLaunchKernelGGL((k44_mfma_dma_kernel<NT, false>), grid, block, 0, stream, a);
    switch (nt) {
    case 32u: K44_DMA(32) break;
    case 64u: K44_DMA(64) break;
    default: return hipErrorInvalidValue;
    }
#undef K44_DMA
    return hipGetLastError();
}

}  // namespace k44dev
