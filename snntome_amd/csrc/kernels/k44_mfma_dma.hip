// Translation unit of the LDS-DMA MFMA tile kernel (512 tokens per workgroup, NT 32 / 64 with
// 2- or 4-stage rings, NT 128 with a 3-stage ring).
#include "k44_launch.hpp"
#include "k44_mfma_dma.hpp"

namespace k44dev {

hipError_t launch_mfma_dma(const MfmaGroup &a, uint32_t nt, uint32_t items, hipStream_t stream,
                           const DmaShape &shape) {
    const dim3 grid(items, 1u, 1u), block(512u, 1u, 1u);
#define K44_DMA(NT, B)                                                                          \
    if (shape.stream_loads)                                                                     \
        hipLaunchKernelGGL((k44_mfma_dma_kernel<NT, true, B>), grid, block, 0, stream, K44_GROUP_ARGS(a));      \
    else                                                                                        \
        hipLaunchKernelGGL((k44_mfma_dma_kernel<NT, false, B>), grid, block, 0, stream, K44_GROUP_ARGS(a));
    if (nt == 32u && shape.nbuf == 4u) {
        K44_DMA(32, 4)
    } else if (nt == 32u && shape.nbuf == 2u) {
        K44_DMA(32, 2)
    } else if (nt == 64u && shape.nbuf == 4u) {
        K44_DMA(64, 4)
    } else if (nt == 64u && shape.nbuf == 2u) {
        K44_DMA(64, 2)
    } else if (nt == 128u && shape.nbuf == 3u) {
        K44_DMA(128, 3)
    } else {
        return hipErrorInvalidValue;
    }
#undef K44_DMA
    return hipGetLastError();
}

}  // namespace k44dev
