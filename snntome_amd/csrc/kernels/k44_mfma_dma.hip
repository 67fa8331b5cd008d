// Translation unit of the LDS-DMA MFMA tile kernel (512 tokens per workgroup, NT 32 / 64 with
// 2- or 4-stage rings, NT 128 with a 3-stage ring; NT 32 / 64 with producer waves, 4 stages).
#include "k44_launch.hpp"
#include "k44_mfma_dma.hpp"

namespace k44dev {

hipError_t launch_mfma_dma(const MfmaGroup &a, uint32_t nt, uint32_t items, hipStream_t stream,
                           const DmaShape &shape) {
    const dim3 grid(items, 1u, 1u), block(512u + 64u * shape.prod, 1u, 1u);
#define K44_DMA_P(NT, B, P)                                                                     \
    if (shape.stream_loads)                                                                     \
        hipLaunchKernelGGL((k44_mfma_dma_kernel<NT, true, B, P>), grid, block, 0, stream,        \
                           K44_GROUP_ARGS(a));                                                  \
    else                                                                                        \
        hipLaunchKernelGGL((k44_mfma_dma_kernel<NT, false, B, P>), grid, block, 0, stream,       \
                           K44_GROUP_ARGS(a));
#define K44_DMA(NT, B) K44_DMA_P(NT, B, 0)
    if (shape.prod != 0u) {
        // Producer/consumer forms: 4-stage rings, one workgroup per CU (8 + P waves).
        if (nt == 32u && shape.nbuf == 4u && shape.prod == 2u) {
            K44_DMA_P(32, 4, 2)
        } else if (nt == 64u && shape.nbuf == 4u && shape.prod == 4u) {
            K44_DMA_P(64, 4, 4)
        } else {
            return hipErrorInvalidValue;
        }
    } else if (nt == 32u && shape.nbuf == 4u) {
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
#undef K44_DMA_P
    return hipGetLastError();
}

}  // namespace k44dev
