// Dispatch of launch_mfma_tile to the per-tile-size translation units.
#include "k44_launch.hpp"

namespace k44dev {

hipError_t launch_mfma_tile_nt16(const MfmaTileArgs &, uint32_t, uint32_t, uint32_t, uint32_t, hipStream_t);
hipError_t launch_mfma_tile_nt32(const MfmaTileArgs &, uint32_t, uint32_t, uint32_t, uint32_t, hipStream_t);
hipError_t launch_mfma_tile_nt64(const MfmaTileArgs &, uint32_t, uint32_t, uint32_t, uint32_t, hipStream_t);
hipError_t launch_mfma_tile_nt128(const MfmaTileArgs &, uint32_t, uint32_t, uint32_t, uint32_t, hipStream_t);

hipError_t launch_mfma_tile(const MfmaTileArgs &a, uint32_t nt, uint32_t mt,
                            uint32_t rows_per_stage, uint32_t tiles, uint32_t tokens,
                            hipStream_t stream) {
    switch (nt) {
    case 16u: return launch_mfma_tile_nt16(a, mt, rows_per_stage, tiles, tokens, stream);
    case 32u: return launch_mfma_tile_nt32(a, mt, rows_per_stage, tiles, tokens, stream);
    case 64u: return launch_mfma_tile_nt64(a, mt, rows_per_stage, tiles, tokens, stream);
    case 128u: return launch_mfma_tile_nt128(a, mt, rows_per_stage, tiles, tokens, stream);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace k44dev
