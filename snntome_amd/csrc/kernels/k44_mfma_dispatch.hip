// Dispatch of launch_mfma_tile to the per-tile-size translation units.
#include "k44_launch.hpp"

namespace k44dev {

hipError_t launch_mfma_tile_nt16(const MfmaGroup &, uint32_t, uint32_t, uint32_t, hipStream_t, bool);
hipError_t launch_mfma_tile_nt32(const MfmaGroup &, uint32_t, uint32_t, uint32_t, hipStream_t, bool);
hipError_t launch_mfma_tile_nt64(const MfmaGroup &, uint32_t, uint32_t, uint32_t, hipStream_t, bool);
hipError_t launch_mfma_tile_nt128(const MfmaGroup &, uint32_t, uint32_t, uint32_t, hipStream_t, bool);

hipError_t launch_mfma_tile(const MfmaGroup &g, uint32_t nt, uint32_t mt, uint32_t rows_per_stage,
                            uint32_t items, hipStream_t stream, bool mis) {
    if (items == 0u) return hipSuccess;
    if (mis && rows_per_stage != 32u) return hipErrorInvalidValue;
    switch (nt) {
    case 16u: return launch_mfma_tile_nt16(g, mt, rows_per_stage, items, stream, mis);
    case 32u: return launch_mfma_tile_nt32(g, mt, rows_per_stage, items, stream, mis);
    case 64u: return launch_mfma_tile_nt64(g, mt, rows_per_stage, items, stream, mis);
    case 128u: return launch_mfma_tile_nt128(g, mt, rows_per_stage, items, stream, mis);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace k44dev
