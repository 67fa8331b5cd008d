// k44_spatial.hpp — kernels of 2-D (spatial) plans: waves over the padded-plane tile layout and
// the spatial aux commands.
//
// 2-D tensor layout (reference wavec/k44_plan_types.hpp:447-569): channel c, frame f, pixel
// (y, x) at c*channel_stride + f*single_stride + (y+1)*W_pad + 4 + x; every other element of a
// plane is zero padding ("halo").  Two modes: W % 64 == 0 (W_pad = W + 8, a 64-token tile is 64
// pixels of one row) and any other W (W_pad = W + 4, a tile is 64 consecutive plane elements
// from (row 1, column 4), spanning rows and halo columns; only pixels are stored).
// 64-frame interleaved images (batches of whole 64-frame blocks, k44_plan_types.hpp:576-598):
// pixel (y, x) of frame f at c*channel_stride + (f/64)*64*single_stride +
// ((y+1)*W_pad + x+1)*64 + f%64 — a 64-token tile is the 64 frames of one pixel, every tile is
// 64-element aligned, and a tap (dy, dx) is a shift by whole pixels of 64 elements.
//
//  * WAVE (2-D): token m of tile t reads X[seg + s*step + tile_x[t] + m] — seg holds the
//    reference's tap-shifted channel offsets ((1+dy)*W_pad + (1+dx) relative to the tile
//    anchor), so 3x3 taps are element-misaligned — and writes Y[y_off + out_j*channel_stride +
//    tile_y[t] + m] for pixels only.  Epilogue as in k44_gather_dot.hpp.
//  * S2D_2X2 (ref kernels/common/kernel44_valu_pack.cuh:80-92): out channel 4c + 2py + px at
//    (y, x) = in channel c at (2y+py, 2x+px).
//  * MAXPOOL_2X2 (:30-38): out (y, x) = max of in (2y..2y+1, 2x..2x+1).
//  * MAXPOOL_5X5, stride 1, pad 2 (:40-55): max over the in-bounds 5x5 window.
//  * UPSAMPLE_2X nearest (:56-64): out (2y+a, 2x+b) = in (y, x).
//  * SCATTER_UP2X2 (:93-103): out channel c at (y, x) = in channel q*Q + c at (y/2, x/2),
//    q = 2*(y&1) + (x&1), Q = quad input channels / 4 (the compiler pads each quad plane group
//    to a multiple of 16 channels; the reference reads q*Cout + c, equal when Cout % 16 == 0).
//  * HALO CLEAR: zero every non-pixel element of each (channel, frame) plane — (channel,
//    64-frame block) plane of 64 * single_stride elements in the interleaved layout — of a
//    tensor (run after every command that writes a 2-D tensor: canvas memory is reused between
//    tensors, and the next 3x3 tap reads the halo as zero padding).
#pragma once
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace k44dev {

struct Plane2D {
    uint32_t H, W, W_pad, frames;
    uint64_t single_stride, channel_stride;
    uint32_t tok64;  // 1: 64-frame interleaved layout (frames a multiple of 64)
};

struct GatherTileArgs {
    const __half *X;         // canvas base
    const uint64_t *seg;     // [rows][K] canvas offsets of segment starts (tile anchor relative)
    const __half *W;         // [cout][K*S] fp16, row-major synapse order
    const __half *bias;      // [cout] or nullptr
    const uint16_t *cmap;    // [cout] or nullptr
    __half *Y;               // canvas + y_off
    const __half *R;         // canvas + res_off, or nullptr
    const uint32_t *tile_x;  // [tiles] gather offset of each 64-token tile
    const uint32_t *tile_y;  // [tiles] store offset of each tile
    uint64_t step;
    uint32_t K, S, cluster, cout, tiles;
    uint64_t out_stride;     // channel stride of the output tensor
    int act;
    Plane2D plane;           // output layout (pixel test of each token)
    uint32_t tiles_per_frame;
    int masked;              // 1: W % 64 != 0 layout (tiles span rows and halo columns)
};

hipError_t launch_gather_tile(const GatherTileArgs &a, hipStream_t stream);
hipError_t launch_halo_clear(__half *base, uint32_t channels, const Plane2D &p,
                             hipStream_t stream);
hipError_t launch_s2d(__half *y, const __half *x, uint32_t cin, const Plane2D &in,
                      const Plane2D &out, hipStream_t stream);
hipError_t launch_maxpool2(__half *y, const __half *x, uint32_t c, const Plane2D &in,
                           const Plane2D &out, hipStream_t stream);
hipError_t launch_maxpool5(__half *y, const __half *x, uint32_t c, const Plane2D &in,
                           const Plane2D &out, hipStream_t stream);
hipError_t launch_upsample2(__half *y, const __half *x, uint32_t c, const Plane2D &in,
                            const Plane2D &out, hipStream_t stream);
// qstride: channels between the quad planes of the input (q * qstride + c).
hipError_t launch_scatter_up2(__half *y, const __half *x, uint32_t cout, uint32_t qstride,
                              const Plane2D &in, const Plane2D &out, hipStream_t stream);

}  // namespace k44dev
