// Kernel argument blocks of the hipRTC preprocess kernels, shared verbatim by the host launcher and the
// runtime-compiled device code (plain pointers and scalars, identical layout on both sides).
#pragma once
#ifndef EFGS_RTC
#include <stdint.h>
#endif

namespace efgs {

struct PrimRecord;

struct CameraArgs {
    const float* w2c;           // rows 0..2 of the world-to-view transform (row-major, 4 floats per row)
    const float* cam_position;  // 3 floats
    uint32_t width, height, grid_w, grid_h;
    float focal_x, focal_y, center_x, center_y, near_plane, far_plane;
    // limits of the projected x / z and y / z that the EWA Jacobian clamps to (1.15x the image, fixed per camera):
    // (-0.15 width - center_x) / focal_x, (1.15 width - center_x) / focal_x, the same in y with height, in fp32
    float clip_left, clip_right, clip_top, clip_bottom;
    uint32_t degree;            // appearance degree used for rendering (0 when the residual is off)
    uint32_t proper_aa;
    uint32_t render_base;
    uint32_t pad_;
};

struct PreprocessForwardArgs {
    const float* means;
    const float* scales;
    const float* rotations;
    const float* opacities;
    const float* precomputed;
    const float* base;
    const float* residual;
    const float* mlp_weights;     // fp32 master weights, flat tcnn layout (rounded to fp16 as they are staged in LDS)
    uint32_t* n_touched;          // (N) 0 for culled primitives
    uint32_t* depth_keys;         // (N) float bits of the view depth
    PrimRecord* records;          // (N) written for visible primitives
    uint32_t* block_counts;       // (2 * blocks) visible count and instance count per block
    uint32_t* block_key_ranges;   // (2 * blocks) min and max depth key of the block's visible primitives
    uint32_t* counters;           // the frame's counters: [2] (instance-emission mismatches) is cleared here
    uint32_t n;
    uint32_t pad_;
    CameraArgs cam;
};

struct PreprocessBackwardArgs {
    const float* means;
    const float* scales;
    const float* rotations;
    const float* opacities;
    const float* base;
    const float* residual;
    const float* mlp_weights;        // fp32 master weights, flat tcnn layout
    const uint32_t* n_touched;
    const uint32_t* prim_offset;     // (N) first emitted instance of each visible primitive
    const PrimRecord* records;
    const float* inst_grads;         // (I x 9, or I x 12 with three densification rows) per-instance blend gradients, emission order
    float* g_means;
    float* g_scales;
    float* g_rotations;
    float* g_opacities;
    float* g_precomputed;
    float* g_base;
    float* g_residual;
    float* g_mlp_partials;           // neural: (blocks x n_params) fp32 per-block weight gradient partials
    float* color_grads;              // neural: (N x 4) dL/d(pre-activation colour), geometry kernel -> MLP kernel
    uint32_t* color_grad_max;        // neural: per geometry block, max |dL/d(pre-activation colour)| as float bits
    const uint32_t* visible_prims;   // neural: (V) the visible primitives in index order (the MLP kernel's work list)
    uint32_t n_visible;
    float* densification_info;       // (rows x N) or null
    uint32_t densification_rows;
    uint32_t n;
    CameraArgs cam;
};

struct NeuralDecodeArgs {
    const float* features;           // (N x n_features) learned per-primitive features
    const float* base;               // (N x 3) base colours (read with base input only)
    const float* dirs;               // (N x 3) unit view directions
    const uint16_t* mlp_weights;     // fp16 bits, flat tcnn layout, 16-byte aligned
    const float* grad_out;           // backward: (N x 3) dL/d(raw MLP output)
    float* out;                      // forward: (N x 3) raw MLP outputs (fp16-rounded values)
    float* g_features;               // backward: (N x n_features) written
    float* g_base;                   // backward: (N x 3) written with base input, or null
    float* g_dirs;                   // backward: (N x 3) dL/d(direction) through the SH encoding, or null
    float* g_mlp_partials;           // backward: (blocks x n_params) per-block weight gradient partials
    uint32_t n;
    uint32_t degree;                 // active SH degree count of the direction encoding
};

}  // namespace efgs
