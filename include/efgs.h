/*
 * efgs.h -- C ABI of the MI355X (gfx950) fused-appearance Gaussian rasterizer (libefgs_hip.so).
 *
 * Plain pointers, sizes and POD structs only. Every tensor argument is a device pointer to contiguous fp32
 * data in the reference's layouts (N x k row-major, quaternions (w, x, y, z), opacity logits, CHW images);
 * `stream` is a hipStream_t. Functions return EFGS_OK or an error code; efgs_last_error() gives the message
 * of the calling thread's last failure.
 *
 * Reference interfaces replaced (paths relative to the reference repository,
 * B/ = FasterGSVDACudaBackend/FasterGSVDACudaBackend/):
 *   _C.set_rtc_dirs ............ B/torch_bindings/bindings.cu:14-28, B/rasterization/src/appearance.cu:16-21
 *   _C.Rasterizer() ............ B/torch_bindings/rasterization.py:8, B/rasterization/include/appearance.h:18-88
 *   Rasterizer.set_appearance .. B/rasterization/src/appearance.cu:166-179
 *   Rasterizer.set_residual_mlp  B/rasterization/src/appearance.cu:181-201
 *   _C.forward ................. B/rasterization/src/rasterization_api.cu:16-123
 *   _C.backward ................ B/rasterization/src/rasterization_api.cu:125-247
 *   _C.inference ............... B/rasterization/src/rasterization_api.cu:249-335
 *   _C.pruning_scores .......... B/rasterization/src/rasterization_api.cu:337-415
 *   _C.adam_step ............... B/adam/src/adam.cu:44-87
 *   _C.add_noise ............... B/densification/src/densification_api.cu:40-72
 *   _C.relocation_adjustment ... B/densification/src/densification_api.cu:13-38
 *   .ngsplat per-splat packing . viewer/export_ngsplat.py:311-400, :576-611, :624-765, :1465-1530 (numpy script)
 */
#ifndef EFGS_H
#define EFGS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    EFGS_OK = 0,
    EFGS_ERR_INVALID_ARGUMENT = 1,  /* bad id, size or null pointer */
    EFGS_ERR_STATE = 2,             /* e.g. forward before set_appearance, set_residual_mlp on a non-neural model */
    EFGS_ERR_HIP = 3,               /* HIP runtime failure */
    EFGS_ERR_RTC = 4,               /* hipRTC compilation or module load failure */
    EFGS_ERR_ALLOC = 5              /* the allocation callback returned NULL */
};

/* appearance model ids (B/torch_bindings/rasterization.py:21-24); 0 is the internal precomputed-colour variant */
enum { EFGS_MODEL_PRECOMPUTED = 0, EFGS_MODEL_SH = 1, EFGS_MODEL_SV = 2, EFGS_MODEL_NASG = 3, EFGS_MODEL_NASGABOR = 4, EFGS_MODEL_NEURAL = 5 };

typedef struct efgs_rasterizer efgs_rasterizer;

/* Caller-owned device allocation: returns a device pointer of at least `bytes` bytes (256-byte aligned) that
 * stays valid until the caller releases it. Used for the forward's persistent buffers (kept for the
 * backward) and for the backward's temporaries. */
typedef void* (*efgs_alloc_fn)(void* ctx, size_t bytes);

/* Bump allocator over one caller-provided device region (no counterpart in the reference: it spares callers
 * a callback per buffer). Pass efgs_workspace_alloc as the efgs_alloc_fn and a workspace as its context: each
 * request takes the next 256-byte-aligned slice of [base, base + capacity); a request that does not fit goes
 * to `fallback` (if set) and the slice is left unused. `requested` accumulates the aligned sizes of all
 * requests, so a caller can size the next call's region. */
typedef struct efgs_workspace {
    void* base;               /* device region, 256-byte aligned */
    size_t capacity;
    size_t used;              /* bytes handed out from the region */
    size_t requested;         /* bytes asked for in total (region + fallback) */
    efgs_alloc_fn fallback;   /* may be NULL: a request that does not fit then fails */
    void* fallback_ctx;
} efgs_workspace;
void* efgs_workspace_alloc(void* workspace, size_t bytes);

/* Message of the calling thread's last error (empty if none). */
const char* efgs_last_error(void);

/* Directory for cached hipRTC code objects and directory holding the preprocess kernel sources.
 * Replaces _C.set_rtc_dirs(cache, include, kernel_dir): B/rasterization/src/appearance.cu:16-21. */
int efgs_set_rtc_dirs(const char* cache_dir, const char* kernel_dir);

/* Replaces the _C.Rasterizer singleton (B/torch_bindings/rasterization.py:8). */
int efgs_rasterizer_create(efgs_rasterizer** out);
void efgs_rasterizer_destroy(efgs_rasterizer* r);

/* Selects the appearance model and activations and invalidates the specialised kernels (compiled lazily).
 * model 1..5; base_act 0 none / 1 exp; residual_act 0 none / 1 tanh / 2 softplus; color_act 0 none /
 * 1 relu / 2 softplus / 3 sigmoid / 4 hardsigmoid / 5 satexp. max_degree: SH degree, SV sites, lobes.
 * Replaces Rasterizer::set_appearance, B/rasterization/src/appearance.cu:166-179. */
int efgs_set_appearance(efgs_rasterizer* r, int model, int max_degree, int base_act, int residual_act, int color_act,
                        int direction_gradient);

/* Residual MLP of the neural model: bias-free, hidden_activation 1 = ReLU (the only one supported),
 * 'None' output activation, tcnn flat parameter layout (row-major [out x in] matrices, input padded to a
 * multiple of 16, output padded to 16 rows). sh_degree_mask: bit l = SH degree l in the direction encoding.
 * Requires efgs_set_appearance(model = 5) first.
 * Replaces Rasterizer::set_residual_mlp, B/rasterization/src/appearance.cu:181-201. */
int efgs_set_residual_mlp(efgs_rasterizer* r, int n_input_dims, int n_output_dims, int n_neurons, int n_hidden_layers,
                          int hidden_activation, int base_input, int n_frequencies, int sh_degree_mask);

/* Number of fp16 parameters of the configured residual MLP (0 if none). */
int64_t efgs_mlp_param_count(const efgs_rasterizer* r);

/* Camera and render settings: RasterizerSettings, B/torch_bindings/rasterization.py:49-83. */
typedef struct efgs_settings {
    const float* w2c;            /* device, >= 12 floats: rows 0..2 of the world-to-view matrix, row-major */
    const float* cam_position;   /* device, 3 floats */
    const float* bg_color;       /* device, 3 floats */
    int appearance_degree;
    int width, height;
    float focal_x, focal_y, center_x, center_y;
    float near_plane, far_plane;
    int proper_antialiasing;
    int render_base;
    int render_residual;         /* 0 renders at appearance degree 0 */
} efgs_settings;

typedef struct efgs_primitives {
    int64_t n_primitives;
    const float* means;               /* (N, 3) */
    const float* scales;              /* (N, 3) log scales */
    const float* rotations;           /* (N, 4) (w, x, y, z), unnormalised */
    const float* opacities;           /* (N, 1) logits */
    const float* precomputed_colors;  /* (N, 3) or NULL; non-NULL selects the precomputed-colour variant */
    const float* base_colors;         /* (N, 3) or NULL */
    const float* residual_params;     /* model-specific (N, ...) or NULL */
    const float* mlp_weights;         /* fp32 master weights, efgs_mlp_param_count entries, 16-byte aligned, neural only
                                         (rounded to fp16, to nearest even, as the kernels stage them) */
} efgs_primitives;

/* Forward state consumed by the backward. The three buffers are caller-owned allocations made through the
 * callback during efgs_forward; the scalars describe their layout. */
typedef struct efgs_frame {
    void* primitive_buffers;
    void* tile_buffers;
    void* instance_buffers;
    int64_t n_primitives;
    int64_t n_visible;
    int64_t n_instances;
    int64_t instance_capacity;   /* instances the instance buffers are laid out for (>= n_instances) */
    int32_t grid_width, grid_height;
    int32_t key_bytes;           /* 2 or 4: width of the tile keys */
    int32_t model;               /* variant used (0 = precomputed colours) */
} efgs_frame;

/* Renders image (device, 3 x H x W fp32, written) and fills *frame. Blocks once on `stream` to read the
 * visible-primitive and instance counts (the reference does the same, B/rasterization/src/forward.cu:82-86);
 * after the first frame of a scene size the read follows the last launch (instance buffers sized from the
 * previous count with headroom; a larger count re-runs the binning and the blend with exact buffers).
 * Replaces _C.forward, B/rasterization/src/rasterization_api.cu:16-123. */
int efgs_forward(efgs_rasterizer* r, const efgs_primitives* prims, const efgs_settings* settings, float* image,
                 efgs_alloc_fn alloc, void* alloc_ctx, efgs_frame* frame, void* stream);

/* Inference render: the same pipeline without the backward state. image (device, fp32) is written 3 x H x W
 * when to_chw != 0, else H x W x 3, clamped to [0, 1] (NaN to 0) when clamp_output != 0. Buffers come from
 * `alloc` and are dead on return (stream-ordered). One blocking counter read, as efgs_forward.
 * Replaces _C.inference, B/rasterization/src/rasterization_api.cu:249-335 (kernels
 * B/rasterization/include/kernels_inference.cuh:11-126). */
int efgs_render(efgs_rasterizer* r, const efgs_primitives* prims, const efgs_settings* settings, float* image, int to_chw, int clamp_output,
                efgs_alloc_fn alloc, void* alloc_ctx, void* stream);

typedef struct efgs_gradients {
    float* means;                 /* (N, 3) written */
    float* scales;                /* (N, 3) written */
    float* rotations;             /* (N, 4) written */
    float* opacities;             /* (N, 1) written */
    float* precomputed_colors;    /* (N, 3) written, precomputed variant only */
    float* base_colors;           /* (N, 3) written */
    float* residual_params;       /* same shape as the parameters, written */
    float* mlp_weights;           /* fp32, efgs_mlp_param_count entries, written (neural only) */
    float* densification_info;    /* (rows, N) accumulated in place, or NULL */
    int densification_rows;       /* 0, 2 or 3 (3 also accumulates the absolute 2D-mean gradient norm) */
} efgs_gradients;

/* Gradients of the image with respect to all inputs. Stream-ordered, no host synchronisation. `prims`,
 * `settings` and `image` must be those of the forward that produced `frame`.
 * Replaces _C.backward, B/rasterization/src/rasterization_api.cu:125-247. */
int efgs_backward(efgs_rasterizer* r, const efgs_primitives* prims, const efgs_settings* settings, const efgs_frame* frame,
                  const float* image, const float* grad_image, efgs_gradients* grads, efgs_alloc_fn alloc, void* alloc_ctx,
                  void* stream);

/* One Adam step over several parameter groups in a single launch. lrs: n_lrs (1..7) learning rates cycled
 * by element index; step counts from 1.
 * Replaces _C.adam_step (one launch per group), B/adam/src/adam.cu:44-87. */
typedef struct efgs_adam_group {
    const float* grad;
    float* param;
    float* exp_avg;
    float* exp_avg_sq;
    int64_t n_elements;
    int64_t step;
    int32_t n_lrs;
    int32_t pad_;
    double lrs[7];
    double beta1, beta2, eps;
} efgs_adam_group;
int efgs_adam_step(const efgs_adam_group* groups, int n_groups, void* stream);

/* Speedy-Splat pruning scores of one view: scores (device, n_primitives fp32) += per primitive the sum over the
 * view's pixels of (o dL/dalpha)^2 for the upstream gradient (1, 1, 1) (o the projected opacity; alpha, the
 * skips and the stop as in the forward). Runs the forward pipeline into a scratch image from `alloc`, then the
 * score pass; one blocking counter read, as efgs_forward. Deterministic (fixed summation order).
 * Replaces _C.pruning_scores, B/rasterization/src/rasterization_api.cu:337-415 (kernels
 * B/rasterization/include/kernels_pruning_scores.cuh:11-171, B/rasterization/src/pruning_scores.cu:11-204). */
int efgs_update_pruning_scores(efgs_rasterizer* r, const efgs_primitives* prims, const efgs_settings* settings, float* scores,
                               efgs_alloc_fn alloc, void* alloc_ctx, void* stream);

/* MCMC noise (3DGS-MCMC): means (n x 3) += current_lr * sigmoid(-(100 sigmoid(raw_opacity) - 0.5)) * Sigma z in
 * place, Sigma from the log-scales (n x 3) and the unnormalised quaternions (n x 4, w x y z; |q|^2 < 1e-8 leaves
 * the mean unchanged), z ~ N(0, I) from Philox4x32-10 with key `seed` and counter (offset / 4, primitive
 * index, 0) through Box-Muller; `offset` must be a multiple of 4 (the caller advances its generator by 4 per
 * call, as PyTorch's philox_engine_inputs(4)). Stream-ordered.
 * Replaces _C.add_noise, B/densification/src/densification_api.cu:40-72 (kernel B/densification/include/
 * kernels_mcmc.cuh:74-144). */
int efgs_add_noise(int64_t n, const float* raw_scales, const float* raw_rotations, const float* raw_opacities, float* means, float current_lr,
                   uint64_t seed, uint64_t offset, void* stream);

/* MCMC relocation: for each of n Gaussians split into n_samples_per_primitive (int64, clamped to 1..50)
 * copies, the new opacity 1 - (1 - o)^(1/n) (n x 1 in, n x 1 out) and the activated scales (n x 3) scaled so
 * that the copies together keep the original's footprint (Eq. 9 of the paper). Outputs are caller-allocated.
 * Replaces _C.relocation_adjustment, B/densification/src/densification_api.cu:13-38 (kernel
 * B/densification/include/kernels_mcmc.cuh:11-56). */
int efgs_relocation_adjustment(int64_t n, const float* old_opacities, const float* old_scales, const int64_t* n_samples_per_primitive,
                               float* new_opacities, float* new_scales, void* stream);

/* ---- .ngsplat export: the per-splat textures of the WebGL viewer's file format ----
 * The reference writes the format with a numpy script (viewer/export_ngsplat.py); these entry points are its
 * per-splat part, run on the device. Splats with sigmoid(raw opacity) < 1/255 are culled, the kept ones are
 * written in source order. Payload kinds (the per-splat residual textures of each appearance model): */
enum {
    EFGS_NGSPLAT_NEURAL_FEATURES = 0,  /* neural, full layout: encoded features as fp16 (1..16 dims) */
    EFGS_NGSPLAT_NEURAL_BAKED = 1,     /* neural, baked layout: h0_static = bake_matrix . encoded + bake_bias as fp16 */
    EFGS_NGSPLAT_SH = 2,               /* raw SH coefficients quantised per level (7 / 8 / 6 bits for degrees 1 / 2 / 3) */
    EFGS_NGSPLAT_SV = 3,               /* spherical Voronoi: unit site, exp temperature, activated colour (7 fp16 per site) */
    EFGS_NGSPLAT_NASG = 4,             /* NASG: frame x, frame z, 2 lambda, a, N, activated colour (12 fp16 per lobe) */
    EFGS_NGSPLAT_NASGABOR = 5          /* NASGabor: the NASG layout plus the Gabor frequency (13 fp16 per lobe) */
};
typedef struct efgs_ngsplat_input {
    int64_t n;                         /* splats */
    const float* means;                /* n x 3 */
    const float* raw_scales;           /* n x 3 log scales */
    const float* raw_rotations;        /* n x 4 (w, x, y, z), unnormalised */
    const float* raw_opacities;        /* n logits */
    const float* base_colors;          /* n x 3 */
    const float* residual_params;      /* n rows of residual_row_stride floats (the model's _residual_params) */
    int64_t residual_row_stride;
    int payload;                       /* EFGS_NGSPLAT_* */
    int n_items;                       /* neural: raw features per row; SH: coefficients exported (0, 3, 8 or 15);
                                          SV: sites (<= 9); NASG: lobes (<= 5); NASGabor: lobes (<= 4) */
    int base_input;                    /* neural: the raw base colours follow the features */
    int n_frequencies;                 /* neural: frequency encoding sin / cos (2^f x), f < k (0 = identity) */
    int n_neurons;                     /* neural baked: rows of bake_matrix (<= 16) */
    int residual_act;                  /* SV / NASG / NASGabor: 0 none, 1 tanh, 2 softplus (baked into the colours) */
    float color_shift;                 /* added to the base colour before its rgb8 quantisation */
    const float* bake_matrix;          /* neural baked, device: n_neurons x encoded width, row-major */
    const float* bake_bias;            /* neural baked, device: n_neurons, or NULL */
} efgs_ngsplat_input;
typedef struct efgs_ngsplat_output {
    int64_t capacity;                  /* rows of every texture: a multiple of 2048 that is >= n */
    uint32_t* splat_words;             /* device, capacity x 4 (RGBA32UI), 16-byte aligned */
    uint32_t* params;                  /* device, the payload textures back to back: texture k holds capacity x
                                          texel_words[k] u32 (efgs_ngsplat_layout), 16-byte aligned */
    int32_t* source_index;             /* device, capacity, optional: source splat of each row, -1 past the kept ones */
    float* kernel_ms;                  /* host, optional (2 floats): milliseconds of the statistics + combine kernels and
                                          of the pack kernel, from HIP events on the stream */
    /* written on return */
    int64_t n_kept;                    /* rows [n_kept, capacity) are zero */
    float base_offset, base_scale;     /* base pre-activation d = base_offset + code8 * base_scale */
    float sh_level_scale[3];           /* SH: max |coefficient| per level (the quantisation scale), 0 when absent */
} efgs_ngsplat_output;
/* Texture count and u32 words per texel of each payload texture (texel_words: 8 entries).
 * Replaces the texture planning of viewer/export_ngsplat.py:372-386 and :576-611. */
int efgs_ngsplat_layout(const efgs_ngsplat_input* in, int* n_textures, int* texel_words);
/* Culls, quantises and packs the splat and payload textures; one blocking read of the 32-byte statistics. Its
 * per-block partials come from `alloc`.
 * Replaces viewer/export_ngsplat.py:1465-1530 (culling, rgb8 base, a8 opacity, layer-0 bake) with the helpers
 * :311-400 (pack_splat_texture, encode_quat_oct, encode_scales, pack_half_textures), :576-611
 * (pack_sh_quantized) and :624-765 (SV / NASG / NASGabor payloads). */
int efgs_ngsplat_pack(const efgs_ngsplat_input* in, efgs_ngsplat_output* out, efgs_alloc_fn alloc, void* alloc_ctx, void* stream);

/* Standalone neural decode: the configured residual MLP (efgs_set_residual_mlp, model 5) on n primitives'
 * features (n x n_features, the learned latents), base colours (n x 3, read with base input only) and unit
 * view directions (n x 3; not read, and may be NULL, when the encoding has no SH degree), encoded as in the
 * rasterizer (frequency encoding, SH degree values of the direction gated by `degree`). With no SH degree, no
 * frequency encoding and no base input the input rows are the features as given: the identity-encoded network
 * of tiny-cuda-nn's NetworkWithInputEncoding (Appearance/Neural.py:40-51,102-111), which efgs.tcnn runs here. Forward writes the raw MLP outputs (n x 3, fp16-rounded values) to `out`.
 * Backward takes dL/d(outputs) (n x 3) and writes the feature gradients (n x n_features), the base-input
 * gradients (n x 3, with base input; may be NULL), the direction gradients (n x 3; may be NULL) and the fp32
 * weight gradients (efgs_mlp_param_count entries); it allocates its per-block partials through `alloc`.
 * Stream-ordered, no host synchronisation. The reference has no Python entry point for this: it is the
 * tiny-cuda-nn MLP that B/rasterization/rtc/appearance_neural.cuh:308-407 calls per primitive
 * (eval_model / backward_eval_model), exposed to measure and test the decode in isolation. */
int efgs_neural_decode_forward(efgs_rasterizer* r, int64_t n, const float* features, const float* base, const float* dirs,
                               const uint16_t* mlp_weights, int degree, float* out, void* stream);
int efgs_neural_decode_backward(efgs_rasterizer* r, int64_t n, const float* features, const float* base, const float* dirs,
                                const uint16_t* mlp_weights, int degree, const float* grad_out, float* g_features, float* g_base,
                                float* g_dirs, float* g_mlp_weights, efgs_alloc_fn alloc, void* alloc_ctx, void* stream);

/* efgs_neural_decode_backward without an allocator, for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). No counterpart in the reference. The
 * per-block weight-gradient partials live in a static 16 MiB device array (4,194,304 floats, one copy per device,
 * held until the process ends); an MLP whose parameter count exceeds that is rejected (EFGS_ERR_INVALID_ARGUMENT),
 * and the block count is min(chunks, 512, 4,194,304 / parameters), so MLPs up to 8,192 parameters get the same
 * blocks, and bit-identical results, as efgs_neural_decode_backward. The first call on a device looks up that
 * device's copy of the array and loads the decode kernels (as any first decode call does); later calls allocate
 * nothing and call no hipMalloc / hipFree. Every call on a device shares its array: calls that overlap on one device
 * (concurrent streams or threads) race and must be serialised by the caller. */
int efgs_neural_decode_backward_no_alloc(efgs_rasterizer* r, int64_t n, const float* features, const float* base, const float* dirs,
                                         const uint16_t* mlp_weights, int degree, const float* grad_out, float* g_features,
                                         float* g_base, float* g_dirs, float* g_mlp_weights, void* stream);

/* Device pointers into a frame's buffers, for inspection (no counterpart in the reference: it lets parity
 * tests compare keys, orders and tile ranges with the CPU oracle). */
typedef struct efgs_frame_views {
    const uint32_t* n_touched;        /* (N) 0 = culled */
    const uint32_t* depth_keys;       /* (N) float bits of the view depth (valid where n_touched > 0) */
    const float* records;             /* (N x 12) mean2d xy, conic xyz, opacity, rgb, packed bounds, pad */
    const uint32_t* visible_prims;       /* (V) the visible primitives in index order */
    const uint32_t* prim_offset;         /* (N) first emission slot of each visible primitive (exclusive scan of
                                            n_touched in index order) */
    const void* instance_keys;           /* (I) tile key of every emission slot, key_bytes wide */
    const uint32_t* instance_primitive;  /* (I) primitive per emission index */
    const void* tile_sorted_keys;        /* (I) key_bytes wide: the tile of every sorted instance */
    const uint32_t* tile_sorted_instances; /* (I) emission index of each instance in (tile, depth, primitive) order */
    const uint32_t* tile_ranges;         /* (T x 2) [start, end) */
    const float* final_transmittance;    /* (T x 192) per tile, row-major 16 x 12 */
    const uint32_t* n_contributors;      /* (T x 192) */
    const uint32_t* counters;            /* (8) V, I, instance-count mismatches, min and max visible depth key, reserved */
} efgs_frame_views;
int efgs_get_frame_views(const efgs_frame* frame, efgs_frame_views* views);

/* Compiles the preprocess kernels of the current configuration into the hipRTC cache for `arch` (e.g.
 * "gfx950") without using a device (no counterpart in the reference; build step). */
int efgs_precompile(const efgs_rasterizer* r, const char* arch);

/* Stage timing (no counterpart in the reference: instrumentation for the roofline report). While enabled,
 * efgs_forward / efgs_backward record a pair of HIP events around each stage on the stream they launch on;
 * efgs_get_stage_times waits for the recorded events and returns, per stage, the summed milliseconds and
 * the number of timed launches since timing was (re-)enabled. Enabling again resets the totals. */
enum {
    EFGS_STAGE_PREPROCESS_FORWARD = 0, /* hipRTC preprocess (projection, culling, appearance, MLP) */
    EFGS_STAGE_COMPACT = 1,            /* per-block count scan + index-ordered compaction with emission offsets */
    EFGS_STAGE_COUNTER_READ = 2,       /* (V, I) device-to-host read and stream synchronisation */
    EFGS_STAGE_CREATE_INSTANCES = 3,   /* (tile, primitive) instances at their emission slots, per-tile counts */
    EFGS_STAGE_TILE_OFFSETS = 4,       /* scan of the per-tile counts: tile ranges */
    EFGS_STAGE_TILE_BUCKETS = 5,       /* instances into their tiles' ranges */
    EFGS_STAGE_TILE_SORT = 6,          /* the tiles' ranges and the blends' tile order (the per-tile (depth, primitive)
                                          sort itself runs inside the forward blend, EFGS_STAGE_BLEND_FORWARD) */
    EFGS_STAGE_BLEND_FORWARD = 7,
    EFGS_STAGE_BLEND_BACKWARD = 8,
    EFGS_STAGE_PREPROCESS_BACKWARD = 9,
    EFGS_STAGE_MLP_REDUCE = 10,        /* reduction of the per-block MLP weight-gradient partials */
    EFGS_STAGE_MLP_BACKWARD = 11,      /* neural: MLP recompute + backward (EFGS_STAGE_PREPROCESS_BACKWARD is the rest) */
    EFGS_N_STAGES = 12
};
int efgs_set_stage_timing(efgs_rasterizer* r, int enable);
int efgs_get_stage_times(efgs_rasterizer* r, double* total_ms, int64_t* launches, int n_stages);

#ifdef __cplusplus
}
#endif

#endif /* EFGS_H */
