// C ABI (include/efgs.h): rasterizer configuration, forward / backward orchestration, Adam.
// Orchestration follows B/rasterization/src/forward.cu:11-246 and backward.cu:8-135 with this build's
// stages: preprocess (hipRTC) -> per-block counts scan -> index-ordered compaction -> one host read of
// (V, I) -> depth radix sort -> gathered scan of tile counts -> instance emission -> tile radix sort ->
// tile ranges -> blend; backward: blend replay -> preprocess backward (per-instance gradient reduction).
#include "../../include/efgs.h"

#include <chrono>
#include <cmath>
#include <cstring>
#include <mutex>
#include <sstream>
#include <string>
#include <vector>

#include "internal.h"
#include "rtc.h"

namespace efgs {

namespace {
thread_local std::string t_error;
}

void set_error(const std::string& msg) { t_error = msg; }
const char* error_message() { return t_error.c_str(); }

// Pairs of HIP events around pipeline stages, recorded on the launching stream while enabled; collect()
// waits for them and folds the elapsed times into per-stage totals. Events are pooled and reused.
class StageTimer {
  public:
    StageTimer() = default;
    StageTimer(const StageTimer&) = delete;
    StageTimer& operator=(const StageTimer&) = delete;
    ~StageTimer() {
        release(open_);
        for (const Pair& p : pending_) release(p);
        for (hipEvent_t e : pool_) (void)hipEventDestroy(e);
    }

    bool enable(bool on) {
        if (!collect()) return false;
        release(open_);
        open_ = Pair{};
        enabled_ = on;
        for (int i = 0; i < EFGS_N_STAGES; i++) {
            totals_[i] = 0.0;
            launches_[i] = 0;
        }
        return true;
    }

    void begin(int stage, hipStream_t s) {
        if (!enabled_) return;
        release(open_);
        open_ = Pair{stage, take(), take()};
        if (!open_.start || !open_.stop || hipEventRecord(open_.start, s) != hipSuccess) {
            release(open_);
            open_ = Pair{};
        }
    }

    void end(hipStream_t s) {
        if (!enabled_ || !open_.start) return;
        if (hipEventRecord(open_.stop, s) == hipSuccess) {
            pending_.push_back(open_);
        } else {
            release(open_);
        }
        open_ = Pair{};
        if (pending_.size() > max_pending) (void)collect();
    }

    bool collect() {
        bool ok = true;
        for (const Pair& p : pending_) {
            float ms = 0.0f;
            if (hipEventSynchronize(p.stop) == hipSuccess && hipEventElapsedTime(&ms, p.start, p.stop) == hipSuccess) {
                totals_[p.stage] += ms;
                launches_[p.stage] += 1;
            } else {
                ok = false;
            }
            release(p);
        }
        pending_.clear();
        if (!ok) set_error("waiting for the stage timing events failed");
        return ok;
    }

    double total_ms(int stage) const { return totals_[stage]; }
    int64_t launches(int stage) const { return launches_[stage]; }

  private:
    struct Pair {
        int stage = 0;
        hipEvent_t start = nullptr;
        hipEvent_t stop = nullptr;
    };
    static constexpr size_t max_pending = 1u << 14;

    hipEvent_t take() {
        if (!pool_.empty()) {
            hipEvent_t e = pool_.back();
            pool_.pop_back();
            return e;
        }
        hipEvent_t e = nullptr;
        return hipEventCreateWithFlags(&e, hipEventDefault) == hipSuccess ? e : nullptr;
    }
    void release(const Pair& p) {
        if (p.start) pool_.push_back(p.start);
        if (p.stop) pool_.push_back(p.stop);
    }

    bool enabled_ = false;
    Pair open_;
    std::vector<Pair> pending_;
    std::vector<hipEvent_t> pool_;
    double totals_[EFGS_N_STAGES] = {};
    int64_t launches_[EFGS_N_STAGES] = {};
};

}  // namespace efgs

using namespace efgs;

struct efgs_rasterizer {
    bool appearance_set = false;
    int model = -1;  // -1 until efgs_set_appearance
    int max_degree = 0;
    int base_act = 0;
    int res_act = 0;
    int color_act = 0;
    bool direction_gradient = false;
    bool mlp_set = false;
    int mlp_n_in = 0;
    int mlp_n_in_padded = 0;
    int mlp_n_neurons = 0;
    int mlp_n_hidden = 0;
    int mlp_n_frequencies = 0;
    int mlp_sh_mask = 0;
    int mlp_n_features = 0;
    bool mlp_base_input = false;
    uint32_t* host_counters = nullptr;      // pinned and mapped, n_counters entries, written by the counter scan
    uint32_t* host_counters_dev = nullptr;  // its device address
    uint32_t counter_seq = 0;               // sequence number of the last frame's counters (never 0 once set)

    // instance count of the last forward and the scene size it was for: sizes the next frame's instance
    // buffers before its counter readback
    uint32_t instance_hint = 0, hint_primitives = 0, hint_tiles = 0;
    efgs::StageTimer timer;
    // specialised preprocess kernels of the current configuration, per variant and direction (forward,
    // backward), for the device they were loaded on; cleared whenever the configuration changes
    struct KernelSlot {
        int device = -1;
        efgs::RtcKernel kernel;
        hipFunction_t mlp = nullptr;  // neural backward: the MLP kernel of the same module
    };
    KernelSlot kernels[6][2];
    KernelSlot decode;  // standalone neural decode: forward kernel + backward kernel (in `mlp`) of one module
    void clear_kernels() {
        for (auto& v : kernels)
            for (auto& k : v) k = KernelSlot{};
        decode = KernelSlot{};
    }
};

namespace {

constexpr size_t buffer_alignment = 256;

struct Carver {
    char* base;
    size_t offset = 0;
    template <typename T>
    T* take(uint64_t count) {
        offset = (offset + buffer_alignment - 1) & ~(buffer_alignment - 1);
        T* p = base ? reinterpret_cast<T*>(base + offset) : nullptr;
        offset += sizeof(T) * count;
        return p;
    }
    void* take_bytes(size_t bytes) { return take<char>(bytes); }
};

struct PrimitiveLayout {
    uint32_t* n_touched;
    uint32_t* depth_keys;
    PrimRecord* records;
    uint32_t* prim_offset;
    uint32_t* block_counts;
    uint32_t* block_key_ranges;
    uint32_t* block_offsets;
    uint32_t* counters;
    uint32_t* visible_prims;
    size_t bytes;

    static PrimitiveLayout carve(char* base, uint64_t n) {
        PrimitiveLayout l;
        Carver c{base};
        const uint64_t nn = n > 0 ? n : 1;
        const uint32_t blocks = div_up(nn, preprocess_block);
        l.n_touched = c.take<uint32_t>(nn);
        l.depth_keys = c.take<uint32_t>(nn);
        l.records = c.take<PrimRecord>(nn);
        l.prim_offset = c.take<uint32_t>(nn);
        l.block_counts = c.take<uint32_t>(2ull * blocks);
        l.block_key_ranges = c.take<uint32_t>(2ull * blocks);
        l.block_offsets = c.take<uint32_t>(2ull * blocks);
        l.counters = c.take<uint32_t>(n_counters);
        l.visible_prims = c.take<uint32_t>(nn);
        l.bytes = c.offset + buffer_alignment;
        return l;
    }
};

struct TileLayout {
    uint2* ranges;
    float* final_T;
    uint32_t* n_contrib;
    uint32_t* tile_max;
    uint32_t* totals;        // instances per tile
    uint32_t* local_start;   // tile start within its 64-tile block
    uint32_t* block_sums;    // instances per 64-tile block
    uint32_t* cursor;        // per-tile bucket cursor of the global-atomic path
    uint32_t* order_runs;    // per 64-tile block and size class: tiles, then the run's first position in the order
    uint32_t* order_rank;    // per tile: size class << 16 | rank in its block's run
    uint32_t* order;         // tile of each blend block, heaviest first
    size_t bytes;

    static TileLayout carve(char* base, uint32_t n_tiles) {
        TileLayout l;
        Carver c{base};
        l.ranges = c.take<uint2>(n_tiles);
        l.final_T = c.take<float>(static_cast<uint64_t>(n_tiles) * tile_pixels);
        l.n_contrib = c.take<uint32_t>(static_cast<uint64_t>(n_tiles) * tile_pixels);
        l.tile_max = c.take<uint32_t>(n_tiles);
        l.totals = c.take<uint32_t>(n_tiles);
        l.local_start = c.take<uint32_t>(n_tiles);
        l.block_sums = c.take<uint32_t>(div_up(n_tiles > 0 ? n_tiles : 1, 64));
        l.cursor = c.take<uint32_t>(n_tiles);
        l.order_runs = c.take<uint32_t>(static_cast<uint64_t>(div_up(n_tiles > 0 ? n_tiles : 1, 64)) * order_classes);
        l.order_rank = c.take<uint32_t>(n_tiles);
        l.order = c.take<uint32_t>(n_tiles);
        l.bytes = c.offset + buffer_alignment;
        return l;
    }
};

struct InstanceLayout {
    void* keys;              // tile key per emission slot
    uint32_t* inst_prim;     // primitive per emission slot
    uint32_t* local_rank;    // rank of each instance among its segment's instances of its tile | segment << 24
    uint32_t* table;         // per segment and tile: the tile's count in the earlier segments (rows for every segment)
    uint4* bucket;           // per tile slot: emission index, depth key, primitive, 0 (sort key: the low 8 bytes)
    uint32_t* sorted_inst;   // emission slots in (tile, depth, primitive) order
    void* sorted_keys;       // tile key of every sorted instance
    uint32_t* sorted_prim;   // primitive of every sorted instance
    size_t bytes;

    static InstanceLayout carve(char* base, uint64_t n_instances, int key_bytes, uint32_t n_tiles) {
        InstanceLayout l;
        Carver c{base};
        const uint64_t ni = n_instances > 0 ? n_instances : 1;
        const bool use_table = fused_binning_fits(n_tiles);
        l.keys = c.take_bytes(key_bytes * ni);
        l.inst_prim = c.take<uint32_t>(ni);
        l.local_rank = c.take<uint32_t>(use_table ? ni : 1);
        l.table = c.take<uint32_t>(use_table ? static_cast<uint64_t>(tile_hist_max_blocks) * n_tiles : 1);
        l.bucket = c.take<uint4>(ni);
        l.sorted_inst = c.take<uint32_t>(ni);
        l.sorted_keys = c.take_bytes(key_bytes * ni);
        l.sorted_prim = c.take<uint32_t>(ni);
        l.bytes = c.offset + buffer_alignment;
        return l;
    }
};

// instances the frame's instance buffers are laid out for (at least its instance count)
uint64_t instance_capacity(const efgs_frame& f) {
    return static_cast<uint64_t>(f.instance_capacity > f.n_instances ? f.instance_capacity : f.n_instances);
}

int fail(int code, const std::string& msg) {
    set_error(msg);
    return code;
}

const char* model_suffix(int model) {
    switch (model) {
        case 0: return "precomputed";
        case 1: return "sh";
        case 2: return "sv";
        case 3: return "nasg";
        case 4: return "nasgabor";
        case 5: return "neural";
    }
    return "unknown";
}

int n_units_of(const efgs_rasterizer* r, int model) {
    switch (model) {
        case 1: return (r->max_degree + 1) * (r->max_degree + 1) - 1;
        case 2:
        case 3:
        case 4: return r->max_degree;
        case 5: return r->mlp_n_features;
    }
    return 0;
}

struct MlpShape {
    uint32_t n_in_padded, n_neurons, n_hidden;
};

MlpShape mlp_shape(const efgs_rasterizer* r) {
    return MlpShape{static_cast<uint32_t>(r->mlp_n_in_padded), static_cast<uint32_t>(r->mlp_n_neurons), static_cast<uint32_t>(r->mlp_n_hidden)};
}

// fp16 weight count of the tcnn-flat layout [W0 n x in_pad][W_h n x n]*(L-1)[W_out 16 x n]
uint32_t mlp_params(const MlpShape& m) { return m.n_neurons * m.n_in_padded + (m.n_hidden - 1) * m.n_neurons * m.n_neurons + 16 * m.n_neurons; }

// fp16 weights W_l and W_l^T with rows padded by 8 halves, as laid out by the neural kernels in LDS
uint32_t mlp_weight_bytes(const MlpShape& m) {
    uint32_t halves = 0;
    for (uint32_t l = 0; l <= m.n_hidden; l++) {
        const uint32_t in = l == 0 ? m.n_in_padded : m.n_neurons;
        const uint32_t out = l == m.n_hidden ? 16u : m.n_neurons;
        halves += out * (in + 8) + in * (out + 8);
    }
    return (halves * 2 + 15) / 16 * 16;
}

// the forward's neural kernels (preprocess, decode): weights + 4 per-wave staging areas of 64 rows of
// (n_in_padded + 4) halves
uint32_t mlp_smem_forward(const MlpShape& m) { return mlp_weight_bytes(m) + 4 * 64 * (m.n_in_padded + 4) * 2; }

constexpr uint32_t max_dynamic_lds = 160 * 1024;  // gfx950: 160 KiB of LDS per block

// the backward's MLP kernels (preprocess, decode): weights + 4 per-wave staging areas of 64 rows of
// (n_in_padded + 4) floats; the whole area is reused for the fp32 block reduction of the weight gradients
uint32_t mlp_smem_backward(const MlpShape& m) {
    const uint32_t f = mlp_weight_bytes(m) + 4 * 64 * (m.n_in_padded + 4) * 4;
    const uint32_t red = mlp_params(m) * 4;
    return f > red ? f : red;
}

// preamble tokens and source files of the preprocess kernel `kind` ("forward" / "backward") for `model`
void kernel_source(const efgs_rasterizer* r, int model, const char* kind, std::string& name, std::string& preamble,
                   std::vector<std::string>& files) {
    name = std::string("preprocess_") + kind + "_" + model_suffix(model);
    const bool pre = model == 0;
    preamble = "#define EFGS_KERNEL_NAME " + name + "\n";
    preamble += "#define EFGS_MODEL " + std::to_string(model) + "\n";
    preamble += "#define EFGS_BASE_ACT " + std::to_string(pre ? 0 : r->base_act) + "\n";
    preamble += "#define EFGS_RES_ACT " + std::to_string(pre ? 0 : r->res_act) + "\n";
    preamble += "#define EFGS_COLOR_ACT " + std::to_string(pre ? 0 : r->color_act) + "\n";
    preamble += "#define EFGS_N_UNITS " + std::to_string(n_units_of(r, model)) + "u\n";
    preamble += "#define EFGS_DIRECTION_GRADIENT " + std::string(!pre && r->direction_gradient ? "1" : "0") + "\n";
    preamble += "#define EFGS_MLP_N_IN " + std::to_string(model == 5 ? r->mlp_n_in : 0) + "u\n";
    preamble += "#define EFGS_MLP_N_IN_PADDED " + std::to_string(model == 5 ? r->mlp_n_in_padded : 0) + "u\n";
    preamble += "#define EFGS_MLP_N_NEURONS " + std::to_string(model == 5 ? r->mlp_n_neurons : 0) + "u\n";
    preamble += "#define EFGS_MLP_N_HIDDEN " + std::to_string(model == 5 ? r->mlp_n_hidden : 0) + "u\n";
    preamble += "#define EFGS_N_FREQUENCIES " + std::to_string(model == 5 ? r->mlp_n_frequencies : 0) + "u\n";
    preamble += "#define EFGS_SH_DEGREE_MASK " + std::to_string(model == 5 ? r->mlp_sh_mask : 0) + "u\n";
    preamble += "#define EFGS_BASE_INPUT " + std::string(model == 5 && r->mlp_base_input ? "1" : "0") + "\n";
    files = {"efgs_common.h", "efgs_args.h", "residual_rows.h"};
    switch (model) {
        case 1: files.push_back("appearance_sh.h"); break;
        case 2: files.push_back("appearance_sv.h"); break;
        case 3:
        case 4: files.push_back("appearance_lobes.h"); break;
        case 5: files.push_back("appearance_neural.h"); break;
    }
    files.push_back(std::string("preprocess_") + kind + ".hip");
}

// preamble tokens and source files of the standalone neural decode module (the configured MLP and encoding)
void decode_source(const efgs_rasterizer* r, std::string& name, std::string& preamble, std::vector<std::string>& files) {
    std::string unused, full;
    kernel_source(r, 5, "forward", unused, full, files);
    name = "neural_decode";
    // the colour activations and the direction-gradient flag do not enter the decode: fixed tokens keep one
    // cached code object per MLP configuration
    preamble = "#define EFGS_KERNEL_NAME " + name + "\n";
    std::istringstream lines(full);
    std::string line;
    while (std::getline(lines, line)) {
        if (line.rfind("#define EFGS_KERNEL_NAME ", 0) == 0) continue;
        for (const char* token : {"EFGS_BASE_ACT ", "EFGS_RES_ACT ", "EFGS_COLOR_ACT ", "EFGS_DIRECTION_GRADIENT "})
            if (line.rfind(std::string("#define ") + token, 0) == 0) line = std::string("#define ") + token + "0";
        preamble += line + "\n";
    }
    files.back() = "neural_decode.hip";
}

bool get_decode_kernels(efgs_rasterizer* r, RtcKernel& forward, hipFunction_t& backward) {
    int device = 0;
    EFGS_HIP_CHECK(hipGetDevice(&device));
    efgs_rasterizer::KernelSlot& slot = r->decode;
    if (slot.device != device || !slot.kernel.function) {
        std::string name, preamble;
        std::vector<std::string> files;
        decode_source(r, name, preamble, files);
        RtcKernel loaded;
        if (!rtc_get_kernel(name, preamble, files, loaded)) return false;
        hipFunction_t bwd = nullptr;
        EFGS_HIP_CHECK(hipModuleGetFunction(&bwd, loaded.module, (name + "_backward").c_str()));
        slot.kernel = loaded;
        slot.mlp = bwd;
        slot.device = device;
    }
    forward = slot.kernel;
    backward = slot.mlp;
    return true;
}

// the specialised preprocess kernel (forward or backward) of `model`, compiled or loaded once per device and
// configuration; for the neural backward `mlp` receives the MLP kernel of the same module
bool get_preprocess_kernel(efgs_rasterizer* r, int model, const char* kind, RtcKernel& k, hipFunction_t* mlp = nullptr) {
    int device = 0;
    EFGS_HIP_CHECK(hipGetDevice(&device));
    const bool backward = kind[0] == 'b';
    efgs_rasterizer::KernelSlot& slot = r->kernels[model][backward ? 1 : 0];
    if (slot.device != device || !slot.kernel.function) {
        std::string name, preamble;
        std::vector<std::string> files;
        kernel_source(r, model, kind, name, preamble, files);
        RtcKernel loaded;
        if (!rtc_get_kernel(name, preamble, files, loaded)) return false;
        hipFunction_t extra = nullptr;
        if (backward && model == 5) EFGS_HIP_CHECK(hipModuleGetFunction(&extra, loaded.module, (name + "_mlp").c_str()));
        slot.kernel = loaded;
        slot.mlp = extra;
        slot.device = device;
    }
    k = slot.kernel;
    if (mlp) *mlp = slot.mlp;
    return true;
}


// persistent grids of the neural kernels: the preprocess forward in 2,048 blocks, two per resident slot (four blocks
// of 256 per CU): each block stages the MLP weights once and takes every 2,048th chunk, which balances the tail better
// than one block per slot (61.1 -> 59.4 us on 1M Gaussians at 1080p, twice); the decode forward, whose blocks do
// little besides the MLP, in 1,024; the backward in 512 blocks, one per slot of its two waves per SIMD, whose
// weight-gradient partials are reduced after it
constexpr uint32_t neural_forward_blocks = 2048;
constexpr uint32_t decode_forward_blocks = 1024;
constexpr uint32_t neural_backward_blocks = 512;

// threads per block of the non-neural preprocess backward of `model` (the kernel's backward_block)
uint32_t preprocess_backward_block(int model) { return model >= 1 && model <= 4 ? 128u : 256u; }

// 0 (precomputed colours) when colours are supplied, else the configured model; -1 if none is configured
int variant_of(const efgs_rasterizer* r, const efgs_primitives* prims) {
    if (prims->precomputed_colors != nullptr) return 0;
    return r->appearance_set ? r->model : -1;
}

int check_config(const efgs_rasterizer* r, const efgs_primitives* prims, int variant) {
    if (variant < 0 || (variant != 0 && !r->appearance_set))
        return fail(EFGS_ERR_STATE, "appearance model is not initialized (efgs_set_appearance)");
    if (variant == 0 && prims->n_primitives > 0 && !prims->precomputed_colors)
        return fail(EFGS_ERR_INVALID_ARGUMENT, "precomputed_colors are required by the precomputed-colour variant");
    if (variant == 5 && !r->mlp_set) return fail(EFGS_ERR_STATE, "residual mlp is not initialized (efgs_set_residual_mlp)");
    if (prims->n_primitives < 0 || prims->n_primitives >= (1ll << 31)) return fail(EFGS_ERR_INVALID_ARGUMENT, "n_primitives out of range");
    if (prims->n_primitives > 0) {
        if (!prims->means || !prims->scales || !prims->rotations || !prims->opacities)
            return fail(EFGS_ERR_INVALID_ARGUMENT, "means, scales, rotations and opacities are required");
        if (variant != 0 && !prims->base_colors) return fail(EFGS_ERR_INVALID_ARGUMENT, "base_colors are required by the appearance model");
        if (variant != 0 && n_units_of(r, variant) > 0 && !prims->residual_params)
            return fail(EFGS_ERR_INVALID_ARGUMENT, "residual_params are required by the appearance model");
        if (variant == 5 && !prims->mlp_weights) return fail(EFGS_ERR_INVALID_ARGUMENT, "mlp_weights are required by the neural model");
        if (variant == 5 && (reinterpret_cast<uintptr_t>(prims->mlp_weights) & 15u) != 0)
            return fail(EFGS_ERR_INVALID_ARGUMENT, "mlp_weights must be 16-byte aligned");
    }
    return EFGS_OK;
}

CameraArgs camera_args(const efgs_rasterizer* r, const efgs_settings* s, int variant, uint32_t grid_w, uint32_t grid_h) {
    CameraArgs c;
    c.w2c = s->w2c;
    c.cam_position = s->cam_position;
    c.width = static_cast<uint32_t>(s->width);
    c.height = static_cast<uint32_t>(s->height);
    c.grid_w = grid_w;
    c.grid_h = grid_h;
    c.focal_x = s->focal_x;
    c.focal_y = s->focal_y;
    c.center_x = s->center_x;
    c.center_y = s->center_y;
    c.near_plane = s->near_plane;
    c.far_plane = s->far_plane;
    {
#pragma clang fp contract(off)
        // the operation sequence the kernels used to evaluate per primitive (IEEE fp32, so the same bits)
        const float wf = static_cast<float>(c.width), hf = static_cast<float>(c.height);
        const float l = -0.15f * wf - c.center_x, rr = 1.15f * wf - c.center_x;
        const float t = -0.15f * hf - c.center_y, b = 1.15f * hf - c.center_y;
        c.clip_left = l / c.focal_x;
        c.clip_right = rr / c.focal_x;
        c.clip_top = t / c.focal_y;
        c.clip_bottom = b / c.focal_y;
    }
    int degree = s->render_residual ? s->appearance_degree : 0;
    if (degree < 0) degree = 0;
    const int max_deg = variant == 5 ? 0 : r->max_degree;
    if (variant >= 1 && variant <= 4 && degree > max_deg) degree = max_deg;
    if (variant == 0) degree = 0;
    c.degree = static_cast<uint32_t>(degree);
    c.proper_aa = s->proper_antialiasing ? 1u : 0u;
    c.render_base = s->render_base ? 1u : 0u;
    c.pad_ = 0;
    return c;
}

bool launch_function(hipFunction_t f, uint32_t blocks, uint32_t threads, uint32_t shared_bytes, void* args, hipStream_t s) {
    void* params[] = {args};
    EFGS_HIP_CHECK(hipModuleLaunchKernel(f, blocks, 1, 1, threads, 1, 1, shared_bytes, s, params, nullptr));
    return true;
}

bool launch_rtc(const RtcKernel& k, uint32_t blocks, uint32_t threads, uint32_t shared_bytes, void* args, hipStream_t s) {
    return launch_function(k.function, blocks, threads, shared_bytes, args, s);
}

}  // namespace


extern "C" {

const char* efgs_last_error(void) { return error_message(); }

void* efgs_workspace_alloc(void* workspace, size_t bytes) {
    efgs_workspace* w = static_cast<efgs_workspace*>(workspace);
    if (!w) return nullptr;
    const size_t aligned = (bytes + buffer_alignment - 1) & ~(buffer_alignment - 1);
    w->requested += aligned;
    if (w->base && w->used + aligned <= w->capacity) {
        void* p = static_cast<char*>(w->base) + w->used;
        w->used += aligned;
        return p;
    }
    return w->fallback ? w->fallback(w->fallback_ctx, bytes) : nullptr;
}

int efgs_set_rtc_dirs(const char* cache_dir, const char* kernel_dir) {
    if (!kernel_dir) return fail(EFGS_ERR_INVALID_ARGUMENT, "kernel_dir is required");
    rtc_set_dirs(cache_dir ? cache_dir : "", kernel_dir);
    return EFGS_OK;
}

int efgs_rasterizer_create(efgs_rasterizer** out) {
    if (!out) return fail(EFGS_ERR_INVALID_ARGUMENT, "null output pointer");
    *out = new efgs_rasterizer();
    return EFGS_OK;
}

void efgs_rasterizer_destroy(efgs_rasterizer* r) {
    if (!r) return;
    if (r->host_counters) (void)hipHostFree(r->host_counters);
    delete r;
}

int efgs_set_appearance(efgs_rasterizer* r, int model, int max_degree, int base_act, int residual_act, int color_act, int direction_gradient) {
    if (!r) return fail(EFGS_ERR_INVALID_ARGUMENT, "null rasterizer");
    if (model < 1 || model > 5) return fail(EFGS_ERR_INVALID_ARGUMENT, "invalid appearance model id");
    if (base_act < 0 || base_act > 1) return fail(EFGS_ERR_INVALID_ARGUMENT, "invalid base activation id");
    if (residual_act < 0 || residual_act > 2) return fail(EFGS_ERR_INVALID_ARGUMENT, "invalid residual activation id");
    if (color_act < 0 || color_act > 5) return fail(EFGS_ERR_INVALID_ARGUMENT, "invalid color activation id");
    if (max_degree < 0 || (model == 1 && max_degree > 3)) return fail(EFGS_ERR_INVALID_ARGUMENT, "invalid max degree (sh supports 0..3)");
    r->clear_kernels();
    r->appearance_set = true;
    r->model = model;
    r->max_degree = model == 5 ? 0 : max_degree;
    r->base_act = base_act;
    r->res_act = residual_act;
    r->color_act = color_act;
    r->direction_gradient = direction_gradient != 0;
    r->mlp_set = false;
    return EFGS_OK;
}

int efgs_set_residual_mlp(efgs_rasterizer* r, int n_input_dims, int n_output_dims, int n_neurons, int n_hidden_layers, int hidden_activation,
                          int base_input, int n_frequencies, int sh_degree_mask) {
    if (!r) return fail(EFGS_ERR_INVALID_ARGUMENT, "null rasterizer");
    if (!r->appearance_set || r->model != 5)
        return fail(EFGS_ERR_STATE, "set_appearance must select the neural appearance model before set_residual_mlp");
    if (n_output_dims != 3) return fail(EFGS_ERR_INVALID_ARGUMENT, "the residual mlp must have 3 outputs");
    if (hidden_activation != 1) return fail(EFGS_ERR_INVALID_ARGUMENT, "only ReLU hidden activations are supported");
    if (n_neurons != 16 && n_neurons != 32 && n_neurons != 64 && n_neurons != 128)
        return fail(EFGS_ERR_INVALID_ARGUMENT, "n_neurons must be 16, 32, 64 or 128");
    if (n_hidden_layers < 1 || n_hidden_layers > 8) return fail(EFGS_ERR_INVALID_ARGUMENT, "n_hidden_layers must be in 1..8");
    if (n_frequencies < 0 || n_frequencies > 8) return fail(EFGS_ERR_INVALID_ARGUMENT, "n_frequencies must be in 0..8");
    if (sh_degree_mask < 0 || sh_degree_mask > 127) return fail(EFGS_ERR_INVALID_ARGUMENT, "sh degrees must lie in 0..6");
    int n_degree_dims = 0, max_degree = 0;
    for (int d = 0; d <= 6; d++) {
        if (sh_degree_mask & (1 << d)) {
            n_degree_dims += 2 * d + 1;
            if (d > 0) max_degree++;
        }
    }
    const int per_feature = n_frequencies > 0 ? 2 * n_frequencies : 1;
    if (n_input_dims <= n_degree_dims || (n_input_dims - n_degree_dims) % per_feature != 0)
        return fail(EFGS_ERR_INVALID_ARGUMENT, "n_input_dims does not match the feature encoding and the sh degrees");
    const int raw_features = (n_input_dims - n_degree_dims) / per_feature;
    const int features = raw_features - (base_input ? 3 : 0);
    if (features < 1) return fail(EFGS_ERR_INVALID_ARGUMENT, "no learned features left for the residual mlp");
    if (n_input_dims > 128) return fail(EFGS_ERR_INVALID_ARGUMENT, "n_input_dims above 128 is not supported");
    const MlpShape probe{static_cast<uint32_t>((n_input_dims + 15) / 16 * 16), static_cast<uint32_t>(n_neurons),
                         static_cast<uint32_t>(n_hidden_layers)};
    if (mlp_smem_backward(probe) > max_dynamic_lds || mlp_smem_forward(probe) > max_dynamic_lds)
        return fail(EFGS_ERR_INVALID_ARGUMENT, "the residual mlp exceeds the 160 KiB LDS budget of the fused kernels");
    r->clear_kernels();
    r->mlp_set = true;
    r->mlp_n_in = n_input_dims;
    r->mlp_n_in_padded = (n_input_dims + 15) / 16 * 16;
    r->mlp_n_neurons = n_neurons;
    r->mlp_n_hidden = n_hidden_layers;
    r->mlp_n_frequencies = n_frequencies;
    r->mlp_sh_mask = sh_degree_mask;
    r->mlp_n_features = features;
    r->mlp_base_input = base_input != 0;
    r->max_degree = max_degree;
    return EFGS_OK;
}

int64_t efgs_mlp_param_count(const efgs_rasterizer* r) {
    if (!r || !r->mlp_set) return 0;
    const int64_t n = r->mlp_n_neurons;
    return n * r->mlp_n_in_padded + (r->mlp_n_hidden - 1) * n * n + 16 * n;
}

namespace {

// The host's pinned, device-mapped copy of the counters (portable: one buffer serves every device).
int prepare_counters(efgs_rasterizer* r) {
    if (!r->host_counters) {
        void* host = nullptr;
        void* dev = nullptr;
        if (hipHostMalloc(&host, n_counters * sizeof(uint32_t), hipHostMallocMapped | hipHostMallocPortable | hipHostMallocCoherent) != hipSuccess)
            return fail(EFGS_ERR_HIP, "hipHostMalloc of the counter buffer failed");
        if (hipHostGetDevicePointer(&dev, host, 0) != hipSuccess) {
            (void)hipHostFree(host);
            return fail(EFGS_ERR_HIP, "hipHostGetDevicePointer of the counter buffer failed");
        }
        std::memset(host, 0, n_counters * sizeof(uint32_t));
        r->host_counters = static_cast<uint32_t*>(host);
        r->host_counters_dev = static_cast<uint32_t*>(dev);
    }
    return EFGS_OK;
}

// Waits until the counter scan of frame `seq` has written the host's copy of the counters: polls the sequence
// word (the scan writes it after the counters, behind a system-scope fence), for up to 20 ms, then waits for the
// stream to drain and looks once more, so an earlier failure on the stream is reported instead of waited on.
int wait_counters(efgs_rasterizer* r, uint32_t seq, hipStream_t s) {
    const uint32_t* word = &r->host_counters[counter_sequence];
    const auto t0 = std::chrono::steady_clock::now();
    for (uint32_t i = 0;; i++) {
        if (__atomic_load_n(word, __ATOMIC_ACQUIRE) == seq) return EFGS_OK;
        if ((i & 1023u) == 1023u && std::chrono::steady_clock::now() - t0 > std::chrono::milliseconds(20)) break;
        __builtin_ia32_pause();
    }
    if (const hipError_t e = hipStreamSynchronize(s); e != hipSuccess)
        return fail(EFGS_ERR_HIP, std::string("reading the visible/instance counters failed: ") + hipGetErrorString(e));
    if (__atomic_load_n(word, __ATOMIC_ACQUIRE) != seq) return fail(EFGS_ERR_HIP, "the counter scan did not write the counters");
    return EFGS_OK;
}

// The forward pipeline. A training forward (frame != null) keeps the backward state (final T, last contributors,
// tile maxima) and writes the image CHW; an inference render (frame == null) writes only the image, in CHW or
// HWC layout, optionally clamped.
int forward_impl(efgs_rasterizer* r, const efgs_primitives* prims, const efgs_settings* settings, float* image, efgs_alloc_fn alloc,
                 void* alloc_ctx, efgs_frame* frame, bool hwc, bool clamp, void* stream) {
    if (!r || !prims || !settings || !image || !alloc) return fail(EFGS_ERR_INVALID_ARGUMENT, "null argument");
    if (settings->width <= 0 || settings->height <= 0 || settings->width > 65535 || settings->height > 65535)
        return fail(EFGS_ERR_INVALID_ARGUMENT, "image size out of range");
    if (!settings->w2c || !settings->cam_position || !settings->bg_color) return fail(EFGS_ERR_INVALID_ARGUMENT, "camera tensors are required");
    const int variant = variant_of(r, prims);
    if (int c = check_config(r, prims, variant)) return c;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const uint32_t n = static_cast<uint32_t>(prims->n_primitives);
    const uint32_t grid_w = div_up(settings->width, tile_width), grid_h = div_up(settings->height, tile_height);
    const uint32_t n_tiles = grid_w * grid_h;
    const int key_bytes = n_tiles <= 65535u ? 2 : 4;
    if (int c = prepare_counters(r)) return c;

    const PrimitiveLayout pl0 = PrimitiveLayout::carve(nullptr, n);
    char* pblob = static_cast<char*>(alloc(alloc_ctx, pl0.bytes));
    if (!pblob) return fail(EFGS_ERR_ALLOC, "allocation of the primitive buffers failed");
    const TileLayout tl0 = TileLayout::carve(nullptr, n_tiles);
    char* tblob = static_cast<char*>(alloc(alloc_ctx, tl0.bytes));
    if (!tblob) return fail(EFGS_ERR_ALLOC, "allocation of the tile buffers failed");
    const PrimitiveLayout pl = PrimitiveLayout::carve(pblob, n);
    const TileLayout tl = TileLayout::carve(tblob, n_tiles);
    const CameraArgs cam = camera_args(r, settings, variant, grid_w, grid_h);
    StageTimer& t = r->timer;
    // Instance buffers are laid out for `capacity` instances. With a count from the previous frame of this scene
    // size, everything after the counter scan is launched at once into buffers with 12.5 % headroom: the scan flags
    // a count above the capacity, the binning and blend kernels then return at once, and the host, which reads the
    // counters only after its last launch, re-runs them with exact buffers. Without one the host reads the
    // counters first.
    const bool speculate = n > 0 && r->instance_hint > 0 && r->hint_primitives == n && r->hint_tiles == n_tiles;
    uint64_t capacity = speculate ? static_cast<uint64_t>(r->instance_hint) + r->instance_hint / 8 + 1024 : 0;
    if (capacity > 0xfffffff0ull) capacity = 0xfffffff0ull;

    uint32_t seq = 0;
    const bool fused = n > 0 && fused_binning_fits(n_tiles);
    if (n > 0) {
        RtcKernel k;
        if (!get_preprocess_kernel(r, variant, "forward", k)) return EFGS_ERR_RTC;
        PreprocessForwardArgs a;
        std::memset(&a, 0, sizeof(a));
        a.means = prims->means;
        a.scales = prims->scales;
        a.rotations = prims->rotations;
        a.opacities = prims->opacities;
        a.precomputed = prims->precomputed_colors;
        a.base = prims->base_colors;
        a.residual = prims->residual_params;
        a.mlp_weights = prims->mlp_weights;
        a.n_touched = pl.n_touched;
        a.depth_keys = pl.depth_keys;
        a.records = pl.records;
        a.block_counts = pl.block_counts;
        a.block_key_ranges = pl.block_key_ranges;
        a.counters = pl.counters;
        a.n = n;
        a.cam = cam;
        const uint32_t chunks = div_up(n, preprocess_block);
        const uint32_t blocks = variant == 5 ? (chunks < neural_forward_blocks ? chunks : neural_forward_blocks) : chunks;
        const uint32_t shared = variant == 5 ? mlp_smem_forward(mlp_shape(r)) : 0u;
        t.begin(EFGS_STAGE_PREPROCESS_FORWARD, s);
        if (!launch_rtc(k, blocks, preprocess_block, shared, &a, s)) return EFGS_ERR_HIP;
        t.end(s);
        // The counter scan writes the counters to the pinned host buffer as well, then the frame's sequence number.
        // With the fused emission (grids whose histogram fits) the emission kernel does the scan and the compaction
        // itself; the scan still runs before a first frame, whose buffers wait for the counts. (The stage is timed
        // only when it launches a kernel.)
        seq = ++r->counter_seq == 0 ? ++r->counter_seq : r->counter_seq;
        const bool scan = !speculate || !fused;
        if (scan || !fused) t.begin(EFGS_STAGE_COMPACT, s);
        if (scan)
            if (!launch_scan_block_counts(pl.block_counts, pl.block_key_ranges, pl.block_offsets, pl.counters, r->host_counters_dev,
                                          speculate ? static_cast<uint32_t>(capacity) : 0xffffffffu, seq, chunks, s))
                return EFGS_ERR_HIP;
        if (!fused && !launch_compact_visible(pl.n_touched, pl.block_offsets, pl.visible_prims, pl.prim_offset, n, s)) return EFGS_ERR_HIP;
        if (scan || !fused) t.end(s);
    } else {
        if (!launch_fill_u32(pl.counters, 0u, n_counters, s)) return EFGS_ERR_HIP;
    }

    // Instance binning and the blend, into instance buffers laid out for `cap` instances (max_visible /
    // max_instances: bounds on the counts, the grid sizes).
    InstanceLayout il{};
    const auto bin_and_blend = [&](char* iblob, uint64_t cap, uint32_t max_visible, uint32_t max_instances) -> int {
        il = InstanceLayout::carve(iblob, cap, key_bytes, n_tiles);
        FusedBinningArgs fa{};
        const TileBinning plan = fused ? fused_binning_plan(n, n_tiles, fa.chunks_per_segment) : TileBinning{false, 0u, 1u};
        fa.block_counts = pl.block_counts;
        fa.key_ranges = pl.block_key_ranges;
        fa.host_counters = r->host_counters_dev;
        fa.n_prims = n;
        fa.n_chunks = div_up(n, preprocess_block);
        fa.capacity = static_cast<uint32_t>(cap);
        fa.seq = seq;
        CreateInstancesArgs ca;
        ca.visible_prims = pl.visible_prims;
        ca.prim_offset = pl.prim_offset;
        ca.visible_prims_out = pl.visible_prims;
        ca.prim_offset_out = pl.prim_offset;
        ca.n_touched = pl.n_touched;
        ca.records = pl.records;
        ca.keys = il.keys;
        ca.inst_prim = il.inst_prim;
        ca.counters = pl.counters;
        ca.grid_w = grid_w;
        ca.max_visible = max_visible;
        ca.n_visible = 0;
        t.begin(EFGS_STAGE_CREATE_INSTANCES, s);
        if (!launch_create_instances(ca, key_bytes, plan, il.local_rank, il.table, n_tiles, fused ? &fa : nullptr, s)) return EFGS_ERR_HIP;
        t.end(s);
        const TileScan ts{tl.totals, tl.local_start, tl.block_sums, tl.cursor, tl.order_runs, tl.order_rank, tl.order, pl.counters};
        t.begin(EFGS_STAGE_TILE_OFFSETS, s);
        if (!launch_tile_counts(plan, il.keys, key_bytes, max_instances, il.table, ts, n_tiles, s)) return EFGS_ERR_HIP;
        t.end(s);
        t.begin(EFGS_STAGE_TILE_BUCKETS, s);
        if (!launch_tile_buckets(plan, il.keys, key_bytes, il.inst_prim, pl.depth_keys, il.table, il.local_rank, ts, il.bucket, max_instances,
                                 n_tiles, s))
            return EFGS_ERR_HIP;
        t.end(s);
        t.begin(EFGS_STAGE_TILE_SORT, s);
        if (!launch_tile_ranges(ts, tl.ranges, n_tiles, s)) return EFGS_ERR_HIP;
        t.end(s);

        BlendForwardArgs b;
        b.ranges = tl.ranges;
        b.bucket = il.bucket;
        b.sorted_inst = il.sorted_inst;
        b.sorted_prim = il.sorted_prim;
        b.sorted_keys = il.sorted_keys;
        b.inst_prim = il.inst_prim;
        b.counters = pl.counters;
        b.key_bytes = static_cast<uint32_t>(key_bytes);
        b.records = pl.records;
        b.bg = settings->bg_color;
        b.image = image;
        b.final_T = tl.final_T;
        b.n_contrib = tl.n_contrib;
        b.tile_max = tl.tile_max;
        b.order = tl.order;
        b.overflow = pl.counters + counter_overflow;
        b.width = static_cast<uint32_t>(settings->width);
        b.height = static_cast<uint32_t>(settings->height);
        b.grid_w = grid_w;
        b.n_tiles = n_tiles;
        b.hwc = hwc ? 1u : 0u;
        b.clamp = clamp ? 1u : 0u;
        if (!frame) b.final_T = nullptr;
        t.begin(EFGS_STAGE_BLEND_FORWARD, s);
        if (!launch_blend_forward(b, s)) return EFGS_ERR_HIP;
        t.end(s);
        return EFGS_OK;
    };

    char* iblob = nullptr;
    if (speculate) {
        iblob = static_cast<char*>(alloc(alloc_ctx, InstanceLayout::carve(nullptr, capacity, key_bytes, n_tiles).bytes));
        if (!iblob) return fail(EFGS_ERR_ALLOC, "allocation of the instance buffers failed");
        if (int c = bin_and_blend(iblob, capacity, n, static_cast<uint32_t>(capacity))) return c;
    }
    t.begin(EFGS_STAGE_COUNTER_READ, s);
    if (n > 0) {
        if (int c = wait_counters(r, seq, s)) return c;
    }
    t.end(s);
    const uint32_t n_visible = n > 0 ? __atomic_load_n(&r->host_counters[0], __ATOMIC_ACQUIRE) : 0u;
    const uint32_t n_instances = n > 0 ? __atomic_load_n(&r->host_counters[1], __ATOMIC_ACQUIRE) : 0u;
    // instance indices are signed 32-bit in the reference (B/rasterization/src/forward.cu:107-221); the emission
    // slots, ranges and records here are unsigned 32-bit indices with 64-bit byte offsets
    if (n_instances > 0x7fffffffu) return fail(EFGS_ERR_INVALID_ARGUMENT, "more than 2^31 - 1 tile instances in one frame");
    r->instance_hint = n_instances;
    r->hint_primitives = n;
    r->hint_tiles = n_tiles;
    if (!speculate || n_instances > capacity) {
        // first frame of this scene size, or more instances than the speculative buffers hold (the device skipped
        // the binning and the blend): exact buffers, with the overflow flag cleared
        if (speculate && !launch_fill_u32(pl.counters + counter_overflow, 0u, 1, s)) return EFGS_ERR_HIP;
        capacity = n_instances;
        iblob = static_cast<char*>(alloc(alloc_ctx, InstanceLayout::carve(nullptr, capacity, key_bytes, n_tiles).bytes));
        if (!iblob) return fail(EFGS_ERR_ALLOC, "allocation of the instance buffers failed");
        if (int c = bin_and_blend(iblob, capacity, n_visible, n_instances)) return c;
    }
    if (!frame) return EFGS_OK;

    frame->primitive_buffers = pblob;
    frame->tile_buffers = tblob;
    frame->instance_buffers = iblob;
    frame->n_primitives = n;
    frame->n_visible = n_visible;
    frame->n_instances = n_instances;
    frame->instance_capacity = static_cast<int64_t>(capacity);
    frame->grid_width = static_cast<int32_t>(grid_w);
    frame->grid_height = static_cast<int32_t>(grid_h);
    frame->key_bytes = key_bytes;
    frame->model = variant;
    return EFGS_OK;
}

}  // namespace

int efgs_forward(efgs_rasterizer* r, const efgs_primitives* prims, const efgs_settings* settings, float* image, efgs_alloc_fn alloc,
                 void* alloc_ctx, efgs_frame* frame, void* stream) {
    if (!frame) return fail(EFGS_ERR_INVALID_ARGUMENT, "null frame");
    return forward_impl(r, prims, settings, image, alloc, alloc_ctx, frame, false, false, stream);
}

int efgs_render(efgs_rasterizer* r, const efgs_primitives* prims, const efgs_settings* settings, float* image, int to_chw, int clamp_output,
                efgs_alloc_fn alloc, void* alloc_ctx, void* stream) {
    return forward_impl(r, prims, settings, image, alloc, alloc_ctx, nullptr, to_chw == 0, clamp_output != 0, stream);
}

int efgs_backward(efgs_rasterizer* r, const efgs_primitives* prims, const efgs_settings* settings, const efgs_frame* frame, const float* image,
                  const float* grad_image, efgs_gradients* grads, efgs_alloc_fn alloc, void* alloc_ctx, void* stream) {
    if (!r || !prims || !settings || !frame || !image || !grad_image || !grads || !alloc)
        return fail(EFGS_ERR_INVALID_ARGUMENT, "null argument");
    const int variant = frame->model;
    if (variant != variant_of(r, prims)) return fail(EFGS_ERR_INVALID_ARGUMENT, "inputs do not match the forward frame");
    if (int c = check_config(r, prims, variant)) return c;
    if (prims->n_primitives != frame->n_primitives) return fail(EFGS_ERR_INVALID_ARGUMENT, "primitive count differs from the forward frame");
    if (grads->densification_rows != 0 && grads->densification_rows != 2 && grads->densification_rows != 3)
        return fail(EFGS_ERR_INVALID_ARGUMENT, "densification_rows must be 0, 2 or 3");
    const uint32_t n = static_cast<uint32_t>(frame->n_primitives);
    if (n == 0) return EFGS_OK;
    if (!grads->means || !grads->scales || !grads->rotations || !grads->opacities)
        return fail(EFGS_ERR_INVALID_ARGUMENT, "geometry gradient outputs are required");
    if (variant == 0 && !grads->precomputed_colors) return fail(EFGS_ERR_INVALID_ARGUMENT, "precomputed colour gradient output is required");
    if (variant != 0 && !grads->base_colors) return fail(EFGS_ERR_INVALID_ARGUMENT, "base colour gradient output is required");
    if (variant != 0 && n_units_of(r, variant) > 0 && !grads->residual_params)
        return fail(EFGS_ERR_INVALID_ARGUMENT, "residual parameter gradient output is required");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const uint32_t grid_w = static_cast<uint32_t>(frame->grid_width), grid_h = static_cast<uint32_t>(frame->grid_height);
    const uint32_t n_tiles = grid_w * grid_h;
    const uint32_t n_instances = static_cast<uint32_t>(frame->n_instances);
    const PrimitiveLayout pl = PrimitiveLayout::carve(static_cast<char*>(frame->primitive_buffers), n);
    const TileLayout tl = TileLayout::carve(static_cast<char*>(frame->tile_buffers), n_tiles);
    const InstanceLayout il = InstanceLayout::carve(static_cast<char*>(frame->instance_buffers), instance_capacity(*frame), frame->key_bytes, n_tiles);
    const uint32_t* sorted_inst = il.sorted_inst;

    const size_t grad_bytes = static_cast<size_t>(n_instances > 0 ? n_instances : 1) *
                              (grads->densification_rows > 2 ? record_floats_abs : record_floats) * sizeof(float);
    float* inst_grads = static_cast<float*>(alloc(alloc_ctx, grad_bytes));
    if (!inst_grads) return fail(EFGS_ERR_ALLOC, "allocation of the instance gradient buffer failed");

    BlendBackwardArgs b;
    b.ranges = tl.ranges;
    b.sorted_inst = sorted_inst;
    b.sorted_prim = il.sorted_prim;
    b.records = pl.records;
    b.bg = settings->bg_color;
    b.image = image;
    b.grad_image = grad_image;
    b.final_T = tl.final_T;
    b.n_contrib = tl.n_contrib;
    b.tile_max = tl.tile_max;
    b.order = tl.order;
    b.inst_grads = inst_grads;
    b.width = static_cast<uint32_t>(settings->width);
    b.height = static_cast<uint32_t>(settings->height);
    b.grid_w = grid_w;
    b.n_tiles = n_tiles;
    b.abs_grads = grads->densification_rows > 2 ? 1u : 0u;
    StageTimer& t = r->timer;
    t.begin(EFGS_STAGE_BLEND_BACKWARD, s);
    if (!launch_blend_backward(b, s)) return EFGS_ERR_HIP;
    t.end(s);

    RtcKernel k;
    hipFunction_t mlp_kernel = nullptr;
    if (!get_preprocess_kernel(r, variant, "backward", k, &mlp_kernel)) return EFGS_ERR_RTC;
    PreprocessBackwardArgs a;
    std::memset(&a, 0, sizeof(a));
    a.means = prims->means;
    a.scales = prims->scales;
    a.rotations = prims->rotations;
    a.opacities = prims->opacities;
    a.base = prims->base_colors;
    a.residual = prims->residual_params;
    a.mlp_weights = prims->mlp_weights;
    a.n_touched = pl.n_touched;
    a.prim_offset = pl.prim_offset;
    a.records = pl.records;
    a.inst_grads = inst_grads;
    a.g_means = grads->means;
    a.g_scales = grads->scales;
    a.g_rotations = grads->rotations;
    a.g_opacities = grads->opacities;
    a.g_precomputed = grads->precomputed_colors;
    a.g_base = grads->base_colors;
    a.g_residual = grads->residual_params;
    a.densification_info = grads->densification_rows > 0 ? grads->densification_info : nullptr;
    a.densification_rows = static_cast<uint32_t>(grads->densification_rows);
    a.n = n;
    a.cam = camera_args(r, settings, variant, grid_w, grid_h);
    const uint32_t chunks = div_up(n, preprocess_block);
    if (variant != 5) {
        const uint32_t bb = preprocess_backward_block(variant);
        t.begin(EFGS_STAGE_PREPROCESS_BACKWARD, s);
        if (!launch_rtc(k, div_up(n, bb), bb, 0u, &a, s)) return EFGS_ERR_HIP;
        t.end(s);
        return EFGS_OK;
    }
    if (!grads->mlp_weights) return fail(EFGS_ERR_INVALID_ARGUMENT, "mlp weight gradient output is required");
    const uint32_t params = mlp_params(mlp_shape(r));
    float* color_grads = static_cast<float*>(alloc(alloc_ctx, static_cast<size_t>(n) * 4 * sizeof(float) + static_cast<size_t>(chunks) * 4));
    if (!color_grads) return fail(EFGS_ERR_ALLOC, "allocation of the colour gradient buffer failed");
    a.color_grads = color_grads;
    a.color_grad_max = reinterpret_cast<uint32_t*>(color_grads + static_cast<size_t>(n) * 4);  // one entry per geometry block
    t.begin(EFGS_STAGE_PREPROCESS_BACKWARD, s);
    if (!launch_rtc(k, chunks, preprocess_block, 0u, &a, s)) return EFGS_ERR_HIP;
    t.end(s);
    if (a.cam.degree == 0) {  // the residual is off: no MLP gradient
        if (!launch_fill_u32(reinterpret_cast<uint32_t*>(grads->mlp_weights), 0u, params, s)) return EFGS_ERR_HIP;
        return EFGS_OK;
    }
    const uint32_t blocks = chunks < neural_backward_blocks ? chunks : neural_backward_blocks;
    float* partials = static_cast<float*>(alloc(alloc_ctx, static_cast<size_t>(blocks) * params * sizeof(float)));
    if (!partials) return fail(EFGS_ERR_ALLOC, "allocation of the mlp gradient partials failed");
    a.g_mlp_partials = partials;
    a.visible_prims = pl.visible_prims;
    a.n_visible = frame->n_visible;
    t.begin(EFGS_STAGE_MLP_BACKWARD, s);
    if (!launch_function(mlp_kernel, blocks, preprocess_block, mlp_smem_backward(mlp_shape(r)), &a, s)) return EFGS_ERR_HIP;
    t.end(s);
    t.begin(EFGS_STAGE_MLP_REDUCE, s);
    if (!launch_reduce_partials(partials, blocks, params, grads->mlp_weights, s)) return EFGS_ERR_HIP;
    t.end(s);
    return EFGS_OK;
}

int efgs_adam_step(const efgs_adam_group* groups, int n_groups, void* stream) {
    if (n_groups < 0 || (n_groups > 0 && !groups)) return fail(EFGS_ERR_INVALID_ARGUMENT, "invalid adam groups");
    std::vector<AdamGroupDevice> dev(static_cast<size_t>(n_groups));
    for (int g = 0; g < n_groups; g++) {
        const efgs_adam_group& in = groups[g];
        if (in.n_lrs < 1 || in.n_lrs > adam_max_lrs) return fail(EFGS_ERR_INVALID_ARGUMENT, "between 1 and 7 learning rates are supported");
        if (in.step < 1) return fail(EFGS_ERR_INVALID_ARGUMENT, "adam step counts from 1");
        if (in.n_elements < 0) return fail(EFGS_ERR_INVALID_ARGUMENT, "negative element count");
        if (in.n_elements > 0 && (!in.grad || !in.param || !in.exp_avg || !in.exp_avg_sq))
            return fail(EFGS_ERR_INVALID_ARGUMENT, "null adam tensor");
        AdamGroupDevice& d = dev[g];
        d.grad = in.grad;
        d.param = in.param;
        d.m = in.exp_avg;
        d.v = in.exp_avg_sq;
        d.n = static_cast<uint64_t>(in.n_elements);
        const double bc1_rcp = 1.0 / (1.0 - std::pow(in.beta1, static_cast<double>(in.step)));
        const double bc2_sqrt_rcp = 1.0 / std::sqrt(1.0 - std::pow(in.beta2, static_cast<double>(in.step)));
        for (int k = 0; k < adam_max_lrs; k++) d.step_sizes[k] = k < in.n_lrs ? static_cast<float>(in.lrs[k] * bc1_rcp) : 0.0f;
        d.n_lrs = in.n_lrs;
        d.beta1 = static_cast<float>(in.beta1);
        d.beta2 = static_cast<float>(in.beta2);
        d.eps = static_cast<float>(in.eps);
        d.bc2_sqrt_rcp = static_cast<float>(bc2_sqrt_rcp);
        d.first_block = 0;
    }
    if (!launch_adam(dev.data(), n_groups, static_cast<hipStream_t>(stream))) return EFGS_ERR_HIP;
    return EFGS_OK;
}

int efgs_update_pruning_scores(efgs_rasterizer* r, const efgs_primitives* prims, const efgs_settings* settings, float* scores,
                               efgs_alloc_fn alloc, void* alloc_ctx, void* stream) {
    if (!r || !prims || !settings || !alloc || (prims->n_primitives > 0 && !scores)) return fail(EFGS_ERR_INVALID_ARGUMENT, "null argument");
    if (settings->width <= 0 || settings->height <= 0 || settings->width > 65535 || settings->height > 65535)
        return fail(EFGS_ERR_INVALID_ARGUMENT, "image size out of range");
    const size_t image_bytes = static_cast<size_t>(settings->width) * static_cast<size_t>(settings->height) * 3 * sizeof(float);
    float* image = static_cast<float*>(alloc(alloc_ctx, image_bytes));
    if (!image) return fail(EFGS_ERR_ALLOC, "allocation of the score pass image failed");
    efgs_frame frame;
    if (int rc = forward_impl(r, prims, settings, image, alloc, alloc_ctx, &frame, false, false, stream)) return rc;
    const uint32_t n = static_cast<uint32_t>(frame.n_primitives);
    if (n == 0 || frame.n_instances == 0) return EFGS_OK;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const uint32_t grid_w = static_cast<uint32_t>(frame.grid_width), grid_h = static_cast<uint32_t>(frame.grid_height);
    const uint32_t n_tiles = grid_w * grid_h;
    const uint32_t n_instances = static_cast<uint32_t>(frame.n_instances);
    const PrimitiveLayout pl = PrimitiveLayout::carve(static_cast<char*>(frame.primitive_buffers), n);
    const TileLayout tl = TileLayout::carve(static_cast<char*>(frame.tile_buffers), n_tiles);
    const InstanceLayout il = InstanceLayout::carve(static_cast<char*>(frame.instance_buffers), instance_capacity(frame), frame.key_bytes, n_tiles);
    float* inst_scores = static_cast<float*>(alloc(alloc_ctx, static_cast<size_t>(n_instances) * sizeof(float)));
    if (!inst_scores) return fail(EFGS_ERR_ALLOC, "allocation of the instance score buffer failed");
    BlendBackwardArgs b;
    std::memset(&b, 0, sizeof(b));
    b.ranges = tl.ranges;
    b.sorted_inst = il.sorted_inst;
    b.sorted_prim = il.sorted_prim;
    b.records = pl.records;
    b.bg = settings->bg_color;
    b.image = image;
    b.final_T = tl.final_T;
    b.n_contrib = tl.n_contrib;
    b.tile_max = tl.tile_max;
    b.order = tl.order;
    b.inst_grads = inst_scores;
    b.width = static_cast<uint32_t>(settings->width);
    b.height = static_cast<uint32_t>(settings->height);
    b.grid_w = grid_w;
    b.n_tiles = n_tiles;
    if (!launch_pruning_scores(b, pl.n_touched, pl.prim_offset, scores, n, s)) return EFGS_ERR_HIP;
    return EFGS_OK;
}

int efgs_add_noise(int64_t n, const float* raw_scales, const float* raw_rotations, const float* raw_opacities, float* means, float current_lr,
                   uint64_t seed, uint64_t offset, void* stream) {
    if (n < 0 || n > static_cast<int64_t>(UINT32_MAX)) return fail(EFGS_ERR_INVALID_ARGUMENT, "primitive count out of range");
    if (n > 0 && (!raw_scales || !raw_rotations || !raw_opacities || !means)) return fail(EFGS_ERR_INVALID_ARGUMENT, "null tensor");
    if (offset % 4 != 0) return fail(EFGS_ERR_INVALID_ARGUMENT, "the philox offset must be a multiple of 4");
    if (!launch_add_noise(raw_scales, raw_rotations, raw_opacities, means, static_cast<uint32_t>(n), current_lr, seed, offset,
                          static_cast<hipStream_t>(stream)))
        return EFGS_ERR_HIP;
    return EFGS_OK;
}

int efgs_relocation_adjustment(int64_t n, const float* old_opacities, const float* old_scales, const int64_t* n_samples_per_primitive,
                               float* new_opacities, float* new_scales, void* stream) {
    if (n < 0 || n > static_cast<int64_t>(UINT32_MAX)) return fail(EFGS_ERR_INVALID_ARGUMENT, "primitive count out of range");
    if (n > 0 && (!old_opacities || !old_scales || !n_samples_per_primitive || !new_opacities || !new_scales))
        return fail(EFGS_ERR_INVALID_ARGUMENT, "null tensor");
    if (!launch_relocation(old_opacities, old_scales, n_samples_per_primitive, new_opacities, new_scales, static_cast<uint32_t>(n),
                           static_cast<hipStream_t>(stream)))
        return EFGS_ERR_HIP;
    return EFGS_OK;
}

int efgs_set_stage_timing(efgs_rasterizer* r, int enable) {
    if (!r) return fail(EFGS_ERR_INVALID_ARGUMENT, "null rasterizer");
    return r->timer.enable(enable != 0) ? EFGS_OK : EFGS_ERR_HIP;
}

int efgs_get_stage_times(efgs_rasterizer* r, double* total_ms, int64_t* launches, int n_stages) {
    if (!r || n_stages < 0 || (n_stages > 0 && (!total_ms || !launches))) return fail(EFGS_ERR_INVALID_ARGUMENT, "invalid argument");
    if (!r->timer.collect()) return EFGS_ERR_HIP;
    for (int i = 0; i < n_stages; i++) {
        total_ms[i] = i < EFGS_N_STAGES ? r->timer.total_ms(i) : 0.0;
        launches[i] = i < EFGS_N_STAGES ? r->timer.launches(i) : 0;
    }
    return EFGS_OK;
}

int efgs_get_frame_views(const efgs_frame* frame, efgs_frame_views* v) {
    if (!frame || !v) return fail(EFGS_ERR_INVALID_ARGUMENT, "null argument");
    const uint32_t n = static_cast<uint32_t>(frame->n_primitives);
    const uint32_t n_tiles = static_cast<uint32_t>(frame->grid_width) * static_cast<uint32_t>(frame->grid_height);
    const PrimitiveLayout pl = PrimitiveLayout::carve(static_cast<char*>(frame->primitive_buffers), n);
    const TileLayout tl = TileLayout::carve(static_cast<char*>(frame->tile_buffers), n_tiles);
    const InstanceLayout il = InstanceLayout::carve(static_cast<char*>(frame->instance_buffers), instance_capacity(*frame), frame->key_bytes, n_tiles);
    v->n_touched = pl.n_touched;
    v->depth_keys = pl.depth_keys;
    v->records = reinterpret_cast<const float*>(pl.records);
    v->visible_prims = pl.visible_prims;
    v->prim_offset = pl.prim_offset;
    v->instance_keys = il.keys;
    v->instance_primitive = il.inst_prim;
    v->tile_sorted_keys = il.sorted_keys;
    v->tile_sorted_instances = il.sorted_inst;
    v->tile_ranges = reinterpret_cast<const uint32_t*>(tl.ranges);
    v->final_transmittance = tl.final_T;
    v->n_contributors = tl.n_contrib;
    v->counters = pl.counters;
    return EFGS_OK;
}

namespace {

int check_decode(const efgs_rasterizer* r, int64_t n, const float* features, const float* base, const float* dirs,
                 const uint16_t* mlp_weights, int degree) {
    if (!r) return fail(EFGS_ERR_INVALID_ARGUMENT, "null rasterizer");
    if (!r->appearance_set || r->model != 5 || !r->mlp_set)
        return fail(EFGS_ERR_STATE, "the neural decode needs the neural model and its residual mlp (efgs_set_residual_mlp)");
    if (n < 0 || n >= (1ll << 31)) return fail(EFGS_ERR_INVALID_ARGUMENT, "n out of range");
    if (degree < 0) return fail(EFGS_ERR_INVALID_ARGUMENT, "negative degree");
    if (n > 0) {
        // (directions are read only with SH degrees in the encoding)
        if ((r->mlp_sh_mask != 0 && !dirs) || !mlp_weights || (r->mlp_n_features > 0 && !features))
            return fail(EFGS_ERR_INVALID_ARGUMENT, "null input");
        if (r->mlp_base_input && !base) return fail(EFGS_ERR_INVALID_ARGUMENT, "base colours are required with base input");
        if ((reinterpret_cast<uintptr_t>(mlp_weights) & 15u) != 0) return fail(EFGS_ERR_INVALID_ARGUMENT, "mlp_weights must be 16-byte aligned");
    }
    return EFGS_OK;
}

NeuralDecodeArgs decode_args(int64_t n, const float* features, const float* base, const float* dirs, const uint16_t* mlp_weights, int degree) {
    NeuralDecodeArgs a;
    std::memset(&a, 0, sizeof(a));
    a.features = features;
    a.base = base;
    a.dirs = dirs;
    a.mlp_weights = mlp_weights;
    a.n = static_cast<uint32_t>(n);
    a.degree = static_cast<uint32_t>(degree);
    return a;
}

}  // namespace

int efgs_neural_decode_forward(efgs_rasterizer* r, int64_t n, const float* features, const float* base, const float* dirs,
                               const uint16_t* mlp_weights, int degree, float* out, void* stream) {
    if (int c = check_decode(r, n, features, base, dirs, mlp_weights, degree)) return c;
    if (n > 0 && !out) return fail(EFGS_ERR_INVALID_ARGUMENT, "null output");
    if (n == 0) return EFGS_OK;
    RtcKernel fwd;
    hipFunction_t bwd = nullptr;
    if (!get_decode_kernels(r, fwd, bwd)) return EFGS_ERR_RTC;
    NeuralDecodeArgs a = decode_args(n, features, base, dirs, mlp_weights, degree);
    a.out = out;
    const uint32_t chunks = div_up(static_cast<uint64_t>(n), preprocess_block);
    const uint32_t blocks = chunks < decode_forward_blocks ? chunks : decode_forward_blocks;
    if (!launch_rtc(fwd, blocks, preprocess_block, mlp_smem_forward(mlp_shape(r)), &a, static_cast<hipStream_t>(stream))) return EFGS_ERR_HIP;
    return EFGS_OK;
}

}  // extern "C"

// Weight-gradient partials of the allocation-free decode backward: one row of mlp_params floats per block of the
// backward kernel, 16 MiB on every device the library runs on, held until the process ends. In host code the name
// `scratch` is a stand-in, not a device address: the host uses only the per-device address that
// hipGetSymbolAddress returns (scratch_device_address), never the name.
constexpr size_t scratch_floats = size_t(4) << 20;
static __device__ __align__(256) float scratch[scratch_floats];

namespace {

constexpr int scratch_max_devices = 64;
std::mutex scratch_mutex;
float* scratch_address[scratch_max_devices] = {};

// The current device's copy of `scratch`, looked up once per device (with that device current) on the first call.
float* scratch_device_address(int device) {
    std::lock_guard<std::mutex> lock(scratch_mutex);
    if (!scratch_address[device]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            fail(EFGS_ERR_HIP, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
            return nullptr;
        }
        scratch_address[device] = static_cast<float*>(p);
    }
    return scratch_address[device];
}

// The decode backward with its partials in `partials` (room for `max_rows` rows of the MLP's parameter count); the
// block count is min(chunks, neural_backward_blocks, max_rows), so every row the reduction reads is written by the
// same launch (nothing has to start at zero).
int decode_backward(efgs_rasterizer* r, int64_t n, const float* features, const float* base, const float* dirs, const uint16_t* mlp_weights,
                    int degree, const float* grad_out, float* g_features, float* g_base, float* g_dirs, float* g_mlp_weights,
                    float* partials, uint32_t blocks, hipStream_t s) {
    RtcKernel fwd;
    hipFunction_t bwd = nullptr;
    if (!get_decode_kernels(r, fwd, bwd)) return EFGS_ERR_RTC;
    NeuralDecodeArgs a = decode_args(n, features, base, dirs, mlp_weights, degree);
    a.grad_out = grad_out;
    a.g_features = g_features;
    a.g_base = r->mlp_base_input ? g_base : nullptr;
    a.g_dirs = g_dirs;
    a.g_mlp_partials = partials;
    if (!launch_function(bwd, blocks, preprocess_block, mlp_smem_backward(mlp_shape(r)), &a, s)) return EFGS_ERR_HIP;
    if (!launch_reduce_partials(partials, blocks, mlp_params(mlp_shape(r)), g_mlp_weights, s)) return EFGS_ERR_HIP;
    return EFGS_OK;
}

int check_decode_backward(const efgs_rasterizer* r, int64_t n, const float* features, const float* base, const float* dirs,
                          const uint16_t* mlp_weights, int degree, const float* grad_out, const float* g_features, const float* g_mlp_weights) {
    if (int c = check_decode(r, n, features, base, dirs, mlp_weights, degree)) return c;
    if (!g_mlp_weights) return fail(EFGS_ERR_INVALID_ARGUMENT, "null weight gradient output");
    if (n > 0 && (!grad_out || (r->mlp_n_features > 0 && !g_features))) return fail(EFGS_ERR_INVALID_ARGUMENT, "null gradient argument");
    return EFGS_OK;
}

uint32_t decode_backward_blocks(int64_t n) {
    const uint32_t chunks = div_up(static_cast<uint64_t>(n), preprocess_block);
    return chunks < neural_backward_blocks ? chunks : neural_backward_blocks;
}

}  // namespace

extern "C" {

int efgs_neural_decode_backward(efgs_rasterizer* r, int64_t n, const float* features, const float* base, const float* dirs,
                                const uint16_t* mlp_weights, int degree, const float* grad_out, float* g_features, float* g_base,
                                float* g_dirs, float* g_mlp_weights, efgs_alloc_fn alloc, void* alloc_ctx, void* stream) {
    if (int c = check_decode_backward(r, n, features, base, dirs, mlp_weights, degree, grad_out, g_features, g_mlp_weights)) return c;
    if (!alloc) return fail(EFGS_ERR_INVALID_ARGUMENT, "null allocator");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const uint32_t params = mlp_params(mlp_shape(r));
    if (n == 0) return launch_fill_u32(reinterpret_cast<uint32_t*>(g_mlp_weights), 0u, params, s) ? EFGS_OK : EFGS_ERR_HIP;
    const uint32_t blocks = decode_backward_blocks(n);
    float* partials = static_cast<float*>(alloc(alloc_ctx, static_cast<size_t>(blocks) * params * sizeof(float)));
    if (!partials) return fail(EFGS_ERR_ALLOC, "allocation of the mlp gradient partials failed");
    return decode_backward(r, n, features, base, dirs, mlp_weights, degree, grad_out, g_features, g_base, g_dirs, g_mlp_weights, partials,
                           blocks, s);
}

int efgs_neural_decode_backward_no_alloc(efgs_rasterizer* r, int64_t n, const float* features, const float* base, const float* dirs,
                                         const uint16_t* mlp_weights, int degree, const float* grad_out, float* g_features,
                                         float* g_base, float* g_dirs, float* g_mlp_weights, void* stream) {
    if (int c = check_decode_backward(r, n, features, base, dirs, mlp_weights, degree, grad_out, g_features, g_mlp_weights)) return c;
    const uint32_t params = mlp_params(mlp_shape(r));
    if (params > scratch_floats)
        return fail(EFGS_ERR_INVALID_ARGUMENT, "the mlp's " + std::to_string(params) + " parameters exceed the static scratch of " +
                                                   std::to_string(scratch_floats) + " floats");
    int device = 0;
    if (const hipError_t e = hipGetDevice(&device); e != hipSuccess) return fail(EFGS_ERR_HIP, std::string("hipGetDevice: ") + hipGetErrorString(e));
    if (device < 0 || device >= scratch_max_devices) return fail(EFGS_ERR_INVALID_ARGUMENT, "device index beyond the scratch table");
    float* partials = scratch_device_address(device);
    if (!partials) return EFGS_ERR_HIP;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (n == 0) return launch_fill_u32(reinterpret_cast<uint32_t*>(g_mlp_weights), 0u, params, s) ? EFGS_OK : EFGS_ERR_HIP;
    const uint32_t rows = static_cast<uint32_t>(scratch_floats / params);
    const uint32_t blocks = decode_backward_blocks(n) < rows ? decode_backward_blocks(n) : rows;
    return decode_backward(r, n, features, base, dirs, mlp_weights, degree, grad_out, g_features, g_base, g_dirs, g_mlp_weights, partials,
                           blocks, s);
}

int efgs_precompile(const efgs_rasterizer* r, const char* arch) {
    if (!r || !arch) return fail(EFGS_ERR_INVALID_ARGUMENT, "null argument");
    std::vector<int> variants = {0};
    if (r->appearance_set && (r->model != 5 || r->mlp_set)) variants.push_back(r->model);
    for (int variant : variants) {
        for (const char* kind : {"forward", "backward"}) {
            std::string name, preamble;
            std::vector<std::string> files;
            kernel_source(r, variant, kind, name, preamble, files);
            if (!rtc_precompile(name, preamble, files, arch)) return EFGS_ERR_RTC;
        }
    }
    if (r->appearance_set && r->model == 5 && r->mlp_set) {
        std::string name, preamble;
        std::vector<std::string> files;
        decode_source(r, name, preamble, files);
        if (!rtc_precompile(name, preamble, files, arch)) return EFGS_ERR_RTC;
    }
    return EFGS_OK;
}

// ---- .ngsplat packing ------------------------------------------------------------------------------------------------

namespace {

struct NgsplatPlan {
    int payload, n_items, n_values, n_encoded, row_used, n_textures;
    uint32_t texel_words[ng_max_textures];
};

int ngsplat_plan(const efgs_ngsplat_input* in, NgsplatPlan& p) {
    if (!in) return fail(EFGS_ERR_INVALID_ARGUMENT, "null ngsplat input");
    p.payload = in->payload;
    p.n_items = in->n_items;
    p.n_encoded = 0;
    switch (in->payload) {
    case EFGS_NGSPLAT_NEURAL_FEATURES:
    case EFGS_NGSPLAT_NEURAL_BAKED: {
        if (in->n_items < 0 || in->n_frequencies < 0 || in->n_frequencies > 16) return fail(EFGS_ERR_INVALID_ARGUMENT, "invalid neural feature layout");
        const int raw = in->n_items + (in->base_input ? 3 : 0);
        p.n_encoded = raw * (in->n_frequencies ? 2 * in->n_frequencies : 1);
        p.row_used = in->n_items;
        if (in->payload == EFGS_NGSPLAT_NEURAL_FEATURES) {
            if (p.n_encoded < 1 || p.n_encoded > 16) return fail(EFGS_ERR_INVALID_ARGUMENT, "stored neural features need 1..16 encoded dims");
            p.n_values = p.n_encoded;
        } else {
            if (in->n_neurons < 1 || in->n_neurons > static_cast<int>(ng_max_baked))
                return fail(EFGS_ERR_INVALID_ARGUMENT, "a baked layer 0 needs 1..16 neurons");
            if (p.n_encoded < 1 || p.n_encoded > 256) return fail(EFGS_ERR_INVALID_ARGUMENT, "a baked layer 0 needs 1..256 encoded features");
            p.n_values = in->n_neurons;
        }
        break;
    }
    case EFGS_NGSPLAT_SH:
        if (in->n_items != 0 && in->n_items != 3 && in->n_items != 8 && in->n_items != 15)
            return fail(EFGS_ERR_INVALID_ARGUMENT, "SH export needs 0, 3, 8 or 15 coefficients (degrees up to 3)");
        p.row_used = 3 * in->n_items;
        p.n_values = 0;
        break;
    case EFGS_NGSPLAT_SV:
        if (in->n_items < 0 || in->n_items > 9) return fail(EFGS_ERR_INVALID_ARGUMENT, "SV export needs at most 9 sites (64 fp16 values)");
        p.row_used = 7 * in->n_items;
        p.n_values = 7 * in->n_items;
        break;
    case EFGS_NGSPLAT_NASG:
        if (in->n_items < 0 || in->n_items > 5) return fail(EFGS_ERR_INVALID_ARGUMENT, "NASG export needs at most 5 lobes (64 fp16 values)");
        p.row_used = 8 * in->n_items;
        p.n_values = 12 * in->n_items;
        break;
    case EFGS_NGSPLAT_NASGABOR:
        if (in->n_items < 0 || in->n_items > 4) return fail(EFGS_ERR_INVALID_ARGUMENT, "NASGabor export needs at most 4 lobes (64 fp16 values)");
        p.row_used = 9 * in->n_items;
        p.n_values = 13 * in->n_items;
        break;
    default: return fail(EFGS_ERR_INVALID_ARGUMENT, "unknown ngsplat payload");
    }
    if (p.row_used > static_cast<int>(ng_max_row)) return fail(EFGS_ERR_INVALID_ARGUMENT, "more than 63 residual parameters per splat");
    if (p.row_used > in->residual_row_stride) return fail(EFGS_ERR_INVALID_ARGUMENT, "residual row stride smaller than the parameters read");
    if (in->residual_act < 0 || in->residual_act > 2) return fail(EFGS_ERR_INVALID_ARGUMENT, "invalid residual activation");
    // the pack kernel stages 256 rows (stride row_used | 1) and, for a baked layer 0, the transposed matrix in LDS
    const size_t lds = sizeof(float) * ((p.row_used ? static_cast<size_t>(ng_block) * (static_cast<uint32_t>(p.row_used) | 1u) : 0) +
                                        (p.payload == EFGS_NGSPLAT_NEURAL_BAKED ? static_cast<size_t>(p.n_encoded) * ng_max_baked : 0));
    if (lds > 65536)
        return fail(EFGS_ERR_INVALID_ARGUMENT, "the per-splat parameters and the baked layer 0 need more than 64 KB of LDS per block");
    p.n_textures = ngsplat_texture_plan(p.payload, p.n_items, p.n_values, p.texel_words);
    return EFGS_OK;
}

}  // namespace

int efgs_ngsplat_layout(const efgs_ngsplat_input* in, int* n_textures, int* texel_words) {
    NgsplatPlan p;
    if (int rc = ngsplat_plan(in, p)) return rc;
    if (!n_textures || !texel_words) return fail(EFGS_ERR_INVALID_ARGUMENT, "null output");
    *n_textures = p.n_textures;
    for (int k = 0; k < static_cast<int>(ng_max_textures); k++) texel_words[k] = k < p.n_textures ? static_cast<int>(p.texel_words[k]) : 0;
    return EFGS_OK;
}

int efgs_ngsplat_pack(const efgs_ngsplat_input* in, efgs_ngsplat_output* out, efgs_alloc_fn alloc, void* alloc_ctx, void* stream) {
    NgsplatPlan p;
    if (int rc = ngsplat_plan(in, p)) return rc;
    if (!out || !alloc) return fail(EFGS_ERR_INVALID_ARGUMENT, "null output or allocator");
    if (in->n < 0 || in->n > (int64_t{1} << 31)) return fail(EFGS_ERR_INVALID_ARGUMENT, "splat count out of range");
    if (out->capacity < in->n || out->capacity % ng_tex_width != 0 || out->capacity > (int64_t{1} << 31))
        return fail(EFGS_ERR_INVALID_ARGUMENT, "output capacity must be a multiple of 2048 rows and hold every splat");
    if (out->capacity > 0 && (!out->splat_words || (p.n_textures > 0 && !out->params)))
        return fail(EFGS_ERR_INVALID_ARGUMENT, "null output texture");
    if (in->n > 0 && (!in->means || !in->raw_scales || !in->raw_rotations || !in->raw_opacities || !in->base_colors ||
                      (p.row_used > 0 && !in->residual_params)))
        return fail(EFGS_ERR_INVALID_ARGUMENT, "null tensor");
    if (p.payload == EFGS_NGSPLAT_NEURAL_BAKED && !in->bake_matrix) return fail(EFGS_ERR_INVALID_ARGUMENT, "null layer-0 bake matrix");
    if ((reinterpret_cast<uintptr_t>(out->splat_words) | reinterpret_cast<uintptr_t>(out->params)) % 16 != 0)
        return fail(EFGS_ERR_INVALID_ARGUMENT, "output textures must be 16-byte aligned");
    out->n_kept = 0;
    out->base_offset = 0.0f;
    out->base_scale = static_cast<float>(1e-6 / 255.0);
    for (int l = 0; l < 3; l++) out->sh_level_scale[l] = 0.0f;
    if (out->capacity == 0) return EFGS_OK;

    hipStream_t s = static_cast<hipStream_t>(stream);
    const uint32_t capacity = static_cast<uint32_t>(out->capacity);
    const size_t partial_bytes = static_cast<size_t>(capacity / ng_block) * 8 * sizeof(uint32_t);
    char* blob = static_cast<char*>(alloc(alloc_ctx, partial_bytes + 256));
    if (!blob) return fail(EFGS_ERR_ALLOC, "allocation of the ngsplat partials failed");
    NgsplatArgs a{};
    a.means = in->means;
    a.raw_scales = in->raw_scales;
    a.raw_rotations = in->raw_rotations;
    a.raw_opacities = in->raw_opacities;
    a.base_colors = in->base_colors;
    a.residual_params = in->residual_params;
    a.bake_matrix = in->bake_matrix;
    a.bake_bias = in->bake_bias;
    a.n = static_cast<uint32_t>(in->n);
    a.row_stride = static_cast<uint32_t>(in->residual_row_stride);
    a.row_used = static_cast<uint32_t>(p.row_used);
    a.payload = p.payload;
    a.n_items = p.n_items;
    a.n_values = p.n_values;
    a.n_encoded = p.n_encoded;
    a.base_input = in->base_input ? 1 : 0;
    a.n_frequencies = in->n_frequencies;
    a.residual_act = in->residual_act;
    a.color_shift = in->color_shift;
    NgsplatTextures t{};
    t.splat_words = out->splat_words;
    t.params = out->params;
    t.source_index = out->source_index;
    t.capacity = capacity;
    t.n_textures = p.n_textures;
    uint64_t offset = 0;
    for (int k = 0; k < p.n_textures; k++) {
        t.texel_words[k] = p.texel_words[k];
        t.texture_offset[k] = offset;
        offset += static_cast<uint64_t>(capacity) * p.texel_words[k];
    }
    NgsplatStats* stats = reinterpret_cast<NgsplatStats*>(blob + partial_bytes);
    hipEvent_t events[3] = {nullptr, nullptr, nullptr};
    const bool timed = out->kernel_ms != nullptr;
    auto destroy_events = [&events]() {
        for (hipEvent_t& e : events)
            if (e) (void)hipEventDestroy(e);
    };
    if (timed)
        for (hipEvent_t& e : events)
            if (hipEventCreate(&e) != hipSuccess) {
                destroy_events();
                return fail(EFGS_ERR_HIP, "creating the ngsplat timing events failed");
            }
    if (!launch_ngsplat_pack(a, t, reinterpret_cast<uint32_t*>(blob), stats, timed ? events : nullptr, s)) {
        destroy_events();
        return EFGS_ERR_HIP;
    }
    NgsplatStats host;
    if (hipMemcpyAsync(&host, stats, sizeof(host), hipMemcpyDeviceToHost, s) != hipSuccess || hipStreamSynchronize(s) != hipSuccess) {
        destroy_events();
        return fail(EFGS_ERR_HIP, "reading the ngsplat statistics failed");
    }
    if (timed) {
        float ms0 = 0.0f, ms1 = 0.0f;
        const bool ok = hipEventElapsedTime(&ms0, events[0], events[1]) == hipSuccess && hipEventElapsedTime(&ms1, events[1], events[2]) == hipSuccess;
        destroy_events();
        if (!ok) return fail(EFGS_ERR_HIP, "reading the ngsplat timing events failed");
        out->kernel_ms[0] = ms0;
        out->kernel_ms[1] = ms1;
    }
    out->n_kept = host.n_kept;
    out->base_offset = host.base_offset;
    out->base_scale = host.base_scale;
    // levels absent from the export carry scale 0 (degree l's coefficients end at (l + 1)^2 - 1)
    for (int l = 0; l < 3; l++)
        out->sh_level_scale[l] = p.payload == EFGS_NGSPLAT_SH && (l + 2) * (l + 2) - 1 <= p.n_items ? host.level_scale[l] : 0.0f;
    return EFGS_OK;
}

}  // extern "C"
