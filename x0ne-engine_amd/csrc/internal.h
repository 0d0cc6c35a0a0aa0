// Host-side structures of the runtime, shared by runtime.hip (device, launch API, arena) and
// engine.hip (the Qwen3 engine).
#pragma once
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>
#include <string>
#include <vector>

#include "../../include/x0ne_core.h"
#include "kernels.h"
#include "launch.h"

namespace x0ne {

// Sets the calling thread's message and returns the status (the reference's Error variants).
x0ne_status fail(x0ne_status s, const std::string& msg);
// X0NE_ERR_GPU with the runtime's error text, for a failed HIP call.
x0ne_status gpu_fail(hipError_t e, const char* what);

struct Counts {
    std::atomic<uint64_t> launches{0}, graph_launches{0}, gemms{0}, htod{0}, dtoh{0}, memsets{0}, syncs{0};
};

}  // namespace x0ne

#define X0NE_HIP(call, what)                                        \
    do {                                                            \
        hipError_t e_ = (call);                                     \
        if (e_ != hipSuccess) return x0ne::gpu_fail(e_, (what));    \
    } while (0)

#define X0NE_TRY(call)                          \
    do {                                        \
        x0ne_status s_ = (call);                \
        if (s_ != X0NE_OK) return s_;           \
    } while (0)

namespace x0ne {
}

struct x0ne_gpu {
    int device = 0;
    hipStream_t stream = nullptr;
    std::string name, arch;
    uint32_t cus = 0;
    int driver_version = 0, runtime_version = 0;
    uint64_t total_mem = 0;
    x0ne::Counts counts;
    bool capturing = false;
    // This device's copy of the library's static scratch array (runtime.hip, `scratch`), as
    // hipGetSymbolAddress gave it at x0ne_gpu_new with the device current.
    void* scratch = nullptr;
};

struct x0ne_graph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    size_t nodes = 0;
    const x0ne_gpu* owner = nullptr;  // the Gpu that captured it: launch_graph refuses any other
};

struct x0ne_arena {
    struct Region {
        std::string label;
        uint32_t cls;
        uint64_t offset, len;
    };
    uint64_t id = 0;
    std::vector<Region> regions;
    uint64_t size = 0;
    bool frozen = false;
    x0ne_gpu* gpu = nullptr;  // null: host backing
    uint8_t* base = nullptr;
    uint64_t len = 0;
};

namespace x0ne {
// Checked offset of `len` bytes at `at` of slice s (arena.rs:229-240).
x0ne_status arena_check(const x0ne_arena* a, x0ne_slice s, uint64_t at, uint64_t len, uint64_t* off);
// Device address of a slice (its first byte).
inline uint8_t* dev(const x0ne_arena* a, x0ne_slice s) { return a->base + s.offset; }
// Launch of a table kernel by index with checked arguments.
x0ne_status launch_checked(x0ne_gpu* g, const X0neKernel& k, uint32_t gx, uint32_t gy, uint32_t block,
                           const x0ne_arg* args, size_t n, uint32_t gz = 1);
// Y[n][rows] = X[n][cols] W^T for 1 <= n <= 64 rows of X with the few-row kernels of gemm.hip
// (mode 0 bf16 Y, 1 f32 Y, 2 SwiGLU over a packed [gate; up] W of 2 rows rows); panels: 2 X in
// panels, 4 Y in panels (bf16 Y), 8 W in panels (rows a multiple of 16), the layout of device.h.
constexpr uint32_t PANEL_X = 2, PANEL_Y = 4, PANEL_W = 8;
// With `work` (a workspace for up to work->groups 16-row groups), a shape whose groups are
// between one and two per CU takes the balanced kernel (x0ne_gemm_few_bal_bf16) instead.
struct FewWork {
    float* ws = nullptr;      // 2 x 256 floats per group
    uint32_t* cnt = nullptr;  // one word per group: zero, left zero by every launch
    uint64_t groups = 0;
};
x0ne_status skinny(x0ne_gpu* g, const void* w, uint64_t rows, uint64_t cols, const void* x, uint64_t n, void* y,
                   uint32_t mode, uint32_t panels, const FewWork* work = nullptr);
// The tiled matrix-core GEMM (gemm.hip) behind x0ne_gpu_gemm_tiled: tile 0 picks per shape;
// layout X0NE_GEMM_W_PANELS | X0NE_GEMM_X_PANELS names the operands held in 16-row panels.
x0ne_status tiled_gemm(x0ne_gpu* g, int tile, uint32_t layout, const void* w, uint64_t rows, uint64_t cols,
                       const void* x, uint64_t n, void* y, bool out_f32);
// Y[n][rows] = X[n][cols] W^T with every product summed in f64 (the exact mode's prefill
// passes; x0ne_gemm_f64_t*_bf16), Y = bf16(f32(sum)) or f32(sum); W and X row-major. ks K slices
// (0: picked per shape, up to what ws_bytes of ws holds) summed in slice order by
// x0ne_gemm_f64_reduce. Launches sharing ws must not overlap.
constexpr uint32_t EXACT_GEMM_MAX_SLICES = 16;
constexpr uint32_t EXACT_GEMM_WAVES_PER_CU = 8;
x0ne_status exact_gemm(x0ne_gpu* g, const void* w, uint64_t rows, uint64_t cols, const void* x, uint64_t n, void* y,
                       bool out_f32, double* ws, uint64_t ws_bytes, uint32_t ks = 0);
// Split plan for a geometry (gpu.rs:958-985), P capped at `cap`.
// exact: the plan of the exact mode's f64 kernel (its occupancy sets P).
x0ne_status split_plan(const x0ne_gpu* g, uint32_t q_heads, uint32_t kv_heads, x0ne_split_plan* out,
                       bool exact = false);
x0ne_status attention_split(x0ne_gpu* g, const x0ne_split_plan& plan, int last_block, const void* q, const void* k,
                            const void* v, const void* pages, void* state, void* counter, void* out, const void* pos,
                            uint32_t q_heads, uint32_t kv_heads, uint32_t max_ctx, float scale);
// The merge kernel over P = plan.splits slices of f32 states (x0ne_attention_merge_bf16).
x0ne_status attention_merge(x0ne_gpu* g, const x0ne_split_plan& plan, const void* state, void* out, const void* pos,
                            uint32_t q_heads, uint32_t max_ctx);
// The decode step's attention in one launch for a grouped plan: QK-norm + RoPE of q, the K/V
// row of position pos written into its page, split-K attention and the last-block merge. rope_cs:
// the RoPE table of positions below max_ctx (x0ne_rope_table_f64 of inv_freq). exact: the exact
// mode's kernel (f64 scores, softmax and sums; its state is f64, twice x0ne_split_state_bytes).
x0ne_status attention_rope_split(x0ne_gpu* g, const x0ne_split_plan& plan, const void* qkv, const void* q_norm,
                                 const void* k_norm, const void* inv_freq, const void* rope_cs, void* k, void* v,
                                 const void* pages,
                                 void* state, void* counter, void* out, const void* pos, uint32_t q_heads,
                                 uint32_t kv_heads, uint32_t max_ctx, float scale, float eps, bool exact = false);
}  // namespace x0ne
