// The device, the kernel-launch API, graph capture and the arena: the reference's
// x0ne-core/runtime/src/{gpu,arena,error}.rs, on the HIP runtime for gfx950.

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <tuple>

#include "internal.h"

namespace x0ne {

static thread_local std::string g_last_error;

x0ne_status fail(x0ne_status s, const std::string& msg) {
    g_last_error = msg;
    return s;
}

x0ne_status gpu_fail(hipError_t e, const char* what) {
    return fail(X0NE_ERR_GPU, std::string(what) + ": " + hipGetErrorName(e) + " (" + hipGetErrorString(e) + ")");
}

static std::atomic<uint64_t> g_next_arena{1};

}  // namespace x0ne

using namespace x0ne;

extern "C" size_t x0ne_last_error(char* buf, size_t len) {
    const std::string& m = g_last_error;
    if (buf && len) {
        const size_t n = m.size() < len - 1 ? m.size() : len - 1;
        std::memcpy(buf, m.data(), n);
        buf[n] = 0;
    }
    return m.size();
}

#ifndef X0NE_KERNEL_SET
#define X0NE_KERNEL_SET "unversioned"
#endif

extern "C" size_t x0ne_kernel_set(char* buf, size_t len) {
    const std::string s = std::string("kernels ") + X0NE_KERNEL_SET + ", gfx950, " + __VERSION__;
    if (buf && len) {
        const size_t n = s.size() < len - 1 ? s.size() : len - 1;
        std::memcpy(buf, s.data(), n);
        buf[n] = 0;
    }
    return s.size();
}

// ---------------------------------------------------------------------------------------------
// The device (gpu.rs:750-928)
// ---------------------------------------------------------------------------------------------

// Split-K workspace for callers that cannot allocate (x0ne_gpu_attention_split_scratch): the
// f32 slice states, then one counter word per kv head. Each GPU holds its own copy for the life
// of the process; every call on a GPU shares it, so calls that overlap on one GPU race.
constexpr uint64_t SCRATCH_STATE_BYTES = 4ull << 20;
constexpr uint64_t SCRATCH_COUNTERS = 256;
constexpr uint64_t SCRATCH_BYTES = SCRATCH_STATE_BYTES + SCRATCH_COUNTERS * 4;
static __device__ __align__(256) uint8_t scratch[SCRATCH_BYTES];

extern "C" x0ne_status x0ne_gpu_new(x0ne_gpu** out) {
    if (!out) return fail(X0NE_ERR_FORMAT, "x0ne_gpu_new: null out");
    *out = nullptr;
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count == 0)
        return fail(X0NE_ERR_GPU, std::string("no HIP device: ") + (e != hipSuccess ? hipGetErrorString(e) : "0 devices"));
    X0NE_HIP(hipSetDevice(0), "hipSetDevice(0)");
    hipDeviceProp_t p;
    X0NE_HIP(hipGetDeviceProperties(&p, 0), "hipGetDeviceProperties");
    const std::string arch = p.gcnArchName;
    if (arch.rfind("gfx950", 0) != 0)
        return fail(X0NE_ERR_GPU, "device 0 is " + arch + ": the kernels are built for gfx950 only");
    x0ne_gpu* g = new x0ne_gpu();
    g->device = 0;
    // The device address of this device's scratch array (device 0 is current): host code uses
    // this pointer, never the array's name, which on the host is only a stand-in.
    e = hipGetSymbolAddress(&g->scratch, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !g->scratch) {
        delete g;
        return gpu_fail(e != hipSuccess ? e : hipErrorInvalidSymbol, "hipGetSymbolAddress(scratch)");
    }
    g->name = p.name;
    g->arch = arch;
    g->cus = (uint32_t)p.multiProcessorCount;
    g->total_mem = (uint64_t)p.totalGlobalMem;
    (void)hipDriverGetVersion(&g->driver_version);
    (void)hipRuntimeGetVersion(&g->runtime_version);
    // One non-blocking stream at the default priority.
    e = hipStreamCreateWithFlags(&g->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete g;
        return gpu_fail(e, "hipStreamCreateWithFlags");
    }
    *out = g;
    return X0NE_OK;
}

namespace x0ne {
}

extern "C" void x0ne_gpu_free(x0ne_gpu* g) {
    if (!g) return;
    if (g->stream) {
        (void)hipStreamSynchronize(g->stream);
        (void)hipStreamDestroy(g->stream);
    }
    delete g;
}

extern "C" x0ne_status x0ne_gpu_sync(x0ne_gpu* g) {
    if (!g) return fail(X0NE_ERR_GPU, "no device");
    g->counts.syncs++;
    X0NE_HIP(hipStreamSynchronize(g->stream), "hipStreamSynchronize");
    return X0NE_OK;
}

extern "C" x0ne_status x0ne_gpu_describe(const x0ne_gpu* g, char* buf, size_t len) {
    if (!g) return fail(X0NE_ERR_GPU, "no device");
    char s[512];
    std::snprintf(s, sizeof s, "%s (%s, %u CUs, %.1f GiB), HIP driver %d, runtime %d", g->name.c_str(),
                  g->arch.c_str(), g->cus, (double)g->total_mem / (1ull << 30), g->driver_version,
                  g->runtime_version);
    if (buf && len) {
        std::strncpy(buf, s, len - 1);
        buf[len - 1] = 0;
    }
    return X0NE_OK;
}

extern "C" uint32_t x0ne_gpu_compute_units(const x0ne_gpu* g) { return g ? g->cus : 0; }

extern "C" x0ne_status x0ne_gpu_mem_info(const x0ne_gpu* g, uint64_t* free_bytes, uint64_t* total_bytes) {
    if (!g) return fail(X0NE_ERR_GPU, "no device");
    size_t f = 0, t = 0;
    X0NE_HIP(hipMemGetInfo(&f, &t), "hipMemGetInfo");
    if (free_bytes) *free_bytes = f;
    if (total_bytes) *total_bytes = t;
    return X0NE_OK;
}

extern "C" x0ne_status x0ne_gpu_counts(const x0ne_gpu* g, x0ne_counts* out) {
    if (!g || !out) return fail(X0NE_ERR_GPU, "no device");
    out->launches = g->counts.launches;
    out->graph_launches = g->counts.graph_launches;
    out->gemms = g->counts.gemms;
    out->htod = g->counts.htod;
    out->dtoh = g->counts.dtoh;
    out->memsets = g->counts.memsets;
    out->syncs = g->counts.syncs;
    return X0NE_OK;
}

// ---------------------------------------------------------------------------------------------
// The kernel table and the checked launch (gpu.rs:281-374, :1031-1086)
// ---------------------------------------------------------------------------------------------

static const X0neKernel* find_kernel(const char* name) {
    if (!name) return nullptr;
    size_t n = 0;
    const X0neKernel* t = x0ne_kernel_table(&n);
    for (size_t i = 0; i < n; ++i)
        if (std::strcmp(t[i].name, name) == 0) return &t[i];
    return nullptr;
}

extern "C" size_t x0ne_kernel_count(void) {
    size_t n = 0;
    x0ne_kernel_table(&n);
    return n;
}

extern "C" const char* x0ne_kernel_name(size_t i) {
    size_t n = 0;
    const X0neKernel* t = x0ne_kernel_table(&n);
    return i < n ? t[i].name : nullptr;
}

static uint32_t kind_of(char c) { return c == 'p' ? X0NE_PARAM_PTR : c == 'u' ? X0NE_PARAM_U32 : X0NE_PARAM_F32; }

extern "C" size_t x0ne_kernel_params(const char* name, uint32_t* out, size_t cap) {
    const X0neKernel* k = find_kernel(name);
    if (!k) return (size_t)-1;
    const size_t n = std::strlen(k->params);
    for (size_t i = 0; i < n && i < cap; ++i) out[i] = kind_of(k->params[i]);
    return n;
}

static const char* kind_name(uint32_t k) {
    return k == X0NE_PARAM_PTR ? "a pointer" : k == X0NE_PARAM_U32 ? "a u32" : k == X0NE_PARAM_F32 ? "an f32" : "unknown";
}

static x0ne_status check_args_of(const X0neKernel& k, const x0ne_arg* args, size_t n) {
    const size_t want = std::strlen(k.params);
    if (n != want)
        return fail(X0NE_ERR_GPU, std::string(k.name) + ": " + std::to_string(n) + " arguments for " +
                                      std::to_string(want) + " parameters");
    for (size_t i = 0; i < n; ++i) {
        const uint32_t p = kind_of(k.params[i]);
        if (args[i].kind != p)
            return fail(X0NE_ERR_GPU, std::string(k.name) + ": argument " + std::to_string(i) + " is " +
                                          kind_name(args[i].kind) + ", the parameter " + kind_name(p));
    }
    return X0NE_OK;
}

extern "C" x0ne_status x0ne_check_args(const char* name, const x0ne_arg* args, size_t n) {
    const X0neKernel* k = find_kernel(name);
    if (!k) return fail(X0NE_ERR_GPU, std::string("no kernel ") + (name ? name : "(null)"));
    return check_args_of(*k, args, n);
}

namespace x0ne {

}  // namespace x0ne

thread_local X0neTimer* x0ne_timer = nullptr;

hipError_t x0ne_launch(const void* fn, dim3 grid, dim3 block, void** args, size_t lds, hipStream_t s) {
    X0neTimer* t = x0ne_timer;
    if (!t) return hipLaunchKernel(fn, grid, block, args, lds, s);
    hipEvent_t start = t->started ? nullptr : t->start;
    t->started = true;
    return hipExtLaunchKernel(fn, grid, block, args, lds, s, start, t->stop, 0);
}

namespace x0ne {

x0ne_status launch_checked(x0ne_gpu* g, const X0neKernel& k, uint32_t gx, uint32_t gy, uint32_t block,
                           const x0ne_arg* args, size_t n, uint32_t gz) {
    X0NE_TRY(check_args_of(k, args, n));
    if (gx == 0 || gy == 0 || gz == 0 || block == 0 || block > k.max_block || block % 64 != 0)
        return fail(X0NE_ERR_GPU, std::string(k.name) + ": launch shape (" + std::to_string(gx) + ", " +
                                      std::to_string(gy) + ", " + std::to_string(gz) + ") x " + std::to_string(block) +
                                      " refused");
    void* ptrs[24];
    if (n > 24) return fail(X0NE_ERR_GPU, "too many arguments");
    for (size_t i = 0; i < n; ++i) {
        switch (args[i].kind) {
            case X0NE_PARAM_PTR: ptrs[i] = (void*)&args[i].ptr; break;
            case X0NE_PARAM_U32: ptrs[i] = (void*)&args[i].u32; break;
            default: ptrs[i] = (void*)&args[i].f32; break;
        }
    }
    g->counts.launches++;
    X0NE_HIP(hipLaunchKernel(k.fn, dim3(gx, gy, gz), dim3(block), ptrs, 0, g->stream), k.name);
    return X0NE_OK;
}

}  // namespace x0ne

extern "C" x0ne_status x0ne_gpu_launch(x0ne_gpu* g, const char* name, uint32_t gx, uint32_t gy, uint32_t block,
                                       const x0ne_arg* args, size_t n) {
    if (!g) return fail(X0NE_ERR_GPU, "no device");
    const X0neKernel* k = find_kernel(name);
    if (!k) return fail(X0NE_ERR_GPU, std::string("no kernel ") + (name ? name : "(null)"));
    return launch_checked(g, *k, gx, gy, block, args, n);
}

extern "C" x0ne_status x0ne_gpu_launch_3d(x0ne_gpu* g, const char* name, uint32_t gx, uint32_t gy, uint32_t gz,
                                          uint32_t block, const x0ne_arg* args, size_t n) {
    if (!g) return fail(X0NE_ERR_GPU, "no device");
    const X0neKernel* k = find_kernel(name);
    if (!k) return fail(X0NE_ERR_GPU, std::string("no kernel ") + (name ? name : "(null)"));
    return launch_checked(g, *k, gx, gy, block, args, n, gz);
}

// Gpu::gemm (gpu.rs:1098-1149). One row: the bandwidth-bound GEMV of gemv.hip. Two to 64 rows:
// the few-row kernel of gemm.hip, still bandwidth-bound (each W row read once). More: the tiled
// matrix-core GEMM. The kernels of gemm.hip take 32-bit buffer offsets.
static constexpr uint64_t SKINNY_MAX_ROWS = 64;
static constexpr uint64_t GEMM_MAX_BYTES = 0xFFFFFFF0ull;

namespace x0ne {

// ---- many rows: the tiled matrix-core GEMM of gemm.hip ----
// The reference hands Gpu::gemm to cuBLAS (gpu.rs:1098-1149); from SKINNY_MAX_ROWS + 1 rows on
// this library runs its own tiled GEMM (x0ne_launch_gemm_tiles), the tile chosen per shape by
// x0ne_gemm_tile_pick unless `tile` names one. A shape always runs the same kernel, and each
// output is summed in a fixed order: results are the same from call to call.
x0ne_status tiled_gemm(x0ne_gpu* g, int tile, uint32_t layout, const void* w, uint64_t rows, uint64_t cols,
                       const void* x, uint64_t n, void* y, bool out_f32) {
    const bool wp = layout & X0NE_GEMM_W_PANELS, xp = layout & X0NE_GEMM_X_PANELS;
    const uint64_t xrows = xp ? (n + 15) / 16 * 16 : n;
    if (rows == 0 || cols == 0 || n == 0 || rows % 4 != 0 || cols % 8 != 0 || (wp && rows % 16 != 0) ||
        layout > 3 || rows > UINT32_MAX || n > UINT32_MAX || rows * cols * 2 > GEMM_MAX_BYTES ||
        xrows * cols * 2 > GEMM_MAX_BYTES || (uintptr_t)w % 16 != 0 || (uintptr_t)x % 16 != 0 ||
        (uintptr_t)y % (out_f32 ? 16 : 8) != 0)
        return fail(X0NE_ERR_FORMAT, "tiled gemm: " + std::to_string(rows) + "x" + std::to_string(cols) + ", n " +
                                         std::to_string(n) + " (rows a multiple of 4, of 16 with W in panels, "
                                         "cols of 8, W and X below 4 GiB, 16-byte aligned operands)");
    if (tile == 0) tile = x0ne_gemm_tile_pick((uint32_t)rows, (uint32_t)cols, (uint32_t)n, g->cus);
    const uint32_t flags = (out_f32 ? X0NE_TILE_F32 : 0u) | (wp ? X0NE_TILE_W_PANEL : 0u) | (xp ? X0NE_TILE_X_PANEL : 0u);
    g->counts.gemms++;
    g->counts.launches++;
    X0NE_HIP(x0ne_launch_gemm_tiles(tile, w, x, y, (uint32_t)rows, (uint32_t)cols, (uint32_t)n, flags, g->stream),
             "tiled gemm");
    return X0NE_OK;
}

x0ne_status skinny(x0ne_gpu* g, const void* w, uint64_t rows, uint64_t cols, const void* x, uint64_t n, void* y,
                   uint32_t mode, uint32_t panels, const FewWork* work) {
    const uint64_t wrows = mode == 2 ? 2 * rows : rows;
    if (n == 0 || n > SKINNY_MAX_ROWS || rows == 0 || cols == 0 || cols % 8 != 0 || mode > 2 || (panels & ~14u) ||
        ((panels & 4) && (mode == 1 || rows % 8 != 0)) || ((panels & 8) && rows % 16 != 0) ||
        wrows * cols * 2 > GEMM_MAX_BYTES || n * cols * 2 > GEMM_MAX_BYTES || (uintptr_t)w % 16 != 0 ||
        (uintptr_t)x % 16 != 0)
        return fail(X0NE_ERR_FORMAT, "few-row gemm: " + std::to_string(rows) + "x" + std::to_string(cols) + ", n " +
                                         std::to_string(n) + ", mode " + std::to_string(mode));
    // Between one and two 16-row groups per CU, each of at least 512 steps, with X and W in
    // panels: one block per CU over an equal run of the steps (gemm.hip, few_bal; 4 wavefronts,
    // swept on MI355X; the 32B O projection's 256-step groups measured no faster). Runs are
    // longer than a group (T >= S), so at most two blocks meet in one.
    const uint64_t groups = rows / 16, steps = (cols + 31) / 32;
    if (work && work->ws && work->cnt && n <= 16 && mode != 2 && (panels & PANEL_X) && (panels & PANEL_W) &&
        rows % 16 == 0 && groups > g->cus && groups < 2ull * g->cus && steps >= 512 && groups <= work->groups) {
        const uint64_t T = (groups * steps + g->cus - 1) / g->cus;
        uint32_t r32 = (uint32_t)rows, c32 = (uint32_t)cols, n32 = (uint32_t)n, t32 = (uint32_t)T;
        uint32_t flags = (mode == 1 ? 1u : 0u) | panels;
        float* wsp = work->ws;
        uint32_t* cntp = work->cnt;
        void* args[] = {(void*)&w,     (void*)&x,  (void*)&y,   (void*)&r32,  (void*)&c32,
                        (void*)&n32,   (void*)&flags, (void*)&t32, (void*)&wsp, (void*)&cntp};
        g->counts.gemms++;
        g->counts.launches++;
        X0NE_HIP(x0ne_launch((const void*)&x0ne_gemm_few_bal_bf16, dim3((uint32_t)((groups * steps + T - 1) / T)),
                             dim3(256), args, 0, g->stream),
                 "balanced few-row gemm");
        return X0NE_OK;
    }
    // Row groups per block (each X piece serves RG W pieces) and wavefronts per block, from sweeps
    // on MI355X over the decode shapes (X in panels, 8 and 16 rows): a CU streams a few hundred
    // KiB of a launch fastest alone, so a launch of up to two blocks per CU takes RG so that at
    // most one block lands on each CU (a CU with two finishes last); large launches (the LM
    // head) take RG 2 at up to 8 rows of X and 8 beyond, where each X piece costs as much as a
    // W piece; SwiGLU launches, two W pieces per X piece already, keep RG 1 over 8 wavefronts
    // (Qwen3-8B at 8 rows 31.6 against 32.4 us over 4, -32B at 16 rows 82.4 against 83.3). With W in panels
    // (PANEL_W) the one-block-per-CU rule extends to RG 4, and a large launch takes RG 2 over 8
    // wavefronts at every n up to 16.
    const bool glu = mode == 2, wpan = panels & PANEL_W;
    auto blocks_of = [&](uint32_t rg) { return (uint32_t)((rows + 16 * rg - 1) / (16 * rg)); };
    uint32_t rg = 1, waves = 4;
    const void* fn = nullptr;
    if (n <= 16) {
        if (glu) {
            fn = (const void*)&x0ne_gemm_few_t1_r1_swiglu_bf16;
            waves = 8;
        } else if (wpan) {
            if (blocks_of(1) <= g->cus)
                rg = 1;
            else if (blocks_of(2) <= g->cus)
                rg = 2;
            else if (blocks_of(4) <= g->cus)
                rg = 4;
            else if (blocks_of(1) >= 8 * g->cus)
                rg = 2, waves = 8;
            fn = rg == 1   ? (const void*)&x0ne_gemm_few_t1_r1_bf16
                 : rg == 2 ? (const void*)&x0ne_gemm_few_t1_r2_bf16
                           : (const void*)&x0ne_gemm_few_t1_r4_bf16;
        } else {
            if (blocks_of(1) <= g->cus)
                rg = 1;
            else if (blocks_of(2) <= g->cus)
                rg = 2;
            else if (blocks_of(1) >= 8 * g->cus)
                rg = n <= 8 ? 2 : 8;
            fn = rg == 1   ? (const void*)&x0ne_gemm_few_t1_r1_bf16
                 : rg == 2 ? (const void*)&x0ne_gemm_few_t1_r2_bf16
                 : rg == 4 ? (const void*)&x0ne_gemm_few_t1_r4_bf16
                           : (const void*)&x0ne_gemm_few_t1_r8_bf16;
        }
    } else if (n <= 32) {
        if (glu) {
            fn = (const void*)&x0ne_gemm_few_t2_r1_swiglu_bf16;
        } else {
            rg = blocks_of(2) >= 160 ? 2 : 1;
            fn = rg == 2 ? (const void*)&x0ne_gemm_few_t2_r2_bf16 : (const void*)&x0ne_gemm_few_t2_r1_bf16;
        }
    } else {
        fn = glu ? (const void*)&x0ne_gemm_few_t4_r1_swiglu_bf16 : (const void*)&x0ne_gemm_few_t4_r1_bf16;
    }
    uint32_t r32 = (uint32_t)rows, c32 = (uint32_t)cols, n32 = (uint32_t)n, flags = (mode == 1 ? 1u : 0u) | panels;
    void* args[] = {(void*)&w, (void*)&x, (void*)&y, (void*)&r32, (void*)&c32, (void*)&n32, (void*)&flags};
    g->counts.gemms++;
    g->counts.launches++;
    X0NE_HIP(x0ne_launch(fn, dim3(blocks_of(rg)), dim3(64 * waves), args, 0, g->stream), "few-row gemm");
    return X0NE_OK;
}

x0ne_status exact_gemm(x0ne_gpu* g, const void* w, uint64_t rows, uint64_t cols, const void* x, uint64_t n, void* y,
                       bool out_f32, double* ws, uint64_t ws_bytes, uint32_t ks) {
    if (rows == 0 || cols == 0 || n == 0 || cols % 8 != 0 || rows > UINT32_MAX || n > UINT32_MAX ||
        rows * cols * 2 > GEMM_MAX_BYTES || n * cols * 2 > GEMM_MAX_BYTES || (uintptr_t)w % 16 != 0 ||
        (uintptr_t)x % 16 != 0 || ks > EXACT_GEMM_MAX_SLICES || (ks > 1 && ws_bytes / 8 / ks / n < rows) ||
        (ks > 1 && ws == nullptr))
        return fail(X0NE_ERR_FORMAT, "exact gemm: " + std::to_string(rows) + "x" + std::to_string(cols) + ", n " +
                                         std::to_string(n) + ", " + std::to_string(ks) + " slices");
    // Tokens per wavefront: up to 32 rows of X in quads of 4 (x0ne_gemm_f64_q*, no padding to 16),
    // beyond that 64 (x0ne_gemm_f64_t4); 64 features per wavefront either way.
    const uint32_t tq = n <= 32 ? (uint32_t)(n + 3) / 4 : 0, tt = 4;
    const uint64_t tiles = (rows + 63) / 64 * (tq ? 1 : (n + 16 * tt - 1) / (16 * tt)), steps = (cols + 31) / 32;
    if (ks == 0) {
        // A wavefront's steps run back to back on its SIMD's f64 matrix core, so a launch wants
        // EXACT_GEMM_WAVES_PER_CU wavefronts per CU: fewer tiles than that cut K into slices of
        // at least 8 steps, as many as the workspace holds.
        ks = 1;
        const uint64_t want = (uint64_t)EXACT_GEMM_WAVES_PER_CU * g->cus;
        if (tiles < want && ws) {
            uint64_t k = std::min<uint64_t>({(want + tiles - 1) / tiles, EXACT_GEMM_MAX_SLICES, steps / 8,
                                             ws_bytes / (n * rows * 8)});
            ks = (uint32_t)std::max<uint64_t>(k, 1);
        }
    }
    static const void* const quads[8] = {(const void*)&x0ne_gemm_f64_q1_bf16, (const void*)&x0ne_gemm_f64_q2_bf16,
                                         (const void*)&x0ne_gemm_f64_q3_bf16, (const void*)&x0ne_gemm_f64_q4_bf16,
                                         (const void*)&x0ne_gemm_f64_q5_bf16, (const void*)&x0ne_gemm_f64_q6_bf16,
                                         (const void*)&x0ne_gemm_f64_q7_bf16, (const void*)&x0ne_gemm_f64_q8_bf16};
    const void* fn = tq ? quads[tq - 1] : (const void*)&x0ne_gemm_f64_t4_bf16;
    uint32_t r32 = (uint32_t)rows, c32 = (uint32_t)cols, n32 = (uint32_t)n, of = out_f32 ? 1u : 0u, k32 = ks;
    double* wsp = ks > 1 ? ws : nullptr;
    void* yp = y;
    void* args[] = {(void*)&w, (void*)&x, (void*)&yp, (void*)&r32, (void*)&c32, (void*)&n32, (void*)&of, (void*)&k32,
                    (void*)&wsp};
    g->counts.gemms++;
    g->counts.launches++;
    X0NE_HIP(x0ne_launch(fn, dim3((uint32_t)((tiles * ks + 3) / 4)), dim3(256), args, 0, g->stream), "exact gemm");
    if (ks > 1) {
        const double* wsc = wsp;
        void* rargs[] = {(void*)&wsc, (void*)&yp, (void*)&r32, (void*)&n32, (void*)&k32, (void*)&of};
        g->counts.launches++;
        X0NE_HIP(x0ne_launch((const void*)&x0ne_gemm_f64_reduce, dim3((uint32_t)((rows * n + 255) / 256)), dim3(256),
                             rargs, 0, g->stream),
                 "exact gemm slices");
    }
    return X0NE_OK;
}

}  // namespace x0ne

// ---- one fused GEMV instance on caller buffers (the kernel-level test surface) ----
namespace {
bool fused_desc(const x0ne_gemv_fused& d, X0neGemv* a, std::string* why) {
    auto aligned = [](uint64_t p) { return p % 16 == 0; };
    if (d.prologue > X0NE_GEMV_PRO_EMBED_NORM || d.epilogue > X0NE_GEMV_EPI_ARGMAX) {
        *why = "unknown prologue or epilogue";
        return false;
    }
    if (!d.w || !d.y || !aligned(d.w)) {
        *why = "W and y are required, W 16-byte aligned";
        return false;
    }
    if (d.prologue == X0NE_GEMV_PRO_X && (!d.x || !aligned(d.x))) {
        *why = "x (16-byte aligned) is required";
        return false;
    }
    if (d.prologue == X0NE_GEMV_PRO_NORM &&
        (!d.res_in || !d.delta || !d.norm_w || !aligned(d.res_in) || !aligned(d.delta) || !aligned(d.norm_w) ||
         !aligned(d.res_out))) {
        *why = "res_in, delta and norm_w (and res_out when given) are required, 16-byte aligned";
        return false;
    }
    if (d.prologue == X0NE_GEMV_PRO_EMBED_NORM &&
        (!d.embed || !d.tokens || !d.norm_w || !d.vocab || !aligned(d.embed) || !aligned(d.norm_w) ||
         !aligned(d.res_out))) {
        *why = "embed, tokens, vocab and norm_w (and res_out when given) are required, 16-byte aligned";
        return false;
    }
    if (d.epilogue == X0NE_GEMV_EPI_ARGMAX && (!d.partial || !d.counter || !d.token_out || (d.advance && !d.pos))) {
        *why = "partial, counter, token_out (and pos when advancing) are required";
        return false;
    }
    *a = X0neGemv{};
    a->w = (const uint16_t*)d.w;
    a->x = (const uint16_t*)d.x;
    a->res_in = (const float*)d.res_in;
    a->res_out = (float*)d.res_out;
    a->delta = (const uint16_t*)d.delta;
    a->norm_w = (const uint16_t*)d.norm_w;
    a->embed = (const uint16_t*)d.embed;
    a->tokens = (const uint32_t*)d.tokens;
    a->y = (void*)d.y;
    a->partial = (float*)d.partial;
    a->counter = (uint32_t*)d.counter;
    a->token_out = (uint32_t*)d.token_out;
    a->pos = (uint32_t*)d.pos;
    a->rows = d.rows;
    a->cols = d.cols;
    a->vocab = d.vocab;
    a->advance = d.advance ? 1u : 0u;
    a->eps = d.eps;
    a->prologue = (int)d.prologue;
    a->epilogue = (int)d.epilogue;
    a->f64acc = d.f64_sums ? 1 : 0;
    return true;
}
}  // namespace

extern "C" uint32_t x0ne_gpu_gemv_fused_blocks(const x0ne_gpu* g, const x0ne_gemv_fused* d) {
    if (!g || !d) return 0;
    X0neGemv a;
    std::string why;
    if (!fused_desc(*d, &a, &why)) return 0;
    return x0ne_gemv_grid(a, g->cus, 0);
}

extern "C" x0ne_status x0ne_gpu_gemv_fused(x0ne_gpu* g, const x0ne_gemv_fused* d) {
    if (!g) return fail(X0NE_ERR_GPU, "no device");
    if (!d) return fail(X0NE_ERR_FORMAT, "fused gemv: no descriptor");
    X0neGemv a;
    std::string why;
    if (!fused_desc(*d, &a, &why)) return fail(X0NE_ERR_FORMAT, "fused gemv: " + why);
    a.grid = x0ne_gemv_grid(a, g->cus, 0);
    if (a.grid == 0)
        return fail(X0NE_ERR_FORMAT, "fused gemv: instance (" + std::to_string(d->prologue) + ", " +
                                         std::to_string(d->epilogue) + ") at " + std::to_string(d->rows) + "x" +
                                         std::to_string(d->cols) + " is not served");
    g->counts.launches++;
    g->counts.gemms++;
    X0NE_HIP(x0ne_launch_gemv(a, g->stream), "fused gemv");
    return X0NE_OK;
}

extern "C" x0ne_status x0ne_gpu_gemm_tiled(x0ne_gpu* g, uint32_t tile, uint32_t layout, uint64_t w, uint64_t rows,
                                           uint64_t cols, uint64_t x, uint64_t n, uint64_t y, int out_f32) {
    if (!g) return fail(X0NE_ERR_GPU, "no device");
    if (tile > X0NE_GEMM_TILE_128x128) return fail(X0NE_ERR_FORMAT, "tiled gemm: tile " + std::to_string(tile));
    return x0ne::tiled_gemm(g, (int)tile, layout, (const void*)w, rows, cols, (const void*)x, n, (void*)y, out_f32 != 0);
}

extern "C" x0ne_status x0ne_gpu_gemv(x0ne_gpu* g, uint64_t w, uint64_t rows, uint64_t cols, uint64_t x, uint64_t n,
                                     uint64_t y, int out_f32) {
    if (!g) return fail(X0NE_ERR_GPU, "no device");
    if (rows == 0 || cols == 0 || n == 0 || rows > UINT32_MAX || cols > UINT32_MAX)
        return fail(X0NE_ERR_FORMAT, "gemv: " + std::to_string(rows) + "x" + std::to_string(cols) + ", n " +
                                         std::to_string(n));
    const uint64_t ob = out_f32 ? 4 : 2;
    if (n >= 2 && n <= SKINNY_MAX_ROWS && cols % 8 == 0 && rows * cols * 2 <= GEMM_MAX_BYTES && w % 16 == 0 &&
        x % 16 == 0)
        return x0ne::skinny(g, (const void*)w, rows, cols, (const void*)x, n, (void*)y, out_f32 ? 1 : 0, 0);
    // Many rows: the tiled matrix-core GEMM (rows a multiple of 4, aligned operands; otherwise the
    // row-by-row GEMV below).
    if (n > SKINNY_MAX_ROWS && cols % 8 == 0 && rows % 4 == 0 && n <= UINT32_MAX &&
        rows * cols * 2 <= GEMM_MAX_BYTES && n * cols * 2 <= GEMM_MAX_BYTES && w % 16 == 0 && x % 16 == 0 &&
        y % 16 == 0)
        return x0ne::tiled_gemm(g, 0, 0, (const void*)w, rows, cols, (const void*)x, n, (void*)y, out_f32 != 0);
    for (uint64_t r = 0; r < n; ++r) {
        const uint16_t* wp = (const uint16_t*)w;
        const uint16_t* xp = (const uint16_t*)(x + r * cols * 2);
        void* yp = (void*)(y + r * rows * ob);
        g->counts.gemms++;
        const bool fast = cols % 8 == 0 && w % 16 == 0 && (x + r * cols * 2) % 16 == 0 && cols <= 32768;
        if (fast) {
            X0neGemv a = {};
            a.w = wp;
            a.x = xp;
            a.y = yp;
            a.rows = (uint32_t)rows;
            a.cols = (uint32_t)cols;
            a.prologue = 0;
            a.epilogue = out_f32 ? 1 : 0;
            a.grid = x0ne_gemv_grid(a, g->cus, 0);
            g->counts.launches++;
            X0NE_HIP(x0ne_launch_gemv(a, g->stream), "gemv");
        } else {
            g->counts.launches++;
            hipLaunchKernelGGL(x0ne_gemv_any, dim3((uint32_t)rows), dim3(256), 0, g->stream, (const bf16_t*)wp,
                               (const bf16_t*)xp, yp, (uint32_t)rows, (uint32_t)cols, (uint32_t)(out_f32 ? 1 : 0));
            X0NE_HIP(hipGetLastError(), "gemv_any");
        }
    }
    return X0NE_OK;
}

// ---------------------------------------------------------------------------------------------
// Split-K attention (gpu.rs:958-985; ops.rs:80-127)
// ---------------------------------------------------------------------------------------------

static const void* group_kernel(uint32_t group) {
    switch (group) {
        case 1: return (const void*)&x0ne_attention_decode_split_g1_bf16;
        case 2: return (const void*)&x0ne_attention_decode_split_g2_bf16;
        case 4: return (const void*)&x0ne_attention_decode_split_g4_bf16;
        case 8: return (const void*)&x0ne_attention_decode_split_g8_bf16;
        default: return nullptr;
    }
}

static const void* rope_group_kernel(uint32_t group) {
    switch (group) {
        case 1: return (const void*)&x0ne_attention_rope_decode_g1_bf16;
        case 2: return (const void*)&x0ne_attention_rope_decode_g2_bf16;
        case 4: return (const void*)&x0ne_attention_rope_decode_g4_bf16;
        case 8: return (const void*)&x0ne_attention_rope_decode_g8_bf16;
        default: return nullptr;
    }
}

static const void* exact_group_kernel(uint32_t group) {
    switch (group) {
        case 1: return (const void*)&x0ne_attention_rope_decode_exact_g1_bf16;
        case 2: return (const void*)&x0ne_attention_rope_decode_exact_g2_bf16;
        case 4: return (const void*)&x0ne_attention_rope_decode_exact_g4_bf16;
        case 8: return (const void*)&x0ne_attention_rope_decode_exact_g8_bf16;
        default: return nullptr;
    }
}

// Most slices a merge reads (the merge keeps one weight per slice in LDS).
static constexpr uint32_t MAX_SPLITS = 256;
// P for a decode step: slices of a kv head beyond this add merge work for nothing at the
// contexts of a decode (a slice of 64-key tiles each).
static constexpr uint32_t DEFAULT_SPLIT_CAP = 128;

namespace x0ne {

x0ne_status split_plan(const x0ne_gpu* g, uint32_t q_heads, uint32_t kv_heads, x0ne_split_plan* out, bool exact) {
    if (kv_heads == 0 || q_heads % kv_heads != 0)
        return fail(X0NE_ERR_GPU, std::to_string(q_heads) + " q heads for " + std::to_string(kv_heads) + " kv heads");
    const uint32_t group = q_heads / kv_heads;
    const void* k = exact ? exact_group_kernel(group) : group_kernel(group);
    if (exact && !k) return fail(X0NE_ERR_GPU, "the exact attention takes 1, 2, 4 or 8 q heads per kv head");
    x0ne_split_plan p = {};
    p.grouped = k != nullptr;
    p.group = p.grouped ? group : 1;
    p.grid_x = p.grouped ? kv_heads : q_heads;
    if (!k) k = (const void*)&x0ne_attention_decode_split_bf16;
    int per = 0;
    X0NE_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, k, 256, 0), "occupancy of the split kernel");
    p.per_cu = per > 0 ? (uint32_t)per : 1;
    // One wave of blocks over the CUs. Measured on MI355X with the coherent last-block merge
    // (32 q / 8 kv heads): 31.1 µs at 32k keys against 39.0 µs at half a wave (P 16), level at
    // 8k, and P does not matter at short contexts (one slice holds them).
    uint32_t splits = g->cus * p.per_cu / p.grid_x;
    if (splits < 1) splits = 1;
    if (splits > DEFAULT_SPLIT_CAP) splits = DEFAULT_SPLIT_CAP;
    p.splits = splits;
    *out = p;
    return X0NE_OK;
}

x0ne_status attention_split(x0ne_gpu* g, const x0ne_split_plan& plan, int last_block, const void* q, const void* k,
                            const void* v, const void* pages, void* state, void* counter, void* out, const void* pos,
                            uint32_t qh, uint32_t kvh, uint32_t max_ctx, float scale) {
    const uint32_t p = plan.splits;
    if (p == 0 || p > MAX_SPLITS) return fail(X0NE_ERR_GPU, "split-K: P " + std::to_string(p) + " outside 1..=256");
    if (kvh == 0 || qh % kvh != 0) return fail(X0NE_ERR_GPU, "split-K: heads");
    if (plan.grouped) {
        const void* kern = group_kernel(plan.group);
        if (!kern || plan.group != qh / kvh) return fail(X0NE_ERR_GPU, "split-K: the plan's group differs");
        // Without the counter the merge kernel below follows; either way a block writes out
        // itself when one slice holds the whole context (and the merge then returns at once).
        void* cnt = last_block ? counter : nullptr;
        void* args[] = {(void*)&q, (void*)&k, (void*)&v, (void*)&pages, (void*)&state, (void*)&cnt,
                        (void*)&out, (void*)&pos, (void*)&qh, (void*)&kvh, (void*)&max_ctx, (void*)&p, (void*)&scale};
        g->counts.launches++;
        X0NE_HIP(x0ne_launch(kern, dim3(kvh, p), dim3(256), args, 0, g->stream), "split-K attention");
        if (last_block) return X0NE_OK;
    } else {
        if (last_block) return fail(X0NE_ERR_GPU, "the last-block merge needs a grouped split-K kernel");
        g->counts.launches++;
        void* args[] = {(void*)&q,   (void*)&k,   (void*)&v,       (void*)&pages, (void*)&state, (void*)&out,
                        (void*)&pos, (void*)&qh,  (void*)&kvh, (void*)&max_ctx, (void*)&p, (void*)&scale};
        X0NE_HIP(x0ne_launch((const void*)&x0ne_attention_decode_split_bf16, dim3(qh, p), dim3(256), args, 0,
                             g->stream),
                 "split-K attention");
    }
    return attention_merge(g, plan, state, out, pos, qh, max_ctx);
}

x0ne_status attention_merge(x0ne_gpu* g, const x0ne_split_plan& plan, const void* state, void* out, const void* pos,
                            uint32_t qh, uint32_t max_ctx) {
    uint32_t p = plan.splits;
    if (p == 0 || p > MAX_SPLITS) return fail(X0NE_ERR_GPU, "split-K: P " + std::to_string(p) + " outside 1..=256");
    g->counts.launches++;
    void* margs[] = {(void*)&state, (void*)&out, (void*)&pos, (void*)&max_ctx, (void*)&p};
    X0NE_HIP(x0ne_launch((const void*)&x0ne_attention_merge_bf16, dim3(qh), dim3(64), margs, 0, g->stream),
             "split-K merge");
    return X0NE_OK;
}

x0ne_status attention_rope_split(x0ne_gpu* g, const x0ne_split_plan& plan, const void* qkv, const void* q_norm,
                                 const void* k_norm, const void* inv_freq, const void* rope_cs, void* k, void* v,
                                 const void* pages,
                                 void* state, void* counter, void* out, const void* pos, uint32_t qh, uint32_t kvh,
                                 uint32_t max_ctx, float scale, float eps, bool exact) {
    const uint32_t p = plan.splits;
    if (p == 0 || p > MAX_SPLITS) return fail(X0NE_ERR_GPU, "split-K: P " + std::to_string(p) + " outside 1..=256");
    if (!plan.grouped || kvh == 0 || qh % kvh != 0 || plan.group != qh / kvh)
        return fail(X0NE_ERR_GPU, "fused attention needs a grouped plan of this geometry");
    const void* kern = exact ? exact_group_kernel(plan.group) : rope_group_kernel(plan.group);
    if (!kern) return fail(X0NE_ERR_GPU, "fused attention: no kernel for this group size");
    void* args[] = {(void*)&qkv,     (void*)&q_norm, (void*)&k_norm, (void*)&inv_freq, (void*)&rope_cs,
                    (void*)&k,       (void*)&v,      (void*)&pages,  (void*)&state,    (void*)&counter,
                    (void*)&out,     (void*)&pos,    (void*)&qh,     (void*)&kvh,      (void*)&max_ctx,
                    (void*)&p,       (void*)&scale,  (void*)&eps};
    g->counts.launches++;
    X0NE_HIP(x0ne_launch(kern, dim3(kvh, p), dim3(256), args, 0, g->stream),
             exact ? "exact decode attention" : "fused decode attention");
    return X0NE_OK;
}

}  // namespace x0ne

extern "C" x0ne_status x0ne_gpu_split_plan(const x0ne_gpu* g, uint32_t q_heads, uint32_t kv_heads,
                                           x0ne_split_plan* out) {
    if (!g || !out) return fail(X0NE_ERR_GPU, "no device");
    return split_plan(g, q_heads, kv_heads, out);
}

// x0ne_gpu_attention_split with its workspace in the library's scratch array: the states at its
// start, the counters after SCRATCH_STATE_BYTES. The counters are zeroed by a fill kernel first
// (a kernel, not a memset, so the call may be captured into a graph); nothing is allocated.
extern "C" x0ne_status x0ne_gpu_attention_split_scratch(x0ne_gpu* g, const x0ne_split_plan* plan, int last_block,
                                                        uint64_t q, uint64_t k, uint64_t v, uint64_t page_table,
                                                        uint64_t out, uint64_t pos, uint32_t q_heads,
                                                        uint32_t kv_heads, uint32_t max_ctx, float scale) {
    if (!g || !plan) return fail(X0NE_ERR_GPU, "no device");
    if (!g->scratch) return fail(X0NE_ERR_GPU, "no scratch array on this device");
    const uint64_t state_bytes = x0ne_split_state_bytes(q_heads, plan->splits);
    if (state_bytes > SCRATCH_STATE_BYTES || kv_heads > SCRATCH_COUNTERS)
        return fail(X0NE_ERR_FORMAT, "split-K scratch: " + std::to_string(q_heads) + " q heads x P " +
                                         std::to_string(plan->splits) + " need " + std::to_string(state_bytes) +
                                         " bytes of states and " + std::to_string(kv_heads) +
                                         " counters; the static scratch holds " +
                                         std::to_string(SCRATCH_STATE_BYTES) + " bytes and " +
                                         std::to_string(SCRATCH_COUNTERS) + " counters");
    uint8_t* base = static_cast<uint8_t*>(g->scratch);
    void* counter = base + SCRATCH_STATE_BYTES;
    if (last_block) {
        g->counts.launches++;
        X0NE_HIP(x0ne_launch_fill_u16(static_cast<uint16_t*>(counter), 2ull * kv_heads, 0, g->stream),
                 "zero the scratch counters");
    }
    return attention_split(g, *plan, last_block, (const void*)q, (const void*)k, (const void*)v, (const void*)page_table,
                           base, counter, (void*)out, (const void*)pos, q_heads, kv_heads, max_ctx, scale);
}

extern "C" x0ne_status x0ne_gpu_attention_split(x0ne_gpu* g, const x0ne_split_plan* plan, int last_block, uint64_t q,
                                                uint64_t k, uint64_t v, uint64_t page_table, uint64_t state,
                                                uint64_t counter, uint64_t out, uint64_t pos, uint32_t q_heads,
                                                uint32_t kv_heads, uint32_t max_ctx, float scale) {
    if (!g || !plan) return fail(X0NE_ERR_GPU, "no device");
    return attention_split(g, *plan, last_block, (const void*)q, (const void*)k, (const void*)v,
                           (const void*)page_table, (void*)state, (void*)counter, (void*)out, (const void*)pos,
                           q_heads, kv_heads, max_ctx, scale);
}

extern "C" x0ne_status x0ne_gpu_time_attention(x0ne_gpu* g, uint32_t q_heads, uint32_t kv_heads, uint32_t ctx,
                                               uint32_t splits, uint32_t iters, uint64_t seed, double* us,
                                               uint32_t* planes_out) {
    if (!g || !us) return fail(X0NE_ERR_GPU, "no device");
    if (ctx == 0 || iters == 0 || kv_heads == 0 || q_heads % kv_heads != 0 || splits == 0 || splits > MAX_SPLITS)
        return fail(X0NE_ERR_FORMAT, "time_attention: geometry");
    x0ne_split_plan plan = {};
    X0NE_TRY(split_plan(g, q_heads, kv_heads, &plan));
    if (!plan.grouped) return fail(X0NE_ERR_NOT_IMPLEMENTED, "time_attention: no grouped kernel for this group");
    plan.splits = splits;
    const uint64_t pages = (ctx + X0NE_PAGE_C - 1) / X0NE_PAGE_C;
    const uint64_t plane = pages * kv_heads * X0NE_PAGE_C * X0NE_HEAD_DIM_C * 2;
    // Enough distinct K/V planes to exceed twice the 256 MiB Infinity Cache, at least 2.
    const uint64_t n_planes = std::max<uint64_t>(2, (512ull << 20) / (2 * plane) + 1);
    std::vector<void*> kv(2 * n_planes, nullptr);
    void *q = nullptr, *out = nullptr, *state = nullptr, *counter = nullptr, *pt = nullptr, *posp = nullptr;
    std::vector<hipEvent_t> ev(2 * (size_t)iters, nullptr);
    x0ne_status st = X0NE_OK;
    auto hip = [&](hipError_t e, const char* what) {
        if (st == X0NE_OK && e != hipSuccess) st = gpu_fail(e, what);
    };
    for (auto& p : kv) hip(hipMalloc(&p, plane), "time_attention: planes");
    hip(hipMalloc(&q, (size_t)q_heads * X0NE_HEAD_DIM_C * 2), "time_attention: q");
    hip(hipMalloc(&out, (size_t)q_heads * X0NE_HEAD_DIM_C * 2), "time_attention: out");
    hip(hipMalloc(&state, x0ne_split_state_bytes(q_heads, splits)), "time_attention: state");
    hip(hipMalloc(&counter, kv_heads * 4), "time_attention: counter");
    hip(hipMalloc(&pt, pages * 4), "time_attention: page table");
    hip(hipMalloc(&posp, 4), "time_attention: pos");
    // Q, K and V N(0, 1) bf16 from the seed; pages in a splitmix64 Fisher-Yates order.
    for (size_t i = 0; i < kv.size() && st == X0NE_OK; ++i)
        hip(x0ne_launch_init_normal((uint16_t*)kv[i], plane / 2, seed + 1 + i, 0, 1.0, g->stream), "time_attention: K/V");
    if (st == X0NE_OK)
        hip(x0ne_launch_init_normal((uint16_t*)q, (uint64_t)q_heads * X0NE_HEAD_DIM_C, seed, 0, 1.0, g->stream),
            "time_attention: q");
    std::vector<uint32_t> order(pages);
    for (uint64_t i = 0; i < pages; ++i) order[i] = (uint32_t)i;
    uint64_t sm = seed;
    for (uint64_t i = pages; i > 1; --i) {
        sm += 0x9E3779B97F4A7C15ull;
        uint64_t z = sm;
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        z ^= z >> 31;
        std::swap(order[i - 1], order[z % i]);
    }
    const uint32_t pos = ctx - 1;
    hip(hipMemcpy(pt, order.data(), pages * 4, hipMemcpyHostToDevice), "time_attention: page table");
    hip(hipMemcpy(posp, &pos, 4, hipMemcpyHostToDevice), "time_attention: pos");
    hip(hipMemset(counter, 0, kv_heads * 4), "time_attention: counter");
    for (auto& x : ev) hip(hipEventCreate(&x), "time_attention: event");
    const float scale = (float)(1.0 / std::sqrt((double)X0NE_HEAD_DIM_C));
    auto launch = [&](uint64_t i) {
        if (st == X0NE_OK)
            st = attention_split(g, plan, 1, q, kv[2 * (i % n_planes)], kv[2 * (i % n_planes) + 1], pt, state, counter,
                                 out, posp, q_heads, kv_heads, ctx, scale);
    };
    for (uint64_t i = 0; i < n_planes; ++i) launch(i);  // warm-up: every plane once
    std::vector<X0neTimer> timers(iters);
    for (uint32_t i = 0; i < iters && st == X0NE_OK; ++i) {
        timers[i] = X0neTimer{ev[2 * i], ev[2 * i + 1], false};
        x0ne_timer = &timers[i];
        launch(n_planes + i);
        x0ne_timer = nullptr;
    }
    if (st == X0NE_OK) hip(hipStreamSynchronize(g->stream), "time_attention: sync");
    double total = 0.0;
    for (uint32_t i = 0; i < iters && st == X0NE_OK; ++i) {
        float ms = 0.f;
        hip(hipEventElapsedTime(&ms, ev[2 * i], ev[2 * i + 1]), "time_attention: elapsed");
        total += ms;
    }
    for (auto& x : ev)
        if (x) (void)hipEventDestroy(x);
    for (void* p : kv)
        if (p) (void)hipFree(p);
    for (void* p : {q, out, state, counter, pt, posp})
        if (p) (void)hipFree(p);
    if (st != X0NE_OK) return st;
    *us = total * 1000.0 / iters;
    if (planes_out) *planes_out = (uint32_t)n_planes;
    return X0NE_OK;
}

extern "C" uint64_t x0ne_split_state_bytes(uint32_t q_heads, uint32_t splits) {
    return (uint64_t)q_heads * splits * X0NE_SPLIT_STATE_C * 4;
}

// ---------------------------------------------------------------------------------------------
// Graph capture (gpu.rs:1170-1238)
// ---------------------------------------------------------------------------------------------

extern "C" x0ne_status x0ne_gpu_capture_begin(x0ne_gpu* g) {
    if (!g) return fail(X0NE_ERR_GPU, "no device");
    if (g->capturing) return fail(X0NE_ERR_GPU, "a capture is already open");
    X0NE_HIP(hipStreamBeginCapture(g->stream, hipStreamCaptureModeGlobal), "hipStreamBeginCapture");
    g->capturing = true;
    return X0NE_OK;
}

extern "C" x0ne_status x0ne_gpu_capture_end(x0ne_gpu* g, x0ne_graph** out) {
    if (!g || !out) return fail(X0NE_ERR_GPU, "no device");
    if (!g->capturing) return fail(X0NE_ERR_GPU, "no capture open");
    g->capturing = false;
    hipGraph_t graph = nullptr;
    X0NE_HIP(hipStreamEndCapture(g->stream, &graph), "hipStreamEndCapture");
    x0ne_graph* gr = new x0ne_graph();
    gr->graph = graph;
    size_t nodes = 0;
    (void)hipGraphGetNodes(graph, nullptr, &nodes);
    gr->nodes = nodes;
    gr->owner = g;
    hipError_t e = hipGraphInstantiate(&gr->exec, graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(graph);
        delete gr;
        return gpu_fail(e, "hipGraphInstantiate");
    }
    *out = gr;
    return X0NE_OK;
}

extern "C" x0ne_status x0ne_gpu_launch_graph(x0ne_gpu* g, const x0ne_graph* graph) {
    if (!g || !graph) return fail(X0NE_ERR_GPU, "no device or graph");
    // A graph's launches address its own Gpu's stream and memory (gpu.rs:1225-1230).
    if (graph->owner != g) return fail(X0NE_ERR_GPU, "graph captured by another Gpu");
    g->counts.graph_launches++;
    X0NE_HIP(hipGraphLaunch(graph->exec, g->stream), "hipGraphLaunch");
    return X0NE_OK;
}

extern "C" size_t x0ne_graph_nodes(const x0ne_graph* graph) { return graph ? graph->nodes : 0; }

extern "C" void x0ne_graph_free(x0ne_graph* graph) {
    if (!graph) return;
    if (graph->exec) (void)hipGraphExecDestroy(graph->exec);
    if (graph->graph) (void)hipGraphDestroy(graph->graph);
    delete graph;
}

// ---------------------------------------------------------------------------------------------
// The arena (arena.rs)
// ---------------------------------------------------------------------------------------------

extern "C" x0ne_status x0ne_arena_new(x0ne_arena** out) {
    if (!out) return fail(X0NE_ERR_ARENA, "null out");
    x0ne_arena* a = new x0ne_arena();
    a->id = g_next_arena.fetch_add(1);
    *out = a;
    return X0NE_OK;
}

extern "C" void x0ne_arena_free(x0ne_arena* a) {
    if (!a) return;
    if (a->base) {
        if (a->gpu) {
            (void)hipStreamSynchronize(a->gpu->stream);
            (void)hipFree(a->base);
        } else {
            std::free(a->base);
        }
    }
    delete a;
}

extern "C" x0ne_status x0ne_arena_alloc(x0ne_arena* a, const char* label, uint64_t len, uint32_t cls,
                                        x0ne_slice* out) {
    if (!a || !out) return fail(X0NE_ERR_ARENA, "null arena");
    const std::string l = label ? label : "";
    if (a->frozen) return fail(X0NE_ERR_ARENA, l + ": the arena is frozen, nothing can be added");
    if (len == 0) return fail(X0NE_ERR_ARENA, l + ": empty region");
    if (cls != X0NE_CLASS_WEIGHTS && cls != X0NE_CLASS_CLIENT_DATA) return fail(X0NE_ERR_ARENA, l + ": class");
    const uint64_t A = X0NE_ARENA_ALIGN;
    if (a->size > UINT64_MAX - (A - 1)) return fail(X0NE_ERR_ARENA, "size overflow");
    const uint64_t off = (a->size + A - 1) / A * A;
    if (off > UINT64_MAX - len) return fail(X0NE_ERR_ARENA, "size overflow");
    a->regions.push_back({l, cls, off, len});
    a->size = off + len;
    *out = {a->id, off, len};
    return X0NE_OK;
}

extern "C" uint64_t x0ne_arena_planned_bytes(const x0ne_arena* a) { return a ? a->size : 0; }

extern "C" x0ne_status x0ne_arena_freeze(x0ne_arena* a, x0ne_gpu* g) {
    if (!a) return fail(X0NE_ERR_ARENA, "null arena");
    if (a->frozen) return fail(X0NE_ERR_ARENA, "already frozen");
    const uint64_t len = a->size ? a->size : 1;
    if (g) {
        void* p = nullptr;
        hipError_t e = hipMalloc(&p, len);
        if (e != hipSuccess) return gpu_fail(e, ("hipMalloc of " + std::to_string(len) + " bytes").c_str());
        a->base = (uint8_t*)p;
        a->gpu = g;
    } else {
        if (len > (uint64_t)SIZE_MAX) return fail(X0NE_ERR_ARENA, "size exceeds host usize");
        void* p = nullptr;  // aligned like a device allocation, so a slice's address is aligned too
        a->base = posix_memalign(&p, X0NE_ARENA_ALIGN, (size_t)len) == 0 ? (uint8_t*)p : nullptr;
        if (!a->base) return fail(X0NE_ERR_ARENA, "host allocation of " + std::to_string(len) + " bytes");
        std::memset(a->base, 0xA5, len);
    }
    a->len = len;
    a->frozen = true;
    return X0NE_OK;
}

namespace x0ne {
x0ne_status arena_check(const x0ne_arena* a, x0ne_slice s, uint64_t at, uint64_t len, uint64_t* off) {
    if (!a->frozen) return fail(X0NE_ERR_ARENA, "the arena is not frozen");
    if (s.arena != a->id) return fail(X0NE_ERR_ARENA, "slice from another arena");
    if (at > UINT64_MAX - len || at + len > s.len)
        return fail(X0NE_ERR_ARENA, std::to_string(len) + " bytes at " + std::to_string(at) + " exceed a " +
                                        std::to_string(s.len) + "-byte slice");
    *off = s.offset + at;
    return X0NE_OK;
}
}  // namespace x0ne

extern "C" x0ne_status x0ne_arena_write(x0ne_arena* a, x0ne_slice s, uint64_t at, const void* data, uint64_t len) {
    if (!a) return fail(X0NE_ERR_ARENA, "null arena");
    uint64_t off;
    X0NE_TRY(arena_check(a, s, at, len, &off));
    if (len == 0) return X0NE_OK;
    if (a->gpu) {
        a->gpu->counts.htod++;
        X0NE_HIP(hipMemcpyAsync(a->base + off, data, len, hipMemcpyHostToDevice, a->gpu->stream), "arena write");
        a->gpu->counts.syncs++;
        X0NE_HIP(hipStreamSynchronize(a->gpu->stream), "arena write");
    } else {
        std::memcpy(a->base + off, data, len);
    }
    return X0NE_OK;
}

extern "C" x0ne_status x0ne_arena_read(const x0ne_arena* a, x0ne_slice s, uint64_t at, void* out, uint64_t len) {
    if (!a) return fail(X0NE_ERR_ARENA, "null arena");
    uint64_t off;
    X0NE_TRY(arena_check(a, s, at, len, &off));
    if (len == 0) return X0NE_OK;
    if (a->gpu) {
        a->gpu->counts.dtoh++;
        X0NE_HIP(hipMemcpyAsync(out, a->base + off, len, hipMemcpyDeviceToHost, a->gpu->stream), "arena read");
        a->gpu->counts.syncs++;
        X0NE_HIP(hipStreamSynchronize(a->gpu->stream), "arena read");
    } else {
        std::memcpy(out, a->base + off, len);
    }
    return X0NE_OK;
}

extern "C" x0ne_status x0ne_arena_addr(const x0ne_arena* a, x0ne_slice s, uint64_t at, uint64_t* out) {
    if (!a || !out) return fail(X0NE_ERR_ARENA, "null arena");
    uint64_t off;
    X0NE_TRY(arena_check(a, s, at, 0, &off));
    if (at >= s.len)
        return fail(X0NE_ERR_ARENA, "address " + std::to_string(at) + " past a " + std::to_string(s.len) + "-byte slice");
    *out = (uint64_t)(uintptr_t)(a->base + off);
    return X0NE_OK;
}

extern "C" x0ne_status x0ne_arena_span(const x0ne_arena* a, x0ne_slice s, uint64_t at, uint64_t len, uint64_t* out) {
    if (!a || !out) return fail(X0NE_ERR_ARENA, "null arena");
    if (len == 0) return fail(X0NE_ERR_ARENA, "empty span");
    uint64_t off;
    X0NE_TRY(arena_check(a, s, at, len, &off));
    *out = (uint64_t)(uintptr_t)(a->base + off);
    return X0NE_OK;
}

extern "C" x0ne_status x0ne_arena_scrub(x0ne_arena* a, uint64_t* zeroed) {
    if (!a) return fail(X0NE_ERR_ARENA, "null arena");
    if (!a->frozen) return fail(X0NE_ERR_ARENA, "the arena is not frozen");
    uint64_t total = 0;
    for (const auto& r : a->regions) {
        if (r.cls != X0NE_CLASS_CLIENT_DATA) continue;
        if (a->gpu) {
            a->gpu->counts.memsets++;
            X0NE_HIP(hipMemsetAsync(a->base + r.offset, 0, r.len, a->gpu->stream), "scrub");
        } else {
            std::memset(a->base + r.offset, 0, r.len);
        }
        total += r.len;
    }
    if (a->gpu) {
        a->gpu->counts.syncs++;
        X0NE_HIP(hipStreamSynchronize(a->gpu->stream), "scrub");
    }
    if (zeroed) *zeroed = total;
    return X0NE_OK;
}

extern "C" size_t x0ne_arena_region_count(const x0ne_arena* a) { return a ? a->regions.size() : 0; }

extern "C" x0ne_status x0ne_arena_region(const x0ne_arena* a, size_t i, char* label_buf, size_t label_len,
                                         uint32_t* cls, uint64_t* offset, uint64_t* len) {
    if (!a || i >= a->regions.size()) return fail(X0NE_ERR_ARENA, "no such region");
    const auto& r = a->regions[i];
    if (label_buf && label_len) {
        std::strncpy(label_buf, r.label.c_str(), label_len - 1);
        label_buf[label_len - 1] = 0;
    }
    if (cls) *cls = r.cls;
    if (offset) *offset = r.offset;
    if (len) *len = r.len;
    return X0NE_OK;
}

extern "C" x0ne_status x0ne_arena_region_slice(const x0ne_arena* a, size_t i, x0ne_slice* out) {
    if (!a || !out || i >= a->regions.size()) return fail(X0NE_ERR_ARENA, "no such region");
    *out = {a->id, a->regions[i].offset, a->regions[i].len};
    return X0NE_OK;
}

extern "C" int x0ne_arena_is_frozen(const x0ne_arena* a) { return a && a->frozen ? 1 : 0; }
