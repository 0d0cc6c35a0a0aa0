// Typed launchers of the fused kernels, for the runtime (host side of this library).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

// One fused GEMV launch (gemv.hip). prologue: 0 x given, 1 add+RMSNorm, 2 embedding+RMSNorm;
// epilogue: 0 bf16 out, 1 f32 out, 2 SwiGLU over [gate; up], 3 f32 logits + argmax.
struct X0neGemv {
    const uint16_t* w;
    const uint16_t* x;
    const float* res_in;
    float* res_out;
    const uint16_t* delta;
    const uint16_t* norm_w;
    const uint16_t* embed;
    const uint32_t* tokens;
    void* y;
    float* partial;
    uint32_t* counter;
    uint32_t* token_out;
    uint32_t* pos;
    uint32_t rows, cols, vocab, advance;
    float eps;
    int prologue, epilogue;
    uint32_t grid;
    int f64acc;  // 1: products added in f64 (the oracle's sums), 0: f32 FMA
};

// Kernel-time measurement. While x0ne_timer is set (this thread only), x0ne_launch records
// `start` at the start of the first kernel it launches and `stop` at the end of each one
// (hipExtLaunchKernel's events carry the kernel's own begin and end), so the pair brackets the
// kernels of one operation and not the gaps before it.
struct X0neTimer {
    hipEvent_t start;
    hipEvent_t stop;
    bool started;
};
extern thread_local X0neTimer* x0ne_timer;
// Every kernel of the decode step is launched through this.
hipError_t x0ne_launch(const void* fn, dim3 grid, dim3 block, void** args, size_t lds, hipStream_t s);

hipError_t x0ne_launch_gemv(const X0neGemv& g, hipStream_t s);
// Blocks for a launch of this shape, prologue, epilogue and accumulation on `cus` CUs (0 for a
// shape the kernel refuses); max_blocks_per_cu 0 means the kernel's occupancy.
uint32_t x0ne_gemv_grid(const X0neGemv& g, uint32_t cus, uint32_t max_blocks_per_cu);

// The tiled matrix-core GEMM for many rows (gemm.hip): Y[n][rows] = X[n][cols] W^T, bf16 W and X,
// f32 accumulation, bf16 or f32 Y (row-major); rows a multiple of 4, cols of 8, W and X below
// 4 GiB - 16 bytes, Y 8-byte (bf16) or 16-byte (f32) aligned. flags: X0NE_TILE_F32 for f32 Y,
// X0NE_TILE_W_PANEL / X0NE_TILE_X_PANEL for W / X in 16-row panels (device.h; W's rows then a
// multiple of 16, X's panels hold ceil(n / 16) whole panels). `tile` names the block tile
// (features x tokens); x0ne_gemm_tile_pick chooses one for a shape.
enum { X0NE_TILE_256x256 = 1, X0NE_TILE_256x128 = 2, X0NE_TILE_128x128 = 3 };
enum { X0NE_TILE_F32 = 1, X0NE_TILE_W_PANEL = 2, X0NE_TILE_X_PANEL = 4 };
int x0ne_gemm_tile_pick(uint32_t rows, uint32_t cols, uint32_t n, uint32_t cus);
hipError_t x0ne_launch_gemm_tiles(int tile, const void* w, const void* x, void* y, uint32_t rows, uint32_t cols,
                                  uint32_t n, uint32_t flags, hipStream_t s);

// Device weight initialisers (init.hip): n values of N(0, std) bf16 from stream `key`
// starting at value `first` (even), and a constant fill.
hipError_t x0ne_launch_init_normal(uint16_t* out, uint64_t n, uint64_t key, uint64_t first, double std_dev,
                                   hipStream_t s);
hipError_t x0ne_launch_fill_u16(uint16_t* out, uint64_t n, uint16_t v, hipStream_t s);
