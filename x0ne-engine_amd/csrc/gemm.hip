// The projections of a pass over a few rows (the batched decode step, a short prompt) on the
// matrix cores: Y[n][rows] = X[n][cols] W^T with W [rows][cols] and X [n][cols] bf16 row-major,
// f32 accumulation, Y bf16 or f32 (the reference's Gpu::gemm, gpu.rs:1098-1149). At one row the
// decode GEMV (gemv.hip) is the right kernel; past 64 rows the work is a compute-bound GEMM,
// which the runtime hands to hipBLASLt as the reference hands it to cuBLAS (runtime.hip).
#include "device.h"

namespace {

constexpr uint32_t RSRC_WORD3 = 0x00020000;
constexpr uint32_t OFF_NONE = 0xFFFFFFF0u;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4 mfma(uint4 a, uint4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint64_t bytes) {
    // A byte count past 4 GiB - 16 is clamped there: offsets are 32-bit.
    const uint32_t n = bytes > OFF_NONE ? OFF_NONE : (uint32_t)bytes;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)n, RSRC_WORD3);
}

// The default cache policy throughout: a non-temporal hint on the few-row GEMM's weight stream
// (which speeds the decode GEMV's, gemv.hip) made its launches 5-15 % slower on MI355X.
__device__ __forceinline__ uint4 bload(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
    return make_uint4((uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]);
}

}  // namespace

// ---- a few rows: Y[n][rows] = X[n][cols] W^T for n <= 64, bandwidth-bound ----
// The batched decode step's projections and a short prompt's. Every W row is read once, so the
// kernel streams W at the HBM rate and the few-row matrix-core products cost nothing beside it:
//  - Block b takes the RG row groups of 16 W rows 16 RG b .. 16 RG b + 16 RG - 1 over all of K;
//    its V wavefronts (V = blockDim / 64, chosen by the host with RG so the launch holds enough
//    loads in flight) take V contiguous runs of K, in whole steps of 32 columns.
//  - A step is TT x RG 16 x 16 x 32 products (TT tiles of 16 tokens, RG row groups) whose A
//    operand is X (row = token, zero past n) and B operand W (column = W row): lane l loads
//    16 bytes, columns k0 + 8 (l / 16) .. + 7, of W row 16 (RG b + g) + l % 16 and of X row
//    16 tt + l % 16; the 4 lane groups cover 64 contiguous bytes of each row. One X piece
//    serves the RG row groups, so X (read from the L2 by every block) costs TT / RG of W's loads.
//  - U steps are in flight per wavefront: the slot a product has consumed is refilled at once
//    with the step U ahead, so U - 1 steps stay in flight while one multiplies. A piece past K
//    (or a token past n, a W row past rows) is a raw buffer load at an offset past the buffer,
//    which returns zeros without touching memory.
//  - The wavefronts' partial tiles are summed in LDS in wavefront order (deterministic).
// flags: FEW_F32 Y f32 (else bf16); FEW_X_PANEL X in panels (below); FEW_Y_PANEL Y in panels
// (bf16); FEW_W_PANEL W in panels (rows a multiple of 16; with SwiGLU the [gate; up] matrix of
// 2 rows rows in panels, so gate and up panels do not mix). GLU: SwiGLU over the packed [gate; up] W of 2 rows rows: the block also takes the up
// rows rows + 16 (RG b + g) .., and writes act[t][r] = bf16(g / (1 + e^-g) u) of the
// bf16-rounded g and u, in f64 (x0ne_swiglu_bf16 of the bf16 projection).
//
// Panels: a [n][cols] bf16 matrix stored as ceil(n / 16) panels of [cols / 8][16][8]: element
// (t, k) at ((t / 16 * cols / 8 + k / 8) 16 + t % 16) 8 + k % 8. One step's X operand is then one
// contiguous KiB; row-major, its 16 rows lie cols apart and meet in the same L2 channels, which
// costs the W stream up to a fifth of its rate at 16 rows (measured on MI355X). W is laid out the
// same way for the same reason: row-major, each step reads 64 bytes of 16 rows cols apart, and
// the W stream of the Qwen3 decode shapes runs at 3.1-5.1 TB/s; in panels each step reads one
// contiguous KiB and a wavefront's steps run through its panel in order, 3.7-5.9 TB/s (MI355X).
namespace {

constexpr uint32_t FEW_F32 = 1, FEW_X_PANEL = 2, FEW_Y_PANEL = 4, FEW_W_PANEL = 8;

template <int TT, int RG, int U, bool GLU, int MAXV>
__device__ __forceinline__ void few_rows(const bf16_t* __restrict__ w, const bf16_t* __restrict__ x,
                                         void* __restrict__ y, uint32_t rows, uint32_t cols, uint32_t n,
                                         uint32_t flags, f32x4* part) {
    constexpr int KINDS = GLU ? 2 : 1;
    const uint32_t b = blockIdx.x, V = blockDim.x >> 6;
    const bool out_f32 = flags & FEW_F32, x_panel = flags & FEW_X_PANEL, y_panel = flags & FEW_Y_PANEL;
    const bool w_panel = flags & FEW_W_PANEL;
    // Grid-uniform exits for a launch that does not fit.
    if (b * 16 * RG >= rows || n == 0 || n > 16 * TT || cols % 8 != 0 || V > MAXV || flags > 15 ||
        (out_f32 && (GLU || y_panel)) || (y_panel && rows % 8 != 0) || (w_panel && rows % 16 != 0))
        return;
    const uint32_t lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t r = lane & 15, q4 = lane >> 4;
    // Panels hold whole tiles of 16 rows.
    const auto xr = rsrc(x, (uint64_t)(x_panel ? (n + 15) / 16 * 16 : n) * cols * 2);
    const auto wr = rsrc(w, (uint64_t)KINDS * rows * cols * 2);
    const uint32_t steps = (cols + 31) / 32, per = (steps + V - 1) / V;
    const uint32_t s_begin = min(wave * per, steps), s_end = min(s_begin + per, steps);
    f32x4 acc[KINDS][RG][TT];
#pragma unroll
    for (int kd = 0; kd < KINDS; ++kd)
#pragma unroll
        for (int g = 0; g < RG; ++g)
#pragma unroll
            for (int tt = 0; tt < TT; ++tt) acc[kd][g][tt] = f32x4{0.f, 0.f, 0.f, 0.f};
    uint4 xa[U][TT], wb[U][KINDS][RG];
    auto request = [&](int u, uint32_t s) {
        const uint32_t k = 32 * s + 8 * q4;
        const bool in = s < s_end && k < cols;  // a K tail: pieces past the row read zeros
#pragma unroll
        for (int tt = 0; tt < TT; ++tt) {
            const uint32_t t = 16 * tt + r;
            const uint32_t off = x_panel ? (uint32_t)panel_index(t, k, cols) * 2 : (t * cols + k) * 2;
            xa[u][tt] = bload(xr, in && t < n ? off : OFF_NONE);
        }
#pragma unroll
        for (int kd = 0; kd < KINDS; ++kd)
#pragma unroll
            for (int g = 0; g < RG; ++g) {
                const uint32_t row = 16 * (RG * b + g) + r;
                const uint32_t wrow = kd * rows + row;
                wb[u][kd][g] = bload(wr, !(in && row < rows) ? OFF_NONE
                                         : w_panel ? (uint32_t)panel_index(wrow, k, cols) * 2
                                                   : (wrow * cols + k) * 2);
            }
    };
#pragma unroll
    for (int u = 0; u < U; ++u) request(u, s_begin + u);
    for (uint32_t s0 = s_begin; s0 < s_end; s0 += U) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
#pragma unroll
            for (int kd = 0; kd < KINDS; ++kd)
#pragma unroll
                for (int g = 0; g < RG; ++g)
#pragma unroll
                    for (int tt = 0; tt < TT; ++tt) acc[kd][g][tt] = mfma(xa[u][tt], wb[u][kd][g], acc[kd][g][tt]);
            request(u, s0 + U + u);
        }
    }
    // part[(((kd V + wave) RG + g) TT + tt) 64 + lane]
    auto at = [&](uint32_t kd, uint32_t v, uint32_t g, uint32_t tt) { return (((kd * V + v) * RG + g) * TT + tt) * 64 + lane; };
#pragma unroll
    for (int kd = 0; kd < KINDS; ++kd)
#pragma unroll
        for (int g = 0; g < RG; ++g)
#pragma unroll
            for (int tt = 0; tt < TT; ++tt) part[at(kd, wave, g, tt)] = acc[kd][g][tt];
    lds_barrier();
    // Wavefront w sums row groups w, w + V, ..: the V partials of each in wavefront order.
    for (uint32_t g = wave; g < (uint32_t)RG; g += V) {
        const uint32_t wrow = 16 * (RG * b + g) + r;
        if (wrow >= rows) continue;
#pragma unroll
        for (int tt = 0; tt < TT; ++tt) {
            f32x4 sg = part[at(0, 0, g, tt)], su = GLU ? part[at(1, 0, g, tt)] : f32x4{0.f, 0.f, 0.f, 0.f};
            for (uint32_t v = 1; v < V; ++v) {
                sg += part[at(0, v, g, tt)];
                if (GLU) su += part[at(1, v, g, tt)];
            }
            // sg[i]: token 16 tt + 4 (lane / 16) + i, W row wrow.
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t t = 16 * tt + 4 * q4 + i;
                if (t >= n) continue;
                const size_t o = y_panel ? panel_index(t, wrow, rows) : (size_t)t * rows + wrow;
                if (GLU) {
                    const double gv = (double)bf2f(f2bf(sg[i])), uv = (double)bf2f(f2bf(su[i]));
                    static_cast<bf16_t*>(y)[o] = f2bf((float)(gv / (1.0 + exp(-gv)) * uv));
                } else if (out_f32) {
                    static_cast<float*>(y)[o] = sg[i];
                } else {
                    static_cast<bf16_t*>(y)[o] = f2bf(sg[i]);
                }
            }
        }
    }
}

}  // namespace

// x0ne_gemm_few_t{TT}_r{RG}[_swiglu]_bf16: grid (ceil(rows / (16 RG))), block 64 V threads
// (V <= MAXV); n in 1 .. 16 TT; cols a multiple of 8 (of 8 and rows of 8 for a Y panel); X, W
// below 4 GiB - 16 bytes; flags as above (FEW_F32 = 1 not with SwiGLU or a Y panel).
#define X0NE_FEW(NAME, TT, RG, U, GLU, MAXV)                                                                     \
    extern "C" __global__ void __launch_bounds__(64 * MAXV)                                                       \
        NAME(const bf16_t* __restrict__ w, const bf16_t* __restrict__ x, void* __restrict__ y, uint32_t rows,     \
             uint32_t cols, uint32_t n, uint32_t flags) {                                                         \
        __shared__ f32x4 part[(GLU ? 2 : 1) * MAXV * RG * TT * 64];                                               \
        few_rows<TT, RG, U, GLU, MAXV>(w, x, y, rows, cols, n, flags, part);                                      \
    }
#ifndef X0NE_FEW_NO_TABLE
X0NE_FEW(x0ne_gemm_few_t1_r1_bf16, 1, 1, 12, false, 8)
X0NE_FEW(x0ne_gemm_few_t1_r2_bf16, 1, 2, 4, false, 8)
X0NE_FEW(x0ne_gemm_few_t1_r4_bf16, 1, 4, 8, false, 8)
X0NE_FEW(x0ne_gemm_few_t1_r8_bf16, 1, 8, 4, false, 8)
X0NE_FEW(x0ne_gemm_few_t1_r1_swiglu_bf16, 1, 1, 4, true, 8)
X0NE_FEW(x0ne_gemm_few_t1_r2_swiglu_bf16, 1, 2, 4, true, 8)
X0NE_FEW(x0ne_gemm_few_t2_r1_bf16, 2, 1, 8, false, 8)
X0NE_FEW(x0ne_gemm_few_t2_r2_bf16, 2, 2, 4, false, 8)
X0NE_FEW(x0ne_gemm_few_t2_r1_swiglu_bf16, 2, 1, 4, true, 8)
X0NE_FEW(x0ne_gemm_few_t4_r1_bf16, 4, 1, 4, false, 8)
X0NE_FEW(x0ne_gemm_few_t4_r1_swiglu_bf16, 4, 1, 4, true, 8)
#endif

// x0ne_panel_bf16: a row-major [rows][cols] bf16 matrix copied into 16-row panels (element (r, k)
// at panel_index(r, k, cols)), one 16-byte chunk per thread in destination order, so the writes
// are contiguous; grid ceil(rows cols / 8 / 256), block 256. rows a multiple of 16 and cols of 8,
// else nothing is written. The source and destination must not overlap.
extern "C" __global__ void __launch_bounds__(256)
    x0ne_panel_bf16(const bf16_t* __restrict__ src, bf16_t* __restrict__ dst, uint32_t rows, uint32_t cols) {
    if (rows % 16 != 0 || cols % 8 != 0) return;  // grid-uniform
    const uint64_t c8 = cols / 8, j = (uint64_t)blockIdx.x * 256 + threadIdx.x;  // destination chunk
    if (j >= (uint64_t)rows * c8) return;
    const uint64_t r = j / (16 * c8) * 16 + j % 16, k8 = j / 16 % c8;
    reinterpret_cast<uint4*>(dst)[j] = reinterpret_cast<const uint4*>(src)[r * c8 + k8];
}
