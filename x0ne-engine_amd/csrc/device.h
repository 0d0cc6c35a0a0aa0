// Device helpers for the gfx950 kernels: bf16 packing, 64-lane wavefront reductions, the KV page
// addressing. Every reduction runs in a fixed order, so a launch is bit-reproducible.
#pragma once
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

// Every attention and RoPE kernel is written for this head size (all Qwen3 dense models;
// x0ne-core/kernels/cuda/common.cuh:10-12).
#define X0NE_HEAD_DIM 128
// Positions per KV page: a page of one layer's K (or V) plane holds [kv_heads][16][128] bf16,
// so one kv head's 16 rows are 4 KiB contiguous.
#define X0NE_PAGE 16
// Split-K decode attention: keys per tile (one wavefront, 4 pages), and floats per partial
// state: m, l, 2 unused, o[128] (the reference's SPLIT_STATE, kernels/src/lib.rs:135-144).
#define X0NE_SPLIT_TILE 64
#define X0NE_SPLIT_STATE (X0NE_HEAD_DIM + 4)

typedef uint16_t bf16_t;

// Maximum and sum over the lanes n, n + 16, n + 32 and n + 48 of a wavefront (its four rows of
// 16), by the gfx950 row swaps (v_permlane16_swap, v_permlane32_swap: VALU, no LDS round trip).
// Each swap of a value with itself leaves a lane its own row's value and the partner row's; the
// sum adds rows 0 + 1 and 2 + 3, then the two pairs: the bits of two xor shuffles by 16 and 32.
__device__ __forceinline__ float rows_max(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float rows_sum(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

__device__ __forceinline__ float bf2f(bf16_t b) { return __uint_as_float((uint32_t)b << 16); }
__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// Nearest bf16, ties to even; a NaN keeps its sign and the high bits of its payload and gets the
// quiet bit (the reference's rounding, x0ne-core/oracle/src/bf16.rs:11-20), stated on the bits:
// adding 0x7FFF plus the kept part's lowest bit carries into the kept part exactly when the
// dropped half is above 0x8000, or equal to it with that bit odd.
__device__ __forceinline__ bf16_t f2bf_bits(float x) {
    const uint32_t b = __float_as_uint(x);
    const uint32_t rounded = (b + 0x7FFFu + ((b >> 16) & 1u)) >> 16;
    return (bf16_t)(x != x ? ((b >> 16) | 0x0040u) : rounded);
}

// The same rounding by the hardware (v_cvt_pk_bf16_f32, nearest-even mode, f32 denormals kept):
// x0ne_probe_bf16_round checks it against f2bf_bits on all 2^32 inputs.
__device__ __forceinline__ bf16_t f2bf(float x) { return __builtin_bit_cast(bf16_t, (__bf16)x); }

__device__ __forceinline__ float bf_round(float x) { return bf2f(f2bf(x)); }

// ---- 64-lane reductions (xor butterflies: every lane ends with the same value) ----

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// A barrier for data exchanged through LDS only: this wavefront's LDS operations are complete,
// then all wavefronts meet. Unlike __syncthreads() it does not wait for outstanding global loads
// (the workgroup fence does), so loads requested before it stay in flight across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Sum over a block of WAVES wavefronts in f64, exchanged through LDS `sh` (one double per
// wavefront) with LDS-only barriers. The block size is a compile-time constant: reading
// blockDim is a memory load, and waiting for it would wait for every load issued before.
template <int WAVES>
__device__ __forceinline__ double block_sum_lds(double v, double* sh) {
    v = wave_sum_d(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    lds_barrier();
    if (lane == 0) sh[wave] = v;
    lds_barrier();
    double t = 0.0;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) t += sh[w];
    return t;
}

// Sum over a block of `blockDim.x` threads (a multiple of 64, at most 1024); every thread gets
// it. `sh` holds 16 doubles. Wave sums, then the wave sums in wave order.
__device__ __forceinline__ double block_sum_d(double v, double* sh) {
    v = wave_sum_d(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if (lane == 0) sh[wave] = v;
    __syncthreads();
    double t = 0.0;
    for (int w = 0; w < nw; ++w) t += sh[w];
    return t;
}

// ---- GEMV row sums (the decode GEMV and the O projection fused behind the decode attention) ----

template <class A>
__device__ __forceinline__ A dot8(const uint4 w, const A* x, A acc);

template <>
__device__ __forceinline__ float dot8<float>(const uint4 w, const float* x, float acc) {
    acc = fmaf(bf_lo(w.x), x[0], acc);
    acc = fmaf(bf_hi(w.x), x[1], acc);
    acc = fmaf(bf_lo(w.y), x[2], acc);
    acc = fmaf(bf_hi(w.y), x[3], acc);
    acc = fmaf(bf_lo(w.z), x[4], acc);
    acc = fmaf(bf_hi(w.z), x[5], acc);
    acc = fmaf(bf_lo(w.w), x[6], acc);
    acc = fmaf(bf_hi(w.w), x[7], acc);
    return acc;
}

// x already in f64. The product of two bf16 values is exact in f64, so each FMA is the exact
// product added to the sum with one rounding, as the f64 oracle sums (w as f64 times x, added).
template <>
__device__ __forceinline__ double dot8<double>(const uint4 w, const double* x, double acc) {
    acc = fma((double)bf_lo(w.x), x[0], acc);
    acc = fma((double)bf_hi(w.x), x[1], acc);
    acc = fma((double)bf_lo(w.y), x[2], acc);
    acc = fma((double)bf_hi(w.y), x[3], acc);
    acc = fma((double)bf_lo(w.z), x[4], acc);
    acc = fma((double)bf_hi(w.z), x[5], acc);
    acc = fma((double)bf_lo(w.w), x[6], acc);
    acc = fma((double)bf_hi(w.w), x[7], acc);
    return acc;
}

// Sum of R values over the 64 lanes. At the first log2(R) steps (lane bits 5, 4, ...) each lane
// keeps half of its values (bit set: the upper half) and adds its partner's copy of them; the
// remaining steps are plain butterflies. Lane l ends with the sum of value reduced_row<R>(l).
template <int N, int K, class A>
struct RowReduce {
    static __device__ __forceinline__ void run(A* v, uint32_t lane) {
        constexpr int H = N >> 1;
        const bool bit = (lane >> K) & 1u;
#pragma unroll
        for (int j = 0; j < H; ++j) {
            const A send = bit ? v[j] : v[j + H];
            const A keep = bit ? v[j + H] : v[j];
            v[j] = keep + __shfl_xor(send, 1 << K, 64);
        }
        RowReduce<H, K - 1, A>::run(v, lane);
    }
};
template <int K, class A>
struct RowReduce<1, K, A> {
    static __device__ __forceinline__ void run(A* v, uint32_t lane) {
        v[0] += __shfl_xor(v[0], 1 << K, 64);
        RowReduce<1, K - 1, A>::run(v, lane);
    }
};
template <class A>
struct RowReduce<1, -1, A> {
    static __device__ __forceinline__ void run(A*, uint32_t) {}
};
// f64 values moved between lanes of a row of 16 by DPP (a VALU operand modifier, no LDS round
// trip), the two 32-bit halves alike: CTRL 0x124 / 0x128 rotate the row by 4 / 8 lanes, 0x4E
// and 0xB1 swap lanes by xor 2 and xor 1 within each group of 4.
template <int CTRL>
__device__ __forceinline__ double dpp_d(double v) {
    const uint64_t u = (uint64_t)__double_as_longlong(v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, 0xF, 0xF, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, 0xF, 0xF, false);
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}
// The last four steps of an f64 sum (lane bits 3..0) within each row of 16: the rotations by 4
// and 8 leave every lane the sum of its 4 lanes of equal index mod 4, the two swaps add the 4
// such sums; each lane ends with the whole row's sum (in an association of its own). The f32
// sums keep their xor butterflies (measured no faster with this, and their bits are the tests'
// recorded ones).
template <>
struct RowReduce<1, 3, double> {
    static __device__ __forceinline__ void run(double* v, uint32_t) {
        double x = v[0];
        x += dpp_d<0x124>(x);
        x += dpp_d<0x128>(x);
        x += dpp_d<0x4E>(x);
        x += dpp_d<0xB1>(x);
        v[0] = x;
    }
};

template <int R, class A>
__device__ __forceinline__ A wave_reduce_rows(A* v) {
    RowReduce<R, 5, A>::run(v, threadIdx.x & 63);
    return v[0];
}

template <int R>
__device__ __forceinline__ uint32_t reduced_row(uint32_t lane) {
    uint32_t idx = 0;
    int n = R;
#pragma unroll
    for (int k = 5; k >= 0; --k) {
        if (n > 1) {
            const int h = n >> 1;
            if ((lane >> k) & 1u) idx += h;
            n = h;
        }
    }
    return idx;
}

// ---- panels ----
// A [rows][cols] bf16 matrix (cols a multiple of 8) kept as ceil(rows / 16) panels of
// [cols / 8][16][8]: element (t, k) at ((t / 16 cols / 8 + k / 8) 16 + t % 16) 8 + k % 8. The
// 16 rows' pieces of 8 columns sit together, so the few-row GEMM (gemm.hip) reads one step of
// its X operand as one contiguous KiB; the batched step's producers of X write this layout.
__device__ __forceinline__ size_t panel_index(uint32_t t, uint32_t k, uint32_t cols) {
    return ((size_t)((t >> 4) * (cols >> 3) + (k >> 3)) * 16 + (t & 15)) * 8 + (k & 7);
}

// ---- KV pages ----
// A layer's K plane is [pages][kv_heads][16][128] bf16 (a key row of 128 dims contiguous); its
// V plane is [pages][kv_heads][128][16] (dim-major within a page: the 16 positions of one dim
// contiguous, the operand layout of the matrix-core P·V product). page_table maps a sequence's
// logical page (position / 16) to its physical page.
__device__ __forceinline__ uint32_t kv_row(const uint32_t* __restrict__ pages, uint32_t pos, uint32_t kh,
                                         uint32_t kv_heads) {
    const uint32_t page = pages[pos / X0NE_PAGE];
    return ((page * kv_heads + kh) * X0NE_PAGE + (pos % X0NE_PAGE)) * X0NE_HEAD_DIM;
}

// Element (pos, dim 0) of a V plane; dim d is at + d * 16.
__device__ __forceinline__ uint32_t v_slot(const uint32_t* __restrict__ pages, uint32_t pos, uint32_t kh,
                                         uint32_t kv_heads) {
    const uint32_t page = pages[pos / X0NE_PAGE];
    return (page * kv_heads + kh) * X0NE_HEAD_DIM * X0NE_PAGE + (pos % X0NE_PAGE);
}
