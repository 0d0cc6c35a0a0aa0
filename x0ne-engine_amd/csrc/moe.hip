// The sparse feed-forward of Qwen3-MoE (the reference's GM1 block, x0ne-core/kernels/cuda/moe.cu):
// the routing of the router's f32 logits, the expert GEMVs through expert ids held in device
// memory (so a captured decode step replays with whatever the routing chose), and the weighted
// combination. A row whose routing is undefined (a non-finite router logit) gets the expert id
// X0NE_MOE_NO_EXPERT and NaN weights; the expert GEMVs then write NaN rows, so the logits are NaN
// and the greedy argmax refuses the token.
//
// Launch shapes are written at each kernel. Wave64 throughout: the routing reduces over 2
// wavefronts, the expert GEMV gives each W row one wavefront (16-byte loads, f32 lanes, a fixed
// xor-butterfly sum), the combination is one thread per output value.
#include "device.h"
#include "kernels.h"

namespace {

constexpr uint32_t MOE_MAX_EXPERTS = 1024;  // kernels/src/lib.rs:147
constexpr uint32_t MOE_NO_EXPERT = 0xFFFFFFFFu;  // kernels/src/lib.rs:151
constexpr uint32_t MOE_MAX_TOP_K = 32;
constexpr uint32_t ROUTE_THREADS = 128;

// The routing order (moe.cu:6-8, lib.rs:268-270): the larger logit, then the smaller index;
// -0.0 equals 0.0.
__device__ __forceinline__ bool route_better(float v, uint32_t i, float bv, uint32_t bi) {
    return v > bv || (v == bv && i < bi);
}

// One W row per wavefront: y[slot][r] = W[ids[slot]][r] . x[slot / x_group], lanes striding
// over the 16-byte chunks of the row, f32 multiply-adds in chunk order, then the butterfly sum.
template <bool F32>
__device__ __forceinline__ void moe_gemv_row(const bf16_t* __restrict__ w, const uint32_t* __restrict__ ids,
                                             const bf16_t* __restrict__ x, void* __restrict__ y, uint32_t rows,
                                             uint32_t cols, uint32_t experts, uint32_t x_group, uint32_t x_stride) {
    const uint32_t lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t r = blockIdx.x * 4 + wave, slot = blockIdx.y;
    if (r >= rows || x_group == 0 || cols % 8 != 0) return;  // wavefront-uniform
    const uint32_t e = __builtin_amdgcn_readfirstlane(ids[slot]);
    const size_t o = (size_t)slot * rows + r;
    if (e >= experts) {  // no expert: the row is NaN
        if (lane == 0) {
            if (F32)
                static_cast<float*>(y)[o] = __uint_as_float(0x7FC00000u);
            else
                static_cast<bf16_t*>(y)[o] = (bf16_t)0x7FC0u;
        }
        return;
    }
    const uint4* wr = reinterpret_cast<const uint4*>(w + ((size_t)e * rows + r) * cols);
    const uint4* xr = reinterpret_cast<const uint4*>(x + (size_t)(slot / x_group) * x_stride);
    float acc = 0.f;
    const uint32_t chunks = cols / 8;
#pragma unroll 4
    for (uint32_t c = lane; c < chunks; c += 64) {
        const uint4 a = wr[c], b = xr[c];
        acc = fmaf(bf_lo(a.x), bf_lo(b.x), acc);
        acc = fmaf(bf_hi(a.x), bf_hi(b.x), acc);
        acc = fmaf(bf_lo(a.y), bf_lo(b.y), acc);
        acc = fmaf(bf_hi(a.y), bf_hi(b.y), acc);
        acc = fmaf(bf_lo(a.z), bf_lo(b.z), acc);
        acc = fmaf(bf_hi(a.z), bf_hi(b.z), acc);
        acc = fmaf(bf_lo(a.w), bf_lo(b.w), acc);
        acc = fmaf(bf_hi(a.w), bf_hi(b.w), acc);
    }
    acc = wave_sum(acc);
    if (lane == 0) {
        if (F32)
            static_cast<float*>(y)[o] = acc;
        else
            static_cast<bf16_t*>(y)[o] = f2bf(acc);
    }
}

}  // namespace

// x0ne_moe_route_f32 (moe.cu:10-80): grid (rows), block 128. Per row of `experts` f32 router
// logits, the top_k experts in routing order into ids[row][..] and their weights
// exp(l_e - l_max) / sum over the chosen, in f64, rounded once to f32 (the softmax denominator
// over every expert cancels in the renormalisation). experts in 1..=1024, top_k in
// 1..=min(32, experts); other launches write nothing.
extern "C" __global__ void __launch_bounds__(ROUTE_THREADS)
    x0ne_moe_route_f32(const float* __restrict__ logits, uint32_t experts, uint32_t top_k, uint32_t* __restrict__ ids,
                       float* __restrict__ weights) {
    __shared__ float vals[MOE_MAX_EXPERTS];
    __shared__ uint8_t taken[MOE_MAX_EXPERTS];
    __shared__ float sv[ROUTE_THREADS / 64];
    __shared__ uint32_t si[ROUTE_THREADS / 64];
    __shared__ uint32_t chosen[MOE_MAX_TOP_K];
    if (experts == 0 || experts > MOE_MAX_EXPERTS || top_k == 0 || top_k > MOE_MAX_TOP_K || top_k > experts ||
        blockDim.x != ROUTE_THREADS)
        return;  // grid-uniform
    const uint32_t t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const float* row = logits + (size_t)blockIdx.x * experts;
    uint32_t* row_ids = ids + (size_t)blockIdx.x * top_k;
    float* row_w = weights + (size_t)blockIdx.x * top_k;
    bool bad = false;
    for (uint32_t i = t; i < experts; i += ROUTE_THREADS) {
        const float v = row[i];
        vals[i] = v;
        taken[i] = 0;
        bad |= !isfinite(v);
    }
    if (__syncthreads_or(bad)) {
        if (t < top_k) {
            row_ids[t] = MOE_NO_EXPERT;
            row_w[t] = __uint_as_float(0x7FC00000u);
        }
        return;
    }
    for (uint32_t s = 0; s < top_k; ++s) {
        float bv = -INFINITY;
        uint32_t bi = 0xFFFFFFFFu;
        for (uint32_t i = t; i < experts; i += ROUTE_THREADS)
            if (!taken[i] && route_better(vals[i], i, bv, bi)) {
                bv = vals[i];
                bi = i;
            }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(bv, o, 64);
            const uint32_t oi = __shfl_xor(bi, o, 64);
            if (route_better(ov, oi, bv, bi)) {
                bv = ov;
                bi = oi;
            }
        }
        if (lane == 0) {
            sv[wave] = bv;
            si[wave] = bi;
        }
        __syncthreads();
        if (t == 0) {
            float v = sv[0];
            uint32_t b = si[0];
            for (uint32_t k = 1; k < ROUTE_THREADS / 64; ++k)
                if (route_better(sv[k], si[k], v, b)) {
                    v = sv[k];
                    b = si[k];
                }
            chosen[s] = b;
            taken[b] = 1;
        }
        __syncthreads();
    }
    if (t == 0) {
        const double m = (double)vals[chosen[0]];
        double e[MOE_MAX_TOP_K], sum = 0.0;
        for (uint32_t s = 0; s < top_k; ++s) {
            e[s] = exp((double)vals[chosen[s]] - m);
            sum += e[s];
        }
        for (uint32_t s = 0; s < top_k; ++s) {
            row_ids[s] = chosen[s];
            row_w[s] = (float)(e[s] / sum);
        }
    }
}

// x0ne_moe_gemv_bf16 / _f32 (moe.cu:84-133): grid (ceil(rows / 4), slots), block 256. For each
// slot s, y[s][0..rows) = W[ids[s]] x[s / x_group], W [experts][rows][cols] bf16, x rows
// x_stride apart; y bf16 (the [gate; up] rows) or f32 (the down rows, kept for the combination).
// cols a multiple of 8, W and x 16-byte aligned. An id >= experts writes a NaN row without
// reading W.
extern "C" __global__ void __launch_bounds__(256)
    x0ne_moe_gemv_bf16(const bf16_t* __restrict__ w, const uint32_t* __restrict__ ids, const bf16_t* __restrict__ x,
                       bf16_t* __restrict__ y, uint32_t rows, uint32_t cols, uint32_t experts, uint32_t x_group,
                       uint32_t x_stride) {
    moe_gemv_row<false>(w, ids, x, y, rows, cols, experts, x_group, x_stride);
}

extern "C" __global__ void __launch_bounds__(256)
    x0ne_moe_gemv_f32(const bf16_t* __restrict__ w, const uint32_t* __restrict__ ids, const bf16_t* __restrict__ x,
                      float* __restrict__ y, uint32_t rows, uint32_t cols, uint32_t experts, uint32_t x_group,
                      uint32_t x_stride) {
    moe_gemv_row<true>(w, ids, x, y, rows, cols, experts, x_group, x_stride);
}

// x0ne_moe_combine_bf16 (moe.cu:136-154): grid (ceil(hidden / 256), rows), block 256.
// out[r][i] = bf16(sum_s weights[r][s] y[r][s][i]), f32 fused multiply-adds in slot order, one
// rounding.
extern "C" __global__ void __launch_bounds__(256)
    x0ne_moe_combine_bf16(const float* __restrict__ y, const float* __restrict__ weights, bf16_t* __restrict__ out,
                          uint32_t hidden, uint32_t top_k) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x, r = blockIdx.y;
    if (i >= hidden) return;
    const float* wr = weights + (size_t)r * top_k;
    const float* yr = y + (size_t)r * top_k * hidden + i;
    float acc = 0.f;
    for (uint32_t s = 0; s < top_k; ++s) acc = fmaf(wr[s], yr[(size_t)s * hidden], acc);
    out[(size_t)r * hidden + i] = f2bf(acc);
}
