// Qwen3-MoE's sparse feed-forward on gfx950: routing of the router's f32 logits, the chosen
// experts' projections read through expert ids held in device memory (so the captured decode
// step replays whatever the routing chose), and their weighted combination. The semantics are
// the reference's (x0ne-core/kernels/cuda/moe.cu, oracle/src/lib.rs:254-329): experts ordered by
// logit then index, weights renormalised over the chosen in f64, an undefined routing (a router
// logit that is not finite) giving the id X0NE_MOE_NO_EXPERT and NaN weights, whose rows come
// out NaN so the greedy argmax refuses the token. The layout of the work is this build's:
//
//  - Routing: one wavefront per row. A lane holds the logits of experts lane, lane + 64, ... in
//    registers (16 at most); each of the top_k picks is a butterfly over the lanes' best untaken
//    candidates, the winner's lane clearing a bit of its taken mask; lane s keeps pick s, and the
//    renormalised weights are computed by the picking lanes with the denominator summed in pick
//    order.
//  - Expert projections: a wavefront owns R rows of one slot's expert; lane l reads 16-byte
//    chunks l, l + 64, ... of each row, two chunks of every row in flight, and the R partial sums
//    meet over the lanes in a transposing butterfly (one shuffle per row). gate/up runs with
//    SwiGLU behind (the gate and up rows of one activation in the same wavefront); down runs over
//    every slot of an output row in one wavefront and adds them with their routing weights in
//    slot order (the combination fused in).
#include "device.h"
#include "kernels.h"

namespace {

constexpr uint32_t MAX_EXPERTS = 1024;     // kernels/src/lib.rs:147
constexpr uint32_t NO_EXPERT = 0xFFFFFFFFu;  // kernels/src/lib.rs:151
constexpr uint32_t MAX_TOP_K = 32;
constexpr uint32_t PER_LANE = MAX_EXPERTS / 64;
constexpr float QNAN = __builtin_nanf("");

// The wavefront's own LDS writes are done (its lanes then read each other's).
__device__ __forceinline__ void wave_lds_wait() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Pick order: the larger logit, then the smaller expert id (-0.0 and 0.0 are equal).
__device__ __forceinline__ bool earlier(float v, uint32_t i, float bv, uint32_t bi) {
    return v > bv || (v == bv && i < bi);
}

// Sum over the 64 lanes of R values, transposing: at each of the first log2(R) steps a lane
// keeps half of its values (lane bit set: the upper half) and adds its partner's copy of them,
// then plain butterflies. Lane l ends with the whole sum of value `row_of_lane<R>(l)`.
template <int R, class Acc>
__device__ __forceinline__ Acc rows_sum(Acc (&v)[R], uint32_t lane) {
    int n = R;
#pragma unroll
    for (int k = 5; k >= 0; --k) {
        const bool up = (lane >> k) & 1u;
        if (n > 1) {
            const int h = n / 2;
#pragma unroll
            for (int j = 0; j < R / 2; ++j)
                if (j < h) {
                    const Acc give = up ? v[j] : v[j + h];
                    const Acc keep = up ? v[j + h] : v[j];
                    v[j] = keep + __shfl_xor(give, 1 << k, 64);
                }
            n = h;
        } else {
            v[0] += __shfl_xor(v[0], 1 << k, 64);
        }
    }
    return v[0];
}
template <int R>
__device__ __forceinline__ uint32_t row_of_lane(uint32_t lane) {
    uint32_t r = 0;
    int n = R;
#pragma unroll
    for (int k = 5; k >= 0; --k)
        if (n > 1) {
            n /= 2;
            if ((lane >> k) & 1u) r += n;
        }
    return r;
}

// Dot products of R rows (16-byte chunk pointers, each `chunks` long) with x over the lanes'
// chunks, two chunks of each row in flight; lane l ends with row row_of_lane<R>(l)'s sum. Acc =
// float: f32 FMA from 0 (each bf16 product exact in f32); double: each exact product added in
// f64 from -0.0, as the oracle's GEMV sums (oracle/src/lib.rs:123-133).
template <int R, class Acc = float>
__device__ __forceinline__ Acc rows_dot(const uint4* const (&w)[R], const uint4* __restrict__ x, uint32_t chunks,
                                        uint32_t lane) {
    constexpr Acc zero = sizeof(Acc) == 8 ? (Acc)-0.0 : (Acc)0.0;
    Acc acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = zero;
    auto madd = [](Acc a, uint4 p, uint4 q) {
        const Acc xs[8] = {(Acc)bf_lo(q.x), (Acc)bf_hi(q.x), (Acc)bf_lo(q.y), (Acc)bf_hi(q.y),
                           (Acc)bf_lo(q.z), (Acc)bf_hi(q.z), (Acc)bf_lo(q.w), (Acc)bf_hi(q.w)};
        return dot8<Acc>(p, xs, a);
    };
    uint32_t c = lane;
    for (; c + 64 < chunks; c += 128) {
        uint4 a[R], b[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            a[r] = w[r][c];
            b[r] = w[r][c + 64];
        }
        const uint4 xa = x[c], xb = x[c + 64];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = madd(madd(acc[r], a[r], xa), b[r], xb);
    }
    if (c < chunks) {
        const uint4 xa = x[c];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = madd(acc[r], w[r][c], xa);
    }
    return rows_sum<R, Acc>(acc, lane);
}

}  // namespace

// x0ne_moe_route_f32: grid (rows), block 64. ids[row][s] and weights[row][s] for the top_k picks
// of the row's `experts` router logits; experts 1..=1024, top_k 1..=min(32, experts), else
// nothing is written.
extern "C" __global__ void __launch_bounds__(64)
    x0ne_moe_route_f32(const float* __restrict__ logits, uint32_t experts, uint32_t top_k, uint32_t* __restrict__ ids,
                       float* __restrict__ weights) {
    if (experts == 0 || experts > MAX_EXPERTS || top_k == 0 || top_k > MAX_TOP_K || top_k > experts ||
        blockDim.x != 64)
        return;  // grid-uniform
    const uint32_t lane = threadIdx.x;
    const float* row = logits + (size_t)blockIdx.x * experts;
    float v[PER_LANE];
    bool finite = true;
#pragma unroll
    for (uint32_t j = 0; j < PER_LANE; ++j) {
        const uint32_t i = lane + 64 * j;
        v[j] = i < experts ? row[i] : -INFINITY;
        finite &= i >= experts || isfinite(v[j]);
    }
    uint32_t* out_ids = ids + (size_t)blockIdx.x * top_k;
    float* out_w = weights + (size_t)blockIdx.x * top_k;
    if (!__all(finite)) {  // an undefined routing: no expert, NaN weights
        if (lane < top_k) {
            out_ids[lane] = NO_EXPERT;
            out_w[lane] = QNAN;
        }
        return;
    }
    uint32_t taken = 0;  // bit j: expert lane + 64 j already picked
    uint32_t mine = NO_EXPERT;
    float mine_v = 0.f, top_v = 0.f;
    for (uint32_t s = 0; s < top_k; ++s) {
        float bv = -INFINITY;
        uint32_t bi = NO_EXPERT;
#pragma unroll
        for (uint32_t j = 0; j < PER_LANE; ++j) {
            const uint32_t i = lane + 64 * j;
            if (i < experts && !((taken >> j) & 1u) && earlier(v[j], i, bv, bi)) {
                bv = v[j];
                bi = i;
            }
        }
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const float ov = __shfl_xor(bv, o, 64);
            const uint32_t oi = __shfl_xor(bi, o, 64);
            if (earlier(ov, oi, bv, bi)) {
                bv = ov;
                bi = oi;
            }
        }
        if (bi % 64 == lane) taken |= 1u << (bi / 64);
        if (s == 0) top_v = bv;
        if (lane == s) {
            mine = bi;
            mine_v = bv;
        }
    }
    // Renormalised weights: exp(l_s - l_top) over their sum, in f64, the sum in pick order.
    const double e = lane < top_k ? exp((double)mine_v - (double)top_v) : 0.0;
    double sum = 0.0;
    for (uint32_t s = 0; s < top_k; ++s) sum += __shfl(e, (int)s, 64);
    if (lane < top_k) {
        out_ids[lane] = mine;
        out_w[lane] = (float)(e / sum);
    }
}

namespace {

// Rows r0 .. r0 + R - 1 of expert `e` of W [experts][rows][cols] (a row past `rows` repeats the
// last one, its sum unused).
template <int R>
__device__ __forceinline__ void expert_rows(const bf16_t* __restrict__ w, uint32_t e, uint32_t rows, uint32_t cols,
                                            uint32_t r0, const uint4* (&out)[R]) {
#pragma unroll
    for (int r = 0; r < R; ++r)
        out[r] = reinterpret_cast<const uint4*>(w + ((size_t)e * rows + min(r0 + r, rows - 1)) * cols);
}

template <bool F32>
__device__ __forceinline__ void expert_gemv(const bf16_t* __restrict__ w, const uint32_t* __restrict__ ids,
                                            const bf16_t* __restrict__ x, void* __restrict__ y, uint32_t rows,
                                            uint32_t cols, uint32_t experts, uint32_t x_group, uint32_t x_stride) {
    constexpr int R = 2;
    const uint32_t lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t r0 = (blockIdx.x * 4 + wave) * R, slot = blockIdx.y;
    if (r0 >= rows || x_group == 0 || cols % 8 != 0) return;  // wavefront-uniform
    const uint32_t e = __builtin_amdgcn_readfirstlane(ids[slot]);
    const uint32_t r = r0 + row_of_lane<R>(lane);
    const bool writer = (lane & 31) == 0 && r < rows;  // one lane per row holds its sum
    const size_t o = (size_t)slot * rows + r;
    float sum = QNAN;
    if (e < experts) {
        const uint4* wr[R];
        expert_rows<R>(w, e, rows, cols, r0, wr);
        sum = rows_dot<R>(wr, reinterpret_cast<const uint4*>(x + (size_t)(slot / x_group) * x_stride), cols / 8, lane);
    }
    if (writer) {
        if (F32)
            static_cast<float*>(y)[o] = sum;
        else
            static_cast<bf16_t*>(y)[o] = f2bf(sum);
    }
}

// out = bf16(sum_s wts[s] y[s * stride]) in f32 fused multiply-adds, slot order, one rounding.
__device__ __forceinline__ bf16_t weigh_slots(const float* __restrict__ wts, const float* y, size_t stride,
                                              uint32_t top_k) {
    float acc = 0.f;
    for (uint32_t s = 0; s < top_k; ++s) acc = fmaf(wts[s], y[s * stride], acc);
    return f2bf(acc);
}

}  // namespace

// x0ne_moe_gemv_bf16 / _f32: grid (ceil(rows / 8), slots), block 256. y[s][0..rows) = W[ids[s]]
// x[s / x_group] (x rows x_stride apart), W [experts][rows][cols] bf16, bf16 or f32 out; cols a
// multiple of 8, W and x 16-byte aligned. An id >= experts gives a NaN row without reading W.
extern "C" __global__ void __launch_bounds__(256)
    x0ne_moe_gemv_bf16(const bf16_t* __restrict__ w, const uint32_t* __restrict__ ids, const bf16_t* __restrict__ x,
                       bf16_t* __restrict__ y, uint32_t rows, uint32_t cols, uint32_t experts, uint32_t x_group,
                       uint32_t x_stride) {
    expert_gemv<false>(w, ids, x, y, rows, cols, experts, x_group, x_stride);
}

extern "C" __global__ void __launch_bounds__(256)
    x0ne_moe_gemv_f32(const bf16_t* __restrict__ w, const uint32_t* __restrict__ ids, const bf16_t* __restrict__ x,
                      float* __restrict__ y, uint32_t rows, uint32_t cols, uint32_t experts, uint32_t x_group,
                      uint32_t x_stride) {
    expert_gemv<true>(w, ids, x, y, rows, cols, experts, x_group, x_stride);
}

// x0ne_moe_combine_bf16: grid (ceil(hidden / 256), rows), block 256. out[r][i] = the routing
// weights of row r over its slots' f32 rows y[r][s][i].
extern "C" __global__ void __launch_bounds__(256)
    x0ne_moe_combine_bf16(const float* __restrict__ y, const float* __restrict__ weights, bf16_t* __restrict__ out,
                          uint32_t hidden, uint32_t top_k) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x, r = blockIdx.y;
    if (i >= hidden) return;
    out[(size_t)r * hidden + i] =
        weigh_slots(weights + (size_t)r * top_k, y + (size_t)r * top_k * hidden + i, hidden, top_k);
}

namespace {

// [gate; up] of expert ids[slot] with SwiGLU behind: a wavefront takes 2 activations (4 rows).
// Each projection's sum is rounded to f32 (the oracle's GEMV output), then to bf16.
template <class Acc>
__device__ __forceinline__ void gate_up_swiglu(const bf16_t* __restrict__ w, const uint32_t* __restrict__ ids,
                                               const bf16_t* __restrict__ x, bf16_t* __restrict__ act, uint32_t inter,
                                               uint32_t cols, uint32_t experts) {
    constexpr int R = 4;  // gate i0, gate i0 + 1, up i0, up i0 + 1
    const uint32_t lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t i0 = (blockIdx.x * 4 + wave) * 2, slot = blockIdx.y;
    if (i0 >= inter || cols % 8 != 0) return;  // wavefront-uniform
    const uint32_t e = __builtin_amdgcn_readfirstlane(ids[slot]);
    const uint32_t k = row_of_lane<R>(lane);  // 0, 1: gate of i0 + k; 2, 3: up of i0 + k - 2
    float sum = QNAN;
    if (e < experts) {
        const uint4* wr[R];
        const size_t base = (size_t)e * 2 * inter;
        for (int j = 0; j < 2; ++j) {
            const uint32_t i = min(i0 + j, inter - 1);
            wr[j] = reinterpret_cast<const uint4*>(w + (base + i) * cols);
            wr[2 + j] = reinterpret_cast<const uint4*>(w + (base + inter + i) * cols);
        }
        sum = (float)rows_dot<R, Acc>(wr, reinterpret_cast<const uint4*>(x), cols / 8, lane);
    }
    // Lanes holding up sums (k = 2, 3) sit 32 above the gate sums of the same activation.
    const float up = __shfl_xor(sum, 32, 64);
    const uint32_t i = i0 + k;
    if ((lane & 15) == 0 && k < 2 && i < inter) {
        const double g = (double)bf_round(sum), u = (double)bf_round(up);
        act[(size_t)slot * inter + i] = f2bf((float)(g / (1.0 + exp(-g)) * u));
    }
}

// Down rows of every slot's expert with the weighted combination behind: a wavefront takes 2
// output rows over every slot (top_k <= 32), each slot's row sum rounded to f32 (the oracle's
// f32 expert GEMV) and staged in LDS, then weighed in slot order: Acc = float, f32 FMA from 0;
// double, each product of two f32 values (exact in f64) added in f64 from -0.0 as the oracle's
// combination (oracle/src/lib.rs:314-329), one rounding to f32 and one to bf16.
template <class Acc>
__device__ __forceinline__ void down_combine(const bf16_t* __restrict__ w, const uint32_t* __restrict__ ids,
                                             const float* __restrict__ wts, const bf16_t* __restrict__ act,
                                             bf16_t* __restrict__ out, uint32_t hidden, uint32_t inter,
                                             uint32_t experts, uint32_t top_k) {
    constexpr int R = 2;
    __shared__ float ys[4][MAX_TOP_K][R];
    const uint32_t lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t r0 = (blockIdx.x * 4 + wave) * R;
    if (r0 >= hidden || top_k == 0 || top_k > MAX_TOP_K || inter % 8 != 0) return;  // wavefront-uniform
    const uint32_t k = row_of_lane<R>(lane);
    for (uint32_t s = 0; s < top_k; ++s) {
        const uint32_t e = __builtin_amdgcn_readfirstlane(ids[s]);
        float sum = QNAN;
        if (e < experts) {
            const uint4* wr[R];
            expert_rows<R>(w, e, hidden, inter, r0, wr);
            sum = (float)rows_dot<R, Acc>(wr, reinterpret_cast<const uint4*>(act + (size_t)s * inter), inter / 8, lane);
        }
        if ((lane & 31) == 0) ys[wave][s][k] = sum;
    }
    wave_lds_wait();
    if (lane < (uint32_t)R && r0 + lane < hidden) {
        if (sizeof(Acc) == 8) {
            double acc = -0.0;
            for (uint32_t s = 0; s < top_k; ++s) acc += (double)wts[s] * (double)ys[wave][s][lane];
            out[r0 + lane] = f2bf((float)acc);
        } else {
            out[r0 + lane] = weigh_slots(wts, &ys[wave][0][lane], R, top_k);
        }
    }
}

}  // namespace

// x0ne_moe_gate_up_swiglu_bf16 / _exact_bf16: grid (ceil(inter / 2 / 4) = ceil(inter / 8),
// slots), block 256. W [experts][2 inter][cols] holds each expert's gate rows then up rows;
// act[s][i] = bf16(silu(bf16 g) bf16 u) for g, u = rows i and inter + i of expert ids[s] against
// x (shared by the slots), summed in f32 (_bf16) or f64 (_exact_bf16). An id >= experts gives NaN.
extern "C" __global__ void __launch_bounds__(256)
    x0ne_moe_gate_up_swiglu_bf16(const bf16_t* __restrict__ w, const uint32_t* __restrict__ ids,
                                 const bf16_t* __restrict__ x, bf16_t* __restrict__ act, uint32_t inter, uint32_t cols,
                                 uint32_t experts) {
    gate_up_swiglu<float>(w, ids, x, act, inter, cols, experts);
}

extern "C" __global__ void __launch_bounds__(256)
    x0ne_moe_gate_up_swiglu_exact_bf16(const bf16_t* __restrict__ w, const uint32_t* __restrict__ ids,
                                       const bf16_t* __restrict__ x, bf16_t* __restrict__ act, uint32_t inter,
                                       uint32_t cols, uint32_t experts) {
    gate_up_swiglu<double>(w, ids, x, act, inter, cols, experts);
}

// x0ne_moe_down_combine_bf16 / _exact_bf16: grid (ceil(hidden / 8)), block 256. out[i] =
// bf16(sum_s wts[s] y_s[i]), y_s[i] = row i of expert ids[s]'s down matrix W
// [experts][hidden][inter] against act[s] (f32), the slots added in order: x0ne_moe_gemv_f32
// then x0ne_moe_combine_bf16 in one launch (_bf16), or the same with f64 sums and an f64
// combination (_exact_bf16).
extern "C" __global__ void __launch_bounds__(256)
    x0ne_moe_down_combine_bf16(const bf16_t* __restrict__ w, const uint32_t* __restrict__ ids,
                               const float* __restrict__ wts, const bf16_t* __restrict__ act, bf16_t* __restrict__ out,
                               uint32_t hidden, uint32_t inter, uint32_t experts, uint32_t top_k) {
    down_combine<float>(w, ids, wts, act, out, hidden, inter, experts, top_k);
}

extern "C" __global__ void __launch_bounds__(256)
    x0ne_moe_down_combine_exact_bf16(const bf16_t* __restrict__ w, const uint32_t* __restrict__ ids,
                                     const float* __restrict__ wts, const bf16_t* __restrict__ act,
                                     bf16_t* __restrict__ out, uint32_t hidden, uint32_t inter, uint32_t experts,
                                     uint32_t top_k) {
    down_combine<double>(w, ids, wts, act, out, hidden, inter, experts, top_k);
}
