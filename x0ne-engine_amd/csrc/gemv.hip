// Bandwidth-bound bf16 GEMV for gfx950: y = W x, W [rows][cols] row-major bf16, x bf16,
// f32 accumulation. It replaces the reference's cuBLAS call at n = 1 (x0ne-core/runtime/src/
// gpu.rs:1098-1149: Y[n][rows] = X[n][cols] W^T, bf16 in, f32 compute, bf16 or f32 out).
//
// Layout of the work (this build's): a block of 256 threads spans one whole row; thread t holds
// the 16-byte chunks t, t + 256, ... of it, so the 256 threads of a block read 4 KiB contiguous
// per load instruction, and thread t's slice of x stays in its registers for every row the
// block visits. A block takes RPB rows at a time (RPB x chunks loads in flight per thread) and
// walks the row groups g, g + gridDim.x, ... (a persistent grid of a few blocks per CU), so the
// prologue below runs once per block, not once per row.
//
// Fused prologue (the engine's; x0ne-core/kernels/cuda/rmsnorm.cu:5-21 and embedding.cu:5-17
// restated): x = bf16(rmsnorm(residual_in + delta) * w_norm), with the residual add in f32 (one
// IEEE addition per value) and the norm in f64 like the oracle (oracle/src/lib.rs:50-67); block 0
// writes residual_in + delta to residual_out (a second buffer, so no block reads a residual
// another has already updated). The first layer's variant adds the embedding row of tokens[0]
// (a token past the table gives a zero row) to a zero residual.
//
// Fused epilogues: bf16 out; f32 out; SwiGLU over the packed [gate; up] rows (gate row i and up
// row inter + i are summed by the same block, act[i] = bf16(silu(bf16 g) bf16 u) in f64,
// oracle/src/lib.rs:205-214); and f32 logits with the greedy argmax (first largest, any NaN
// gives 0xFFFFFFFF; kernels/cuda/argmax.cu:11-58) reduced by the last block to finish, which
// writes the token to device memory and can advance the position (advance.cu:5-7).
#include "device.h"

namespace {

constexpr int BLOCK = 256;
constexpr uint32_t NO_TOKEN = 0xFFFFFFFFu;

enum Pro : int { PRO_X = 0, PRO_NORM = 1, PRO_EMBED_NORM = 2 };
enum Epi : int { EPI_BF16 = 0, EPI_F32 = 1, EPI_SWIGLU = 2, EPI_ARGMAX = 3 };

struct GemvArgs {
    const bf16_t* w;
    const bf16_t* x;          // PRO_X
    const float* res_in;      // PRO_NORM
    float* res_out;           // PRO_NORM, PRO_EMBED_NORM (block 0 writes it; may be null)
    const bf16_t* delta;      // PRO_NORM
    const bf16_t* norm_w;     // PRO_NORM, PRO_EMBED_NORM
    const bf16_t* embed;      // PRO_EMBED_NORM: [vocab][cols]
    const uint32_t* tokens;   // PRO_EMBED_NORM: tokens[0]
    void* y;                  // bf16 [rows] / f32 [rows] / bf16 act [rows/2]
    float* partial;           // EPI_ARGMAX: 3 words per block
    uint32_t* counter;        // EPI_ARGMAX: one word, left at 0
    uint32_t* token_out;      // EPI_ARGMAX
    uint32_t* pos;            // EPI_ARGMAX: advanced when advance != 0
    uint32_t rows;            // output rows (SwiGLU: 2 x inter)
    uint32_t cols;
    uint32_t vocab;           // PRO_EMBED_NORM
    uint32_t advance;         // EPI_ARGMAX
    float eps;
};

__device__ __forceinline__ bool better(float v, uint32_t i, float bv, uint32_t bi) {
    return v > bv || (v == bv && i < bi);
}

// x of this thread: chunk j covers columns 8 (t + 256 j) .. + 7 (as f32 values of bf16).
template <int KMAX, int PRO>
__device__ __forceinline__ void prologue(const GemvArgs& a, float xs[KMAX][8], double* sh) {
    const uint32_t t = threadIdx.x, nch = (a.cols / 8 + BLOCK - 1) / BLOCK, C = a.cols / 8;
    if (PRO == PRO_X) {
#pragma unroll
        for (int j = 0; j < KMAX; ++j) {
            const uint32_t c = t + BLOCK * j;
            uint4 u = make_uint4(0, 0, 0, 0);
            if (j < (int)nch && c < C) u = *reinterpret_cast<const uint4*>(a.x + 8 * (size_t)c);
            xs[j][0] = bf_lo(u.x); xs[j][1] = bf_hi(u.x); xs[j][2] = bf_lo(u.y); xs[j][3] = bf_hi(u.y);
            xs[j][4] = bf_lo(u.z); xs[j][5] = bf_hi(u.z); xs[j][6] = bf_lo(u.w); xs[j][7] = bf_hi(u.w);
        }
        return;
    }
    // r = residual_in + delta (f32), or the embedding row over a zero residual.
    const bf16_t* drow = a.delta;
    bool zero_row = false;
    if (PRO == PRO_EMBED_NORM) {
        const uint32_t tok = a.tokens[0];
        zero_row = tok >= a.vocab;
        drow = a.embed + (size_t)(zero_row ? 0 : tok) * a.cols;
    }
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < KMAX; ++j) {
        const uint32_t c = t + BLOCK * j;
        float r[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        if (j < (int)nch && c < C) {
            uint4 u = *reinterpret_cast<const uint4*>(drow + 8 * (size_t)c);
            if (zero_row) u = make_uint4(0, 0, 0, 0);
            const float d[8] = {bf_lo(u.x), bf_hi(u.x), bf_lo(u.y), bf_hi(u.y),
                                bf_lo(u.z), bf_hi(u.z), bf_lo(u.w), bf_hi(u.w)};
            if (PRO == PRO_NORM) {
                const float4 r0 = *reinterpret_cast<const float4*>(a.res_in + 8 * (size_t)c);
                const float4 r1 = *reinterpret_cast<const float4*>(a.res_in + 8 * (size_t)c + 4);
                r[0] = r0.x + d[0]; r[1] = r0.y + d[1]; r[2] = r0.z + d[2]; r[3] = r0.w + d[3];
                r[4] = r1.x + d[4]; r[5] = r1.y + d[5]; r[6] = r1.z + d[6]; r[7] = r1.w + d[7];
            } else {
#pragma unroll
                for (int k = 0; k < 8; ++k) r[k] = 0.f + d[k];
            }
            if (blockIdx.x == 0 && a.res_out != nullptr) {
                float4* o = reinterpret_cast<float4*>(a.res_out + 8 * (size_t)c);
                o[0] = make_float4(r[0], r[1], r[2], r[3]);
                o[1] = make_float4(r[4], r[5], r[6], r[7]);
            }
#pragma unroll
            for (int k = 0; k < 8; ++k) ss += (double)r[k] * (double)r[k];
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) xs[j][k] = r[k];
    }
    const double total = block_sum_d(ss, sh);
    const double scale = 1.0 / sqrt(total / (double)a.cols + (double)a.eps);
#pragma unroll
    for (int j = 0; j < KMAX; ++j) {
        const uint32_t c = t + BLOCK * j;
        if (j < (int)nch && c < C) {
            const uint4 u = *reinterpret_cast<const uint4*>(a.norm_w + 8 * (size_t)c);
            const float w[8] = {bf_lo(u.x), bf_hi(u.x), bf_lo(u.y), bf_hi(u.y),
                                bf_lo(u.z), bf_hi(u.z), bf_lo(u.w), bf_hi(u.w)};
#pragma unroll
            for (int k = 0; k < 8; ++k) xs[j][k] = bf_round((float)((double)xs[j][k] * scale * (double)w[k]));
        } else {
#pragma unroll
            for (int k = 0; k < 8; ++k) xs[j][k] = 0.f;
        }
    }
}

__device__ __forceinline__ float dot8(const uint4 w, const float* x, float acc) {
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

// RPB rows per step. For EPI_SWIGLU a step is RPB / 2 pairs: gate rows i.. and up rows inter + i..
template <int KMAX, int RPB, int PRO, int EPI>
__device__ __forceinline__ void gemv_body(const GemvArgs& a) {
    __shared__ double sh[16];
    __shared__ float part[2][BLOCK / 64][RPB];
    __shared__ float best_v[BLOCK / 64];
    __shared__ uint32_t best_i[BLOCK / 64];
    __shared__ uint32_t last;
    const uint32_t t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const uint32_t C = a.cols / 8, nch = (C + BLOCK - 1) / BLOCK;
    float xs[KMAX][8];
    prologue<KMAX, PRO>(a, xs, sh);

    constexpr int PAIRS = RPB / 2;
    const uint32_t inter = a.rows / 2;
    const uint32_t groups = EPI == EPI_SWIGLU ? (inter + PAIRS - 1) / PAIRS : (a.rows + RPB - 1) / RPB;
    float bv = -INFINITY;
    uint32_t bi = NO_TOKEN;
    bool nan = false;
    int parity = 0;
    for (uint32_t g = blockIdx.x; g < groups; g += gridDim.x) {
        uint32_t row[RPB];
#pragma unroll
        for (int rr = 0; rr < RPB; ++rr) {
            if (EPI == EPI_SWIGLU)
                row[rr] = rr < PAIRS ? g * PAIRS + rr : inter + g * PAIRS + (rr - PAIRS);
            else
                row[rr] = g * RPB + rr;
        }
        bool in[RPB];
#pragma unroll
        for (int rr = 0; rr < RPB; ++rr)
            in[rr] = EPI == EPI_SWIGLU ? (rr < PAIRS ? row[rr] < inter : row[rr] - inter < inter) : row[rr] < a.rows;
        uint4 wv[RPB][KMAX];
#pragma unroll
        for (int rr = 0; rr < RPB; ++rr) {
            const bf16_t* wr = a.w + (size_t)row[rr] * a.cols;
#pragma unroll
            for (int j = 0; j < KMAX; ++j) {
                const uint32_t c = t + BLOCK * j;
                wv[rr][j] = (in[rr] && j < (int)nch && c < C) ? *reinterpret_cast<const uint4*>(wr + 8 * (size_t)c)
                                                                : make_uint4(0, 0, 0, 0);
            }
        }
        float acc[RPB];
#pragma unroll
        for (int rr = 0; rr < RPB; ++rr) {
            float s = 0.f;
#pragma unroll
            for (int j = 0; j < KMAX; ++j) s = dot8(wv[rr][j], xs[j], s);
            acc[rr] = wave_sum(s);
        }
        if (lane == 0) {
#pragma unroll
            for (int rr = 0; rr < RPB; ++rr) part[parity][wave][rr] = acc[rr];
        }
        __syncthreads();
        if (EPI == EPI_SWIGLU) {
            const uint32_t i = g * PAIRS + t;
            if (t < (uint32_t)PAIRS && i < inter) {
                float gs = 0.f, us = 0.f;
#pragma unroll
                for (int w = 0; w < BLOCK / 64; ++w) {
                    gs += part[parity][w][t];
                    us += part[parity][w][PAIRS + t];
                }
                const double gd = (double)bf_round(gs), ud = (double)bf_round(us);
                reinterpret_cast<bf16_t*>(a.y)[i] = f2bf((float)(gd / (1.0 + exp(-gd)) * ud));
            }
        } else {
            const uint32_t r = g * RPB + t;
            if (t < (uint32_t)RPB && r < a.rows) {
                float s = 0.f;
#pragma unroll
                for (int w = 0; w < BLOCK / 64; ++w) s += part[parity][w][t];
                if (EPI == EPI_BF16) reinterpret_cast<bf16_t*>(a.y)[r] = f2bf(s);
                if (EPI == EPI_F32 || EPI == EPI_ARGMAX) reinterpret_cast<float*>(a.y)[r] = s;
                if (EPI == EPI_ARGMAX) {
                    nan |= s != s;
                    if (better(s, r, bv, bi)) {
                        bv = s;
                        bi = r;
                    }
                }
            }
        }
        parity ^= 1;
    }
    if (EPI != EPI_ARGMAX) return;

    // This block's candidate: lanes 0..RPB-1 of wave 0 hold one each.
    if (wave == 0) {
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const float ov = __shfl_xor(bv, o, 64);
            const uint32_t oi = __shfl_xor(bi, o, 64);
            if (better(ov, oi, bv, bi)) {
                bv = ov;
                bi = oi;
            }
        }
        const bool any_nan = __any(nan);
        if (lane == 0) {
            a.partial[3 * blockIdx.x] = bv;
            a.partial[3 * blockIdx.x + 1] = __uint_as_float(bi);
            a.partial[3 * blockIdx.x + 2] = any_nan ? 1.f : 0.f;
        }
    }
    __threadfence();
    __syncthreads();
    if (t == 0) last = atomicAdd(a.counter, 1u) == gridDim.x - 1;
    __syncthreads();
    if (!last) return;
    __threadfence();
    // The last block: candidates of blocks 0..gridDim.x-1, thread t takes t, t + 256, ...
    float v = -INFINITY;
    uint32_t i = NO_TOKEN;
    bool n = false;
    for (uint32_t k = t; k < gridDim.x; k += BLOCK) {
        const float kv = __hip_atomic_load(a.partial + 3 * k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint32_t ki = __float_as_uint(
            __hip_atomic_load(a.partial + 3 * k + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        n |= __hip_atomic_load(a.partial + 3 * k + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0.f;
        if (better(kv, ki, v, i)) {
            v = kv;
            i = ki;
        }
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const float ov = __shfl_xor(v, o, 64);
        const uint32_t oi = __shfl_xor(i, o, 64);
        if (better(ov, oi, v, i)) {
            v = ov;
            i = oi;
        }
    }
    const bool wn = __any(n);
    if (lane == 0) {
        best_v[wave] = wn ? NAN : v;
        best_i[wave] = wn ? NO_TOKEN : i;
    }
    __syncthreads();
    if (t == 0) {
        bool any = false;
        float fv = -INFINITY;
        uint32_t fi = NO_TOKEN;
        for (int w = 0; w < BLOCK / 64; ++w) {
            if (best_i[w] == NO_TOKEN && best_v[w] != best_v[w]) any = true;
            if (better(best_v[w], best_i[w], fv, fi)) {
                fv = best_v[w];
                fi = best_i[w];
            }
        }
        a.token_out[0] = any ? NO_TOKEN : fi;
        if (a.advance) a.pos[0] += 1u;
        a.counter[0] = 0;  // ready for the next launch
    }
}

}  // namespace

// ---- host-side dispatch: one kernel per (KMAX, RPB, prologue, epilogue) ----

template <int KMAX, int RPB, int PRO, int EPI>
__global__ void __launch_bounds__(256) gemv_kernel(GemvArgs a) {
    gemv_body<KMAX, RPB, PRO, EPI>(a);
}

// Plain GEMV for the kernel table and tests: y[rows] = W x, bf16 or f32 out, any cols that is
// a multiple of 8 up to 16384 (16-byte chunks); grid (blocks), block 256.
#define X0NE_GEMV_PLAIN(NAME, EPI)                                                                                \
    extern "C" __global__ void __launch_bounds__(256) NAME(const bf16_t* __restrict__ w, const bf16_t* __restrict__ x, \
                                                          void* __restrict__ y, uint32_t rows, uint32_t cols) {     \
        GemvArgs a = {};                                                                                          \
        a.w = w;                                                                                                  \
        a.x = x;                                                                                                  \
        a.y = y;                                                                                                  \
        a.rows = rows;                                                                                            \
        a.cols = cols;                                                                                            \
        gemv_body<8, 2, PRO_X, EPI>(a);                                                                          \
    }
X0NE_GEMV_PLAIN(x0ne_gemv_bf16, EPI_BF16)
X0NE_GEMV_PLAIN(x0ne_gemv_f32, EPI_F32)

// Any cols (the reference's cuBLAS call takes any shape): one block per row, scalar loads,
// thread t sums columns t, t + 256, ... in order, then the block sums the threads in order.
extern "C" __global__ void __launch_bounds__(256)
    x0ne_gemv_any(const bf16_t* __restrict__ w, const bf16_t* __restrict__ x, void* __restrict__ y, uint32_t rows,
                  uint32_t cols, uint32_t f32_out) {
    __shared__ float sh[BLOCK / 64];
    const uint32_t row = blockIdx.x, t = threadIdx.x;
    if (row >= rows) return;
    float s = 0.f;
    for (uint32_t c = t; c < cols; c += BLOCK) s = fmaf(bf2f(w[(size_t)row * cols + c]), bf2f(x[c]), s);
    s = wave_sum(s);
    if ((t & 63) == 0) sh[t >> 6] = s;
    __syncthreads();
    if (t == 0) {
        float tot = 0.f;
        for (int k = 0; k < BLOCK / 64; ++k) tot += sh[k];
        if (f32_out)
            reinterpret_cast<float*>(y)[row] = tot;
        else
            reinterpret_cast<bf16_t*>(y)[row] = f2bf(tot);
    }
}

// ---- typed launchers (called by the runtime) ----

#include "launch.h"

namespace {

template <int RPB, int PRO, int EPI>
hipError_t launch_k(const GemvArgs& a, uint32_t grid, hipStream_t s) {
    const uint32_t nch = (a.cols / 8 + BLOCK - 1) / BLOCK;
    if (nch <= 1) return (gemv_kernel<1, RPB * 4 <= 8 ? RPB * 4 : 8, PRO, EPI><<<grid, BLOCK, 0, s>>>(a), hipGetLastError());
    if (nch <= 2) return (gemv_kernel<2, RPB * 2 <= 8 ? RPB * 2 : 8, PRO, EPI><<<grid, BLOCK, 0, s>>>(a), hipGetLastError());
    if (nch <= 4) return (gemv_kernel<4, RPB, PRO, EPI><<<grid, BLOCK, 0, s>>>(a), hipGetLastError());
    if (nch <= 8) return (gemv_kernel<8, RPB / 2 >= 2 ? RPB / 2 : 2, PRO, EPI><<<grid, BLOCK, 0, s>>>(a), hipGetLastError());
    if (nch <= 16) return (gemv_kernel<16, 2, PRO, EPI><<<grid, BLOCK, 0, s>>>(a), hipGetLastError());
    return hipErrorInvalidValue;
}

template <int PRO, int EPI>
hipError_t launch_pe(const GemvArgs& a, uint32_t grid, hipStream_t s) {
    return launch_k<2, PRO, EPI>(a, grid, s);
}

}  // namespace

// Rows per step the launch above picks for cols (EPI_SWIGLU counts rows of both halves).
uint32_t x0ne_gemv_rows_per_step(uint32_t cols) {
    const uint32_t nch = (cols / 8 + BLOCK - 1) / BLOCK;
    if (nch <= 1) return 8;
    if (nch <= 2) return 4;
    if (nch <= 4) return 2;
    return 2;
}

hipError_t x0ne_launch_gemv(const X0neGemv& g, hipStream_t s) {
    if (g.cols == 0 || g.cols % 8 != 0 || (g.cols / 8 + BLOCK - 1) / BLOCK > 16 || g.rows == 0 || g.grid == 0)
        return hipErrorInvalidValue;
    GemvArgs a = {};
    a.w = g.w;
    a.x = g.x;
    a.res_in = g.res_in;
    a.res_out = g.res_out;
    a.delta = g.delta;
    a.norm_w = g.norm_w;
    a.embed = g.embed;
    a.tokens = g.tokens;
    a.y = g.y;
    a.partial = g.partial;
    a.counter = g.counter;
    a.token_out = g.token_out;
    a.pos = g.pos;
    a.rows = g.rows;
    a.cols = g.cols;
    a.vocab = g.vocab;
    a.advance = g.advance;
    a.eps = g.eps;
    const int pro = g.prologue, epi = g.epilogue;
#define X0NE_CASE(P, E) \
    if (pro == P && epi == E) return launch_pe<P, E>(a, g.grid, s);
    X0NE_CASE(PRO_X, EPI_BF16)
    X0NE_CASE(PRO_X, EPI_F32)
    X0NE_CASE(PRO_NORM, EPI_BF16)
    X0NE_CASE(PRO_NORM, EPI_SWIGLU)
    X0NE_CASE(PRO_NORM, EPI_ARGMAX)
    X0NE_CASE(PRO_NORM, EPI_F32)
    X0NE_CASE(PRO_EMBED_NORM, EPI_BF16)
#undef X0NE_CASE
    return hipErrorInvalidValue;
}
