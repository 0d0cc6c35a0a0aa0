// Bandwidth-bound bf16 GEMV for gfx950: y = W x, W [rows][cols] row-major bf16, x bf16. It
// replaces the reference's cuBLAS call at n = 1 (x0ne-core/runtime/src/gpu.rs:1098-1149:
// Y[n][rows] = X[n][cols] W^T, bf16 in, f32 compute, bf16 or f32 out).
//
// Layout of the work (this build's): a block of 256 threads (4 wavefronts) first stages x in LDS
// (bf16, after the fused prologue below), then each wavefront works alone, with no barrier: it
// takes R whole rows at a time (row groups w, w + W, ... of a persistent grid of W wavefronts),
// lane l reading the 16-byte chunks l, l + 64, ... of each row, so one load instruction of a
// wavefront covers 1 KiB contiguous of one row and R x 8 such loads are in flight per wavefront.
// The R partial sums of a lane are reduced over the 64 lanes by a transposing butterfly (the R
// values halve at the first log2(R) steps), so a row costs about one shuffle.
//
// Accumulation: `Acc` = float (f32 FMA, products of two bf16 exact in f32) or double (each exact
// product added in f64, as the oracle sums, oracle/src/lib.rs:123-133).
//
// Fused prologue (the engine's; x0ne-core/kernels/cuda/rmsnorm.cu:5-21 and embedding.cu:5-17
// restated): x = bf16(rmsnorm(residual_in + delta) * w_norm), with the residual add in f32 (one
// IEEE addition per value) and the norm in f64 like the oracle (oracle/src/lib.rs:50-67); block 0
// writes residual_in + delta to residual_out (a second buffer, so no block reads a residual
// another has already updated). The first layer's variant adds the embedding row of tokens[0]
// (a token past the table gives a zero row) to a zero residual.
//
// Fused epilogues: bf16 out; f32 out; SwiGLU over the packed [gate; up] rows (gate row i and up
// row inter + i are summed by the same wavefront, act[i] = bf16(silu(bf16 g) bf16 u) in f64,
// oracle/src/lib.rs:205-214); and f32 logits with the greedy argmax (first largest, any NaN
// gives 0xFFFFFFFF; kernels/cuda/argmax.cu:11-58) reduced by the last block to finish, which
// writes the token to device memory and can advance the position (advance.cu:5-7).
#include "device.h"

namespace {

constexpr int BLOCK = 256;
constexpr int WAVES = BLOCK / 64;
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

__device__ __forceinline__ uint32_t pack2(bf16_t lo, bf16_t hi) { return (uint32_t)lo | ((uint32_t)hi << 16); }

// Stages x (bf16) in LDS: the given x, or bf16(rmsnorm(residual + delta) * w_norm). Block-wide;
// ends with a barrier. The residual sums of a thread's first KEEP chunks stay in registers between
// the two passes (hidden sizes up to 256 x 8 x KEEP need no second read); later chunks are read
// again and recomputed (the same f32 additions, the same bits).
template <int PRO>
__device__ __forceinline__ void stage_x(const GemvArgs& a, uint4* xl, double* sh) {
    constexpr uint32_t KEEP = 2;
    const uint32_t t = threadIdx.x, C = a.cols / 8;
    if (PRO == PRO_X) {
        for (uint32_t c = t; c < C; c += BLOCK) xl[c] = *reinterpret_cast<const uint4*>(a.x + 8 * (size_t)c);
        __syncthreads();
        return;
    }
    const bf16_t* drow = a.delta;
    bool zero_row = false;
    if (PRO == PRO_EMBED_NORM) {
        const uint32_t tok = a.tokens[0];
        zero_row = tok >= a.vocab;
        drow = a.embed + (size_t)(zero_row ? 0 : tok) * a.cols;
    }
    auto residual = [&](uint32_t c, float* r) {
        uint4 u = *reinterpret_cast<const uint4*>(drow + 8 * (size_t)c);
        if (zero_row) u = make_uint4(0, 0, 0, 0);
        const float d[8] = {bf_lo(u.x), bf_hi(u.x), bf_lo(u.y), bf_hi(u.y), bf_lo(u.z), bf_hi(u.z), bf_lo(u.w), bf_hi(u.w)};
        if (PRO == PRO_NORM) {
            const float4 r0 = *reinterpret_cast<const float4*>(a.res_in + 8 * (size_t)c);
            const float4 r1 = *reinterpret_cast<const float4*>(a.res_in + 8 * (size_t)c + 4);
            r[0] = r0.x + d[0]; r[1] = r0.y + d[1]; r[2] = r0.z + d[2]; r[3] = r0.w + d[3];
            r[4] = r1.x + d[4]; r[5] = r1.y + d[5]; r[6] = r1.z + d[6]; r[7] = r1.w + d[7];
        } else {
#pragma unroll
            for (int k = 0; k < 8; ++k) r[k] = 0.f + d[k];
        }
    };
    // Pass 1: r = residual + delta (f32), block 0 writes it out, squares summed in f64.
    float keep[KEEP][8];
    double ss = 0.0;
    uint32_t it = 0;
    for (uint32_t c = t; c < C; c += BLOCK, ++it) {
        float r[8];
        residual(c, r);
        if (blockIdx.x == 0 && a.res_out != nullptr) {
            float4* o = reinterpret_cast<float4*>(a.res_out + 8 * (size_t)c);
            o[0] = make_float4(r[0], r[1], r[2], r[3]);
            o[1] = make_float4(r[4], r[5], r[6], r[7]);
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) ss += (double)r[k] * (double)r[k];
#pragma unroll
        for (uint32_t q = 0; q < KEEP; ++q)
            if (it == q) {
#pragma unroll
                for (int k = 0; k < 8; ++k) keep[q][k] = r[k];
            }
    }
    const double total = block_sum_d(ss, sh);
    const double scale = 1.0 / sqrt(total / (double)a.cols + (double)a.eps);
    // Pass 2: x = bf16(r * scale * w) in f64.
    it = 0;
    for (uint32_t c = t; c < C; c += BLOCK, ++it) {
        float r[8];
        if (it < KEEP) {
#pragma unroll
            for (uint32_t q = 0; q < KEEP; ++q)
                if (it == q) {
#pragma unroll
                    for (int k = 0; k < 8; ++k) r[k] = keep[q][k];
                }
        } else {
            residual(c, r);
        }
        const uint4 wn = *reinterpret_cast<const uint4*>(a.norm_w + 8 * (size_t)c);
        const float w[8] = {bf_lo(wn.x), bf_hi(wn.x), bf_lo(wn.y), bf_hi(wn.y), bf_lo(wn.z), bf_hi(wn.z), bf_lo(wn.w), bf_hi(wn.w)};
        bf16_t o[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) o[k] = f2bf((float)((double)r[k] * scale * (double)w[k]));
        xl[c] = make_uint4(pack2(o[0], o[1]), pack2(o[2], o[3]), pack2(o[4], o[5]), pack2(o[6], o[7]));
    }
    __syncthreads();
}

template <class A>
__device__ __forceinline__ A dot8(const uint4 w, const float* x, A acc);

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

// Each product of two bf16 is exact in f32; it is added in f64.
template <>
__device__ __forceinline__ double dot8<double>(const uint4 w, const float* x, double acc) {
    acc += (double)(bf_lo(w.x) * x[0]);
    acc += (double)(bf_hi(w.x) * x[1]);
    acc += (double)(bf_lo(w.y) * x[2]);
    acc += (double)(bf_hi(w.y) * x[3]);
    acc += (double)(bf_lo(w.z) * x[4]);
    acc += (double)(bf_hi(w.z) * x[5]);
    acc += (double)(bf_lo(w.w) * x[6]);
    acc += (double)(bf_hi(w.w) * x[7]);
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

// A wavefront's work is a sequence of tiles: row group g (R rows; for EPI_SWIGLU R / 2 gate rows
// i.. and the up rows inter + i..) times batch b (chunks 64 BATCH b + lane + 64 j, j < BATCH, of
// each row). Tiles are double-buffered in registers: while one is summed the next is in flight,
// and the first two are requested before the prologue, so the weights' latency overlaps the
// staging of x. A group's sums are reduced over the wavefront after its last batch.
struct TilePos {
    uint32_t g, b;
};

template <int R, int BATCH, int PRO, int EPI, class Acc>
__device__ __forceinline__ void gemv_body(const GemvArgs& a, uint4* xl) {
    __shared__ double sh[16];
    __shared__ float best_v[WAVES];
    __shared__ uint32_t best_i[WAVES];
    __shared__ int any_nan;
    __shared__ uint32_t last;
    const uint32_t t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const uint32_t C = a.cols / 8;
    const uint32_t NB = (C + 64 * BATCH - 1) / (64 * BATCH);  // batches per row group
    constexpr int PAIRS = R / 2;
    const uint32_t inter = a.rows / 2;
    const uint32_t groups = EPI == EPI_SWIGLU ? (inter + PAIRS - 1) / PAIRS : (a.rows + R - 1) / R;
    const uint32_t gw = blockIdx.x * WAVES + wave, nw = gridDim.x * WAVES;
    const uint32_t my_groups = gw < groups ? (groups - gw + nw - 1) / nw : 0;
    const uint32_t T = my_groups * NB;  // wavefront-uniform
    if (EPI == EPI_ARGMAX && t == 0) any_nan = 0;

    auto row_of = [&](uint32_t g, int r, bool& in) -> uint32_t {
        if (EPI == EPI_SWIGLU) {
            const uint32_t i = g * PAIRS + (r % PAIRS);
            in = i < inter;
            return r < PAIRS ? i : inter + i;
        }
        const uint32_t row = g * R + r;
        in = row < a.rows;
        return row;
    };
    auto load = [&](uint4 (&w)[R][BATCH], TilePos p) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            bool in;
            const uint32_t row = row_of(p.g, r, in);
            const bf16_t* wr = a.w + (size_t)row * a.cols;
#pragma unroll
            for (int j = 0; j < BATCH; ++j) {
                const uint32_t c = lane + 64 * (BATCH * p.b + j);
                w[r][j] = (in && c < C) ? *reinterpret_cast<const uint4*>(wr + 8 * (size_t)c) : make_uint4(0, 0, 0, 0);
            }
        }
    };
    auto advance = [&](TilePos& p) {
        if (++p.b == NB) {
            p.b = 0;
            p.g += nw;
        }
    };

    uint4 w0[R][BATCH], w1[R][BATCH];
    TilePos lp = {gw, 0};  // next tile to request
    if (T > 0) {
        load(w0, lp);
        advance(lp);
    }
    if (T > 1) {
        load(w1, lp);
        advance(lp);
    }

    stage_x<PRO>(a, xl, sh);

    float bv = -INFINITY;
    uint32_t bi = NO_TOKEN;
    bool nan = false;
    Acc acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = (Acc)0;

    auto consume = [&](const uint4 (&w)[R][BATCH], TilePos p) {
#pragma unroll
        for (int j = 0; j < BATCH; ++j) {
            const uint32_t c = lane + 64 * (BATCH * p.b + j);
            if (c < C) {
                const uint4 u = xl[c];
                const float x[8] = {bf_lo(u.x), bf_hi(u.x), bf_lo(u.y), bf_hi(u.y),
                                    bf_lo(u.z), bf_hi(u.z), bf_lo(u.w), bf_hi(u.w)};
#pragma unroll
                for (int r = 0; r < R; ++r) acc[r] = dot8<Acc>(w[r][j], x, acc[r]);
            }
        }
        if (p.b + 1 != NB) return;
        // The group's last batch: reduce and write.
        const Acc sum = wave_reduce_rows<R, Acc>(acc);
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = (Acc)0;
        const uint32_t k = reduced_row<R>(lane);
        const bool holder = (lane & (64 / R - 1)) == 0;  // one lane per row holds its sum
        if (EPI == EPI_SWIGLU) {
            // Gate k < PAIRS sits in the lower lanes, up k + PAIRS in the upper: bring up down.
            const Acc up = __shfl_xor(sum, 32, 64);
            const uint32_t i = p.g * PAIRS + k;
            if (holder && k < (uint32_t)PAIRS && i < inter) {
                const double gd = (double)bf_round((float)sum), ud = (double)bf_round((float)up);
                reinterpret_cast<bf16_t*>(a.y)[i] = f2bf((float)(gd / (1.0 + exp(-gd)) * ud));
            }
        } else if (holder) {
            const uint32_t r = p.g * R + k;
            if (r < a.rows) {
                const float s = (float)sum;
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
    };

    TilePos cp = {gw, 0};  // next tile to sum
    for (uint32_t i = 0; i < T; i += 2) {
        consume(w0, cp);
        advance(cp);
        if (i + 2 < T) {
            load(w0, lp);
            advance(lp);
        }
        if (i + 1 >= T) break;
        consume(w1, cp);
        advance(cp);
        if (i + 3 < T) {
            load(w1, lp);
            advance(lp);
        }
    }
    if (EPI != EPI_ARGMAX) return;

    // This block's candidate: each wave's over its lanes, then the waves' in LDS.
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const uint32_t oi = __shfl_xor(bi, o, 64);
        if (better(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    }
    if (__any(nan) && lane == 0) atomicOr(&any_nan, 1);
    if (lane == 0) {
        best_v[wave] = bv;
        best_i[wave] = bi;
    }
    __syncthreads();
    if (t == 0) {
        float fv = -INFINITY;
        uint32_t fi = NO_TOKEN;
        for (int w = 0; w < WAVES; ++w)
            if (better(best_v[w], best_i[w], fv, fi)) {
                fv = best_v[w];
                fi = best_i[w];
            }
        a.partial[3 * blockIdx.x] = fv;
        a.partial[3 * blockIdx.x + 1] = __uint_as_float(fi);
        a.partial[3 * blockIdx.x + 2] = any_nan ? 1.f : 0.f;
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
    __syncthreads();
    if (lane == 0) {
        best_v[wave] = v;
        best_i[wave] = i;
        if (wn) atomicOr(&any_nan, 2);
    }
    __syncthreads();
    if (t == 0) {
        float fv = -INFINITY;
        uint32_t fi = NO_TOKEN;
        for (int w = 0; w < WAVES; ++w)
            if (better(best_v[w], best_i[w], fv, fi)) {
                fv = best_v[w];
                fi = best_i[w];
            }
        a.token_out[0] = (any_nan & 2) ? NO_TOKEN : fi;
        if (a.advance) a.pos[0] += 1u;
        a.counter[0] = 0;  // ready for the next launch
    }
}

}  // namespace

template <int R, int BATCH, int PRO, int EPI, class Acc>
__global__ void __launch_bounds__(256) gemv_kernel(GemvArgs a) {
    extern __shared__ uint4 xl[];
    gemv_body<R, BATCH, PRO, EPI, Acc>(a, xl);
}

// Plain GEMV for the kernel table and tests: y[rows] = W x, bf16 or f32 out, f32 accumulation,
// cols a multiple of 8 up to 16384 (x staged in 32 KiB of static LDS); any grid (persistent),
// block 256.
#define X0NE_GEMV_PLAIN(NAME, EPI)                                                                                \
    extern "C" __global__ void __launch_bounds__(256) NAME(const bf16_t* __restrict__ w, const bf16_t* __restrict__ x, \
                                                          void* __restrict__ y, uint32_t rows, uint32_t cols) {     \
        __shared__ uint4 xs[16384 / 8];                                                                           \
        if (cols > 16384 || cols % 8) return;                                                                     \
        GemvArgs a = {};                                                                                          \
        a.w = w;                                                                                                  \
        a.x = x;                                                                                                  \
        a.y = y;                                                                                                  \
        a.rows = rows;                                                                                            \
        a.cols = cols;                                                                                            \
        gemv_body<4, 4, PRO_X, EPI, float>(a, xs);                                                                   \
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

constexpr int TILE_R = 4;      // rows per row group
constexpr int TILE_BATCH = 4;  // 16-byte chunks per lane per row in one tile

template <int P, int E>
const void* instance(int f64acc) {
    return f64acc ? (const void*)&gemv_kernel<TILE_R, TILE_BATCH, P, E, double>
                  : (const void*)&gemv_kernel<TILE_R, TILE_BATCH, P, E, float>;
}

const void* pick(int pro, int epi, int f64acc) {
#define X0NE_CASE(P, E) \
    if (pro == P && epi == E) return instance<P, E>(f64acc);
    X0NE_CASE(PRO_X, EPI_BF16)
    X0NE_CASE(PRO_X, EPI_F32)
    X0NE_CASE(PRO_NORM, EPI_BF16)
    X0NE_CASE(PRO_NORM, EPI_SWIGLU)
    X0NE_CASE(PRO_NORM, EPI_ARGMAX)
    X0NE_CASE(PRO_NORM, EPI_F32)
    X0NE_CASE(PRO_EMBED_NORM, EPI_BF16)
#undef X0NE_CASE
    return nullptr;
}

bool shape_ok(const X0neGemv& g) {
    return g.cols != 0 && g.cols % 8 == 0 && g.cols <= 32768 && g.rows != 0 &&
           (g.epilogue != EPI_SWIGLU || g.rows % 2 == 0);
}

}  // namespace

// The grid of a launch: as many wavefronts as can be resident at once (the kernel's occupancy
// on `cus` CUs, capped at `max_blocks_per_cu` blocks per CU when that is not 0), then cut so the
// row groups divide as evenly as they can: each wavefront takes ceil(groups / waves) of them,
// and no more wavefronts are launched than that split needs.
uint32_t x0ne_gemv_grid(const X0neGemv& g, uint32_t cus, uint32_t max_blocks_per_cu) {
    if (!shape_ok(g) || cus == 0) return 0;
    const void* fn = pick(g.prologue, g.epilogue, g.f64acc);
    if (!fn) return 0;
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, BLOCK, (size_t)g.cols * 2) != hipSuccess ||
        per_cu <= 0)
        per_cu = 1;
    if (max_blocks_per_cu != 0 && (uint32_t)per_cu > max_blocks_per_cu) per_cu = (int)max_blocks_per_cu;
    const uint64_t groups = g.epilogue == EPI_SWIGLU ? ((uint64_t)g.rows / 2 + TILE_R / 2 - 1) / (TILE_R / 2)
                                                     : ((uint64_t)g.rows + TILE_R - 1) / TILE_R;
    const uint64_t waves_max = (uint64_t)cus * (uint64_t)per_cu * WAVES;
    const uint64_t per_wave = (groups + waves_max - 1) / waves_max;
    const uint64_t waves = (groups + per_wave - 1) / per_wave;
    return (uint32_t)((waves + WAVES - 1) / WAVES);
}

hipError_t x0ne_launch_gemv(const X0neGemv& g, hipStream_t s) {
    if (!shape_ok(g) || g.grid == 0) return hipErrorInvalidValue;
    const void* fn = pick(g.prologue, g.epilogue, g.f64acc);
    if (!fn) return hipErrorInvalidValue;
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
    void* args[] = {(void*)&a};
    return x0ne_launch(fn, dim3(g.grid), dim3(BLOCK), args, (size_t)g.cols * 2, s);
}
