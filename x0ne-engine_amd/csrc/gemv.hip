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

// ---- branch-free loads ----
// A raw buffer resource over `bytes` bytes at `base` (gfx9 word 3: 32-bit data format). A load
// whose 16 bytes are not all inside gives zeros and touches no memory, so a row past the matrix,
// a chunk past the row or a prefetch past the last tile needs no branch: every load of the
// pipeline is an instruction the compiler can count, and its waits cover only what is needed.
constexpr int RSRC_WORD3 = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, RSRC_WORD3);
}

// Cache policy of the weight stream: non-temporal (each weight byte is read once per step, so
// keeping it in the L2 or the Infinity Cache only evicts what is reused). Measured on MI355X: a
// streaming read of the LM head's 1.25 GB takes 201 µs with it, 218 µs without.
constexpr int CPOL_NT = 2;

template <int CPOL = 0>
__device__ __forceinline__ uint4 load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, CPOL);
    return make_uint4((uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]);
}

// The prologue's inputs, XC 16-byte chunks per thread (chunk t + 256 i): requested first, used
// after the first weight tiles are in flight.
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4 load16f(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}

template <int PRO, int XC>
struct XIn {
    uint4 d[XC];                // x (PRO_X) or delta / the embedding row (norm prologues)
    f32x4 r0[XC], r1[XC];       // the f32 residual (PRO_NORM)
    uint4 w[XC];                // the norm weight (norm prologues)
};

template <int PRO, int XC>
__device__ __forceinline__ void x_request(const GemvArgs& a, XIn<PRO, XC>& in) {
    const uint32_t t = threadIdx.x;
    if (PRO == PRO_X) {
        const auto xr = rsrc(a.x, a.cols * 2);
#pragma unroll
        for (int i = 0; i < XC; ++i) in.d[i] = load16(xr, (t + BLOCK * i) * 16);
        return;
    }
    __amdgpu_buffer_rsrc_t dr;
    if (PRO == PRO_EMBED_NORM) {
        const uint32_t tok = a.tokens[0];
        // A token past the table gives a zero row (embedding.cu:5-17).
        dr = rsrc(a.embed + (size_t)(tok < a.vocab ? tok : 0) * a.cols, tok < a.vocab ? a.cols * 2 : 0);
    } else {
        dr = rsrc(a.delta, a.cols * 2);
    }
    const auto nr = rsrc(a.norm_w, a.cols * 2);
#pragma unroll
    for (int i = 0; i < XC; ++i) {
        const uint32_t c = t + BLOCK * i;
        in.d[i] = load16(dr, c * 16);
        in.w[i] = load16(nr, c * 16);
        if (PRO == PRO_NORM) {
            const auto rr = rsrc(a.res_in, a.cols * 4);
            in.r0[i] = load16f(rr, c * 32);
            in.r1[i] = load16f(rr, c * 32 + 16);
        }
    }
}

// Stages x (bf16) in LDS from the requested inputs: the given x, or bf16(rmsnorm(residual +
// delta) * w_norm) with the residual add in f32 and the norm in f64; block 0 writes the new
// residual. Block-wide; ends with a barrier.
template <int PRO, int XC>
__device__ __forceinline__ void x_stage(const GemvArgs& a, const XIn<PRO, XC>& in, uint4* xl, double* sh) {
    const uint32_t t = threadIdx.x, C = a.cols / 8;
    if (PRO == PRO_X) {
#pragma unroll
        for (int i = 0; i < XC; ++i)
            if (t + BLOCK * i < C) xl[t + BLOCK * i] = in.d[i];
        lds_barrier();
        return;
    }
    float r[XC][8];
    double ss = 0.0;
#pragma unroll
    for (int i = 0; i < XC; ++i) {
        const uint4 u = in.d[i];
        const float d[8] = {bf_lo(u.x), bf_hi(u.x), bf_lo(u.y), bf_hi(u.y), bf_lo(u.z), bf_hi(u.z), bf_lo(u.w), bf_hi(u.w)};
        if (PRO == PRO_NORM) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                r[i][k] = in.r0[i][k] + d[k];
                r[i][k + 4] = in.r1[i][k] + d[k + 4];
            }
        } else {
#pragma unroll
            for (int k = 0; k < 8; ++k) r[i][k] = 0.f + d[k];
        }
        const uint32_t c = t + BLOCK * i;
        if (blockIdx.x == 0 && a.res_out != nullptr && c < C) {
            float4* o = reinterpret_cast<float4*>(a.res_out + 8 * (size_t)c);
            o[0] = make_float4(r[i][0], r[i][1], r[i][2], r[i][3]);
            o[1] = make_float4(r[i][4], r[i][5], r[i][6], r[i][7]);
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) ss += (double)r[i][k] * (double)r[i][k];  // chunks past C are 0
    }
    const double total = block_sum_lds<WAVES>(ss, sh);
    const double scale = 1.0 / sqrt(total / (double)a.cols + (double)a.eps);
#pragma unroll
    for (int i = 0; i < XC; ++i) {
        const uint32_t c = t + BLOCK * i;
        const uint4 wn = in.w[i];
        const float w[8] = {bf_lo(wn.x), bf_hi(wn.x), bf_lo(wn.y), bf_hi(wn.y), bf_lo(wn.z), bf_hi(wn.z), bf_lo(wn.w), bf_hi(wn.w)};
        bf16_t o[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) o[k] = f2bf((float)((double)r[i][k] * scale * (double)w[k]));
        if (c < C) xl[c] = make_uint4(pack2(o[0], o[1]), pack2(o[2], o[3]), pack2(o[4], o[5]), pack2(o[6], o[7]));
    }
    lds_barrier();
}

// A wavefront's work is a sequence of tiles: row group g (R rows; for EPI_SWIGLU R / 2 gate rows
// i.. and the up rows inter + i..) times batch b (chunks 64 BATCH b + lane + 64 j, j < BATCH, of
// each row). Tiles are double-buffered in registers: while one is summed the next is in flight,
// and the first is requested right after the prologue's inputs, so waiting for x leaves it in
// flight (the prologue's barriers wait for LDS only). Every load is unconditional (buffer resources bound rows and chunks), so
// the compiler's waits before a tile cover that tile only. A group's sums are reduced over the
// wavefront after its last batch.
struct TilePos {
    uint32_t g, b;
};

// Work mapping (MAP bits). MAP_CONTIGUOUS: wavefront w takes row groups [w per, w per + per)
// instead of w, w + W, ... MAP_XCD: launch ids alternate between the 8 XCDs (each with its own
// L2), so block id (b % 8) (grid / 8) + b / 8 gives each XCD a contiguous range of blocks (the
// grid is then a multiple of 8).
constexpr int MAP_CONTIGUOUS = 1;
constexpr int MAP_XCD = 2;
// MAP_SPREAD: batch b of a row takes chunks lane + 64 (b + NB j), spread over the whole row,
// instead of a contiguous run. MAP_STAGGER: wavefront w starts each row group at batch w % NB,
// so wavefronts in step do not all read the same part of their rows.
constexpr int MAP_SPREAD = 4;
constexpr int MAP_STAGGER = 8;

template <int R, int BATCH, int PRO, int EPI, class Acc, int XC, int MAP>
__device__ __forceinline__ void gemv_body(const GemvArgs& a, uint4* xl) {
    __shared__ double sh[16];
    __shared__ float best_v[WAVES];
    __shared__ uint32_t best_i[WAVES];
    __shared__ int any_nan;
    __shared__ uint32_t last;
    const uint32_t t = threadIdx.x, lane = t & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(t >> 6);  // uniform: row resources in SGPRs
    const uint32_t C = a.cols / 8;
    const uint32_t NB = (C + 64 * BATCH - 1) / (64 * BATCH);  // batches per row group
    constexpr int PAIRS = R / 2;
    const uint32_t inter = a.rows / 2;
    const uint32_t groups = EPI == EPI_SWIGLU ? (inter + PAIRS - 1) / PAIRS : (a.rows + R - 1) / R;
    const uint32_t bid = (MAP & MAP_XCD) ? (blockIdx.x & 7) * (gridDim.x >> 3) + (blockIdx.x >> 3) : blockIdx.x;
    const uint32_t gw = bid * WAVES + wave, nw = gridDim.x * WAVES;
    uint32_t g0, gstep, my_groups;
    if (MAP & MAP_CONTIGUOUS) {
        const uint32_t per = (groups + nw - 1) / nw;
        g0 = gw * per;
        gstep = 1;
        my_groups = g0 < groups ? min(per, groups - g0) : 0;
    } else {
        g0 = gw;
        gstep = nw;
        my_groups = gw < groups ? (groups - gw + nw - 1) / nw : 0;
    }
    const uint32_t T = my_groups * NB;  // wavefront-uniform
    if (EPI == EPI_ARGMAX && t == 0) any_nan = 0;

    // Chunk j of batch b.
    auto chunk = [&](uint32_t b, int j) -> uint32_t {
        return (MAP & MAP_SPREAD) ? lane + 64 * (b + NB * j) : lane + 64 * (BATCH * b + j);
    };
    const uint32_t b0 = (MAP & MAP_STAGGER) ? gw % NB : 0;  // first batch of each row group
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
    // live = false: a prefetch past the wavefront's last tile (reads nothing).
    auto load = [&](uint4 (&w)[R][BATCH], TilePos p, bool live) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            bool in;
            const uint32_t row = row_of(p.g, r, in);
            const auto rs = rsrc(a.w + (size_t)(in && live ? row : 0) * a.cols, in && live ? a.cols * 2 : 0);
#pragma unroll
            for (int j = 0; j < BATCH; ++j) w[r][j] = load16<CPOL_NT>(rs, chunk(p.b, j) * 16);
        }
    };
    // Batches of a group run b0, b0 + 1, ..., NB - 1, 0, ..., b0 - 1; the group ends at its last.
    auto advance = [&](TilePos& p) {
        if (++p.b == NB) p.b = 0;
        if (p.b == b0) p.g += gstep;
    };

    uint4 w0[R][BATCH], w1[R][BATCH];
    TilePos lp = {g0, b0};  // next tile to request
    {
        XIn<PRO, XC> xin;
        x_request<PRO, XC>(a, xin);
        __builtin_amdgcn_sched_barrier(0);  // keep the request order: x first, then the weights
        load(w0, lp, T > 0);
        advance(lp);
        __builtin_amdgcn_sched_barrier(0);
        x_stage<PRO, XC>(a, xin, xl, sh);
    }
    load(w1, lp, T > 1);
    advance(lp);

    float bv = -INFINITY;
    uint32_t bi = NO_TOKEN;
    bool nan = false;
    // Sums start from -0.0, the neutral element of the reference's f64 sums (Rust's
    // Iterator::sum, oracle/src/lib.rs:123-133): a row whose products are all negative zeros
    // sums to -0.0, any other as from +0.0.
    Acc acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = (Acc)-0.0f;

    auto consume = [&](const uint4 (&w)[R][BATCH], TilePos p) {
#pragma unroll
        for (int j = 0; j < BATCH; ++j) {
            const uint32_t c = chunk(p.b, j);
            const bool ok = c < C;
            const uint4 u = xl[ok ? c : 0];
            // A chunk past the row: its weights are zeros, and x is -0.0 (0 times a value that
            // is not finite would not be 0), so each product is -0.0 and leaves a sum as it is.
            // x in the accumulation type, converted once for the R rows.
            const Acc x[8] = {(Acc)(ok ? bf_lo(u.x) : -0.f), (Acc)(ok ? bf_hi(u.x) : -0.f), (Acc)(ok ? bf_lo(u.y) : -0.f),
                              (Acc)(ok ? bf_hi(u.y) : -0.f), (Acc)(ok ? bf_lo(u.z) : -0.f), (Acc)(ok ? bf_hi(u.z) : -0.f),
                              (Acc)(ok ? bf_lo(u.w) : -0.f), (Acc)(ok ? bf_hi(u.w) : -0.f)};
#pragma unroll
            for (int r = 0; r < R; ++r) acc[r] = dot8<Acc>(w[r][j], x, acc[r]);
        }
        if ((p.b + 1 == NB ? 0 : p.b + 1) != b0) return;
        // The group's last batch: reduce and write.
        const Acc sum = wave_reduce_rows<R, Acc>(acc);
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = (Acc)-0.0f;
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

    TilePos cp = {g0, b0};  // next tile to sum
    for (uint32_t i = 0; i < T; i += 2) {
        consume(w0, cp);
        advance(cp);
        load(w0, lp, i + 2 < T);
        advance(lp);
        if (i + 1 >= T) break;
        consume(w1, cp);
        advance(cp);
        load(w1, lp, i + 3 < T);
        advance(lp);
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

template <int R, int BATCH, int PRO, int EPI, class Acc, int XC, int MAP>
__global__ void __launch_bounds__(256) gemv_kernel(GemvArgs a) {
    extern __shared__ uint4 xl[];
    gemv_body<R, BATCH, PRO, EPI, Acc, XC, MAP>(a, xl);
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
        gemv_body<4, 4, PRO_X, EPI, float, 8, 0>(a, xs);                                                             \
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

// Tile shape and residency per epilogue, measured on MI355X over 36 distinct matrices of each
// Qwen3-8B projection: narrow tiles (2 rows x 4 chunks) at one block per CU for the plain and
// normed projections, 4 x 4 tiles at the kernel's occupancy for gate/up (both rows of a SwiGLU
// pair in one wavefront), and whole-row 4 x 8 tiles at one block per CU for the LM head. More
// resident wavefronts than that (more rows streamed at once) lowered the achieved bandwidth.
// Rows of at most 1024 columns (Qwen3-0.6B's hidden size: 128 chunks, two per lane) take tiles
// of two chunks per lane and as many more rows, so a tile is the same size and every load reads
// weights (a 4- or 8-chunk tile of a 2 KiB row would leave half or three quarters of its loads
// past the row). Each lane sums the same chunks in the same order and the lane sums meet in the
// same butterfly, so the sums are the same bits.
constexpr uint32_t NARROW_COLS = 1024;
template <int E, bool NARROW = false>
struct Tile {
    static constexpr int R = NARROW ? 4 : 2, BATCH = NARROW ? 2 : 4, BLOCKS_PER_CU = 1;
};
template <bool NARROW>
struct Tile<EPI_SWIGLU, NARROW> {
    static constexpr int R = NARROW ? 8 : 4, BATCH = NARROW ? 2 : 4, BLOCKS_PER_CU = 0;  // 0: the occupancy
};
template <bool NARROW>
struct Tile<EPI_ARGMAX, NARROW> {
    static constexpr int R = NARROW ? 16 : 4, BATCH = NARROW ? 2 : 8, BLOCKS_PER_CU = 1;
};
constexpr int TILE_MAP = 0;  // strided row groups, launch order

// 16-byte chunks of x per thread the prologue requests: the smallest of 2, 4, 8, 16 that covers
// cols / 8 over 256 threads (the norm prologues keep four registers per chunk and stop at 8).
int x_chunks(uint32_t cols) {
    const uint32_t per = (cols / 8 + BLOCK - 1) / BLOCK;
    return per <= 2 ? 2 : per <= 4 ? 4 : per <= 8 ? 8 : 16;
}

template <int P, int E, int XC, bool NARROW = false>
const void* instance(int f64acc) {
    constexpr int R = Tile<E, NARROW>::R, B = Tile<E, NARROW>::BATCH;
    return f64acc ? (const void*)&gemv_kernel<R, B, P, E, double, XC, TILE_MAP>
                  : (const void*)&gemv_kernel<R, B, P, E, float, XC, TILE_MAP>;
}

// A narrow row (at most 1024 columns) always takes 2 x chunks per thread.
template <int P, int E>
const void* instance_x(int f64acc, int xc, bool narrow) {
    if (narrow) return xc == 2 ? instance<P, E, 2, true>(f64acc) : nullptr;
    if (xc == 2) return instance<P, E, 2>(f64acc);
    if (xc == 4) return instance<P, E, 4>(f64acc);
    if (xc == 8) return instance<P, E, 8>(f64acc);
    if constexpr (P == PRO_X) {
        if (xc == 16) return instance<P, E, 16>(f64acc);
    }
    return nullptr;
}

const void* pick(int pro, int epi, int f64acc, uint32_t cols) {
    const int xc = x_chunks(cols);
    const bool narrow = cols <= NARROW_COLS;
#define X0NE_CASE(P, E) \
    if (pro == P && epi == E) return instance_x<P, E>(f64acc, xc, narrow);
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

// Rows per row group and the default blocks-per-CU cap of an epilogue's tile at this width.
template <bool NARROW>
void tile_of_w(int epi, uint32_t* rows, uint32_t* blocks_per_cu) {
    if (epi == EPI_SWIGLU) {
        *rows = Tile<EPI_SWIGLU, NARROW>::R;
        *blocks_per_cu = Tile<EPI_SWIGLU, NARROW>::BLOCKS_PER_CU;
    } else if (epi == EPI_ARGMAX) {
        *rows = Tile<EPI_ARGMAX, NARROW>::R;
        *blocks_per_cu = Tile<EPI_ARGMAX, NARROW>::BLOCKS_PER_CU;
    } else {
        *rows = Tile<EPI_BF16, NARROW>::R;
        *blocks_per_cu = Tile<EPI_BF16, NARROW>::BLOCKS_PER_CU;
    }
}
void tile_of(int epi, uint32_t cols, uint32_t* rows, uint32_t* blocks_per_cu) {
    if (cols <= NARROW_COLS)
        tile_of_w<true>(epi, rows, blocks_per_cu);
    else
        tile_of_w<false>(epi, rows, blocks_per_cu);
}

bool shape_ok(const X0neGemv& g) {
    return g.cols != 0 && g.cols % 8 == 0 && g.cols <= (g.prologue == PRO_X ? 32768u : 16384u) && g.rows != 0 &&
           (g.epilogue != EPI_SWIGLU || g.rows % 2 == 0);
}

}  // namespace

// The grid of a launch: as many wavefronts as the epilogue's tile keeps resident (its
// blocks-per-CU cap, or the kernel's occupancy; `max_blocks_per_cu`, when not 0, overrides
// both), then cut so the row groups divide as evenly as they can: each wavefront takes
// ceil(groups / waves) of them, and no more wavefronts are launched than that split needs.
uint32_t x0ne_gemv_grid(const X0neGemv& g, uint32_t cus, uint32_t max_blocks_per_cu) {
    if (!shape_ok(g) || cus == 0) return 0;
    const void* fn = pick(g.prologue, g.epilogue, g.f64acc, g.cols);
    if (!fn) return 0;
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, BLOCK, (size_t)g.cols * 2) != hipSuccess ||
        per_cu <= 0)
        per_cu = 1;
    uint32_t rows = 0, cap = 0;
    tile_of(g.epilogue, g.cols, &rows, &cap);
    if (max_blocks_per_cu != 0) cap = max_blocks_per_cu;
    if (cap != 0 && (uint32_t)per_cu > cap) per_cu = (int)cap;
    const uint64_t groups = g.epilogue == EPI_SWIGLU ? ((uint64_t)g.rows / 2 + rows / 2 - 1) / (rows / 2)
                                                     : ((uint64_t)g.rows + rows - 1) / rows;
    const uint64_t waves_max = (uint64_t)cus * (uint64_t)per_cu * WAVES;
    const uint64_t per_wave = (groups + waves_max - 1) / waves_max;
    const uint64_t waves = (groups + per_wave - 1) / per_wave;
    return (uint32_t)((waves + WAVES - 1) / WAVES);
}

hipError_t x0ne_launch_gemv(const X0neGemv& g, hipStream_t s) {
    if (!shape_ok(g) || g.grid == 0) return hipErrorInvalidValue;
    const void* fn = pick(g.prologue, g.epilogue, g.f64acc, g.cols);
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
