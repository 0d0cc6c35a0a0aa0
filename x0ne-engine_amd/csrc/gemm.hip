// The projections of a pass over a few rows (the batched decode step, a short prompt) on the
// matrix cores: Y[n][rows] = X[n][cols] W^T with W [rows][cols] and X [n][cols] bf16 row-major,
// f32 accumulation, Y bf16 or f32 (the reference's Gpu::gemm, gpu.rs:1098-1149). At one row the
// decode GEMV (gemv.hip) is the right kernel; past 64 rows the work is a compute-bound GEMM,
// the tiled kernels further down.
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

// CPOL: the cache policy (0 the default; CPOL_NT non-temporal, for a stream read once).
constexpr int CPOL_NT = 2;
template <int CPOL = 0>
__device__ __forceinline__ uint4 bload(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, CPOL);
    return make_uint4((uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]);
}

}  // namespace

// ---- a few rows: Y[n][rows] = X[n][cols] W^T for n <= 64, bandwidth-bound ----
// The batched decode step's projections and a short prompt's. Every W row is read once, so the
// kernel streams W at the HBM rate and the few-row matrix-core products cost nothing beside it:
//  - Block b takes the RG row groups of 16 W rows 16 RG b .. 16 RG b + 16 RG - 1 over all of K;
//    its V wavefronts (V = blockDim / 64, chosen by the host with RG so the launch holds enough
//    loads in flight) take its steps of 32 columns in turn (wavefront w: steps w, w + V, ..), so
//    at any time a block reads one contiguous run of each of its panels.
//  - W is read with a non-temporal hint (each byte read once), X with the default policy (every
//    block reads it, from the L2). Measured on MI355X on the batched Qwen3-8B and -32B shapes
//    (W and X in panels): 3-19 % faster than each wavefront reading its own quarter of K with the
//    default policy.
//  - A step is TT x RG 16 x 16 x 32 products (TT tiles of 16 tokens, RG row groups) whose A
//    operand is X (row = token, zero past n) and B operand W (column = W row): lane l loads
//    16 bytes, columns k0 + 8 (l / 16) .. + 7, of W row 16 (RG b + g) + l % 16 and of X row
//    16 tt + l % 16; the 4 lane groups cover 64 contiguous bytes of each row. One X piece
//    serves the RG row groups, so X (read from the L2 by every block) costs TT / RG of W's loads.
//  - U steps are in flight per wavefront: the slot a product has consumed is refilled at once
//    with the wavefront's step U ahead, so U - 1 steps stay in flight while one multiplies. A piece past K
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
// contiguous KiB and a block's steps run through its panel in order, 3.7-5.9 TB/s (MI355X).
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
    const uint32_t steps = (cols + 31) / 32;
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
        const bool in = s < steps && k < cols;  // a K tail: pieces past the row read zeros
#pragma unroll
        for (int tt = 0; tt < TT; ++tt) {
            const uint32_t t = 16 * tt + r;
            const uint32_t off = x_panel ? (uint32_t)panel_index(t, k, cols) * 2 : (t * cols + k) * 2;
            xa[u][tt] = bload<>(xr, in && t < n ? off : OFF_NONE);
        }
#pragma unroll
        for (int kd = 0; kd < KINDS; ++kd)
#pragma unroll
            for (int g = 0; g < RG; ++g) {
                const uint32_t row = 16 * (RG * b + g) + r;
                const uint32_t wrow = kd * rows + row;
                wb[u][kd][g] = bload<CPOL_NT>(wr, !(in && row < rows) ? OFF_NONE
                                         : w_panel ? (uint32_t)panel_index(wrow, k, cols) * 2
                                                   : (wrow * cols + k) * 2);
            }
    };
#pragma unroll
    for (int u = 0; u < U; ++u) request(u, wave + V * u);
    for (uint32_t s0 = wave; s0 < steps; s0 += U * V) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
#pragma unroll
            for (int kd = 0; kd < KINDS; ++kd)
#pragma unroll
                for (int g = 0; g < RG; ++g)
#pragma unroll
                    for (int tt = 0; tt < TT; ++tt) acc[kd][g][tt] = mfma(xa[u][tt], wb[u][kd][g], acc[kd][g][tt]);
            request(u, s0 + V * (U + u));
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

// ---- a few rows balanced over the CUs: one block per CU, an equal run of the steps ----
// Where the 16-row groups are between one and two per CU (the Qwen3-32B O and down projections:
// 320 groups on 256 CUs), whole groups per block leave CUs idle (RG 2: 160 blocks) or doubled
// (RG 1). Here the steps of all groups, group-major (G groups x S steps of 32 columns), are cut
// into runs of T steps, one run per block and one block per CU, and the block's V wavefronts
// take its run's steps in turn (wavefront w: steps Lb + w, Lb + w + V, ..), so every block
// streams the same bytes as one contiguous run through the panels (a run crosses a group's end
// where one panel ends and the next begins).
//  - A wavefront sums its steps in order, one accumulator at a time: where its next step is in
//    the next group, the sums go to LDS (slot g - g0), so its loads never wait on a store.
//  - The block sums each group's wavefront partials in wavefront order. A group inside its run is
//    written at once. A group cut between runs (at most two blocks meet in a group here) is
//    finished by the last of its blocks to count: each stores its sums in slot (g, block - first
//    block of g) through agent-scope stores (coherent across the XCDs' L2s), waits for their
//    acknowledgment and counts in cnt[g]; the one that completes the count adds the slots in
//    slot order, writes Y and sets the count back to 0 for the next launch.
// Every sum's order is fixed by (rows, cols, T, V): the same bits whatever n, the timing or
// which block finishes a group. Measured on MI355X (32B down, 16 rows, 262 MB): 48.1 against
// 53.0 us for RG 2 (160 blocks); shapes whose groups are not cut this way (the 8B projections,
// SwiGLU, 640 or 1600 groups) measured no faster than whole groups per block.
namespace {

__device__ __forceinline__ void bal_put(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float bal_get(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int U, int MAXG, int MAXV>
__device__ __forceinline__ void few_bal(const bf16_t* __restrict__ w, const bf16_t* __restrict__ x,
                                        void* __restrict__ y, uint32_t rows, uint32_t cols, uint32_t n,
                                        uint32_t flags, uint32_t T, float* __restrict__ ws,
                                        uint32_t* __restrict__ cnt, f32x4* stash) {
    const bool out_f32 = flags & FEW_F32, y_panel = flags & FEW_Y_PANEL;
    const uint32_t S = (cols + 31) / 32, G = rows / 16, V = blockDim.x >> 6;
    const uint64_t total = (uint64_t)G * S;
    // Grid-uniform exits for a launch that does not fit: a run touches at most MAXG groups and
    // gives every wavefront a step; X and W in panels.
    if (n == 0 || n > 16 || cols % 8 != 0 || rows % 16 != 0 || T < V || (uint64_t)T > (uint64_t)(MAXG - 2) * S + 1 ||
        total >= (1ull << 31) || V > MAXV || S < V || flags > 15 || !(flags & FEW_W_PANEL) || !(flags & FEW_X_PANEL) ||
        (out_f32 && y_panel) || (y_panel && rows % 8 != 0) || ws == nullptr || cnt == nullptr)
        return;
    const uint32_t b = blockIdx.x;
    if ((uint64_t)b * T >= total) return;  // block-uniform
    const uint32_t lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t r = lane & 15, q4 = lane >> 4;
    const uint32_t Lb = b * T, Le = (uint32_t)min<uint64_t>((uint64_t)Lb + T, total), g0 = Lb / S;
    const uint32_t cmax = (S + T - 1) / T + 1;  // blocks that can meet in one group
    const auto xr = rsrc(x, (uint64_t)16 * cols * 2);
    const auto wr = rsrc(w, (uint64_t)rows * cols * 2);
    f32x4* mine = stash + (size_t)wave * MAXG * 64 + lane;
#pragma unroll
    for (int j = 0; j < MAXG; ++j) mine[j * 64] = f32x4{0.f, 0.f, 0.f, 0.f};
    uint4 xa[U], wb[U];
    // Requests run through the wavefront's steps: (rg, rs) is request rq's group and step.
    const uint32_t L0 = Lb + wave;
    uint32_t rq = L0, rg = L0 / S, rs = L0 - rg * S;
    auto request = [&](int u) {
        const uint32_t k = 32 * rs + 8 * q4;
        const bool in = rq < Le && k < cols;  // a K tail: pieces past the row read zeros
        xa[u] = bload<>(xr, in && r < n ? (uint32_t)panel_index(r, k, cols) * 2 : OFF_NONE);
        wb[u] = bload<CPOL_NT>(wr, in ? (uint32_t)panel_index(16 * rg + r, k, cols) * 2 : OFF_NONE);
        rq += V;
        rs += V;
        if (rs >= S) {
            rs -= S;
            ++rg;
        }
    };
#pragma unroll
    for (int u = 0; u < U; ++u) request(u);
    uint32_t cq = L0, cg = L0 / S, cs = L0 - cg * S;  // the consumed step, its group and place
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
    for (uint32_t q0 = L0; q0 < Le; q0 += U * V) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (cq < Le) {  // wavefront-uniform
                acc = mfma(xa[u], wb[u], acc);
                cq += V;
                cs += V;
                if (cs >= S) {  // this wavefront's part of group cg ends: its sums to LDS
                    mine[(cg - g0) * 64] = acc;
                    acc = f32x4{0.f, 0.f, 0.f, 0.f};
                    cs -= S;
                    ++cg;
                }
            }
            request(u);
        }
    }
    if (cs != 0) mine[(cg - g0) * 64] = acc;  // the run ends inside group cg
    lds_barrier();
    // sg[i]: token 4 (lane / 16) + i, W row 16 g + lane % 16.
    auto emit = [&](uint32_t g, const f32x4& sg) {
        const uint32_t wrow = 16 * g + r;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t t = 4 * q4 + i;
            if (t >= n) continue;
            const size_t o = y_panel ? panel_index(t, wrow, rows) : (size_t)t * rows + wrow;
            if (out_f32)
                static_cast<float*>(y)[o] = sg[i];
            else
                static_cast<bf16_t*>(y)[o] = f2bf(sg[i]);
        }
    };
    auto slot = [&](uint32_t g, uint32_t c) { return ws + ((size_t)g * cmax + c) * 256 + lane * 4; };
    const uint32_t ng = (Le - 1) / S - g0 + 1;
    // Wavefront w finishes the block's groups w, w + V, ..
    for (uint32_t j = wave; j < ng; j += V) {
        const uint32_t g = g0 + j;
        f32x4 sg = stash[j * 64 + lane];
        for (uint32_t v = 1; v < V; ++v) sg += stash[(v * MAXG + j) * 64 + lane];
        const uint32_t fb = (uint32_t)((uint64_t)g * S / T), lb = (uint32_t)(((uint64_t)g * S + S - 1) / T);
        if (fb == lb) {
            emit(g, sg);
            continue;
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) bal_put(slot(g, b - fb) + e, sg[e]);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the slot acknowledged, then the count
        uint32_t old = 0;
        if (lane == 0) old = __hip_atomic_fetch_add(cnt + g, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (__builtin_amdgcn_readfirstlane(old) != lb - fb) continue;
#pragma unroll
        for (int e = 0; e < 4; ++e) sg[e] = bal_get(slot(g, 0) + e);
        for (uint32_t c = 1; c <= lb - fb; ++c)
#pragma unroll
            for (int e = 0; e < 4; ++e) sg[e] += bal_get(slot(g, c) + e);
        emit(g, sg);
        if (lane == 0) __hip_atomic_store(cnt + g, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

}  // namespace

// x0ne_gemm_few_bal_bf16: grid ceil(G S / T) for G = rows / 16 groups and S = ceil(cols / 32)
// steps, block 64 V threads (V <= 8, V <= T <= 4 S + 1); n in 1 .. 16; rows a multiple of 16,
// cols of 8; X and W in panels (flags FEW_X_PANEL | FEW_W_PANEL, FEW_F32 or FEW_Y_PANEL as
// above; no SwiGLU); ws: G (ceil(S / T) + 1) 256 floats, cnt: G words, zero before the first
// launch and left zero by every launch. Launches sharing ws and cnt must not overlap.
extern "C" __global__ void __launch_bounds__(512)
    x0ne_gemm_few_bal_bf16(const bf16_t* __restrict__ w, const bf16_t* __restrict__ x, void* __restrict__ y,
                           uint32_t rows, uint32_t cols, uint32_t n, uint32_t flags, uint32_t T, float* __restrict__ ws,
                           uint32_t* __restrict__ cnt) {
    __shared__ f32x4 stash[8 * 6 * 64];
    few_bal<8, 6, 8>(w, x, y, rows, cols, n, flags, T, ws, cnt, stash);
}

// ---- exact sums: Y[n][rows] = X[n][cols] W^T, every product summed in f64 ----
// The exact mode's prefill passes (the f64 sums of the exact GEMV, gemv.hip, over many rows):
// W [rows][cols] and X [n][cols] bf16 row-major, the products exact on the f64 matrix cores
// (v_mfma_f64_16x16x4_f64, W the A operand: 16 features x 4 k; X the B operand: 4 k x 16
// tokens), f64 accumulators, and Y = bf16(f32(sum)) or f32(sum): the exact GEMV's rounding.
//  - A wavefront owns 16 TF features x 16 TT tokens over all of K and works alone (no LDS, no
//    barrier): at 64 cycles per product on MI355X the matrix cores, not the loads, bound it, so
//    its operands come straight from memory (the L2), one step of 32 columns ahead.
//  - In a step lane l loads 16 bytes, columns k0 + 8 (l / 16) .. + 7, of W row 16 f + l % 16
//    and of X row 16 t + l % 16; product e (0..7) of the step feeds element e of both, so lane
//    group l / 16 supplies column k0 + 8 (l / 16) + e and each product sums 4 columns.
//  - Each output is summed in a fixed order (steps, then products within a step, then the
//    product's own 4 columns): the same bits from call to call, within f64 rounding of the
//    oracle's sequential sum.
//  - A wavefront's steps run one after the other (8 x 16 products of 64 cycles per step at
//    64 x 64 outputs), so a launch of few tiles (a short prompt) is latency-bound: with ks > 1
//    the steps are cut into ks equal runs, wavefront (tile, slice) writes its f64 partial sums
//    to ws[slice][token][feature], and x0ne_gemm_f64_reduce adds the slices in slice order.
// Wavefronts are numbered tokens fastest, then slices, so neighbouring wavefronts share W rows.
namespace {

typedef double f64x4 __attribute__((ext_vector_type(4)));

template <int TF, int TT>
__device__ __forceinline__ void gemm_f64(const bf16_t* __restrict__ w, const bf16_t* __restrict__ x,
                                         void* __restrict__ y, uint32_t rows, uint32_t cols, uint32_t n,
                                         uint32_t out_f32, uint32_t ks, double* __restrict__ ws) {
    const uint32_t lane = threadIdx.x & 63, V = blockDim.x >> 6;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t tiles_t = (n + 16 * TT - 1) / (16 * TT), tiles_f = (rows + 16 * TF - 1) / (16 * TF);
    const uint32_t id = blockIdx.x * V + wave;
    if (cols % 8 != 0 || out_f32 > 1 || ks == 0 || (ks > 1 && ws == nullptr) ||
        (uint64_t)id >= (uint64_t)tiles_f * tiles_t * ks)
        return;  // wavefront-uniform; no barrier
    const uint32_t tile = id / (tiles_t * ks) * tiles_t + id % tiles_t, slice = id / tiles_t % ks;
    const uint32_t ft = tile / tiles_t, tt = tile % tiles_t, r = lane & 15, q = lane >> 4;
    const auto wr = rsrc(w, (uint64_t)rows * cols * 2);
    const auto xr = rsrc(x, (uint64_t)n * cols * 2);
    f64x4 acc[TF][TT];
#pragma unroll
    for (int f = 0; f < TF; ++f)
#pragma unroll
        for (int t = 0; t < TT; ++t) acc[f][t] = f64x4{0.0, 0.0, 0.0, 0.0};
    uint4 a[2][TF], b[2][TT];
    const uint32_t all = (cols + 31) / 32, s_lo = all * slice / ks, steps = all * (slice + 1) / ks;
    auto load = [&](int buf, uint32_t s) {
        const uint32_t k = 32 * s + 8 * q;
        const bool in = s < steps && k < cols;  // a K tail: pieces past the row read zeros
#pragma unroll
        for (int f = 0; f < TF; ++f) {
            const uint32_t row = 16 * (TF * ft + f) + r;
            a[buf][f] = bload<>(wr, in && row < rows ? (row * cols + k) * 2 : OFF_NONE);
        }
#pragma unroll
        for (int t = 0; t < TT; ++t) {
            const uint32_t tok = 16 * (TT * tt + t) + r;
            b[buf][t] = bload<>(xr, in && tok < n ? (tok * cols + k) * 2 : OFF_NONE);
        }
    };
    auto elem = [](const uint4& v, int e) -> double {
        const uint32_t u = e < 2 ? v.x : e < 4 ? v.y : e < 6 ? v.z : v.w;
        return (double)((e & 1) ? bf_hi(u) : bf_lo(u));
    };
    auto step = [&](int buf) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            double av[TF], bv[TT];
#pragma unroll
            for (int f = 0; f < TF; ++f) av[f] = elem(a[buf][f], e);
#pragma unroll
            for (int t = 0; t < TT; ++t) bv[t] = elem(b[buf][t], e);
#pragma unroll
            for (int f = 0; f < TF; ++f)
#pragma unroll
                for (int t = 0; t < TT; ++t) acc[f][t] = __builtin_amdgcn_mfma_f64_16x16x4f64(av[f], bv[t], acc[f][t], 0, 0, 0);
        }
    };
    // Steps in pairs, so each register set is named statically.
    load(0, s_lo);
    for (uint32_t s = s_lo; s < steps; s += 2) {
        load(1, s + 1);
        step(0);
        if (s + 1 >= steps) break;  // wavefront-uniform
        load(0, s + 2);
        step(1);
    }
    // acc[f][t][i]: feature 16 (TF ft + f) + l / 16 + 4 i, token 16 (TT tt + t) + l % 16 (the
    // f64 product's result rows interleave over the lane groups).
#pragma unroll
    for (int f = 0; f < TF; ++f)
#pragma unroll
        for (int t = 0; t < TT; ++t) {
            const uint32_t tok = 16 * (TT * tt + t) + r;
            if (tok >= n) continue;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t feat = 16 * (TF * ft + f) + q + 4 * i;
                if (feat >= rows) continue;
                if (ks > 1) {
                    ws[((size_t)slice * n + tok) * rows + feat] = acc[f][t][i];
                    continue;
                }
                const float v = (float)acc[f][t][i];
                if (out_f32)
                    static_cast<float*>(y)[(size_t)tok * rows + feat] = v;
                else
                    static_cast<bf16_t*>(y)[(size_t)tok * rows + feat] = f2bf(v);
            }
        }
}

}  // namespace

// x0ne_gemm_f64_t{TT}_bf16: grid ceil(ceil(rows / 64) ceil(n / (16 TT)) ks / V), block 64 V
// threads (any V); cols a multiple of 8; W and X below 4 GiB - 16 bytes; out_f32 0 (bf16 Y) or
// 1 (f32 Y); ks 1 (Y written) or more (the partial sums into ws: [ks][n][rows] f64, then
// x0ne_gemm_f64_reduce).
#define X0NE_GEMM_F64(NAME, TT)                                                                                   \
    extern "C" __global__ void __launch_bounds__(256)                                                              \
        NAME(const bf16_t* __restrict__ w, const bf16_t* __restrict__ x, void* __restrict__ y, uint32_t rows,      \
             uint32_t cols, uint32_t n, uint32_t out_f32, uint32_t ks, double* __restrict__ ws) {                 \
        gemm_f64<4, TT>(w, x, y, rows, cols, n, out_f32, ks, ws);                                                  \
    }
X0NE_GEMM_F64(x0ne_gemm_f64_t1_bf16, 1)
X0NE_GEMM_F64(x0ne_gemm_f64_t2_bf16, 2)
X0NE_GEMM_F64(x0ne_gemm_f64_t4_bf16, 4)

// ---- exact sums for a few rows: 4-token quads ----
// The same product for n <= 32 rows of X on v_mfma_f64_4x4x4f64, which computes 4 blocks b of
// D[4][4] += A[4][4] B[4][4] with lane l = 16 k + 4 b + x holding A_b[x][k], B_b[k][x] and
// D_b[l / 16][x] (about 18 cycles per product against 64 for the 16x16x4 product, the same f64
// rate): A is W as in gemm_f64 (lane l loads row 16 f + l % 16, columns k0 + 8 (l / 16) ..), B
// the quad's 4 tokens (lane l loads token 4 t + l % 4, the same columns), so a wavefront covers
// 16 TF features x 4 TQ tokens without padding 20 rows to 32. D of lane l: feature
// 16 f + 4 ((l % 16) / 4) + l / 16, token 4 t + l % 4.
namespace {

template <int TF, int TQ>
__device__ __forceinline__ void gemm_f64_quads(const bf16_t* __restrict__ w, const bf16_t* __restrict__ x,
                                               void* __restrict__ y, uint32_t rows, uint32_t cols, uint32_t n,
                                               uint32_t out_f32, uint32_t ks, double* __restrict__ ws) {
    const uint32_t lane = threadIdx.x & 63, V = blockDim.x >> 6;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t tiles_f = (rows + 16 * TF - 1) / (16 * TF);
    const uint32_t id = blockIdx.x * V + wave;
    if (cols % 8 != 0 || out_f32 > 1 || ks == 0 || (ks > 1 && ws == nullptr) || n > 4u * TQ ||
        (uint64_t)id >= (uint64_t)tiles_f * ks)
        return;  // wavefront-uniform; no barrier
    const uint32_t ft = id / ks, slice = id % ks;
    const uint32_t r = lane & 15, q = lane >> 4, xq = lane & 3;
    const auto wr = rsrc(w, (uint64_t)rows * cols * 2);
    const auto xr = rsrc(x, (uint64_t)n * cols * 2);
    double acc[TF][TQ];
#pragma unroll
    for (int f = 0; f < TF; ++f)
#pragma unroll
        for (int t = 0; t < TQ; ++t) acc[f][t] = 0.0;
    uint4 a[2][TF], b[2][TQ];
    const uint32_t all = (cols + 31) / 32, s_lo = all * slice / ks, steps = all * (slice + 1) / ks;
    auto load = [&](int buf, uint32_t s) {
        const uint32_t k = 32 * s + 8 * q;
        const bool in = s < steps && k < cols;
#pragma unroll
        for (int f = 0; f < TF; ++f) {
            const uint32_t row = 16 * (TF * ft + f) + r;
            a[buf][f] = bload<>(wr, in && row < rows ? (row * cols + k) * 2 : OFF_NONE);
        }
#pragma unroll
        for (int t = 0; t < TQ; ++t) {
            const uint32_t tok = 4 * t + xq;
            b[buf][t] = bload<>(xr, in && tok < n ? (tok * cols + k) * 2 : OFF_NONE);
        }
    };
    auto elem = [](const uint4& v, int e) -> double {
        const uint32_t u = e < 2 ? v.x : e < 4 ? v.y : e < 6 ? v.z : v.w;
        return (double)((e & 1) ? bf_hi(u) : bf_lo(u));
    };
    auto step = [&](int buf) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            double av[TF], bv[TQ];
#pragma unroll
            for (int f = 0; f < TF; ++f) av[f] = elem(a[buf][f], e);
#pragma unroll
            for (int t = 0; t < TQ; ++t) bv[t] = elem(b[buf][t], e);
#pragma unroll
            for (int f = 0; f < TF; ++f)
#pragma unroll
                for (int t = 0; t < TQ; ++t) acc[f][t] = __builtin_amdgcn_mfma_f64_4x4x4f64(av[f], bv[t], acc[f][t], 0, 0, 0);
        }
    };
    load(0, s_lo);
    for (uint32_t s = s_lo; s < steps; s += 2) {
        load(1, s + 1);
        step(0);
        if (s + 1 >= steps) break;  // wavefront-uniform
        load(0, s + 2);
        step(1);
    }
#pragma unroll
    for (int f = 0; f < TF; ++f)
#pragma unroll
        for (int t = 0; t < TQ; ++t) {
            const uint32_t tok = 4 * t + xq, feat = 16 * (TF * ft + f) + 4 * (r / 4) + q;
            if (tok >= n || feat >= rows) continue;
            if (ks > 1) {
                ws[((size_t)slice * n + tok) * rows + feat] = acc[f][t];
                continue;
            }
            const float v = (float)acc[f][t];
            if (out_f32)
                static_cast<float*>(y)[(size_t)tok * rows + feat] = v;
            else
                static_cast<bf16_t*>(y)[(size_t)tok * rows + feat] = f2bf(v);
        }
}

}  // namespace

// x0ne_gemm_f64_q{TQ}_bf16: x0ne_gemm_f64_t*_bf16's arguments for 1 <= n <= 4 TQ rows; grid
// ceil(ceil(rows / 64) ks / V), block 64 V threads (any V).
#define X0NE_GEMM_F64_Q(TQ)                                                                                       \
    extern "C" __global__ void __launch_bounds__(256) x0ne_gemm_f64_q##TQ##_bf16(                                 \
        const bf16_t* __restrict__ w, const bf16_t* __restrict__ x, void* __restrict__ y, uint32_t rows,          \
        uint32_t cols, uint32_t n, uint32_t out_f32, uint32_t ks, double* __restrict__ ws) {                      \
        gemm_f64_quads<4, TQ>(w, x, y, rows, cols, n, out_f32, ks, ws);                                            \
    }
X0NE_GEMM_F64_Q(1)
X0NE_GEMM_F64_Q(2)
X0NE_GEMM_F64_Q(3)
X0NE_GEMM_F64_Q(4)
X0NE_GEMM_F64_Q(5)
X0NE_GEMM_F64_Q(6)
X0NE_GEMM_F64_Q(7)
X0NE_GEMM_F64_Q(8)

// x0ne_gemm_f64_reduce: y[t][f] = the f32 (out_f32 1) or bf16 of the f32 of sum over slices 0 ..
// ks - 1, in that order, of ws[slice][t][f] (f64); grid ceil(n rows / 256), block 256.
extern "C" __global__ void __launch_bounds__(256)
    x0ne_gemm_f64_reduce(const double* __restrict__ ws, void* __restrict__ y, uint32_t rows, uint32_t n, uint32_t ks,
                         uint32_t out_f32) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x, total = (uint64_t)rows * n;
    if (i >= total || ks == 0 || out_f32 > 1) return;
    double sum = ws[i];
    for (uint32_t s = 1; s < ks; ++s) sum += ws[(uint64_t)s * total + i];
    if (out_f32)
        static_cast<float*>(y)[i] = (float)sum;
    else
        static_cast<bf16_t*>(y)[i] = f2bf((float)sum);
}

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

// ---- many rows: Y[n][rows] = X[n][cols] W^T, compute-bound, on the matrix cores ----
// The prefill passes' projections (2048 rows of X at Qwen3 widths: 0.07-0.41 TFLOP a launch).
// A block of NWF x NWT wavefronts computes a tile of BF = NWF WF output features (W rows) by
// BT = NWT WT tokens (X rows); wavefront (wf, wt) holds WF x WT of it in f32 accumulators as
// (WF / 16) x (WT / 16) products v_mfma_f32_16x16x32_bf16 with W as the A operand (16 features x
// 32 k) and X as the B operand (16 tokens x 32 k), so each lane ends with 4 consecutive
// features of one token and stores them as one 8-byte (bf16) or 16-byte (f32) write.
//  - K passes in stages of KS x 32 columns through a ring of STAGES buffers in LDS, filled by
//    direct buffer-to-LDS loads (buffer_load_dwordx4 ... lds: no registers, no VALU) issued
//    STAGES stages ahead. One barrier per stage.
//  - The operands of each 32-column step are read from LDS into a second register set while the
//    products of the step before run, the reads interleaved with the products (one read, then
//    products), so the matrix cores do not wait for LDS. Measured on MI355X (Qwen3-8B shapes,
//    2048 rows): 0.4-0.47 of bf16 peak against 0.36-0.43 without the overlap.
//  - LDS holds operand fragments in the order the products read them: a fragment is 16 rows x
//    32 k (1 KiB), lane l's 16 bytes (row l % 16, k 8 (l / 16) .. + 7) at byte 16 l, so each
//    ds_read_b128 reads 1 KiB contiguous in lane order (no bank conflicts).
//  - Operands in 16-row panels (device.h: [rows / 16][cols / 8][16][8]) hold a fragment as
//    1 KiB contiguous in exactly that order, so one load instruction fetches it whole. Row-major
//    operands (Gpu::gemm's) give each load 16 rows x 64 bytes: measured on MI355X, a tile's
//    loads stream from the L2 at 25 TB/s (all CUs) from panels against 9.5 TB/s row-major, so
//    the engine's prefill passes keep W and X in panels.
//  - A load past the matrix (a token past n, a feature past rows, k past cols) is a buffer load
//    at an offset past the buffer: zeros, no memory touched.
//  - Tiles in launch order go round the 8 XCDs (each with its own L2): the launch's blocks are
//    renumbered so each XCD takes a contiguous run of tiles, and runs are ordered TILE_GROUP
//    feature tiles wide, tokens fastest, so the blocks an XCD holds at once share their W and X
//    pieces in its L2.
// Each output is summed over k by one wavefront in a fixed order: bit-reproducible, and the
// same bits whatever the operands' layout.
namespace {

constexpr int TILE_GROUP = 4;  // feature tiles side by side in one run of tiles
constexpr uint32_t TILE_F32 = 1, TILE_W_PANEL = 2, TILE_X_PANEL = 4;

template <int WF, int WT, int NWF, int NWT, int STAGES, int KS>
struct TileCfg {
    static constexpr int NW = NWF * NWT;
    static constexpr int BF = NWF * WF, BT = NWT * WT;  // block tile: features x tokens
    static constexpr int WFR = BF / 16, XFR = BT / 16;   // fragments per 32-column step
    static constexpr int FR = WFR + XFR;
    static constexpr int LOADS = KS * FR / NW;          // load instructions per wavefront per stage
    static constexpr int BYTES = KS * FR * 1024;        // one stage (KS steps) in LDS
    static constexpr int RA = WF / 16, RB = WT / 16;    // fragments a wavefront reads per step
    static_assert((KS * FR) % NW == 0 && WF % 16 == 0 && WT % 16 == 0, "tile shape");
    static_assert(STAGES >= 2 && STAGES * BYTES <= 160 * 1024, "LDS");
};

typedef int i32x4 __attribute__((ext_vector_type(4)));

// A raw buffer descriptor (the 48-bit base, stride 0, `bytes` records, word 3 of
// make_buffer_rsrc) as four scalar words, for the load below.
__device__ __forceinline__ i32x4 rsrc_words(const void* base, uint64_t bytes) {
    const uint64_t a = (uint64_t)base;
    const uint32_t n = bytes > OFF_NONE ? OFF_NONE : (uint32_t)bytes;
    return i32x4{(int)(uint32_t)a, (int)((uint32_t)(a >> 32) & 0xFFFFu), (int)n, (int)RSRC_WORD3};
}

// One direct buffer-to-LDS load (buffer_load_dwordx4 ... lds): lane l's 16 bytes at byte offset
// `off` of the buffer (zeros past it) land at LDS byte lds + 16 l. Written as an instruction of
// its own so the compiler adds no wait of its own for it: the loop below counts these loads and
// waits for them itself. M0 holds the LDS address; nothing else in these kernels uses M0.
__device__ __forceinline__ void load_lds16(const i32x4& r, uint32_t lds, uint32_t off) {
    // The descriptor and the LDS address are wavefront-uniform; read from lane 0 so they are
    // scalar registers whatever the compiler concluded.
    const i32x4 u = {__builtin_amdgcn_readfirstlane(r[0]), __builtin_amdgcn_readfirstlane(r[1]),
                     __builtin_amdgcn_readfirstlane(r[2]), __builtin_amdgcn_readfirstlane(r[3])};
    asm volatile("s_mov_b32 m0, %1\n\tbuffer_load_dwordx4 %0, %2, 0 offen lds" ::"v"(off),
                 "s"(__builtin_amdgcn_readfirstlane(lds)), "s"(u)
                 : "memory");
}

__device__ __forceinline__ uint32_t lds_addr(const uint8_t* p) {
    return __builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)(p));
}

// s_waitcnt lgkmcnt(0) (vmcnt and expcnt at their maxima) through the compiler's builtin, so its
// own wait bookkeeping knows the LDS reads are done.
constexpr int WAIT_LGKM0 = 0xC07F;

template <int WF, int WT, int NWF, int NWT, int STAGES, int KS>
__device__ __forceinline__ void gemm_tiles(const bf16_t* __restrict__ w, const bf16_t* __restrict__ x,
                                           void* __restrict__ y, uint32_t rows, uint32_t cols, uint32_t n,
                                           uint32_t flags, uint8_t* lds) {
    using C = TileCfg<WF, WT, NWF, NWT, STAGES, KS>;
    const uint32_t tiles_f = (rows + C::BF - 1) / C::BF, tiles_t = (n + C::BT - 1) / C::BT;
    const uint32_t tiles = tiles_f * tiles_t;
    // Launch id -> tile: ids alternate over the 8 XCDs, so id b runs on XCD b % 8; the XCD's
    // ids b % 8, b % 8 + 8, .. take the run of tiles (b % 8) (tiles / 8) + b / 8.
    const uint32_t b = blockIdx.x;
    const uint32_t seq = tiles % 8 == 0 ? (b & 7) * (tiles >> 3) + (b >> 3) : b;
    const uint32_t group = seq / (TILE_GROUP * tiles_t), in_group = seq % (TILE_GROUP * tiles_t);
    const uint32_t width = min((uint32_t)TILE_GROUP, tiles_f - group * TILE_GROUP);
    const uint32_t f0 = (group * TILE_GROUP + in_group % width) * C::BF, t0 = in_group / width * C::BT;

    const uint32_t lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t wf = wave % NWF, wt = wave / NWF;
    const bool w_panel = flags & TILE_W_PANEL, x_panel = flags & TILE_X_PANEL;
    // Panels hold whole groups of 16 rows.
    const i32x4 wr = rsrc_words(w, (uint64_t)(w_panel ? (rows + 15) / 16 * 16 : rows) * cols * 2);
    const i32x4 xr = rsrc_words(x, (uint64_t)(x_panel ? (n + 15) / 16 * 16 : n) * cols * 2);
    const uint32_t steps = (cols + 31) / 32, stages = (steps + KS - 1) / KS, c8 = cols / 8;

    // This wavefront's loads of a stage: fragment f = wave + NW q of the stage's KS x FR (step
    // kk = f / FR, fragment f % FR, W fragments first), lane l fetching row 16 g + l % 16,
    // columns 32 (KS s + kk) + 8 (l / 16) .. + 7 of its operand: byte base[q] + step[q] KS s of
    // the buffer while those columns exist and the row (panel: its group of 16) does.
    uint32_t base[C::LOADS], step[C::LOADS], chunk0[C::LOADS];
    bool row_in[C::LOADS];
#pragma unroll
    for (int q = 0; q < C::LOADS; ++q) {
        const int f = (int)wave + C::NW * q, kk = f / C::FR, fr = f % C::FR;
        const bool is_w = fr < C::WFR;
        const uint32_t g16 = ((is_w ? f0 : t0) >> 4) + (uint32_t)(is_w ? fr : fr - C::WFR);
        const uint32_t row = 16 * g16 + (lane & 15);
        const bool panel = is_w ? w_panel : x_panel;
        row_in[q] = (panel ? 16 * g16 : row) < (is_w ? rows : n);
        step[q] = panel ? 1024 : 64;
        base[q] = (panel ? g16 * c8 * 256 + lane * 16 : row * cols * 2 + (lane >> 4) * 16) + step[q] * kk;
        chunk0[q] = 4 * kk + (lane >> 4);
    }
    auto issue = [&](uint32_t s) {
        uint8_t* dst = lds + (s % STAGES) * C::BYTES;
#pragma unroll
        for (int q = 0; q < C::LOADS; ++q) {
            const int f = (int)wave + C::NW * q;
            const bool is_w = f % C::FR < C::WFR;
            const bool in = row_in[q] && 4 * KS * s + chunk0[q] < c8;
            load_lds16(is_w ? wr : xr, lds_addr(dst + f * 1024), in ? base[q] + step[q] * KS * s : OFF_NONE);
        }
    };

    f32x4 acc[C::RA][C::RB];
#pragma unroll
    for (int i = 0; i < C::RA; ++i)
#pragma unroll
        for (int j = 0; j < C::RB; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    uint4 a0[C::RA], b0[C::RB], a1[C::RA], b1[C::RB];
    auto read = [&](uint32_t s, int kk, uint4 (&a)[C::RA], uint4 (&bx)[C::RB]) {
        const uint8_t* src = lds + (s % STAGES) * C::BYTES + kk * C::FR * 1024;
#pragma unroll
        for (int i = 0; i < C::RA; ++i)
            a[i] = *reinterpret_cast<const uint4*>(src + (wf * C::RA + i) * 1024 + lane * 16);
#pragma unroll
        for (int j = 0; j < C::RB; ++j)
            bx[j] = *reinterpret_cast<const uint4*>(src + (C::WFR + wt * C::RB + j) * 1024 + lane * 16);
    };
    // The products of one stage, with the reads issued just before them interleaved: one LDS
    // read, then its share of the products.
    auto compute = [&](const uint4 (&a)[C::RA], const uint4 (&bx)[C::RB]) {
#pragma unroll
        for (int i = 0; i < C::RA; ++i)
#pragma unroll
            for (int j = 0; j < C::RB; ++j) acc[i][j] = mfma(a[i], bx[j], acc[i][j]);
        constexpr int R = C::RA + C::RB, M = C::RA * C::RB;
#pragma unroll
        for (int i = 0; i < R; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);      // one LDS read
            __builtin_amdgcn_sched_group_barrier(0x008, M / R, 0);  // then products
        }
        if (M % R) __builtin_amdgcn_sched_group_barrier(0x008, M % R, 0);
    };

    // Prologue: stages 0 .. STAGES - 1 in flight, stage 0 complete (this wavefront's loads: at
    // most the later stages' in flight; then the barrier: every wavefront's), its first step's
    // operands read.
#pragma unroll
    for (int p = 0; p < STAGES; ++p)
        if ((uint32_t)p < stages) issue(p);
    if (stages >= (uint32_t)STAGES) {
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(C::LOADS * (STAGES - 1)) : "memory");
    } else {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    asm volatile("s_barrier" ::: "memory");
    read(0, 0, a0, b0);
    // Step kk of stage s: its products run while the next step's operands are read. Before the
    // last step of stage s: stage s + 1 complete in this wavefront (at most min(stages - s - 2,
    // STAGES - 2) later stages' loads in flight) and its own reads of stage s done; the barrier:
    // the same in every wavefront, so stage s's slot is no longer read and takes stage
    // s + STAGES. The next step after the last one reads stage s's last step again (a harmless
    // read that keeps the reads unconditional). Stages go in pairs so each step's register set
    // is fixed at compile time.
    for (uint32_t s2 = 0; s2 < stages; s2 += 2) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t s = s2 + h;
            if (s >= stages) break;
#pragma unroll
            for (int kk = 0; kk < KS; ++kk) {
                uint32_t ns = s;
                int nk = kk + 1;
                if (kk == KS - 1) {
                    if (s + 1 < stages) {
                        if (stages - s - 2 >= (uint32_t)(STAGES - 2)) {
                            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(C::LOADS * (STAGES - 2)) : "memory");
                        } else {
                            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                        }
                    }
                    __builtin_amdgcn_s_waitcnt(WAIT_LGKM0);
                    asm volatile("s_barrier" ::: "memory");
                    if (s + STAGES < stages) issue(s + STAGES);
                    ns = s + 1 < stages ? s + 1 : s;
                    nk = s + 1 < stages ? 0 : kk;
                }
                if (((h * KS + kk) & 1) == 0) {
                    read(ns, nk, a1, b1);
                    compute(a0, b0);
                } else {
                    read(ns, nk, a0, b0);
                    compute(a1, b1);
                }
            }
        }
    }

    // acc[i][j][r]: feature f0 + WF wf + 16 i + 4 (lane / 16) + r, token t0 + WT wt + 16 j + lane % 16.
    const bool out_f32 = flags & TILE_F32;
#pragma unroll
    for (int j = 0; j < C::RB; ++j) {
        const uint32_t t = t0 + WT * wt + 16 * j + (lane & 15);
        if (t >= n) continue;
#pragma unroll
        for (int i = 0; i < C::RA; ++i) {
            const uint32_t f = f0 + WF * wf + 16 * i + 4 * (lane >> 4);
            if (f >= rows) continue;
            const f32x4 v = acc[i][j];
            const size_t o = (size_t)t * rows + f;
            if (out_f32) {
                *reinterpret_cast<f32x4*>(static_cast<float*>(y) + o) = v;
            } else {
                const uint32_t lo = (uint32_t)f2bf(v[0]) | ((uint32_t)f2bf(v[1]) << 16);
                const uint32_t hi = (uint32_t)f2bf(v[2]) | ((uint32_t)f2bf(v[3]) << 16);
                *reinterpret_cast<uint2*>(static_cast<bf16_t*>(y) + o) = make_uint2(lo, hi);
            }
        }
    }
}

}  // namespace

// Tiled GEMM kernels: grid ceil(rows / BF) ceil(n / BT), block 64 NWF NWT; rows a multiple of 4,
// cols of 8 (and rows of 16 with W in panels), W and X below 4 GiB - 16 bytes, Y 8-byte (bf16)
// or 16-byte (f32) aligned; flags TILE_F32 | TILE_W_PANEL | TILE_X_PANEL.
#define X0NE_TILES(NAME, WF, WT, NWF, NWT, STAGES, KS)                                                          \
    extern "C" __global__ void __launch_bounds__(64 * NWF * NWT)                                                      \
        NAME(const bf16_t* __restrict__ w, const bf16_t* __restrict__ x, void* __restrict__ y, uint32_t rows,         \
             uint32_t cols, uint32_t n, uint32_t flags) {                                                             \
        __shared__ __attribute__((aligned(1024))) uint8_t lds[STAGES * TileCfg<WF, WT, NWF, NWT, STAGES, KS>::BYTES]; \
        if (rows % 4 != 0 || cols % 8 != 0 || n == 0 || ((flags & TILE_W_PANEL) && rows % 16 != 0)) return;         \
        gemm_tiles<WF, WT, NWF, NWT, STAGES, KS>(w, x, y, rows, cols, n, flags, lds);                                 \
    }
// Block tiles from sweeps on MI355X over the Qwen3-8B prefill shapes at 2048 rows, operands in
// panels, all in four stages of 32 columns (64-column stages, two of them for 256 x 256 and three
// for 256 x 128, measured 3-10 % slower in the engine's prefill): 256 x 256 of 8 wavefronts
// (64 features x 128 tokens each; two per SIMD), 256 x 128 of 8 (64 x 64 each), and 128 x 128 of
// 4 (64 x 64 each; two blocks per CU).
X0NE_TILES(x0ne_gemm_tiles_256x256_bf16, 64, 128, 4, 2, 4, 1)
X0NE_TILES(x0ne_gemm_tiles_256x128_bf16, 64, 64, 4, 2, 4, 1)
X0NE_TILES(x0ne_gemm_tiles_128x128_bf16, 64, 64, 2, 2, 4, 1)

// ---- typed launchers of the tiled GEMM (called by the runtime) ----

#include "launch.h"

namespace {

struct TileKind {
    const void* fn;
    uint32_t bf, bt;    // block tile: features x tokens
    uint32_t threads;
};

TileKind tile_kind(int tile) {
    switch (tile) {
        case X0NE_TILE_256x256: return {(const void*)&x0ne_gemm_tiles_256x256_bf16, 256, 256, 512};
        case X0NE_TILE_256x128: return {(const void*)&x0ne_gemm_tiles_256x128_bf16, 256, 128, 512};
        case X0NE_TILE_128x128: return {(const void*)&x0ne_gemm_tiles_128x128_bf16, 128, 128, 256};
        default: return {nullptr, 0, 0, 0};
    }
}

}  // namespace

// The tile for a shape, from the MI355X sweeps at 2048 rows of X (operands in panels): the
// 256 x 256 tile while it gives at least 0.7 of a tile per CU (gate/up 24576 rows: 335-360 us;
// QKV 6144 rows: 98-106 us against 125 for 256 x 128), else 256 x 128 while that does (O and down,
// 4096 rows: 68 and 186 us against 99 and 278 for 256 x 256), else 128 x 128.
int x0ne_gemm_tile_pick(uint32_t rows, uint32_t cols, uint32_t n, uint32_t cus) {
    auto tiles = [&](uint32_t bf, uint32_t bt) { return (uint64_t)((rows + bf - 1) / bf) * ((n + bt - 1) / bt); };
    if (10 * tiles(256, 256) >= 7ull * cus) return X0NE_TILE_256x256;
    if (10 * tiles(256, 128) >= 7ull * cus) return X0NE_TILE_256x128;
    return X0NE_TILE_128x128;
}

hipError_t x0ne_launch_gemm_tiles(int tile, const void* w, const void* x, void* y, uint32_t rows, uint32_t cols,
                                  uint32_t n, uint32_t flags, hipStream_t s) {
    const TileKind k = tile_kind(tile);
    if (!k.fn || rows % 4 != 0 || cols % 8 != 0 || n == 0 || flags > 7 || ((flags & TILE_W_PANEL) && rows % 16 != 0))
        return hipErrorInvalidValue;
    const uint64_t blocks = (uint64_t)((rows + k.bf - 1) / k.bf) * ((n + k.bt - 1) / k.bt);
    if (blocks > 0x7FFFFFFFull) return hipErrorInvalidValue;
    void* args[] = {(void*)&w, (void*)&x, (void*)&y, (void*)&rows, (void*)&cols, (void*)&n, (void*)&flags};
    return x0ne_launch(k.fn, dim3((uint32_t)blocks), dim3(k.threads), args, 0, s);
}
