// GQA decode attention over the paged KV arena, for gfx950 (64-lane wavefronts).
//
// Semantics follow x0ne-core/kernels/cuda/attention.cu: the query at position pos[0] attends
// keys 0..pos[0] (ctx = min(pos + 1, max_ctx)); q head h reads kv head h / (q_heads / kv_heads);
// scores q.k / sqrt(128); softmax with the maximum subtracted; f32 accumulation. Split-K
// (attention.cu:161-251): keys in tiles at absolute positions, block (kh, y) takes tiles
// y, y + P, y + 2P, ... below ctx and writes a partial state (m, l, o[128]) per q head at
// state[(h * P + y) * 132]; the merge (attention.cu:253-280) combines slices 0..active-1 in that
// fixed order. The result depends on the inputs, ctx and P only.
//
// The layout and the work split are this build's own, shaped for CDNA:
//  - K and V planes are paged: [pages][kv_heads][16][128] bf16, page_table[pos / 16] the
//    physical page. A tile is 64 keys (4 pages); one wavefront takes a tile per step.
//  - Each 16-byte load of a wavefront covers 4 whole rows of one page (1 KiB contiguous). Lane
//    (r = lane / 16, b = lane % 16) holds dims 8b..8b+7 of rows 4i + r, i = 0..15.
//  - The partial dot products of a lane (16 rows x G heads) are summed over the 16 lanes of a row
//    by a transposing butterfly (xor 1, 2, 4, 8; each step halves the vector), so a lane ends
//    with whole scores without reducing every value separately.
//  - Scores and softmax weights go through LDS once per tile, so each lane runs the online
//    softmax for one key and the V accumulation for its own rows, with no further shuffles.
#include "device.h"

namespace {

// One step of the transposing butterfly: lanes b and b ^ 2^K exchange halves of an N-vector;
// the lane whose bit K is 0 keeps the lower half, its partner the upper.
template <int N, int K>
__device__ __forceinline__ void butterfly_step(float* a, uint32_t b) {
    constexpr int H = N >> 1;
    const bool bit = (b >> K) & 1u;
#pragma unroll
    for (int j = 0; j < H; ++j) {
        const float send = bit ? a[j] : a[j + H];
        const float keep = bit ? a[j + H] : a[j];
        a[j] = keep + __shfl_xor(send, 1 << K, 64);
    }
}

// Sum over the 16 lanes of a row, transposing: lane b (of a row) ends with values
// (N/16) * rev4(b) + e, e < N/16, of the original vector, in a[0..N/16).
template <int N>
__device__ __forceinline__ void butterfly16(float* a, uint32_t b) {
    butterfly_step<N, 0>(a, b);
    butterfly_step<N / 2, 1>(a, b);
    butterfly_step<N / 4, 2>(a, b);
    butterfly_step<N / 8, 3>(a, b);
}

__device__ __forceinline__ uint32_t rev4(uint32_t b) {
    return ((b & 1u) << 3) | ((b & 2u) << 1) | ((b & 4u) >> 1) | ((b & 8u) >> 3);
}

// One wavefront: the G q heads at `q` (G x 128 bf16, consecutive) over kv head kh, tiles
// t0, t0 + tstep, ... below ntiles. Leaves per head the running max m, the sum l (whole, every
// lane) and o = sum exp(s - m) v for dims 8b..8b+7 (summed over the 4 rows of a lane, valid in
// every lane). lds: 2 * G * 64 floats.
template <int G>
__device__ __forceinline__ void attend_wave(const bf16_t* __restrict__ q, const bf16_t* __restrict__ kc,
                                            const bf16_t* __restrict__ vc, const uint32_t* __restrict__ pages,
                                            uint32_t kh, uint32_t kv_heads, uint32_t ctx, uint32_t t0,
                                            uint32_t tstep, float scale, float* lds, float m[G], float l[G],
                                            float o[G][8]) {
    constexpr int HG = G < 4 ? G : 4;  // heads per score pass
    constexpr int PASSES = G / HG;
    float* s_lds = lds;           // [G][64] scores of the tile's keys
    float* p_lds = lds + G * 64;  // [G][64] their softmax weights
    const uint32_t lane = threadIdx.x & 63, r = lane >> 4, b = lane & 15;
    const uint32_t ntiles = (ctx + X0NE_SPLIT_TILE - 1) / X0NE_SPLIT_TILE;

    float lsum[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        m[g] = -INFINITY;
        lsum[g] = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) o[g][j] = 0.f;
    }

    for (uint32_t t = t0; t < ntiles; t += tstep) {
        const uint32_t base = t * X0NE_SPLIT_TILE;
        // Rows 4i + r of the tile: page base/16 + i/4, slot 4 (i % 4) + r. A page is looked up
        // only when its first key is below ctx (the table holds ceil(ctx / 16) pages at least).
        uint32_t pg[4];
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
            const uint32_t first = base + X0NE_PAGE * ii;
            pg[ii] = first < ctx ? pages[first / X0NE_PAGE] : 0u;
        }
        uint32_t off[16];
        bool valid[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            valid[i] = base + 4 * i + r < ctx;
            off[i] = ((pg[i >> 2] * kv_heads + kh) * X0NE_PAGE + 4 * (i & 3) + r) * X0NE_HEAD_DIM + 8 * b;
        }
        uint4 kv[16];
#pragma unroll
        for (int i = 0; i < 16; ++i)
            kv[i] = valid[i] ? *reinterpret_cast<const uint4*>(kc + off[i]) : make_uint4(0, 0, 0, 0);

#pragma unroll
        for (int pass = 0; pass < PASSES; ++pass) {
            float qf[HG][8];
#pragma unroll
            for (int g = 0; g < HG; ++g) {
                const uint4 u = *reinterpret_cast<const uint4*>(q + (pass * HG + g) * X0NE_HEAD_DIM + 8 * b);
                qf[g][0] = bf_lo(u.x); qf[g][1] = bf_hi(u.x);
                qf[g][2] = bf_lo(u.y); qf[g][3] = bf_hi(u.y);
                qf[g][4] = bf_lo(u.z); qf[g][5] = bf_hi(u.z);
                qf[g][6] = bf_lo(u.w); qf[g][7] = bf_hi(u.w);
            }
            float part[16 * HG];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float k0 = bf_lo(kv[i].x), k1 = bf_hi(kv[i].x), k2 = bf_lo(kv[i].y), k3 = bf_hi(kv[i].y);
                const float k4 = bf_lo(kv[i].z), k5 = bf_hi(kv[i].z), k6 = bf_lo(kv[i].w), k7 = bf_hi(kv[i].w);
#pragma unroll
                for (int g = 0; g < HG; ++g) {
                    float d = qf[g][0] * k0;
                    d = fmaf(qf[g][1], k1, d);
                    d = fmaf(qf[g][2], k2, d);
                    d = fmaf(qf[g][3], k3, d);
                    d = fmaf(qf[g][4], k4, d);
                    d = fmaf(qf[g][5], k5, d);
                    d = fmaf(qf[g][6], k6, d);
                    d = fmaf(qf[g][7], k7, d);
                    part[i * HG + g] = d;
                }
            }
            butterfly16<16 * HG>(part, b);
            // Lane holds values HG * rev4(b) + e: row slot i = v / HG, head g = v % HG.
            constexpr int VPL = HG;
#pragma unroll
            for (int e = 0; e < VPL; ++e) {
                const uint32_t v = VPL * rev4(b) + e;
                const uint32_t i = v / HG, g = v % HG;
                const uint32_t row = 4 * i + r;
                const float s = (base + row < ctx) ? part[e] * scale : -INFINITY;
                s_lds[(pass * HG + g) * 64 + row] = s;
            }
        }
        __syncthreads();

        // Online softmax, lane = key of the tile.
        float alpha[G];
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float s = s_lds[g * 64 + lane];
            const float mn = fmaxf(m[g], wave_max(s));  // key `base` is below ctx: mn is finite
            alpha[g] = expf(m[g] - mn);
            const float p = expf(s - mn);
            lsum[g] = lsum[g] * alpha[g] + p;
            m[g] = mn;
            p_lds[g * 64 + lane] = p;
        }
        __syncthreads();

        // V rows 4i + r, dims 8b..8b+7; rows past ctx are zero (their weight is 0, and a zero
        // keeps a value that is not a number out of the sum).
        uint4 vv[16];
#pragma unroll
        for (int i = 0; i < 16; ++i)
            vv[i] = valid[i] ? *reinterpret_cast<const uint4*>(vc + off[i]) : make_uint4(0, 0, 0, 0);
#pragma unroll
        for (int g = 0; g < G; ++g) {
#pragma unroll
            for (int j = 0; j < 8; ++j) o[g][j] *= alpha[g];
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float v0 = bf_lo(vv[i].x), v1 = bf_hi(vv[i].x), v2 = bf_lo(vv[i].y), v3 = bf_hi(vv[i].y);
            const float v4 = bf_lo(vv[i].z), v5 = bf_hi(vv[i].z), v6 = bf_lo(vv[i].w), v7 = bf_hi(vv[i].w);
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const float p = p_lds[g * 64 + 4 * i + r];
                o[g][0] = fmaf(p, v0, o[g][0]);
                o[g][1] = fmaf(p, v1, o[g][1]);
                o[g][2] = fmaf(p, v2, o[g][2]);
                o[g][3] = fmaf(p, v3, o[g][3]);
                o[g][4] = fmaf(p, v4, o[g][4]);
                o[g][5] = fmaf(p, v5, o[g][5]);
                o[g][6] = fmaf(p, v6, o[g][6]);
                o[g][7] = fmaf(p, v7, o[g][7]);
            }
        }
        __syncthreads();  // the next tile rewrites s_lds and p_lds
    }
    // Whole sums: l over the 64 keys' lanes, o over the 4 rows of a lane (lanes b, b+16, ...).
#pragma unroll
    for (int g = 0; g < G; ++g) {
        l[g] = wave_sum(lsum[g]);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            float x = o[g][j];
            x += __shfl_xor(x, 16, 64);
            x += __shfl_xor(x, 32, 64);
            o[g][j] = x;
        }
    }
}

// The state of one (q head, slice): [0] m, [1] l, [4..131] o. Lanes 0..15 write o.
template <int G>
__device__ __forceinline__ void write_states(float* __restrict__ state, uint32_t h0, uint32_t splits, uint32_t y,
                                             const float m[G], const float l[G], const float o[G][8]) {
    const uint32_t lane = threadIdx.x & 63;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        float* st = state + ((size_t)(h0 + g) * splits + y) * X0NE_SPLIT_STATE;
        if (lane < 16) {
            float4* d = reinterpret_cast<float4*>(st + 4 + 8 * lane);
            d[0] = make_float4(o[g][0], o[g][1], o[g][2], o[g][3]);
            d[1] = make_float4(o[g][4], o[g][5], o[g][6], o[g][7]);
        }
        if (lane == 0) {
            st[0] = m[g];
            st[1] = l[g];
        }
    }
}

__device__ __forceinline__ float ld_agent(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Merge of one q head's slices 0..active-1 in that order (FlashInfer's: M = max m_y,
// f_y = exp(m_y - M), l = sum l_y f_y, o = sum o_y f_y; one rounding, of o / l). One wavefront;
// lane d owns dims d and d + 64. lds: at least `active` floats. Every active slice saw a key,
// so each m is finite. States are read with agent-coherent loads: other workgroups wrote them.
__device__ __forceinline__ void merge_head(const float* __restrict__ s, bf16_t* __restrict__ out_h,
                                           uint32_t active, float* lds) {
    const uint32_t lane = threadIdx.x & 63;
    float mx = -INFINITY;
    for (uint32_t y = 0; y < active; ++y)
        mx = fmaxf(mx, ld_agent(s + (size_t)y * X0NE_SPLIT_STATE));
    for (uint32_t y = lane; y < active; y += 64)
        lds[y] = expf(ld_agent(s + (size_t)y * X0NE_SPLIT_STATE) - mx);
    __syncthreads();
    float l = 0.f, o0 = 0.f, o1 = 0.f;
    for (uint32_t y = 0; y < active; ++y) {
        const float* st = s + (size_t)y * X0NE_SPLIT_STATE;
        const float f = lds[y];
        l += ld_agent(st + 1) * f;
        o0 += ld_agent(st + 4 + lane) * f;
        o1 += ld_agent(st + 4 + 64 + lane) * f;
    }
    out_h[lane] = f2bf(o0 / l);
    out_h[lane + 64] = f2bf(o1 / l);
    __syncthreads();
}

constexpr int MERGE_LDS = 1024;  // most slices a merge takes (P is capped at this)

template <int G>
__device__ __forceinline__ void split_group(const bf16_t* __restrict__ q, const bf16_t* __restrict__ kc,
                                            const bf16_t* __restrict__ vc, const uint32_t* __restrict__ pages,
                                            float* __restrict__ state, uint32_t* __restrict__ counter,
                                            bf16_t* __restrict__ out, const uint32_t* __restrict__ pos,
                                            uint32_t kv_heads, uint32_t max_ctx, uint32_t splits, float scale) {
    __shared__ float lds[2 * G * 64 > MERGE_LDS ? 2 * G * 64 : MERGE_LDS];
    __shared__ uint32_t last;
    const uint32_t kh = blockIdx.x, y = blockIdx.y;
    const uint32_t ctx = min(pos[0] + 1u, max_ctx);
    const uint32_t ntiles = (ctx + X0NE_SPLIT_TILE - 1) / X0NE_SPLIT_TILE;
    if (y >= ntiles) return;  // block-uniform
    float m[G], l[G], o[G][8];
    attend_wave<G>(q + (size_t)kh * G * X0NE_HEAD_DIM, kc, vc, pages, kh, kv_heads, ctx, y, splits, scale, lds, m,
                   l, o);
    write_states<G>(state, kh * G, splits, y, m, l, o);
    if (counter == nullptr) return;  // grid-uniform: the merge kernel follows
    const uint32_t active = min(splits, ntiles);
    __threadfence();  // this block's states, visible to the block that merges
    __syncthreads();
    if (threadIdx.x == 0) last = atomicAdd(counter + kh, 1u) == active - 1;
    __syncthreads();
    if (!last) return;  // block-uniform
    __threadfence();
#pragma unroll 1
    for (int g = 0; g < G; ++g) {
        const uint32_t h = kh * G + g;
        merge_head(state + (size_t)h * splits * X0NE_SPLIT_STATE, out + (size_t)h * X0NE_HEAD_DIM, active, lds);
    }
    if (threadIdx.x == 0) counter[kh] = 0;  // ready for the next step
}

}  // namespace

// Split-K, one block (one wavefront) per (kv head, slice) serving the G q heads of the group:
// grid (kv_heads, P), block 64. With counter != 0 the last block of a kv head to finish merges
// its G heads into out (same code and order as x0ne_attention_merge_bf16, so the same bits)
// and sets counter[kh] back to 0; with counter == 0, out is unused and the merge kernel follows.
#define X0NE_SPLIT_GROUP(G)                                                                                        \
    extern "C" __global__ void __launch_bounds__(64) x0ne_attention_decode_split_g##G##_bf16(                     \
        const bf16_t* __restrict__ q, const bf16_t* __restrict__ k_cache, const bf16_t* __restrict__ v_cache,    \
        const uint32_t* __restrict__ pages, float* __restrict__ state, uint32_t* __restrict__ counter,           \
        bf16_t* __restrict__ out, const uint32_t* __restrict__ pos, uint32_t q_heads, uint32_t kv_heads,         \
        uint32_t max_ctx, uint32_t splits, float scale) {                                                         \
        (void)q_heads;                                                                                             \
        split_group<G>(q, k_cache, v_cache, pages, state, counter, out, pos, kv_heads, max_ctx, splits, scale);    \
    }
X0NE_SPLIT_GROUP(1)
X0NE_SPLIT_GROUP(2)
X0NE_SPLIT_GROUP(4)
X0NE_SPLIT_GROUP(8)

// Split-K, one block per (q head, slice), for group sizes without a grouped kernel:
// grid (q_heads, P), block 64. The merge kernel follows.
extern "C" __global__ void __launch_bounds__(64)
    x0ne_attention_decode_split_bf16(const bf16_t* __restrict__ q, const bf16_t* __restrict__ k_cache,
                                     const bf16_t* __restrict__ v_cache, const uint32_t* __restrict__ pages,
                                     float* __restrict__ state, const uint32_t* __restrict__ pos, uint32_t q_heads,
                                     uint32_t kv_heads, uint32_t max_ctx, uint32_t splits, float scale) {
    __shared__ float lds[2 * 64];
    const uint32_t h = blockIdx.x, y = blockIdx.y, kh = h / (q_heads / kv_heads);
    const uint32_t ctx = min(pos[0] + 1u, max_ctx);
    const uint32_t ntiles = (ctx + X0NE_SPLIT_TILE - 1) / X0NE_SPLIT_TILE;
    if (y >= ntiles) return;
    float m[1], l[1], o[1][8];
    attend_wave<1>(q + (size_t)h * X0NE_HEAD_DIM, k_cache, v_cache, pages, kh, kv_heads, ctx, y, splits, scale, lds,
                   m, l, o);
    write_states<1>(state, h, splits, y, m, l, o);
}

// Merge of the split-K states: grid (q_heads), block 64, active = min(P, ceil(ctx / 64)).
extern "C" __global__ void __launch_bounds__(64)
    x0ne_attention_merge_bf16(const float* __restrict__ state, bf16_t* __restrict__ out,
                              const uint32_t* __restrict__ pos, uint32_t max_ctx, uint32_t splits) {
    __shared__ float lds[MERGE_LDS];
    const uint32_t h = blockIdx.x;
    const uint32_t ctx = min(pos[0] + 1u, max_ctx);
    const uint32_t active = min(splits, (ctx + X0NE_SPLIT_TILE - 1) / X0NE_SPLIT_TILE);
    merge_head(state + (size_t)h * splits * X0NE_SPLIT_STATE, out + (size_t)h * X0NE_HEAD_DIM, active, lds);
}

// Per-head decode over the whole context in one block (the reference's E2 witness,
// attention.cu:9-81): grid (q_heads), block 64; one slice, normalised in the block.
extern "C" __global__ void __launch_bounds__(64)
    x0ne_attention_decode_bf16(const bf16_t* __restrict__ q, const bf16_t* __restrict__ k_cache,
                               const bf16_t* __restrict__ v_cache, const uint32_t* __restrict__ pages,
                               bf16_t* __restrict__ out, const uint32_t* __restrict__ pos, uint32_t q_heads,
                               uint32_t kv_heads, uint32_t max_ctx, float scale) {
    __shared__ float lds[2 * 64];
    const uint32_t h = blockIdx.x, kh = h / (q_heads / kv_heads);
    const uint32_t ctx = min(pos[0] + 1u, max_ctx);
    float m[1], l[1], o[1][8];
    attend_wave<1>(q + (size_t)h * X0NE_HEAD_DIM, k_cache, v_cache, pages, kh, kv_heads, ctx, 0, 1, scale, lds, m,
                   l, o);
    const uint32_t lane = threadIdx.x & 63;
    if (lane < 16) {
        bf16_t* d = out + (size_t)h * X0NE_HEAD_DIM + 8 * lane;
#pragma unroll
        for (int j = 0; j < 8; ++j) d[j] = f2bf(o[0][j] / l[0]);
    }
}

// Causal prefill: rows at positions pos0[0] + r over the cache (already holding their keys).
// grid (q_heads, rows), block 64: one wavefront per (q head, row), the decode arithmetic over
// keys 0..min(pos0 + r, max_ctx - 1). q and out are [rows][q_heads][128].
extern "C" __global__ void __launch_bounds__(64)
    x0ne_attention_prefill_bf16(const bf16_t* __restrict__ q, const bf16_t* __restrict__ k_cache,
                                const bf16_t* __restrict__ v_cache, const uint32_t* __restrict__ pages,
                                bf16_t* __restrict__ out, const uint32_t* __restrict__ pos0, uint32_t rows,
                                uint32_t q_heads, uint32_t kv_heads, uint32_t max_ctx, float scale) {
    __shared__ float lds[2 * 64];
    const uint32_t h = blockIdx.x, row = blockIdx.y, kh = h / (q_heads / kv_heads);
    if (row >= rows) return;
    const uint32_t ctx = min(pos0[0] + row + 1u, max_ctx);
    const size_t at = ((size_t)row * q_heads + h) * X0NE_HEAD_DIM;
    float m[1], l[1], o[1][8];
    attend_wave<1>(q + at, k_cache, v_cache, pages, kh, kv_heads, ctx, 0, 1, scale, lds, m, l, o);
    const uint32_t lane = threadIdx.x & 63;
    if (lane < 16) {
#pragma unroll
        for (int j = 0; j < 8; ++j) out[at + 8 * lane + j] = f2bf(o[0][j] / l[0]);
    }
}
