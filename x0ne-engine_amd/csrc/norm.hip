// The small kernels of the decode step, for gfx950: embedding, residual add + RMSNorm, per-head
// QK-norm + RoPE + the paged KV write, SwiGLU, greedy argmax, the position advance. Each follows
// its reference kernel in x0ne-core/kernels/cuda/ (cited per kernel), with 64-lane reductions;
// the norms, RoPE and SwiGLU compute in f64 like the reference's oracle (oracle/src/lib.rs), so
// their bf16 results are the oracle's except where an f64 result sits on a rounding boundary.
#include "device.h"

// Smallest kernel that proves the build path end to end (probe.cu:4-9): out[i] = i.
// grid (ceil(n / 256)), block 256.
extern "C" __global__ void __launch_bounds__(256) x0ne_probe_iota_u32(uint32_t* out, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = i;
}

// Probe of the bf16 rounding: for the f32 values whose bits are base + i, i < n, out[i] = f2bf
// (when out is given) and counter[0] += how many differ from f2bf_bits. Any grid of 256-thread
// blocks (grid-stride).
extern "C" __global__ void __launch_bounds__(256)
    x0ne_probe_bf16_round(uint32_t base, uint32_t n, bf16_t* __restrict__ out, uint32_t* __restrict__ counter) {
    uint32_t differ = 0;
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (uint64_t)gridDim.x * 256) {
        const float x = __uint_as_float(base + (uint32_t)i);
        const bf16_t h = f2bf(x);
        differ += h != f2bf_bits(x);
        if (out) out[i] = h;
    }
    if (differ) atomicAdd(counter, differ);
}

// out[r] = table[tokens[r]] (embedding.cu:5-17): grid (rows), block 128, hidden % 8 == 0,
// 16-byte copies. An id >= vocab writes a zero row.
extern "C" __global__ void __launch_bounds__(128)
    x0ne_embedding_bf16(const bf16_t* __restrict__ table, const uint32_t* __restrict__ tokens,
                        bf16_t* __restrict__ out, uint32_t hidden, uint32_t vocab) {
    const uint32_t row = blockIdx.x;
    const uint32_t t = tokens[row];
    uint4* dst = reinterpret_cast<uint4*>(out + (size_t)row * hidden);
    const uint32_t n = hidden / 8;
    if (t >= vocab) {
        for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) dst[i] = make_uint4(0, 0, 0, 0);
        return;
    }
    const uint4* src = reinterpret_cast<const uint4*>(table + (size_t)t * hidden);
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) dst[i] = src[i];
}

// residual[r] += x[r] (f32, one addition per value); out[r] = bf16(residual / rms * w), the rms
// and the product in f64 (rmsnorm.cu:5-21; oracle/src/lib.rs:50-67). grid (rows), block 256.
// Thread t owns the 8-value chunks t, t + 256, .. of its row (values 8 chunk .. 8 chunk + 7); the
// first NORM_CHUNKS of them are loaded into registers at once (every load in flight together,
// one memory round trip per row), the rest of a wider row in a loop. Each thread sums its squares
// chunk by chunk in that order, then the block (block_sum_d): every norm kernel of this file sums
// in this order, so they give the same bits for the same row.
constexpr uint32_t NORM_CHUNKS = 4;  // 8-value chunks per thread kept in registers: hidden <= 8192 at 256

template <class Src, class Dst>
__device__ __forceinline__ void rmsnorm_row(float* __restrict__ residual, Src&& src, const bf16_t* __restrict__ w,
                                            Dst&& out, uint32_t hidden, float eps) {
    __shared__ double sh[16];
    const uint32_t t = threadIdx.x, step = blockDim.x;
    float r[NORM_CHUNKS][8], wv[NORM_CHUNKS][8];
    double ss = 0.0;
    // Loads of a clamped index, selected after: no branch between them, so all (the row's values
    // and the norm weights) are in flight at once.
#pragma unroll
    for (uint32_t c = 0; c < NORM_CHUNKS; ++c)
#pragma unroll
        for (uint32_t e = 0; e < 8; ++e) {
            const uint32_t i = 8 * (t + c * step) + e;
            const uint32_t j = i < hidden ? i : 0u;
            const float v = src(j);
            wv[c][e] = bf2f(w[j]);
            r[c][e] = i < hidden ? v : 0.0f;
        }
#pragma unroll
    for (uint32_t c = 0; c < NORM_CHUNKS; ++c)
#pragma unroll
        for (uint32_t e = 0; e < 8; ++e) {
            const uint32_t i = 8 * (t + c * step) + e;
            if (i < hidden) {
                residual[i] = r[c][e];
                ss += (double)r[c][e] * (double)r[c][e];
            }
        }
    for (uint32_t k = t + NORM_CHUNKS * step; 8 * k < hidden; k += step)  // rows wider than held
        for (uint32_t i = 8 * k; i < min(8 * k + 8, hidden); ++i) {
            const float v = src(i);
            residual[i] = v;
            ss += (double)v * (double)v;
        }
    const double total = block_sum_d(ss, sh);
    const double scale = 1.0 / sqrt(total / (double)hidden + (double)eps);
#pragma unroll
    for (uint32_t c = 0; c < NORM_CHUNKS; ++c)
#pragma unroll
        for (uint32_t e = 0; e < 8; ++e) {
            const uint32_t i = 8 * (t + c * step) + e;
            if (i < hidden) out(i) = f2bf((float)((double)r[c][e] * scale * (double)wv[c][e]));
        }
    for (uint32_t k = t + NORM_CHUNKS * step; 8 * k < hidden; k += step)
        for (uint32_t i = 8 * k; i < min(8 * k + 8, hidden); ++i)
            out(i) = f2bf((float)((double)residual[i] * scale * (double)bf2f(w[i])));
}

// rmsnorm_row's chunks, order and arithmetic with 16-byte memory operations: load(j, v) gives the
// 8 f32 values of chunk j (residual + x), the residual is written as two float4 at res + 8 k and
// out chunk k as 8 bf16 by store(k, value). For hidden a multiple of 8 and at most 8192, a
// 256-thread block and 16-byte aligned rows (the callers check and fall back to rmsnorm_row).
template <class Load, class Store>
__device__ __forceinline__ void rmsnorm_row_vec(float* __restrict__ res, Load&& load, const bf16_t* __restrict__ w,
                                                Store&& store, uint32_t hidden, float eps) {
    __shared__ double sh[16];
    const uint32_t t = threadIdx.x, chunks = hidden / 8;
    float r[NORM_CHUNKS][8];
    uint4 wv[NORM_CHUNKS];
#pragma unroll
    for (uint32_t c = 0; c < NORM_CHUNKS; ++c) {
        const uint32_t k = t + 256 * c;
        const uint32_t j = k < chunks ? k : 0u;  // loads of a clamped chunk, selected after
        load(j, r[c]);
        wv[c] = reinterpret_cast<const uint4*>(w)[j];
    }
    double ss = 0.0;
#pragma unroll
    for (uint32_t c = 0; c < NORM_CHUNKS; ++c) {
        const uint32_t k = t + 256 * c;
        if (k < chunks) {
            reinterpret_cast<float4*>(res)[2 * k] = make_float4(r[c][0], r[c][1], r[c][2], r[c][3]);
            reinterpret_cast<float4*>(res)[2 * k + 1] = make_float4(r[c][4], r[c][5], r[c][6], r[c][7]);
#pragma unroll
            for (int e = 0; e < 8; ++e) ss += (double)r[c][e] * (double)r[c][e];
        }
    }
    const double total = block_sum_d(ss, sh);
    const double scale = 1.0 / sqrt(total / (double)hidden + (double)eps);
#pragma unroll
    for (uint32_t c = 0; c < NORM_CHUNKS; ++c) {
        const uint32_t k = t + 256 * c;
        if (k >= chunks) continue;
        const uint32_t ww[4] = {wv[c].x, wv[c].y, wv[c].z, wv[c].w};
        uint32_t ow[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const bf16_t lo = f2bf((float)((double)r[c][2 * e] * scale * (double)bf_lo(ww[e])));
            const bf16_t hi = f2bf((float)((double)r[c][2 * e + 1] * scale * (double)bf_hi(ww[e])));
            ow[e] = (uint32_t)lo | ((uint32_t)hi << 16);
        }
        store(k, make_uint4(ow[0], ow[1], ow[2], ow[3]));
    }
}

__device__ __forceinline__ bool vec_norm_ok(uint32_t hidden, uintptr_t ptrs) {
    return hidden % 8 == 0 && hidden <= 8 * 256 * NORM_CHUNKS && blockDim.x == 256 && (ptrs & 15) == 0;
}

// The 8 values of chunk j of a row: an f32 residual plus a bf16 x.
__device__ __forceinline__ void add_chunk(const float* __restrict__ res, const bf16_t* __restrict__ x, uint32_t j,
                                          float (&v)[8]) {
    const float4 r0 = reinterpret_cast<const float4*>(res)[2 * j], r1 = reinterpret_cast<const float4*>(res)[2 * j + 1];
    const uint4 xv = reinterpret_cast<const uint4*>(x)[j];
    const float rv[8] = {r0.x, r0.y, r0.z, r0.w, r1.x, r1.y, r1.z, r1.w};
    const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = rv[e] + (e & 1 ? bf_hi(xw[e / 2]) : bf_lo(xw[e / 2]));
}

// The prefill pass's rows. grid (rows), block 256.
extern "C" __global__ void __launch_bounds__(256)
    x0ne_add_rmsnorm_bf16(float* __restrict__ residual, const bf16_t* __restrict__ x, const bf16_t* __restrict__ w,
                          bf16_t* __restrict__ out, uint32_t hidden, float eps) {
    const size_t base = (size_t)blockIdx.x * hidden;
    float* res = residual + base;
    const bf16_t* xr = x + base;
    bf16_t* o = out + base;
    if (!vec_norm_ok(hidden, (uintptr_t)residual | (uintptr_t)x | (uintptr_t)w | (uintptr_t)out)) {  // grid-uniform
        rmsnorm_row(res, [&](uint32_t i) { return res[i] + bf2f(xr[i]); }, w,
                    [&](uint32_t i) -> bf16_t& { return o[i]; }, hidden, eps);
        return;
    }
    rmsnorm_row_vec(res, [&](uint32_t j, float (&v)[8]) { add_chunk(res, xr, j, v); }, w,
                    [&](uint32_t k, uint4 v) { reinterpret_cast<uint4*>(o)[k] = v; }, hidden, eps);
}

// x0ne_add_rmsnorm_bf16 with the residual read from res_in and the sum written to res_out (the
// decode step's two residual buffers, which the MoE feed-forward keeps: the GEMV prologues read
// one and write the other). The same arithmetic as x0ne_add_rmsnorm_bf16. grid (rows), block 256;
// res_in and res_out must not overlap.
extern "C" __global__ void __launch_bounds__(256)
    x0ne_add_rmsnorm_to_bf16(const float* __restrict__ res_in, float* __restrict__ res_out,
                             const bf16_t* __restrict__ x, const bf16_t* __restrict__ w, bf16_t* __restrict__ out,
                             uint32_t hidden, float eps) {
    const size_t base = (size_t)blockIdx.x * hidden;
    const float* ri = res_in + base;
    const bf16_t* xr = x + base;
    bf16_t* o = out + base;
    if (!vec_norm_ok(hidden, (uintptr_t)res_in | (uintptr_t)res_out | (uintptr_t)x | (uintptr_t)w | (uintptr_t)out)) {
        rmsnorm_row(res_out + base, [&](uint32_t i) { return ri[i] + bf2f(xr[i]); }, w,
                    [&](uint32_t i) -> bf16_t& { return o[i]; }, hidden, eps);
        return;
    }
    rmsnorm_row_vec(res_out + base, [&](uint32_t j, float (&v)[8]) { add_chunk(ri, xr, j, v); }, w,
                    [&](uint32_t k, uint4 v) { reinterpret_cast<uint4*>(o)[k] = v; }, hidden, eps);
}

// x0ne_add_rmsnorm_bf16 with out in panels (hidden a multiple of 8): the batched step's norms,
// whose rows feed the few-row GEMM. The same bits at the panel positions (a chunk of 8 values is
// 8 consecutive panel elements). grid (rows), block 256.
extern "C" __global__ void __launch_bounds__(256)
    x0ne_add_rmsnorm_panel_bf16(float* __restrict__ residual, const bf16_t* __restrict__ x,
                                const bf16_t* __restrict__ w, bf16_t* __restrict__ out, uint32_t hidden, float eps) {
    const uint32_t row = blockIdx.x;
    const size_t base = (size_t)row * hidden;
    float* res = residual + base;
    const bf16_t* xr = x + base;
    if (hidden % 8 != 0) return;
    if (!vec_norm_ok(hidden, (uintptr_t)residual | (uintptr_t)x | (uintptr_t)w | (uintptr_t)out)) {
        rmsnorm_row(res, [&](uint32_t i) { return res[i] + bf2f(xr[i]); }, w,
                    [&](uint32_t i) -> bf16_t& { return out[panel_index(row, i, hidden)]; }, hidden, eps);
        return;
    }
    rmsnorm_row_vec(res, [&](uint32_t j, float (&v)[8]) { add_chunk(res, xr, j, v); }, w,
                    [&](uint32_t k, uint4 v) { *reinterpret_cast<uint4*>(out + panel_index(row, 8 * k, hidden)) = v; },
                    hidden, eps);
}

// The first norm of a batched step: residual[r] = 0 + table[tokens[r]] (f32; an id >= vocab gives
// a zero row) and row r of out (in panels, hidden a multiple of 8) its RMSNorm: the bits
// x0ne_embedding_bf16 followed by x0ne_add_rmsnorm_bf16 on a zero residual give. grid (rows),
// block 256.
extern "C" __global__ void __launch_bounds__(256)
    x0ne_embed_rmsnorm_panel_bf16(const bf16_t* __restrict__ table, const uint32_t* __restrict__ tokens,
                                  float* __restrict__ residual, const bf16_t* __restrict__ w, bf16_t* __restrict__ out,
                                  uint32_t hidden, uint32_t vocab, float eps) {
    const uint32_t row = blockIdx.x;
    if (hidden % 8 != 0) return;
    const size_t base = (size_t)row * hidden;
    const uint32_t tok = tokens[blockIdx.x];
    const bf16_t* src = table + (size_t)(tok < vocab ? tok : 0) * hidden;
    const bool in = tok < vocab;
    if (!vec_norm_ok(hidden, (uintptr_t)table | (uintptr_t)residual | (uintptr_t)w | (uintptr_t)out)) {
        rmsnorm_row(residual + base, [&](uint32_t i) {
            const float v = bf2f(src[i]);  // row 0 for an id past the table, then not used
            return 0.0f + (in ? v : 0.0f);
        }, w, [&](uint32_t i) -> bf16_t& { return out[panel_index(row, i, hidden)]; }, hidden, eps);
        return;
    }
    rmsnorm_row_vec(residual + base, [&](uint32_t j, float (&v)[8]) {
        const uint4 sv = reinterpret_cast<const uint4*>(src)[j];
        const uint32_t sw[4] = {sv.x, sv.y, sv.z, sv.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = 0.0f + (in ? (e & 1 ? bf_hi(sw[e / 2]) : bf_lo(sw[e / 2])) : 0.0f);
    }, w, [&](uint32_t k, uint4 v) { *reinterpret_cast<uint4*>(out + panel_index(row, 8 * k, hidden)) = v; },
                    hidden, eps);
}

// Per-head RMSNorm of q and k, rotate-half RoPE, and the K/V write into the paged cache
// (rope.cu:7-47; oracle/src/lib.rs:82-120). grid (q_heads + kv_heads, rows), block 64: lane i
// owns the pair (i, i + 64) of one head. Row r sits at position pos0[0] + r, written at
// physical page page_table[pos / 16], slot pos % 16 of the layer's K plane
// ([pages][kv_heads][16][128]) and V plane ([pages][kv_heads][128][16]). A position >= max_ctx
// writes nothing into the cache. The angle
// is the f32 product pos * inv_freq[i] (inv_freq computed on the host in f32), its sine and
// cosine in f64. Blocks of k heads also copy v, bit for bit.
extern "C" __global__ void __launch_bounds__(64)
    x0ne_qk_norm_rope_kv_write_bf16(const bf16_t* __restrict__ qkv, const bf16_t* __restrict__ q_norm,
                                    const bf16_t* __restrict__ k_norm, const float* __restrict__ inv_freq,
                                    bf16_t* __restrict__ q_out, bf16_t* __restrict__ k_cache,
                                    bf16_t* __restrict__ v_cache, const uint32_t* __restrict__ pages,
                                    const uint32_t* __restrict__ pos0, uint32_t q_heads, uint32_t kv_heads,
                                    uint32_t max_ctx, float eps) {
    constexpr uint32_t HD = X0NE_HEAD_DIM, HALF = HD / 2;
    const uint32_t head = blockIdx.x, row = blockIdx.y, i = threadIdx.x;
    const uint32_t q_dim = q_heads * HD, kv_dim = kv_heads * HD, qkv_dim = q_dim + 2 * kv_dim;
    const uint32_t pos = pos0[0] + row;
    const bool is_q = head < q_heads;
    const uint32_t kh = is_q ? 0 : head - q_heads;
    const bf16_t* src = qkv + (size_t)row * qkv_dim + (is_q ? head * HD : q_dim + kh * HD);
    const bf16_t* nw = is_q ? q_norm : k_norm;

    const float a = bf2f(src[i]), b = bf2f(src[i + HALF]);
    const double ss = wave_sum_d((double)a * (double)a + (double)b * (double)b);
    const double scale = 1.0 / sqrt(ss / (double)HD + (double)eps);
    const double na = (double)a * scale * (double)bf2f(nw[i]);
    const double nb = (double)b * scale * (double)bf2f(nw[i + HALF]);
    const double angle = (double)((float)pos * inv_freq[i]);
    const double s = sin(angle), c = cos(angle);
    const float ra = (float)(na * c - nb * s);
    const float rb = (float)(nb * c + na * s);

    if (is_q) {
        bf16_t* d = q_out + (size_t)row * q_dim + head * HD;
        d[i] = f2bf(ra);
        d[i + HALF] = f2bf(rb);
        return;
    }
    if (pos >= max_ctx) return;
    const uint32_t at = kv_row(pages, pos, kh, kv_heads);
    k_cache[at + i] = f2bf(ra);
    k_cache[at + i + HALF] = f2bf(rb);
    const bf16_t* vs = qkv + (size_t)row * qkv_dim + q_dim + kv_dim + kh * HD;
    const uint32_t vat = v_slot(pages, pos, kh, kv_heads);
    v_cache[vat + i * X0NE_PAGE] = vs[i];
    v_cache[vat + (i + HALF) * X0NE_PAGE] = vs[i + HALF];
}

// x0ne_qk_norm_rope_kv_write_bf16 for the rows of a prefill pass: the same arithmetic and
// writes, with each position's cos and sin read from the RoPE table cs (x0ne_rope_table_f64 below,
// positions < max_ctx) instead of computed, and four heads of one row per 256-thread block (one
// per wavefront). The table holds the f64 values the direct kernel computes, so the two give
// the same bits. grid (ceil((q_heads + kv_heads) / 4), rows), block 256.
extern "C" __global__ void __launch_bounds__(256)
    x0ne_qk_norm_rope_kv_write_rows_bf16(const bf16_t* __restrict__ qkv, const bf16_t* __restrict__ q_norm,
                                         const bf16_t* __restrict__ k_norm, const double* __restrict__ cs,
                                         bf16_t* __restrict__ q_out, bf16_t* __restrict__ k_cache,
                                         bf16_t* __restrict__ v_cache, const uint32_t* __restrict__ pages,
                                         const uint32_t* __restrict__ pos0, uint32_t q_heads, uint32_t kv_heads,
                                         uint32_t max_ctx, float eps) {
    constexpr uint32_t HD = X0NE_HEAD_DIM, HALF = HD / 2;
    const uint32_t head = blockIdx.x * 4 + (threadIdx.x >> 6), row = blockIdx.y, i = threadIdx.x & 63;
    if (head >= q_heads + kv_heads) return;  // wavefront-uniform
    const uint32_t q_dim = q_heads * HD, kv_dim = kv_heads * HD, qkv_dim = q_dim + 2 * kv_dim;
    const uint32_t pos = pos0[0] + row;
    if (pos >= max_ctx) return;  // no table entry, and no cache slot; a pass never reaches it
    const bool is_q = head < q_heads;
    const uint32_t kh = is_q ? 0 : head - q_heads;
    const bf16_t* src = qkv + (size_t)row * qkv_dim + (is_q ? head * HD : q_dim + kh * HD);
    const bf16_t* nw = is_q ? q_norm : k_norm;

    const double2 t = reinterpret_cast<const double2*>(cs)[(size_t)pos * HALF + i];  // (cos, sin)
    const float a = bf2f(src[i]), b = bf2f(src[i + HALF]);
    const double ss = wave_sum_d((double)a * (double)a + (double)b * (double)b);
    const double scale = 1.0 / sqrt(ss / (double)HD + (double)eps);
    const double na = (double)a * scale * (double)bf2f(nw[i]);
    const double nb = (double)b * scale * (double)bf2f(nw[i + HALF]);
    const float ra = (float)(na * t.x - nb * t.y);
    const float rb = (float)(nb * t.x + na * t.y);

    if (is_q) {
        bf16_t* d = q_out + (size_t)row * q_dim + head * HD;
        d[i] = f2bf(ra);
        d[i + HALF] = f2bf(rb);
        return;
    }
    const uint32_t at = kv_row(pages, pos, kh, kv_heads);
    k_cache[at + i] = f2bf(ra);
    k_cache[at + i + HALF] = f2bf(rb);
    const bf16_t* vs = qkv + (size_t)row * qkv_dim + q_dim + kv_dim + kh * HD;
    const uint32_t vat = v_slot(pages, pos, kh, kv_heads);
    v_cache[vat + i * X0NE_PAGE] = vs[i];
    v_cache[vat + (i + HALF) * X0NE_PAGE] = vs[i + HALF];
}

// The RoPE table of the fused decode attention: cs[2 (p 64 + i)] = cos and cs[2 (p 64 + i) + 1] =
// sin of the f64 angle (double)((float)p * inv_freq[i]), positions p < positions: the values the
// rotation above computes, so a kernel that reads them rotates to the same bits. grid
// (ceil(positions * 64 / 256)), block 256.
extern "C" __global__ void __launch_bounds__(256)
    x0ne_rope_table_f64(const float* __restrict__ inv_freq, double* __restrict__ cs, uint32_t positions) {
    const uint64_t k = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (k >= (uint64_t)positions * (X0NE_HEAD_DIM / 2)) return;
    const uint32_t p = (uint32_t)(k / (X0NE_HEAD_DIM / 2)), i = (uint32_t)(k % (X0NE_HEAD_DIM / 2));
    const double angle = (double)((float)p * inv_freq[i]);
    cs[2 * k] = cos(angle);
    cs[2 * k + 1] = sin(angle);
}

// SwiGLU on the packed [gate; up] row: out[i] = g / (1 + e^-g) * u, in f64 (swiglu.cu:5-11;
// oracle/src/lib.rs:205-214). Thread t of block x takes values 8 (256 x + t) .. + 7 of row y:
// 16-byte loads of gate and up and one 16-byte store where inter is a multiple of 8 and both
// pointers are 16-byte aligned (single values otherwise). grid (ceil(inter / 2048), rows), block 256.
__device__ __forceinline__ bf16_t swiglu1(bf16_t g16, bf16_t u16) {
    const double g = (double)bf2f(g16), u = (double)bf2f(u16);
    return f2bf((float)(g / (1.0 + exp(-g)) * u));
}
extern "C" __global__ void __launch_bounds__(256)
    x0ne_swiglu_bf16(const bf16_t* __restrict__ gate_up, bf16_t* __restrict__ out, uint32_t inter) {
    const uint32_t i0 = 8 * (blockIdx.x * blockDim.x + threadIdx.x), r = blockIdx.y;
    if (i0 >= inter) return;
    const bf16_t* row = gate_up + (size_t)r * 2 * inter;
    bf16_t* o = out + (size_t)r * inter;
    if (inter % 8 == 0 && (((uintptr_t)gate_up | (uintptr_t)out) & 15) == 0) {  // grid-uniform
        const uint4 g = *reinterpret_cast<const uint4*>(row + i0);
        const uint4 u = *reinterpret_cast<const uint4*>(row + inter + i0);
        const uint32_t gw[4] = {g.x, g.y, g.z, g.w}, uw[4] = {u.x, u.y, u.z, u.w};
        uint32_t ow[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            ow[j] = (uint32_t)swiglu1((bf16_t)(gw[j] & 0xFFFFu), (bf16_t)(uw[j] & 0xFFFFu)) |
                    ((uint32_t)swiglu1((bf16_t)(gw[j] >> 16), (bf16_t)(uw[j] >> 16)) << 16);
        *reinterpret_cast<uint4*>(o + i0) = make_uint4(ow[0], ow[1], ow[2], ow[3]);
        return;
    }
    for (uint32_t i = i0; i < min(i0 + 8, inter); ++i) o[i] = swiglu1(row[i], row[inter + i]);
}

// x0ne_swiglu_bf16 with out in 16-row panels (device.h) of inter columns, for the prefill pass's
// down projection: the same values (swiglu1 of each gate and up pair), stored at panel_index.
// grid (ceil(inter / 2048), rows), block 256.
extern "C" __global__ void __launch_bounds__(256)
    x0ne_swiglu_panel_bf16(const bf16_t* __restrict__ gate_up, bf16_t* __restrict__ out, uint32_t inter) {
    const uint32_t i0 = 8 * (blockIdx.x * blockDim.x + threadIdx.x), r = blockIdx.y;
    if (i0 >= inter) return;
    const bf16_t* row = gate_up + (size_t)r * 2 * inter;
    if (inter % 8 == 0 && ((uintptr_t)gate_up & 15) == 0 && ((uintptr_t)out & 15) == 0) {  // grid-uniform
        const uint4 g = *reinterpret_cast<const uint4*>(row + i0);
        const uint4 u = *reinterpret_cast<const uint4*>(row + inter + i0);
        const uint32_t gw[4] = {g.x, g.y, g.z, g.w}, uw[4] = {u.x, u.y, u.z, u.w};
        uint32_t ow[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            ow[j] = (uint32_t)swiglu1((bf16_t)(gw[j] & 0xFFFFu), (bf16_t)(uw[j] & 0xFFFFu)) |
                    ((uint32_t)swiglu1((bf16_t)(gw[j] >> 16), (bf16_t)(uw[j] >> 16)) << 16);
        *reinterpret_cast<uint4*>(out + panel_index(r, i0, inter)) = make_uint4(ow[0], ow[1], ow[2], ow[3]);
        return;
    }
    for (uint32_t i = i0; i < min(i0 + 8, inter); ++i) out[panel_index(r, i, inter)] = swiglu1(row[i], row[inter + i]);
}

__device__ __forceinline__ bool better(float v, uint32_t i, float bv, uint32_t bi) {
    return v > bv || (v == bv && i < bi);
}

// The first largest value of row[0 .. n) with its index (0xFFFFFFFF and -inf for an empty
// row) and whether the row holds a NaN, for thread 0 of a block of whole wavefronts (at most 16).
struct ArgBest {
    float v;
    uint32_t i;
    bool nan;
};

__device__ __forceinline__ ArgBest argmax_block(const float* __restrict__ row, uint32_t n) {
    __shared__ float sv[16];
    __shared__ uint32_t si[16];
    __shared__ int snan;
    const uint32_t t = threadIdx.x, lane = t & 63, wave = t >> 6, nw = blockDim.x >> 6;
    if (t == 0) snan = 0;
    __syncthreads();
    float bv = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu;
    bool nan = false;
    for (uint32_t i = t; i < n; i += blockDim.x) {
        const float v = row[i];
        nan |= v != v;
        if (better(v, i, bv, bi)) {
            bv = v;
            bi = i;
        }
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const uint32_t oi = __shfl_xor(bi, o, 64);
        if (better(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    }
    if (__any(nan) && lane == 0) atomicOr(&snan, 1);
    if (lane == 0) {
        sv[wave] = bv;
        si[wave] = bi;
    }
    __syncthreads();
    ArgBest best = {-INFINITY, 0xFFFFFFFFu, snan != 0};
    if (t == 0) {
        for (uint32_t w = 0; w < nw; ++w) {
            if (better(sv[w], si[w], best.v, best.i)) {
                best.v = sv[w];
                best.i = si[w];
            }
        }
    }
    return best;
}

// Greedy pick (argmax.cu:11-58): index of the largest logit of each row, lowest index on ties;
// a row holding any NaN yields 0xFFFFFFFF. grid (rows), block 1024 (16 wavefronts).
extern "C" __global__ void __launch_bounds__(1024)
    x0ne_argmax_f32(const float* __restrict__ logits, uint32_t n, uint32_t* __restrict__ out) {
    const ArgBest b = argmax_block(logits + (size_t)blockIdx.x * n, n);
    if (threadIdx.x == 0) out[blockIdx.x] = b.nan ? 0xFFFFFFFFu : b.i;
}

// The batched step's pick in two launches, so many blocks share a row: slice s of row r (grid
// (rows, slices), block 256) takes values s per .. (s + 1) per - 1, per = ceil(n / slices), and
// writes its first largest value, that value's index in the row and its NaN flag into
// partial[3 (r slices + s) ..]; then x0ne_argmax_pick_advance (grid (rows), block 64) takes the
// first largest over the slices in slice order (so the lowest index on ties, as x0ne_argmax_f32),
// 0xFFFFFFFF when any slice saw a NaN, into tokens[r], and advances pos[r].
extern "C" __global__ void __launch_bounds__(256)
    x0ne_argmax_slices_f32(const float* __restrict__ logits, uint32_t n, uint32_t slices,
                           uint32_t* __restrict__ partial) {
    const uint32_t r = blockIdx.x, s = blockIdx.y;
    const uint32_t per = (n + slices - 1) / slices, begin = min(s * per, n), len = min(per, n - begin);
    const ArgBest b = argmax_block(logits + (size_t)r * n + begin, len);
    if (threadIdx.x == 0) {
        uint32_t* p = partial + 3 * ((size_t)r * slices + s);
        p[0] = __float_as_uint(b.v);
        p[1] = b.i == 0xFFFFFFFFu ? 0xFFFFFFFFu : begin + b.i;
        p[2] = b.nan ? 1u : 0u;
    }
}

extern "C" __global__ void __launch_bounds__(64)
    x0ne_argmax_pick_advance(const uint32_t* __restrict__ partial, uint32_t slices, uint32_t* __restrict__ tokens,
                             uint32_t* __restrict__ pos) {
    const uint32_t r = blockIdx.x, lane = threadIdx.x;
    float bv = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu;
    bool nan = false;
    for (uint32_t s = lane; s < slices; s += 64) {  // lane order = slice order within a lane
        const uint32_t* p = partial + 3 * ((size_t)r * slices + s);
        const float v = __uint_as_float(p[0]);
        nan |= p[2] != 0;
        if (better(v, p[1], bv, bi)) {
            bv = v;
            bi = p[1];
        }
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const uint32_t oi = __shfl_xor(bi, o, 64);
        if (better(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    }
    nan = __any(nan);
    if (lane == 0) {
        tokens[r] = nan ? 0xFFFFFFFFu : bi;
        pos[r] += 1u;
    }
}

// Position advance, the last node of the decode step (advance.cu:5-7): pos[0] += 1.
// grid (1), block 64.
extern "C" __global__ void __launch_bounds__(64) x0ne_advance_u32(uint32_t* __restrict__ pos) {
    if (threadIdx.x == 0 && blockIdx.x == 0) pos[0] += 1u;
}

// Prefill feed (this build's): token ids[i] into tokens[0] and position i into pos[0], so the
// decode step that reads both on the device runs on prompt token i. grid (1), block 64.
extern "C" __global__ void __launch_bounds__(64)
    x0ne_feed_u32(const uint32_t* __restrict__ ids, uint32_t i, uint32_t* __restrict__ tokens,
                  uint32_t* __restrict__ pos) {
    if (threadIdx.x == 0 && blockIdx.x == 0) {
        tokens[0] = ids[i];
        pos[0] = i;
    }
}
