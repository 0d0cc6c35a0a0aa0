// The projections of a many-row pass (prefill, batched rows) on the matrix cores:
// Y[n][rows] = X[n][cols] W^T with W [rows][cols] and X [n][cols] bf16 row-major, f32
// accumulation, Y bf16 or f32 (the reference's Gpu::gemm, gpu.rs:1098-1149, which hands this to
// cuBLAS). At one row the decode GEMV (gemv.hip) is the right kernel; from a few rows on the work
// is compute-bound and belongs here.
//
// Tiling, for gfx950 (wave64, 16x16x32 bf16 MFMA, 160 KiB LDS per CU):
//  - A block (256 threads, 4 wavefronts as 2 x 2) computes a 128 (tokens) x 128 (W rows) tile
//    of Y; a wavefront 64 x 64, as 4 x 4 blocks of 16 x 16, 16 f32x4 accumulators.
//  - K advances 64 columns at a time: each thread requests its 4 + 4 16-byte pieces of the next
//    X and W slices (raw buffer loads: a piece past the matrix or past a row's end gives zeros
//    without a branch) while the matrix cores work on the current slice, then writes them into
//    the other half of a double-buffered LDS tile. LDS rows are 64 + 8 bf16 (the pad spreads
//    the 16 rows a fragment read touches over the banks).
//  - The linear block index is dealt round-robin over the 8 XCDs; it is remapped so each XCD
//    takes a contiguous run of tiles, W-row tile major: the token tiles that reuse one 1 MiB W
//    slice run on one XCD and meet it in that XCD's L2.
#include "device.h"

namespace {

constexpr int BM = 128, BN = 128, BK = 64, LDT = BK + 8;  // LDS row: 72 bf16 = 144 bytes
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

__device__ __forceinline__ uint4 bload(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
    return make_uint4((uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]);
}

struct Lds {
    bf16_t a[2][BM][LDT];
    bf16_t b[2][BN][LDT];
};

}  // namespace

// grid (ceil(rows / 128) * ceil(n / 128)), block 256. cols a multiple of 8 (16-byte pieces);
// X and W below 4 GiB - 16 bytes each (32-bit buffer offsets).
extern "C" __global__ void __launch_bounds__(256)
    x0ne_gemm_bf16(const bf16_t* __restrict__ w, const bf16_t* __restrict__ x, void* __restrict__ y, uint32_t rows,
                   uint32_t cols, uint32_t n, uint32_t out_f32) {
    __shared__ Lds sh;
    const uint32_t tw = (rows + BN - 1) / BN, tn = (n + BM - 1) / BM, total = tw * tn;
    uint32_t tile = blockIdx.x;
    if (tile >= total || cols % 8 != 0) return;
    if (total % 8 == 0) tile = (tile % 8) * (total / 8) + tile / 8;  // XCD-contiguous runs
    const uint32_t wt = tile / tn, nt = tile % tn;
    const uint32_t row0 = wt * BN, tok0 = nt * BM;

    const uint32_t t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const uint32_t wm = wave >> 1, wn = wave & 1;  // the wavefront's 64 x 64 of the tile
    const auto xr = rsrc(x, (uint64_t)n * cols * 2), wr = rsrc(w, (uint64_t)rows * cols * 2);

    // This thread's pieces of a 128 x 64 slice: rows t / 8 + 32 i, 16-byte column c8 = t % 8.
    const uint32_t prow = t >> 3, c8 = t & 7;
    uint4 pa[4], pb[4];
    auto request = [&](uint32_t k0) {
        const uint32_t col = k0 + 8 * c8;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t tr = tok0 + prow + 32 * i, wrow = row0 + prow + 32 * i;
            pa[i] = bload(xr, tr < n && col < cols ? (tr * cols + col) * 2 : OFF_NONE);
            pb[i] = bload(wr, wrow < rows && col < cols ? (wrow * cols + col) * 2 : OFF_NONE);
        }
    };
    auto stage = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            *reinterpret_cast<uint4*>(&sh.a[buf][prow + 32 * i][8 * c8]) = pa[i];
            *reinterpret_cast<uint4*>(&sh.b[buf][prow + 32 * i][8 * c8]) = pb[i];
        }
    };

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const uint32_t nk = (cols + BK - 1) / BK;
    request(0);
    stage(0);
    lds_barrier();
    const uint32_t fr = lane & 15, fk = 8 * (lane >> 4);  // fragment row and k offset
    for (uint32_t ks = 0; ks < nk; ++ks) {
        const int cur = ks & 1;
        if (ks + 1 < nk) request((ks + 1) * BK);
#pragma unroll
        for (int kk = 0; kk < BK; kk += 32) {
            uint4 fa[4], fb[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                fa[i] = *reinterpret_cast<const uint4*>(&sh.a[cur][64 * wm + 16 * i + fr][kk + fk]);
                fb[i] = *reinterpret_cast<const uint4*>(&sh.b[cur][64 * wn + 16 * i + fr][kk + fk]);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = mfma(fa[i], fb[j], acc[i][j]);
        }
        if (ks + 1 < nk) stage(cur ^ 1);
        lds_barrier();
    }

    // acc[i][j][r]: token tok0 + 64 wm + 16 i + 4 (lane / 16) + r, W row row0 + 64 wn + 16 j + lane % 16.
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t tok = tok0 + 64 * wm + 16 * i + 4 * (lane >> 4) + r;
            if (tok >= n) continue;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t col = row0 + 64 * wn + 16 * j + (lane & 15);
                if (col >= rows) continue;
                const size_t at = (size_t)tok * rows + col;
                if (out_f32)
                    static_cast<float*>(y)[at] = acc[i][j][r];
                else
                    static_cast<bf16_t*>(y)[at] = f2bf(acc[i][j][r]);
            }
        }
}
