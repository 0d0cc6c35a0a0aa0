// Synthetic weights drawn on the device: N(0, std) bf16 from a counter-based splitmix64 stream,
// through Box-Muller with log and sin/cos written from +, -, *, / only. The CPU oracle's
// generator (oracle/x0ne_oracle.c, xo_normal_at) is the same code operation for operation; with
// contraction off on both sides (this file is compiled with -ffp-contract=off, and the pragma
// below repeats it), the device and the host draw the same bits, which a GPU test checks.
//
// Stream: value i of tensor key K takes splitmix64 outputs 2k and 2k + 1 (k = i / 2) of a
// generator seeded with K: r = fmix(K + (j + 1) * 0x9E3779B97F4A7C15). u1 = (r1 >> 11 + 1) 2^-53,
// u2 = (r2 >> 11) 2^-53; value 2k = sqrt(-2 ln u1) cos(2 pi u2), value 2k + 1 the sine.
#include "device.h"
#include "launch.h"

#pragma clang fp contract(off)

namespace {

constexpr uint64_t GOLDEN = 0x9E3779B97F4A7C15ull;

__device__ __forceinline__ uint64_t fmix(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ double det_log(double x) {
    uint64_t b = __double_as_longlong(x);
    int e = (int)((b >> 52) & 0x7FF) - 1023;
    double m = __longlong_as_double((long long)((b & 0x000FFFFFFFFFFFFFull) | 0x3FF0000000000000ull));
    if (m > 1.4142135623730951) {
        m = m * 0.5;
        e += 1;
    }
    const double f = (m - 1.0) / (m + 1.0);
    const double f2 = f * f;
    const double c[14] = {1.0,        1.0 / 3.0,  1.0 / 5.0,  1.0 / 7.0,  1.0 / 9.0,
                          1.0 / 11.0, 1.0 / 13.0, 1.0 / 15.0, 1.0 / 17.0, 1.0 / 19.0,
                          1.0 / 21.0, 1.0 / 23.0, 1.0 / 25.0, 1.0 / 27.0};
    double p = c[13];
#pragma unroll
    for (int k = 12; k >= 0; --k) p = p * f2 + c[k];
    return (double)e * 0.6931471805599453 + 2.0 * f * p;
}

__device__ void det_sincos_turn(double u, double* s, double* c) {
    const double t = u * 4.0;
    const int q = (int)t;
    const double r = t - (double)q;
    const double phi = r * 1.5707963267948966;
    const double p2 = phi * phi;
    const double sc[12] = {
        1.0,
        -1.0 / 6.0,
        1.0 / 120.0,
        -1.0 / 5040.0,
        1.0 / 362880.0,
        -1.0 / 39916800.0,
        1.0 / 6227020800.0,
        -1.0 / 1307674368000.0,
        1.0 / 355687428096000.0,
        -1.0 / 121645100408832000.0,
        1.0 / 51090942171709440000.0,
        -1.0 / 25852016738884976640000.0,
    };
    const double cc[13] = {
        1.0,
        -1.0 / 2.0,
        1.0 / 24.0,
        -1.0 / 720.0,
        1.0 / 40320.0,
        -1.0 / 3628800.0,
        1.0 / 479001600.0,
        -1.0 / 87178291200.0,
        1.0 / 20922789888000.0,
        -1.0 / 6402373705728000.0,
        1.0 / 2432902008176640000.0,
        -1.0 / 1124000727777607680000.0,
        1.0 / 620448401733239439360000.0,
    };
    double ps = sc[11];
#pragma unroll
    for (int k = 10; k >= 0; --k) ps = ps * p2 + sc[k];
    const double S = phi * ps;
    double pc = cc[12];
#pragma unroll
    for (int k = 11; k >= 0; --k) pc = pc * p2 + cc[k];
    const double C = pc;
    switch (q & 3) {
        case 0: *s = S; *c = C; break;
        case 1: *s = C; *c = -S; break;
        case 2: *s = -S; *c = -C; break;
        default: *s = -C; *c = S; break;
    }
}

// Values 2k and 2k + 1 of stream `key`, as bf16 bits of std * z.
__device__ __forceinline__ void normal_pair(uint64_t key, uint64_t k, double std_dev, bf16_t* z0, bf16_t* z1) {
    const uint64_t r1 = fmix(key + (2 * k + 1) * GOLDEN);
    const uint64_t r2 = fmix(key + (2 * k + 2) * GOLDEN);
    const double u1 = (double)((r1 >> 11) + 1) * 0x1p-53;
    const double u2 = (double)(r2 >> 11) * 0x1p-53;
    const double rad = sqrt(-2.0 * det_log(u1));
    double s, c;
    det_sincos_turn(u2, &s, &c);
    *z0 = f2bf((float)(std_dev * (rad * c)));
    *z1 = f2bf((float)(std_dev * (rad * s)));
}

// out[j] = value first + j of stream `key`, j < n; first is even. grid-stride over pairs.
__global__ void __launch_bounds__(256)
    init_normal_bf16(bf16_t* __restrict__ out, uint64_t n, uint64_t key, uint64_t first, double std_dev) {
    const uint64_t pairs = (n + 1) / 2;
    for (uint64_t p = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; p < pairs;
         p += (uint64_t)gridDim.x * blockDim.x) {
        bf16_t z0, z1;
        normal_pair(key, first / 2 + p, std_dev, &z0, &z1);
        out[2 * p] = z0;
        if (2 * p + 1 < n) out[2 * p + 1] = z1;
    }
}

__global__ void __launch_bounds__(256) fill_u16(uint16_t* __restrict__ out, uint64_t n, uint16_t v) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        out[i] = v;
}

}  // namespace

hipError_t x0ne_launch_init_normal(uint16_t* out, uint64_t n, uint64_t key, uint64_t first, double std_dev,
                                   hipStream_t s) {
    if (first % 2 != 0) return hipErrorInvalidValue;
    const uint64_t pairs = (n + 1) / 2;
    uint64_t blocks = (pairs + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (blocks == 0) return hipSuccess;
    init_normal_bf16<<<(uint32_t)blocks, 256, 0, s>>>(out, n, key, first, std_dev);
    return hipGetLastError();
}

hipError_t x0ne_launch_fill_u16(uint16_t* out, uint64_t n, uint16_t v, hipStream_t s) {
    uint64_t blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (blocks == 0) return hipSuccess;
    fill_u16<<<(uint32_t)blocks, 256, 0, s>>>(out, n, v);
    return hipGetLastError();
}
