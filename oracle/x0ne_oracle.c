/*
 * CPU oracle of x0ne Core's Qwen3 bf16 decode path (the dense forward, and the Qwen3-MoE block's
 * routing, expert GEMVs and combination). TEST INFRASTRUCTURE, NOT PRODUCT:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.
 *
 * Restates x0ne-core/oracle/src/{bf16,lib,model}.rs operation for operation: f64 inside, the
 * reference's summation orders, bf16 rounding at the engine's points. Build with
 * -ffp-contract=off: the reference (Rust) never fuses a multiply and an add, so neither may
 * this code, or the bits move.
 *
 * Parity pins (see tests/test_oracle_*.py):
 *  - bf16: exhaustive over all 2^32 f32 patterns against torch's RNE cast;
 *  - splitmix64: the reference's known-answer ids (x0ne-infer/src/bench_tests.rs:1072-1081);
 *  - the forward's mathematics: the transformers F32 fixture x0ne-infer/tests/arch/qwen3/
 *    (logits at 1e-4, greedy tokens exact), plus the closed forms of cpu_oracle.rs:315-447;
 *  - the cache: a recompute equals the carried cache, bit for bit (cpu_oracle.rs:502-565).
 */
#include "x0ne_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------------------------ */
/* bf16 (bf16.rs)                                                                               */
/* ------------------------------------------------------------------------------------------ */

static uint32_t f32_bits(float x) {
    uint32_t b;
    memcpy(&b, &x, 4);
    return b;
}

static float f32_of(uint32_t b) {
    float x;
    memcpy(&x, &b, 4);
    return x;
}

/* bf16.rs:11-20: the upper half, plus one when the lower half is above the middle or at it
   with an odd upper half. A NaN keeps its sign and gets the quiet bit 0x0040. */
uint16_t xo_bf16_bits(float x) {
    uint32_t b = f32_bits(x);
    uint32_t hi = b >> 16, lo = b & 0xFFFFu;
    if (x != x) return (uint16_t)(hi | 0x0040u);
    uint32_t up = (lo > 0x8000u) || (lo == 0x8000u && (hi & 1u));
    return (uint16_t)(hi + up);
}

/* bf16.rs:5-7 */
static inline float bf16v(uint16_t b) { return f32_of((uint32_t)b << 16); }
float xo_bf16_value(uint16_t b) { return bf16v(b); }

/* bf16.rs:23-25 */
float xo_bf16_round(float x) { return xo_bf16_value(xo_bf16_bits(x)); }

void xo_bf16_round_all(float* x, size_t n) {
    for (size_t i = 0; i < n; ++i) x[i] = xo_bf16_round(x[i]);
}

void xo_bf16_encode(const float* x, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = xo_bf16_bits(x[i]);
}

void xo_bf16_decode(const uint16_t* b, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = xo_bf16_value(b[i]);
}

/* bf16.rs:48-54 */
double xo_bf16_ulp(float x) {
    uint16_t bits = xo_bf16_bits(fabsf(x));
    if (bits >= 0x7F80u) return INFINITY;
    return (double)xo_bf16_value((uint16_t)(bits + 1)) - (double)xo_bf16_value(bits);
}

/* ------------------------------------------------------------------------------------------ */
/* splitmix64 (oracle/tests/common/mod.rs:8-53)                                                 */
/* ------------------------------------------------------------------------------------------ */

#define GOLDEN 0x9E3779B97F4A7C15ull

static uint64_t fmix(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* common/mod.rs:15-21 */
uint64_t xo_rng_next(uint64_t* state) {
    *state += GOLDEN;
    return fmix(*state);
}

/* common/mod.rs:23-25 */
uint64_t xo_rng_below(uint64_t* state, uint64_t n) { return xo_rng_next(state) % n; }

/* common/mod.rs:37-39: ((next >> 40) / 2^24) * 2 - 1, in f32 (every step exact). */
float xo_rng_unit(uint64_t* state) {
    return ((float)(xo_rng_next(state) >> 40) / (float)(1u << 24)) * 2.0f - 1.0f;
}

/* common/mod.rs:50-52 */
void xo_rng_tokens(uint64_t* state, uint32_t* out, size_t n, uint64_t vocab) {
    for (size_t i = 0; i < n; ++i) out[i] = (uint32_t)xo_rng_below(state, vocab);
}

/* common/mod.rs:44-46 */
void xo_rng_bf16s(uint64_t* state, float* out, size_t n, float scale) {
    for (size_t i = 0; i < n; ++i) out[i] = xo_bf16_round(xo_rng_unit(state) * scale);
}

/* ------------------------------------------------------------------------------------------ */
/* Deterministic N(0, 1): splitmix64 outputs into Box-Muller, log and sin/cos from +,-,*,/.     */
/* The device initialiser (x0ne-engine_amd/csrc/init.hip) repeats this code; both sides are     */
/* compiled without contraction, so the two draw the same bits.                                 */
/* ------------------------------------------------------------------------------------------ */

/* ln x for x > 0 finite and normal: x = m 2^e with m in [sqrt(1/2), sqrt(2)); ln m = 2 atanh(f),
   f = (m - 1) / (m + 1), |f| <= 0.1716, series to f^27 (error below 1e-17 of the result). */
double xo_det_log(double x) {
    uint64_t b;
    memcpy(&b, &x, 8);
    int e = (int)((b >> 52) & 0x7FF) - 1023;
    uint64_t mb = (b & 0x000FFFFFFFFFFFFFull) | 0x3FF0000000000000ull;
    double m;
    memcpy(&m, &mb, 8);
    if (m > 1.4142135623730951) {
        m = m * 0.5;
        e += 1;
    }
    double f = (m - 1.0) / (m + 1.0);
    double f2 = f * f;
    static const double c[14] = {1.0,        1.0 / 3.0,  1.0 / 5.0,  1.0 / 7.0,  1.0 / 9.0,
                                 1.0 / 11.0, 1.0 / 13.0, 1.0 / 15.0, 1.0 / 17.0, 1.0 / 19.0,
                                 1.0 / 21.0, 1.0 / 23.0, 1.0 / 25.0, 1.0 / 27.0};
    double p = c[13];
    for (int k = 12; k >= 0; --k) p = p * f2 + c[k];
    return (double)e * 0.6931471805599453 + 2.0 * f * p;
}

/* sin and cos of 2 pi u for u in [0, 1): quadrant q = floor(4u) (exact), phi = (4u - q) pi/2,
   Taylor series to phi^23 and phi^24 (error below 1e-17 on [0, pi/2)). */
void xo_det_sincos_turn(double u, double* s, double* c) {
    double t = u * 4.0;
    int q = (int)t;
    double r = t - (double)q;
    double phi = r * 1.5707963267948966;
    double p2 = phi * phi;
    static const double sc[12] = {
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
    static const double cc[13] = {
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
    for (int k = 10; k >= 0; --k) ps = ps * p2 + sc[k];
    double S = phi * ps;
    double pc = cc[12];
    for (int k = 11; k >= 0; --k) pc = pc * p2 + cc[k];
    double C = pc;
    switch (q & 3) {
        case 0: *s = S; *c = C; break;
        case 1: *s = C; *c = -S; break;
        case 2: *s = -S; *c = -C; break;
        default: *s = -C; *c = S; break;
    }
}

/* Value i of stream `key`: pair k = i / 2 takes splitmix64 outputs 2k and 2k + 1 of a generator
   seeded with `key`; u1 = (r1 >> 11 + 1) 2^-53 in (0, 1], u2 = (r2 >> 11) 2^-53 in [0, 1);
   value 2k = sqrt(-2 ln u1) cos(2 pi u2), value 2k + 1 = sqrt(-2 ln u1) sin(2 pi u2). */
static void normal_pair(uint64_t key, uint64_t k, double* z0, double* z1) {
    uint64_t r1 = fmix(key + (2 * k + 1) * GOLDEN);
    uint64_t r2 = fmix(key + (2 * k + 2) * GOLDEN);
    double u1 = (double)((r1 >> 11) + 1) * 0x1p-53;
    double u2 = (double)(r2 >> 11) * 0x1p-53;
    double rad = sqrt(-2.0 * xo_det_log(u1));
    double s, c;
    xo_det_sincos_turn(u2, &s, &c);
    *z0 = rad * c;
    *z1 = rad * s;
}

double xo_normal_at(uint64_t key, uint64_t i) {
    double z0, z1;
    normal_pair(key, i >> 1, &z0, &z1);
    return (i & 1) ? z1 : z0;
}

void xo_normal_bf16(uint64_t key, uint64_t first, size_t n, double std_dev, uint16_t* out) {
    size_t j = 0;
    while (j < n) {
        uint64_t i = first + j;
        double z0, z1;
        normal_pair(key, i >> 1, &z0, &z1);
        if ((i & 1) == 0) {
            out[j++] = xo_bf16_bits((float)(std_dev * z0));
            if (j < n) out[j++] = xo_bf16_bits((float)(std_dev * z1));
        } else {
            out[j++] = xo_bf16_bits((float)(std_dev * z1));
        }
    }
}

/* Output `index` of a splitmix64 seeded with `seed`. */
uint64_t xo_tensor_key(uint64_t seed, uint64_t index) { return fmix(seed + (index + 1) * GOLDEN); }

/* ------------------------------------------------------------------------------------------ */
/* Row-parallel thread pool. A task splits [0, n) into contiguous ranges, one per thread.       */
/* ------------------------------------------------------------------------------------------ */

typedef void (*xo_task)(void* arg, size_t begin, size_t end);

static struct {
    pthread_mutex_t mu;
    pthread_cond_t go, done;
    pthread_t tid[256];
    int threads;    /* workers + the caller */
    int started;    /* workers running */
    uint64_t round; /* bumped per task */
    int pending;
    xo_task task;
    void* arg;
    size_t n;
    int stop;
} P = {PTHREAD_MUTEX_INITIALIZER, PTHREAD_COND_INITIALIZER, PTHREAD_COND_INITIALIZER};

static pthread_mutex_t call_mu = PTHREAD_MUTEX_INITIALIZER;

static void range_of(int t, int threads, size_t n, size_t* b, size_t* e) {
    size_t per = (n + (size_t)threads - 1) / (size_t)threads;
    *b = per * (size_t)t;
    *e = *b + per;
    if (*b > n) *b = n;
    if (*e > n) *e = n;
}

/* A worker starts having seen every task posted before it was created (the round set_threads
   hands it), so it never runs a finished task's stale arguments. */
static uint64_t start_round[256];

static void* worker(void* p) {
    int me = (int)(intptr_t)p;
    pthread_mutex_lock(&P.mu);
    uint64_t seen = start_round[me];
    for (;;) {
        while (P.round == seen && !P.stop) pthread_cond_wait(&P.go, &P.mu);
        if (P.stop) break;
        seen = P.round;
        xo_task f = P.task;
        void* arg = P.arg;
        size_t n = P.n;
        int threads = P.threads;
        pthread_mutex_unlock(&P.mu);
        size_t b, e;
        range_of(me, threads, n, &b, &e);
        if (b < e) f(arg, b, e);
        pthread_mutex_lock(&P.mu);
        if (--P.pending == 0) pthread_cond_signal(&P.done);
    }
    pthread_mutex_unlock(&P.mu);
    return NULL;
}

static void pool_stop(void) {
    pthread_mutex_lock(&P.mu);
    P.stop = 1;
    pthread_cond_broadcast(&P.go);
    pthread_mutex_unlock(&P.mu);
    for (int i = 1; i < P.started; ++i) pthread_join(P.tid[i], NULL);
    P.started = 0;
    P.stop = 0;
}

void xo_set_threads(int n) {
    pthread_mutex_lock(&call_mu);
    if (n < 1) n = 1;
    if (n > 256) n = 256;
    if (P.started) pool_stop();
    P.threads = n;
    pthread_mutex_lock(&P.mu);
    for (int i = 1; i < n; ++i) start_round[i] = P.round;
    pthread_mutex_unlock(&P.mu);
    for (int i = 1; i < n; ++i) pthread_create(&P.tid[i], NULL, worker, (void*)(intptr_t)i);
    P.started = n;
    pthread_mutex_unlock(&call_mu);
}

int xo_threads(void) { return P.threads < 1 ? 1 : P.threads; }

static void pool_run(xo_task f, void* arg, size_t n) {
    pthread_mutex_lock(&call_mu);
    int threads = P.threads < 1 ? 1 : P.threads;
    if (threads == 1 || n < 64) {
        if (n) f(arg, 0, n);
        pthread_mutex_unlock(&call_mu);
        return;
    }
    pthread_mutex_lock(&P.mu);
    P.task = f;
    P.arg = arg;
    P.n = n;
    P.pending = threads - 1;
    P.round++;
    pthread_cond_broadcast(&P.go);
    pthread_mutex_unlock(&P.mu);
    size_t b, e;
    range_of(0, threads, n, &b, &e);
    if (b < e) f(arg, b, e);
    pthread_mutex_lock(&P.mu);
    while (P.pending) pthread_cond_wait(&P.done, &P.mu);
    pthread_mutex_unlock(&P.mu);
    pthread_mutex_unlock(&call_mu);
}

/* ------------------------------------------------------------------------------------------ */
/* Kernels (oracle/src/lib.rs)                                                                  */
/* ------------------------------------------------------------------------------------------ */

/* lib.rs:39-46: a token outside the table gives a zero row. */
void xo_embedding(const float* table, size_t vocab, size_t hidden, uint32_t token, float* out) {
    if ((size_t)token >= vocab) {
        for (size_t i = 0; i < hidden; ++i) out[i] = 0.0f;
        return;
    }
    memcpy(out, table + (size_t)token * hidden, hidden * sizeof(float));
}

/* lib.rs:64-67: 1 / sqrt(sum(x^2) / n + eps), the sum a sequential f64 fold. Every sum the
   reference forms with Iterator::sum::<f64>() starts from -0.0, the neutral element of f64's Sum
   in the Rust the reference pins (rust-toolchain.toml: 1.98.1), so a sum of nothing or of
   negative zeros only is -0.0 here too; a sum it folds from an explicit 0f64 starts at +0.0. */
double xo_rms_scale(const float* x, size_t n, float eps) {
    double ss = -0.0;
    for (size_t i = 0; i < n; ++i) ss += (double)x[i] * (double)x[i];
    return 1.0 / sqrt(ss / (double)n + (double)eps);
}

/* lib.rs:50-62: residual += x in f32 (one addition per value), then (r * scale) * w in f64. */
void xo_add_rmsnorm(float* residual, const float* x, const float* w, size_t h, float eps,
                    float* out) {
    for (size_t i = 0; i < h; ++i) residual[i] = residual[i] + x[i];
    double scale = xo_rms_scale(residual, h, eps);
    for (size_t i = 0; i < h; ++i) out[i] = (float)((double)residual[i] * scale * (double)w[i]);
}

/* lib.rs:72-76 */
void xo_inv_freq_f64(size_t head_dim, double theta, double* out) {
    for (size_t i = 0; i < head_dim / 2; ++i)
        out[i] = 1.0 / pow(theta, (double)(2 * i) / (double)head_dim);
}

/* x0ne-core/runtime/src/ops.rs:210-214: 1 / theta^(2i / d) in f32, what the host gives the
   device. Rust's f32::powf is the platform's powf. */
void xo_inv_freq_f32(size_t head_dim, float theta, float* out) {
    for (size_t i = 0; i < head_dim / 2; ++i)
        out[i] = 1.0f / powf(theta, (float)(2 * i) / (float)head_dim);
}

/* ops.rs:217-219 */
float xo_attn_scale(size_t head_dim) { return (float)(1.0 / sqrt((double)head_dim)); }

/* lib.rs:95-110: one head: f64 RMSNorm, then the rotate-half pair (i, i + d/2) turned by
   angle = f32(pos * inv_freq[i]), sin and cos in f64. */
static void rope_head(const float* x, const float* w, const float* inv_freq, size_t hd,
                      uint32_t pos, float eps, float* out) {
    size_t half = hd / 2;
    double scale = xo_rms_scale(x, hd, eps);
    double n[1024];
    for (size_t i = 0; i < hd; ++i) n[i] = (double)x[i] * scale * (double)w[i];
    for (size_t i = 0; i < half; ++i) {
        double angle = (double)((float)pos * inv_freq[i]);
        double s = sin(angle), c = cos(angle);
        out[i] = (float)(n[i] * c - n[i + half] * s);
        out[i + half] = (float)(n[i + half] * c + n[i] * s);
    }
}

/* lib.rs:82-120. q: q_heads * hd, k: kv_heads * hd, v: kv_heads * hd (copied). */
void xo_qk_norm_rope(const float* qkv, const float* q_norm, const float* k_norm,
                     const float* inv_freq, size_t q_heads, size_t kv_heads, size_t hd,
                     uint32_t pos, float eps, float* q, float* k, float* v) {
    size_t qd = q_heads * hd, kvd = kv_heads * hd;
    for (size_t h = 0; h < q_heads; ++h)
        rope_head(qkv + h * hd, q_norm, inv_freq, hd, pos, eps, q + h * hd);
    for (size_t h = 0; h < kv_heads; ++h)
        rope_head(qkv + qd + h * hd, k_norm, inv_freq, hd, pos, eps, k + h * hd);
    memcpy(v, qkv + qd + kvd, kvd * sizeof(float));
}

/* lib.rs:123-133: each row a sequential f64 sum of exact products. Threads split rows; four
   rows are summed side by side (each still in its own order). */
typedef struct {
    const void* w;
    int bf16;
    size_t cols;
    const double* x;
    float* y;
} gemv_job;

static inline double wval(const gemv_job* j, size_t idx) {
    if (j->bf16) return (double)bf16v(((const uint16_t*)j->w)[idx]);
    return (double)((const float*)j->w)[idx];
}

static void gemv_rows(void* p, size_t b, size_t e) {
    const gemv_job* j = (const gemv_job*)p;
    size_t cols = j->cols, r = b;
    const double* x = j->x;
    for (; r + 4 <= e; r += 4) {
        double s0 = -0.0, s1 = -0.0, s2 = -0.0, s3 = -0.0; /* lib.rs:130, .sum::<f64>() */
        if (j->bf16) {
            const uint16_t* w0 = (const uint16_t*)j->w + r * cols;
            const uint16_t* w1 = w0 + cols;
            const uint16_t* w2 = w1 + cols;
            const uint16_t* w3 = w2 + cols;
            for (size_t c = 0; c < cols; ++c) {
                s0 += (double)bf16v(w0[c]) * x[c];
                s1 += (double)bf16v(w1[c]) * x[c];
                s2 += (double)bf16v(w2[c]) * x[c];
                s3 += (double)bf16v(w3[c]) * x[c];
            }
        } else {
            const float* w0 = (const float*)j->w + r * cols;
            const float* w1 = w0 + cols;
            const float* w2 = w1 + cols;
            const float* w3 = w2 + cols;
            for (size_t c = 0; c < cols; ++c) {
                s0 += (double)w0[c] * x[c];
                s1 += (double)w1[c] * x[c];
                s2 += (double)w2[c] * x[c];
                s3 += (double)w3[c] * x[c];
            }
        }
        j->y[r] = (float)s0;
        j->y[r + 1] = (float)s1;
        j->y[r + 2] = (float)s2;
        j->y[r + 3] = (float)s3;
    }
    for (; r < e; ++r) {
        double s = -0.0;
        for (size_t c = 0; c < cols; ++c) s += wval(j, r * cols + c) * x[c];
        j->y[r] = (float)s;
    }
}

static void gemv_any(const void* w, int bf16, size_t rows, size_t cols, const float* x,
                     float* y) {
    double* xd = (double*)malloc(cols * sizeof(double));
    for (size_t c = 0; c < cols; ++c) xd[c] = (double)x[c];
    gemv_job j = {w, bf16, cols, xd, y};
    pool_run(gemv_rows, &j, rows);
    free(xd);
}

void xo_gemv(const float* w, size_t rows, size_t cols, const float* x, float* y) {
    gemv_any(w, 0, rows, cols, x, y);
}

void xo_gemv_bf16w(const uint16_t* w, size_t rows, size_t cols, const float* x, float* y) {
    gemv_any(w, 1, rows, cols, x, y);
}

/* lib.rs:136-146 */
void xo_gemv_magnitude(const float* w, size_t rows, size_t cols, const float* x, double* y) {
    for (size_t r = 0; r < rows; ++r) {
        double s = -0.0;
        for (size_t c = 0; c < cols; ++c) s += fabs((double)w[r * cols + c] * (double)x[c]);
        y[r] = s;
    }
}

/* lib.rs:150-174: scores q.k_j / sqrt(d) in f64, max subtracted, weights exp(s - m), l their
   sum, out = sum_j p_j v_j / l; every sum sequential over j. */
static void attend(const float* q, const float* k, const float* v, size_t keys, size_t kh,
                   size_t hd, size_t kvd, double* scores, double* acc, float* out) {
    double scale = 1.0 / sqrt((double)hd);
    double m = -INFINITY;
    for (size_t j = 0; j < keys; ++j) {
        const float* kr = k + j * kvd + kh * hd;
        double d = -0.0; /* lib.rs:160, .sum::<f64>() */
        for (size_t i = 0; i < hd; ++i) d += (double)q[i] * (double)kr[i];
        scores[j] = d * scale;
        /* f64::max: a NaN operand gives the other one */
        if (scores[j] > m || m != m) m = (scores[j] != scores[j]) ? m : scores[j];
    }
    double l = -0.0;                              /* lib.rs:166, .sum() */
    for (size_t i = 0; i < hd; ++i) acc[i] = 0.0; /* lib.rs:167, vec![0f64; hd] */
    for (size_t j = 0; j < keys; ++j) {
        double p = exp(scores[j] - m);
        scores[j] = p;
        l += p;
    }
    for (size_t j = 0; j < keys; ++j) {
        const float* vr = v + j * kvd + kh * hd;
        for (size_t i = 0; i < hd; ++i) acc[i] += scores[j] * (double)vr[i];
    }
    for (size_t i = 0; i < hd; ++i) out[i] = (float)(acc[i] / l);
}

/* lib.rs:178-185: q head h reads kv head h / (q_heads / kv_heads); cache [pos][kv_heads][hd]. */
void xo_attention_decode(const float* q, const float* k, const float* v, size_t ctx,
                         size_t q_heads, size_t kv_heads, size_t hd, float* out) {
    size_t kvd = kv_heads * hd, group = q_heads / kv_heads;
    double* scores = (double*)malloc((ctx ? ctx : 1) * sizeof(double));
    double* acc = (double*)malloc(hd * sizeof(double));
    for (size_t h = 0; h < q_heads; ++h)
        attend(q + h * hd, k, v, ctx, h / group, hd, kvd, scores, acc, out + h * hd);
    free(scores);
    free(acc);
}

/* lib.rs:205-214: g / (1 + e^-g) * u in f64. */
void xo_swiglu(const float* gate_up, size_t inter, float* out) {
    for (size_t i = 0; i < inter; ++i) {
        double g = (double)gate_up[i], u = (double)gate_up[inter + i];
        out[i] = (float)(g / (1.0 + exp(-g)) * u);
    }
}

/* lib.rs:254-282: routing of `rows` rows of `experts` router logits: per row the top_k experts,
   larger logit first then the smaller index (-0.0 equals 0.0), and exp(l_e - l_max) renormalised
   over the chosen in f64, rounded once to f32; a row with a non-finite logit gets
   XO_MOE_NO_EXPERT and NaN. The selection is a stable order of the indices by decreasing logit
   (the reference sorts stably), done here by repeated extraction of the best remaining. */
void xo_moe_route(const float* logits, size_t rows, size_t experts, size_t top_k, uint32_t* ids, float* weights) {
    unsigned char* taken = (unsigned char*)calloc(experts ? experts : 1, 1);
    for (size_t r = 0; r < rows; ++r) {
        const float* row = logits + r * experts;
        uint32_t* ri = ids + r * top_k;
        float* rw = weights + r * top_k;
        int bad = 0;
        for (size_t i = 0; i < experts; ++i) bad |= !isfinite(row[i]);
        if (bad) {
            for (size_t s = 0; s < top_k; ++s) {
                ri[s] = XO_MOE_NO_EXPERT;
                rw[s] = NAN;
            }
            continue;
        }
        memset(taken, 0, experts);
        for (size_t s = 0; s < top_k; ++s) {
            size_t best = experts;
            for (size_t i = 0; i < experts; ++i)
                if (!taken[i] && (best == experts || row[i] > row[best])) best = i;
            taken[best] = 1;
            ri[s] = (uint32_t)best;
        }
        const double m = (double)row[ri[0]];
        double e[64], sum = -0.0;
        for (size_t s = 0; s < top_k; ++s) {
            e[s] = exp((double)row[ri[s]] - m);
            sum += e[s];
        }
        for (size_t s = 0; s < top_k; ++s) rw[s] = (float)(e[s] / sum);
    }
    free(taken);
}

/* lib.rs:284-312: y[s] = W[ids[s]] x[s / x_group] for W [experts][rows][cols] (bf16 values as
   f32) and x [slots / x_group][cols]; an id outside the experts gives a NaN row. */
void xo_moe_gemv(const float* w, size_t experts, size_t rows, size_t cols, const uint32_t* ids, size_t slots,
                 const float* x, size_t x_group, float* y) {
    for (size_t s = 0; s < slots; ++s) {
        float* ys = y + s * rows;
        if ((size_t)ids[s] >= experts) {
            for (size_t r = 0; r < rows; ++r) ys[r] = NAN;
            continue;
        }
        gemv_any(w + (size_t)ids[s] * rows * cols, 0, rows, cols, x + (s / x_group) * cols, ys);
    }
}

/* lib.rs:314-329: out[r][i] = sum_s weights[r][s] y[r][s][i] in f64, in slot order, rounded once. */
void xo_moe_combine(const float* y, const float* weights, size_t rows, size_t hidden, size_t top_k, float* out) {
    for (size_t r = 0; r < rows; ++r)
        for (size_t i = 0; i < hidden; ++i) {
            double acc = -0.0;
            for (size_t s = 0; s < top_k; ++s) acc += (double)weights[r * top_k + s] * (double)y[(r * top_k + s) * hidden + i];
            out[r * hidden + i] = (float)acc;
        }
}

/* lib.rs:218-230: the first index of the largest value; none for an empty row or a NaN. */
int64_t xo_argmax(const float* x, size_t n) {
    int64_t best = -1;
    for (size_t i = 0; i < n; ++i) {
        if (x[i] != x[i]) return -1;
        if (best < 0 || !(x[best] >= x[i])) best = (int64_t)i;
    }
    return best;
}

/* lib.rs:233-239 */
double xo_logsumexp(const float* x, size_t n) {
    double m = -INFINITY;
    for (size_t i = 0; i < n; ++i) {
        double v = (double)x[i];
        if (v > m || m != m) m = (v != v) ? m : v;
    }
    if (!isfinite(m)) return m;
    double s = -0.0;
    for (size_t i = 0; i < n; ++i) s += exp((double)x[i] - m);
    return m + log(s);
}

/* lib.rs:242-252 */
double xo_kl(const float* p, const float* q, size_t n) {
    double lp = xo_logsumexp(p, n), lq = xo_logsumexp(q, n);
    double s = -0.0;
    for (size_t i = 0; i < n; ++i) {
        double a = (double)p[i] - lp, b = (double)q[i] - lq;
        s += exp(a) * (a - b);
    }
    return s;
}

/* ------------------------------------------------------------------------------------------ */
/* The forward (oracle/src/model.rs)                                                            */
/* ------------------------------------------------------------------------------------------ */

enum { T_INPUT_NORM, T_Q, T_K, T_V, T_QN, T_KN, T_O, T_POST_NORM, T_GATE, T_UP, T_DOWN, T_PER };

typedef struct {
    void* t[T_PER];
} xo_layer;

struct xo_model {
    xo_config c;
    int bf16;
    void* embed;
    xo_layer* layers;
    void* final_norm;
    void* lm_head;
    float* inv_freq;
    /* cache: per layer K and V, [pos][kv_dim] f32 values */
    float** k;
    float** v;
    size_t len, cap;
    /* scratch */
    float *delta, *residual, *normed, *qkv, *q, *kr, *vr, *attn, *gate_up, *act;
    double *scores, *acc;
    size_t scores_cap;
};

static size_t qdim(const xo_config* c) { return (size_t)c->q_heads * c->head_dim; }
static size_t kvdim(const xo_config* c) { return (size_t)c->kv_heads * c->head_dim; }

size_t xo_tensor_count(const xo_config* c) {
    return 1 + (size_t)c->layers * T_PER + 1 + (c->tied ? 0 : 1);
}

/* model.rs:63-89: names and element counts, in the checkpoint's order. */
size_t xo_tensor_info(const xo_config* c, size_t index, char* name, size_t len) {
    size_t h = c->hidden, in = c->inter, hd = c->head_dim, qd = qdim(c), kvd = kvdim(c);
    size_t n = 0;
    char buf[128];
    if (index == 0) {
        snprintf(buf, sizeof buf, "model.embed_tokens.weight");
        n = (size_t)c->vocab * h;
    } else if (index <= (size_t)c->layers * T_PER) {
        size_t l = (index - 1) / T_PER, t = (index - 1) % T_PER;
        static const char* leaf[T_PER] = {
            "input_layernorm",        "self_attn.q_proj", "self_attn.k_proj",
            "self_attn.v_proj",       "self_attn.q_norm", "self_attn.k_norm",
            "self_attn.o_proj",       "post_attention_layernorm",
            "mlp.gate_proj",          "mlp.up_proj",      "mlp.down_proj"};
        size_t sizes[T_PER] = {h, qd * h, kvd * h, kvd * h, hd, hd, h * qd, h, in * h, in * h, h * in};
        snprintf(buf, sizeof buf, "model.layers.%zu.%s.weight", l, leaf[t]);
        n = sizes[t];
    } else if (index == (size_t)c->layers * T_PER + 1) {
        snprintf(buf, sizeof buf, "model.norm.weight");
        n = h;
    } else if (!c->tied && index == (size_t)c->layers * T_PER + 2) {
        snprintf(buf, sizeof buf, "lm_head.weight");
        n = (size_t)c->vocab * h;
    } else {
        buf[0] = 0;
        n = 0;
    }
    if (name && len) {
        strncpy(name, buf, len - 1);
        name[len - 1] = 0;
    }
    return n;
}

static void** tensor_slot(xo_model* m, size_t index) {
    const xo_config* c = &m->c;
    if (index == 0) return &m->embed;
    if (index <= (size_t)c->layers * T_PER) {
        size_t l = (index - 1) / T_PER, t = (index - 1) % T_PER;
        return &m->layers[l].t[t];
    }
    if (index == (size_t)c->layers * T_PER + 1) return &m->final_norm;
    if (!c->tied && index == (size_t)c->layers * T_PER + 2) return &m->lm_head;
    return NULL;
}

xo_model* xo_model_new(const xo_config* c, const float* inv_freq, int weights_bf16) {
    if (!c->hidden || !c->layers || !c->q_heads || !c->kv_heads || !c->head_dim || !c->vocab ||
        c->q_heads % c->kv_heads || c->head_dim % 2 || c->head_dim > 1024)
        return NULL;
    xo_model* m = (xo_model*)calloc(1, sizeof(xo_model));
    m->c = *c;
    m->bf16 = weights_bf16 ? 1 : 0;
    size_t es = m->bf16 ? 2 : 4;
    m->layers = (xo_layer*)calloc(c->layers, sizeof(xo_layer));
    size_t count = xo_tensor_count(c);
    for (size_t i = 0; i < count; ++i) {
        size_t n = xo_tensor_info(c, i, NULL, 0);
        void* p = calloc(n, es);
        if (!p) {
            xo_model_free(m);
            return NULL;
        }
        *tensor_slot(m, i) = p;
    }
    m->inv_freq = (float*)malloc(c->head_dim / 2 * sizeof(float));
    memcpy(m->inv_freq, inv_freq, c->head_dim / 2 * sizeof(float));
    m->k = (float**)calloc(c->layers, sizeof(float*));
    m->v = (float**)calloc(c->layers, sizeof(float*));
    size_t h = c->hidden, qd = qdim(c), kvd = kvdim(c), in = c->inter;
    m->delta = (float*)calloc(h, 4);
    m->residual = (float*)calloc(h, 4);
    m->normed = (float*)calloc(h, 4);
    m->qkv = (float*)calloc(qd + 2 * kvd, 4);
    m->q = (float*)calloc(qd, 4);
    m->kr = (float*)calloc(kvd, 4);
    m->vr = (float*)calloc(kvd, 4);
    m->attn = (float*)calloc(qd, 4);
    m->gate_up = (float*)calloc(2 * in, 4);
    m->act = (float*)calloc(in, 4);
    m->acc = (double*)calloc(c->head_dim, 8);
    return m;
}

void xo_model_free(xo_model* m) {
    if (!m) return;
    size_t count = xo_tensor_count(&m->c);
    for (size_t i = 0; i < count; ++i) {
        void** s = tensor_slot(m, i);
        if (s) free(*s);
    }
    for (size_t l = 0; l < m->c.layers && m->k; ++l) {
        free(m->k[l]);
        free(m->v[l]);
    }
    free(m->k);
    free(m->v);
    free(m->layers);
    free(m->inv_freq);
    free(m->delta);
    free(m->residual);
    free(m->normed);
    free(m->qkv);
    free(m->q);
    free(m->kr);
    free(m->vr);
    free(m->attn);
    free(m->gate_up);
    free(m->act);
    free(m->scores);
    free(m->acc);
    free(m);
}

int xo_model_set(xo_model* m, size_t index, size_t at, const void* data, size_t n) {
    if (index >= xo_tensor_count(&m->c)) return -1;
    size_t total = xo_tensor_info(&m->c, index, NULL, 0);
    if (at > total || n > total - at) return -1;
    size_t es = m->bf16 ? 2 : 4;
    memcpy((char*)*tensor_slot(m, index) + at * es, data, n * es);
    return 0;
}

static int is_norm(size_t index, const xo_config* c) {
    if (index == 0) return 0;
    if (index == (size_t)c->layers * T_PER + 1) return 1;
    if (index > (size_t)c->layers * T_PER) return 0;
    size_t t = (index - 1) % T_PER;
    return t == T_INPUT_NORM || t == T_POST_NORM || t == T_QN || t == T_KN;
}

typedef struct {
    uint16_t* out;
    uint64_t key;
    double std_dev;
} normal_job;

static void normal_rows(void* p, size_t b, size_t e) {
    normal_job* j = (normal_job*)p;
    /* ranges of 4096 values */
    for (size_t r = b; r < e; ++r) xo_normal_bf16(j->key, r * 4096, 4096, j->std_dev, j->out + r * 4096);
}

int xo_model_init_normal(xo_model* m, uint64_t seed, double std_dev) {
    if (!m->bf16) return -1;
    size_t count = xo_tensor_count(&m->c);
    for (size_t i = 0; i < count; ++i) {
        size_t n = xo_tensor_info(&m->c, i, NULL, 0);
        uint16_t* t = (uint16_t*)*tensor_slot(m, i);
        if (is_norm(i, &m->c)) {
            for (size_t j = 0; j < n; ++j) t[j] = 0x3F80; /* 1.0 */
            continue;
        }
        uint64_t key = xo_tensor_key(seed, i);
        normal_job j = {t, key, std_dev};
        size_t full = n / 4096;
        pool_run(normal_rows, &j, full);
        if (n % 4096) xo_normal_bf16(key, full * 4096, n % 4096, std_dev, t + full * 4096);
    }
    return 0;
}

/* common/mod.rs:199-221: norms bf16(1 + 0.25 unit), embedding and lm_head bf16(unit), the
   projections bf16(unit * 2 / sqrt(fan_in)), one splitmix64 stream in checkpoint order. */
int xo_model_init_reference(xo_model* m, uint64_t seed) {
    uint64_t st = seed;
    size_t count = xo_tensor_count(&m->c);
    for (size_t i = 0; i < count; ++i) {
        char name[128];
        size_t n = xo_tensor_info(&m->c, i, name, sizeof name);
        float* vals = (float*)malloc(n * sizeof(float));
        int vector = 0;
        size_t fan_in = 0;
        if (i == 0 || strstr(name, "lm_head")) {
            xo_rng_bf16s(&st, vals, n, 1.0f);
        } else {
            if (is_norm(i, &m->c)) vector = 1;
            if (vector) {
                for (size_t j = 0; j < n; ++j) vals[j] = xo_bf16_round(1.0f + 0.25f * xo_rng_unit(&st));
            } else {
                size_t t = (i - 1) % T_PER;
                const xo_config* c = &m->c;
                fan_in = (t == T_O) ? qdim(c) : (t == T_DOWN) ? c->inter : c->hidden;
                xo_rng_bf16s(&st, vals, n, 2.0f / sqrtf((float)fan_in));
            }
        }
        if (m->bf16) {
            uint16_t* t = (uint16_t*)*tensor_slot(m, i);
            xo_bf16_encode(vals, t, n);
        } else {
            memcpy(*tensor_slot(m, i), vals, n * sizeof(float));
        }
        free(vals);
    }
    return 0;
}

void xo_model_reset(xo_model* m) { m->len = 0; }
size_t xo_model_len(const xo_model* m) { return m->len; }
void xo_model_truncate(xo_model* m, size_t len) {
    if (len < m->len) m->len = len;
}

int xo_model_cache_row(const xo_model* m, size_t layer, size_t pos, float* k, float* v) {
    if (layer >= m->c.layers || pos >= m->len) return -1;
    size_t kvd = kvdim(&m->c);
    memcpy(k, m->k[layer] + pos * kvd, kvd * 4);
    memcpy(v, m->v[layer] + pos * kvd, kvd * 4);
    return 0;
}

/* A vector tensor (norm weights) as f32. */
static void vec_f32(const xo_model* m, const void* t, size_t n, float* out) {
    if (m->bf16)
        xo_bf16_decode((const uint16_t*)t, out, n);
    else
        memcpy(out, t, n * 4);
}

static void gemv_w(const xo_model* m, const void* w, size_t rows, size_t cols, const float* x,
                   float* y) {
    gemv_any(w, m->bf16, rows, cols, x, y);
}

static void maybe_round(const xo_model* m, float* x, size_t n) {
    if (m->c.round_bf16) xo_bf16_round_all(x, n);
}

/* A packed pair of weight matrices [a; b] the reference builds (model.rs:160-167) is two
   GEMVs here, rows of a then rows of b: the same sums. */
static void gemv2(const xo_model* m, const void* a, size_t ra, const void* b, size_t rb,
                  size_t cols, const float* x, float* y) {
    gemv_w(m, a, ra, cols, x, y);
    gemv_w(m, b, rb, cols, x, y + ra);
}

static void reserve(xo_model* m, size_t need) {
    if (need <= m->cap) return;
    size_t cap = m->cap ? m->cap : 64;
    while (cap < need) cap *= 2;
    size_t kvd = kvdim(&m->c);
    for (size_t l = 0; l < m->c.layers; ++l) {
        m->k[l] = (float*)realloc(m->k[l], cap * kvd * 4);
        m->v[l] = (float*)realloc(m->v[l], cap * kvd * 4);
    }
    m->cap = cap;
    free(m->scores);
    m->scores = (double*)malloc(cap * sizeof(double));
}

/* model.rs:196-262: one token at position len. */
int xo_model_step(xo_model* m, uint32_t token, float* logits) {
    const xo_config* c = &m->c;
    size_t h = c->hidden, hd = c->head_dim, qd = qdim(c), kvd = kvdim(c), in = c->inter;
    size_t pos = m->len;
    if (c->max_pos && pos >= c->max_pos) return -1;
    reserve(m, pos + 1);
    float* w1 = (float*)malloc((h > 2 * hd ? h : 2 * hd) * sizeof(float));
    float* w2 = (float*)malloc(hd * sizeof(float));
    /* embedding (lib.rs:39) */
    if ((size_t)token >= c->vocab) {
        for (size_t i = 0; i < h; ++i) m->delta[i] = 0.0f;
    } else if (m->bf16) {
        xo_bf16_decode((const uint16_t*)m->embed + (size_t)token * h, m->delta, h);
    } else {
        memcpy(m->delta, (const float*)m->embed + (size_t)token * h, h * 4);
    }
    for (size_t i = 0; i < h; ++i) m->residual[i] = 0.0f;
    size_t group = c->q_heads / c->kv_heads;
    for (size_t l = 0; l < c->layers; ++l) {
        xo_layer* L = &m->layers[l];
        vec_f32(m, L->t[T_INPUT_NORM], h, w1);
        xo_add_rmsnorm(m->residual, m->delta, w1, h, c->eps, m->normed);
        maybe_round(m, m->normed, h);
        gemv_w(m, L->t[T_Q], qd, h, m->normed, m->qkv);
        gemv2(m, L->t[T_K], kvd, L->t[T_V], kvd, h, m->normed, m->qkv + qd);
        maybe_round(m, m->qkv, qd + 2 * kvd);
        float* qn = w1;
        float* kn = w1 + hd;
        vec_f32(m, L->t[T_QN], hd, qn);
        vec_f32(m, L->t[T_KN], hd, kn);
        xo_qk_norm_rope(m->qkv, qn, kn, m->inv_freq, c->q_heads, c->kv_heads, hd, (uint32_t)pos,
                        c->eps, m->q, m->kr, m->vr);
        maybe_round(m, m->kr, kvd);
        memcpy(m->k[l] + pos * kvd, m->kr, kvd * 4);
        memcpy(m->v[l] + pos * kvd, m->vr, kvd * 4);
        maybe_round(m, m->q, qd);
        for (size_t hh = 0; hh < c->q_heads; ++hh)
            attend(m->q + hh * hd, m->k[l], m->v[l], pos + 1, hh / group, hd, kvd, m->scores,
                   m->acc, m->attn + hh * hd);
        maybe_round(m, m->attn, qd);
        gemv_w(m, L->t[T_O], h, qd, m->attn, m->delta);
        maybe_round(m, m->delta, h);
        vec_f32(m, L->t[T_POST_NORM], h, w1);
        xo_add_rmsnorm(m->residual, m->delta, w1, h, c->eps, m->normed);
        maybe_round(m, m->normed, h);
        gemv2(m, L->t[T_GATE], in, L->t[T_UP], in, h, m->normed, m->gate_up);
        maybe_round(m, m->gate_up, 2 * in);
        xo_swiglu(m->gate_up, in, m->act);
        maybe_round(m, m->act, in);
        gemv_w(m, L->t[T_DOWN], h, in, m->act, m->delta);
        maybe_round(m, m->delta, h);
    }
    m->len = pos + 1;
    vec_f32(m, m->final_norm, h, w1);
    xo_add_rmsnorm(m->residual, m->delta, w1, h, c->eps, m->normed);
    maybe_round(m, m->normed, h);
    gemv_w(m, c->tied ? m->embed : m->lm_head, c->vocab, h, m->normed, logits);
    free(w1);
    free(w2);
    return 0;
}

size_t xo_model_greedy(xo_model* m, const uint32_t* prompt, size_t n_prompt, size_t n,
                       uint32_t* out, float* margins) {
    float* logits = (float*)malloc((size_t)m->c.vocab * sizeof(float));
    size_t got = 0;
    for (size_t i = 0; i < n_prompt; ++i)
        if (xo_model_step(m, prompt[i], logits)) goto done;
    for (size_t i = 0; i < n; ++i) {
        int64_t t = xo_argmax(logits, m->c.vocab);
        if (t < 0) break;
        float first = logits[t], second = -INFINITY;
        for (size_t j = 0; j < m->c.vocab; ++j)
            if ((int64_t)j != t && logits[j] > second) second = logits[j];
        out[got] = (uint32_t)t;
        if (margins) margins[got] = first - second;
        got++;
        if (i + 1 < n && xo_model_step(m, (uint32_t)t, logits)) break;
    }
done:
    free(logits);
    return got;
}
