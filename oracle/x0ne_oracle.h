/*
 * CPU oracle of x0ne Core's Qwen3 dense bf16 decode path.
 *
 * TEST INFRASTRUCTURE, NOT PRODUCT. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load this library, and only as the checker (or, for cpu_baseline, as the
 * CPU path timed beside the GPU). The GPU product path never links or calls it.
 *
 * A restatement in C of the reference's Rust oracle (x0ne-core/oracle/src/{bf16,lib,model}.rs):
 * plain loops, f64 inside, bf16 rounding (nearest, ties to even) at the points where the engine
 * stores bf16, the residual stream in f32, the logits in f32. Each function names the reference
 * lines it follows. Summation orders are the reference's (sequential left folds), so a result
 * does not depend on the number of threads: threads split rows, never a sum.
 *
 * Two additions of this build, not in the reference:
 *  - a counter-based N(0, std) weight generator (splitmix64 + Box-Muller, with log and sin/cos
 *    written here from +, -, *, / only), whose code the device initialiser repeats operation
 *    for operation, so the host and the device draw the same bf16 weights;
 *  - a row-parallel thread pool (xo_set_threads), used by the GEMVs.
 */
#ifndef X0NE_ORACLE_H
#define X0NE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- bf16 (x0ne-core/oracle/src/bf16.rs) ---- */
uint16_t xo_bf16_bits(float x);  /* bf16.rs:11-20: RNE, NaN -> hi | 0x0040 */
float xo_bf16_value(uint16_t b); /* bf16.rs:5-7 */
float xo_bf16_round(float x);    /* bf16.rs:23-25 */
void xo_bf16_round_all(float* x, size_t n);
void xo_bf16_encode(const float* x, uint16_t* out, size_t n);
void xo_bf16_decode(const uint16_t* b, float* out, size_t n);
double xo_bf16_ulp(float x); /* bf16.rs:48-54 */

/* ---- splitmix64 (x0ne-core/oracle/tests/common/mod.rs:8-53) ---- */
uint64_t xo_rng_next(uint64_t* state);
uint64_t xo_rng_below(uint64_t* state, uint64_t n);
float xo_rng_unit(uint64_t* state); /* uniform in [-1, 1) */
void xo_rng_tokens(uint64_t* state, uint32_t* out, size_t n, uint64_t vocab);
/* n values of bf16(unit * scale), as f32 (common/mod.rs:44-46) */
void xo_rng_bf16s(uint64_t* state, float* out, size_t n, float scale);

/* ---- deterministic normal generator (this build) ---- */
double xo_det_log(double x);
void xo_det_sincos_turn(double u, double* s, double* c); /* sin, cos of 2 pi u, u in [0, 1) */
/* Element i of the stream `key`: value index i of N(0, 1) pairs, see the .c file. */
double xo_normal_at(uint64_t key, uint64_t i);
/* bf16 bits of std * N(0,1), elements first..first+n of stream `key`. */
void xo_normal_bf16(uint64_t key, uint64_t first, size_t n, double std_dev, uint16_t* out);
/* The stream key of tensor number `index` (checkpoint order) under `seed`. */
uint64_t xo_tensor_key(uint64_t seed, uint64_t index);

/* ---- threads ---- */
void xo_set_threads(int n);
int xo_threads(void);

/* ---- kernels (x0ne-core/oracle/src/lib.rs) ---- */
void xo_embedding(const float* table, size_t vocab, size_t hidden, uint32_t token, float* out);
void xo_add_rmsnorm(float* residual, const float* x, const float* w, size_t h, float eps,
                    float* out);
double xo_rms_scale(const float* x, size_t n, float eps);
void xo_inv_freq_f64(size_t head_dim, double theta, double* out);
void xo_inv_freq_f32(size_t head_dim, float theta, float* out);
float xo_attn_scale(size_t head_dim);
void xo_qk_norm_rope(const float* qkv, const float* q_norm, const float* k_norm,
                     const float* inv_freq, size_t q_heads, size_t kv_heads, size_t head_dim,
                     uint32_t pos, float eps, float* q, float* k, float* v);
void xo_gemv(const float* w, size_t rows, size_t cols, const float* x, float* y);
void xo_gemv_bf16w(const uint16_t* w, size_t rows, size_t cols, const float* x, float* y);
void xo_gemv_magnitude(const float* w, size_t rows, size_t cols, const float* x, double* y);
void xo_attention_decode(const float* q, const float* k, const float* v, size_t ctx,
                         size_t q_heads, size_t kv_heads, size_t head_dim, float* out);
void xo_swiglu(const float* gate_up, size_t inter, float* out);
/* GM1, Qwen3-MoE (lib.rs:254-329). */
#define XO_MOE_NO_EXPERT 0xFFFFFFFFu
void xo_moe_route(const float* logits, size_t rows, size_t experts, size_t top_k, uint32_t* ids, float* weights);
void xo_moe_gemv(const float* w, size_t experts, size_t rows, size_t cols, const uint32_t* ids, size_t slots,
                 const float* x, size_t x_group, float* y);
void xo_moe_combine(const float* y, const float* weights, size_t rows, size_t hidden, size_t top_k, float* out);
int64_t xo_argmax(const float* x, size_t n); /* -1: empty or a NaN */
double xo_logsumexp(const float* x, size_t n);
double xo_kl(const float* p, const float* q, size_t n);

/* ---- the forward (x0ne-core/oracle/src/model.rs) ---- */
typedef struct {
    uint32_t hidden, inter, layers, q_heads, kv_heads, head_dim, vocab, max_pos;
    float eps;
    uint32_t tied;
    /* 1: round to bf16 at the engine's points (model.rs:209-261); 0: plain f32 (for the
       transformers F32 fixture, whose arithmetic stores f32 everywhere). */
    uint32_t round_bf16;
} xo_config;

typedef struct xo_model xo_model;

/* A model whose weights are bf16 bit patterns (weights_bf16 = 1) or f32 values. Tensor
   `index` follows model.rs:63-89: embed, then per layer input_norm, q, k, v, q_norm, k_norm, o,
   post_norm, gate, up, down, then the final norm, then lm_head when untied. */
xo_model* xo_model_new(const xo_config* c, const float* inv_freq, int weights_bf16);
void xo_model_free(xo_model* m);
size_t xo_tensor_count(const xo_config* c);
/* Element count of tensor `index`, its name into name_buf. */
size_t xo_tensor_info(const xo_config* c, size_t index, char* name_buf, size_t name_len);
/* Copies n elements (bf16 bits or f32, by the model's kind) into tensor `index` at `at`. */
int xo_model_set(xo_model* m, size_t index, size_t at, const void* data, size_t n);
/* Draws every projection and the embedding (and lm_head) as N(0, std) bf16 from `seed`,
   norm weights 1.0. Only for bf16 models. */
int xo_model_init_normal(xo_model* m, uint64_t seed, double std_dev);
/* Draws the reference tests' init (common/mod.rs:199-221) from one splitmix64 stream. */
int xo_model_init_reference(xo_model* m, uint64_t seed);

/* Cache handling: the model keeps one cache. */
void xo_model_reset(xo_model* m);
size_t xo_model_len(const xo_model* m);
void xo_model_truncate(xo_model* m, size_t len);
/* Feeds `token` at position len: writes K/V and returns the f32 logits (vocab values). */
int xo_model_step(xo_model* m, uint32_t token, float* logits);
/* K, V rows of layer l at position p (kv_dim values each). */
int xo_model_cache_row(const xo_model* m, size_t layer, size_t pos, float* k, float* v);
/* Greedy: feeds prompt, then n tokens, each the argmax of the last logits (the first from the
   prompt). out[i]: token i; margins[i]: top-1 minus top-2 logit of the row that chose it.
   Returns tokens produced (< n when a row has a NaN). */
size_t xo_model_greedy(xo_model* m, const uint32_t* prompt, size_t n_prompt, size_t n,
                       uint32_t* out, float* margins);

#ifdef __cplusplus
}
#endif
#endif
