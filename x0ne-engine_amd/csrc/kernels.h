// The kernel ABI of this library (the analogue of x0ne-core/kernels/cuda/x0ne_kernels.h): C
// linkage, row-major bf16, f32 accumulation, positions and token ids read from device memory,
// bounds checked without trap. KV planes are paged: [pages][kv_heads][16][128] bf16 with a
// page table mapping position / 16 to a physical page. Launch shapes are documented at each
// definition (attention.hip, norm.hip, gemv.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef uint16_t bf16_t;

extern "C" {
__global__ void x0ne_probe_iota_u32(uint32_t* out, uint32_t n);
__global__ void x0ne_probe_bf16_round(uint32_t base, uint32_t n, bf16_t* out, uint32_t* counter);
__global__ void x0ne_embedding_bf16(const bf16_t* table, const uint32_t* tokens, bf16_t* out, uint32_t hidden,
                                    uint32_t vocab);
__global__ void x0ne_add_rmsnorm_bf16(float* residual, const bf16_t* x, const bf16_t* w, bf16_t* out,
                                      uint32_t hidden, float eps);
__global__ void x0ne_qk_norm_rope_kv_write_bf16(const bf16_t* qkv, const bf16_t* q_norm, const bf16_t* k_norm,
                                                const float* inv_freq, bf16_t* q_out, bf16_t* k_cache,
                                                bf16_t* v_cache, const uint32_t* pages, const uint32_t* pos0,
                                                uint32_t q_heads, uint32_t kv_heads, uint32_t max_ctx, float eps);
__global__ void x0ne_qk_norm_rope_kv_write_rows_bf16(const bf16_t* qkv, const bf16_t* q_norm, const bf16_t* k_norm,
                                                     const double* cs, bf16_t* q_out, bf16_t* k_cache,
                                                     bf16_t* v_cache, const uint32_t* pages, const uint32_t* pos0,
                                                     uint32_t q_heads, uint32_t kv_heads, uint32_t max_ctx, float eps);
__global__ void x0ne_attention_decode_bf16(const bf16_t* q, const bf16_t* k_cache, const bf16_t* v_cache,
                                           const uint32_t* pages, bf16_t* out, const uint32_t* pos, uint32_t q_heads,
                                           uint32_t kv_heads, uint32_t max_ctx, float scale);
__global__ void x0ne_attention_decode_split_bf16(const bf16_t* q, const bf16_t* k_cache, const bf16_t* v_cache,
                                                 const uint32_t* pages, float* state, bf16_t* out, const uint32_t* pos,
                                                 uint32_t q_heads, uint32_t kv_heads, uint32_t max_ctx,
                                                 uint32_t splits, float scale);
#define X0NE_DECLARE_SPLIT_GROUP(G)                                                                              \
    __global__ void x0ne_attention_decode_split_g##G##_bf16(                                                    \
        const bf16_t* q, const bf16_t* k_cache, const bf16_t* v_cache, const uint32_t* pages, float* state,     \
        uint32_t* counter, bf16_t* out, const uint32_t* pos, uint32_t q_heads, uint32_t kv_heads, uint32_t max_ctx, \
        uint32_t splits, float scale);                                                                            \
    __global__ void x0ne_attention_rope_decode_g##G##_bf16(                                                     \
        const bf16_t* qkv, const bf16_t* q_norm, const bf16_t* k_norm, const float* inv_freq,                    \
        const double* rope_cs, bf16_t* k_cache, bf16_t* v_cache, const uint32_t* pages, float* state,           \
        uint32_t* counter, bf16_t* out, const uint32_t* pos, uint32_t q_heads, uint32_t kv_heads,                \
        uint32_t max_ctx, uint32_t splits, float scale, float eps);                                              \
    __global__ void x0ne_attention_rope_decode_batch_g##G##_bf16(                                               \
        const bf16_t* qkv, const bf16_t* q_norm, const bf16_t* k_norm, const float* inv_freq,                    \
        const double* rope_cs, bf16_t* k_cache, bf16_t* v_cache, const uint32_t* pages, float* state,           \
        uint32_t* counter, bf16_t* out, const uint32_t* pos, uint32_t q_heads, uint32_t kv_heads,                \
        uint32_t max_ctx, uint32_t splits, float scale, float eps, uint32_t seq_pages);                          \
    __global__ void x0ne_attention_rope_decode_exact_g##G##_bf16(                                               \
        const bf16_t* qkv, const bf16_t* q_norm, const bf16_t* k_norm, const float* inv_freq,                    \
        const double* rope_cs, bf16_t* k_cache, bf16_t* v_cache, const uint32_t* pages, float* state,           \
        uint32_t* counter, bf16_t* out, const uint32_t* pos, uint32_t q_heads, uint32_t kv_heads,                \
        uint32_t max_ctx, uint32_t splits, float scale, float eps);
X0NE_DECLARE_SPLIT_GROUP(1)
X0NE_DECLARE_SPLIT_GROUP(2)
X0NE_DECLARE_SPLIT_GROUP(4)
X0NE_DECLARE_SPLIT_GROUP(8)
#undef X0NE_DECLARE_SPLIT_GROUP
__global__ void x0ne_attention_merge_bf16(const float* state, bf16_t* out, const uint32_t* pos, uint32_t max_ctx,
                                          uint32_t splits);
__global__ void x0ne_attention_prefill_bf16(const bf16_t* q, const bf16_t* k_cache, const bf16_t* v_cache,
                                            const uint32_t* pages, bf16_t* out, const uint32_t* pos0, uint32_t rows,
                                            uint32_t q_heads, uint32_t kv_heads, uint32_t max_ctx, float scale);
__global__ void x0ne_rope_table_f64(const float* inv_freq, double* cs, uint32_t positions);
// Columns (row, q head) per block of x0ne_attention_prefill_g{G}_bf16 and its threads: its grid
// is (kv_heads, ceil(rows / (X0NE_PREFILL_COLS / G))), its block X0NE_PREFILL_THREADS (a block
// of another size does nothing).
#define X0NE_PREFILL_COLS 128
#define X0NE_PREFILL_THREADS 256
#define X0NE_DECLARE_PREFILL_GROUP(G)                                                                            \
    __global__ void x0ne_attention_prefill_g##G##_bf16(const bf16_t* q, const bf16_t* k_cache, const bf16_t* v_cache, \
                                                      const uint32_t* pages, bf16_t* out, const uint32_t* pos0,  \
                                                      uint32_t rows, uint32_t q_heads, uint32_t kv_heads,        \
                                                      uint32_t max_ctx, float scale);                    \
    __global__ void x0ne_attention_prefill_panel_g##G##_bf16(                                                    \
        const bf16_t* q, const bf16_t* k_cache, const bf16_t* v_cache, const uint32_t* pages, bf16_t* out,       \
        const uint32_t* pos0, uint32_t rows, uint32_t q_heads, uint32_t kv_heads, uint32_t max_ctx, float scale);
X0NE_DECLARE_PREFILL_GROUP(1)
X0NE_DECLARE_PREFILL_GROUP(2)
X0NE_DECLARE_PREFILL_GROUP(4)
X0NE_DECLARE_PREFILL_GROUP(8)
#undef X0NE_DECLARE_PREFILL_GROUP
// x0ne_attention_prefill_exact_g{G}_bf16: the exact mode's causal prefill; grid (kv_heads,
// ceil(rows / (X0NE_PREFILL_EXACT_COLS / G))), block X0NE_PREFILL_EXACT_THREADS (a block of
// another size does nothing).
#define X0NE_PREFILL_EXACT_COLS 64
#define X0NE_PREFILL_EXACT_THREADS 256
#define X0NE_DECLARE_PREFILL_EXACT(G)                                                                            \
    __global__ void x0ne_attention_prefill_exact_g##G##_bf16(                                                    \
        const bf16_t* q, const bf16_t* k_cache, const bf16_t* v_cache, const uint32_t* pages, bf16_t* out,       \
        const uint32_t* pos0, uint32_t rows, uint32_t q_heads, uint32_t kv_heads, uint32_t max_ctx, float scale);
X0NE_DECLARE_PREFILL_EXACT(1)
X0NE_DECLARE_PREFILL_EXACT(2)
X0NE_DECLARE_PREFILL_EXACT(4)
X0NE_DECLARE_PREFILL_EXACT(8)
#undef X0NE_DECLARE_PREFILL_EXACT
__global__ void x0ne_swiglu_bf16(const bf16_t* gate_up, bf16_t* out, uint32_t inter);
__global__ void x0ne_swiglu_panel_bf16(const bf16_t* gate_up, bf16_t* out, uint32_t inter);
__global__ void x0ne_argmax_f32(const float* logits, uint32_t n, uint32_t* out);
__global__ void x0ne_argmax_slices_f32(const float* logits, uint32_t n, uint32_t slices, uint32_t* partial);
__global__ void x0ne_argmax_pick_advance(const uint32_t* partial, uint32_t slices, uint32_t* tokens, uint32_t* pos);
__global__ void x0ne_embed_rmsnorm_panel_bf16(const bf16_t* table, const uint32_t* tokens, float* residual,
                                              const bf16_t* w, bf16_t* out, uint32_t hidden, uint32_t vocab,
                                              float eps);
__global__ void x0ne_add_rmsnorm_to_bf16(const float* res_in, float* res_out, const bf16_t* x, const bf16_t* w,
                                         bf16_t* out, uint32_t hidden, float eps);
__global__ void x0ne_add_rmsnorm_panel_bf16(float* residual, const bf16_t* x, const bf16_t* w, bf16_t* out,
                                            uint32_t hidden, float eps);
__global__ void x0ne_advance_u32(uint32_t* pos);
__global__ void x0ne_feed_u32(const uint32_t* ids, uint32_t i, uint32_t* tokens, uint32_t* pos);
#define X0NE_DECLARE_FEW(V)                                                                                      \
    __global__ void x0ne_gemm_few_##V##_bf16(const bf16_t* w, const bf16_t* x, void* y, uint32_t rows, uint32_t cols, \
                                             uint32_t n, uint32_t out_f32);
X0NE_DECLARE_FEW(t1_r1)
X0NE_DECLARE_FEW(t1_r2)
X0NE_DECLARE_FEW(t1_r4)
X0NE_DECLARE_FEW(t1_r8)
X0NE_DECLARE_FEW(t1_r1_swiglu)
X0NE_DECLARE_FEW(t1_r2_swiglu)
X0NE_DECLARE_FEW(t2_r1)
X0NE_DECLARE_FEW(t2_r2)
X0NE_DECLARE_FEW(t2_r1_swiglu)
X0NE_DECLARE_FEW(t4_r1)
X0NE_DECLARE_FEW(t4_r1_swiglu)
#undef X0NE_DECLARE_FEW
#define X0NE_DECLARE_GEMM_F64(V)                                                                                 \
    __global__ void x0ne_gemm_f64_##V##_bf16(const bf16_t* w, const bf16_t* x, void* y, uint32_t rows, uint32_t cols, \
                                             uint32_t n, uint32_t out_f32, uint32_t ks, double* ws);
X0NE_DECLARE_GEMM_F64(t1)
X0NE_DECLARE_GEMM_F64(t2)
X0NE_DECLARE_GEMM_F64(t4)
X0NE_DECLARE_GEMM_F64(q1)
X0NE_DECLARE_GEMM_F64(q2)
X0NE_DECLARE_GEMM_F64(q3)
X0NE_DECLARE_GEMM_F64(q4)
X0NE_DECLARE_GEMM_F64(q5)
X0NE_DECLARE_GEMM_F64(q6)
X0NE_DECLARE_GEMM_F64(q7)
X0NE_DECLARE_GEMM_F64(q8)
#undef X0NE_DECLARE_GEMM_F64
__global__ void x0ne_gemm_f64_reduce(const double* ws, void* y, uint32_t rows, uint32_t n, uint32_t ks,
                                     uint32_t out_f32);
__global__ void x0ne_gemm_few_bal_bf16(const bf16_t* w, const bf16_t* x, void* y, uint32_t rows, uint32_t cols,
                                       uint32_t n, uint32_t flags, uint32_t T, float* ws, uint32_t* cnt);
__global__ void x0ne_moe_route_f32(const float* logits, uint32_t experts, uint32_t top_k, uint32_t* ids,
                                   float* weights);
__global__ void x0ne_moe_gemv_bf16(const bf16_t* w, const uint32_t* ids, const bf16_t* x, bf16_t* y, uint32_t rows,
                                   uint32_t cols, uint32_t experts, uint32_t x_group, uint32_t x_stride);
__global__ void x0ne_moe_gemv_f32(const bf16_t* w, const uint32_t* ids, const bf16_t* x, float* y, uint32_t rows,
                                  uint32_t cols, uint32_t experts, uint32_t x_group, uint32_t x_stride);
__global__ void x0ne_moe_combine_bf16(const float* y, const float* weights, bf16_t* out, uint32_t hidden,
                                      uint32_t top_k);
__global__ void x0ne_moe_gate_up_swiglu_bf16(const bf16_t* w, const uint32_t* ids, const bf16_t* x, bf16_t* act,
                                             uint32_t inter, uint32_t cols, uint32_t experts);
__global__ void x0ne_moe_down_combine_bf16(const bf16_t* w, const uint32_t* ids, const float* wts, const bf16_t* act,
                                           bf16_t* out, uint32_t hidden, uint32_t inter, uint32_t experts,
                                           uint32_t top_k);
__global__ void x0ne_moe_gate_up_swiglu_exact_bf16(const bf16_t* w, const uint32_t* ids, const bf16_t* x, bf16_t* act,
                                                   uint32_t inter, uint32_t cols, uint32_t experts);
__global__ void x0ne_moe_down_combine_exact_bf16(const bf16_t* w, const uint32_t* ids, const float* wts,
                                                 const bf16_t* act, bf16_t* out, uint32_t hidden, uint32_t inter,
                                                 uint32_t experts, uint32_t top_k);
__global__ void x0ne_panel_bf16(const bf16_t* src, bf16_t* dst, uint32_t rows, uint32_t cols);
__global__ void x0ne_gemv_bf16(const bf16_t* w, const bf16_t* x, void* y, uint32_t rows, uint32_t cols);
__global__ void x0ne_gemv_f32(const bf16_t* w, const bf16_t* x, void* y, uint32_t rows, uint32_t cols);
__global__ void x0ne_gemv_any(const bf16_t* w, const bf16_t* x, void* y, uint32_t rows, uint32_t cols,
                              uint32_t f32_out);
}

// The table: name, host stub, parameter kinds (0 pointer, 1 u32, 2 f32), most threads a block
// may have.
struct X0neKernel {
    const char* name;
    const void* fn;
    const char* params;  // one character per parameter: 'p', 'u', 'f'
    uint32_t max_block;
};

const X0neKernel* x0ne_kernel_table(size_t* n);
