// The kernel table (the analogue of KERNEL_NAMES / KERNEL_PARAMS, x0ne-core/kernels/src/
// lib.rs:39-124): every kernel the launch API accepts, with its parameter kinds in order.
// A CPU test parses the declarations in kernels.h and checks this table against them.
#include "kernels.h"

static const X0neKernel TABLE[] = {
    {"x0ne_probe_iota_u32", (const void*)&x0ne_probe_iota_u32, "pu", 256},
    {"x0ne_gemm_bf16", (const void*)&x0ne_gemm_bf16, "pppuuuu", 256},
    {"x0ne_gemm_few_t1_r1_bf16", (const void*)&x0ne_gemm_few_t1_r1_bf16, "pppuuuu", 512},
    {"x0ne_gemm_few_t1_r2_bf16", (const void*)&x0ne_gemm_few_t1_r2_bf16, "pppuuuu", 512},
    {"x0ne_gemm_few_t1_r4_bf16", (const void*)&x0ne_gemm_few_t1_r4_bf16, "pppuuuu", 512},
    {"x0ne_gemm_few_t1_r8_bf16", (const void*)&x0ne_gemm_few_t1_r8_bf16, "pppuuuu", 512},
    {"x0ne_gemm_few_t1_r1_swiglu_bf16", (const void*)&x0ne_gemm_few_t1_r1_swiglu_bf16, "pppuuuu", 512},
    {"x0ne_gemm_few_t1_r2_swiglu_bf16", (const void*)&x0ne_gemm_few_t1_r2_swiglu_bf16, "pppuuuu", 512},
    {"x0ne_gemm_few_t2_r1_bf16", (const void*)&x0ne_gemm_few_t2_r1_bf16, "pppuuuu", 512},
    {"x0ne_gemm_few_t2_r2_bf16", (const void*)&x0ne_gemm_few_t2_r2_bf16, "pppuuuu", 512},
    {"x0ne_gemm_few_t2_r1_swiglu_bf16", (const void*)&x0ne_gemm_few_t2_r1_swiglu_bf16, "pppuuuu", 512},
    {"x0ne_gemm_few_t4_r1_bf16", (const void*)&x0ne_gemm_few_t4_r1_bf16, "pppuuuu", 512},
    {"x0ne_gemm_few_t4_r1_swiglu_bf16", (const void*)&x0ne_gemm_few_t4_r1_swiglu_bf16, "pppuuuu", 512},
    {"x0ne_probe_bf16_round", (const void*)&x0ne_probe_bf16_round, "uupp", 256},
    {"x0ne_embedding_bf16", (const void*)&x0ne_embedding_bf16, "pppuu", 128},
    {"x0ne_add_rmsnorm_bf16", (const void*)&x0ne_add_rmsnorm_bf16, "ppppuf", 256},
    {"x0ne_rope_table_f64", (const void*)&x0ne_rope_table_f64, "ppu", 256},
    {"x0ne_qk_norm_rope_kv_write_bf16", (const void*)&x0ne_qk_norm_rope_kv_write_bf16, "pppppppppuuuf", 64},
    {"x0ne_attention_decode_bf16", (const void*)&x0ne_attention_decode_bf16, "ppppppuuuf", 256},
    {"x0ne_attention_decode_split_bf16", (const void*)&x0ne_attention_decode_split_bf16, "pppppppuuuuf", 256},
    {"x0ne_attention_decode_split_g1_bf16", (const void*)&x0ne_attention_decode_split_g1_bf16, "ppppppppuuuuf", 256},
    {"x0ne_attention_decode_split_g2_bf16", (const void*)&x0ne_attention_decode_split_g2_bf16, "ppppppppuuuuf", 256},
    {"x0ne_attention_decode_split_g4_bf16", (const void*)&x0ne_attention_decode_split_g4_bf16, "ppppppppuuuuf", 256},
    {"x0ne_attention_decode_split_g8_bf16", (const void*)&x0ne_attention_decode_split_g8_bf16, "ppppppppuuuuf", 256},
    {"x0ne_attention_rope_decode_g1_bf16", (const void*)&x0ne_attention_rope_decode_g1_bf16, "ppppppppppppuuuuff", 256},
    {"x0ne_attention_rope_decode_g2_bf16", (const void*)&x0ne_attention_rope_decode_g2_bf16, "ppppppppppppuuuuff", 256},
    {"x0ne_attention_rope_decode_g4_bf16", (const void*)&x0ne_attention_rope_decode_g4_bf16, "ppppppppppppuuuuff", 256},
    {"x0ne_attention_rope_decode_g8_bf16", (const void*)&x0ne_attention_rope_decode_g8_bf16, "ppppppppppppuuuuff", 256},
    {"x0ne_attention_rope_decode_batch_g1_bf16", (const void*)&x0ne_attention_rope_decode_batch_g1_bf16, "ppppppppppppuuuuffu", 256},
    {"x0ne_attention_rope_decode_exact_g1_bf16", (const void*)&x0ne_attention_rope_decode_exact_g1_bf16, "pppppppppuuuf", 256},
    {"x0ne_attention_rope_decode_batch_g2_bf16", (const void*)&x0ne_attention_rope_decode_batch_g2_bf16, "ppppppppppppuuuuffu", 256},
    {"x0ne_attention_rope_decode_exact_g2_bf16", (const void*)&x0ne_attention_rope_decode_exact_g2_bf16, "pppppppppuuuf", 256},
    {"x0ne_attention_rope_decode_batch_g4_bf16", (const void*)&x0ne_attention_rope_decode_batch_g4_bf16, "ppppppppppppuuuuffu", 256},
    {"x0ne_attention_rope_decode_exact_g4_bf16", (const void*)&x0ne_attention_rope_decode_exact_g4_bf16, "pppppppppuuuf", 256},
    {"x0ne_attention_rope_decode_batch_g8_bf16", (const void*)&x0ne_attention_rope_decode_batch_g8_bf16, "ppppppppppppuuuuffu", 256},
    {"x0ne_attention_rope_decode_exact_g8_bf16", (const void*)&x0ne_attention_rope_decode_exact_g8_bf16, "pppppppppuuuf", 256},
    {"x0ne_attention_merge_bf16", (const void*)&x0ne_attention_merge_bf16, "pppuu", 64},
    {"x0ne_attention_prefill_g1_bf16", (const void*)&x0ne_attention_prefill_g1_bf16, "ppppppuuuuf", 256},
    {"x0ne_attention_prefill_g2_bf16", (const void*)&x0ne_attention_prefill_g2_bf16, "ppppppuuuuf", 256},
    {"x0ne_attention_prefill_g4_bf16", (const void*)&x0ne_attention_prefill_g4_bf16, "ppppppuuuuf", 256},
    {"x0ne_attention_prefill_g8_bf16", (const void*)&x0ne_attention_prefill_g8_bf16, "ppppppuuuuf", 256},
    {"x0ne_attention_prefill_bf16", (const void*)&x0ne_attention_prefill_bf16, "ppppppuuuuf", 256},
    {"x0ne_swiglu_bf16", (const void*)&x0ne_swiglu_bf16, "ppu", 256},
    {"x0ne_argmax_f32", (const void*)&x0ne_argmax_f32, "pup", 1024},
    {"x0ne_argmax_slices_f32", (const void*)&x0ne_argmax_slices_f32, "puup", 256},
    {"x0ne_argmax_pick_advance", (const void*)&x0ne_argmax_pick_advance, "pupp", 64},
    {"x0ne_embed_rmsnorm_bf16", (const void*)&x0ne_embed_rmsnorm_bf16, "pppppuuf", 256},
    {"x0ne_advance_u32", (const void*)&x0ne_advance_u32, "p", 64},
    {"x0ne_feed_u32", (const void*)&x0ne_feed_u32, "pupp", 64},
    {"x0ne_gemv_bf16", (const void*)&x0ne_gemv_bf16, "pppuu", 256},
    {"x0ne_gemv_f32", (const void*)&x0ne_gemv_f32, "pppuu", 256},
    {"x0ne_gemv_any", (const void*)&x0ne_gemv_any, "pppuuu", 256},
};

const X0neKernel* x0ne_kernel_table(size_t* n) {
    *n = sizeof(TABLE) / sizeof(TABLE[0]);
    return TABLE;
}
