/*
 * x0ne Core for MI355X: the C ABI of the decode engine, its kernel-launch API and its arena.
 *
 * This is the drop-in boundary for the reference's x0ne-core runtime crate
 * (x0ne-core/runtime/src/, Rust): every entry point below names the Rust item it replaces,
 * file:line in the reference. Plain pointers and sizes only. A Rust FFI crate binds these
 * functions one to one, and safe wrappers over them give back the reference's Engine / Session /
 * Greedy / Gpu / Arena types.
 *
 * Conventions:
 *  - Every call returns an x0ne_status; X0NE_OK is 0. The other codes are the variants of the
 *    reference's Error (x0ne-core/runtime/src/error.rs:4-15). x0ne_last_error copies the calling
 *    thread's message of its last failed call.
 *  - Format errors (bad config, bad ids, sizes) are raised before any device work, as in the
 *    reference.
 *  - Handles are not thread-safe: one thread at a time per engine (the reference's Gpu is Send,
 *    not Sync, and x0ne-infer serialises through a Mutex, core_backend.rs:106,281).
 *  - No call keeps caller memory after it returns, except the logits pointer of a session, valid
 *    until the next step or finish (engine.rs:1141-1160).
 */
#ifndef X0NE_CORE_H
#define X0NE_CORE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- errors (x0ne-core/runtime/src/error.rs:4-40) ---- */
typedef enum {
    X0NE_OK = 0,
    X0NE_ERR_IO = 1,              /* Error::Io */
    X0NE_ERR_FORMAT = 2,          /* Error::Format(String) */
    X0NE_ERR_ARENA = 3,           /* Error::Arena(String) */
    X0NE_ERR_NOT_IMPLEMENTED = 4, /* Error::NotImplemented(&'static str) */
    X0NE_ERR_GPU = 5,             /* Error::Gpu(String) */
} x0ne_status;

/* The message of the calling thread's last failed call, truncated to len - 1 bytes. Returns the
   full length. */
size_t x0ne_last_error(char* buf, size_t len);

/* Library facts: kernel-set fingerprint and the compiler it was built with
   (x0ne-core/runtime/src/lib.rs: kernel_set()). */
size_t x0ne_kernel_set(char* buf, size_t len);

/* ---- the device (x0ne-core/runtime/src/gpu.rs) ---- */
typedef struct x0ne_gpu x0ne_gpu;

/* Gpu::new (gpu.rs:799-928): device 0, one non-blocking stream at the default priority, the
   kernel table checked against the loaded code object. X0NE_ERR_GPU without a usable GPU. */
x0ne_status x0ne_gpu_new(x0ne_gpu** out);
void x0ne_gpu_free(x0ne_gpu* g);
/* Gpu::sync: waits for the stream. */
x0ne_status x0ne_gpu_sync(x0ne_gpu* g);
/* Name, architecture, compute units, driver and runtime versions (Engine::describe's GPU part,
   engine.rs:578-606). */
x0ne_status x0ne_gpu_describe(const x0ne_gpu* g, char* buf, size_t len);
uint32_t x0ne_gpu_compute_units(const x0ne_gpu* g);
/* Free and total device bytes (Engine::device_free_bytes, engine.rs:632-635). */
x0ne_status x0ne_gpu_mem_info(const x0ne_gpu* g, uint64_t* free_bytes, uint64_t* total_bytes);

/* Driver-call tallies (gpu.rs:93-103, Counts): the witness of "one graph launch and one 4-byte
   copy per token". */
typedef struct {
    uint64_t launches, graph_launches, gemms, htod, dtoh, memsets, syncs;
} x0ne_counts;
x0ne_status x0ne_gpu_counts(const x0ne_gpu* g, x0ne_counts* out);

/* ---- the kernel table (x0ne-core/kernels/src/lib.rs:39-132: KERNEL_NAMES, KERNEL_PARAMS) ---- */
typedef enum { X0NE_PARAM_PTR = 0, X0NE_PARAM_U32 = 1, X0NE_PARAM_F32 = 2 } x0ne_param;

/* Arg::{Ptr(u64), U32, F32} (gpu.rs:281-314). */
typedef struct {
    uint32_t kind; /* x0ne_param */
    uint32_t u32;
    float f32;
    uint32_t pad;
    uint64_t ptr;
} x0ne_arg;

size_t x0ne_kernel_count(void);
/* Name of kernel i, or NULL past the table. */
const char* x0ne_kernel_name(size_t i);
/* params_of (lib.rs:146-151): the parameter kinds of `name` into out (up to cap); returns the
   count, or (size_t)-1 for an unknown name. */
size_t x0ne_kernel_params(const char* name, uint32_t* out, size_t cap);
/* check_args (gpu.rs:317-333): X0NE_ERR_GPU naming the first argument whose kind differs, or a
   count that differs. No device needed. */
x0ne_status x0ne_check_args(const char* name, const x0ne_arg* args, size_t n);
/* Gpu::launch / launch! (gpu.rs:1031-1086, :1383-1387): kernel `name` on the stream, grid
   (gx, gy), `block` threads, the arguments checked against the table first. Not synchronised. */
x0ne_status x0ne_gpu_launch(x0ne_gpu* g, const char* name, uint32_t gx, uint32_t gy, uint32_t block,
                            const x0ne_arg* args, size_t n);
/* x0ne_gpu_launch with a third grid dimension, for the kernels that take one sequence per
   blockIdx.z (x0ne_attention_rope_decode_batch_g*_bf16); no counterpart in the reference, whose
   launch grids are two-dimensional (gpu.rs:1031-1086). */
x0ne_status x0ne_gpu_launch_3d(x0ne_gpu* g, const char* name, uint32_t gx, uint32_t gy, uint32_t gz, uint32_t block,
                               const x0ne_arg* args, size_t n);

/* Gpu::gemm (gpu.rs:1098-1149), the projection the reference hands cuBLAS: Y[n][rows] =
   X[n][cols] W^T, W [rows][cols] row-major bf16, X bf16, f32 accumulation; out_f32 = 0 gives
   bf16 Y, 1 f32 Y. Device addresses. One row of X: the bandwidth-bound GEMV; 2 to 64 rows (cols
   a multiple of 8, W and X each below 4 GiB): one few-row matrix-core launch that reads each W
   row once (x0ne_gemm_few_*); more rows (rows a multiple of 4, 16-byte aligned operands): this
   library's tiled matrix-core GEMM (x0ne_gpu_gemm_tiled with the tile chosen for the shape);
   other shapes: one GEMV per row of X. */
x0ne_status x0ne_gpu_gemv(x0ne_gpu* g, uint64_t w, uint64_t rows, uint64_t cols, uint64_t x, uint64_t n, uint64_t y,
                          int out_f32);
/* The tiled matrix-core GEMM of x0ne_gpu_gemv past 64 rows with an explicit block tile (output
   features x tokens; AUTO: the one x0ne_gpu_gemv picks) and operand layout, for kernel tests and
   tuning; no counterpart in the reference, whose Gpu::gemm is one cuBLAS call
   (gpu.rs:1098-1149). Y[n][rows] = X[n][cols] W^T, bf16 W and X, f32 accumulation in a fixed
   order (the same bits from call to call), bf16 or f32 Y row-major. layout: X0NE_GEMM_W_PANELS
   and/or X0NE_GEMM_X_PANELS for W and/or X in 16-row panels (element (r, k) at
   ((r / 16 * cols / 8 + k / 8) * 16 + r % 16) * 8 + k % 8; X's last panel whole, the rows past n
   any value), else row-major. rows a multiple of 4 (of 16 with W in panels), cols of 8, W and
   X below 4 GiB, 16-byte aligned operands, else X0NE_ERR_FORMAT. It may be captured into a
   graph. */
enum {
    X0NE_GEMM_TILE_AUTO = 0,
    X0NE_GEMM_TILE_256x256 = 1,
    X0NE_GEMM_TILE_256x128 = 2,
    X0NE_GEMM_TILE_128x128 = 3
};
enum { X0NE_GEMM_W_PANELS = 1, X0NE_GEMM_X_PANELS = 2 };
x0ne_status x0ne_gpu_gemm_tiled(x0ne_gpu* g, uint32_t tile, uint32_t layout, uint64_t w, uint64_t rows, uint64_t cols,
                                uint64_t x, uint64_t n, uint64_t y, int out_f32);

/* One launch of a fused decode GEMV instance on caller buffers: the kernels the decode step runs
   for its projections, each with its prologue and epilogue, driven alone for kernel-level
   parity tests. No counterpart in the reference, whose projections are cuBLAS calls beside
   separate norm, SwiGLU and argmax kernels (gpu.rs:1098-1149; rmsnorm.cu, swiglu.cu, argmax.cu).
   Device addresses; 0 for what the instance does not read or write.
   prologue X0NE_GEMV_PRO_X: x given (bf16 [cols]). X0NE_GEMV_PRO_NORM: x = bf16(rmsnorm(res_in +
   delta) * norm_w) (res_in f32, delta and norm_w bf16, [cols]), and res_out (may be 0) receives
   res_in + delta. X0NE_GEMV_PRO_EMBED_NORM: the same on row tokens[0] of embed ([vocab][cols];
   an id past vocab gives a zero row) over a zero residual.
   epilogue X0NE_GEMV_EPI_BF16 / _F32: y[rows]. X0NE_GEMV_EPI_SWIGLU: W is [gate; up] (rows = 2
   inter) and y[inter] = bf16(silu(bf16 gate) * bf16 up). X0NE_GEMV_EPI_ARGMAX: f32 logits in y,
   the first largest index into token_out (0xFFFFFFFF when the row holds a NaN), pos[0] += 1 when
   advance != 0; partial holds 3 words per block, counter one zeroed word that is left at zero.
   Instances: (X, BF16), (X, F32), (NORM, BF16), (NORM, F32), (NORM, SWIGLU), (NORM, ARGMAX),
   (EMBED_NORM, BF16); cols a multiple of 8, at most 32768 (X) or 16384 (the norm prologues).
   f64_sums: each exact product added in f64 (the exact mode). X0NE_ERR_FORMAT for another
   instance or shape, a missing or misaligned (16-byte) buffer. */
enum { X0NE_GEMV_PRO_X = 0, X0NE_GEMV_PRO_NORM = 1, X0NE_GEMV_PRO_EMBED_NORM = 2 };
enum { X0NE_GEMV_EPI_BF16 = 0, X0NE_GEMV_EPI_F32 = 1, X0NE_GEMV_EPI_SWIGLU = 2, X0NE_GEMV_EPI_ARGMAX = 3 };
typedef struct {
    uint64_t w, x, res_in, res_out, delta, norm_w, embed, tokens, y, partial, counter, token_out, pos;
    uint32_t rows, cols, vocab, advance;
    float eps;
    uint32_t prologue, epilogue, f64_sums;
} x0ne_gemv_fused;
/* The blocks of that launch (the engine's grid for the shape), 0 for a refused instance. */
uint32_t x0ne_gpu_gemv_fused_blocks(const x0ne_gpu* g, const x0ne_gemv_fused* d);
x0ne_status x0ne_gpu_gemv_fused(x0ne_gpu* g, const x0ne_gemv_fused* d);

/* Split-K plan (gpu.rs:958-985, SplitPlan): P for a geometry, and whether a grouped kernel
   serves it (group sizes 1, 2, 4, 8). */
typedef struct {
    uint32_t splits, grid_x, group, grouped, per_cu;
} x0ne_split_plan;
x0ne_status x0ne_gpu_split_plan(const x0ne_gpu* g, uint32_t q_heads, uint32_t kv_heads, x0ne_split_plan* out);
/* launch_split (ops.rs:80-122): the split kernel, then the merge kernel (last_block = 0), or the
   grouped kernel merging in its last block (last_block = 1, `counter` holds kv_heads zeroed
   words and is left at zero). The KV planes are paged: [pages][kv_heads][16][128] bf16. */
x0ne_status x0ne_gpu_attention_split(x0ne_gpu* g, const x0ne_split_plan* plan, int last_block, uint64_t q,
                                     uint64_t k, uint64_t v, uint64_t page_table, uint64_t state, uint64_t counter,
                                     uint64_t out, uint64_t pos, uint32_t q_heads, uint32_t kv_heads,
                                     uint32_t max_ctx, float scale);
/* x0ne_gpu_attention_split without a workspace argument and without allocating: no counterpart
   in the reference. For callers that cannot allocate device memory (code under HIP graph
   capture, tight serving loops, harnesses that forbid hipMalloc). The split-K states and the
   last-block counters live in a static device array of this library (4 MiB of states and 256
   counter words per GPU, held until the process ends); the counters are zeroed by a fill kernel
   at the start of each call. X0NE_ERR_FORMAT when x0ne_split_state_bytes(q_heads, P) exceeds
   4 MiB or kv_heads exceeds 256. Every call on a GPU shares that GPU's array and it keeps the
   last call's contents: calls that overlap on one GPU (other streams, other threads) race. */
x0ne_status x0ne_gpu_attention_split_scratch(x0ne_gpu* g, const x0ne_split_plan* plan, int last_block, uint64_t q,
                                             uint64_t k, uint64_t v, uint64_t page_table, uint64_t out, uint64_t pos,
                                             uint32_t q_heads, uint32_t kv_heads, uint32_t max_ctx, float scale);
/* split_state_bytes (ops.rs:125-127) */
uint64_t x0ne_split_state_bytes(uint32_t q_heads, uint32_t splits);
/* BASELINE.json config 2, the isolated decode attention of ops.rs:585-681: the grouped split-K
   kernel (P = splits, last-block merge) at position ctx - 1 over ctx keys, Q, K and V N(0, 1) bf16
   drawn from `seed`, pages in a seeded permutation, each launch on the next of *planes_out
   distinct K/V plane pairs (together more than 512 MiB, so the 256 MiB Infinity Cache serves
   none of them). *us: the mean kernel time of `iters` launches (events around each kernel). */
x0ne_status x0ne_gpu_time_attention(x0ne_gpu* g, uint32_t q_heads, uint32_t kv_heads, uint32_t ctx, uint32_t splits,
                                    uint32_t iters, uint64_t seed, double* us, uint32_t* planes_out);

/* Graph capture (gpu.rs:1170-1238): every launch between begin and end is recorded, then
   replayed by x0ne_gpu_launch_graph on the Gpu that captured it (another Gpu is refused with
   X0NE_ERR_GPU, gpu.rs:1225-1230). */
typedef struct x0ne_graph x0ne_graph;
x0ne_status x0ne_gpu_capture_begin(x0ne_gpu* g);
x0ne_status x0ne_gpu_capture_end(x0ne_gpu* g, x0ne_graph** out);
x0ne_status x0ne_gpu_launch_graph(x0ne_gpu* g, const x0ne_graph* graph);
size_t x0ne_graph_nodes(const x0ne_graph* graph);
void x0ne_graph_free(x0ne_graph* graph);

/* ---- the arena (x0ne-core/runtime/src/arena.rs) ---- */
typedef enum { X0NE_CLASS_WEIGHTS = 0, X0NE_CLASS_CLIENT_DATA = 1 } x0ne_class; /* arena.rs:42-45 */

/* A planned region (arena.rs:49-53); only valid for the arena that issued it. */
typedef struct {
    uint64_t arena, offset, len;
} x0ne_slice;

typedef struct x0ne_arena x0ne_arena;
#define X0NE_ARENA_ALIGN 256 /* arena.rs:37 */

/* Arena::new (arena.rs:163-172): a Building arena. */
x0ne_status x0ne_arena_new(x0ne_arena** out);
void x0ne_arena_free(x0ne_arena* a);
/* Arena<Building>::alloc (arena.rs:174-198); refused once frozen (the reference's typestate
   makes that a compile error; here it is X0NE_ERR_ARENA). */
x0ne_status x0ne_arena_alloc(x0ne_arena* a, const char* label, uint64_t len, uint32_t cls, x0ne_slice* out);
uint64_t x0ne_arena_planned_bytes(const x0ne_arena* a);
/* freeze (arena.rs:210-225): the one allocation, on `g`'s device; g == NULL gives host memory
   poisoned with 0xA5 (HostBacking, arena.rs:91-136). */
x0ne_status x0ne_arena_freeze(x0ne_arena* a, x0ne_gpu* g);
/* write / read (arena.rs:242-250): checked against the slice. Device arenas copy synchronously
   on `g`'s stream. */
x0ne_status x0ne_arena_write(x0ne_arena* a, x0ne_slice s, uint64_t at, const void* data, uint64_t len);
x0ne_status x0ne_arena_read(const x0ne_arena* a, x0ne_slice s, uint64_t at, void* out, uint64_t len);
/* addr / span (arena.rs:276-303): the device (or host) address of byte `at` of a slice. */
x0ne_status x0ne_arena_addr(const x0ne_arena* a, x0ne_slice s, uint64_t at, uint64_t* out);
x0ne_status x0ne_arena_span(const x0ne_arena* a, x0ne_slice s, uint64_t at, uint64_t len, uint64_t* out);
/* scrub_client_data (arena.rs:252-265): zeroes every ClientData region, returns the bytes. */
x0ne_status x0ne_arena_scrub(x0ne_arena* a, uint64_t* zeroed);
/* Regions in plan order: label into label_buf, class, offset and length. */
size_t x0ne_arena_region_count(const x0ne_arena* a);
x0ne_status x0ne_arena_region(const x0ne_arena* a, size_t i, char* label_buf, size_t label_len, uint32_t* cls,
                              uint64_t* offset, uint64_t* len);
/* The slice of region i, as alloc returned it (for reading a planned buffer back). */
x0ne_status x0ne_arena_region_slice(const x0ne_arena* a, size_t i, x0ne_slice* out);
int x0ne_arena_is_frozen(const x0ne_arena* a);

/* ---- the engine (x0ne-core/runtime/src/engine.rs) ---- */
typedef struct x0ne_engine x0ne_engine;
typedef struct x0ne_session x0ne_session;
typedef struct x0ne_greedy x0ne_greedy;

/* EngineOptions (engine.rs:38-40), plus this build's choices:
   - page_seed: 0 keeps logical KV page i at physical page i, another seed shuffles the pages
     with a seeded permutation;
   - sums: the accumulation of the projections and of decode attention.
     X0NE_SUMS_F64 is the exact mode: the projections add their exact bf16 products in f64, and
     decode attention computes scores, softmax and sums in f64 with the f64 scale 1/sqrt(128)
     (split-K with f64 states merged in f64), so every rounding point of the step is the f64
     oracle's (oracle/src/lib.rs:123-187) and the greedy tokens are the oracle's; its prefill
     passes sum in f64 too (the same bits as feeding the prompt one decode step per token). It
     serves a dense or MoE model decoding one sequence with 1, 2, 4 or 8 q
     heads per kv head (X0NE_ERR_NOT_IMPLEMENTED otherwise).
     X0NE_SUMS_F32 is the fp32-accumulating path (the reference engine's arithmetic: f32 sums,
     matrix-core prefill passes).
     X0NE_SUMS_DEFAULT (0, what EngineOptions { max_ctx } gives) is the exact mode wherever the
     engine can serve it, else the f32 path (max_batch > 1).
   - prefill_chunk: prompt rows per prefill pass (engine.rs:67, PREFILL_CHUNK); 0 takes
     min(2048, max_ctx x max_batch). A pass runs every layer over its rows with matrix-core
     GEMMs and the causal prefill attention (the exact mode's in f64; a MoE engine feeds a
     prompt one decode step per token).
   - max_batch: independent sequences the batched greedy entry points serve (0 or 1: the
     single-sequence engine). Each sequence has its own max_ctx positions of KV pages (the page
     table holds max_batch runs of ceil(max_ctx / 16) pages) and its own position; the batched
     step's projections read every weight once for all sequences. 1 to 64; the f32 path only
     (X0NE_ERR_NOT_IMPLEMENTED with X0NE_SUMS_F64 or a group size without a grouped kernel). */
#define X0NE_SUMS_DEFAULT 0u
#define X0NE_SUMS_F64 1u
#define X0NE_SUMS_F32 2u
typedef struct {
    uint64_t max_ctx;
    uint64_t page_seed;
    uint32_t sums;
    uint32_t prefill_chunk;
    uint32_t max_batch;
    uint32_t reserved; /* 0 */
} x0ne_engine_options;

/* Engine::load_from (engine.rs:301-309) over safetensors files already in memory (the
   reference's st::SliceSource::new(index_json, files), st.rs:216-277): `n_files` files named
   names[i] with bytes data[i][0..lens[i]]; index_json may be NULL. BF16 tensors of a Qwen3 dense
   checkpoint; [q;k;v] and [gate;up] rows are packed at upload (weights.rs:420-429). */
x0ne_status x0ne_engine_load_from(const char* config_json, size_t n_files, const char* const* names,
                                  const uint8_t* const* data, const uint64_t* lens, const char* index_json,
                                  const x0ne_engine_options* opts, x0ne_engine** out);
/* Engine::load (engine.rs:292-297) with Safetensors::open_dir (st.rs:158-181): model_dir's
   config.json (X0NE_ERR_IO when it cannot be read), then model.safetensors or the shards named
   by model.safetensors.index.json, mapped read-only, each at most 64 GiB (st.rs:11, :55-67); both
   present or neither is X0NE_ERR_FORMAT, a shard that cannot be opened X0NE_ERR_IO. The files then
   pass x0ne_engine_load_from's checks. */
x0ne_status x0ne_engine_load(const char* model_dir, const x0ne_engine_options* opts, x0ne_engine** out);
/* This build's synthetic load: the checkpoint of `config_json` drawn on the device, every
   projection and the embedding N(0, std) bf16 from `seed` (tensor i of the checkpoint order,
   oracle/src/model.rs:63-89, takes stream key splitmix64 output i of `seed`), norm weights 1.0. */
x0ne_status x0ne_engine_load_synthetic(const char* config_json, uint64_t seed, double std_dev,
                                       const x0ne_engine_options* opts, x0ne_engine** out);
void x0ne_engine_free(x0ne_engine* e);

/* Engine::session (engine.rs:389-406): prefills `prompt` and holds the last position's logits.
   One session at a time per engine (a Session borrows the Engine mutably). */
x0ne_status x0ne_engine_session(x0ne_engine* e, const uint32_t* prompt, size_t n, x0ne_session** out);
/* Session::logits (engine.rs:1141-1149): vocab_size f32, valid until the next step or finish. */
x0ne_status x0ne_session_logits(const x0ne_session* s, const float** ptr, size_t* len);
size_t x0ne_session_position(const x0ne_session* s);
/* Session::step (engine.rs:1159-1178). */
x0ne_status x0ne_session_step(x0ne_session* s, uint32_t token);
/* Session::finish (engine.rs:1181-1184): zeroes client bytes, frees the session. */
x0ne_status x0ne_session_finish(x0ne_session* s);
/* Drop for Session (engine.rs:1346-1353): scrubs, frees. */
void x0ne_session_drop(x0ne_session* s);
/* Session::into_greedy_ahead (engine.rs:1199-1243): consumes the session (freed even on error;
   a failure then scrubs, as the reference's drop does). ahead in 1..=15. */
x0ne_status x0ne_session_into_greedy(x0ne_session* s, size_t max_tokens, size_t ahead, x0ne_greedy** out);
/* Greedy::next_token / taken / position / finish (engine.rs:1250-1344). */
x0ne_status x0ne_greedy_next(x0ne_greedy* g, uint32_t* token);
size_t x0ne_greedy_taken(const x0ne_greedy* g);
size_t x0ne_greedy_position(const x0ne_greedy* g);
x0ne_status x0ne_greedy_finish(x0ne_greedy* g);
void x0ne_greedy_drop(x0ne_greedy* g);

/* Engine::greedy_timed (engine.rs:1026-1038): n greedy tokens after prompt, with the wall time
   (seconds from the call) each was back on the host. times may be NULL (Engine::greedy). */
x0ne_status x0ne_engine_greedy_timed(x0ne_engine* e, const uint32_t* prompt, size_t n_prompt, size_t n,
                                     uint32_t* tokens, double* times);
/* Engine::greedy_with_last_logits (engine.rs:1042-1063): logits holds vocab_size floats. */
x0ne_status x0ne_engine_greedy_with_last_logits(x0ne_engine* e, const uint32_t* prompt, size_t n_prompt, size_t n,
                                                uint32_t* tokens, float* logits);

/* The bench's decode measure (the method of x0ne-core/oracle/examples/core-perf.rs:77-94, with
   the timed region bracketed by stream synchronisations): prefill `prompt`, run `warmup` decode
   steps, synchronise, then time `steps` decode steps to a final synchronisation. tokens receives
   warmup + steps + 1 greedy tokens; seconds the timed region. Client bytes are zeroed after. */
x0ne_status x0ne_engine_decode_timed(x0ne_engine* e, const uint32_t* prompt, size_t n_prompt, size_t warmup,
                                     size_t steps, uint32_t* tokens, double* seconds);

/* Batched greedy decoding of `batch` independent sequences (1 <= batch <= max_batch): no
   counterpart in the reference, whose engine serves one sequence at a time (engine.rs:389-406);
   it is Engine::greedy_timed applied to each of `batch` prompts at once. prompts holds
   batch rows of n_prompt ids. Each prompt is prefilled into its own KV pages: prompts of more
   than 64 ids that fit a pass share passes (prefill_chunk / n_prompt of them side by side),
   longer ones take passes of up to prefill_chunk rows each. Then every decode step advances
   all sequences: one graph launch (or the eager launches) and one copy of `batch` token words. tokens receives batch rows of n tokens;
   times (may be NULL) the wall time of each step's tokens, seconds from the call; last_logits
   (may be NULL) batch rows of vocab_size floats, the logits of each sequence's last token.
   A sequence's tokens and logits do not depend on the other sequences of the batch: the same
   bits alone or beside any others. Client bytes are zeroed after. */
x0ne_status x0ne_engine_greedy_batch(x0ne_engine* e, const uint32_t* prompts, size_t n_prompt, size_t batch, size_t n,
                                     uint32_t* tokens, double* times, float* last_logits);
/* The bench's batched decode measure: as x0ne_engine_decode_timed for `batch` sequences (tokens:
   batch rows of warmup + steps + 1 tokens). */
x0ne_status x0ne_engine_decode_batch_timed(x0ne_engine* e, const uint32_t* prompts, size_t n_prompt, size_t batch,
                                           size_t warmup, size_t steps, uint32_t* tokens, double* seconds);

/* Route (engine.rs:44-48) and DecodeMode (engine.rs:51-55). */
typedef enum { X0NE_ROUTE_PREFILL = 0, X0NE_ROUTE_DECODE = 1 } x0ne_route;
typedef enum { X0NE_DECODE_EAGER = 0, X0NE_DECODE_GRAPH = 1 } x0ne_decode_mode;
x0ne_status x0ne_engine_set_decode_mode(x0ne_engine* e, uint32_t mode);
uint32_t x0ne_engine_decode_mode(const x0ne_engine* e);

/* DecodeAttention (ops.rs:55-62) and SplitMerge (ops.rs:64-70). Engine::set_decode_attention
   (engine.rs:531-539): split-K (the default; one fused launch per layer on a grouped plan) or the
   per-head kernel (the reference's E2 witness, after the QK-norm/RoPE kernel). Engine::
   set_split_merge (engine.rs:547-560): the split-K states merged by the merge kernel or by the
   last block of each kv head (X0NE_ERR_GPU without a grouped kernel). Either re-captures the
   decode graph, which zeroes the client buffers: call them between requests (X0NE_ERR_FORMAT
   while a session is open); if the capture fails no graph is left and the engine runs eager.
   This build's default merge is the last block on a grouped plan (the reference's is the merge
   kernel, engine.rs:35). The exact mode has only its f64 split-K kernel with the last-block merge
   (X0NE_ERR_NOT_IMPLEMENTED for the others). */
typedef enum { X0NE_ATTENTION_SPLIT_K = 0, X0NE_ATTENTION_PER_HEAD = 1 } x0ne_decode_attention;
typedef enum { X0NE_MERGE_KERNEL = 0, X0NE_MERGE_LAST_BLOCK = 1 } x0ne_split_merge;
x0ne_status x0ne_engine_set_decode_attention(x0ne_engine* e, uint32_t attention);
uint32_t x0ne_engine_decode_attention(const x0ne_engine* e);
x0ne_status x0ne_engine_set_split_merge(x0ne_engine* e, uint32_t merge);
uint32_t x0ne_engine_split_merge(const x0ne_engine* e);

/* Engine::logits_at (engine.rs:1012-1020): teacher-forced f32 logits at `positions` of ids,
   rows[k * vocab ..] for positions[k]: x0ne_engine_run's kept rows (and its refusals). */
x0ne_status x0ne_engine_logits_at(x0ne_engine* e, const uint32_t* ids, size_t n, const size_t* positions,
                                  size_t n_positions, uint32_t route, float* rows);

/* PosStats (engine.rs:60-64) and Engine::run (engine.rs:928-1006): the teacher-forced pass of
   ids with, for each of the n positions, stats[p] (the device's argmax of the row; the row's
   logsumexp, metrics.rs:4-7; the log-probability of ids[p + 1], NaN at the last position), and
   the f32 rows at keep[k] in rows[k * vocab ..]. A row without a finite maximum (a NaN in it)
   refuses the whole pass with X0NE_ERR_GPU, as the reference's argmax read does
   (engine.rs:855-864). Engine::stats is this with n_keep 0, Engine::logits_at its kept rows. */
typedef struct {
    uint32_t argmax;
    float logsumexp;
    float next_logprob;
} x0ne_pos_stats;
x0ne_status x0ne_engine_run(x0ne_engine* e, const uint32_t* ids, size_t n, uint32_t route, const size_t* keep,
                            size_t n_keep, x0ne_pos_stats* stats, float* rows);

/* Engine::moe_routing (engine.rs:612-640): the experts every layer of a Qwen3-MoE engine chose
   at each position of ids (fed one per step through the decode route), [position][layer][top_k]
   into out (room for cap entries; X0NE_ERR_FORMAT when short); *written their count, 0 for a
   dense engine. */
x0ne_status x0ne_engine_moe_routing(x0ne_engine* e, const uint32_t* ids, size_t n, uint32_t* out, size_t cap,
                                    size_t* written);

/* Engine::describe, graph_nodes, splits, counts, client_data_is_zero, host_buffers_are_zero
   (engine.rs:563-670). */
x0ne_status x0ne_engine_describe(const x0ne_engine* e, char* buf, size_t len);
size_t x0ne_engine_graph_nodes(const x0ne_engine* e);
uint32_t x0ne_engine_splits(const x0ne_engine* e);
x0ne_status x0ne_engine_counts(const x0ne_engine* e, x0ne_counts* out);
x0ne_status x0ne_engine_client_data_is_zero(const x0ne_engine* e, int* out);
int x0ne_engine_host_buffers_are_zero(const x0ne_engine* e);
uint64_t x0ne_engine_max_ctx(const x0ne_engine* e);
/* The accumulation the engine runs with, X0NE_SUMS_F64 or X0NE_SUMS_F32 (the default resolved;
   this build's, no counterpart in the reference, whose engine has the f32 path only). */
uint32_t x0ne_engine_sums(const x0ne_engine* e);
/* The engine's arena, for tests that read a buffer back (KV pages, residual). Not owned. */
const x0ne_arena* x0ne_engine_arena(const x0ne_engine* e);
/* Physical page of logical page i (this build's paged KV arena). */
x0ne_status x0ne_engine_page(const x0ne_engine* e, uint64_t i, uint32_t* out);

/* One kernel of the decode step timed alone with HIP events on the engine's stream (this
   build's measurement hook, the analogue of ops.rs:585-681 attention_decode_timed): `iters`
   rounds over every layer's weights (so no cache holds them), launched back to back after one
   warm-up round. kernel_us: the average duration of one launch's kernels, from the start and
   stop events hipExtLaunchKernel records at the kernel's own begin and end (the figure a kernel
   trace reports); wall_us: the average time per launch between events around the whole run,
   gaps between launches included (either pointer may be NULL). The attention runs with every
   sequence at position max_ctx - 1, the longest context the engine holds. Client bytes are
   zeroed afterwards. */
typedef enum {
    X0NE_KERNEL_QKV = 0,
    X0NE_KERNEL_ATTENTION = 1,
    X0NE_KERNEL_O = 2,
    X0NE_KERNEL_GATE_UP = 3,
    X0NE_KERNEL_DOWN = 4,
    X0NE_KERNEL_HEAD = 5,
} x0ne_step_kernel;
x0ne_status x0ne_engine_time_kernel(x0ne_engine* e, uint32_t which, uint32_t iters, double* kernel_us,
                                    double* wall_us, uint64_t* launches);
/* The same measurement for the batched step's kernel at `batch` sequences (1 <= batch <=
   max_batch of an engine loaded with max_batch > 1): the few-row GEMM projections, the batched
   attention, the LM head with the per-sequence argmax. No counterpart in the reference. */
x0ne_status x0ne_engine_time_batch_kernel(x0ne_engine* e, uint32_t which, uint32_t batch, uint32_t iters,
                                          double* kernel_us, double* wall_us, uint64_t* launches);

/* The reference's constants (engine.rs:67-79; kernels/src/lib.rs:135-144). */
#define X0NE_GREEDY_AHEAD 2
#define X0NE_GREEDY_AHEAD_MAX 15
#define X0NE_HEAD_DIM_C 128
#define X0NE_SPLIT_STATE_C 132
#define X0NE_PAGE_C 16

#ifdef __cplusplus
}
#endif
#endif
