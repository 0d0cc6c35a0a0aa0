// The Qwen3 dense bf16 engine on MI355X: x0ne-core/runtime/src/engine.rs (with config.rs,
// weights.rs and st.rs for loading), re-planned for gfx950.
//
// One arena, frozen at load: weights, the paged KV cache, activations, logits, split-K state.
// The decode step reads its token and position from device memory and leaves the argmax in
// tokens[0] and pos + 1, so it is captured once into a HIP graph and replayed per token; the
// host receives 4 bytes per token (engine.rs:1-14, :484-501, :718-839).
//
// Per layer the step is 5 launches (the reference's is 10 plus cuBLAS nodes): the QKV GEMV with
// the residual add + RMSNorm fused in front (layer 0: the embedding too); one attention launch
// doing QK-norm + RoPE, the paged KV write and split-K attention whose last block merges; the O
// GEMV; the gate/up GEMV with the add + RMSNorm in front and SwiGLU behind; the down GEMV. Then
// the LM-head GEMV with the final norm in front and the greedy argmax + position advance behind.
// The residual stream is two f32 buffers used in turn (norm j reads buffer j % 2 and writes
// j + 1 % 2), so no block of a GEMV reads a residual another block has already advanced.
//
// A prompt is prefilled in passes of up to `chunk` rows through the MFMA GEMMs and the causal
// matrix-core attention (prefill_pass); the exact mode's passes sum in f64 on the f64 matrix
// cores and vector units with the decode step's roundings. With chunk 1 (a MoE engine) it is
// fed through the decode step one position at a time (a feed kernel puts ids[i] and i where the
// step reads them).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <map>
#include <vector>

#include "internal.h"
#include "json.h"
#include "ring.h"

using namespace x0ne;

namespace {

// Prompt rows per prefill pass by default (engine.rs:67 has 512; the matrix-core GEMM's tiles are
// 128 rows, and 2048 rows keep it compute-bound).
constexpr uint64_t PREFILL_CHUNK = 2048;
// The exact mode's prefill GEMM: f64 parts of up to this many bytes (a short pass cuts K into
// slices to fill the chip).
constexpr uint64_t EXACT_PARTS_BYTES = 32ull << 20;
constexpr uint64_t MAX_BATCH = 64;  // the few-row GEMM's most rows
constexpr uint32_t ARGMAX_SLICES = 64;  // blocks per logits row of the batched step's argmax
constexpr uint64_t MOE_MAX_EXPERTS = 1024;  // kernels/src/lib.rs:147 (moe.hip)
constexpr uint64_t MOE_MAX_TOP_K = 32;
// The largest K or V plane the attention kernels' 32-bit byte offsets address (attention.hip).
constexpr uint64_t KV_PLANE_MAX_BYTES = 0xFFFFFFF0ull;

struct Cfg {
    uint64_t hidden = 0, inter = 0, layers = 0, q_heads = 0, kv_heads = 0, head_dim = 0, vocab = 0, max_pos = 0;
    double eps = 0, theta = 0;
    bool tied = false;
    // Qwen3-MoE (config.rs:218-335): every layer's feed-forward routes a token to top_k of
    // `experts` SwiGLU experts of width moe_inter (intermediate_size is then unused).
    bool moe = false;
    uint64_t experts = 0, top_k = 0, moe_inter = 0;
    uint64_t q_dim() const { return q_heads * head_dim; }
    uint64_t kv_dim() const { return kv_heads * head_dim; }
    uint64_t qkv_rows() const { return q_dim() + 2 * kv_dim(); }
};

// ---- config.json ----
//
// The accept/refuse rules are the reference's (x0ne-core/runtime/src/config.rs:59-118 dense,
// :218-335 MoE; x0ne-infer/src/core_backend.rs:28-55 for rope_parameters), so a checkpoint it
// serves loads here and one it turns away is turned away here too. The reader and its messages
// are this build's: each refusal names the field and what the engine needs of it.
struct ConfigReader {
    const Json& root;
    std::string refusal;  // the first rule broken, empty while every rule holds

    bool refuse(const std::string& what) {
        if (refusal.empty()) refusal = "config.json: " + what;
        return false;
    }
    // `key` must hold a whole number of at least 1, written without sign, fraction or exponent.
    bool count(const char* key, uint64_t* out) {
        const Json* f = root.get(key);
        if (!f) return refuse(std::string("no \"") + key + "\" field");
        uint64_t n = 0;
        if (!f->as_u64(&n) || n == 0) return refuse(std::string("\"") + key + "\" must be a whole number >= 1");
        *out = n;
        return true;
    }
    // `f` (field `key`) must be a finite number above zero.
    bool positive(const Json* f, const char* key, double* out) {
        if (!f) return refuse(std::string("no \"") + key + "\" field");
        if (f->kind != Json::Number || !std::isfinite(f->num) || !(f->num > 0))
            return refuse(std::string("\"") + key + "\" must be a finite number above zero");
        *out = f->num;
        return true;
    }
    // `key` is absent, null or false: a feature the kernels do not have is not asked for.
    bool unset(const char* key) {
        const Json* f = root.get(key);
        if (!f || f->kind == Json::Null || (f->kind == Json::Bool && !f->b)) return true;
        return refuse(std::string("\"") + key + "\" asks for a feature this engine lacks");
    }
    // `f` is the string `want`.
    bool text(const Json* f, const char* key, const char* want) {
        if (f && f->kind == Json::String && f->text == want) return true;
        return refuse(std::string("\"") + key + "\" must be \"" + want + "\"");
    }
};

x0ne_status parse_config(const char* json_text, Cfg* c) {
    if (!json_text) return fail(X0NE_ERR_FORMAT, "config.json: no text given");
    Json root;
    try {
        root = parse_json(json_text);
    } catch (const std::exception& ex) {
        return fail(X0NE_ERR_FORMAT, std::string("config.json: ") + ex.what());
    }
    if (root.kind != Json::Object) return fail(X0NE_ERR_FORMAT, "config.json: the top level must be an object");
    ConfigReader r{root, {}};
    // The architecture: Qwen3 dense, or Qwen3-MoE with its sparse block (config.rs:329-335).
    const Json* arch = root.get("model_type");
    const bool dense = arch && arch->kind == Json::String && arch->text == "qwen3";
    c->moe = arch && arch->kind == Json::String && arch->text == "qwen3_moe";
    if (!dense && !c->moe) r.refuse("\"model_type\" must be \"qwen3\" or \"qwen3_moe\"");
    // Arithmetic: bf16 weights ("dtype", or the older "torch_dtype" when "dtype" is absent), a
    // SiLU-gated MLP, and none of bias, sliding windows or RoPE scaling.
    const Json* dtype = root.get("dtype") ? root.get("dtype") : root.get("torch_dtype");
    r.text(dtype, "dtype", "bfloat16");
    r.text(root.get("hidden_act"), "hidden_act", "silu");
    r.unset("attention_bias");
    r.unset("use_sliding_window");
    r.unset("rope_scaling");
    const Json* tie = root.get("tie_word_embeddings");
    if (tie && tie->kind != Json::Bool) r.refuse("\"tie_word_embeddings\" must be true or false");
    c->tied = tie && tie->kind == Json::Bool && tie->b;
    if (!r.refusal.empty()) return fail(X0NE_ERR_FORMAT, r.refusal);
    // The shape.
    const struct {
        const char* key;
        uint64_t* dst;
    } sizes[] = {{"hidden_size", &c->hidden},          {"intermediate_size", &c->inter},
                 {"num_hidden_layers", &c->layers},     {"num_attention_heads", &c->q_heads},
                 {"num_key_value_heads", &c->kv_heads}, {"head_dim", &c->head_dim},
                 {"vocab_size", &c->vocab},             {"max_position_embeddings", &c->max_pos}};
    for (const auto& s : sizes)
        if (!r.count(s.key, s.dst)) return fail(X0NE_ERR_FORMAT, r.refusal);
    if (!r.positive(root.get("rms_norm_eps"), "rms_norm_eps", &c->eps)) return fail(X0NE_ERR_FORMAT, r.refusal);
    // RoPE base: at the top level, or inside "rope_parameters" as transformers 5 writes it.
    const Json* theta = root.get("rope_theta");
    if (!theta && root.get("rope_parameters")) theta = root.get("rope_parameters")->get("rope_theta");
    if (!r.positive(theta, "rope_theta", &c->theta)) return fail(X0NE_ERR_FORMAT, r.refusal);
    if (c->moe) {
        // Every layer sparse, no shared expert, renormalised top-k routing.
        for (const char* key : {"shared_expert_intermediate_size", "n_shared_experts"}) {
            const Json* f = root.get(key);
            if (f && f->kind != Json::Null) r.refuse(std::string("\"") + key + "\": shared experts are not served");
        }
        uint64_t every = 0;
        if (r.count("decoder_sparse_step", &every) && every != 1)
            r.refuse("\"decoder_sparse_step\" must be 1: every layer sparse");
        const Json* dense_layers = root.get("mlp_only_layers");
        if (dense_layers && dense_layers->kind != Json::Null &&
            !(dense_layers->kind == Json::Array && dense_layers->items.empty()))
            r.refuse("\"mlp_only_layers\" must be empty: every layer sparse");
        const Json* renorm = root.get("norm_topk_prob");
        if (!renorm || renorm->kind != Json::Bool || !renorm->b)
            r.refuse("\"norm_topk_prob\" must be true: the chosen experts' weights are renormalised");
        if (!r.refusal.empty()) return fail(X0NE_ERR_FORMAT, r.refusal);
        if (!r.count("num_experts", &c->experts) || !r.count("num_experts_per_tok", &c->top_k) ||
            !r.count("moe_intermediate_size", &c->moe_inter))
            return fail(X0NE_ERR_FORMAT, r.refusal);
        if (c->top_k > c->experts) r.refuse("more experts per token than experts");
        if (c->experts > UINT32_MAX) r.refuse("expert ids must fit 32 bits");
    }
    // Relations between the sizes.
    if (c->q_heads % c->kv_heads != 0) r.refuse("every KV head must serve the same number of query heads");
    if (c->head_dim % 2 != 0) r.refuse("RoPE rotates pairs of dimensions: head_dim must be even");
    if (c->vocab > UINT32_MAX) r.refuse("token ids must fit 32 bits: vocab_size too large");
    // No size derived from the shape may overflow (config.rs check_sizes): weights of every
    // layer plus both vocabulary matrices, bounded well inside 64 bits.
    const long double mlp = c->moe ? (long double)c->experts * (3.0L * c->moe_inter * c->hidden + c->hidden)
                                   : 3.0L * c->inter * c->hidden;
    const long double params = (long double)c->layers * ((long double)c->qkv_rows() * c->hidden + mlp) +
                               2.0L * c->vocab * c->hidden;
    if (params > 1e18L) r.refuse("the shape's sizes overflow");
    if (!r.refusal.empty()) return fail(X0NE_ERR_FORMAT, r.refusal);
    return X0NE_OK;
}

// The accumulation an engine runs with: f64 when asked, or by default wherever this build has the
// exact kernels (a dense or MoE model decoding one sequence, 1, 2, 4 or 8 q heads per kv head);
// f32 when asked, and by default for batched engines (check_config has refused an f64 request
// those cannot serve).
bool exact_sums(const Cfg& c, const x0ne_engine_options& o) {
    if (o.sums == X0NE_SUMS_F64) return true;
    if (o.sums == X0NE_SUMS_F32) return false;
    const uint64_t grp = c.kv_heads ? c.q_heads / c.kv_heads : 0;
    return (o.max_batch == 0 || o.max_batch == 1) && (grp == 1 || grp == 2 || grp == 4 || grp == 8);
}

// What the kernels and the arena of this build accept (engine.rs:236-289 for the reference's
// own limits), for a checked config and the load's options; all of it before any device work.
x0ne_status check_config(const Cfg& c, const x0ne_engine_options& o) {
    const uint64_t max_ctx = o.max_ctx;
    auto no = [](const std::string& why) { return fail(X0NE_ERR_FORMAT, why); };
    if (c.moe) {  // expert count and width (kernels/src/lib.rs:147; engine.rs:236-262)
        if (c.experts == 0 || c.experts > MOE_MAX_EXPERTS)
            return no("MoE: " + std::to_string(c.experts) + " experts, the routing kernel takes 1 to " +
                      std::to_string(MOE_MAX_EXPERTS));
        if (c.top_k == 0 || c.top_k > MOE_MAX_TOP_K)
            return no("MoE: " + std::to_string(c.top_k) + " experts per token, the routing kernel takes 1 to " +
                      std::to_string(MOE_MAX_TOP_K));
        if (c.moe_inter == 0 || c.moe_inter % 8 != 0) return no("MoE: the expert width must be a multiple of 8");
        if (c.experts * 2 * c.moe_inter > UINT32_MAX || c.top_k * c.hidden > UINT32_MAX)
            return no("MoE: the expert matrices' rows must fit 32 bits");
    }
    if (c.head_dim != 128) return no("head_dim " + std::to_string(c.head_dim) + ": the attention kernels take 128");
    if (c.hidden % 8 != 0 || c.inter % 8 != 0)
        return no("hidden and intermediate sizes must be multiples of 8 (16-byte rows)");
    if (max_ctx == 0 || max_ctx > c.max_pos)
        return no("max_ctx " + std::to_string(max_ctx) + ": must be 1 to max_position_embeddings (" +
                  std::to_string(c.max_pos) + ")");
    const uint64_t seq_pages = (max_ctx + X0NE_PAGE_C - 1) / X0NE_PAGE_C;
    for (uint64_t s : {c.vocab, c.hidden, 2 * c.inter, c.qkv_rows(), max_ctx * c.kv_dim(),
                       seq_pages * X0NE_PAGE_C * c.kv_dim()})
        if (s > UINT32_MAX) return no("a row count or KV-plane element count exceeds 32 bits");
    // x is staged whole in LDS: a normed x (hidden) up to 16384 values, an attention output or an
    // activation (q_dim, intermediate) up to 32768.
    if (c.hidden > 16384) return no("hidden_size above 16384, the GEMV's staged x");
    if (c.q_dim() > 32768 || c.inter > 32768) return no("a projection wider than 32768 columns");
    // The options.
    const uint64_t batch = o.max_batch ? o.max_batch : 1;
    if (batch > MAX_BATCH) return no("max_batch " + std::to_string(batch) + " above " + std::to_string(MAX_BATCH));
    if (o.sums > X0NE_SUMS_F32) return no("sums " + std::to_string(o.sums) + ": 0 (default), 1 (f64) or 2 (f32)");
    if (o.sums == X0NE_SUMS_F64) {
        if (batch > 1) return fail(X0NE_ERR_NOT_IMPLEMENTED, "batched decoding with f64 sums");
        const uint64_t grp = c.q_heads / c.kv_heads;
        if (grp != 1 && grp != 2 && grp != 4 && grp != 8)
            return fail(X0NE_ERR_NOT_IMPLEMENTED,
                        "f64 sums: the exact attention kernels take 1, 2, 4 or 8 q heads per kv head, not " +
                            std::to_string(grp));
    }
    if (c.moe && batch > 1) return fail(X0NE_ERR_NOT_IMPLEMENTED, "a MoE engine decodes one sequence");
    // The attention kernels address a K or V plane (every sequence's pages of one layer) by 32-bit
    // byte offsets into a buffer resource of 0xFFFFFFF0 bytes, the offset 0xFFFFFFF0 standing for
    // "no key" (attention.hip, OFF_NONE). A plane must therefore end at or below that offset;
    // a larger one would wrap onto other pages (other sequences' keys), so it is refused here.
    const uint64_t plane = batch * seq_pages * X0NE_PAGE_C * c.kv_dim() * 2;
    if (plane > KV_PLANE_MAX_BYTES)
        return no("KV plane of " + std::to_string(plane) + " bytes (max_batch " + std::to_string(batch) + " x " +
                  std::to_string(seq_pages) + " pages of " + std::to_string(X0NE_PAGE_C * c.kv_dim() * 2) +
                  " bytes) above the attention kernels' " + std::to_string(KV_PLANE_MAX_BYTES) +
                  "-byte addressing: lower max_batch or max_ctx");
    return X0NE_OK;
}

// ---- the checkpoint's tensors (oracle/src/model.rs:63-89; weights.rs) ----

enum Leaf { L_INPUT_NORM, L_Q, L_K, L_V, L_QN, L_KN, L_O, L_POST_NORM, L_GATE, L_UP, L_DOWN, L_COUNT };
const char* LEAF_NAMES[L_COUNT] = {"input_layernorm", "self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj",
                                   "self_attn.q_norm", "self_attn.k_norm", "self_attn.o_proj",
                                   "post_attention_layernorm", "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj"};

std::vector<uint64_t> leaf_shape(const Cfg& c, int leaf) {
    switch (leaf) {
        case L_INPUT_NORM:
        case L_POST_NORM: return {c.hidden};
        case L_Q: return {c.q_dim(), c.hidden};
        case L_K:
        case L_V: return {c.kv_dim(), c.hidden};
        case L_QN:
        case L_KN: return {c.head_dim};
        case L_O: return {c.hidden, c.q_dim()};
        case L_GATE:
        case L_UP: return {c.inter, c.hidden};
        default: return {c.hidden, c.inter};
    }
}

std::string layer_name(uint64_t l, int leaf) {
    return "model.layers." + std::to_string(l) + "." + LEAF_NAMES[leaf] + ".weight";
}

// A Qwen3-MoE layer's feed-forward tensors (weights.rs:371-389): the router mlp.gate
// [experts][hidden] and per expert e mlp.experts.e.{gate,up}_proj [moe_inter][hidden] and
// down_proj [hidden][moe_inter].
std::string expert_name(uint64_t l, uint64_t e, const char* leaf) {
    return "model.layers." + std::to_string(l) + ".mlp.experts." + std::to_string(e) + "." + leaf + ".weight";
}
std::string router_name(uint64_t l) { return "model.layers." + std::to_string(l) + ".mlp.gate.weight"; }

// ---- safetensors in memory (st.rs:21-277) ----

struct TensorView {
    std::string dtype;
    std::vector<uint64_t> shape;
    const uint8_t* data = nullptr;
    uint64_t len = 0;
};

x0ne_status parse_safetensors(const std::string& file, const uint8_t* bytes, uint64_t len,
                              std::map<std::string, TensorView>* out) {
    if (len < 8) return fail(X0NE_ERR_FORMAT, file + ": shorter than a header length");
    uint64_t n = 0;
    for (int i = 7; i >= 0; --i) n = (n << 8) | bytes[i];
    if (n > len - 8 || n > (100ull << 20)) return fail(X0NE_ERR_FORMAT, file + ": header length " + std::to_string(n));
    Json h;
    try {
        h = parse_json(std::string((const char*)bytes + 8, n));
    } catch (const std::exception& ex) {
        return fail(X0NE_ERR_FORMAT, file + ": header: " + ex.what());
    }
    if (h.kind != Json::Object) return fail(X0NE_ERR_FORMAT, file + ": header is not an object");
    const uint8_t* data = bytes + 8 + n;
    const uint64_t data_len = len - 8 - n;
    for (const auto& f : h.fields) {
        if (f.first == "__metadata__") continue;
        const Json& t = f.second;
        const Json* dt = t.get("dtype");
        const Json* sh = t.get("shape");
        const Json* of = t.get("data_offsets");
        if (!dt || dt->kind != Json::String || !sh || sh->kind != Json::Array || !of || of->kind != Json::Array ||
            of->items.size() != 2)
            return fail(X0NE_ERR_FORMAT, file + ": " + f.first + ": malformed entry");
        TensorView v;
        v.dtype = dt->text;
        uint64_t count = 1;
        for (const auto& d : sh->items) {
            uint64_t x = 0;
            if (!d.as_u64(&x)) return fail(X0NE_ERR_FORMAT, file + ": " + f.first + ": bad shape");
            if (x && count > UINT64_MAX / x) return fail(X0NE_ERR_FORMAT, file + ": " + f.first + ": shape overflows");
            count *= x;
            v.shape.push_back(x);
        }
        uint64_t b = 0, e = 0;
        if (!of->items[0].as_u64(&b) || !of->items[1].as_u64(&e) || b > e || e > data_len)
            return fail(X0NE_ERR_FORMAT, file + ": " + f.first + ": data offsets outside the file");
        const uint64_t es = v.dtype == "BF16" || v.dtype == "F16" ? 2 : v.dtype == "F32" ? 4 : v.dtype == "F64" ? 8 : 0;
        if (es && (count > UINT64_MAX / es || count * es != e - b))
            return fail(X0NE_ERR_FORMAT, file + ": " + f.first + ": size does not match the shape");
        v.data = data + b;
        v.len = e - b;
        if (out->count(f.first)) return fail(X0NE_ERR_FORMAT, f.first + ": in two files");
        (*out)[f.first] = v;
    }
    return X0NE_OK;
}

// weights.rs:124-165: the exact tensor set, all BF16, every shape; a tied checkpoint may carry
// lm_head.weight only if it equals the embedding.
x0ne_status check_tensors(const Cfg& c, const std::map<std::string, TensorView>& t) {
    std::map<std::string, std::vector<uint64_t>> want;
    want["model.embed_tokens.weight"] = {c.vocab, c.hidden};
    for (uint64_t l = 0; l < c.layers; ++l) {
        for (int leaf = 0; leaf < L_COUNT; ++leaf) {
            if (c.moe && (leaf == L_GATE || leaf == L_UP || leaf == L_DOWN)) continue;
            want[layer_name(l, leaf)] = leaf_shape(c, leaf);
        }
        if (c.moe) {
            want[router_name(l)] = {c.experts, c.hidden};
            for (uint64_t e = 0; e < c.experts; ++e) {
                want[expert_name(l, e, "gate_proj")] = {c.moe_inter, c.hidden};
                want[expert_name(l, e, "up_proj")] = {c.moe_inter, c.hidden};
                want[expert_name(l, e, "down_proj")] = {c.hidden, c.moe_inter};
            }
        }
    }
    want["model.norm.weight"] = {c.hidden};
    if (!c.tied) want["lm_head.weight"] = {c.vocab, c.hidden};
    for (const auto& kv : t) {
        if (want.count(kv.first)) continue;
        if (c.tied && kv.first == "lm_head.weight") continue;
        return fail(X0NE_ERR_FORMAT, kv.first + ": unexpected tensor");
    }
    for (const auto& w : want) {
        auto it = t.find(w.first);
        if (it == t.end()) return fail(X0NE_ERR_FORMAT, w.first + ": missing tensor");
        if (it->second.dtype != "BF16") return fail(X0NE_ERR_FORMAT, w.first + ": dtype " + it->second.dtype + ", expected BF16");
        if (it->second.shape != w.second) return fail(X0NE_ERR_FORMAT, w.first + ": shape differs from the config's");
    }
    if (c.tied) {
        auto h = t.find("lm_head.weight");
        if (h != t.end()) {
            const auto& e = t.at("model.embed_tokens.weight");
            if (h->second.dtype != "BF16" || h->second.shape != e.shape || h->second.len != e.len ||
                std::memcmp(h->second.data, e.data, e.len) != 0)
                return fail(X0NE_ERR_FORMAT, "tied config, but lm_head.weight differs from the embedding");
        }
    }
    return X0NE_OK;
}

// splitmix64 output `index` of a generator seeded with `seed` (the tensor keys of the synthetic
// checkpoint; the oracle's xo_tensor_key).
uint64_t tensor_key(uint64_t seed, uint64_t index) {
    uint64_t z = seed + (index + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

}  // namespace

struct LayerW {
    x0ne_slice input_norm, qkv, q_norm, k_norm, o, post_norm, gate_up, down;
    x0ne_slice qkv_p{}, o_p{}, gate_up_p{}, down_p{};  // copies in 16-row panels (wpanel)
    x0ne_slice router{};  // MoE: [experts][hidden]; gate_up is then [experts][2 moe_inter][hidden],
                          // down [experts][hidden][moe_inter]
};

struct x0ne_engine {
    Cfg c;
    uint64_t max_ctx = 0, pages = 0, page_seed = 0;
    uint64_t chunk = 1;  // prompt rows per prefill pass; 1: one decode step per token
    uint64_t max_batch = 1, seq_pages = 0;  // sequences of the batched step; pages per sequence
    int f64_sums = 0;
    x0ne_gpu* gpu = nullptr;
    x0ne_arena* arena = nullptr;
    // weights
    x0ne_slice embed{}, final_norm{}, lm_head{};
    x0ne_slice head_p{};  // the LM head (or tied embedding) in 16-row panels (hpanel)
    bool has_lm_head = false;
    bool wpanel = false;  // the projections' panel copies exist: the batched step reads them
    bool ppanel = false;  // the prefill pass keeps W and X in panels (wpanel too)
    bool hpanel = false;  // the batched LM head reads head_p
    std::vector<LayerW> L;
    // buffers
    x0ne_slice inv_freq{}, rope_cs{}, page_table{}, kv{}, prompt{}, tokens{}, pos{}, residual{}, delta{}, qkv{}, q{}, attn{},
        act{}, logits{}, head_partial{}, head_counter{}, attn_state{}, attn_counter{};
    // A prefill pass's rows: f32 residual, bf16 delta, normed x, qkv, q, attention, [gate; up], act.
    x0ne_slice p_res{}, p_delta{}, p_x{}, p_qkv{}, p_q{}, p_attn{}, p_gu{}, p_act{};
    x0ne_slice p_tok{};  // a batched engine's pass of several sequences: their ids side by side
    x0ne_slice p_parts{};  // the exact mode's prefill GEMM: f64 partial sums of K slices
    // The batched step's rows ([max_batch][...]): f32 residual, bf16 delta, normed x, qkv,
    // attention, SwiGLU activation, f32 logits; its split-K state and counters.
    x0ne_slice b_res{}, b_delta{}, b_x{}, b_qkv{}, b_attn{}, b_act{}, b_logits{}, b_state{}, b_counter{}, b_argmax{};
    // The balanced few-row GEMM's parts and counts (runtime.hip, skinny).
    x0ne_slice b_few_ws{}, b_few_cnt{};
    // The MoE feed-forward's rows: the normed x, the router's f32 logits, each layer's chosen
    // expert ids and weights ([layers][top_k], read back by x0ne_engine_moe_routing), the chosen
    // experts' SwiGLU activations.
    x0ne_slice m_x{}, m_logits{}, m_ids{}, m_w{}, m_act{};
    std::vector<uint32_t> page_of;
    x0ne_split_plan split{}, bsplit{};
    uint32_t grid_qkv = 0, grid_o = 0, grid_gu = 0, grid_down = 0, grid_head = 0;
    x0ne_graph* graph = nullptr;
    x0ne_graph* bgraph = nullptr;  // the batched step for bgraph_batch sequences
    uint64_t bgraph_batch = 0;
    uint32_t mode = X0NE_DECODE_GRAPH;
    // The decode step's attention (Engine::decode_attention / split_merge, engine.rs:526-560):
    // split-K (the fused kernel for a grouped plan) or per head; the split-K states merged by the
    // last block of each kv head (grouped plans) or by the merge kernel.
    uint32_t attention = X0NE_ATTENTION_SPLIT_K;
    uint32_t merge = X0NE_MERGE_KERNEL;
    // host side (pinned)
    uint32_t* ring = nullptr;
    uint32_t* bring = nullptr;  // RING slots of max_batch token words
    hipEvent_t ring_ev[RING] = {};
    float* host_logits = nullptr;
    hipEvent_t logits_ev = nullptr;
    uint32_t* host_token = nullptr;
    bool poisoned = false;
    bool session_open = false;

    ~x0ne_engine() {
        // Drain the stream first: a graph's executable must not be destroyed while a replay of it
        // is still queued (a caller that frees the engine with steps in flight).
        if (gpu && gpu->stream) (void)hipStreamSynchronize(gpu->stream);
        if (graph) x0ne_graph_free(graph);
        if (bgraph) x0ne_graph_free(bgraph);
        for (auto& ev : ring_ev)
            if (ev) (void)hipEventDestroy(ev);
        if (logits_ev) (void)hipEventDestroy(logits_ev);
        if (ring) (void)hipHostFree(ring);
        if (bring) (void)hipHostFree(bring);
        if (host_logits) (void)hipHostFree(host_logits);
        if (host_token) (void)hipHostFree(host_token);
        if (arena) x0ne_arena_free(arena);
        if (gpu) x0ne_gpu_free(gpu);
    }
    uint8_t* d(x0ne_slice s) const { return dev(arena, s); }
    uint64_t plane_bytes() const { return pages * X0NE_PAGE_C * c.kv_dim() * 2; }
    // K (kv = 0) or V (kv = 1) plane of layer l.
    uint8_t* plane(uint64_t l, int kvsel) const { return d(kv) + (2 * l + kvsel) * plane_bytes(); }
    // Sequence b's page table, position, token and prompt row (b = 0: the single-sequence ones).
    const uint32_t* pages_of(uint64_t b) const { return (const uint32_t*)d(page_table) + b * seq_pages; }
    uint32_t* pos_of(uint64_t b) const { return (uint32_t*)d(pos) + b; }
    uint32_t* token_of(uint64_t b) const { return (uint32_t*)d(tokens) + b; }
    const uint32_t* prompt_of(uint64_t b) const { return (const uint32_t*)d(prompt) + b * max_ctx; }
};

struct x0ne_session {
    x0ne_engine* e = nullptr;
    size_t pos = 0;
    bool open = true;
    bool failed = false;
};

struct x0ne_greedy {
    x0ne_session* s = nullptr;
    size_t max_tokens = 0, ahead = 0, taken = 0, launched = 0;
    uint32_t first = 0;
};

namespace {

x0ne_status plan(x0ne_engine* e) {
    x0ne_arena* a = e->arena;
    const Cfg& c = e->c;
    const uint32_t W = X0NE_CLASS_WEIGHTS, CD = X0NE_CLASS_CLIENT_DATA;
    auto al = [&](const char* label, uint64_t len, uint32_t cls, x0ne_slice* s) {
        return x0ne_arena_alloc(a, label, len, cls, s);
    };
    X0NE_TRY(al("embed", c.vocab * c.hidden * 2, W, &e->embed));
    e->L.resize(c.layers);
    for (uint64_t l = 0; l < c.layers; ++l) {
        LayerW& w = e->L[l];
        X0NE_TRY(al("input_norm", c.hidden * 2, W, &w.input_norm));
        X0NE_TRY(al("qkv", c.qkv_rows() * c.hidden * 2, W, &w.qkv));
        X0NE_TRY(al("q_norm", c.head_dim * 2, W, &w.q_norm));
        X0NE_TRY(al("k_norm", c.head_dim * 2, W, &w.k_norm));
        X0NE_TRY(al("o", c.hidden * c.q_dim() * 2, W, &w.o));
        X0NE_TRY(al("post_norm", c.hidden * 2, W, &w.post_norm));
        if (c.moe) {
            X0NE_TRY(al("router", c.experts * c.hidden * 2, W, &w.router));
            X0NE_TRY(al("experts_gate_up", c.experts * 2 * c.moe_inter * c.hidden * 2, W, &w.gate_up));
            X0NE_TRY(al("experts_down", c.experts * c.hidden * c.moe_inter * 2, W, &w.down));
        } else {
            X0NE_TRY(al("gate_up", 2 * c.inter * c.hidden * 2, W, &w.gate_up));
            X0NE_TRY(al("down", c.hidden * c.inter * 2, W, &w.down));
        }
    }
    X0NE_TRY(al("final_norm", c.hidden * 2, W, &e->final_norm));
    e->has_lm_head = !c.tied;
    if (e->has_lm_head) X0NE_TRY(al("lm_head", c.vocab * c.hidden * 2, W, &e->lm_head));
    // A second copy of the projections in 16-row panels (device.h), filled from the row-major
    // copy at load, for a batched engine (the few-row GEMM then reads one contiguous KiB of W per
    // step instead of 64 bytes of 16 rows) and for a prefill pass of more than one row (the
    // tiled GEMM's loads fetch whole 1 KiB fragments: 25 TB/s from the L2 against 9.5
    // row-major on MI355X). The prefill pass's GEMM inputs (normed rows, attention, SwiGLU) are
    // then written in panels too. A batched engine's LM head has a panel copy as well.
    const bool dims16 = c.qkv_rows() % 16 == 0 && c.hidden % 16 == 0 && c.inter % 16 == 0;
    const uint64_t group = c.q_heads / c.kv_heads;
    e->ppanel = dims16 && e->chunk > 1 && !c.moe && !e->f64_sums && (group == 1 || group == 2 || group == 4 || group == 8);
    e->hpanel = dims16 && e->max_batch > 1 && c.vocab % 16 == 0;
    e->wpanel = e->ppanel || (dims16 && e->max_batch > 1);
    if (e->wpanel) {
        for (uint64_t l = 0; l < c.layers; ++l) {
            LayerW& w = e->L[l];
            X0NE_TRY(al("qkv_panel", c.qkv_rows() * c.hidden * 2, W, &w.qkv_p));
            X0NE_TRY(al("o_panel", c.hidden * c.q_dim() * 2, W, &w.o_p));
            X0NE_TRY(al("gate_up_panel", 2 * c.inter * c.hidden * 2, W, &w.gate_up_p));
            X0NE_TRY(al("down_panel", c.hidden * c.inter * 2, W, &w.down_p));
        }
    }
    if (e->hpanel) X0NE_TRY(al("lm_head_panel", c.vocab * c.hidden * 2, W, &e->head_p));
    // Engine tables, not client data: the host's f32 inverse frequencies and the page order.
    X0NE_TRY(al("inv_freq", c.head_dim / 2 * 4, W, &e->inv_freq));
    X0NE_TRY(al("rope_cs", e->max_ctx * (c.head_dim / 2) * 16, W, &e->rope_cs));
    X0NE_TRY(al("page_table", e->pages * 4, W, &e->page_table));
    // Client data.
    X0NE_TRY(al("kv_cache", 2 * c.layers * e->plane_bytes(), CD, &e->kv));
    X0NE_TRY(al("prompt", e->max_batch * e->max_ctx * 4, CD, &e->prompt));
    X0NE_TRY(al("tokens", e->max_batch * 4, CD, &e->tokens));
    X0NE_TRY(al("pos", e->max_batch * 4, CD, &e->pos));
    X0NE_TRY(al("residual", 2 * c.hidden * 4, CD, &e->residual));
    X0NE_TRY(al("delta", c.hidden * 2, CD, &e->delta));
    X0NE_TRY(al("qkv_out", c.qkv_rows() * 2, CD, &e->qkv));
    X0NE_TRY(al("q", c.q_dim() * 2, CD, &e->q));
    X0NE_TRY(al("attn", c.q_dim() * 2, CD, &e->attn));
    X0NE_TRY(al("act", c.inter * 2, CD, &e->act));
    X0NE_TRY(al("logits", c.vocab * 4, CD, &e->logits));
    X0NE_TRY(al("head_partial", (uint64_t)e->grid_head * 3 * 4, CD, &e->head_partial));
    X0NE_TRY(al("head_counter", 4, CD, &e->head_counter));
    // The exact mode's split state is f64: twice the bytes.
    X0NE_TRY(al("attention_split_state",
                x0ne_split_state_bytes((uint32_t)c.q_heads, e->split.splits) * (e->f64_sums ? 2 : 1), CD,
                &e->attn_state));
    X0NE_TRY(al("attention_split_counter", c.kv_heads * 4, CD, &e->attn_counter));
    if (c.moe) {
        X0NE_TRY(al("moe_normed", c.hidden * 2, CD, &e->m_x));
        X0NE_TRY(al("moe_router_logits", c.experts * 4, CD, &e->m_logits));
        X0NE_TRY(al("moe_ids", c.layers * c.top_k * 4, CD, &e->m_ids));
        X0NE_TRY(al("moe_weights", c.layers * c.top_k * 4, CD, &e->m_w));
        X0NE_TRY(al("moe_act", c.top_k * c.moe_inter * 2, CD, &e->m_act));
    }
    if (e->chunk > 1) {
        // The GEMM inputs in panels hold whole tiles of 16 rows.
        const uint64_t n = e->chunk, np = e->ppanel ? (n + 15) / 16 * 16 : n;
        X0NE_TRY(al("prefill_residual", n * c.hidden * 4, CD, &e->p_res));
        X0NE_TRY(al("prefill_delta", n * c.hidden * 2, CD, &e->p_delta));
        X0NE_TRY(al("prefill_normed", np * c.hidden * 2, CD, &e->p_x));
        X0NE_TRY(al("prefill_qkv", n * c.qkv_rows() * 2, CD, &e->p_qkv));
        X0NE_TRY(al("prefill_q", n * c.q_dim() * 2, CD, &e->p_q));
        X0NE_TRY(al("prefill_attn", np * c.q_dim() * 2, CD, &e->p_attn));
        X0NE_TRY(al("prefill_gate_up", n * 2 * c.inter * 2, CD, &e->p_gu));
        X0NE_TRY(al("prefill_act", np * c.inter * 2, CD, &e->p_act));
        if (e->max_batch > 1) X0NE_TRY(al("prefill_ids", n * 4, CD, &e->p_tok));
        if (e->f64_sums) X0NE_TRY(al("prefill_f64_parts", EXACT_PARTS_BYTES, CD, &e->p_parts));
    }
    if (e->max_batch > 1) {
        const uint64_t b = e->max_batch, bp = (b + 15) / 16 * 16;  // panels hold whole tiles of 16 rows
        X0NE_TRY(al("batch_residual", b * c.hidden * 4, CD, &e->b_res));
        X0NE_TRY(al("batch_delta", b * c.hidden * 2, CD, &e->b_delta));
        X0NE_TRY(al("batch_normed", bp * c.hidden * 2, CD, &e->b_x));
        X0NE_TRY(al("batch_qkv", b * c.qkv_rows() * 2, CD, &e->b_qkv));
        X0NE_TRY(al("batch_attn", bp * c.q_dim() * 2, CD, &e->b_attn));
        X0NE_TRY(al("batch_act", bp * c.inter * 2, CD, &e->b_act));
        X0NE_TRY(al("batch_logits", b * c.vocab * 4, CD, &e->b_logits));
        X0NE_TRY(al("batch_split_state", b * x0ne_split_state_bytes((uint32_t)c.q_heads, e->bsplit.splits), CD,
                    &e->b_state));
        X0NE_TRY(al("batch_split_counter", b * c.kv_heads * 4, CD, &e->b_counter));
        X0NE_TRY(al("batch_argmax", b * ARGMAX_SLICES * 3 * 4, CD, &e->b_argmax));
        const uint64_t groups = std::max<uint64_t>(c.hidden, c.qkv_rows()) / 16;
        X0NE_TRY(al("batch_gemm_parts", groups * 2 * 256 * 4, CD, &e->b_few_ws));
        X0NE_TRY(al("batch_gemm_counts", groups * 4, CD, &e->b_few_cnt));
    }
    return X0NE_OK;
}

// The GEMV grids of a decode step: the kernel's occupancy on this device, the row groups split
// evenly over the resident wavefronts (x0ne_gemv_grid). X0NE_GEMV_BLOCKS_PER_CU caps the blocks
// per CU (a tuning knob; unset, the occupancy decides).
x0ne_status plan_grids(x0ne_engine* e) {
    const Cfg& c = e->c;
    static const char* env = std::getenv("X0NE_GEMV_BLOCKS_PER_CU");
    const uint32_t cap = env && std::atoi(env) > 0 ? (uint32_t)std::atoi(env) : 0;
    auto grid = [&](uint64_t rows, uint64_t cols, int pro, int epi, uint32_t* out) -> x0ne_status {
        X0neGemv a = {};
        a.rows = (uint32_t)rows;
        a.cols = (uint32_t)cols;
        a.prologue = pro;
        a.epilogue = epi;
        a.f64acc = e->f64_sums;
        *out = x0ne_gemv_grid(a, e->gpu->cus, cap);
        if (*out == 0) return fail(X0NE_ERR_FORMAT, "a projection shape the GEMV refuses");
        return X0NE_OK;
    };
    X0NE_TRY(grid(c.qkv_rows(), c.hidden, 1, 0, &e->grid_qkv));
    X0NE_TRY(grid(c.hidden, c.q_dim(), 0, 0, &e->grid_o));
    X0NE_TRY(grid(2 * c.inter, c.hidden, 1, 2, &e->grid_gu));
    X0NE_TRY(grid(c.hidden, c.inter, 0, 0, &e->grid_down));
    return grid(c.vocab, c.hidden, 1, 3, &e->grid_head);
}

// The kernels of one decode step, one helper each. Norm j of the step reads residual buffer
// j % 2 and writes (j + 1) % 2: layer l's QKV norm is j = 2l, its gate/up norm 2l + 1, the final
// norm 2L.
float* residual_buf(const x0ne_engine* e, int k) { return (float*)e->d(e->residual) + (k & 1) * e->c.hidden; }

x0ne_status launch_qkv(x0ne_engine* e, uint64_t l) {
    const Cfg& c = e->c;
    const LayerW& w = e->L[l];
    X0neGemv a = {};
    a.w = (const uint16_t*)e->d(w.qkv);
    a.res_in = residual_buf(e, 0);
    a.res_out = residual_buf(e, 1);
    a.delta = (const uint16_t*)e->d(e->delta);
    a.norm_w = (const uint16_t*)e->d(w.input_norm);
    a.embed = (const uint16_t*)e->d(e->embed);
    a.tokens = (const uint32_t*)e->d(e->tokens);
    a.vocab = (uint32_t)c.vocab;
    a.y = e->d(e->qkv);
    a.rows = (uint32_t)c.qkv_rows();
    a.cols = (uint32_t)c.hidden;
    a.eps = (float)c.eps;
    a.prologue = l == 0 ? 2 : 1;  // layer 0 adds the embedding row to a zero residual
    a.epilogue = 0;
    a.grid = e->grid_qkv;
    a.f64acc = e->f64_sums;
    e->gpu->counts.launches++;
    X0NE_HIP(x0ne_launch_gemv(a, e->gpu->stream), "qkv gemv");
    return X0NE_OK;
}

x0ne_status launch_rope(x0ne_engine* e, uint64_t l) {
    const Cfg& c = e->c;
    const LayerW& w = e->L[l];
    const uint32_t qh = (uint32_t)c.q_heads, kvh = (uint32_t)c.kv_heads;
    e->gpu->counts.launches++;
    const void* qkv = e->d(e->qkv);
    const void* qn = e->d(w.q_norm);
    const void* kn = e->d(w.k_norm);
    const void* inv = e->d(e->inv_freq);
    void* q = e->d(e->q);
    void* kc = e->plane(l, 0);
    void* vc = e->plane(l, 1);
    const void* pt = e->d(e->page_table);
    const void* pos = e->d(e->pos);
    uint32_t max_ctx = (uint32_t)e->max_ctx;
    float eps = (float)c.eps;
    void* args[] = {(void*)&qkv, (void*)&qn, (void*)&kn,      (void*)&inv, (void*)&q,   (void*)&kc,  (void*)&vc,
                    (void*)&pt,  (void*)&pos, (void*)&qh, (void*)&kvh, (void*)&max_ctx, (void*)&eps};
    X0NE_HIP(x0ne_launch((const void*)&x0ne_qk_norm_rope_kv_write_bf16, dim3(qh + kvh, 1), dim3(64), args, 0,
                         e->gpu->stream),
             "qk_norm_rope_kv_write");
    return X0NE_OK;
}

// The decode attention of layer l. Split-K on a grouped plan is one fused launch (QK-norm +
// RoPE + K/V write + split-K), merged by its last block or followed by the merge kernel; the
// exact mode's fused kernel always merges in its last block. Otherwise the QK-norm/RoPE kernel,
// then split-K and the merge kernel, or the per-head kernel (engine.rs:744-764).
x0ne_status launch_attention(x0ne_engine* e, uint64_t l) {
    const Cfg& c = e->c;
    const float scale = (float)(1.0 / std::sqrt((double)c.head_dim));  // ops.rs:217-219
    const uint32_t qh = (uint32_t)c.q_heads, kvh = (uint32_t)c.kv_heads, max_ctx = (uint32_t)e->max_ctx;
    if (e->attention == X0NE_ATTENTION_SPLIT_K && e->split.grouped) {  // the exact mode is grouped (load check)
        const LayerW& w = e->L[l];
        const bool last = e->f64_sums || e->merge == X0NE_MERGE_LAST_BLOCK;
        X0NE_TRY(attention_rope_split(e->gpu, e->split, e->d(e->qkv), e->d(w.q_norm), e->d(w.k_norm),
                                      e->d(e->inv_freq), e->d(e->rope_cs), e->plane(l, 0), e->plane(l, 1),
                                      e->d(e->page_table), e->d(e->attn_state),
                                      last ? e->d(e->attn_counter) : nullptr, e->d(e->attn), e->d(e->pos), qh, kvh,
                                      max_ctx, scale, (float)c.eps, e->f64_sums != 0));
        return last ? X0NE_OK : attention_merge(e->gpu, e->split, e->d(e->attn_state), e->d(e->attn), e->d(e->pos),
                                                qh, max_ctx);
    }
    X0NE_TRY(launch_rope(e, l));
    if (e->attention == X0NE_ATTENTION_PER_HEAD) {
        const void* q = e->d(e->q);
        const void* kc = e->plane(l, 0);
        const void* vc = e->plane(l, 1);
        const void* pt = e->d(e->page_table);
        void* out = e->d(e->attn);
        const void* pos = e->d(e->pos);
        uint32_t mc = max_ctx;
        float sc = scale;
        void* args[] = {(void*)&q,   (void*)&kc, (void*)&vc,  (void*)&pt, (void*)&out,
                        (void*)&pos, (void*)&qh, (void*)&kvh, (void*)&mc, (void*)&sc};
        e->gpu->counts.launches++;
        X0NE_HIP(x0ne_launch((const void*)&x0ne_attention_decode_bf16, dim3(qh), dim3(256), args, 0, e->gpu->stream),
                 "per-head decode attention");
        return X0NE_OK;
    }
    return attention_split(e->gpu, e->split, e->merge == X0NE_MERGE_LAST_BLOCK ? 1 : 0, e->d(e->q), e->plane(l, 0),
                           e->plane(l, 1), e->d(e->page_table), e->d(e->attn_state), e->d(e->attn_counter),
                           e->d(e->attn), e->d(e->pos), qh, kvh, max_ctx, scale);
}

x0ne_status launch_o(x0ne_engine* e, uint64_t l) {
    const Cfg& c = e->c;
    X0neGemv o = {};
    o.w = (const uint16_t*)e->d(e->L[l].o);
    o.x = (const uint16_t*)e->d(e->attn);
    o.y = e->d(e->delta);
    o.rows = (uint32_t)c.hidden;
    o.cols = (uint32_t)c.q_dim();
    o.prologue = 0;
    o.epilogue = 0;
    o.grid = e->grid_o;
    o.f64acc = e->f64_sums;
    e->gpu->counts.launches++;
    X0NE_HIP(x0ne_launch_gemv(o, e->gpu->stream), "o gemv");
    return X0NE_OK;
}

x0ne_status launch_gate_up(x0ne_engine* e, uint64_t l) {
    const Cfg& c = e->c;
    X0neGemv gu = {};
    gu.w = (const uint16_t*)e->d(e->L[l].gate_up);
    gu.res_in = residual_buf(e, 1);
    gu.res_out = residual_buf(e, 0);
    gu.delta = (const uint16_t*)e->d(e->delta);
    gu.norm_w = (const uint16_t*)e->d(e->L[l].post_norm);
    gu.y = e->d(e->act);
    gu.rows = (uint32_t)(2 * c.inter);
    gu.cols = (uint32_t)c.hidden;
    gu.eps = (float)c.eps;
    gu.prologue = 1;
    gu.epilogue = 2;  // SwiGLU over [gate; up]
    gu.grid = e->grid_gu;
    gu.f64acc = e->f64_sums;
    e->gpu->counts.launches++;
    X0NE_HIP(x0ne_launch_gemv(gu, e->gpu->stream), "gate_up gemv");
    return X0NE_OK;
}

x0ne_status launch_down(x0ne_engine* e, uint64_t l) {
    const Cfg& c = e->c;
    X0neGemv dn = {};
    dn.w = (const uint16_t*)e->d(e->L[l].down);
    dn.x = (const uint16_t*)e->d(e->act);
    dn.y = e->d(e->delta);
    dn.rows = (uint32_t)c.hidden;
    dn.cols = (uint32_t)c.inter;
    dn.prologue = 0;
    dn.epilogue = 0;
    dn.grid = e->grid_down;
    dn.f64acc = e->f64_sums;
    e->gpu->counts.launches++;
    X0NE_HIP(x0ne_launch_gemv(dn, e->gpu->stream), "down gemv");
    return X0NE_OK;
}

// Final norm, the LM head (f32 logits), the argmax into tokens[0] and pos += 1.
x0ne_status launch_head(x0ne_engine* e) {
    const Cfg& c = e->c;
    X0neGemv hd = {};
    hd.w = (const uint16_t*)e->d(e->has_lm_head ? e->lm_head : e->embed);
    hd.res_in = residual_buf(e, 0);
    hd.res_out = nullptr;
    hd.delta = (const uint16_t*)e->d(e->delta);
    hd.norm_w = (const uint16_t*)e->d(e->final_norm);
    hd.y = e->d(e->logits);
    hd.partial = (float*)e->d(e->head_partial);
    hd.counter = (uint32_t*)e->d(e->head_counter);
    hd.token_out = (uint32_t*)e->d(e->tokens);
    hd.pos = (uint32_t*)e->d(e->pos);
    hd.advance = 1;
    hd.rows = (uint32_t)c.vocab;
    hd.cols = (uint32_t)c.hidden;
    hd.eps = (float)c.eps;
    hd.prologue = 1;
    hd.epilogue = 3;
    hd.grid = e->grid_head;
    hd.f64acc = e->f64_sums;
    e->gpu->counts.launches++;
    X0NE_HIP(x0ne_launch_gemv(hd, e->gpu->stream), "lm_head gemv");
    return X0NE_OK;
}

// The launches of one decode step at the device's pos on the device's tokens[0]: forward,
// logits, argmax into tokens[0], pos += 1. No host copy and no synchronisation, so the
// sequence can be captured (engine.rs:495-501, :718-839).
x0ne_status launch_rows(x0ne_engine* e, const void* fn, dim3 grid, dim3 block, void** args, const char* what);

// The sparse feed-forward of layer l (engine.rs:795-815): add + RMSNorm from residual buffer 1
// into buffer 0 (the norm the dense gate/up GEMV fuses), the router GEMV (f32 logits), the
// routing into layer l's ids and weights, the chosen experts' [gate; up] projections with SwiGLU
// behind, and their down projections with the weighted combination behind, into delta.
x0ne_status launch_moe(x0ne_engine* e, uint64_t l) {
    const Cfg& c = e->c;
    const LayerW& w = e->L[l];
    const uint32_t h = (uint32_t)c.hidden, ne = (uint32_t)c.experts, k = (uint32_t)c.top_k, mi = (uint32_t)c.moe_inter;
    {
        const void* rin = residual_buf(e, 1);
        void* rout = residual_buf(e, 0);
        const void* dl = e->d(e->delta);
        const void* nw = e->d(w.post_norm);
        void* xo = e->d(e->m_x);
        float eps = (float)c.eps;
        void* args[] = {(void*)&rin, (void*)&rout, (void*)&dl, (void*)&nw, (void*)&xo, (void*)&h, (void*)&eps};
        X0NE_TRY(launch_rows(e, (const void*)&x0ne_add_rmsnorm_to_bf16, dim3(1), dim3(256), args, "moe norm"));
    }
    {  // router logits in f32, summed as the engine sums
        X0neGemv r = {};
        r.w = (const uint16_t*)e->d(w.router);
        r.x = (const uint16_t*)e->d(e->m_x);
        r.y = e->d(e->m_logits);
        r.rows = ne;
        r.cols = h;
        r.prologue = 0;
        r.epilogue = 1;
        r.grid = x0ne_gemv_grid(r, e->gpu->cus, 0);
        r.f64acc = e->f64_sums;
        e->gpu->counts.gemms++;
        e->gpu->counts.launches++;
        X0NE_HIP(x0ne_launch_gemv(r, e->gpu->stream), "router gemv");
    }
    void* ids = e->d(e->m_ids) + l * c.top_k * 4;
    void* wts = e->d(e->m_w) + l * c.top_k * 4;
    {
        const void* lg = e->d(e->m_logits);
        void* args[] = {(void*)&lg, (void*)&ne, (void*)&k, (void*)&ids, (void*)&wts};
        X0NE_TRY(launch_rows(e, (const void*)&x0ne_moe_route_f32, dim3(1), dim3(64), args, "moe route"));
    }
    {
        const void* wg = e->d(w.gate_up);
        const void* x = e->d(e->m_x);
        void* act = e->d(e->m_act);
        void* args[] = {(void*)&wg, (void*)&ids, (void*)&x, (void*)&act, (void*)&mi, (void*)&h, (void*)&ne};
        X0NE_TRY(launch_rows(e,
                             e->f64_sums ? (const void*)&x0ne_moe_gate_up_swiglu_exact_bf16
                                         : (const void*)&x0ne_moe_gate_up_swiglu_bf16,
                             dim3((mi + 7) / 8, k), dim3(256), args, "moe gate_up + swiglu"));
    }
    const void* wd = e->d(w.down);
    const void* wc = wts;
    const void* act = e->d(e->m_act);
    void* out = e->d(e->delta);
    void* args[] = {(void*)&wd, (void*)&ids, (void*)&wc, (void*)&act, (void*)&out, (void*)&h, (void*)&mi, (void*)&ne,
                    (void*)&k};
    return launch_rows(e,
                       e->f64_sums ? (const void*)&x0ne_moe_down_combine_exact_bf16
                                   : (const void*)&x0ne_moe_down_combine_bf16,
                       dim3((h + 7) / 8), dim3(256), args, "moe down + combination");
}

x0ne_status step_launches(x0ne_engine* e) {
    for (uint64_t l = 0; l < e->c.layers; ++l) {
        X0NE_TRY(launch_qkv(e, l));
        X0NE_TRY(launch_attention(e, l));
        X0NE_TRY(launch_o(e, l));
        if (e->c.moe) {
            X0NE_TRY(launch_moe(e, l));
            continue;
        }
        X0NE_TRY(launch_gate_up(e, l));
        X0NE_TRY(launch_down(e, l));
    }
    return launch_head(e);
}

x0ne_status run_step(x0ne_engine* e) {
    if (e->mode == X0NE_DECODE_GRAPH) {
        if (!e->graph) return fail(X0NE_ERR_GPU, "no decode graph captured");
        return x0ne_gpu_launch_graph(e->gpu, e->graph);
    }
    return step_launches(e);
}

// Prompt token i through the step: ids[i] into tokens[0], i into pos (from the prompt buffer).
x0ne_status feed(x0ne_engine* e, uint32_t i) {
    e->gpu->counts.launches++;
    hipLaunchKernelGGL(x0ne_feed_u32, dim3(1), dim3(64), 0, e->gpu->stream, (const uint32_t*)e->d(e->prompt), i,
                       (uint32_t*)e->d(e->tokens), (uint32_t*)e->d(e->pos));
    X0NE_HIP(hipGetLastError(), "feed");
    return run_step(e);
}

x0ne_status put_prompt(x0ne_engine* e, const uint32_t* ids, size_t n) {
    return x0ne_arena_write(e->arena, e->prompt, 0, ids, n * 4);
}

// Sequence b's token = its prompt[i], its position = i, without a step.
x0ne_status set_position(x0ne_engine* e, uint64_t i, uint64_t b = 0) {
    e->gpu->counts.launches++;
    hipLaunchKernelGGL(x0ne_feed_u32, dim3(1), dim3(64), 0, e->gpu->stream, e->prompt_of(b), (uint32_t)i,
                       e->token_of(b), e->pos_of(b));
    X0NE_HIP(hipGetLastError(), "position");
    return X0NE_OK;
}

x0ne_status launch_rows(x0ne_engine* e, const void* fn, dim3 grid, dim3 block, void** args, const char* what) {
    e->gpu->counts.launches++;
    X0NE_HIP(x0ne_launch(fn, grid, block, args, 0, e->gpu->stream), what);
    return X0NE_OK;
}

// Y[n][rows] = X[n][cols] W^T on arena slices (Gpu::gemm, bf16 out). A panel prefill pass
// (ppanel) passes W's panel copy and X in panels: up to 64 rows the few-row GEMM, more the tiled
// GEMM. The exact mode's: the f64-sum GEMM (its K slices' parts in p_parts). Y is row-major.
x0ne_status gemm(x0ne_engine* e, x0ne_slice w, x0ne_slice w_panels, uint64_t rows, uint64_t cols, x0ne_slice x,
                 uint64_t n, x0ne_slice y) {
    if (e->f64_sums)
        return exact_gemm(e->gpu, e->d(w), rows, cols, e->d(x), n, e->d(y), false, (double*)e->d(e->p_parts),
                          EXACT_PARTS_BYTES);
    if (!e->ppanel)
        return x0ne_gpu_gemv(e->gpu, (uint64_t)(uintptr_t)e->d(w), rows, cols, (uint64_t)(uintptr_t)e->d(x), n,
                             (uint64_t)(uintptr_t)e->d(y), 0);
    if (n <= 64) return skinny(e->gpu, e->d(w_panels), rows, cols, e->d(x), n, e->d(y), 0, PANEL_X | PANEL_W);
    return tiled_gemm(e->gpu, 0, X0NE_GEMM_W_PANELS | X0NE_GEMM_X_PANELS, e->d(w_panels), rows, cols, e->d(x), n,
                      e->d(y), false);
}

// Prompt rows pos0 .. pos0 + n - 1 through every layer (engine.rs:729-839 with n rows): the
// embedding into delta and a zero residual, then per layer add + RMSNorm, the QKV GEMM, QK-norm
// + RoPE with the K/V rows written at their positions, the causal attention (matrix-core kernel
// for 1, 2, 4 or 8 q heads per kv head), the O GEMM, add + RMSNorm, the gate/up GEMM, SwiGLU,
// the down GEMM. Leaves the rows' residual and last delta for the final norm. Sequence b: its
// prompt row, position and KV pages. With ppanel the GEMM inputs are written in panels (the same
// values at panel_index) and the GEMMs read W's panel copies.
// seqs > 1 (a batched engine's prompts of one length): sequences b .. b + seqs - 1 in one pass,
// n rows each at the same positions, side by side (rows s n .. s n + n - 1 are sequence b + s):
// the GEMMs, norms and SwiGLU take all seqs n rows at once, QK-norm + RoPE and the attention run
// per sequence on its rows, pages and position. With panels n is a multiple of 16, so each
// sequence's rows start a panel.
x0ne_status prefill_pass(x0ne_engine* e, uint64_t pos0, uint64_t n, uint64_t b = 0, uint64_t seqs = 1) {
    const Cfg& c = e->c;
    if (e->chunk < 2 || n == 0 || seqs == 0 || n * seqs > e->chunk || pos0 + n > e->max_ctx || b + seqs > e->max_batch ||
        (seqs > 1 && e->ppanel && n % 16 != 0))
        return fail(X0NE_ERR_FORMAT, "prefill: " + std::to_string(seqs) + " x " + std::to_string(n) + " rows at " +
                                         std::to_string(pos0));
    for (uint64_t s = 0; s < seqs; ++s) X0NE_TRY(set_position(e, pos0, b + s));
    const uint32_t sn = (uint32_t)n;  // rows of one sequence
    n *= seqs;
    const uint32_t rows = (uint32_t)n, h = (uint32_t)c.hidden, vocab = (uint32_t)c.vocab, inter = (uint32_t)c.inter;
    const uint32_t qh = (uint32_t)c.q_heads, kvh = (uint32_t)c.kv_heads, max_ctx = (uint32_t)e->max_ctx;
    const float eps = (float)c.eps, scale = (float)(1.0 / std::sqrt((double)c.head_dim));
    {
        const void* table = e->d(e->embed);
        const void* toks = e->prompt_of(b) + pos0;
        if (seqs > 1) {  // the sequences' ids of this pass side by side
            e->gpu->counts.launches++;
            X0NE_HIP(hipMemcpy2DAsync(e->d(e->p_tok), (size_t)sn * 4, toks, e->max_ctx * 4, (size_t)sn * 4, seqs,
                                      hipMemcpyDeviceToDevice, e->gpu->stream),
                     "pass ids");
            toks = e->d(e->p_tok);
        }
        void* out = e->d(e->p_delta);
        void* args[] = {(void*)&table, (void*)&toks, (void*)&out, (void*)&h, (void*)&vocab};
        X0NE_TRY(launch_rows(e, (const void*)&x0ne_embedding_bf16, dim3(rows), dim3(128), args, "embedding"));
    }
    e->gpu->counts.memsets++;
    X0NE_HIP(hipMemsetAsync(e->d(e->p_res), 0, n * c.hidden * 4, e->gpu->stream), "residual");
    void* res = e->d(e->p_res);
    void* dl = e->d(e->p_delta);
    void* xn = e->d(e->p_x);
    auto norm = [&](x0ne_slice w) {
        const void* wp = e->d(w);
        void* args[] = {(void*)&res, (void*)&dl, (void*)&wp, (void*)&xn, (void*)&h, (void*)&eps};
        return launch_rows(e, e->ppanel ? (const void*)&x0ne_add_rmsnorm_panel_bf16 : (const void*)&x0ne_add_rmsnorm_bf16,
                           dim3(rows), dim3(256), args, "add_rmsnorm");
    };
    const uint32_t group = qh / kvh;
    const bool pp = e->ppanel;
    const void* grouped = group == 1   ? (pp ? (const void*)&x0ne_attention_prefill_panel_g1_bf16 : (const void*)&x0ne_attention_prefill_g1_bf16)
                          : group == 2 ? (pp ? (const void*)&x0ne_attention_prefill_panel_g2_bf16 : (const void*)&x0ne_attention_prefill_g2_bf16)
                          : group == 4 ? (pp ? (const void*)&x0ne_attention_prefill_panel_g4_bf16 : (const void*)&x0ne_attention_prefill_g4_bf16)
                          : group == 8 ? (pp ? (const void*)&x0ne_attention_prefill_panel_g8_bf16 : (const void*)&x0ne_attention_prefill_g8_bf16)
                                       : nullptr;
    // The exact mode (1, 2, 4 or 8 q heads per kv head, check_config): f64 scores and sums.
    const void* exact = group == 1   ? (const void*)&x0ne_attention_prefill_exact_g1_bf16
                        : group == 2 ? (const void*)&x0ne_attention_prefill_exact_g2_bf16
                        : group == 4 ? (const void*)&x0ne_attention_prefill_exact_g4_bf16
                        : group == 8 ? (const void*)&x0ne_attention_prefill_exact_g8_bf16
                                     : nullptr;
    if (e->f64_sums && !exact) return fail(X0NE_ERR_FORMAT, "exact prefill: a group of " + std::to_string(group));
    for (uint64_t l = 0; l < c.layers; ++l) {
        const LayerW& w = e->L[l];
        X0NE_TRY(norm(w.input_norm));
        X0NE_TRY(gemm(e, w.qkv, w.qkv_p, c.qkv_rows(), c.hidden, e->p_x, n, e->p_qkv));
        for (uint64_t sq = 0; sq < seqs; ++sq) {
            const void* qkv = e->d(e->p_qkv) + sq * sn * c.qkv_rows() * 2;
            const void* qn = e->d(w.q_norm);
            const void* kn = e->d(w.k_norm);
            const void* cs = e->d(e->rope_cs);
            void* q = e->d(e->p_q) + sq * sn * c.q_dim() * 2;
            void* kc = e->plane(l, 0);
            void* vc = e->plane(l, 1);
            const void* pt = e->pages_of(b + sq);
            const void* pos = e->pos_of(b + sq);
            void* args[] = {(void*)&qkv, (void*)&qn, (void*)&kn, (void*)&cs, (void*)&q,       (void*)&kc, (void*)&vc,
                            (void*)&pt,  (void*)&pos, (void*)&qh, (void*)&kvh, (void*)&max_ctx, (void*)&eps};
            X0NE_TRY(launch_rows(e, (const void*)&x0ne_qk_norm_rope_kv_write_rows_bf16, dim3((qh + kvh + 3) / 4, sn),
                                 dim3(256), args, "qk_norm_rope_kv_write"));
        }
        for (uint64_t sq = 0; sq < seqs; ++sq) {
            const void* q = e->d(e->p_q) + sq * sn * c.q_dim() * 2;
            const void* kc = e->plane(l, 0);
            const void* vc = e->plane(l, 1);
            const void* pt = e->pages_of(b + sq);
            void* out = e->d(e->p_attn) + sq * sn * c.q_dim() * 2;  // a whole number of panels
            const void* pos = e->pos_of(b + sq);
            void* args[] = {(void*)&q,  (void*)&kc, (void*)&vc,  (void*)&pt,      (void*)&out, (void*)&pos,
                            (void*)&sn, (void*)&qh, (void*)&kvh, (void*)&max_ctx, (void*)&scale};
            if (e->f64_sums) {
                const uint32_t per = X0NE_PREFILL_EXACT_COLS / group;  // rows per block
                X0NE_TRY(launch_rows(e, exact, dim3(kvh, (sn + per - 1) / per), dim3(X0NE_PREFILL_EXACT_THREADS), args,
                                     "exact prefill attention"));
            } else if (grouped) {
                const uint32_t per = X0NE_PREFILL_COLS / group;  // rows per block
                X0NE_TRY(launch_rows(e, grouped, dim3(kvh, (sn + per - 1) / per), dim3(X0NE_PREFILL_THREADS), args,
                                     "prefill attention"));
            } else {
                X0NE_TRY(launch_rows(e, (const void*)&x0ne_attention_prefill_bf16, dim3(qh, sn), dim3(256), args,
                                     "prefill attention"));
            }
        }
        X0NE_TRY(gemm(e, w.o, w.o_p, c.hidden, c.q_dim(), e->p_attn, n, e->p_delta));
        X0NE_TRY(norm(w.post_norm));
        X0NE_TRY(gemm(e, w.gate_up, w.gate_up_p, 2 * c.inter, c.hidden, e->p_x, n, e->p_gu));
        {
            const void* gu = e->d(e->p_gu);
            void* act = e->d(e->p_act);
            void* args[] = {(void*)&gu, (void*)&act, (void*)&inter};
            X0NE_TRY(launch_rows(e, pp ? (const void*)&x0ne_swiglu_panel_bf16 : (const void*)&x0ne_swiglu_bf16,
                                 dim3((inter + 2047) / 2048, rows), dim3(256), args, "swiglu"));
        }
        X0NE_TRY(gemm(e, w.down, w.down_p, c.hidden, c.inter, e->p_act, n, e->p_delta));
    }
    return X0NE_OK;
}

// The final norm and the LM head on row r of the last pass, at position p: f32 logits, the argmax
// into tokens[0] and, with advance, pos = p + 1 for the decode step that follows (sequence b's
// token and position).
x0ne_status prefill_head(x0ne_engine* e, uint64_t r, uint64_t p, bool advance, uint64_t b = 0) {
    const Cfg& c = e->c;
    X0NE_TRY(set_position(e, p, b));
    X0neGemv hd = {};
    hd.w = (const uint16_t*)e->d(e->has_lm_head ? e->lm_head : e->embed);
    hd.res_in = (const float*)e->d(e->p_res) + r * c.hidden;
    hd.res_out = nullptr;
    hd.delta = (const uint16_t*)e->d(e->p_delta) + r * c.hidden;
    hd.norm_w = (const uint16_t*)e->d(e->final_norm);
    hd.y = e->d(e->logits);
    hd.partial = (float*)e->d(e->head_partial);
    hd.counter = (uint32_t*)e->d(e->head_counter);
    hd.token_out = e->token_of(b);
    hd.pos = e->pos_of(b);
    hd.advance = advance ? 1 : 0;
    hd.rows = (uint32_t)c.vocab;
    hd.cols = (uint32_t)c.hidden;
    hd.eps = (float)c.eps;
    hd.prologue = 1;
    hd.epilogue = 3;
    hd.grid = e->grid_head;
    hd.f64acc = e->f64_sums;
    e->gpu->counts.launches++;
    X0NE_HIP(x0ne_launch_gemv(hd, e->gpu->stream), "prefill lm_head gemv");
    return X0NE_OK;
}

// The ids of a request: 1..=max_ctx of them, each inside the vocabulary (engine.rs:637-645).
x0ne_status check_ids(const x0ne_engine* e, const uint32_t* ids, size_t n) {
    if (n == 0 || n > e->max_ctx)
        return fail(X0NE_ERR_FORMAT, std::to_string(n) + " tokens for max_ctx " + std::to_string(e->max_ctx));
    for (size_t i = 0; i < n; ++i)
        if (ids[i] >= e->c.vocab) return fail(X0NE_ERR_FORMAT, "token " + std::to_string(ids[i]) + " outside the vocabulary");
    return X0NE_OK;
}

// Zeroes every client byte: the arena's, then the host buffers once the stream is drained. A
// failure poisons the engine (engine.rs:453-468).
x0ne_status scrub(x0ne_engine* e) {
    e->poisoned = true;
    X0NE_TRY(x0ne_arena_scrub(e->arena, nullptr));
    if (e->host_logits) std::memset(e->host_logits, 0, e->c.vocab * 4);
    if (e->host_token) *e->host_token = 0;
    if (e->ring) std::memset(e->ring, 0, RING * 4);
    if (e->bring) std::memset(e->bring, 0, RING * e->max_batch * 4);
    e->poisoned = false;
    return X0NE_OK;
}

// The logits row into the pinned host row: one asynchronous copy, then its event.
x0ne_status pull_logits(x0ne_engine* e) {
    e->gpu->counts.dtoh++;
    X0NE_HIP(hipMemcpyAsync(e->host_logits, e->d(e->logits), e->c.vocab * 4, hipMemcpyDeviceToHost, e->gpu->stream),
             "logits copy");
    X0NE_HIP(hipEventRecord(e->logits_ev, e->gpu->stream), "logits event");
    X0NE_HIP(hipEventSynchronize(e->logits_ev), "logits wait");
    return X0NE_OK;
}

// tokens[0] into ring word j % RING, then its event.
x0ne_status ring_fetch(x0ne_engine* e, size_t j) {
    e->gpu->counts.dtoh++;
    X0NE_HIP(hipMemcpyAsync(&e->ring[ring_word(j)], e->d(e->tokens), 4, hipMemcpyDeviceToHost, e->gpu->stream),
             "ring copy");
    X0NE_HIP(hipEventRecord(e->ring_ev[ring_word(j)], e->gpu->stream), "ring event");
    return X0NE_OK;
}

x0ne_status ring_take(x0ne_engine* e, size_t j, uint32_t* out) {
    X0NE_HIP(hipEventSynchronize(e->ring_ev[ring_word(j)]), "ring wait");
    *out = e->ring[ring_word(j)];
    return X0NE_OK;
}

// tokens[0] after the stream is drained; refused when the row had no finite maximum.
x0ne_status read_token(x0ne_engine* e, uint32_t* out) {
    uint32_t t = 0;
    X0NE_TRY(x0ne_arena_read(e->arena, e->tokens, 0, &t, 4));
    if (t >= e->c.vocab) return fail(X0NE_ERR_GPU, "argmax: a logits row has no finite maximum");
    *out = t;
    return X0NE_OK;
}

// A prompt into the cache: passes of up to `chunk` rows, then the last row's logits and argmax
// (engine.rs:408-425); tokens[0] holds the first generated token and pos the prompt's length.
// With chunk 1 (a MoE engine) one decode step per token.
// The passes of sequence b's prompt (n ids, already in its prompt row) and its first token.
x0ne_status prefill_passes(x0ne_engine* e, size_t n, uint64_t b) {
    size_t start = 0;
    for (;;) {
        const size_t len = std::min<size_t>(e->chunk, n - start);
        X0NE_TRY(prefill_pass(e, start, len, b));
        if (start + len == n) return prefill_head(e, len - 1, n - 1, true, b);
        start += len;
    }
}

x0ne_status prefill(x0ne_engine* e, const uint32_t* ids, size_t n) {
    X0NE_TRY(put_prompt(e, ids, n));
    if (e->chunk < 2) {
        for (size_t i = 0; i < n; ++i) X0NE_TRY(feed(e, (uint32_t)i));
        return X0NE_OK;
    }
    return prefill_passes(e, n, 0);
}

x0ne_status capture(x0ne_engine* e) {
    // One eager step on zeroed client buffers (the runtime loads code lazily, which a capture
    // must not see), then the capture of the same launches; the client bytes are zeroed after.
    X0NE_TRY(step_launches(e));
    X0NE_TRY(x0ne_gpu_sync(e->gpu));
    if (e->graph) {
        x0ne_graph_free(e->graph);
        e->graph = nullptr;
    }
    X0NE_TRY(x0ne_gpu_capture_begin(e->gpu));
    x0ne_status st = step_launches(e);
    x0ne_graph* gr = nullptr;
    x0ne_status st2 = x0ne_gpu_capture_end(e->gpu, &gr);
    if (st != X0NE_OK) {
        if (gr) x0ne_graph_free(gr);
        return st;
    }
    X0NE_TRY(st2);
    e->graph = gr;
    return x0ne_arena_scrub(e->arena, nullptr);
}

// Seeded page order: logical page i -> physical page page_of[i] (Fisher-Yates over splitmix64),
// or the identity for seed 0.
void page_order(x0ne_engine* e) {
    e->page_of.resize(e->pages);
    for (uint64_t i = 0; i < e->pages; ++i) e->page_of[i] = (uint32_t)i;
    if (e->page_seed == 0) return;
    uint64_t st = e->page_seed;
    for (uint64_t i = e->pages; i > 1; --i) {
        st += 0x9E3779B97F4A7C15ull;
        uint64_t z = st;
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        z ^= z >> 31;
        const uint64_t j = z % i;
        std::swap(e->page_of[i - 1], e->page_of[j]);
    }
}

// The device, the plan, the one allocation, and the tables; weights are written by the caller.
x0ne_status build_begin(const Cfg& c, const x0ne_engine_options* opts, x0ne_engine** out) {
    x0ne_engine* e = new x0ne_engine();
    e->c = c;
    e->max_ctx = opts->max_ctx;
    e->page_seed = opts->page_seed;
    e->f64_sums = exact_sums(c, *opts) ? 1 : 0;
    // A MoE engine prefills through the decode route (engine.rs:322-328).
    // A pass holds up to max_ctx rows of one sequence, or of several for a batched engine (its
    // prompts of one length share a pass).
    e->max_batch = opts->max_batch ? opts->max_batch : 1;  // check_config bounded it
    e->chunk = c.moe ? 1
                     : std::min<uint64_t>(opts->prefill_chunk ? opts->prefill_chunk : PREFILL_CHUNK,
                                          opts->max_ctx * e->max_batch);
    if (e->chunk == 0) e->chunk = 1;
    e->seq_pages = (e->max_ctx + X0NE_PAGE_C - 1) / X0NE_PAGE_C;
    e->pages = e->max_batch * e->seq_pages;
    x0ne_status st = x0ne_gpu_new(&e->gpu);
    if (st != X0NE_OK) {
        delete e;
        return st;
    }
    auto bail = [&](x0ne_status s) {
        delete e;
        return s;
    };
    if ((st = split_plan(e->gpu, (uint32_t)c.q_heads, (uint32_t)c.kv_heads, &e->split, e->f64_sums != 0)) != X0NE_OK)
        return bail(st);
    if (e->f64_sums) {
        static const char* env = std::getenv("X0NE_EXACT_SPLITS");  // a tuning knob
        if (env && std::atoi(env) > 0) e->split.splits = (uint32_t)std::min(std::atoi(env), 256);
    }
    // A grouped plan merges in its last block by default (one launch per layer); the reference's
    // default is the merge kernel (engine.rs:35), which set_split_merge selects.
    e->merge = e->split.grouped ? X0NE_MERGE_LAST_BLOCK : X0NE_MERGE_KERNEL;
    if (e->max_batch > 1) {
        if (!e->split.grouped)
            return bail(fail(X0NE_ERR_NOT_IMPLEMENTED, "batched decoding needs 1, 2, 4 or 8 q heads per kv head"));
        // The batched step's attention grid is max_batch times wider: fewer slices per sequence,
        // about one block per CU in all (measured at 8 and 16 sequences of 8 kv heads, 640 and
        // 8.7k positions: P 4 and 2 beat half and twice as many blocks).
        e->bsplit = e->split;
        const uint64_t p = (uint64_t)e->gpu->cus * e->split.per_cu / (e->split.grid_x * e->max_batch);
        e->bsplit.splits = (uint32_t)std::max<uint64_t>(1, std::min<uint64_t>(p, e->split.splits));
        static const char* env = std::getenv("X0NE_BATCH_SPLITS");  // a tuning knob
        if (env && std::atoi(env) > 0) e->bsplit.splits = (uint32_t)std::min(std::atoi(env), 256);
    }
    if ((st = plan_grids(e)) != X0NE_OK) return bail(st);
    if ((st = x0ne_arena_new(&e->arena)) != X0NE_OK) return bail(st);
    if ((st = plan(e)) != X0NE_OK) return bail(st);
    if ((st = x0ne_arena_freeze(e->arena, e->gpu)) != X0NE_OK) return bail(st);
    // inv_freq in f32 on the host (ops.rs:210-214), and the page table.
    std::vector<float> inv(c.head_dim / 2);
    for (size_t i = 0; i < inv.size(); ++i)
        inv[i] = 1.0f / std::pow((float)c.theta, (float)(2 * i) / (float)c.head_dim);
    if ((st = x0ne_arena_write(e->arena, e->inv_freq, 0, inv.data(), inv.size() * 4)) != X0NE_OK) return bail(st);
    page_order(e);
    if ((st = x0ne_arena_write(e->arena, e->page_table, 0, e->page_of.data(), e->pages * 4)) != X0NE_OK)
        return bail(st);
    *out = e;
    return X0NE_OK;
}

// The fused decode attention's RoPE table: cos and sin per position below max_ctx and pair, from
// inv_freq, on the device (the functions the rotation kernels call, so the same bits).
x0ne_status fill_rope_table(x0ne_engine* e) {
    const void* inv = e->d(e->inv_freq);
    void* cs = e->d(e->rope_cs);
    uint32_t positions = (uint32_t)e->max_ctx;
    void* args[] = {(void*)&inv, (void*)&cs, (void*)&positions};
    const uint32_t blocks = (uint32_t)((e->max_ctx * (e->c.head_dim / 2) + 255) / 256);
    X0NE_HIP(x0ne_launch((const void*)&x0ne_rope_table_f64, dim3(blocks), dim3(256), args, 0, e->gpu->stream),
             "rope table");
    X0NE_HIP(hipStreamSynchronize(e->gpu->stream), "rope table");
    return X0NE_OK;
}

// The panel copies of a batched engine's weights (x0ne_panel_bf16), from the row-major ones.
x0ne_status fill_panels(x0ne_engine* e) {
    if (!e->wpanel) return X0NE_OK;
    const Cfg& c = e->c;
    auto panel = [&](x0ne_slice src, x0ne_slice dst, uint64_t rows, uint64_t cols) -> x0ne_status {
        if (rows % 16 != 0 || cols % 8 != 0 || src.len != rows * cols * 2 || dst.len != src.len ||
            rows * cols / 8 > (uint64_t)UINT32_MAX * 256)
            return fail(X0NE_ERR_FORMAT, "panel copy of a " + std::to_string(rows) + "x" + std::to_string(cols) +
                                             " matrix");
        const void* sp = e->d(src);
        void* dp = e->d(dst);
        uint32_t r32 = (uint32_t)rows, c32 = (uint32_t)cols;
        void* args[] = {(void*)&sp, (void*)&dp, (void*)&r32, (void*)&c32};
        const uint32_t blocks = (uint32_t)((rows * cols / 8 + 255) / 256);
        X0NE_HIP(x0ne_launch((const void*)&x0ne_panel_bf16, dim3(blocks), dim3(256), args, 0, e->gpu->stream),
                 "panel copy");
        return X0NE_OK;
    };
    for (uint64_t l = 0; l < c.layers; ++l) {
        const LayerW& w = e->L[l];
        X0NE_TRY(panel(w.qkv, w.qkv_p, c.qkv_rows(), c.hidden));
        X0NE_TRY(panel(w.o, w.o_p, c.hidden, c.q_dim()));
        X0NE_TRY(panel(w.gate_up, w.gate_up_p, 2 * c.inter, c.hidden));
        X0NE_TRY(panel(w.down, w.down_p, c.hidden, c.inter));
    }
    if (e->hpanel) X0NE_TRY(panel(e->has_lm_head ? e->lm_head : e->embed, e->head_p, c.vocab, c.hidden));
    X0NE_HIP(hipStreamSynchronize(e->gpu->stream), "panel copies");
    return X0NE_OK;
}

x0ne_status build_end(x0ne_engine* e) {
    X0NE_TRY(x0ne_arena_scrub(e->arena, nullptr));
    X0NE_TRY(fill_rope_table(e));
    X0NE_TRY(fill_panels(e));
    X0NE_HIP(hipHostMalloc((void**)&e->ring, RING * 4, hipHostMallocDefault), "pinned ring");
    X0NE_HIP(hipHostMalloc((void**)&e->host_logits, e->c.vocab * 4, hipHostMallocDefault), "pinned logits");
    X0NE_HIP(hipHostMalloc((void**)&e->host_token, 4, hipHostMallocDefault), "pinned token");
    std::memset(e->ring, 0, RING * 4);
    if (e->max_batch > 1) {
        X0NE_HIP(hipHostMalloc((void**)&e->bring, RING * e->max_batch * 4, hipHostMallocDefault), "pinned batch ring");
        std::memset(e->bring, 0, RING * e->max_batch * 4);
    }
    std::memset(e->host_logits, 0, e->c.vocab * 4);
    *e->host_token = 0;
    for (auto& ev : e->ring_ev) X0NE_HIP(hipEventCreateWithFlags(&ev, hipEventDisableTiming), "ring event");
    X0NE_HIP(hipEventCreateWithFlags(&e->logits_ev, hipEventDisableTiming), "logits event");
    return capture(e);
}

}  // namespace

// ---------------------------------------------------------------------------------------------
// Load
// ---------------------------------------------------------------------------------------------

namespace {
// A shard name an index may give (st.rs:83-87): no directory part and not hidden.
bool plain_shard_name(const std::string& f) {
    return f.find('/') == std::string::npos && f.find('\\') == std::string::npos && (f.empty() || f[0] != '.');
}
}  // namespace

extern "C" x0ne_status x0ne_engine_load_from(const char* config_json, size_t n_files, const char* const* names,
                                             const uint8_t* const* data, const uint64_t* lens, const char* index_json,
                                             const x0ne_engine_options* opts, x0ne_engine** out) {
    if (!out || !opts) return fail(X0NE_ERR_FORMAT, "null argument");
    *out = nullptr;
    Cfg c;
    X0NE_TRY(parse_config(config_json, &c));
    X0NE_TRY(check_config(c, *opts));
    // Every format check before the device is touched. The files and the index agree exactly
    // (st.rs:216-277): without an index, one file; with one, every file it names given once,
    // no other file, each listed tensor in the shard it names, and every tensor listed.
    if (n_files == 0) return fail(X0NE_ERR_FORMAT, "no checkpoint file");
    if (!index_json && n_files != 1)
        return fail(X0NE_ERR_FORMAT, std::to_string(n_files) + " files without an index");
    std::map<std::string, TensorView> tensors;
    std::map<std::string, std::string> file_of;
    std::map<std::string, size_t> seen_files;
    for (size_t i = 0; i < n_files; ++i) {
        std::map<std::string, TensorView> one;
        const std::string fname = names && names[i] ? names[i] : ("file" + std::to_string(i));
        if (seen_files.count(fname)) return fail(X0NE_ERR_FORMAT, fname + ": given twice");
        seen_files[fname] = i;
        if (!data || (!data[i] && lens[i] != 0)) return fail(X0NE_ERR_FORMAT, fname + ": no bytes");
        X0NE_TRY(parse_safetensors(fname, data[i], lens[i], &one));
        for (auto& kv : one) {
            if (tensors.count(kv.first)) return fail(X0NE_ERR_FORMAT, kv.first + ": in two files");
            tensors[kv.first] = kv.second;
            file_of[kv.first] = fname;
        }
    }
    if (index_json) {
        Json idx;
        try {
            idx = parse_json(index_json);
        } catch (const std::exception& ex) {
            return fail(X0NE_ERR_FORMAT, std::string("index: ") + ex.what());
        }
        if (idx.kind != Json::Object) return fail(X0NE_ERR_FORMAT, "index: not an object");
        const Json* wm = idx.get("weight_map");
        if (!wm || wm->kind != Json::Object) return fail(X0NE_ERR_FORMAT, "index: no weight_map");
        std::map<std::string, int> named;
        for (const auto& f : wm->fields) {
            if (f.second.kind != Json::String) return fail(X0NE_ERR_FORMAT, "index: " + f.first + ": file is not a string");
            if (!plain_shard_name(f.second.text))
                return fail(X0NE_ERR_FORMAT, "index: shard name \"" + f.second.text + "\" is not a plain file name");
            named[f.second.text] = 1;
            auto it = file_of.find(f.first);
            if (it == file_of.end() || it->second != f.second.text)
                return fail(X0NE_ERR_FORMAT, f.first + ": not in " + f.second.text);
        }
        for (const auto& kv : file_of)
            if (!wm->get(kv.first)) return fail(X0NE_ERR_FORMAT, kv.first + ": in " + kv.second + " but not in the index");
        for (const auto& f : seen_files)
            if (!named.count(f.first)) return fail(X0NE_ERR_FORMAT, f.first + ": a file the index does not name");
        for (const auto& f : named)
            if (!seen_files.count(f.first)) return fail(X0NE_ERR_FORMAT, f.first + ": named by the index, not given");
    }
    X0NE_TRY(check_tensors(c, tensors));
    x0ne_engine* e = nullptr;
    X0NE_TRY(build_begin(c, opts, &e));
    auto put = [&](x0ne_slice s, std::initializer_list<std::string> names_) -> x0ne_status {
        uint64_t at = 0;
        for (const auto& n : names_) {
            const TensorView& t = tensors.at(n);
            X0NE_TRY(x0ne_arena_write(e->arena, s, at, t.data, t.len));
            at += t.len;
        }
        if (at != s.len) return fail(X0NE_ERR_FORMAT, "wrote " + std::to_string(at) + " bytes into a " + std::to_string(s.len) + "-byte slice");
        return X0NE_OK;
    };
    auto put_all = [&](x0ne_slice s, const std::vector<std::string>& names_) -> x0ne_status {
        uint64_t at = 0;
        for (const auto& n : names_) {
            const TensorView& t = tensors.at(n);
            X0NE_TRY(x0ne_arena_write(e->arena, s, at, t.data, t.len));
            at += t.len;
        }
        if (at != s.len) return fail(X0NE_ERR_FORMAT, "wrote " + std::to_string(at) + " bytes into a " + std::to_string(s.len) + "-byte slice");
        return X0NE_OK;
    };
    x0ne_status st = put(e->embed, {"model.embed_tokens.weight"});
    for (uint64_t l = 0; l < c.layers && st == X0NE_OK; ++l) {
        const LayerW& w = e->L[l];
        if ((st = put(w.input_norm, {layer_name(l, L_INPUT_NORM)})) != X0NE_OK) break;
        if ((st = put(w.qkv, {layer_name(l, L_Q), layer_name(l, L_K), layer_name(l, L_V)})) != X0NE_OK) break;
        if ((st = put(w.q_norm, {layer_name(l, L_QN)})) != X0NE_OK) break;
        if ((st = put(w.k_norm, {layer_name(l, L_KN)})) != X0NE_OK) break;
        if ((st = put(w.o, {layer_name(l, L_O)})) != X0NE_OK) break;
        if ((st = put(w.post_norm, {layer_name(l, L_POST_NORM)})) != X0NE_OK) break;
        if (c.moe) {  // weights.rs:371-389: per expert its [gate; up] rows, then the down rows
            std::vector<std::string> gu, dn;
            for (uint64_t x = 0; x < c.experts; ++x) {
                gu.push_back(expert_name(l, x, "gate_proj"));
                gu.push_back(expert_name(l, x, "up_proj"));
                dn.push_back(expert_name(l, x, "down_proj"));
            }
            if ((st = put_all(w.gate_up, gu)) != X0NE_OK) break;
            if ((st = put_all(w.down, dn)) != X0NE_OK) break;
            st = put(w.router, {router_name(l)});
            continue;
        }
        if ((st = put(w.gate_up, {layer_name(l, L_GATE), layer_name(l, L_UP)})) != X0NE_OK) break;
        st = put(w.down, {layer_name(l, L_DOWN)});
    }
    if (st == X0NE_OK) st = put(e->final_norm, {"model.norm.weight"});
    if (st == X0NE_OK && e->has_lm_head) st = put(e->lm_head, {"lm_head.weight"});
    if (st == X0NE_OK) st = build_end(e);
    if (st != X0NE_OK) {
        delete e;
        return st;
    }
    *out = e;
    return X0NE_OK;
}

namespace {

// Per-file size cap of a directory load (st.rs:11, DEFAULT_FILE_CAP).
constexpr uint64_t FILE_CAP = 64ull << 30;

// A read-only mapping of one checkpoint file (st.rs:55-67), released when it goes out of scope.
struct MappedFile {
    void* p = nullptr;
    size_t n = 0;
    MappedFile() = default;
    MappedFile(const MappedFile&) = delete;
    MappedFile& operator=(const MappedFile&) = delete;
    ~MappedFile() {
        if (p) munmap(p, n);
    }
};

x0ne_status io_fail(const std::string& path) {
    return fail(X0NE_ERR_IO, path + ": " + std::strerror(errno));
}

x0ne_status map_capped(const std::string& path, uint64_t cap, MappedFile* m) {
    if (path.find('\0') != std::string::npos) return fail(X0NE_ERR_IO, "a path with a NUL byte");
    const int fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) return io_fail(path);
    struct stat sb;
    if (fstat(fd, &sb) != 0) {
        const x0ne_status s = io_fail(path);
        close(fd);
        return s;
    }
    if (!S_ISREG(sb.st_mode)) {
        close(fd);
        return fail(X0NE_ERR_IO, path + ": not a regular file");
    }
    const uint64_t len = (uint64_t)sb.st_size;
    if (len > cap) {
        close(fd);
        return fail(X0NE_ERR_FORMAT, path + ": " + std::to_string(len) + " bytes exceeds the " + std::to_string(cap) +
                                         "-byte cap");
    }
    if (len != 0) {  // an empty file stays unmapped: the header check refuses it
        void* p = mmap(nullptr, (size_t)len, PROT_READ, MAP_PRIVATE, fd, 0);
        if (p == MAP_FAILED) {
            const x0ne_status s = io_fail(path);
            close(fd);
            return s;
        }
        m->p = p;
        m->n = (size_t)len;
    }
    close(fd);
    return X0NE_OK;
}

x0ne_status read_text(const std::string& path, std::string* out) {
    MappedFile m;
    X0NE_TRY(map_capped(path, FILE_CAP, &m));
    out->assign(static_cast<const char*>(m.p ? m.p : ""), m.n);
    return X0NE_OK;
}

bool file_exists(const std::string& path) {
    struct stat sb;
    return stat(path.c_str(), &sb) == 0;
}

}  // namespace

// Engine::load (engine.rs:292-297) with Safetensors::open_dir (st.rs:158-181): config.json is
// read and checked first; then model.safetensors, or the shards model.safetensors.index.json
// names (in first-seen order), each mapped read-only under the per-file cap; both present, or
// neither, is a format error. The mapped files go through x0ne_engine_load_from's checks.
extern "C" x0ne_status x0ne_engine_load(const char* model_dir, const x0ne_engine_options* opts, x0ne_engine** out) {
    if (!out || !opts || !model_dir) return fail(X0NE_ERR_FORMAT, "null argument");
    *out = nullptr;
    const std::string dir = model_dir;
    auto at = [&](const std::string& f) { return dir + "/" + f; };
    std::string config;
    X0NE_TRY(read_text(at("config.json"), &config));
    {
        Cfg c;
        X0NE_TRY(parse_config(config.c_str(), &c));
        X0NE_TRY(check_config(c, *opts));
    }
    const std::string single = at("model.safetensors"), index = at("model.safetensors.index.json");
    const bool has_single = file_exists(single), has_index = file_exists(index);
    if (has_single && has_index) return fail(X0NE_ERR_FORMAT, dir + ": both model.safetensors and its index");
    if (!has_single && !has_index) return fail(X0NE_ERR_FORMAT, dir + ": no safetensors file");
    std::vector<std::string> files;
    std::string index_text;
    if (has_single) {
        files.push_back("model.safetensors");
    } else {
        X0NE_TRY(read_text(index, &index_text));
        Json idx;
        try {
            idx = parse_json(index_text);
        } catch (const std::exception& ex) {
            return fail(X0NE_ERR_FORMAT, std::string("index: ") + ex.what());
        }
        const Json* wm = idx.kind == Json::Object ? idx.get("weight_map") : nullptr;
        if (!wm || wm->kind != Json::Object) return fail(X0NE_ERR_FORMAT, "index: no weight_map");
        for (const auto& f : wm->fields) {
            if (f.second.kind != Json::String)
                return fail(X0NE_ERR_FORMAT, "index: " + f.first + ": file is not a string");
            if (!plain_shard_name(f.second.text))
                return fail(X0NE_ERR_FORMAT, "index: shard name \"" + f.second.text + "\" is not a plain file name");
            bool seen = false;
            for (const auto& g : files) seen = seen || g == f.second.text;
            if (!seen) files.push_back(f.second.text);
        }
    }
    std::vector<MappedFile> maps(files.size());
    std::vector<const char*> names;
    std::vector<const uint8_t*> data;
    std::vector<uint64_t> lens;
    for (size_t i = 0; i < files.size(); ++i) {
        X0NE_TRY(map_capped(at(files[i]), FILE_CAP, &maps[i]));
        names.push_back(files[i].c_str());
        data.push_back(static_cast<const uint8_t*>(maps[i].p));
        lens.push_back(maps[i].n);
    }
    return x0ne_engine_load_from(config.c_str(), files.size(), names.data(), data.data(), lens.data(),
                                 has_index ? index_text.c_str() : nullptr, opts, out);
}

extern "C" x0ne_status x0ne_engine_load_synthetic(const char* config_json, uint64_t seed, double std_dev,
                                                  const x0ne_engine_options* opts, x0ne_engine** out) {
    if (!out || !opts) return fail(X0NE_ERR_FORMAT, "null argument");
    *out = nullptr;
    Cfg c;
    X0NE_TRY(parse_config(config_json, &c));
    X0NE_TRY(check_config(c, *opts));
    if (!(std_dev > 0) || !std::isfinite(std_dev)) return fail(X0NE_ERR_FORMAT, "std is not a positive number");
    if (c.moe) return fail(X0NE_ERR_NOT_IMPLEMENTED, "synthetic weights of a MoE model (load its checkpoint)");
    x0ne_engine* e = nullptr;
    X0NE_TRY(build_begin(c, opts, &e));
    hipStream_t s = e->gpu->stream;
    auto normal = [&](x0ne_slice sl, uint64_t at_elems, uint64_t n, uint64_t index) -> x0ne_status {
        X0NE_HIP(x0ne_launch_init_normal((uint16_t*)(e->d(sl)) + at_elems, n, tensor_key(seed, index), 0, std_dev, s),
                 "weight init");
        return X0NE_OK;
    };
    auto ones = [&](x0ne_slice sl) -> x0ne_status {
        X0NE_HIP(x0ne_launch_fill_u16((uint16_t*)e->d(sl), sl.len / 2, 0x3F80, s), "norm init");
        return X0NE_OK;
    };
    // Tensor index i of the checkpoint order: 0 embed, 1 + 11 l + leaf, then the final norm,
    // then lm_head.
    x0ne_status st = normal(e->embed, 0, c.vocab * c.hidden, 0);
    for (uint64_t l = 0; l < c.layers && st == X0NE_OK; ++l) {
        const LayerW& w = e->L[l];
        const uint64_t base = 1 + l * L_COUNT;
        const uint64_t h = c.hidden;
        if ((st = ones(w.input_norm)) != X0NE_OK) break;
        if ((st = normal(w.qkv, 0, c.q_dim() * h, base + L_Q)) != X0NE_OK) break;
        if ((st = normal(w.qkv, c.q_dim() * h, c.kv_dim() * h, base + L_K)) != X0NE_OK) break;
        if ((st = normal(w.qkv, (c.q_dim() + c.kv_dim()) * h, c.kv_dim() * h, base + L_V)) != X0NE_OK) break;
        if ((st = ones(w.q_norm)) != X0NE_OK) break;
        if ((st = ones(w.k_norm)) != X0NE_OK) break;
        if ((st = normal(w.o, 0, h * c.q_dim(), base + L_O)) != X0NE_OK) break;
        if ((st = ones(w.post_norm)) != X0NE_OK) break;
        if ((st = normal(w.gate_up, 0, c.inter * h, base + L_GATE)) != X0NE_OK) break;
        if ((st = normal(w.gate_up, c.inter * h, c.inter * h, base + L_UP)) != X0NE_OK) break;
        st = normal(w.down, 0, h * c.inter, base + L_DOWN);
    }
    if (st == X0NE_OK) st = ones(e->final_norm);
    if (st == X0NE_OK && e->has_lm_head) st = normal(e->lm_head, 0, c.vocab * c.hidden, 1 + c.layers * L_COUNT + 1);
    if (st == X0NE_OK) st = x0ne_gpu_sync(e->gpu);
    if (st == X0NE_OK) st = build_end(e);
    if (st != X0NE_OK) {
        delete e;
        return st;
    }
    *out = e;
    return X0NE_OK;
}

extern "C" void x0ne_engine_free(x0ne_engine* e) { delete e; }

// ---------------------------------------------------------------------------------------------
// Sessions (engine.rs:389-452, :1137-1344)
// ---------------------------------------------------------------------------------------------

extern "C" x0ne_status x0ne_engine_session(x0ne_engine* e, const uint32_t* prompt, size_t n, x0ne_session** out) {
    if (!e || !out) return fail(X0NE_ERR_FORMAT, "null argument");
    *out = nullptr;
    if (e->session_open) return fail(X0NE_ERR_FORMAT, "a session is open on this engine");
    if (e->poisoned) X0NE_TRY(scrub(e));
    X0NE_TRY(check_ids(e, prompt, n));
    x0ne_status st = prefill(e, prompt, n);
    if (st == X0NE_OK) st = pull_logits(e);
    if (st != X0NE_OK) {
        scrub(e);
        return st;
    }
    x0ne_session* s = new x0ne_session();
    s->e = e;
    s->pos = n;
    e->session_open = true;
    *out = s;
    return X0NE_OK;
}

extern "C" x0ne_status x0ne_session_logits(const x0ne_session* s, const float** ptr, size_t* len) {
    if (!s || !ptr || !len) return fail(X0NE_ERR_FORMAT, "null argument");
    if (s->failed) {
        *ptr = nullptr;
        *len = 0;
        return X0NE_OK;
    }
    *ptr = s->e->host_logits;
    *len = s->e->c.vocab;
    return X0NE_OK;
}

extern "C" size_t x0ne_session_position(const x0ne_session* s) { return s ? s->pos : 0; }

extern "C" x0ne_status x0ne_session_step(x0ne_session* s, uint32_t token) {
    if (!s) return fail(X0NE_ERR_FORMAT, "null session");
    if (s->failed) return fail(X0NE_ERR_GPU, "a previous step failed");
    x0ne_engine* e = s->e;
    if (token >= e->c.vocab) return fail(X0NE_ERR_FORMAT, "token " + std::to_string(token) + " outside the vocabulary");
    if (s->pos >= e->max_ctx)
        return fail(X0NE_ERR_FORMAT, "position " + std::to_string(s->pos) + " at max_ctx " + std::to_string(e->max_ctx));
    // The token goes up from a pinned word; the step reads it and pos on the device.
    *e->host_token = token;
    e->gpu->counts.htod++;
    hipError_t he = hipMemcpyAsync(e->d(e->tokens), e->host_token, 4, hipMemcpyHostToDevice, e->gpu->stream);
    x0ne_status st = he == hipSuccess ? X0NE_OK : gpu_fail(he, "token copy");
    if (st == X0NE_OK) st = run_step(e);
    if (st == X0NE_OK) st = pull_logits(e);
    if (st != X0NE_OK) {
        s->failed = true;
        return st;
    }
    s->pos += 1;
    return X0NE_OK;
}

static x0ne_status session_close(x0ne_session* s) {
    x0ne_status st = X0NE_OK;
    if (s->open) {
        s->open = false;
        st = scrub(s->e);
    }
    s->e->session_open = false;
    return st;
}

extern "C" x0ne_status x0ne_session_finish(x0ne_session* s) {
    if (!s) return fail(X0NE_ERR_FORMAT, "null session");
    x0ne_status st = session_close(s);
    delete s;
    return st;
}

extern "C" void x0ne_session_drop(x0ne_session* s) {
    if (!s) return;
    session_close(s);
    delete s;
}

namespace {

// Keeps the device busy ahead of the caller: queues decode steps (graph replay, then the copy
// of the step's token into ring word j % RING) while fewer than `ahead` of them sit beyond the
// last token the caller has taken and the request still wants tokens. A queued step's word
// cannot be overwritten before it is read: at most `ahead` (< RING) steps are ever outstanding.
// The semantics of the reference's Greedy ring (engine.rs:1322-1343).
x0ne_status greedy_fill(x0ne_greedy* g) {
    x0ne_engine* e = g->s->e;
    while (greedy_may_launch(g->launched, g->taken, g->max_tokens, g->ahead)) {
        const size_t j = g->launched + 1;
        x0ne_status st = run_step(e);
        if (st == X0NE_OK) st = ring_fetch(e, j);
        if (st != X0NE_OK) {
            g->s->failed = true;
            return st;
        }
        g->launched = j;
        g->s->pos += 1;
    }
    return X0NE_OK;
}

}  // namespace

extern "C" x0ne_status x0ne_session_into_greedy(x0ne_session* s, size_t max_tokens, size_t ahead, x0ne_greedy** out) {
    if (!s || !out) return fail(X0NE_ERR_FORMAT, "null argument");
    *out = nullptr;
    auto refuse = [&](x0ne_status st) {
        x0ne_session_drop(s);
        return st;
    };
    if (ahead < 1 || ahead > X0NE_GREEDY_AHEAD_MAX)
        return refuse(fail(X0NE_ERR_FORMAT, std::to_string(ahead) + " greedy steps ahead: 1 to 15"));
    if (s->failed) return refuse(fail(X0NE_ERR_GPU, "a previous step failed"));
    if (max_tokens == 0) return refuse(fail(X0NE_ERR_FORMAT, "0 greedy tokens asked"));
    const size_t room = s->e->max_ctx > s->pos ? s->e->max_ctx - s->pos : 0;
    if (max_tokens - 1 > room)
        return refuse(fail(X0NE_ERR_FORMAT, std::to_string(max_tokens) + " greedy tokens at position " +
                                                std::to_string(s->pos) + " pass max_ctx " + std::to_string(s->e->max_ctx)));
    x0ne_greedy* g = new x0ne_greedy();
    g->s = s;
    g->max_tokens = max_tokens;
    g->ahead = ahead;
    // The argmax of the current position is in tokens[0] already (the step wrote it).
    x0ne_status st = read_token(s->e, &g->first);
    if (st == X0NE_OK) st = greedy_fill(g);
    if (st != X0NE_OK) {
        s->failed = true;
        x0ne_greedy_drop(g);
        return st;
    }
    *out = g;
    return X0NE_OK;
}

extern "C" x0ne_status x0ne_greedy_next(x0ne_greedy* g, uint32_t* token) {
    if (!g || !token) return fail(X0NE_ERR_FORMAT, "null argument");
    if (g->s->failed) return fail(X0NE_ERR_GPU, "a previous step failed");
    if (g->taken == g->max_tokens)
        return fail(X0NE_ERR_FORMAT, "all " + std::to_string(g->max_tokens) + " greedy tokens taken");
    uint32_t t = g->first;
    if (g->taken > 0) {
        x0ne_status st = ring_take(g->s->e, g->taken, &t);
        if (st != X0NE_OK) {
            g->s->failed = true;
            return st;
        }
    }
    if (t >= g->s->e->c.vocab) {
        g->s->failed = true;
        return fail(X0NE_ERR_GPU, "argmax: a logits row has no finite maximum");
    }
    g->taken += 1;
    X0NE_TRY(greedy_fill(g));
    *token = t;
    return X0NE_OK;
}

extern "C" size_t x0ne_greedy_taken(const x0ne_greedy* g) { return g ? g->taken : 0; }
extern "C" size_t x0ne_greedy_position(const x0ne_greedy* g) { return g ? g->s->pos : 0; }

extern "C" x0ne_status x0ne_greedy_finish(x0ne_greedy* g) {
    if (!g) return fail(X0NE_ERR_FORMAT, "null greedy");
    x0ne_status st = x0ne_session_finish(g->s);
    delete g;
    return st;
}

extern "C" void x0ne_greedy_drop(x0ne_greedy* g) {
    if (!g) return;
    x0ne_session_drop(g->s);
    delete g;
}

// ---------------------------------------------------------------------------------------------
// Greedy passes (engine.rs:1026-1135)
// ---------------------------------------------------------------------------------------------

namespace {

x0ne_status greedy_inner(x0ne_engine* e, const uint32_t* prompt, size_t np, size_t n, uint32_t* out, double* times) {
    const auto t0 = std::chrono::steady_clock::now();
    auto now = [&]() { return std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count(); };
    X0NE_TRY(prefill(e, prompt, np));
    // The first token comes from the prefill's last step; it is in tokens[0] for the next.
    X0NE_TRY(read_token(e, &out[0]));
    if (times) times[0] = now();
    if (e->mode == X0NE_DECODE_EAGER) {
        for (size_t i = 1; i < n; ++i) {
            X0NE_TRY(step_launches(e));
            X0NE_TRY(read_token(e, &out[i]));
            if (times) times[i] = now();
        }
        return X0NE_OK;
    }
    // Per token: one graph launch, one 4-byte copy into a host word, one event; the host runs
    // up to RING - 1 steps ahead and collects tokens in order.
    size_t next = 1;
    auto collect = [&](size_t j) -> x0ne_status {
        uint32_t t = 0;
        X0NE_TRY(ring_take(e, j, &t));
        if (t >= e->c.vocab) return fail(X0NE_ERR_GPU, "argmax: a logits row has no finite maximum");
        out[j] = t;
        if (times) times[j] = now();
        return X0NE_OK;
    };
    for (size_t i = 1; i < n; ++i) {
        X0NE_TRY(run_step(e));
        X0NE_TRY(ring_fetch(e, i));
        if (timed_must_collect(i, next)) {
            X0NE_TRY(collect(next));
            next += 1;
        }
    }
    while (next < n) {
        X0NE_TRY(collect(next));
        next += 1;
    }
    return X0NE_OK;
}

// ---- the batched step: B independent sequences, each weight read once for all of them ----

// The launches of one batched decode step on sequences 0 .. B - 1, each at its own position with
// its own token and KV pages: per layer add + RMSNorm (layer 0: the embedding row on a zero
// residual), the QKV projection, the fused QK-norm + RoPE + K/V write + split-K attention over
// each sequence's pages, the O projection, add + RMSNorm, the gate/up projection with SwiGLU
// behind, the down projection; then the final norm, the f32 LM head and per sequence the
// argmax into its token and its position + 1. The projections are the few-row GEMM (each weight
// row read once for all B rows); the rounding points are those of the single-sequence step.
// Add + RMSNorm of the B rows (residual += delta, normed x out).
x0ne_status batch_norm(x0ne_engine* e, uint32_t B, x0ne_slice w) {
    const uint32_t h = (uint32_t)e->c.hidden;
    const float eps = (float)e->c.eps;
    void* res = e->d(e->b_res);
    const void* dl = e->d(e->b_delta);
    const void* wp = e->d(w);
    void* xn = e->d(e->b_x);
    void* args[] = {(void*)&res, (void*)&dl, (void*)&wp, (void*)&xn, (void*)&h, (void*)&eps};
    return launch_rows(e, (const void*)&x0ne_add_rmsnorm_panel_bf16, dim3(B), dim3(256), args, "batch add_rmsnorm");
}

// Layer 0's norm: each sequence's embedding row on a zero residual.
x0ne_status batch_embed_norm(x0ne_engine* e, uint32_t B) {
    const uint32_t h = (uint32_t)e->c.hidden, vocab = (uint32_t)e->c.vocab;
    const float eps = (float)e->c.eps;
    const void* table = e->d(e->embed);
    const void* toks = e->token_of(0);
    void* res = e->d(e->b_res);
    const void* wp = e->d(e->L[0].input_norm);
    void* xn = e->d(e->b_x);
    void* args[] = {(void*)&table, (void*)&toks, (void*)&res, (void*)&wp, (void*)&xn, (void*)&h, (void*)&vocab,
                    (void*)&eps};
    return launch_rows(e, (const void*)&x0ne_embed_rmsnorm_panel_bf16, dim3(B), dim3(256), args, "batch embedding");
}

uint32_t wpanel_bit(const x0ne_engine* e) { return e->wpanel ? PANEL_W : 0u; }

// The workspace of the batched projections' balanced kernel.
FewWork few_work(x0ne_engine* e) {
    FewWork w;
    w.ws = reinterpret_cast<float*>(e->d(e->b_few_ws));
    w.cnt = reinterpret_cast<uint32_t*>(e->d(e->b_few_cnt));
    w.groups = e->b_few_cnt.len / 4;
    return w;
}

x0ne_status batch_qkv(x0ne_engine* e, uint32_t B, uint64_t l) {
    const Cfg& c = e->c;
    const LayerW& w = e->L[l];
    const FewWork fw = few_work(e);
    return skinny(e->gpu, e->d(e->wpanel ? w.qkv_p : w.qkv), c.qkv_rows(), c.hidden, e->d(e->b_x), B, e->d(e->b_qkv),
                  0, PANEL_X | wpanel_bit(e), &fw);
}

x0ne_status batch_attention(x0ne_engine* e, uint32_t B, uint64_t l) {
    const Cfg& c = e->c;
    const void* kern = nullptr;
    switch (e->bsplit.group) {
        case 1: kern = (const void*)&x0ne_attention_rope_decode_batch_g1_bf16; break;
        case 2: kern = (const void*)&x0ne_attention_rope_decode_batch_g2_bf16; break;
        case 4: kern = (const void*)&x0ne_attention_rope_decode_batch_g4_bf16; break;
        case 8: kern = (const void*)&x0ne_attention_rope_decode_batch_g8_bf16; break;
        default: return fail(X0NE_ERR_NOT_IMPLEMENTED, "batched attention for this group size");
    }
    const LayerW& w = e->L[l];
    const void* qkv = e->d(e->b_qkv);
    const void* qn = e->d(w.q_norm);
    const void* kn = e->d(w.k_norm);
    const void* inv = e->d(e->inv_freq);
    const void* cs = e->d(e->rope_cs);
    void* kc = e->plane(l, 0);
    void* vc = e->plane(l, 1);
    const void* pt = e->d(e->page_table);
    void* st = e->d(e->b_state);
    void* cnt = e->d(e->b_counter);
    void* out = e->d(e->b_attn);
    const void* pos = e->d(e->pos);
    uint32_t qh = (uint32_t)c.q_heads, kvh = (uint32_t)c.kv_heads, max_ctx = (uint32_t)e->max_ctx;
    uint32_t P = e->bsplit.splits, sp = (uint32_t)e->seq_pages;
    float scale = (float)(1.0 / std::sqrt((double)c.head_dim)), eps = (float)c.eps;
    void* args[] = {(void*)&qkv, (void*)&qn,  (void*)&kn,      (void*)&inv, (void*)&cs,    (void*)&kc, (void*)&vc,
                    (void*)&pt,  (void*)&st,  (void*)&cnt,     (void*)&out, (void*)&pos,   (void*)&qh, (void*)&kvh,
                    (void*)&max_ctx, (void*)&P, (void*)&scale, (void*)&eps, (void*)&sp};
    return launch_rows(e, kern, dim3(kvh, P, B), dim3(256), args, "batch attention");
}

x0ne_status batch_o(x0ne_engine* e, uint32_t B, uint64_t l) {
    const Cfg& c = e->c;
    const LayerW& w = e->L[l];
    const FewWork fw = few_work(e);
    return skinny(e->gpu, e->d(e->wpanel ? w.o_p : w.o), c.hidden, c.q_dim(), e->d(e->b_attn), B, e->d(e->b_delta), 0,
                  PANEL_X | wpanel_bit(e), &fw);
}

x0ne_status batch_gate_up(x0ne_engine* e, uint32_t B, uint64_t l) {
    const Cfg& c = e->c;
    const LayerW& w = e->L[l];
    return skinny(e->gpu, e->d(e->wpanel ? w.gate_up_p : w.gate_up), c.inter, c.hidden, e->d(e->b_x), B,
                  e->d(e->b_act), 2, PANEL_X | PANEL_Y | wpanel_bit(e));
}

x0ne_status batch_down(x0ne_engine* e, uint32_t B, uint64_t l) {
    const Cfg& c = e->c;
    const LayerW& w = e->L[l];
    const FewWork fw = few_work(e);
    return skinny(e->gpu, e->d(e->wpanel ? w.down_p : w.down), c.hidden, c.inter, e->d(e->b_act), B, e->d(e->b_delta),
                  0, PANEL_X | wpanel_bit(e), &fw);
}

// The f32 LM head over the B normed rows, then each row's argmax into its token, position + 1.
x0ne_status batch_head(x0ne_engine* e, uint32_t B) {
    const Cfg& c = e->c;
    const x0ne_slice head = e->hpanel ? e->head_p : e->has_lm_head ? e->lm_head : e->embed;
    X0NE_TRY(skinny(e->gpu, e->d(head), c.vocab, c.hidden, e->d(e->b_x), B, e->d(e->b_logits), 1,
                    PANEL_X | (e->hpanel ? PANEL_W : 0u)));
    const void* lg = e->d(e->b_logits);
    uint32_t vocab = (uint32_t)c.vocab, slices = ARGMAX_SLICES;
    void* part = e->d(e->b_argmax);
    void* args[] = {(void*)&lg, (void*)&vocab, (void*)&slices, (void*)&part};
    X0NE_TRY(launch_rows(e, (const void*)&x0ne_argmax_slices_f32, dim3(B, slices), dim3(256), args, "batch argmax"));
    void* toks = e->token_of(0);
    void* pos = e->pos_of(0);
    void* args2[] = {(void*)&part, (void*)&slices, (void*)&toks, (void*)&pos};
    return launch_rows(e, (const void*)&x0ne_argmax_pick_advance, dim3(B), dim3(64), args2, "batch argmax pick");
}

// The launches of one batched decode step on sequences 0 .. B - 1, each at its own position with
// its own token and KV pages: per layer add + RMSNorm (layer 0: the embedding row on a zero
// residual), the QKV projection, the fused QK-norm + RoPE + K/V write + split-K attention over
// each sequence's pages, the O projection, add + RMSNorm, the gate/up projection with SwiGLU
// behind, the down projection; then the final norm, the f32 LM head and per sequence the
// argmax into its token and its position + 1. The projections are the few-row GEMM (each weight
// row read once for all B rows); the rounding points are those of the single-sequence step.
x0ne_status batch_step_launches(x0ne_engine* e, uint32_t B) {
    for (uint64_t l = 0; l < e->c.layers; ++l) {
        X0NE_TRY(l == 0 ? batch_embed_norm(e, B) : batch_norm(e, B, e->L[l].input_norm));
        X0NE_TRY(batch_qkv(e, B, l));
        X0NE_TRY(batch_attention(e, B, l));
        X0NE_TRY(batch_o(e, B, l));
        X0NE_TRY(batch_norm(e, B, e->L[l].post_norm));
        X0NE_TRY(batch_gate_up(e, B, l));
        X0NE_TRY(batch_down(e, B, l));
    }
    X0NE_TRY(batch_norm(e, B, e->final_norm));
    return batch_head(e, B);
}

// The batched step's graph for B sequences, captured as the single-sequence one is (an eager
// step on zeroed client buffers first); the client bytes are zeroed after, so this runs before
// any sequence is prefilled.
x0ne_status batch_capture(x0ne_engine* e, uint32_t B) {
    if (e->bgraph && e->bgraph_batch == B) return X0NE_OK;
    X0NE_TRY(batch_step_launches(e, B));
    X0NE_TRY(x0ne_gpu_sync(e->gpu));
    if (e->bgraph) {
        x0ne_graph_free(e->bgraph);
        e->bgraph = nullptr;
        e->bgraph_batch = 0;
    }
    X0NE_TRY(x0ne_gpu_capture_begin(e->gpu));
    x0ne_status st = batch_step_launches(e, B);
    x0ne_graph* gr = nullptr;
    x0ne_status st2 = x0ne_gpu_capture_end(e->gpu, &gr);
    if (st != X0NE_OK) {
        if (gr) x0ne_graph_free(gr);
        return st;
    }
    X0NE_TRY(st2);
    e->bgraph = gr;
    e->bgraph_batch = B;
    return x0ne_arena_scrub(e->arena, nullptr);
}

// The B token words into ring slot j % RING, then its event.
x0ne_status batch_ring_fetch(x0ne_engine* e, size_t j, uint32_t B) {
    e->gpu->counts.dtoh++;
    X0NE_HIP(hipMemcpyAsync(e->bring + ring_word(j) * e->max_batch, e->token_of(0), B * 4, hipMemcpyDeviceToHost,
                            e->gpu->stream),
             "batch ring copy");
    X0NE_HIP(hipEventRecord(e->ring_ev[ring_word(j)], e->gpu->stream), "ring event");
    return X0NE_OK;
}

// Step j's tokens out of the ring into column j of the [B][n] token rows.
x0ne_status batch_ring_take(x0ne_engine* e, size_t j, uint32_t B, size_t n, uint32_t* out) {
    X0NE_HIP(hipEventSynchronize(e->ring_ev[ring_word(j)]), "ring wait");
    for (uint32_t b = 0; b < B; ++b) {
        const uint32_t t = e->bring[ring_word(j) * e->max_batch + b];
        if (t >= e->c.vocab) return fail(X0NE_ERR_GPU, "argmax: a logits row has no finite maximum");
        out[b * n + j] = t;
    }
    return X0NE_OK;
}

x0ne_status batch_checks(x0ne_engine* e, const uint32_t* prompts, size_t np, size_t B, size_t n) {
    if (e->session_open) return fail(X0NE_ERR_FORMAT, "a session is open on this engine");
    if (e->poisoned) X0NE_TRY(scrub(e));
    if (B == 0 || B > e->max_batch)
        return fail(X0NE_ERR_FORMAT, "batch " + std::to_string(B) + " for max_batch " + std::to_string(e->max_batch));
    if (e->chunk < 2 || e->max_batch < 2)
        return fail(X0NE_ERR_NOT_IMPLEMENTED, "batched decoding needs an engine loaded with max_batch > 1");
    if (!prompts) return fail(X0NE_ERR_FORMAT, "null argument");
    for (size_t b = 0; b < B; ++b) X0NE_TRY(check_ids(e, prompts + b * np, np));
    if (n == 0 || np + n - 1 > e->max_ctx)
        return fail(X0NE_ERR_FORMAT, std::to_string(np) + " + " + std::to_string(n) + " tokens exceed max_ctx " +
                                         std::to_string(e->max_ctx));
    return X0NE_OK;
}

// The batch's graph (or nothing in eager mode), the prompts into their rows and their passes,
// and each sequence's first token into column 0 of tokens ([B][n]).
x0ne_status batch_prefill(x0ne_engine* e, const uint32_t* prompts, size_t np, uint32_t B, size_t n, uint32_t* tokens) {
    if (e->mode == X0NE_DECODE_GRAPH) X0NE_TRY(batch_capture(e, B));
    for (uint32_t b = 0; b < B; ++b)
        X0NE_TRY(x0ne_arena_write(e->arena, e->prompt, (uint64_t)b * e->max_ctx * 4, prompts + (size_t)b * np, np * 4));
    // Prompts that fit a pass several at a time go together (chunk / np of them; with panels np
    // a multiple of 16), the others one sequence at a time in passes of up to chunk rows. Only
    // prompts of more than 64 rows: a sequence alone then runs the same tiled GEMM as the shared
    // pass (64 rows or fewer take the few-row kernel), so each sequence's bits do not depend on
    // the batch.
    const uint64_t per_pass =
        np > 64 && np <= e->chunk && (!e->ppanel || np % 16 == 0) ? e->chunk / np : 1;
    // Its logits row where the batched step leaves the others' (the last token's logits of a
    // one-token request).
    auto keep_logits = [&](uint32_t b) -> x0ne_status {
        X0NE_HIP(hipMemcpyAsync(e->d(e->b_logits) + (uint64_t)b * e->c.vocab * 4, e->d(e->logits), e->c.vocab * 4,
                                hipMemcpyDeviceToDevice, e->gpu->stream),
                 "first logits");
        return X0NE_OK;
    };
    for (uint32_t b = 0; b < B;) {
        if (per_pass > 1) {
            const uint32_t seqs = (uint32_t)std::min<uint64_t>(per_pass, B - b);
            X0NE_TRY(prefill_pass(e, 0, np, b, seqs));
            for (uint32_t s = 0; s < seqs; ++s) {
                X0NE_TRY(prefill_head(e, (uint64_t)s * np + np - 1, np - 1, true, b + s));
                X0NE_TRY(keep_logits(b + s));
            }
            b += seqs;
        } else {
            X0NE_TRY(prefill_passes(e, np, b));
            X0NE_TRY(keep_logits(b));
            ++b;
        }
    }
    std::vector<uint32_t> first(B);
    X0NE_TRY(x0ne_arena_read(e->arena, e->tokens, 0, first.data(), B * 4));
    for (uint32_t b = 0; b < B; ++b) {
        if (first[b] >= e->c.vocab) return fail(X0NE_ERR_GPU, "argmax: a logits row has no finite maximum");
        tokens[b * n] = first[b];
    }
    return X0NE_OK;
}

x0ne_status batch_run_step(x0ne_engine* e, uint32_t B) {
    if (e->mode == X0NE_DECODE_GRAPH) {
        if (!e->bgraph || e->bgraph_batch != B) return fail(X0NE_ERR_GPU, "no batched decode graph captured");
        return x0ne_gpu_launch_graph(e->gpu, e->bgraph);
    }
    return batch_step_launches(e, B);
}

// Decode steps first .. last (each one launch and one copy of B words, up to RING - 1 in
// flight), collecting column j of tokens ([B][n]) as step j's words arrive.
x0ne_status batch_steps(x0ne_engine* e, uint32_t B, size_t first, size_t last, size_t n, uint32_t* tokens,
                        const std::function<void(size_t)>& arrived) {
    size_t next = first;
    for (size_t i = first; i <= last; ++i) {
        X0NE_TRY(batch_run_step(e, B));
        X0NE_TRY(batch_ring_fetch(e, i, B));
        if (timed_must_collect(i, next)) {
            X0NE_TRY(batch_ring_take(e, next, B, n, tokens));
            arrived(next++);
        }
    }
    while (next <= last) {
        X0NE_TRY(batch_ring_take(e, next, B, n, tokens));
        arrived(next++);
    }
    return X0NE_OK;
}

x0ne_status greedy_checks(x0ne_engine* e, const uint32_t* prompt, size_t np, size_t n) {
    if (e->session_open) return fail(X0NE_ERR_FORMAT, "a session is open on this engine");
    if (e->poisoned) X0NE_TRY(scrub(e));
    X0NE_TRY(check_ids(e, prompt, np));
    if (n == 0 || np + n - 1 > e->max_ctx)
        return fail(X0NE_ERR_FORMAT, std::to_string(np) + " + " + std::to_string(n) + " tokens exceed max_ctx " +
                                         std::to_string(e->max_ctx));
    return X0NE_OK;
}

}  // namespace

extern "C" x0ne_status x0ne_engine_greedy_timed(x0ne_engine* e, const uint32_t* prompt, size_t np, size_t n,
                                                uint32_t* tokens, double* times) {
    if (!e || !tokens) return fail(X0NE_ERR_FORMAT, "null argument");
    X0NE_TRY(greedy_checks(e, prompt, np, n));
    x0ne_status st = greedy_inner(e, prompt, np, n, tokens, times);
    x0ne_status sc = scrub(e);
    return st != X0NE_OK ? st : sc;
}

// The bench's decode measure: the prompt, `warmup` decode steps, a stream synchronisation, then
// `steps` decode steps timed on the host clock between two synchronisations. Per step one
// graph launch and one 4-byte copy into the host ring, RING - 1 steps in flight, as in
// greedy_inner. tokens gets warmup + steps + 1 tokens (the first from the prompt).
extern "C" x0ne_status x0ne_engine_decode_timed(x0ne_engine* e, const uint32_t* prompt, size_t np, size_t warmup,
                                                size_t steps, uint32_t* tokens, double* seconds) {
    if (!e || !tokens || !seconds || steps == 0) return fail(X0NE_ERR_FORMAT, "null argument");
    const size_t n = warmup + steps + 1;
    X0NE_TRY(greedy_checks(e, prompt, np, n));
    auto body = [&]() -> x0ne_status {
        X0NE_TRY(prefill(e, prompt, np));
        X0NE_TRY(read_token(e, &tokens[0]));
        size_t next = 1;
        auto collect = [&](size_t j) -> x0ne_status {
            uint32_t t = 0;
            X0NE_TRY(ring_take(e, j, &t));
            if (t >= e->c.vocab) return fail(X0NE_ERR_GPU, "argmax: a logits row has no finite maximum");
            tokens[j] = t;
            return X0NE_OK;
        };
        auto run = [&](size_t first, size_t last) -> x0ne_status {
            for (size_t i = first; i <= last; ++i) {
                X0NE_TRY(run_step(e));
                X0NE_TRY(ring_fetch(e, i));
                if (i + 1 - next >= RING - 1) X0NE_TRY(collect(next++));
            }
            while (next <= last) X0NE_TRY(collect(next++));
            return x0ne_gpu_sync(e->gpu);
        };
        if (warmup) X0NE_TRY(run(1, warmup));
        X0NE_TRY(x0ne_gpu_sync(e->gpu));
        const auto t0 = std::chrono::steady_clock::now();
        X0NE_TRY(run(warmup + 1, warmup + steps));
        *seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
        return X0NE_OK;
    };
    x0ne_status st = body();
    x0ne_status sc = scrub(e);
    return st != X0NE_OK ? st : sc;
}

extern "C" x0ne_status x0ne_engine_greedy_batch(x0ne_engine* e, const uint32_t* prompts, size_t np, size_t batch,
                                                size_t n, uint32_t* tokens, double* times, float* last_logits) {
    if (!e || !tokens) return fail(X0NE_ERR_FORMAT, "null argument");
    X0NE_TRY(batch_checks(e, prompts, np, batch, n));
    const uint32_t B = (uint32_t)batch;
    const auto t0 = std::chrono::steady_clock::now();
    auto now = [&]() { return std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count(); };
    auto body = [&]() -> x0ne_status {
        X0NE_TRY(batch_prefill(e, prompts, np, B, n, tokens));
        if (times) times[0] = now();
        if (n > 1)
            X0NE_TRY(batch_steps(e, B, 1, n - 1, n, tokens, [&](size_t j) {
                if (times) times[j] = now();
            }));
        if (!last_logits) return X0NE_OK;
        return x0ne_arena_read(e->arena, e->b_logits, 0, last_logits, (uint64_t)B * e->c.vocab * 4);
    };
    x0ne_status st = body();
    x0ne_status sc = scrub(e);
    return st != X0NE_OK ? st : sc;
}

extern "C" x0ne_status x0ne_engine_decode_batch_timed(x0ne_engine* e, const uint32_t* prompts, size_t np, size_t batch,
                                                      size_t warmup, size_t steps, uint32_t* tokens, double* seconds) {
    if (!e || !tokens || !seconds || steps == 0) return fail(X0NE_ERR_FORMAT, "null argument");
    const size_t n = warmup + steps + 1;
    X0NE_TRY(batch_checks(e, prompts, np, batch, n));
    const uint32_t B = (uint32_t)batch;
    auto body = [&]() -> x0ne_status {
        X0NE_TRY(batch_prefill(e, prompts, np, B, n, tokens));
        auto none = [](size_t) {};
        if (warmup) X0NE_TRY(batch_steps(e, B, 1, warmup, n, tokens, none));
        X0NE_TRY(x0ne_gpu_sync(e->gpu));
        const auto t0 = std::chrono::steady_clock::now();
        X0NE_TRY(batch_steps(e, B, warmup + 1, warmup + steps, n, tokens, none));
        X0NE_TRY(x0ne_gpu_sync(e->gpu));
        *seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
        return X0NE_OK;
    };
    x0ne_status st = body();
    x0ne_status sc = scrub(e);
    return st != X0NE_OK ? st : sc;
}

extern "C" x0ne_status x0ne_engine_greedy_with_last_logits(x0ne_engine* e, const uint32_t* prompt, size_t np, size_t n,
                                                           uint32_t* tokens, float* logits) {
    if (!e || !tokens || !logits) return fail(X0NE_ERR_FORMAT, "null argument");
    X0NE_TRY(greedy_checks(e, prompt, np, n));
    x0ne_status st = greedy_inner(e, prompt, np, n, tokens, nullptr);
    if (st == X0NE_OK) st = x0ne_arena_read(e->arena, e->logits, 0, logits, e->c.vocab * 4);
    x0ne_status sc = scrub(e);
    return st != X0NE_OK ? st : sc;
}

namespace {

// metrics::logsumexp (metrics.rs:4-7): the f32 maximum (NaN values skipped, as f32::max does),
// then m + ln of the f64 sum, in order, of e^(v - m).
double logsumexp_row(const float* x, size_t n) {
    float m = -INFINITY;
    for (size_t i = 0; i < n; ++i) m = std::fmax(m, x[i]);
    double sum = 0.0;
    for (size_t i = 0; i < n; ++i) sum += std::exp((double)x[i] - (double)m);
    return (double)m + std::log(sum);
}

}  // namespace

namespace {
// The teacher-forced pass of Engine::run (engine.rs:928-1006) over ids by `route`: every
// position's row computed (per row the LM head with the final norm on the prefill route, or the
// decode step) and its device argmax read, a row without a finite maximum refusing the pass
// (engine.rs:855-864); with `stats`, each position's PosStats (the argmax, the row's logsumexp,
// the log-probability of the next id, NaN at the last position); the full f32 rows at `keep`.
// Client bytes are scrubbed after, on success and on failure.
x0ne_status teacher_forced(x0ne_engine* e, const uint32_t* ids, size_t n, uint32_t route, const size_t* keep,
                           size_t n_keep, x0ne_pos_stats* stats, float* rows) {
    if (route != X0NE_ROUTE_PREFILL && route != X0NE_ROUTE_DECODE) return fail(X0NE_ERR_FORMAT, "unknown route");
    if (e->session_open) return fail(X0NE_ERR_FORMAT, "a session is open on this engine");
    if (e->poisoned) X0NE_TRY(scrub(e));
    X0NE_TRY(check_ids(e, ids, n));
    for (size_t k = 0; k < n_keep; ++k)
        if (keep[k] >= n)
            return fail(X0NE_ERR_FORMAT, "position " + std::to_string(keep[k]) + " outside " + std::to_string(n) + " tokens");
    const size_t vocab = e->c.vocab;
    std::vector<float> row(vocab);
    auto collect = [&](size_t p) -> x0ne_status {
        uint32_t am = 0;
        X0NE_TRY(x0ne_arena_read(e->arena, e->tokens, 0, &am, 4));
        if (am >= vocab) return fail(X0NE_ERR_GPU, "argmax: a logits row has no finite maximum");
        bool kept = false;
        for (size_t k = 0; k < n_keep; ++k) kept |= keep[k] == p;
        if (!stats && !kept) return X0NE_OK;  // the row is not asked for
        X0NE_TRY(x0ne_arena_read(e->arena, e->logits, 0, row.data(), vocab * 4));
        if (stats) {
            const double lse = logsumexp_row(row.data(), vocab);
            stats[p].argmax = am;
            stats[p].logsumexp = (float)lse;
            stats[p].next_logprob = p + 1 < n ? (float)((double)row[ids[p + 1]] - lse) : NAN;
        }
        for (size_t k = 0; k < n_keep; ++k)
            if (keep[k] == p) std::memcpy(rows + k * vocab, row.data(), vocab * 4);
        return X0NE_OK;
    };
    x0ne_status st = put_prompt(e, ids, n);
    if (route == X0NE_ROUTE_PREFILL && e->chunk > 1) {
        for (size_t start = 0; start < n && st == X0NE_OK;) {
            const size_t len = std::min<size_t>(e->chunk, n - start);
            st = prefill_pass(e, start, len);
            for (size_t p = start; p < start + len && st == X0NE_OK; ++p) {
                st = prefill_head(e, p - start, p, false);
                if (st == X0NE_OK) st = collect(p);
            }
            start += len;
        }
    } else {
        for (size_t p = 0; p < n && st == X0NE_OK; ++p) {
            st = feed(e, (uint32_t)p);
            if (st == X0NE_OK) st = collect(p);
        }
    }
    x0ne_status sc = scrub(e);
    return st != X0NE_OK ? st : sc;
}
}  // namespace

extern "C" x0ne_status x0ne_engine_run(x0ne_engine* e, const uint32_t* ids, size_t n, uint32_t route,
                                       const size_t* keep, size_t n_keep, x0ne_pos_stats* stats, float* rows) {
    if (!e || !ids || !stats || (!rows && n_keep) || (!keep && n_keep)) return fail(X0NE_ERR_FORMAT, "null argument");
    return teacher_forced(e, ids, n, route, keep, n_keep, stats, rows);
}

// Engine::logits_at (engine.rs:1012-1020) is Engine::run's kept rows: the same pass, the same
// refusal of a row without a finite maximum.
extern "C" x0ne_status x0ne_engine_logits_at(x0ne_engine* e, const uint32_t* ids, size_t n, const size_t* positions,
                                             size_t n_positions, uint32_t route, float* rows) {
    if (!e || !ids || (!rows && n_positions) || (!positions && n_positions)) return fail(X0NE_ERR_FORMAT, "null argument");
    return teacher_forced(e, ids, n, route, positions, n_positions, nullptr, rows);
}

// Engine::moe_routing (engine.rs:612-640): the experts every layer chose at each position of
// ids, fed one token per step through the decode route, [position][layer][top_k] into out
// (cap entries); *written the count (0 for a dense engine). Client bytes are scrubbed after.
extern "C" x0ne_status x0ne_engine_moe_routing(x0ne_engine* e, const uint32_t* ids, size_t n, uint32_t* out,
                                               size_t cap, size_t* written) {
    if (!e || !ids || !written) return fail(X0NE_ERR_FORMAT, "null argument");
    *written = 0;
    if (e->session_open) return fail(X0NE_ERR_FORMAT, "a session is open on this engine");
    if (e->poisoned) X0NE_TRY(scrub(e));
    X0NE_TRY(check_ids(e, ids, n));
    if (!e->c.moe) return X0NE_OK;
    const size_t per = e->c.layers * e->c.top_k;
    if (cap < n * per || !out) return fail(X0NE_ERR_FORMAT, std::to_string(n * per) + " routing entries, room for " + std::to_string(cap));
    x0ne_status st = put_prompt(e, ids, n);
    for (size_t p = 0; p < n && st == X0NE_OK; ++p) {
        st = feed(e, (uint32_t)p);
        if (st == X0NE_OK) st = x0ne_arena_read(e->arena, e->m_ids, 0, out + p * per, per * 4);
    }
    if (st == X0NE_OK) *written = n * per;
    x0ne_status sc = scrub(e);
    return st != X0NE_OK ? st : sc;
}

// ---------------------------------------------------------------------------------------------
// Introspection
// ---------------------------------------------------------------------------------------------

extern "C" x0ne_status x0ne_engine_set_decode_mode(x0ne_engine* e, uint32_t mode) {
    if (!e) return fail(X0NE_ERR_FORMAT, "null engine");
    if (mode != X0NE_DECODE_EAGER && mode != X0NE_DECODE_GRAPH) return fail(X0NE_ERR_FORMAT, "unknown decode mode");
    if (mode == X0NE_DECODE_GRAPH && !e->graph) return fail(X0NE_ERR_GPU, "no decode graph captured");
    e->mode = mode;
    return X0NE_OK;
}

extern "C" uint32_t x0ne_engine_decode_mode(const x0ne_engine* e) { return e ? e->mode : 0; }

namespace {
// A new decode attention or merge: the graph is captured again (which zeroes the client
// buffers); a failed capture leaves no graph and eager mode (engine.rs:531-560).
// The caller has already refused an open session (before changing any state), so the graph, the
// getters and the eager path always use the same kernel.
x0ne_status recapture(x0ne_engine* e) {
    x0ne_status st = capture(e);
    if (st != X0NE_OK) {
        if (e->graph) x0ne_graph_free(e->graph);
        e->graph = nullptr;
        e->mode = X0NE_DECODE_EAGER;
    }
    return st;
}
}  // namespace

extern "C" x0ne_status x0ne_engine_set_decode_attention(x0ne_engine* e, uint32_t a) {
    if (!e) return fail(X0NE_ERR_FORMAT, "null engine");
    if (a != X0NE_ATTENTION_SPLIT_K && a != X0NE_ATTENTION_PER_HEAD) return fail(X0NE_ERR_FORMAT, "unknown decode attention");
    if (e->f64_sums && a != X0NE_ATTENTION_SPLIT_K)
        return fail(X0NE_ERR_NOT_IMPLEMENTED, "the exact mode has one decode attention kernel (f64 split-K)");
    // A session borrows the engine (engine.rs:389-406): refused before anything changes.
    if (e->session_open) return fail(X0NE_ERR_FORMAT, "a session is open: change the decode attention between requests");
    if (a == e->attention && e->graph) return X0NE_OK;
    e->attention = a;
    return recapture(e);
}

extern "C" uint32_t x0ne_engine_decode_attention(const x0ne_engine* e) { return e ? e->attention : 0; }

extern "C" x0ne_status x0ne_engine_set_split_merge(x0ne_engine* e, uint32_t m) {
    if (!e) return fail(X0NE_ERR_FORMAT, "null engine");
    if (m != X0NE_MERGE_KERNEL && m != X0NE_MERGE_LAST_BLOCK) return fail(X0NE_ERR_FORMAT, "unknown split merge");
    if (m == X0NE_MERGE_LAST_BLOCK && !e->split.grouped)
        return fail(X0NE_ERR_GPU, "the last-block merge needs a grouped split-K kernel");
    if (e->f64_sums && m != X0NE_MERGE_LAST_BLOCK)
        return fail(X0NE_ERR_NOT_IMPLEMENTED, "the exact mode merges its f64 states in the last block");
    if (e->session_open) return fail(X0NE_ERR_FORMAT, "a session is open: change the split merge between requests");
    if (m == e->merge && e->graph) return X0NE_OK;
    e->merge = m;
    return recapture(e);
}

extern "C" uint32_t x0ne_engine_split_merge(const x0ne_engine* e) { return e ? e->merge : 0; }

extern "C" x0ne_status x0ne_engine_describe(const x0ne_engine* e, char* buf, size_t len) {
    if (!e) return fail(X0NE_ERR_FORMAT, "null engine");
    char gpu[512];
    x0ne_gpu_describe(e->gpu, gpu, sizeof gpu);
    const std::string moe_text =
        e->c.moe ? "MoE, " + std::to_string(e->c.experts) + " experts of width " + std::to_string(e->c.moe_inter) + ", " +
                       std::to_string(e->c.top_k) + " per token (prefill through the decode route)"
                 : std::string("dense");
    char s[1024];
    std::snprintf(s, sizeof s,
                  "%s, arena %llu bytes, decode graph %zu nodes, decode attention %s P %u (grid %u x %u, %u q "
                  "heads per block, %u blocks per CU, merge %s), KV pages of %d positions (%llu pages, %s order), "
                  "GEMV grids qkv %u o %u gate_up %u down %u head %u (%s sums), prefill passes of %llu rows, "
                  "batch %llu (weights %s), feed-forward %s",
                  gpu, (unsigned long long)e->arena->len, e->graph ? e->graph->nodes : (size_t)0,
                  e->attention == X0NE_ATTENTION_PER_HEAD ? "per head (E2), split-K" : "split-K", e->split.splits,
                  e->split.grid_x, e->split.splits, e->split.group, e->split.per_cu,
                  (e->f64_sums || e->merge == X0NE_MERGE_LAST_BLOCK) ? "LastBlock" : "Kernel", X0NE_PAGE_C, (unsigned long long)e->pages,
                  e->page_seed ? "shuffled" : "identity", e->grid_qkv, e->grid_o, e->grid_gu, e->grid_down,
                  e->grid_head, e->f64_sums ? "f64" : "f32", (unsigned long long)e->chunk,
                  (unsigned long long)e->max_batch, e->wpanel ? "row-major and in 16-row panels" : "row-major",
                  moe_text.c_str());
    if (buf && len) {
        std::strncpy(buf, s, len - 1);
        buf[len - 1] = 0;
    }
    return X0NE_OK;
}

extern "C" size_t x0ne_engine_graph_nodes(const x0ne_engine* e) { return e && e->graph ? e->graph->nodes : 0; }
extern "C" uint32_t x0ne_engine_splits(const x0ne_engine* e) { return e ? e->split.splits : 0; }
extern "C" uint64_t x0ne_engine_max_ctx(const x0ne_engine* e) { return e ? e->max_ctx : 0; }
extern "C" uint32_t x0ne_engine_sums(const x0ne_engine* e) {
    return e ? (e->f64_sums ? X0NE_SUMS_F64 : X0NE_SUMS_F32) : 0;
}
extern "C" const x0ne_arena* x0ne_engine_arena(const x0ne_engine* e) { return e ? e->arena : nullptr; }

extern "C" x0ne_status x0ne_engine_counts(const x0ne_engine* e, x0ne_counts* out) {
    if (!e) return fail(X0NE_ERR_FORMAT, "null engine");
    return x0ne_gpu_counts(e->gpu, out);
}

namespace {

x0ne_status time_kernel(x0ne_engine* e, uint32_t which, uint32_t batch, uint32_t iters, double* kernel_us,
                        double* wall_us, uint64_t* launches) {
    if (!e || iters == 0) return fail(X0NE_ERR_FORMAT, "null argument");
    if (which > X0NE_KERNEL_HEAD) return fail(X0NE_ERR_FORMAT, "unknown kernel");
    if (e->session_open) return fail(X0NE_ERR_FORMAT, "a session is open on this engine");
    if (batch > 0 && (batch > e->max_batch || e->max_batch < 2))
        return fail(X0NE_ERR_FORMAT, "batch " + std::to_string(batch) + " for max_batch " + std::to_string(e->max_batch));
    auto one = [&](uint64_t l) -> x0ne_status {
        if (batch > 0) {
            switch (which) {
                case X0NE_KERNEL_QKV: return batch_qkv(e, batch, l);
                case X0NE_KERNEL_ATTENTION: return batch_attention(e, batch, l);
                case X0NE_KERNEL_O: return batch_o(e, batch, l);
                case X0NE_KERNEL_GATE_UP: return batch_gate_up(e, batch, l);
                case X0NE_KERNEL_DOWN: return batch_down(e, batch, l);
                default: return batch_head(e, batch);
            }
        }
        switch (which) {
            case X0NE_KERNEL_QKV: return launch_qkv(e, e->c.layers > 1 ? l + 1 : 0);
            case X0NE_KERNEL_ATTENTION: return launch_attention(e, l);
            case X0NE_KERNEL_O: return launch_o(e, l);
            case X0NE_KERNEL_GATE_UP: return launch_gate_up(e, l);
            case X0NE_KERNEL_DOWN: return launch_down(e, l);
            default: return launch_head(e);
        }
    };
    // The attention is timed at the longest context the engine holds: every sequence at
    // position max_ctx - 1 (the client state, zeroed between calls, would leave it at 1 key).
    if (which == X0NE_KERNEL_ATTENTION) {
        const std::vector<uint32_t> at(batch > 0 ? batch : 1, (uint32_t)(e->max_ctx - 1));
        X0NE_HIP(hipMemcpyAsync(e->d(e->pos), at.data(), at.size() * 4, hipMemcpyHostToDevice, e->gpu->stream),
                 "timing position");
        X0NE_HIP(hipStreamSynchronize(e->gpu->stream), "timing position");
    }
    // Layer 0's QKV kernel also reads the embedding; the others are timed.
    const uint64_t per = which == X0NE_KERNEL_HEAD ? 1
                         : which == X0NE_KERNEL_QKV ? (e->c.layers > 1 ? e->c.layers - 1 : 1)
                                                    : e->c.layers;
    const uint64_t n = (uint64_t)iters * per;
    std::vector<hipEvent_t> ev(2 * n + 2, nullptr);
    x0ne_status st = X0NE_OK;
    for (auto& x : ev)
        if (st == X0NE_OK && hipEventCreate(&x) != hipSuccess) st = fail(X0NE_ERR_GPU, "event create");
    for (uint64_t l = 0; l < per && st == X0NE_OK; ++l) st = one(l);  // warm-up round
    if (st == X0NE_OK && hipEventRecord(ev[2 * n], e->gpu->stream) != hipSuccess) st = fail(X0NE_ERR_GPU, "event");
    std::vector<X0neTimer> timers(n);
    for (uint64_t i = 0; i < n && st == X0NE_OK; ++i) {
        timers[i] = X0neTimer{ev[2 * i], ev[2 * i + 1], false};
        x0ne_timer = &timers[i];
        st = one(i % per);
        x0ne_timer = nullptr;
    }
    if (st == X0NE_OK && hipEventRecord(ev[2 * n + 1], e->gpu->stream) != hipSuccess) st = fail(X0NE_ERR_GPU, "event");
    if (st == X0NE_OK && hipEventSynchronize(ev[2 * n + 1]) != hipSuccess) st = fail(X0NE_ERR_GPU, "event wait");
    double kern_ms = 0.0;
    float wall_ms = 0.f;
    for (uint64_t i = 0; i < n && st == X0NE_OK; ++i) {
        float ms = 0.f;
        if (hipEventElapsedTime(&ms, ev[2 * i], ev[2 * i + 1]) != hipSuccess) st = fail(X0NE_ERR_GPU, "elapsed time");
        kern_ms += ms;
    }
    if (st == X0NE_OK && hipEventElapsedTime(&wall_ms, ev[2 * n], ev[2 * n + 1]) != hipSuccess)
        st = fail(X0NE_ERR_GPU, "elapsed time");
    for (auto& x : ev)
        if (x) (void)hipEventDestroy(x);
    x0ne_status sc = scrub(e);
    if (st != X0NE_OK) return st;
    if (kernel_us) *kernel_us = kern_ms * 1000.0 / (double)n;
    if (wall_us) *wall_us = (double)wall_ms * 1000.0 / (double)n;
    if (launches) *launches = n;
    return sc;
}

}  // namespace

extern "C" x0ne_status x0ne_engine_time_kernel(x0ne_engine* e, uint32_t which, uint32_t iters, double* kernel_us,
                                              double* wall_us, uint64_t* launches) {
    return time_kernel(e, which, 0, iters, kernel_us, wall_us, launches);
}

extern "C" x0ne_status x0ne_engine_time_batch_kernel(x0ne_engine* e, uint32_t which, uint32_t batch, uint32_t iters,
                                                    double* kernel_us, double* wall_us, uint64_t* launches) {
    if (batch == 0) return fail(X0NE_ERR_FORMAT, "batch 0");
    return time_kernel(e, which, batch, iters, kernel_us, wall_us, launches);
}

extern "C" x0ne_status x0ne_engine_page(const x0ne_engine* e, uint64_t i, uint32_t* out) {
    if (!e || !out || i >= e->pages) return fail(X0NE_ERR_FORMAT, "no such page");
    *out = e->page_of[i];
    return X0NE_OK;
}

extern "C" x0ne_status x0ne_engine_client_data_is_zero(const x0ne_engine* e, int* out) {
    if (!e || !out) return fail(X0NE_ERR_FORMAT, "null argument");
    const uint64_t STEP = 64ull << 20;
    std::vector<uint8_t> buf(STEP);
    *out = 1;
    for (const auto& r : e->arena->regions) {
        if (r.cls != X0NE_CLASS_CLIENT_DATA) continue;
        for (uint64_t at = 0; at < r.len; at += STEP) {
            const uint64_t n = r.len - at < STEP ? r.len - at : STEP;
            X0NE_HIP(hipMemcpy(buf.data(), e->arena->base + r.offset + at, n, hipMemcpyDeviceToHost), "read back");
            for (uint64_t i = 0; i < n; ++i)
                if (buf[i]) {
                    *out = 0;
                    return X0NE_OK;
                }
        }
    }
    return X0NE_OK;
}

extern "C" int x0ne_engine_host_buffers_are_zero(const x0ne_engine* e) {
    if (!e) return 0;
    for (uint64_t i = 0; i < e->c.vocab; ++i)
        if (e->host_logits[i] != 0.0f || std::signbit(e->host_logits[i])) return 0;
    if (*e->host_token) return 0;
    for (size_t i = 0; i < RING; ++i)
        if (e->ring[i]) return 0;
    for (size_t i = 0; e->bring && i < RING * e->max_batch; ++i)
        if (e->bring[i]) return 0;
    return 1;
}
