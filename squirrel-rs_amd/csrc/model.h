// Llama model and inference context on one GPU.
#pragma once
#include <hip/hip_runtime.h>

#include <functional>
#include <string>
#include <vector>

#include "gguf.h"
#include "launch.h"

namespace sq {

// LlamaConfig (src/models/llama/config.rs:10-26).
struct Config {
    int n_layers = 0, dim = 0, ffn = 0, n_heads = 0, n_kv_heads = 0, head_dim = 0, vocab = 0;
    int context_length = 0;
    uint32_t bos = 0, eos = 0;
    float rope_base = 0.f, eps = 0.f;
    std::vector<float> inv_freq;  // head_dim / 2
};

// LlamaConfig::from_gguf (config.rs:29-73) incl. compute_rope_inv_freq
// (config.rs:83-127).  SQ_ERR_CONFIG on MissingMetadata / WrongMetadataType.
int read_config(const GGUFFile& f, Config* cfg);
void rope_inv_freq(int head_dim, float base, float factor, float low, float high, float orig_ctx,
                   float* out);

// Upload `rows` rows of GGUF blocks into the device layout (DevMatrix).
int upload_matrix(int wtype, const uint8_t* blocks, size_t rows, size_t k, DevMatrix* out);
// Upload several GGUF matrices with equal k as one stacked device matrix.
int upload_stacked(int wtype, const std::vector<const uint8_t*>& parts,
                   const std::vector<size_t>& rows, size_t k, DevMatrix* out);
void free_matrix(DevMatrix* m);

struct Layer {
    float* attn_norm = nullptr;
    DevMatrix qkv;     // [q rows; k rows; v rows]
    DevMatrix o;
    float* ffn_norm = nullptr;
    DevMatrix gateup;  // [gate rows; up rows]
    DevMatrix down;
};

}  // namespace sq

struct sq_model {
    sq::Config cfg;
    int wtype = 0;
    bool tied = true;
    std::vector<sq::Layer> layers;
    sq::DevMatrix embd;     // token_embd rows: the embedding table
    sq::DevMatrix head;     // LM head rows (aliases embd when tied)
    float* out_norm = nullptr;
    uint64_t weight_bytes = 0;
    int device = 0;
};

struct sq_ctx {
    const sq_model* m = nullptr;
    hipStream_t stream = nullptr;
    size_t max_pos = 0;
    uint32_t flags = 0;
    bool a8 = true;           // quantized activations on the matvecs
    size_t seq_len = 0;       // host mirror of *d_pos

    float* kcache = nullptr;  // [layer][max_pos][kv_dim]
    float* vcache = nullptr;
    float2* rope = nullptr;   // [max_pos][head_dim/2] (cos, sin)
    int* d_pos = nullptr;
    uint32_t* d_token = nullptr;
    uint32_t* d_ids = nullptr;   // prompt ids [max_pos]
    uint32_t* d_hist = nullptr;  // generated ids [max_pos]
    int* d_nhist = nullptr;

    // decode workspace
    float* hidden = nullptr;
    float* q = nullptr;
    float* attn = nullptr;
    float* ffn_act = nullptr;
    float* logits = nullptr;
    // Q8_0 activations of every quantization site of a decode step, per
    // layer l at l * tap_width: the attention-norm output [dim], the attention
    // output [q_dim], the FFN-norm output [dim], the FFN activation [ffn]
    // (payload tap_q, fp16 block scales tap_d at the same offset / 32).  The
    // one-kernel-per-op step reads its activations from here; the persistent
    // step writes layer 0's attention-norm site, and every site when taps
    // are on.  The LM-head input is head_qs / head_d.
    int8_t* tap_q = nullptr;
    uint16_t* tap_d = nullptr;
    bool taps = false;             // record every site (persistent step, prefill)
    int8_t* ptap_q = nullptr;      // the prefill's sites: rows x the decode layout
    uint16_t* ptap_d = nullptr;
    size_t ptap_rows = 0;
    size_t last_rows = 0;          // rows of the most recent forward
    bool last_tapped = false;      // its sites were recorded
    float *part_m = nullptr, *part_l = nullptr, *part_o = nullptr;
    int max_tiles = 0;               // 64-position attention tiles of max_pos
    unsigned* attn_counters = nullptr;  // one per kv head, zero between launches
    float* pv = nullptr;
    int* pi = nullptr;
    int* pn = nullptr;
    int n_parts = 0;
    float* dbg_normed = nullptr;   // layer-0 attention norm of the last decode step
    float* last_hidden = nullptr;  // final norm of the last forward
    int8_t* head_qs = nullptr;
    uint16_t* head_d = nullptr;

    // prefill workspace, grown on demand
    size_t cap_rows = 0;
    float* p_hidden = nullptr;
    float* p_normed = nullptr;
    float* p_qkv = nullptr;
    float* p_q = nullptr;
    float* p_attn = nullptr;
    float* p_gu = nullptr;
    float* p_act = nullptr;
    int8_t* p_aq = nullptr;
    uint16_t* p_ad = nullptr;
    float* p_split = nullptr;  // partial tiles of a K-split prefill matmul (kPrefillSplitFloats)
    uint32_t* p_kvs = nullptr;  // one layer's K and V split into f16 halves (attn_split_words(max_pos))

    // persistent decode step (one launch per token)
    bool persist = false;
    int step_grid = 0;
    sq::StepArgs step{};
    sq::StepLayer* d_layers = nullptr;
    uint8_t* s_stream = nullptr;  // per-CU weight streams
    unsigned long long* s_xchg = nullptr;  // exchange words
    unsigned* s_epoch = nullptr;
    int* s_error = nullptr;
    unsigned long long* s_trace = nullptr;  // step timeline when enabled

    // Set by a kernel that met a token id past the embedding table (the
    // reference's slice index panics there, embedding.rs:43-44); the read
    // itself is clamped in bounds.  Checked by ctx_check, cleared by reset.
    uint32_t* d_id_error = nullptr;
    uint32_t* d_sids = nullptr;    // the window being scored [max_pos + 1]
    double* d_logp = nullptr;      // its log-probabilities [max_pos + 1]
    uint32_t* h_pinned = nullptr;  // pinned staging for ids / tokens
    hipGraphExec_t graph = nullptr;
    hipGraph_t graph_def = nullptr;

    // Prefill phase timing (measurement only): events recorded between
    // launch groups, each interval charged to the kind of its first launch.
    bool prof = false;
    std::vector<hipEvent_t> prof_ev;
    std::vector<int> prof_kind;

    // Per-kernel relaunchers of the decode step (measurement only).
    std::vector<std::function<int()>> kernels;
    std::vector<uint64_t> kernel_bytes;
};

namespace sq {
// Quantization sites of one layer, in activation elements: the
// attention-norm output, the attention output, the FFN-norm output and the
// FFN activation; tap_width is their sum.
inline size_t tap_width(const Config& g) { return 2 * (size_t)g.dim + (size_t)g.n_heads * g.head_dim + g.ffn; }
inline size_t tap_offset(const Config& g, int site) {
    const size_t D = g.dim, QD = (size_t)g.n_heads * g.head_dim;
    return site == 0 ? 0 : site == 1 ? D : site == 2 ? D + QD : 2 * D + QD;
}
}  // namespace sq

// A weight matrix uploaded through the operator-level entry points.
struct sq_weight {
    sq::DevMatrix m;
};

namespace sq {
int ctx_create(const sq_model* m, size_t max_pos, uint32_t flags, sq_ctx** out);
void ctx_destroy(sq_ctx* c);
int ctx_forward(sq_ctx* c, const uint32_t* ids, size_t n);
int ctx_generate(sq_ctx* c, const uint32_t* prompt, size_t n_prompt, size_t max_tokens, uint32_t flags,
                 uint32_t* out, size_t* n_out, double* step_ms);
int ctx_time_kernel(sq_ctx* c, int which, int iters, double* mean_us, uint64_t* bytes);
int ctx_set_taps(sq_ctx* c, bool on);
// Teacher-forced scoring of one window on a reset context (perplexity.rs:61-110):
// prefill ids[0, burn), then for i in [burn, n): logp[i - burn] = log p(ids[i])
// and, while i + 1 < n, one decode step on ids[i].
int ctx_score(sq_ctx* c, const uint32_t* ids, size_t n, size_t burn, double* logp);
// Runs a prefill of ids on a reset context with HIP events between launch
// groups; ms[0..3] = int8 matmuls, attention, everything else, whole prefill.
int ctx_prefill_phases(sq_ctx* c, const uint32_t* ids, size_t n, double* ms);
// Host copy of the most recent forward's quantized activations as GGUF
// Q8_0 blocks: per layer, per site, rows x k/32 blocks; then the LM-head row.
int ctx_read_taps(sq_ctx* c, void* blocks, size_t n_blocks);
// Status of the device error words: a token id past the embedding table, and
// the persistent decode step's wait limit (synchronizes the stream).
int ctx_check(sq_ctx* c);
// A fresh sequence on the context (ModelContext::clear, context.rs:9-27):
// position 0, empty token history, device error words cleared and, for the
// persistent step, the tag epoch moved past every tag an abandoned step may
// have written.  Synchronizes the stream.
int ctx_reset(sq_ctx* c);
int model_load(const char* path, sq_model** out);
// Parse + config + tensor checks only (no device allocation).
int model_inspect(const char* path, sq_model** out);
void model_free(sq_model* m);
}  // namespace sq
