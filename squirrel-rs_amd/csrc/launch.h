// Host-side launchers for the HIP kernels.  Every launcher enqueues on the
// given stream and returns 0 or a status code; none of them synchronizes.
#pragma once
#include "sq_common.h"

namespace sq {

// ---- decode matvec (k_gemv.hip) -------------------------------------------
enum GemvPro : int {
    PRO_NORM = 0,  // RMSNorm(x) * norm_w computed in every workgroup, then
                   // quantized (A8) or kept f32 (A32) in LDS
    PRO_Q8 = 1,    // quantized activation blocks read from global memory
    PRO_F32 = 2,   // f32 activations read from global memory
};
enum GemvEpi : int {
    EPI_STORE = 0,   // out[row] = v
    EPI_QKV = 1,     // RoPE on q/k rows, q -> q_out, k/v -> cache row `pos`
    EPI_RESID = 2,   // out[row] += v  (residual add into hidden)
    EPI_GATEUP = 3,  // silu(gate)*up -> ffn_act (+ Q8_0 blocks)
    EPI_LOGITS = 4,  // logits[row] = v, per-workgroup argmax partials
};

// Workgroups of the LM-head matvec; its argmax partials have this many slots.
constexpr int kLogitsGrid = 1024;

struct GemvArgs {
    MatView w;
    int n_rows;        // logical output rows (EPI_GATEUP: ffn width)
    // prologue inputs
    const float* x;        // PRO_NORM / PRO_F32
    const float* norm_w;   // PRO_NORM
    float eps;
    const int8_t* aq;      // PRO_Q8: activation payload [k]
    const uint16_t* ad;    // PRO_Q8: activation scales [k/32]
    // epilogue outputs
    float* out;
    float* q_out;          // EPI_QKV
    float* kcache;
    float* vcache;
    const float2* rope;    // [max_pos][head_dim/2] (cos, sin)
    const int* pos;        // device position counter
    int q_rows, kv_rows, half;
    float* ffn_act;        // EPI_GATEUP
    int8_t* act_q;
    uint16_t* act_d;
    float* part_val;       // EPI_LOGITS
    int* part_idx;
    int* part_nan;
    // PRO_NORM from the embedding table: x = dequantized row *token of embd
    // (when embd.qs is non-null); workgroup 0 also stores x to hidden_out.
    MatView embd;
    const uint32_t* token;
    uint32_t* id_error;  // set when *token is past the table (the read is clamped)
    float* hidden_out;
    // taps of the prologue, written by workgroup 0 when non-null: the
    // normalized row (f32) and, on the integer path, its Q8_0 blocks
    float* dbg_normed;
    int8_t* dbg_qs;
    uint16_t* dbg_d;
};

// a8: quantized activations (false: f32 activations).  Returns the number of
// workgroups launched through *grid_out when not null.
int launch_gemv(hipStream_t s, int pro, int epi, bool a8, const GemvArgs& a, int* grid_out);

// ---- attention (k_attn.hip) ------------------------------------------------
// Decode: one query row per head at position *pos, keys 0..*pos (inclusive),
// tiles of 64 positions (grid n_kv_heads x max_tiles).  Writes attn f32 and,
// when act_q is non-null, Q8_0 blocks of each head's output.  part_* hold
// n_heads * max_tiles partials; counters (n_kv_heads) must start at zero and
// are left at zero.
int launch_attn_decode(hipStream_t s, const float* q, const float* kcache, const float* vcache,
                       const int* pos, int n_heads, int n_kv_heads, int head_dim, int max_tiles,
                       float* part_m, float* part_l, float* part_o, unsigned* counters, float* attn,
                       int8_t* act_q, uint16_t* act_d);
// Prefill: m query rows at positions pos0 .. pos0+m-1 against keys 0..pos0+m-1.
// Writes the rows to out and/or, when act_q is non-null, their Q8_0 blocks
// ([m][n_heads*64] and [m][n_heads*2]: what launch_quantize_rows makes of
// out, bit for bit); either may be null.
// kv_split: attn_split_words(max_keys, n_kv_heads) words of workspace, into
// which the layer's K and V rows are split (f16 halves) before the
// attention; pos0 + m may not exceed max_keys.
size_t attn_split_words(int max_keys, int n_kv_heads);
int launch_attn_prefill(hipStream_t s, const float* q, const float* kcache, const float* vcache,
                        int pos0, int m, int n_heads, int n_kv_heads, int head_dim,
                        uint32_t* kv_split, int max_keys,
                        float* out, int8_t* act_q = nullptr, uint16_t* act_d = nullptr);
// Any head_dim: one wavefront per (query, head) row; op-level entry point.
int launch_sdpa_generic(hipStream_t s, const float* q, const float* k, const float* v, float* out,
                        int seq_q, int seq_k, int n_heads, int n_kv_heads, int head_dim);

// ---- row kernels (k_misc.hip) -------------------------------------------
// An id past the table sets *id_error (the row read is clamped in bounds).
int launch_embed(hipStream_t s, const MatView& table, int wtype, const uint32_t* tokens,
                 int n_tokens, int dim, float* out, uint32_t* id_error);
int launch_rmsnorm_rows(hipStream_t s, const float* x, const float* w, int rows, int dim,
                        float eps, float* out, int8_t* act_q, uint16_t* act_d);
int launch_quantize_rows(hipStream_t s, const float* x, size_t n, int8_t* qs, uint16_t* d);
int launch_pack_q8_blocks(hipStream_t s, const int8_t* qs, const uint16_t* d, size_t nblocks,
                          void* gguf_blocks);
int launch_unpack_q8_blocks(hipStream_t s, const void* gguf_blocks, size_t nblocks, int8_t* qs,
                            uint16_t* d);
// Row m of qkv ([m][ld], q | k | v) is at position pos0 + m: q is rotated into
// q_out [m][q_dim], k rotated and v copied into cache row pos0 + m.
int launch_rope_kv_rows(hipStream_t s, const float* qkv, int ld, int rows, int q_dim, int kv_dim,
                        int head_dim, int pos0, const float2* rope, float* q_out, float* kcache,
                        float* vcache);
int launch_rope_rows_table(hipStream_t s, float* t, int rows, int row_dim, int head_dim,
                           const float2* cs_rows);
// gu holds [gate | up] rows of 2*ffn; writes silu(gate)*up for n = rows*ffn
// values (and their Q8_0 blocks when act_q is non-null).
int launch_silu_mul_rows(hipStream_t s, const float* gu, int ffn, size_t n, float* out,
                         int8_t* act_q, uint16_t* act_d);
int launch_silu(hipStream_t s, float* x, size_t n);
int launch_mul(hipStream_t s, const float* a, const float* b, float* out, size_t n);
int launch_add_inplace(hipStream_t s, float* a, const float* b, size_t n);
int launch_softmax_row(hipStream_t s, const float* in, float* out, int n);
// Final argmax over the LM head partials (or a full scan when a NaN was
// seen); writes token[0], appends to history[*pos_hist] when history is
// non-null, and advances *pos by `advance`.
int launch_argmax_final(hipStream_t s, const float* logits, int n, const float* part_val,
                        const int* part_idx, const int* part_nan, int n_parts, uint32_t* token,
                        int* pos, int advance, uint32_t* history, int* n_hist);
int launch_argmax_partials(hipStream_t s, const float* logits, int n, float* part_val,
                           int* part_idx, int* part_nan, int n_parts);
int launch_block_isums(hipStream_t s, const int8_t* aq, const MatView& w, int wtype, int row,
                       int32_t* out);
int launch_copy_i32(hipStream_t s, const int* src, int* dst);
// out = log p(*idx) under softmax(logits[0..n)) in f64 (*idx < n).
int launch_log_softmax_at(hipStream_t s, const float* logits, int n, const uint32_t* idx, double* out,
                          uint32_t* id_error);

// ---- prefill matmul (k_gemm.hip) ----------------------------------------
// out[m, rows] (+)= in[m, k] @ W.  a8: activations given as Q8_0 (aq/ad,
// [m][k] / [m][k/32]); otherwise f32 activations x [m][k].
// ws: room for ws_floats floats of partial tiles, for a K split of the
// integer path when the output has few tiles (null: no split).
constexpr size_t kGemmSplitFloats = (size_t)4 << 20;
// The model context's K-split workspace: three partial 2048 x 2048 tiles
// (the FFN down projection of a 2048-token prompt) and more.
constexpr size_t kPrefillSplitFloats = (size_t)16 << 20;
// Integer matmul launches on the matrix cores since the last reset: out[0]
// all, [1] with a K split, [2] on 128 x 128 tiles, [3] the largest split.
void gemm_counters(bool reset, uint64_t* out);
int launch_gemm(hipStream_t s, const MatView& w, int wtype, bool a8, const int8_t* aq,
                const uint16_t* ad, const float* x, int m, float* out, int ldo, bool accumulate,
                float* ws = nullptr, size_t ws_floats = 0);
// The FFN gate/up projection (w: [gate | up], 2 * ffn rows) of m prompt rows
// given as Q8_0, with silu(gate) * up written as Q8_0 blocks (act_q [m][ffn],
// act_d [m][ffn / 32]) in the same launch: what launch_gemm followed by
// launch_silu_mul_rows writes, bit for bit.  act_q/act_d must not overlap
// aq/ad (every workgroup reads every row).  ws_floats: the workspace size
// launch_gemm would be given (it picks the same tiling).  Returns -1
// (nothing launched) where the fused form does not apply (small grids,
// K-split tilings, pinned tilings).
int launch_gateup_silu(hipStream_t s, const MatView& w, int wtype, const int8_t* aq, const uint16_t* ad, int m,
                       int8_t* act_q, uint16_t* act_d, size_t ws_floats = 0);
// The stacked q|k|v projection (w: q_dim + 2 kv_dim rows) of m prompt rows
// at positions pos0.. given as Q8_0, with RoPE on q and k and the KV-cache
// append in the same launch (or, on a K-split tiling, in the launch that sums
// the partials in ws): what launch_gemm with the same workspace followed by
// launch_rope_kv_rows writes, bit for bit (q_out [m][q_dim], the caches
// [position][kv_dim]).  Returns -1 (nothing launched) where the fused form
// does not apply.
int launch_qkv_rope(hipStream_t s, const MatView& w, int wtype, const int8_t* aq, const uint16_t* ad, int m,
                    int q_dim, int kv_dim, int head_dim, int pos0, const float2* rope, float* q_out, float* kcache,
                    float* vcache, float* ws = nullptr, size_t ws_floats = 0);

// ---- persistent decode step (k_step.hip) -----------------------------------
struct StepLayer {
    MatView qkv, o, gateup, down;
    const float* attn_norm;
    const float* ffn_norm;
};

// Exchange words of the persistent decode step: payload in the low 32 bits,
// the producing phase's tag in the high 32 bits.
struct Xchg {
    unsigned long long* h;  // hidden row [dim]
    unsigned long long* q;  // q after RoPE [n_heads*64]
    unsigned long long* k;  // new K row [n_kv_heads*64]
    unsigned long long* v;  // new V row [n_kv_heads*64]
    unsigned long long* a;  // attention row as Q8_0: payload [q_dim/4] then scales [q_dim/32]
    unsigned long long* f;  // FFN activation as Q8_0: payload [ffn/4] then scales [ffn/32]
    unsigned long long* p;  // argmax partials [3 * grid]
    unsigned long long* t;  // attention tile partials [n_heads][max_tiles][64 + 2]
};
size_t exchange_words(int dim, int ffn, int n_heads, int n_kv_heads, int max_tiles, int grid);

// Everything one decode step reads and writes.  The launch reads *pos,
// *token and *epoch; workgroup 0 writes the next token, appends it to
// history[*n_hist], advances *pos and *epoch.  *epoch starts at zero and is
// never rewound; *error is raised when a wait exceeds spin_limit wall-clock
// ticks, after which every workgroup leaves.
struct StepArgs {
    const StepLayer* layers;  // device array [n_layers]
    // The weight rows in the order each CU multiplies them (launch_build_stream):
    // CU w's stream starts at unit w * stream_stride (16-byte units).
    const void* stream;
    size_t stream_stride;
    MatView embd, head;
    const float* out_norm;
    int n_layers, dim, ffn, n_heads, n_kv_heads, vocab;
    float eps;
    Xchg x;
    float* kcache;
    float* vcache;
    size_t kv_layer;  // floats per layer of each cache
    const float2* rope;
    int* pos;
    uint32_t* token;
    uint32_t* history;
    int* n_hist;
    float* logits;
    int max_tiles;
    unsigned* epoch;
    int* error;
    uint32_t* id_error;  // set when *token is past the embedding table
    long long spin_limit;
    float* dbg_normed;  // layer-0 attention norm (workgroup 0), optional
    // Quantized activations of every site (the context's tap_q / tap_d
    // layout): layer 0's attention-norm site always, every site when taps
    // is non-zero (written by workgroup 0).
    int8_t* dbg_qs;
    uint16_t* dbg_d;
    int taps;
    float* last_hidden;  // final norm (workgroup 0), optional
    int8_t* head_qs;
    uint16_t* head_d;
    // Optional timeline (measurement): per workgroup, trace_stride wall-clock
    // stamps, 20 slots per layer (k_step.hip TraceSlot) after slot 0 (start).
    unsigned long long* trace;
    int trace_stride;
};

// True when the step kernel can run the model with `grid` workgroups.
bool decode_step_fits(int dim, int ffn, int n_heads, int n_kv_heads, int grid);
// 16-byte units per CU in the weight stream of a model run over `grid` CUs.
size_t decode_stream_stride(int wtype, int n_layers, int dim, int ffn, int n_heads, int n_kv_heads, int vocab,
                            int grid);
// Fills dst (grid * stride units) with the per-CU weight streams of the
// layers, head and geometry in `a` (a.stream_stride must be the stride).
int launch_build_stream(hipStream_t s, int wtype, const StepArgs& a, int grid, void* dst);
// Launch of one decode step over `grid` workgroups (one per CU).  pos, the
// position the step decodes as the host counts it, picks the kernel instance
// (any instance computes every position).
int launch_decode_step(hipStream_t s, int wtype, const StepArgs& a, int grid, int pos);
// Workgroups for the decode step on the current device (one per CU).
int decode_step_max_grid(int wtype, int* grid);

}  // namespace sq
