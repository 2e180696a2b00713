/*
 * Oracle: a CPU restatement of squirrel-rs's Llama token loop arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the reference arithmetic the HIP
 * implementation is tested against, and the timed CPU baseline.  Only tests/, the smoke() entry
 * and bench.py's cpu_baseline leg may load it; the product path never does.
 *
 * Every function follows one reference function (cited file:line, paths
 * relative to the squirrel-rs repository root) with the same operation order,
 * so that float results are bit-identical to the reference as compiled for
 * x86_64 (scalar fallbacks, no FMA contraction, sequential folds).  Build with
 * -ffp-contract=off and without -ffast-math.
 *
 * Status codes mirror KernelError (src/kernels/kernel_error.rs:2-7):
 *   0 ok, 1 ShapeMismatch, 2 InvalidType, 3 EmptyInput, 4 TensorAlignmentError.
 */
#ifndef SQ_ORACLE_H
#define SQ_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { OR_OK = 0, OR_SHAPE = 1, OR_INVALID_TYPE = 2, OR_EMPTY = 3, OR_ALIGN = 4 };

/* GGML type ids (src/file_parser/ggml_type.rs:8-41). */
enum { OR_F32 = 0, OR_Q4_0 = 2, OR_Q8_0 = 8, OR_BF16 = 30 };

/* Linear-layer arithmetic modes.
 *   OR_W8A32:     f32 activations against the weight blocks; the path every
 *                 non-aarch64 build runs (src/kernels/matmul.rs:102-103,
 *                 src/ops/linear.rs:160-167).
 *   OR_W8A8:      activations quantized to Q8_0 once per projection group,
 *                 integer block dots, scalar-twin combine order
 *                 (src/ops/linear.rs:83-143, src/kernels/dot_prod.rs:378-403).
 *   OR_W8A8_NEON: same integer sums, combined in the order of the aarch64
 *                 NEON kernels (src/kernels/dot_prod.rs:189-252,306-374);
 *                 used to measure the reference's own order sensitivity.
 * BF16 weights always use f32 activations (src/ops/linear.rs:34). */
enum { OR_W8A32 = 0, OR_W8A8 = 1, OR_W8A8_NEON = 2 };

#pragma pack(push, 1)
typedef struct { uint16_t d; int8_t qs[32]; } or_block_q8_0;  /* 34 B, tensor.rs:10-15 */
typedef struct { uint16_t d; uint8_t qs[16]; } or_block_q4_0; /* 18 B, tensor.rs:17-25 */
#pragma pack(pop)

/* ---- scalar conversions (crate `half` 2.7.1 semantics) ---- */
uint16_t or_f32_to_f16(float f);     /* IEEE-754 binary16, round to nearest even */
float or_f16_to_f32(uint16_t h);     /* exact widening */
float or_bf16_to_f32(uint16_t b);    /* exact widening */
void or_f32_to_f16_array(const float* x, size_t n, uint16_t* out);

/* ---- threading (stands in for rayon's global pool) ---- */
int or_set_threads(int n);           /* returns the thread count in effect */
int or_get_threads(void);

/* ---- dot_prod.rs ---- */
void or_quantize_row_q8_0(const float* src, size_t n, or_block_q8_0* out);
float or_dot_f32_q8_0(const float* a, const or_block_q8_0* b, size_t nblocks);
float or_dot_f32_q4_0(const float* a, const or_block_q4_0* b, size_t nblocks);
float or_dot_f32_bf16(const float* a, const uint16_t* b, size_t n);
float or_dot_q8_0_q8_0(const or_block_q8_0* a, const or_block_q8_0* b, size_t nblocks);
float or_dot_q8_0_q4_0(const or_block_q8_0* a, const or_block_q4_0* b, size_t nblocks);
float or_dot_q8_0_q8_0_neon(const or_block_q8_0* a, const or_block_q8_0* b, size_t nblocks);
float or_dot_q8_0_q4_0_neon(const or_block_q8_0* a, const or_block_q4_0* b, size_t nblocks);
int32_t or_isum_q8_0_q8_0(const or_block_q8_0* a, const or_block_q8_0* b);
int32_t or_isum_q8_0_q4_0(const or_block_q8_0* a, const or_block_q4_0* b);
int or_dot_f32_f32(const float* a, size_t na, const float* b, size_t nb, float* out);
void or_dequantize_row(int wtype, const void* blocks, size_t n, float* out);

/* ---- matmul.rs / ops/linear.rs ----
 * out[m, n_out] = in[m, k] @ W, W stored as n_out rows of k/32 blocks
 * (GGUF dims [k, n_out]).  Rows of `in` are processed serially, output
 * columns in parallel (src/kernels/matmul.rs:28-64). */
int or_linear(const float* in, size_t m, size_t k, int wtype, const void* w, size_t n_out,
              float* out, int mode);
/* Integer-path per-block sums for one (activation row, weight row) pair:
 * isums[b] = sum_i qa[b,i] * qw[b,i], the exact i32 the reference forms
 * before any scale is applied. */
int or_block_isums(const or_block_q8_0* a, int wtype, const void* w_row, size_t nblocks,
                   int32_t* isums);

/* ---- softmax.rs, rms_norm.rs, rope.rs, silu.rs, sigmoid.rs ---- */
int or_softmax(const float* a, float* out, size_t n);
int or_rms_norm_rows(const float* in, const float* w, float* out, size_t rows, size_t dim,
                     float eps);
int or_rope_rows(float* t, size_t rows, size_t row_dim, size_t base_pos, const float* inv_freq,
                 size_t half);
float or_sigmoid(float x);
void or_silu(float* x, size_t n);
void or_rope_inv_freq(size_t head_dim, float base, float factor, float low, float high,
                      float orig_ctx, float* out);

/* ---- attention.rs ---- */
int or_sdpa(const float* q, const float* k, const float* v, float* out, size_t seq_q,
            size_t seq_k, size_t n_heads, size_t n_kv_heads, size_t head_dim);

/* ---- samplers/greedy.rs ---- */
int64_t or_greedy(const float* logits, size_t n);

/* ---- embedding.rs ---- */
int or_embed(const uint32_t* tokens, size_t n_tokens, int wtype, const void* table,
             size_t embed_dim, size_t vocab, float* out);

/* ---- models/llama: the whole forward pass ---- */
typedef struct {
    int n_layers, dim, ffn_dim, n_heads, n_kv_heads, head_dim, vocab;
    float eps;
    int wtype;               /* GGML type of every matrix (Q8_0, Q4_0 or BF16) */
    const void* tok_embd;    /* [vocab rows x dim] */
    const void* output;      /* LM head rows; equal to tok_embd when tied */
    const float* output_norm;
    const void* const* layer; /* 9 per layer: attn_norm, q, k, v, o, ffn_norm, gate, up, down */
    const float* inv_freq;   /* head_dim / 2 entries */
} or_llama;

typedef struct or_ctx or_ctx;
or_ctx* or_ctx_new(const or_llama* m, size_t max_positions, int mode);
void or_ctx_free(or_ctx* c);
void or_ctx_reset(or_ctx* c);
size_t or_ctx_seq_len(const or_ctx* c);
/* One Llama3_2::forward (src/models/llama/model.rs:45-97).  Logits of the
 * last token are left in the context.  Status as above; 5 = cache full. */
int or_forward(const or_llama* m, or_ctx* c, const uint32_t* ids, size_t n);
const float* or_ctx_logits(const or_ctx* c);
/* Debug views of the most recent forward: the final normed last row. */
const float* or_ctx_last_hidden(const or_ctx* c);

/* matmul_prequant_q (src/kernels/matmul.rs:133-171): linear on activations
 * already quantized to Q8_0 blocks (m rows of k/32 blocks). */
int or_linear_prequant(const or_block_q8_0* aq, size_t m, size_t k, int wtype, const void* w,
                       size_t n_out, float* out, int mode);

/* Phase lock of the integer path.  Every quantization site of a forward
 * (per layer: 0 the attention-norm output, 1 the attention output, 2 the
 * FFN-norm output, 3 the FFN activation, each n rows; then site 0 of layer
 * n_layers, the final norm's last row) is quantized by the oracle and
 * compared block by block with an implementation's blocks, given in that
 * order in `blocks`.  An element may differ by one step only where the
 * oracle's scaled value x * (1/scale) lies within `tol` quanta of a rounding
 * midpoint (a flip that any f32 rounding difference upstream can cause); a
 * block scale may differ by one binary16 step only where the f32 scale lies
 * at the midpoint of the two.  Everything else counts as bad.  The forward
 * then continues with the implementation's blocks, so the logits compare the
 * two at f32 rounding level.  Integer modes only.  Sites are numbered 0
 * attention-norm output, 1 attention output, 2 FFN-norm output, 3 FFN
 * activation (layers 0..n-1), and 4 the LM-head input (layer n). */
typedef struct {
    const or_block_q8_0* blocks;
    float tol;
    uint64_t values, flips, scale_flips, bad;
    int first_bad_layer, first_bad_site;
    size_t first_bad_index;
    float first_bad_dist; /* distance from the midpoint, -1 for a scale mismatch */
    /* the largest distance from a midpoint (quanta) of an accepted element
     * flip, and the largest |scale - midpoint| / midpoint of an accepted
     * scale flip */
    float max_flip_dist;
    float max_scale_rel;
    uint64_t site_values[5], site_flips[5];
    /* Test hook, a planted systematic error: when plant_quanta is non-zero,
     * the implementation's blocks of site (plant_layer, plant_site) are
     * replaced, before the check, by the oracle's own quantization of that
     * site with every scaled value moved by plant_quanta quanta. */
    int plant_layer, plant_site;
    float plant_quanta;
} or_lock;
int or_forward_locked(const or_llama* m, or_ctx* c, const uint32_t* ids, size_t n, or_lock* lock);

#ifdef __cplusplus
}
#endif
#endif
