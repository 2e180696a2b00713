/*
 * squirrel-hip: MI355X (gfx950) implementation of squirrel-rs's Llama token
 * loop behind a C ABI.
 *
 * Every entry point returns an int status:
 *   0            ok
 *   1..4         KernelError in declaration order (src/kernels/kernel_error.rs:2-7):
 *                ShapeMismatch, InvalidType, EmptyInput, TensorAlignmentError
 *   16..         load-path errors (IO, malformed GGUF, ConfigError, WeightsError,
 *                UnsupportedQuantScheme, cache full)
 *   64           a HIP runtime error
 * sq_last_error() returns a message for the most recent failure on the
 * calling thread.
 *
 * Pointers named d_* are device pointers (HBM); everything else is host
 * memory.  Model handles are read-only after load and may be shared between
 * threads; a context belongs to one thread at a time (the reference's
 * `forward(&self, &mut ModelContext)` rule, src/models/common/model.rs:16).
 */
#ifndef SQUIRREL_HIP_H
#define SQUIRREL_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---------------------------------------------------- */
#define SQ_OK 0
#define SQ_ERR_SHAPE 1        /* KernelError::ShapeMismatch */
#define SQ_ERR_INVALID_TYPE 2 /* KernelError::InvalidType */
#define SQ_ERR_EMPTY 3        /* KernelError::EmptyInput */
#define SQ_ERR_ALIGN 4        /* KernelError::TensorAlignmentError */
#define SQ_ERR_IO 16          /* file open / read / mmap failure */
#define SQ_ERR_FORMAT 17      /* malformed GGUF (truncated, bad type id, bad bool) */
#define SQ_ERR_CONFIG 18      /* ConfigError (config.rs:3-7) */
#define SQ_ERR_WEIGHTS 19     /* WeightsError::MissingTensor (weights.rs:10-16) */
#define SQ_ERR_UNSUPPORTED 20 /* gguf_tensor_info::Error::UnsupportedQuantScheme */
#define SQ_ERR_CACHE_FULL 21  /* more positions than the context was created for */
#define SQ_ERR_ARG 22         /* null handle or invalid argument */
#define SQ_ERR_HIP 64

/* GGML type ids (src/file_parser/ggml_type.rs:8-41) */
#define SQ_F32 0
#define SQ_Q4_0 2
#define SQ_Q8_0 8
#define SQ_BF16 30

/* Context flags */
#define SQ_CTX_F32_ACTS 1u  /* SQUIRREL_F32_ACTS=1 (src/ops/linear.rs:14-19): W8A32 matvecs */
#define SQ_CTX_NO_GRAPH 2u  /* multi-kernel decode: launch kernel by kernel (no hipGraph) */
#define SQ_CTX_MULTI_KERNEL 4u /* decode with one kernel per op (a hipGraph) instead of the
                                  persistent one-launch-per-token kernel */

/* Generation flags */
#define SQ_GEN_IGNORE_EOS 1u  /* SQUIRREL_IGNORE_EOS=1 (src/text_generator.rs:15-19) */
#define SQ_GEN_NO_KV_CACHE 2u /* SQUIRREL_NO_KV_CACHE=1 (src/text_generator.rs:9-13) */

const char* sq_last_error(void);
const char* sq_version(void);

/* ---- device plumbing (for FFI callers without their own allocator) ---- */
int sq_device_count(int* n);
int sq_malloc(void** d_ptr, size_t bytes);
int sq_free(void* d_ptr);
int sq_memcpy_h2d(void* d_dst, const void* src, size_t bytes);
int sq_memcpy_d2h(void* dst, const void* d_src, size_t bytes);
int sq_memset(void* d_dst, int value, size_t bytes);
int sq_synchronize(void);

/* ---- GGUF files --------------------------------------------------------
 * Synthetic Llama GGUF writer: the seeded random-init models the benchmarks
 * run on (no reference counterpart; the reference downloads real files).
 * Matrices ~ N(0, std) quantized per 32-block; norm gains 1.0 (F32); tied
 * embeddings (no output.weight); metadata keys per config.rs:29-106. */
typedef struct {
    uint32_t n_layers, dim, ffn_dim, n_heads, n_kv_heads, vocab, context_length;
    uint32_t wtype;       /* SQ_Q8_0, SQ_Q4_0 or SQ_BF16 */
    uint64_t seed;
    float std_dev;        /* 0.02 */
    float rope_base;      /* 500000 */
    float rms_eps;        /* 1e-5 */
    uint32_t bos, eos;
} sq_synth_spec;
int sq_synth_write_gguf(const char* path, const sq_synth_spec* spec);

/* ---- model / context: the `Model` trait (src/models/common/model.rs:6-26) */
typedef struct sq_model sq_model;
typedef struct sq_ctx sq_ctx;

typedef struct {
    uint32_t n_layers, dim, ffn_dim, n_heads, n_kv_heads, head_dim, vocab;
    uint32_t context_length, bos, eos, wtype, tied_output;
    float rope_base, rms_eps;
    uint64_t weight_bytes; /* bytes of every matrix as uploaded */
} sq_model_info;

/* Parse a GGUF file, read its LlamaConfig (config.rs:29-73) and resolve and
 * check every tensor LlamaWeights::from_gguf needs (weights.rs:50-97)
 * without touching the GPU.  inv_freq (head_dim/2 floats) may be null.
 * Returns the same status the loader would return before uploading. */
int sq_gguf_inspect(const char* path, sq_model_info* info, float* inv_freq, size_t n);

/* Llama3_2::from_gguf (src/models/llama/model.rs:20-32) minus the tokenizer:
 * parse GGUF, read LlamaConfig (config.rs:29-73), resolve tensors
 * (weights.rs:50-97) and upload them to the current device. */
int sq_model_load_gguf(const char* path, sq_model** out);
int sq_model_info_get(const sq_model* m, sq_model_info* info);
/* The RoPE inverse-frequency table the model uses (config.rs:83-127). */
int sq_model_rope_inv_freq(const sq_model* m, float* out, size_t n);
void sq_model_free(sq_model* m);

/* Model::new_context (model.rs:36-43): a device KV cache preallocated for
 * max_positions, the workspace, one HIP stream and the decode hipGraph. */
int sq_ctx_new(const sq_model* m, size_t max_positions, uint32_t flags, sq_ctx** out);
void sq_ctx_free(sq_ctx* c);
/* ModelContext::reset_cache (context.rs:25-27). */
int sq_ctx_reset(sq_ctx* c);
/* How decode steps run: 1 = the persistent one-launch-per-token kernel
 * (Q8_0 / Q4_0 integer path, head_dim 64, width <= 2048), 0 = one kernel per
 * op replayed as a hipGraph.  No reference counterpart (measurement aid).
 * The persistent kernel occupies one workgroup per CU; the environment
 * variable SQUIRREL_STEP_GRID, read by sq_ctx_new, caps that count (a cap the
 * shape does not fit in selects the multi-kernel path). */
int sq_ctx_decode_kernel(const sq_ctx* c);
/* Timeline of the persistent decode step (measurement aid, no reference
 * counterpart).  With tracing enabled every step records, per workgroup,
 * `stride` wall-clock stamps (device wall clock, hipDeviceAttributeWallClockRate
 * kHz): [0] start; for layer l at [1 + 20l + j]: j = 0 QKV input row gathered
 * and quantized, 1 QKV done, 2 attention done, 3 tile merge done, 4 o-projection
 * inputs gathered, 5 o-projection done, 6 gate/up input row gathered and
 * quantized, 7 gate/up dot done, 8 gate/up done, 9 down inputs gathered,
 * 10 down done, 11-13 the first attention item's q gathered / scores /
 * outputs published, 14-15 durations (ticks) the first compute wavefront
 * waited for weights in the gate/up phase / the layer, 16 the QKV input
 * row's polls begin; then [1 + 20L] LM-head inputs gathered,
 * [2 + 20L] LM head done, [3 + 20L] token resolved (workgroup 0 only); 0 where
 * a slot was not reached.
 * _read copies the most recent step's stamps (grid * stride values); with
 * out == NULL it only reports grid and stride.  While the trace or the
 * activation taps below are on, decode steps run a kernel instance built
 * with these outputs, about 3.5% slower per token than the one used
 * otherwise; both compute the same logits bit for bit. */
int sq_ctx_step_trace(sq_ctx* c, int enable);
/* The current device's wall-clock rate in kHz (the unit of the step trace). */
int sq_device_wall_clock_khz(int* khz);
int sq_ctx_step_trace_read(sq_ctx* c, uint64_t* out, size_t n, int* grid, int* stride);
size_t sq_ctx_seq_len(const sq_ctx* c);
/* Quantized-activation taps (measurement and parity aid, no reference
 * counterpart).  The integer path quantizes activations to Q8_0 at four sites
 * per layer -- the attention-norm output and the attention output (inputs of
 * linear_shared / linear in layers::attention, src/models/llama/layers.rs:24-58),
 * the FFN-norm output and the FFN activation (layers::ffn, layers.rs:64-77) --
 * and once for the LM head.  With taps enabled every forward records them;
 * the one-kernel-per-op decode step always does.  _read copies those of the
 * most recent forward (n rows) as GGUF Q8_0 blocks (34 B each): per layer, per
 * site, n rows of k/32 blocks (k = dim, q_dim, dim, ffn_dim), then the
 * LM-head input row (dim/32 blocks).  n_blocks must hold them all. */
int sq_ctx_act_taps(sq_ctx* c, int enable);
int sq_ctx_act_tap_read(sq_ctx* c, void* blocks, size_t n_blocks);

/* Model::forward (model.rs:45-97): n > 1 runs the batched prefill, n == 1 a
 * decode step.  Asynchronous on the context stream. */
int sq_forward(const sq_model* m, sq_ctx* c, const uint32_t* ids, size_t n);
/* ModelContext::logits (context.rs:20-22): copies the last token's logits
 * (vocab floats); synchronizes. */
int sq_logits(sq_ctx* c, float* out, size_t n);
/* GreedySampler::sample (src/samplers/greedy.rs:6-15) of the last forward,
 * computed on the device with the reference's tie rule; synchronizes. */
int sq_argmax(sq_ctx* c, uint32_t* token);
/* Debug view: the final normed hidden row fed to the LM head (dim floats). */
int sq_ctx_last_hidden(sq_ctx* c, float* out, size_t n);
/* Debug view of layer 0's first attention-norm output of the most recent
 * decode step: f32 row (dim floats) and its Q8_0 blocks (dim/32 * 34 B, GGUF
 * layout).  Lets tests check the fused norm+quantize kernel bit for bit. */
int sq_ctx_debug_act(sq_ctx* c, float* normed, void* blocks);

/* One window of the perplexity harness (src/bin/perplexity.rs:61-110): on a
 * reset context, prefill ids[0, burn) (the burn-in), then for every i in
 * [burn, n) write log p(ids[i]) of the current logits to logp[i - burn]
 * (f64, as sq_log_softmax_at) and, while i + 1 < n, teacher-force ids[i]
 * with one decode step.  The whole window is enqueued on the context stream
 * and the n - burn values come back with one copy.  Needs 1 <= burn < n and
 * n - 1 <= max_positions; every id below the vocabulary size. */
int sq_ctx_score(sq_ctx* c, const uint32_t* ids, size_t n, size_t burn, double* logp);

/* TextTokenGenerator::generate (src/text_generator.rs:38-101) on token ids:
 * prefill `prompt`, then greedy decode until max_tokens tokens or EOS.
 * out_tokens receives the generated ids (max_tokens capacity); step_ms, when
 * not null, receives the wall time of every step as the reference's per-step
 * timer measures it (forward + logits + sample; step 1 includes the prefill).
 * Decode steps replay the captured hipGraph with the next step launched
 * before the previous token is read back. */
int sq_generate(const sq_model* m, sq_ctx* c, const uint32_t* prompt, size_t n_prompt,
                size_t max_tokens, uint32_t flags, uint32_t* out_tokens, size_t* n_out,
                double* step_ms);

/* ---- operator level: mirrors the src/ops files on device buffers -------- */

/* A weight matrix uploaded in the device layout (the WeightBlock extension
 * point, src/kernels/tensor.rs:37-69): `blocks` holds `rows` rows of k/32
 * GGUF blocks (host memory). */
typedef struct sq_weight sq_weight;
int sq_weight_upload(int wtype, const void* blocks, size_t rows, size_t k, sq_weight** out);
void sq_weight_free(sq_weight* w);

/* quantize_row_q8_0 (src/kernels/dot_prod.rs:10-31): n/32 blocks of 34 B in
 * GGUF layout. */
int sq_quantize_row_q8_0(const float* d_x, size_t n, void* d_blocks);
/* linear (src/ops/linear.rs:26-70): d_out[m, rows] = d_in[m, k] @ W.  Q8_0 /
 * Q4_0 quantize the activations (the reference's aarch64 path).  The
 * f32-activation kernels (SQ_CTX_F32_ACTS in flags, and BF16 weights, which
 * always take f32 activations) are disabled in this build and return
 * SQ_ERR_UNSUPPORTED. */
int sq_linear(const float* d_in, size_t m, size_t k, const sq_weight* w, float* d_out,
              uint32_t flags);
/* No counterpart in the reference: sq_linear for callers that cannot
 * allocate device memory (tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments, kernels and results as sq_linear, but the
 * scratch (Q8_0 activations and K-split partial tiles) is a static per-GPU
 * device array of 20.25 MiB: m * k may not exceed 4 Mi elements
 * (SQ_ERR_SHAPE otherwise).  Calls that overlap on one GPU share that array
 * and race.  Each call runs on the null stream and synchronizes it, so it
 * cannot be recorded under a stream capture. */
int sq_linear_noalloc(const float* d_in, size_t m, size_t k, const sq_weight* w, float* d_out,
                      uint32_t flags);
/* linear_shared (src/ops/linear.rs:73-168): several projections of one input,
 * its activations quantized once. */
int sq_linear_shared(const float* d_in, size_t m, size_t k, const sq_weight* const* ws,
                     float* const* d_outs, size_t n_weights, uint32_t flags);
/* Per-block integer sums of one quantized activation row against weight row
 * `row` (the exact i32 of dot_prod.rs:381-384 / 394-399): nblocks int32. */
int sq_block_isums(const void* d_act_blocks, const sq_weight* w, size_t row, int32_t* d_isums);
/* embed (src/ops/embedding.rs:10-52). */
int sq_embed(const uint32_t* d_tokens, size_t n, const sq_weight* table, float* d_out);
/* rms_norm (src/ops/rms_norm.rs:13-43) over `rows` rows of `dim`. */
int sq_rms_norm(const float* d_in, const float* d_w, float* d_out, size_t rows, size_t dim,
                float eps);
/* rope_rows (src/ops/rope.rs:6-32), in place; inv_freq is host memory. */
int sq_rope_rows(float* d_t, size_t rows, size_t row_dim, size_t base_pos,
                 const float* inv_freq, size_t half);
/* sdpa_cached (src/ops/sdpa.rs:8-38) / sdpa_f32 (src/kernels/attention.rs:11-70). */
int sq_sdpa(const float* d_q, const float* d_k, const float* d_v, float* d_out, size_t seq_q,
            size_t seq_k, size_t n_heads, size_t n_kv_heads, size_t head_dim);
/* silu (src/ops/silu.rs:4-8), in place. */
int sq_silu(float* d_x, size_t n);
/* elementwise_mul (src/ops/elementwise_mul.rs:8-22). */
int sq_elementwise_mul(const float* d_a, const float* d_b, float* d_out, size_t n);
/* elementwise_add (src/ops/elementwise_add.rs:8-15): d_a += d_b. */
int sq_elementwise_add(float* d_a, const float* d_b, size_t n);
/* GreedySampler::sample (src/samplers/greedy.rs:6-15) over d_logits. */
int sq_greedy(const float* d_logits, size_t n, uint32_t* token);
/* softmax_f32 (src/kernels/softmax.rs:4-27) over one row. */
int sq_softmax(const float* d_in, float* d_out, size_t n);
/* log_softmax_at (src/bin/perplexity.rs:112-117): log p(idx) under
 * softmax(d_logits[0..n)) in f64 -- the maximum folded in f32, the sum of
 * exp(l - max) in f64 (a fixed-order tree rather than a sequential fold).
 * idx >= n is SQ_ERR_ARG (the reference would panic on the index). */
int sq_log_softmax_at(const float* d_logits, size_t n, uint32_t idx, double* out);

/* ---- measurement -----------------------------------------------------
 * Replays one kernel of the context's decode step `iters` times on the
 * context stream between two HIP events and returns the mean duration.
 * which: 0 = fused gate/up matvec, 1 = LM head (+ argmax), 2 = down matvec,
 * 3 = QKV matvec, 4 = attention, 5 = o-projection; the per-layer kernels are
 * those of layer 1 (layer 0 when the model has one layer).  The context must
 * have run at least one decode step and have a free KV position (replays
 * write the KV row at the current position); the replays write the same
 * buffers the step does, so reset or re-prefill the context afterwards. */
int sq_ctx_time_kernel(sq_ctx* c, int which, int iters, double* mean_us, uint64_t* bytes);
/* Phase split of a batched prefill (measurement aid, no reference
 * counterpart): resets the context, prefills ids (n >= 2) with HIP events
 * between launch groups, and returns in ms[0..3] the milliseconds spent in the
 * integer matmuls (matrix cores, including a K split's sum), in the causal
 * attention, in everything else (embedding, norms, quantization, RoPE,
 * SiLU, LM head, argmax), and in the whole prefill.  The context holds the
 * prompt afterwards, as after sq_forward. */
int sq_ctx_prefill_phases(sq_ctx* c, const uint32_t* ids, size_t n, double* ms);
/* Matrix-core matmul launches in this process since the last reset
 * (measurement and test aid, no reference counterpart): out[0] all, [1] those
 * that split K over workgroups, [2] those on the full-rate kernel's 128 x 128
 * tiles, [3] the largest split count, [4] those on the full-rate kernel's
 * 128 x 64 tiles, [5] those on the few-rows kernel (32 x 32 tiles, inputs of
 * at most 32 rows) (out holds 6 values).  out may be null; reset != 0 zeroes
 * the counters afterwards. */
int sq_gemm_counters(int reset, uint64_t* out);

#ifdef __cplusplus
}
#endif
#endif
