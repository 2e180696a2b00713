// extern "C" entry points declared in include/squirrel_hip.h.
#include <cmath>
#include <cstring>
#include <string>
#include <vector>

#include "model.h"

namespace sq {

thread_local std::string g_err;

int set_error(int code, const std::string& msg) {
    g_err = msg;
    return code;
}

int synth_write(const std::string& path, const sq_synth_spec& s);

}  // namespace sq

using namespace sq;

namespace {

// Temporary device buffer for the operator-level entry points.
struct Tmp {
    void* p = nullptr;
    ~Tmp() {
        if (p) (void)hipFree(p);
    }
    int alloc(size_t n) {
        hipError_t e = hipMalloc(&p, n ? n : 1);
        if (e != hipSuccess) return set_error(SQ_ERR_HIP, std::string("hipMalloc: ") + hipGetErrorString(e));
        return 0;
    }
};

int finish(int st) {
    if (st) return st;
    hipError_t e = hipStreamSynchronize(nullptr);
    if (e != hipSuccess) return set_error(SQ_ERR_HIP, std::string("kernel: ") + hipGetErrorString(e));
    return 0;
}

}  // namespace

extern "C" {

const char* sq_last_error(void) { return g_err.c_str(); }
const char* sq_version(void) { return "squirrel-hip 0.1 (gfx950)"; }

int sq_device_count(int* n) {
    hipError_t e = hipGetDeviceCount(n);
    if (e != hipSuccess) {
        *n = 0;
        return set_error(SQ_ERR_HIP, std::string("hipGetDeviceCount: ") + hipGetErrorString(e));
    }
    return 0;
}

int sq_malloc(void** p, size_t bytes) {
    SQ_HIP_CHECK(hipMalloc(p, bytes ? bytes : 1));
    return 0;
}
int sq_free(void* p) {
    SQ_HIP_CHECK(hipFree(p));
    return 0;
}
int sq_memcpy_h2d(void* d, const void* s, size_t n) {
    SQ_HIP_CHECK(hipMemcpy(d, s, n, hipMemcpyHostToDevice));
    return 0;
}
int sq_memcpy_d2h(void* d, const void* s, size_t n) {
    SQ_HIP_CHECK(hipMemcpy(d, s, n, hipMemcpyDeviceToHost));
    return 0;
}
int sq_memset(void* d, int v, size_t n) {
    SQ_HIP_CHECK(hipMemset(d, v, n));
    return 0;
}
int sq_synchronize(void) {
    SQ_HIP_CHECK(hipDeviceSynchronize());
    return 0;
}

int sq_synth_write_gguf(const char* path, const sq_synth_spec* spec) {
    if (!path || !spec) return set_error(SQ_ERR_ARG, "synth: null argument");
    return synth_write(path, *spec);
}

// ------------------------------------------------------------ model / context

int sq_model_load_gguf(const char* path, sq_model** out) {
    if (!path || !out) return set_error(SQ_ERR_ARG, "load: null argument");
    return model_load(path, out);
}

int sq_gguf_inspect(const char* path, sq_model_info* info, float* inv_freq, size_t n) {
    if (!path || !info) return set_error(SQ_ERR_ARG, "inspect: null argument");
    sq_model* m = nullptr;
    int st = model_inspect(path, &m);
    if (st) return st;
    st = sq_model_info_get(m, info);
    if (!st && inv_freq) st = sq_model_rope_inv_freq(m, inv_freq, n);
    model_free(m);
    return st;
}

int sq_model_info_get(const sq_model* m, sq_model_info* i) {
    if (!m || !i) return set_error(SQ_ERR_ARG, "info: null argument");
    const Config& c = m->cfg;
    i->n_layers = c.n_layers;
    i->dim = c.dim;
    i->ffn_dim = c.ffn;
    i->n_heads = c.n_heads;
    i->n_kv_heads = c.n_kv_heads;
    i->head_dim = c.head_dim;
    i->vocab = c.vocab;
    i->context_length = c.context_length;
    i->bos = c.bos;
    i->eos = c.eos;
    i->wtype = m->wtype;
    i->tied_output = m->tied ? 1 : 0;
    i->rope_base = c.rope_base;
    i->rms_eps = c.eps;
    i->weight_bytes = m->weight_bytes;
    return 0;
}

int sq_model_rope_inv_freq(const sq_model* m, float* out, size_t n) {
    if (!m || !out || n < m->cfg.inv_freq.size()) return set_error(SQ_ERR_ARG, "rope_inv_freq: bad argument");
    memcpy(out, m->cfg.inv_freq.data(), m->cfg.inv_freq.size() * 4);
    return 0;
}

void sq_model_free(sq_model* m) { model_free(m); }

int sq_ctx_new(const sq_model* m, size_t max_positions, uint32_t flags, sq_ctx** out) {
    if (!out) return set_error(SQ_ERR_ARG, "ctx_new: null argument");
    return ctx_create(m, max_positions, flags, out);
}

void sq_ctx_free(sq_ctx* c) { ctx_destroy(c); }

int sq_ctx_reset(sq_ctx* c) {
    if (!c) return set_error(SQ_ERR_ARG, "reset: null context");
    return ctx_reset(c);
}

int sq_ctx_decode_kernel(const sq_ctx* c) { return c && c->persist ? 1 : 0; }

int sq_ctx_step_trace(sq_ctx* c, int enable) {
    if (!c) return set_error(SQ_ERR_ARG, "step_trace: null context");
    if (!c->persist) return set_error(SQ_ERR_UNSUPPORTED, "step_trace: the context has no persistent decode step");
    SQ_HIP_CHECK(hipStreamSynchronize(c->stream));
    if (!enable) {
        c->step.trace = nullptr;
        return 0;
    }
    const int stride = 20 * c->m->cfg.n_layers + 4;
    if (!c->s_trace) SQ_HIP_CHECK(hipMalloc((void**)&c->s_trace, (size_t)c->step_grid * stride * 8));
    SQ_HIP_CHECK(hipMemset(c->s_trace, 0, (size_t)c->step_grid * stride * 8));
    c->step.trace = c->s_trace;
    c->step.trace_stride = stride;
    return 0;
}

int sq_ctx_step_trace_read(sq_ctx* c, uint64_t* out, size_t n, int* grid, int* stride) {
    if (!c || !grid || !stride) return set_error(SQ_ERR_ARG, "step_trace_read: null argument");
    if (!c->s_trace || !c->step.trace) return set_error(SQ_ERR_ARG, "step_trace_read: tracing is not enabled");
    *grid = c->step_grid;
    *stride = c->step.trace_stride;
    const size_t need = (size_t)c->step_grid * c->step.trace_stride;
    if (!out) return 0;
    if (n < need) return set_error(SQ_ERR_ARG, "step_trace_read: buffer too small");
    SQ_HIP_CHECK(hipStreamSynchronize(c->stream));
    SQ_HIP_CHECK(hipMemcpy(out, c->s_trace, need * 8, hipMemcpyDeviceToHost));
    return 0;
}

size_t sq_ctx_seq_len(const sq_ctx* c) { return c ? c->seq_len : 0; }

int sq_device_wall_clock_khz(int* khz) {
    if (!khz) return set_error(SQ_ERR_ARG, "wall_clock_khz: null argument");
    int dev = 0;
    SQ_HIP_CHECK(hipGetDevice(&dev));
    SQ_HIP_CHECK(hipDeviceGetAttribute(khz, hipDeviceAttributeWallClockRate, dev));
    return 0;
}

int sq_ctx_prefill_phases(sq_ctx* c, const uint32_t* ids, size_t n, double* ms) {
    if (!c || !ids || !ms) return set_error(SQ_ERR_ARG, "prefill_phases: null argument");
    if (n > c->max_pos) return set_error(SQ_ERR_CACHE_FULL, "prefill_phases: prompt longer than the context");
    return ctx_prefill_phases(c, ids, n, ms);
}

int sq_ctx_score(sq_ctx* c, const uint32_t* ids, size_t n, size_t burn, double* logp) {
    if (!c) return set_error(SQ_ERR_ARG, "score: null context");
    return ctx_score(c, ids, n, burn, logp);
}

int sq_gemm_counters(int reset, uint64_t* out) {
    gemm_counters(reset != 0, out);
    return 0;
}

int sq_ctx_act_taps(sq_ctx* c, int enable) {
    if (!c) return set_error(SQ_ERR_ARG, "act_taps: null context");
    return ctx_set_taps(c, enable != 0);
}

int sq_ctx_act_tap_read(sq_ctx* c, void* blocks, size_t n_blocks) {
    if (!c || !blocks) return set_error(SQ_ERR_ARG, "act_tap_read: null argument");
    return ctx_read_taps(c, blocks, n_blocks);
}

int sq_forward(const sq_model* m, sq_ctx* c, const uint32_t* ids, size_t n) {
    if (!m || !c || c->m != m) return set_error(SQ_ERR_ARG, "forward: context does not belong to this model");
    return ctx_forward(c, ids, n);
}

int sq_logits(sq_ctx* c, float* out, size_t n) {
    if (!c || !out || n < (size_t)c->m->cfg.vocab) return set_error(SQ_ERR_ARG, "logits: buffer too small");
    SQ_HIP_CHECK(hipStreamSynchronize(c->stream));
    if (int st = ctx_check(c)) return st;
    SQ_HIP_CHECK(hipMemcpy(out, c->logits, (size_t)c->m->cfg.vocab * 4, hipMemcpyDeviceToHost));
    return 0;
}

int sq_argmax(sq_ctx* c, uint32_t* token) {
    if (!c || !token) return set_error(SQ_ERR_ARG, "argmax: null argument");
    SQ_HIP_CHECK(hipStreamSynchronize(c->stream));
    if (int st = ctx_check(c)) return st;
    SQ_HIP_CHECK(hipMemcpy(token, c->d_token, 4, hipMemcpyDeviceToHost));
    return 0;
}

int sq_ctx_last_hidden(sq_ctx* c, float* out, size_t n) {
    if (!c || !out || n < (size_t)c->m->cfg.dim) return set_error(SQ_ERR_ARG, "last_hidden: buffer too small");
    SQ_HIP_CHECK(hipStreamSynchronize(c->stream));
    if (int st = ctx_check(c)) return st;
    SQ_HIP_CHECK(hipMemcpy(out, c->last_hidden, (size_t)c->m->cfg.dim * 4, hipMemcpyDeviceToHost));
    return 0;
}

int sq_ctx_debug_act(sq_ctx* c, float* normed, void* blocks) {
    if (!c) return set_error(SQ_ERR_ARG, "debug_act: null context");
    const size_t D = c->m->cfg.dim;
    SQ_HIP_CHECK(hipStreamSynchronize(c->stream));
    if (int st = ctx_check(c)) return st;
    if (normed) SQ_HIP_CHECK(hipMemcpy(normed, c->dbg_normed, D * 4, hipMemcpyDeviceToHost));
    if (blocks) {
        std::vector<int8_t> qs(D);
        std::vector<uint16_t> d(D / 32);
        SQ_HIP_CHECK(hipMemcpy(qs.data(), c->tap_q, D, hipMemcpyDeviceToHost));
        SQ_HIP_CHECK(hipMemcpy(d.data(), c->tap_d, D / 32 * 2, hipMemcpyDeviceToHost));
        uint8_t* o = (uint8_t*)blocks;
        for (size_t b = 0; b < D / 32; b++) {
            memcpy(o + b * 34, &d[b], 2);
            memcpy(o + b * 34 + 2, &qs[b * 32], 32);
        }
    }
    return 0;
}

int sq_generate(const sq_model* m, sq_ctx* c, const uint32_t* prompt, size_t n_prompt, size_t max_tokens,
                uint32_t flags, uint32_t* out_tokens, size_t* n_out, double* step_ms) {
    if (!m || !c || c->m != m || !n_out || (max_tokens && !out_tokens))
        return set_error(SQ_ERR_ARG, "generate: bad argument");
    int st = ctx_generate(c, prompt, n_prompt, max_tokens, flags, out_tokens, n_out, step_ms);
    if (st) return st;
    return ctx_check(c);
}

int sq_ctx_time_kernel(sq_ctx* c, int which, int iters, double* mean_us, uint64_t* bytes) {
    if (!c || !mean_us) return set_error(SQ_ERR_ARG, "time_kernel: null argument");
    if (c->seq_len == 0 || c->seq_len >= c->max_pos)
        return set_error(SQ_ERR_ARG, "time_kernel: needs a context with 1 <= positions < max_positions");
    return ctx_time_kernel(c, which, iters, mean_us, bytes);
}

// ------------------------------------------------------------ operator level

int sq_weight_upload(int wtype, const void* blocks, size_t rows, size_t k, sq_weight** out) {
    if (!blocks || !out) return set_error(SQ_ERR_ARG, "weight_upload: null argument");
    if (wtype != SQ_Q8_0 && wtype != SQ_Q4_0 && wtype != SQ_BF16)
        return set_error(SQ_ERR_INVALID_TYPE, "weight_upload: InvalidType");
    if (k == 0 || k % 32) return set_error(SQ_ERR_SHAPE, "weight_upload: k must be a multiple of 32");
    sq_weight* w = new sq_weight();
    int st = upload_matrix(wtype, (const uint8_t*)blocks, rows, k, &w->m);
    if (st) {
        free_matrix(&w->m);
        delete w;
        return st;
    }
    *out = w;
    return 0;
}

void sq_weight_free(sq_weight* w) {
    if (!w) return;
    free_matrix(&w->m);
    delete w;
}

int sq_quantize_row_q8_0(const float* d_x, size_t n, void* d_blocks) {
    if (n % 32) return set_error(SQ_ERR_SHAPE, "quantize: length must be a multiple of 32");
    if (n == 0) return 0;
    Tmp qs, d;
    int st;
    if ((st = qs.alloc(n)) || (st = d.alloc(n / 16))) return st;
    if ((st = launch_quantize_rows(nullptr, d_x, n, (int8_t*)qs.p, (uint16_t*)d.p))) return st;
    st = launch_pack_q8_blocks(nullptr, (int8_t*)qs.p, (uint16_t*)d.p, n / 32, d_blocks);
    return finish(st);
}

namespace {

int linear_impl(const float* d_in, size_t m, size_t k, const sq_weight* w, float* d_out, uint32_t flags,
                const int8_t* pre_q, const uint16_t* pre_d) {
    if (!w || !d_in || !d_out) return set_error(SQ_ERR_ARG, "linear: null argument");
    if (k != (size_t)w->m.k) return set_error(SQ_ERR_SHAPE, "linear: ShapeMismatch (in_dim != weight k)");
    if (m == 0) return 0;
    const bool a8 = w->m.wtype != WT_BF16 && !(flags & SQ_CTX_F32_ACTS);
    if (!a8) return set_error(SQ_ERR_UNSUPPORTED, kA32Disabled);
    Tmp tq, td;
    int st;
    const int8_t* aq = pre_q;
    const uint16_t* ad = pre_d;
    if (a8 && !aq) {
        if ((st = tq.alloc(m * k)) || (st = td.alloc(m * k / 16))) return st;
        if ((st = launch_quantize_rows(nullptr, d_in, m * k, (int8_t*)tq.p, (uint16_t*)td.p))) return st;
        aq = (const int8_t*)tq.p;
        ad = (const uint16_t*)td.p;
    }
    if (m == 1 && (k / 32 <= 256)) {
        GemvArgs a{};
        a.w = view(w->m);
        a.n_rows = w->m.rows;
        a.aq = aq;
        a.ad = ad;
        a.x = d_in;
        a.out = d_out;
        st = launch_gemv(nullptr, a8 ? PRO_Q8 : PRO_F32, EPI_STORE, a8, a, nullptr);
    } else {
        Tmp ws;  // partial tiles of a K split
        if ((st = ws.alloc(kGemmSplitFloats * sizeof(float)))) return st;
        st = launch_gemm(nullptr, view(w->m), w->m.wtype, a8, aq, ad, d_in, (int)m, d_out, w->m.rows, false,
                         (float*)ws.p, kGemmSplitFloats);
        if (!st) st = finish(st);  // the workspace is freed on return
    }
    return finish(st);
}

}  // namespace

int sq_linear(const float* d_in, size_t m, size_t k, const sq_weight* w, float* d_out, uint32_t flags) {
    return linear_impl(d_in, m, k, w, d_out, flags, nullptr, nullptr);
}

int sq_linear_shared(const float* d_in, size_t m, size_t k, const sq_weight* const* ws, float* const* d_outs,
                     size_t n_weights, uint32_t flags) {
    if (n_weights == 0 || !ws || !d_outs) return set_error(SQ_ERR_SHAPE, "linear_shared: ShapeMismatch (no weights)");
    const int wt = ws[0]->m.wtype;
    for (size_t i = 0; i < n_weights; i++) {
        if (!ws[i]) return set_error(SQ_ERR_ARG, "linear_shared: null weight");
        if ((size_t)ws[i]->m.k != k) return set_error(SQ_ERR_SHAPE, "linear_shared: ShapeMismatch");
        if (ws[i]->m.wtype != wt) return set_error(SQ_ERR_INVALID_TYPE, "linear_shared: InvalidType (mixed types)");
    }
    const bool a8 = wt != WT_BF16 && !(flags & SQ_CTX_F32_ACTS);
    if (!a8) return set_error(SQ_ERR_UNSUPPORTED, kA32Disabled);
    Tmp tq, td;
    int st;
    if (a8 && m) {
        // One quantization shared by every projection (linear.rs:117-127).
        if ((st = tq.alloc(m * k)) || (st = td.alloc(m * k / 16))) return st;
        if ((st = launch_quantize_rows(nullptr, d_in, m * k, (int8_t*)tq.p, (uint16_t*)td.p))) return st;
    }
    for (size_t i = 0; i < n_weights; i++)
        if ((st = linear_impl(d_in, m, k, ws[i], d_outs[i], flags, (const int8_t*)tq.p, (const uint16_t*)td.p)))
            return st;
    return 0;
}

int sq_block_isums(const void* d_act_blocks, const sq_weight* w, size_t row, int32_t* d_isums) {
    if (!w || !d_act_blocks || !d_isums) return set_error(SQ_ERR_ARG, "block_isums: null argument");
    if (w->m.wtype == WT_BF16) return set_error(SQ_ERR_INVALID_TYPE, "block_isums: BF16 has no integer path");
    if (row >= (size_t)w->m.rows) return set_error(SQ_ERR_SHAPE, "block_isums: row out of range");
    const size_t kb = w->m.k / 32;
    Tmp qs, d;
    int st;
    if ((st = qs.alloc(kb * 32)) || (st = d.alloc(kb * 2))) return st;
    if ((st = launch_unpack_q8_blocks(nullptr, d_act_blocks, kb, (int8_t*)qs.p, (uint16_t*)d.p))) return st;
    return finish(launch_block_isums(nullptr, (const int8_t*)qs.p, view(w->m), w->m.wtype, (int)row, d_isums));
}

int sq_embed(const uint32_t* d_tokens, size_t n, const sq_weight* table, float* d_out) {
    if (!table) return set_error(SQ_ERR_ARG, "embed: null table");
    if (table->m.wtype == WT_BF16) return set_error(SQ_ERR_UNSUPPORTED, kA32Disabled);
    if (n == 0) return 0;
    Tmp err;
    int st;
    if ((st = err.alloc(4))) return st;
    SQ_HIP_CHECK(hipMemsetAsync(err.p, 0, 4, nullptr));
    if ((st = finish(launch_embed(nullptr, view(table->m), table->m.wtype, d_tokens, (int)n, table->m.k, d_out,
                                  (uint32_t*)err.p))))
        return st;
    uint32_t bad = 0;
    SQ_HIP_CHECK(hipMemcpy(&bad, err.p, 4, hipMemcpyDeviceToHost));
    if (bad) return set_error(SQ_ERR_ARG, "embed: a token id is past the embedding table (embedding.rs:43-44)");
    return 0;
}

int sq_rms_norm(const float* d_in, const float* d_w, float* d_out, size_t rows, size_t dim, float eps) {
    if (dim == 0) return set_error(SQ_ERR_SHAPE, "rms_norm: ShapeMismatch (empty last dim)");
    if (rows == 0) return 0;
    return finish(launch_rmsnorm_rows(nullptr, d_in, d_w, (int)rows, (int)dim, eps, d_out, nullptr, nullptr));
}

int sq_rope_rows(float* d_t, size_t rows, size_t row_dim, size_t base_pos, const float* inv_freq, size_t half) {
    const size_t head_dim = 2 * half;
    if (head_dim == 0 || row_dim == 0 || row_dim % head_dim)
        return set_error(SQ_ERR_SHAPE, "rope_rows: ShapeMismatch");
    if (rows == 0) return 0;
    // (cos, sin) of f32(pos) * inv_freq[j] with the host libm, as the
    // reference computes them (src/kernels/rope.rs:24-26).
    std::vector<float2> cs(rows * half);
    for (size_t r = 0; r < rows; r++)
        for (size_t j = 0; j < half; j++) {
            volatile float th = (float)(base_pos + r) * inv_freq[j];
            cs[r * half + j] = make_float2(cosf(th), sinf(th));
        }
    Tmp d;
    int st;
    if ((st = d.alloc(cs.size() * sizeof(float2)))) return st;
    SQ_HIP_CHECK(hipMemcpy(d.p, cs.data(), cs.size() * sizeof(float2), hipMemcpyHostToDevice));
    return finish(launch_rope_rows_table(nullptr, d_t, (int)rows, (int)row_dim, (int)head_dim, (const float2*)d.p));
}

int sq_sdpa(const float* d_q, const float* d_k, const float* d_v, float* d_out, size_t seq_q, size_t seq_k,
            size_t n_heads, size_t n_kv_heads, size_t head_dim) {
    if (n_kv_heads == 0 || head_dim == 0 || n_heads % n_kv_heads) return set_error(SQ_ERR_SHAPE, "sdpa: ShapeMismatch");
    if (seq_k < seq_q) return set_error(SQ_ERR_SHAPE, "sdpa: ShapeMismatch (seq_k < seq_q)");
    if (seq_q == 0) return 0;
    const size_t G = n_heads / n_kv_heads;
    const bool model_kernels = head_dim == 64 && (G == 1 || G == 2 || G == 4 || G == 8);
    int st;
    if (model_kernels && seq_q == 1) {
        // The decode kernel: the query sits at position seq_k - 1.
        const int tiles = (int)((seq_k + 63) / 64);
        Tmp pos, pm, pl, po, cnt, aq, ad;
        const int p = (int)seq_k - 1;
        if ((st = pos.alloc(4)) || (st = pm.alloc(n_heads * tiles * 4)) || (st = pl.alloc(n_heads * tiles * 4)) ||
            (st = po.alloc(n_heads * tiles * 64 * 4)) || (st = cnt.alloc(n_kv_heads * 4)))
            return st;
        SQ_HIP_CHECK(hipMemcpy(pos.p, &p, 4, hipMemcpyHostToDevice));
        SQ_HIP_CHECK(hipMemset(cnt.p, 0, n_kv_heads * 4));
        return finish(launch_attn_decode(nullptr, d_q, d_k, d_v, (const int*)pos.p, (int)n_heads, (int)n_kv_heads, 64,
                                         tiles, (float*)pm.p, (float*)pl.p, (float*)po.p, (unsigned*)cnt.p, d_out,
                                         nullptr, nullptr));
    }
    if (model_kernels) {
        Tmp kvs;
        if ((st = kvs.alloc(attn_split_words((int)seq_k, (int)n_kv_heads) * 4))) return st;
        return finish(launch_attn_prefill(nullptr, d_q, d_k, d_v, (int)(seq_k - seq_q), (int)seq_q, (int)n_heads,
                                          (int)n_kv_heads, 64, (uint32_t*)kvs.p, (int)seq_k, d_out));
    }
    return finish(launch_sdpa_generic(nullptr, d_q, d_k, d_v, d_out, (int)seq_q, (int)seq_k, (int)n_heads,
                                      (int)n_kv_heads, (int)head_dim));
}

int sq_silu(float* d_x, size_t n) {
    if (n == 0) return 0;
    return finish(launch_silu(nullptr, d_x, n));
}

int sq_elementwise_mul(const float* d_a, const float* d_b, float* d_out, size_t n) {
    if (n == 0) return 0;
    return finish(launch_mul(nullptr, d_a, d_b, d_out, n));
}

int sq_elementwise_add(float* d_a, const float* d_b, size_t n) {
    if (n == 0) return 0;
    return finish(launch_add_inplace(nullptr, d_a, d_b, n));
}

int sq_softmax(const float* d_in, float* d_out, size_t n) {
    if (n == 0) return set_error(SQ_ERR_EMPTY, "softmax: EmptyInput");
    return finish(launch_softmax_row(nullptr, d_in, d_out, (int)n));
}

int sq_log_softmax_at(const float* d_logits, size_t n, uint32_t idx, double* out) {
    if (!d_logits || !out) return set_error(SQ_ERR_ARG, "log_softmax_at: null argument");
    if (n == 0) return set_error(SQ_ERR_EMPTY, "log_softmax_at: EmptyInput");
    if (idx >= n) return set_error(SQ_ERR_ARG, "log_softmax_at: index out of range");
    if (n > (size_t)INT32_MAX) return set_error(SQ_ERR_SHAPE, "log_softmax_at: row too long");
    Tmp id, val, err;
    int st;
    if ((st = id.alloc(4)) || (st = val.alloc(8)) || (st = err.alloc(4))) return st;
    SQ_HIP_CHECK(hipMemcpy(id.p, &idx, 4, hipMemcpyHostToDevice));
    SQ_HIP_CHECK(hipMemsetAsync(err.p, 0, 4, nullptr));
    if ((st = launch_log_softmax_at(nullptr, d_logits, (int)n, (const uint32_t*)id.p, (double*)val.p,
                                    (uint32_t*)err.p)))
        return st;
    if ((st = finish(0))) return st;
    SQ_HIP_CHECK(hipMemcpy(out, val.p, 8, hipMemcpyDeviceToHost));
    return 0;
}

int sq_greedy(const float* d_logits, size_t n, uint32_t* token) {
    if (n == 0 || !token) return set_error(SQ_ERR_EMPTY, "greedy: empty logits");
    const int parts = (int)std::min<size_t>(256, (n + 1023) / 1024);
    Tmp pv, pi, pn, tok;
    int st;
    if ((st = pv.alloc(parts * 4)) || (st = pi.alloc(parts * 4)) || (st = pn.alloc(parts * 4)) || (st = tok.alloc(4)))
        return st;
    if ((st = launch_argmax_partials(nullptr, d_logits, (int)n, (float*)pv.p, (int*)pi.p, (int*)pn.p, parts))) return st;
    if ((st = launch_argmax_final(nullptr, d_logits, (int)n, (float*)pv.p, (int*)pi.p, (int*)pn.p, parts,
                                  (uint32_t*)tok.p, nullptr, 0, nullptr, nullptr)))
        return st;
    if ((st = finish(0))) return st;
    SQ_HIP_CHECK(hipMemcpy(token, tok.p, 4, hipMemcpyDeviceToHost));
    return 0;
}

}  // extern "C"
