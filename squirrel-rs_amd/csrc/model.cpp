// Model load, inference context and the forward pass orchestration.
//
// Decode (one token): 6 launches per layer plus embed / LM head / argmax, all
// captured once into a hipGraph.  Every launch reads the position and the
// input token from device memory, so one graph serves every step and a step
// needs no host round trip.
//
//   embed(token)                                        model.rs:57-62
//   per layer (layers.rs:81-109):
//     QKV matvec   <- RMSNorm+quantize prologue          layers.rs:89-94, 33-38
//                  -> RoPE(q, k), K/V into the cache     layers.rs:42-46
//     attention split + combine(+quantize)               layers.rs:47-55
//     o matvec     -> hidden += ...                      layers.rs:57, 96
//     gate/up      <- RMSNorm+quantize prologue          layers.rs:99-104, 66-71
//                  -> silu(gate)*up (+quantize)          layers.rs:73-74
//     down matvec  -> hidden += ...                      layers.rs:76, 106
//   LM head        <- final RMSNorm+quantize prologue    model.rs:72-95
//                  -> logits + argmax partials
//   argmax final   -> token, position += 1               greedy.rs:6-15
//
// Prefill (n tokens): the same math over n rows with multi-row matmuls and a
// tiled causal attention; only the last row feeds the LM head.
#include "model.h"

#include <algorithm>
#include <chrono>
#include <memory>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <thread>

namespace sq {

namespace {

struct MetaErr {
    int code;
};

const GGUFValue* find_meta(const GGUFFile& f, const char* key) {
    auto it = f.meta.find(key);
    return it == f.meta.end() ? nullptr : &it->second;
}

// read_u32 / read_f32 (config.rs:129-149).
int read_u32(const GGUFFile& f, const char* key, uint32_t* out) {
    const GGUFValue* v = find_meta(f, key);
    if (!v) return set_error(SQ_ERR_CONFIG, std::string("MissingMetadata(") + key + ")");
    if (v->type != GT_U32) return set_error(SQ_ERR_CONFIG, std::string("WrongMetadataType(") + key + ", u32)");
    *out = (uint32_t)v->u;
    return 0;
}

int read_f32(const GGUFFile& f, const char* key, float* out) {
    const GGUFValue* v = find_meta(f, key);
    if (!v) return set_error(SQ_ERR_CONFIG, std::string("MissingMetadata(") + key + ")");
    if (v->type != GT_F32) return set_error(SQ_ERR_CONFIG, std::string("WrongMetadataType(") + key + ", f32)");
    *out = v->f32;
    return 0;
}

bool opt_u32(const GGUFFile& f, const char* key, uint32_t* out) {
    const GGUFValue* v = find_meta(f, key);
    if (!v || v->type != GT_U32) return false;
    *out = (uint32_t)v->u;
    return true;
}

bool opt_f32(const GGUFFile& f, const char* key, float* out) {
    const GGUFValue* v = find_meta(f, key);
    if (!v || v->type != GT_F32) return false;
    *out = v->f32;
    return true;
}

size_t row_payload_bytes(int wtype, size_t k) {
    if (wtype == WT_Q8_0) return k;
    if (wtype == WT_Q4_0) return k / 2;
    return k * 2;
}

size_t gguf_row_bytes(int wtype, size_t k) {
    if (wtype == WT_Q8_0) return (k / 32) * 34;
    if (wtype == WT_Q4_0) return (k / 32) * 18;
    return k * 2;
}

template <typename T>
int dmalloc(T** p, size_t count) {
    if (count == 0) count = 1;
    hipError_t e = hipMalloc((void**)p, count * sizeof(T));
    if (e != hipSuccess)
        return set_error(SQ_ERR_HIP, "hipMalloc(" + std::to_string(count * sizeof(T)) + "): " + hipGetErrorString(e));
    return 0;
}

template <typename T>
void dfree(T*& p) {
    if (p) (void)hipFree((void*)p);
    p = nullptr;
}

}  // namespace

size_t DevMatrix::payload_bytes() const { return (size_t)rows * row_payload_bytes(wtype, (size_t)k); }
size_t DevMatrix::scale_bytes() const { return wtype == WT_BF16 ? 0 : (size_t)rows * (k / 32) * 2; }

// compute_rope_inv_freq (src/models/llama/config.rs:83-127).  Compiled without
// FMA contraction so every product and sum rounds as the reference's does.
#pragma STDC FP_CONTRACT OFF
void rope_inv_freq(int head_dim, float base, float factor, float low, float high, float orig_ctx,
                   float* out) {
    const int half = head_dim / 2;
    const float inv_head_dim = 1.0f / (float)head_dim;
    for (int j = 0; j < half; j++) {
        volatile float e = -2.0f * (float)j;
        e = e * inv_head_dim;
        out[j] = powf(base, e);
    }
    const float two_pi = 6.28318530717958647692f;
    const float low_wl = orig_ctx / low;
    const float high_wl = orig_ctx / high;
    for (int j = 0; j < half; j++) {
        const float f = out[j];
        const float wavelen = two_pi / f;
        if (wavelen > low_wl) {
            out[j] = f / factor;
        } else if (wavelen >= high_wl) {
            volatile float smooth = (orig_ctx / wavelen - low) / (high - low);
            volatile float a = (1.0f - smooth) * (f / factor);
            volatile float b = smooth * f;
            out[j] = a + b;
        }
    }
}

int read_config(const GGUFFile& f, Config* c) {
    uint32_t u;
    int st;
    if ((st = read_u32(f, "llama.block_count", &u))) return st;
    c->n_layers = (int)u;
    if ((st = read_u32(f, "llama.embedding_length", &u))) return st;
    c->dim = (int)u;
    if ((st = read_u32(f, "llama.feed_forward_length", &u))) return st;
    c->ffn = (int)u;
    if ((st = read_u32(f, "llama.attention.head_count", &u))) return st;
    c->n_heads = (int)u;
    if ((st = read_u32(f, "llama.attention.head_count_kv", &u))) return st;
    c->n_kv_heads = (int)u;
    if (c->n_heads == 0) return set_error(SQ_ERR_CONFIG, "llama.attention.head_count is 0");
    c->head_dim = opt_u32(f, "llama.rope.dimension_count", &u) ? (int)u : c->dim / c->n_heads;
    if ((st = read_f32(f, "llama.rope.freq_base", &c->rope_base))) return st;
    if ((st = read_f32(f, "llama.attention.layer_norm_rms_epsilon", &c->eps))) return st;
    if ((st = read_u32(f, "llama.context_length", &u))) return st;
    c->context_length = (int)u;
    if ((st = read_u32(f, "tokenizer.ggml.bos_token_id", &c->bos))) return st;
    if ((st = read_u32(f, "tokenizer.ggml.eos_token_id", &c->eos))) return st;
    if (opt_u32(f, "llama.vocab_size", &u)) {
        c->vocab = (int)u;
    } else {
        const GGUFValue* t = find_meta(f, "tokenizer.ggml.tokens");
        if (!t || t->type != GT_ARRAY)
            return set_error(SQ_ERR_CONFIG, "MissingMetadata(llama.vocab_size / tokenizer.ggml.tokens)");
        c->vocab = (int)t->arr.size();
    }
    float factor = 32.0f, low = 1.0f, high = 4.0f;
    opt_f32(f, "llama.rope.scaling.factor", &factor);
    opt_f32(f, "llama.rope.scaling.low_freq_factor", &low);
    opt_f32(f, "llama.rope.scaling.high_freq_factor", &high);
    float orig = 8192.0f;
    if (opt_u32(f, "llama.rope.scaling.original_context_length", &u)) orig = (float)u;
    c->inv_freq.assign(c->head_dim / 2, 0.0f);
    rope_inv_freq(c->head_dim, c->rope_base, factor, low, high, orig, c->inv_freq.data());
    return 0;
}

int upload_stacked(int wtype, const std::vector<const uint8_t*>& parts, const std::vector<size_t>& rows,
                   size_t k, DevMatrix* out) {
    size_t total = 0;
    for (size_t r : rows) total += r;
    out->wtype = wtype;
    out->rows = (int)total;
    out->k = (int)k;
    const size_t kb = k / 32;
    const size_t pay = row_payload_bytes(wtype, k);
    std::vector<uint8_t> h_qs(total * pay);
    std::vector<uint16_t> h_sc(wtype == WT_BF16 ? 0 : total * kb);
    size_t r0 = 0;
    for (size_t p = 0; p < parts.size(); p++) {
        const uint8_t* src = parts[p];
        const size_t grb = gguf_row_bytes(wtype, k);
        for (size_t r = 0; r < rows[p]; r++) {
            const uint8_t* row = src + r * grb;
            uint8_t* dq = h_qs.data() + (r0 + r) * pay;
            if (wtype == WT_BF16) {
                memcpy(dq, row, pay);
                continue;
            }
            const size_t bb = wtype == WT_Q8_0 ? 34 : 18, pb = bb - 2;
            for (size_t b = 0; b < kb; b++) {
                const uint8_t* blk = row + b * bb;
                memcpy(&h_sc[(r0 + r) * kb + b], blk, 2);
                memcpy(dq + b * pb, blk + 2, pb);
            }
        }
        r0 += rows[p];
    }
    int st;
    if ((st = dmalloc((uint8_t**)&out->qs, h_qs.size()))) return st;
    SQ_HIP_CHECK(hipMemcpy(out->qs, h_qs.data(), h_qs.size(), hipMemcpyHostToDevice));
    if (!h_sc.empty()) {
        if ((st = dmalloc(&out->scale, h_sc.size()))) return st;
        SQ_HIP_CHECK(hipMemcpy(out->scale, h_sc.data(), h_sc.size() * 2, hipMemcpyHostToDevice));
    }
    return 0;
}

int upload_matrix(int wtype, const uint8_t* blocks, size_t rows, size_t k, DevMatrix* out) {
    return upload_stacked(wtype, {blocks}, {rows}, k, out);
}

void free_matrix(DevMatrix* m) {
    if (m->qs) (void)hipFree(m->qs);
    if (m->scale) (void)hipFree(m->scale);
    m->qs = nullptr;
    m->scale = nullptr;
}

// ---------------------------------------------------------------- model load

namespace {

// A tensor of the expected GGML dims ([k, n] for matrices, [n] for norms).
int get_tensor(const GGUFFile& f, const std::string& name, const std::vector<uint64_t>& dims,
               const uint8_t** data, uint32_t* type) {
    int st;
    *data = f.tensor_data(name, &st);
    if (!*data) return st;
    const GGUFTensorInfo& ti = f.tensors.at(name);
    if (ti.dims != dims) {
        std::string got, want;
        for (auto d : ti.dims) got += std::to_string(d) + ",";
        for (auto d : dims) want += std::to_string(d) + ",";
        return set_error(SQ_ERR_SHAPE, "tensor " + name + " has dims [" + got + "] expected [" + want + "]");
    }
    *type = ti.ggml_type;
    return 0;
}

}  // namespace

int model_load_impl(const char* path, sq_model** out, bool upload) {
    GGUFFile f;
    int st = f.open(path);
    if (st) return st;
    sq_model* m = new sq_model();
    Config& c = m->cfg;
    if ((st = read_config(f, &c))) {
        delete m;
        return st;
    }
    if (c.n_kv_heads == 0 || c.n_heads % c.n_kv_heads != 0) {
        delete m;
        return set_error(SQ_ERR_CONFIG, "n_heads must be a multiple of n_kv_heads");
    }
    const int G = c.n_heads / c.n_kv_heads;
    if (c.head_dim != 64 || c.dim % 32 || c.ffn % 32 || c.dim > 2048 || c.ffn > 8192 ||
        (G != 1 && G != 2 && G != 4 && G != 8) || c.n_heads * c.head_dim > 2048) {
        delete m;
        return set_error(SQ_ERR_UNSUPPORTED,
                         "shape outside the built kernels (head_dim 64, dim <= 2048, ffn <= 8192, GQA 1/2/4/8)");
    }
    if (hipGetDevice(&m->device) != hipSuccess) m->device = 0;
    const uint64_t D = c.dim, F = c.ffn, QD = (uint64_t)c.n_heads * c.head_dim,
                   KVD = (uint64_t)c.n_kv_heads * c.head_dim, V = c.vocab;
    auto fail = [&](int code) {
        model_free(m);
        return code;
    };
    // Pass 1: resolve and check every tensor (LlamaWeights::from_gguf,
    // weights.rs:50-97) before any device allocation.
    int wtype = -1;
    auto norm = [&](const std::string& name, const uint8_t** p) -> int {
        uint32_t t;
        int s = get_tensor(f, name, {D}, p, &t);
        if (s) return s;
        if (t != WT_F32) return set_error(SQ_ERR_INVALID_TYPE, "norm " + name + " must be F32");
        return 0;
    };
    auto mat = [&](const std::string& name, uint64_t k, uint64_t n, const uint8_t** p) -> int {
        uint32_t t;
        int s = get_tensor(f, name, {k, n}, p, &t);
        if (s) return s;
        if (t != WT_Q8_0 && t != WT_Q4_0 && t != WT_BF16)
            return set_error(SQ_ERR_INVALID_TYPE, "matrix " + name + " has unsupported type " + std::to_string(t));
        if (wtype < 0) wtype = (int)t;
        if ((int)t != wtype) return set_error(SQ_ERR_UNSUPPORTED, "mixed matrix types are not supported: " + name);
        return 0;
    };
    struct LayerSrc {
        const uint8_t *an, *wq, *wk, *wv, *wo, *fn, *wg, *wu, *wd;
    };
    std::vector<LayerSrc> src(c.n_layers);
    for (int i = 0; i < c.n_layers; i++) {
        LayerSrc& S = src[i];
        const std::string pre = "blk." + std::to_string(i) + ".";
        if ((st = norm(pre + "attn_norm.weight", &S.an)) || (st = mat(pre + "attn_q.weight", D, QD, &S.wq)) ||
            (st = mat(pre + "attn_k.weight", D, KVD, &S.wk)) || (st = mat(pre + "attn_v.weight", D, KVD, &S.wv)) ||
            (st = mat(pre + "attn_output.weight", QD, D, &S.wo)) || (st = norm(pre + "ffn_norm.weight", &S.fn)) ||
            (st = mat(pre + "ffn_gate.weight", D, F, &S.wg)) || (st = mat(pre + "ffn_up.weight", D, F, &S.wu)) ||
            (st = mat(pre + "ffn_down.weight", F, D, &S.wd)))
            return fail(st);
    }
    const uint8_t *we, *wn, *wout = nullptr;
    if ((st = mat("token_embd.weight", D, V, &we)) || (st = norm("output_norm.weight", &wn))) return fail(st);
    // Tied LM head when output.weight is absent (weights.rs:87-89).
    const bool tied = f.tensors.count("output.weight") == 0;
    if (!tied && (st = mat("output.weight", D, V, &wout))) return fail(st);

    m->wtype = wtype;
    m->tied = tied;
    if (!upload) {
        for (int i = 0; i < c.n_layers; i++) {
            const uint64_t mats[4] = {(QD + 2 * KVD) * D, QD * D, 2 * F * D, D * F};
            for (uint64_t e : mats)
                m->weight_bytes += wtype == WT_BF16 ? 2 * e : e + e / 16 - (wtype == WT_Q4_0 ? e / 2 : 0);
        }
        m->weight_bytes += wtype == WT_BF16 ? 2 * V * D : V * D + V * D / 16 - (wtype == WT_Q4_0 ? V * D / 2 : 0);
        *out = m;
        return 0;
    }
    if (wtype == WT_BF16) return fail(set_error(SQ_ERR_UNSUPPORTED, kA32Disabled));

    // Pass 2: upload.
    auto up_norm = [&](const uint8_t* p, float** dst) -> int {
        int s;
        if ((s = dmalloc(dst, D))) return s;
        SQ_HIP_CHECK(hipMemcpy(*dst, p, D * 4, hipMemcpyHostToDevice));
        return 0;
    };
    m->layers.resize(c.n_layers);
    for (int i = 0; i < c.n_layers; i++) {
        Layer& L = m->layers[i];
        const LayerSrc& S = src[i];
        if ((st = up_norm(S.an, &L.attn_norm)) || (st = up_norm(S.fn, &L.ffn_norm)) ||
            (st = upload_stacked(wtype, {S.wq, S.wk, S.wv}, {QD, KVD, KVD}, D, &L.qkv)) ||
            (st = upload_matrix(wtype, S.wo, D, QD, &L.o)) ||
            (st = upload_stacked(wtype, {S.wg, S.wu}, {F, F}, D, &L.gateup)) ||
            (st = upload_matrix(wtype, S.wd, D, F, &L.down)))
            return fail(st);
        m->weight_bytes += L.qkv.payload_bytes() + L.qkv.scale_bytes() + L.o.payload_bytes() +
                           L.o.scale_bytes() + L.gateup.payload_bytes() + L.gateup.scale_bytes() +
                           L.down.payload_bytes() + L.down.scale_bytes();
    }
    if ((st = upload_matrix(wtype, we, V, D, &m->embd)) || (st = up_norm(wn, &m->out_norm))) return fail(st);
    if (tied) {
        m->head = m->embd;
    } else if ((st = upload_matrix(wtype, wout, V, D, &m->head))) {
        return fail(st);
    }
    m->tied = tied;
    m->weight_bytes += m->head.payload_bytes() + m->head.scale_bytes();
    m->wtype = wtype;
    *out = m;
    return 0;
}

int model_load(const char* path, sq_model** out) { return model_load_impl(path, out, true); }
int model_inspect(const char* path, sq_model** out) { return model_load_impl(path, out, false); }

void model_free(sq_model* m) {
    if (!m) return;
    for (Layer& L : m->layers) {
        if (L.attn_norm) (void)hipFree(L.attn_norm);
        if (L.ffn_norm) (void)hipFree(L.ffn_norm);
        free_matrix(&L.qkv);
        free_matrix(&L.o);
        free_matrix(&L.gateup);
        free_matrix(&L.down);
    }
    if (!m->tied) free_matrix(&m->head);
    free_matrix(&m->embd);
    if (m->out_norm) (void)hipFree(m->out_norm);
    delete m;
}

// ---------------------------------------------------------------- context

namespace {

int build_decode_step(sq_ctx* c);

int ensure_prefill(sq_ctx* c, size_t n) {
    if (n <= c->cap_rows) return 0;
    const Config& g = c->m->cfg;
    const size_t D = g.dim, F = g.ffn, QD = (size_t)g.n_heads * g.head_dim, KVD = (size_t)g.n_kv_heads * g.head_dim;
    dfree(c->p_hidden); dfree(c->p_normed); dfree(c->p_qkv); dfree(c->p_q); dfree(c->p_attn);
    dfree(c->p_gu); dfree(c->p_act); dfree(c->p_aq); dfree(c->p_ad);
    int st;
    const size_t wmax = std::max(std::max(D, F), QD);
    if ((st = dmalloc(&c->p_hidden, n * D)) || (st = dmalloc(&c->p_normed, n * D)) ||
        (st = dmalloc(&c->p_qkv, n * (QD + 2 * KVD))) || (st = dmalloc(&c->p_q, n * QD)) ||
        (st = dmalloc(&c->p_attn, n * QD)) || (st = dmalloc(&c->p_gu, n * 2 * F)) ||
        (st = dmalloc(&c->p_act, n * F)) || (st = dmalloc(&c->p_aq, n * wmax)) ||
        (st = dmalloc(&c->p_ad, n * wmax / 32)))
        return st;
    if (!c->p_split && (st = dmalloc(&c->p_split, kPrefillSplitFloats))) return st;
    if (!c->p_kvs && (st = dmalloc(&c->p_kvs, attn_split_words((int)c->max_pos, g.n_kv_heads)))) return st;
    c->cap_rows = n;
    return 0;
}

// Decode step launches, in order.  Indices of the kernels the measurement
// entry point can replay are recorded in c->kernels.
struct StepBuilder {
    sq_ctx* c;
    std::vector<std::function<int()>> launches;
};

enum KernelId { K_GATEUP = 0, K_HEAD = 1, K_DOWN = 2, K_QKV = 3, K_ATTN = 4, K_OPROJ = 5, K_COUNT = 6 };

int build_decode_step(sq_ctx* c) {
    const sq_model* m = c->m;
    const Config& g = m->cfg;
    const int D = g.dim, F = g.ffn, QD = g.n_heads * g.head_dim, KVD = g.n_kv_heads * g.head_dim;
    const bool a8 = c->a8;
    hipStream_t s = c->stream;
    std::vector<std::function<int()>>& L = c->kernels;
    L.clear();
    c->kernel_bytes.assign(K_COUNT, 0);
    std::vector<std::function<int()>> step;
    std::vector<int> named(K_COUNT, -1);

    const size_t kv_layer = c->max_pos * (size_t)KVD;
    const size_t TW = tap_width(g);
    // quantized activations of layer l, site j (see sq_ctx::tap_q)
    auto tq = [&](int l, int j) { return c->tap_q + l * TW + tap_offset(g, j); };
    auto td = [&](int l, int j) { return c->tap_d + (l * TW + tap_offset(g, j)) / 32; };
    auto mat_bytes = [](const DevMatrix& x) { return (uint64_t)(x.payload_bytes() + x.scale_bytes()); };
    // Kernels replayed by the measurement entry point come from layer 1 (layer
    // 0's QKV also performs the embedding lookup).
    const int lt = g.n_layers > 1 ? 1 : 0;
    for (int l = 0; l < g.n_layers; l++) {
        const Layer& Ly = m->layers[l];
        float* kc = c->kcache + l * kv_layer;
        float* vc = c->vcache + l * kv_layer;
        GemvArgs q{};
        q.w = view(Ly.qkv);
        q.n_rows = QD + 2 * KVD;
        q.x = c->hidden;
        q.norm_w = Ly.attn_norm;
        q.eps = g.eps;
        q.q_out = c->q;
        q.kcache = kc;
        q.vcache = vc;
        q.rope = c->rope;
        q.pos = c->d_pos;
        q.q_rows = QD;
        q.kv_rows = KVD;
        q.half = g.head_dim / 2;
        q.dbg_qs = a8 ? tq(l, 0) : nullptr;
        q.dbg_d = td(l, 0);
        if (l == 0) {
            // embed (model.rs:57-62) fused into the first norm prologue
            q.embd = view(m->embd);
            q.token = c->d_token;
            q.id_error = c->d_id_error;
            q.hidden_out = c->hidden;
            q.dbg_normed = c->dbg_normed;
        }
        if (l == lt) {
            named[K_QKV] = (int)step.size();
            c->kernel_bytes[K_QKV] = mat_bytes(Ly.qkv) + 2ull * D * 4 + (uint64_t)(QD + 2 * KVD) * 4;
        }
        step.push_back([=]() { return launch_gemv(s, PRO_NORM, EPI_QKV, a8, q, nullptr); });
        if (l == lt) {
            named[K_ATTN] = (int)step.size();
            c->kernel_bytes[K_ATTN] = 0;  // depends on the position; filled at measurement time
        }
        int8_t* const attn_q = a8 ? tq(l, 1) : nullptr;
        uint16_t* const attn_d = td(l, 1);
        step.push_back([=]() {
            return launch_attn_decode(s, c->q, kc, vc, c->d_pos, g.n_heads, g.n_kv_heads, g.head_dim, c->max_tiles,
                                      c->part_m, c->part_l, c->part_o, c->attn_counters, c->attn, attn_q, attn_d);
        });
        GemvArgs o{};
        o.w = view(Ly.o);
        o.n_rows = D;
        o.aq = tq(l, 1);
        o.ad = td(l, 1);
        o.x = c->attn;
        o.out = c->hidden;
        if (l == lt) {
            named[K_OPROJ] = (int)step.size();
            c->kernel_bytes[K_OPROJ] = mat_bytes(Ly.o) + (a8 ? (uint64_t)QD + QD / 16 : (uint64_t)QD * 4) + 2ull * D * 4;
        }
        step.push_back([=]() { return launch_gemv(s, a8 ? PRO_Q8 : PRO_F32, EPI_RESID, a8, o, nullptr); });
        GemvArgs gu{};
        gu.w = view(Ly.gateup);
        gu.n_rows = F;
        gu.x = c->hidden;
        gu.norm_w = Ly.ffn_norm;
        gu.eps = g.eps;
        gu.ffn_act = c->ffn_act;
        gu.act_q = a8 ? tq(l, 3) : nullptr;
        gu.act_d = td(l, 3);
        gu.dbg_qs = a8 ? tq(l, 2) : nullptr;
        gu.dbg_d = td(l, 2);
        if (l == lt) {
            named[K_GATEUP] = (int)step.size();
            c->kernel_bytes[K_GATEUP] = mat_bytes(Ly.gateup) + 2ull * D * 4 + (uint64_t)F * 4 +
                                        (a8 ? (uint64_t)F + F / 16 : 0);
        }
        step.push_back([=]() { return launch_gemv(s, PRO_NORM, EPI_GATEUP, a8, gu, nullptr); });
        GemvArgs dn{};
        dn.w = view(Ly.down);
        dn.n_rows = D;
        dn.aq = tq(l, 3);
        dn.ad = td(l, 3);
        dn.x = c->ffn_act;
        dn.out = c->hidden;
        if (l == lt) {
            named[K_DOWN] = (int)step.size();
            c->kernel_bytes[K_DOWN] = mat_bytes(Ly.down) + (a8 ? (uint64_t)F + F / 16 : (uint64_t)F * 4) + 2ull * D * 4;
        }
        step.push_back([=]() { return launch_gemv(s, a8 ? PRO_Q8 : PRO_F32, EPI_RESID, a8, dn, nullptr); });
    }
    GemvArgs h{};
    h.w = view(m->head);
    h.n_rows = g.vocab;
    h.x = c->hidden;
    h.norm_w = m->out_norm;
    h.eps = g.eps;
    h.out = c->logits;
    h.part_val = c->pv;
    h.part_idx = c->pi;
    h.part_nan = c->pn;
    h.dbg_normed = c->last_hidden;
    h.dbg_qs = c->head_qs;
    h.dbg_d = c->head_d;
    named[K_HEAD] = (int)step.size();
    c->kernel_bytes[K_HEAD] = mat_bytes(m->head) + 2ull * D * 4 + (uint64_t)g.vocab * 4;
    step.push_back([=]() { return launch_gemv(s, PRO_NORM, EPI_LOGITS, a8, h, nullptr); });
    step.push_back([=]() {
        return launch_argmax_final(s, c->logits, g.vocab, c->pv, c->pi, c->pn, c->n_parts, c->d_token, c->d_pos, 1,
                                   c->d_hist, c->d_nhist);
    });
    for (int k = 0; k < K_COUNT; k++) L.push_back(step[named[k]]);
    // The whole step as one launcher.
    auto all = std::make_shared<std::vector<std::function<int()>>>(std::move(step));
    L.push_back([all]() {
        for (auto& f : *all) {
            int st = f();
            if (st) return st;
        }
        return 0;
    });
    return 0;
}

int run_decode_step(sq_ctx* c) {
    if (c->persist) return launch_decode_step(c->stream, c->m->wtype, c->step, c->step_grid, (int)c->seq_len);
    if (c->graph) {
        SQ_HIP_CHECK(hipGraphLaunch(c->graph, c->stream));
        return 0;
    }
    return c->kernels.back()();
}

// Final norm + LM head + argmax for the last row (prefill tail).
int run_head(sq_ctx* c, int advance) {
    const sq_model* m = c->m;
    const Config& g = m->cfg;
    GemvArgs h{};
    h.w = view(m->head);
    h.n_rows = g.vocab;
    h.x = c->hidden;
    h.norm_w = m->out_norm;
    h.eps = g.eps;
    h.out = c->logits;
    h.part_val = c->pv;
    h.part_idx = c->pi;
    h.part_nan = c->pn;
    h.dbg_normed = c->last_hidden;
    h.dbg_qs = c->head_qs;
    h.dbg_d = c->head_d;
    int st = launch_gemv(c->stream, PRO_NORM, EPI_LOGITS, c->a8, h, nullptr);
    if (st) return st;
    return launch_argmax_final(c->stream, c->logits, g.vocab, c->pv, c->pi, c->pn, c->n_parts, c->d_token,
                               c->d_pos, advance, c->d_hist, c->d_nhist);
}

int run_prefill(sq_ctx* c, size_t n) {
    const sq_model* m = c->m;
    const Config& g = m->cfg;
    const int D = g.dim, F = g.ffn, QD = g.n_heads * g.head_dim, KVD = g.n_kv_heads * g.head_dim;
    const int hd = g.head_dim;
    const bool a8 = c->a8;
    hipStream_t s = c->stream;
    int st;
    if ((st = ensure_prefill(c, n))) return st;
    const size_t TW = tap_width(g);
    const bool taps = c->taps && a8;
    if (taps && c->ptap_rows < n) {
        dfree(c->ptap_q);
        dfree(c->ptap_d);
        c->ptap_rows = 0;
        if ((st = dmalloc(&c->ptap_q, n * g.n_layers * TW)) || (st = dmalloc(&c->ptap_d, n * g.n_layers * TW / 32)))
            return st;
        c->ptap_rows = n;
    }
    // the n rows of site j of layer l, just quantized into p_aq / p_ad
    auto tap = [&](int l, int j, size_t k, const int8_t* q = nullptr, const uint16_t* d = nullptr) -> int {
        if (!taps) return 0;
        const size_t off = n * (l * TW + tap_offset(g, j));
        SQ_HIP_CHECK(hipMemcpyAsync(c->ptap_q + off, q ? q : c->p_aq, n * k, hipMemcpyDeviceToDevice, s));
        SQ_HIP_CHECK(hipMemcpyAsync(c->ptap_d + off / 32, d ? d : c->p_ad, n * k / 16, hipMemcpyDeviceToDevice, s));
        return 0;
    };
    // phase boundary for the measurement entry point (kind: 0 matmul,
    // 1 attention, 2 other, 3 end)
    auto phase = [&](int kind) -> int {
        if (!c->prof) return 0;
        hipEvent_t e;
        SQ_HIP_CHECK(hipEventCreate(&e));
        c->prof_ev.push_back(e);
        c->prof_kind.push_back(kind);
        SQ_HIP_CHECK(hipEventRecord(e, s));
        return 0;
    };
    if ((st = phase(2))) return st;
    SQ_HIP_CHECK(hipMemcpyAsync(c->d_ids, c->h_pinned, n * 4, hipMemcpyHostToDevice, s));
    if ((st = launch_embed(s, view(m->embd), m->wtype, c->d_ids, (int)n, D, c->p_hidden, c->d_id_error))) return st;
    const int pos0 = (int)c->seq_len;
    const int N = (int)n;
    const size_t kv_layer = c->max_pos * (size_t)KVD;
    for (int l = 0; l < g.n_layers; l++) {
        const Layer& L = m->layers[l];
        float* kc = c->kcache + l * kv_layer;
        float* vc = c->vcache + l * kv_layer;
        if ((st = launch_rmsnorm_rows(s, c->p_hidden, L.attn_norm, N, D, g.eps, a8 ? nullptr : c->p_normed,
                                      a8 ? c->p_aq : nullptr, c->p_ad)) ||
            (st = tap(l, 0, D)))
            return st;
        // the q|k|v projection with RoPE and the KV append in its epilogue
        if ((st = phase(0))) return st;
        const int fused_qkv = a8 ? launch_qkv_rope(s, view(L.qkv), m->wtype, c->p_aq, c->p_ad, N, QD, KVD, hd, pos0,
                                                   c->rope, c->p_q, kc, vc, c->p_split, kPrefillSplitFloats)
                                 : -1;
        if (fused_qkv > 0) return fused_qkv;
        if (fused_qkv != 0) {
            if ((st = launch_gemm(s, view(L.qkv), m->wtype, a8, c->p_aq, c->p_ad, c->p_normed, N, c->p_qkv,
                                  QD + 2 * KVD, false, c->p_split, kPrefillSplitFloats)) ||
                (st = phase(2)) ||
                (st = launch_rope_kv_rows(s, c->p_qkv, QD + 2 * KVD, N, QD, KVD, hd, pos0, c->rope, c->p_q, kc, vc)))
                return st;
        } else if ((st = phase(2))) {
            return st;
        }
        // the integer path takes the attention rows as Q8_0 blocks, formed by
        // the attention kernel itself (the f32 rows are not stored)
        if ((st = phase(1)) ||
            (st = launch_attn_prefill(s, c->p_q, kc, vc, pos0, N, g.n_heads, g.n_kv_heads, hd, c->p_kvs,
                                      (int)c->max_pos, a8 ? nullptr : c->p_attn, a8 ? c->p_aq : nullptr,
                                      a8 ? c->p_ad : nullptr)) ||
            (st = phase(2)))
            return st;
        if (a8 && (st = tap(l, 1, QD))) return st;
        if ((st = phase(0)) ||
            (st = launch_gemm(s, view(L.o), m->wtype, a8, c->p_aq, c->p_ad, c->p_attn, N, c->p_hidden, D, true,
                              c->p_split, kPrefillSplitFloats)) ||
            (st = phase(2)))
            return st;
        if ((st = launch_rmsnorm_rows(s, c->p_hidden, L.ffn_norm, N, D, g.eps, a8 ? nullptr : c->p_normed,
                                      a8 ? c->p_aq : nullptr, c->p_ad)) ||
            (st = tap(l, 2, D)))
            return st;
        // Short prompts: gate/up, SiLU * up and its Q8_0 blocks in one launch.
        // Every workgroup of it reads every prompt row's FFN-norm blocks in
        // p_aq, so it writes the FFN activation's blocks apart, into p_act's
        // bytes (unused by the integer path), and the down projection reads
        // them there.
        const int8_t* fq = c->p_aq;
        const uint16_t* fd = c->p_ad;
        int fused = -1;
        if ((st = phase(0))) return st;
        if (a8) {
            int8_t* aq2 = (int8_t*)c->p_act;
            uint16_t* ad2 = (uint16_t*)(aq2 + (size_t)N * F);
            fused = launch_gateup_silu(s, view(L.gateup), m->wtype, c->p_aq, c->p_ad, N, aq2, ad2,
                                       kPrefillSplitFloats);
            if (fused > 0) return fused;
            if (fused == 0) {
                fq = aq2;
                fd = ad2;
            }
        }
        if (fused != 0) {
            if ((st = launch_gemm(s, view(L.gateup), m->wtype, a8, c->p_aq, c->p_ad, c->p_normed, N, c->p_gu, 2 * F,
                                  false, c->p_split, kPrefillSplitFloats)) ||
                (st = phase(2)) ||
                (st = launch_silu_mul_rows(s, c->p_gu, F, (size_t)N * F, a8 ? nullptr : c->p_act,
                                           a8 ? c->p_aq : nullptr, c->p_ad)))
                return st;
        } else if ((st = phase(2))) {
            return st;
        }
        if ((a8 && (st = tap(l, 3, F, fq, fd)))) return st;
        if ((st = phase(0)) ||
            (st = launch_gemm(s, view(L.down), m->wtype, a8, fq, fd, c->p_act, N, c->p_hidden, D, true,
                              c->p_split, kPrefillSplitFloats)) ||
            (st = phase(2)))
            return st;
    }
    SQ_HIP_CHECK(hipMemcpyAsync(c->hidden, c->p_hidden + (size_t)(N - 1) * D, (size_t)D * 4,
                                hipMemcpyDeviceToDevice, s));
    if ((st = run_head(c, N))) return st;
    return phase(3);
}

}  // namespace

// The persistent decode step serves integer-path Q8_0 / Q4_0 models with
// head_dim 64 (the multi-kernel hipGraph path serves the rest, and any context
// created with SQ_CTX_MULTI_KERNEL).
int setup_persistent(sq_ctx* c) {
    const sq_model* m = c->m;
    const Config& g = m->cfg;
    if ((c->flags & SQ_CTX_MULTI_KERNEL) || !c->a8 || (m->wtype != WT_Q8_0 && m->wtype != WT_Q4_0) ||
        g.head_dim != 64)
        return 0;
    int grid = 0, st;
    if ((st = decode_step_max_grid(m->wtype, &grid))) return st;
    // SQUIRREL_STEP_GRID sets the workgroup count (one per CU by default):
    // below the CU count it leaves CUs to other work on the device; a count
    // the shape does not fit in selects the multi-kernel path; a count above
    // what the device holds at once is refused at launch.
    if (const char* e = getenv("SQUIRREL_STEP_GRID")) {
        const int req = atoi(e);
        if (req > 0) grid = req;
    }
    if (!decode_step_fits(g.dim, g.ffn, g.n_heads, g.n_kv_heads, grid)) return 0;
    const int QD = g.n_heads * g.head_dim, KVD = g.n_kv_heads * g.head_dim;
    std::vector<StepLayer> hl(g.n_layers);
    for (int l = 0; l < g.n_layers; l++) {
        const Layer& L = m->layers[l];
        hl[l] = StepLayer{view(L.qkv), view(L.o), view(L.gateup), view(L.down), L.attn_norm, L.ffn_norm};
    }
    const size_t nx = exchange_words(g.dim, g.ffn, g.n_heads, g.n_kv_heads, c->max_tiles, grid);
    if ((st = dmalloc(&c->d_layers, (size_t)g.n_layers)) || (st = dmalloc(&c->s_xchg, nx)) ||
        (st = dmalloc(&c->s_epoch, 1)) || (st = dmalloc(&c->s_error, 1)))
        return st;
    SQ_HIP_CHECK(hipMemcpy(c->d_layers, hl.data(), hl.size() * sizeof(StepLayer), hipMemcpyHostToDevice));
    SQ_HIP_CHECK(hipMemset(c->s_xchg, 0, nx * 8));
    SQ_HIP_CHECK(hipMemset(c->s_epoch, 0, 4));
    SQ_HIP_CHECK(hipMemset(c->s_error, 0, 4));
    int dev = 0, khz = 0;
    SQ_HIP_CHECK(hipGetDevice(&dev));
    SQ_HIP_CHECK(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev));
    StepArgs& a = c->step;
    a.layers = c->d_layers;
    a.embd = view(m->embd);
    a.head = view(m->head);
    a.out_norm = m->out_norm;
    a.n_layers = g.n_layers;
    a.dim = g.dim;
    a.ffn = g.ffn;
    a.n_heads = g.n_heads;
    a.n_kv_heads = g.n_kv_heads;
    a.vocab = g.vocab;
    a.eps = g.eps;
    unsigned long long* x = c->s_xchg;
    a.x.h = x; x += g.dim;
    a.x.q = x; x += QD;
    a.x.k = x; x += KVD;
    a.x.v = x; x += KVD;
    a.x.a = x; x += QD / 4 + QD / 32;
    a.x.f = x; x += g.ffn / 4 + g.ffn / 32;
    a.x.p = x; x += 3 * (size_t)grid;
    a.x.t = x;
    a.kcache = c->kcache;
    a.vcache = c->vcache;
    a.kv_layer = c->max_pos * (size_t)KVD;
    a.rope = c->rope;
    a.pos = c->d_pos;
    a.token = c->d_token;
    a.history = c->d_hist;
    a.n_hist = c->d_nhist;
    a.logits = c->logits;
    a.max_tiles = c->max_tiles;
    a.epoch = c->s_epoch;
    a.error = c->s_error;
    a.id_error = c->d_id_error;
    a.spin_limit = (long long)khz * 250;  // 250 ms
    a.dbg_normed = c->dbg_normed;
    a.dbg_qs = c->tap_q;
    a.dbg_d = c->tap_d;
    a.taps = c->taps ? 1 : 0;
    a.last_hidden = c->last_hidden;
    a.head_qs = c->head_qs;
    a.head_d = c->head_d;
    a.trace = nullptr;
    a.trace_stride = 0;
    a.stream_stride = decode_stream_stride(m->wtype, g.n_layers, g.dim, g.ffn, g.n_heads, g.n_kv_heads, g.vocab, grid);
    if ((st = dmalloc(&c->s_stream, a.stream_stride * 16 * (size_t)grid))) return st;
    a.stream = c->s_stream;
    if ((st = launch_build_stream(c->stream, m->wtype, a, grid, c->s_stream))) return st;
    SQ_HIP_CHECK(hipStreamSynchronize(c->stream));
    c->step_grid = grid;
    c->persist = true;
    return 0;
}

int ctx_check(sq_ctx* c) {
    SQ_HIP_CHECK(hipStreamSynchronize(c->stream));
    uint32_t id_err = 0;
    SQ_HIP_CHECK(hipMemcpy(&id_err, c->d_id_error, 4, hipMemcpyDeviceToHost));
    if (id_err)
        return set_error(SQ_ERR_ARG, "forward: a token id on the device is past the embedding table "
                                     "(embedding.rs:43-44); the context must be reset");
    if (!c->persist) return 0;
    int err = 0;
    SQ_HIP_CHECK(hipMemcpy(&err, c->s_error, 4, hipMemcpyDeviceToHost));
    if (err)
        return set_error(SQ_ERR_HIP, "decode step: a grid barrier wait timed out; the context must be reset");
    return 0;
}

int ctx_reset(sq_ctx* c) {
    SQ_HIP_CHECK(hipStreamSynchronize(c->stream));
    c->seq_len = 0;
    // every write on the context's own stream, so the next launch there is
    // ordered after them
    SQ_HIP_CHECK(hipMemsetAsync(c->d_pos, 0, 4, c->stream));
    SQ_HIP_CHECK(hipMemsetAsync(c->d_nhist, 0, 4, c->stream));
    SQ_HIP_CHECK(hipMemsetAsync(c->d_id_error, 0, 4, c->stream));
    if (c->persist) {
        unsigned epoch = 0;
        SQ_HIP_CHECK(hipMemcpyAsync(&epoch, c->s_epoch, 4, hipMemcpyDeviceToHost, c->stream));
        SQ_HIP_CHECK(hipStreamSynchronize(c->stream));
        epoch += 2u * (6u * (unsigned)c->m->cfg.n_layers + 2u);
        c->h_pinned[0] = epoch;
        SQ_HIP_CHECK(hipMemcpyAsync(c->s_epoch, c->h_pinned, 4, hipMemcpyHostToDevice, c->stream));
        SQ_HIP_CHECK(hipMemsetAsync(c->s_error, 0, 4, c->stream));
    }
    SQ_HIP_CHECK(hipStreamSynchronize(c->stream));
    return 0;
}

int ctx_create(const sq_model* m, size_t max_pos, uint32_t flags, sq_ctx** out) {
    if (!m || max_pos == 0) return set_error(SQ_ERR_ARG, "ctx_new: null model or zero positions");
    if (flags & SQ_CTX_F32_ACTS) return set_error(SQ_ERR_UNSUPPORTED, kA32Disabled);
    SQ_HIP_CHECK(hipSetDevice(m->device));
    sq_ctx* c = new sq_ctx();
    c->m = m;
    c->max_pos = max_pos;
    c->flags = flags;
    c->a8 = m->wtype != WT_BF16 && !(flags & SQ_CTX_F32_ACTS);
    const Config& g = m->cfg;
    const size_t D = g.dim, F = g.ffn, QD = (size_t)g.n_heads * g.head_dim, KVD = (size_t)g.n_kv_heads * g.head_dim;
    const int half = g.head_dim / 2;
    auto fail = [&](int st) {
        ctx_destroy(c);
        return st;
    };
    int st;
    hipError_t he = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
    if (he != hipSuccess) return fail(set_error(SQ_ERR_HIP, std::string("hipStreamCreate: ") + hipGetErrorString(he)));
    c->max_tiles = (int)((max_pos + 63) / 64);
    c->n_parts = kLogitsGrid;
    if ((st = dmalloc(&c->kcache, (size_t)g.n_layers * max_pos * KVD)) ||
        (st = dmalloc(&c->vcache, (size_t)g.n_layers * max_pos * KVD)) || (st = dmalloc(&c->rope, max_pos * half)) ||
        (st = dmalloc(&c->d_pos, 1)) || (st = dmalloc(&c->d_token, 1)) || (st = dmalloc(&c->d_ids, max_pos)) ||
        (st = dmalloc(&c->d_hist, max_pos + 1)) || (st = dmalloc(&c->d_nhist, 1)) || (st = dmalloc(&c->hidden, D)) ||
        (st = dmalloc(&c->q, QD)) || (st = dmalloc(&c->attn, QD)) || (st = dmalloc(&c->ffn_act, F)) ||
        (st = dmalloc(&c->tap_q, g.n_layers * tap_width(g))) ||
        (st = dmalloc(&c->tap_d, g.n_layers * tap_width(g) / 32)) || (st = dmalloc(&c->logits, (size_t)g.vocab)) ||
        (st = dmalloc(&c->part_m, (size_t)g.n_heads * c->max_tiles)) ||
        (st = dmalloc(&c->part_l, (size_t)g.n_heads * c->max_tiles)) ||
        (st = dmalloc(&c->part_o, (size_t)g.n_heads * c->max_tiles * g.head_dim)) ||
        (st = dmalloc(&c->attn_counters, (size_t)g.n_kv_heads)) ||
        (st = dmalloc(&c->pv, c->n_parts)) ||
        (st = dmalloc(&c->pi, c->n_parts)) || (st = dmalloc(&c->pn, c->n_parts)) ||
        (st = dmalloc(&c->dbg_normed, D)) || (st = dmalloc(&c->last_hidden, D)) || (st = dmalloc(&c->head_qs, D)) ||
        (st = dmalloc(&c->head_d, D / 32)) || (st = dmalloc(&c->d_sids, max_pos + 1)) ||
        (st = dmalloc(&c->d_logp, max_pos + 1)) || (st = dmalloc(&c->d_id_error, 1)))
        return fail(st);
    he = hipHostMalloc((void**)&c->h_pinned, (max_pos + 16) * sizeof(uint32_t), hipHostMallocDefault);
    if (he != hipSuccess) return fail(set_error(SQ_ERR_HIP, std::string("hipHostMalloc: ") + hipGetErrorString(he)));

    // RoPE (cos, sin) per position, computed on the host exactly as the
    // reference: theta = f32(pos) * inv_freq[j], then libm sinf / cosf
    // (src/kernels/rope.rs:24-26).
    std::vector<float2> h_rope(max_pos * half);
    for (size_t p = 0; p < max_pos; p++)
        for (int j = 0; j < half; j++) {
            volatile float theta = (float)p * g.inv_freq[j];
            h_rope[p * half + j] = make_float2(cosf(theta), sinf(theta));
        }
    SQ_HIP_CHECK(hipMemcpy(c->rope, h_rope.data(), h_rope.size() * sizeof(float2), hipMemcpyHostToDevice));
    std::vector<float> init_v(c->n_parts, -INFINITY);
    std::vector<int> init_i(c->n_parts, -1);
    SQ_HIP_CHECK(hipMemcpy(c->pv, init_v.data(), c->n_parts * 4, hipMemcpyHostToDevice));
    SQ_HIP_CHECK(hipMemcpy(c->pi, init_i.data(), c->n_parts * 4, hipMemcpyHostToDevice));
    SQ_HIP_CHECK(hipMemcpy(c->pn, init_i.data(), c->n_parts * 4, hipMemcpyHostToDevice));
    SQ_HIP_CHECK(hipMemset(c->attn_counters, 0, (size_t)g.n_kv_heads * 4));
    SQ_HIP_CHECK(hipMemset(c->d_pos, 0, 4));
    SQ_HIP_CHECK(hipMemset(c->d_nhist, 0, 4));
    SQ_HIP_CHECK(hipMemset(c->d_token, 0, 4));
    SQ_HIP_CHECK(hipMemset(c->d_id_error, 0, 4));
    SQ_HIP_CHECK(hipMemset(c->kcache, 0, (size_t)g.n_layers * max_pos * KVD * 4));
    SQ_HIP_CHECK(hipMemset(c->vcache, 0, (size_t)g.n_layers * max_pos * KVD * 4));

    if ((st = build_decode_step(c))) return fail(st);
    if (!(flags & SQ_CTX_NO_GRAPH)) {
        SQ_HIP_CHECK(hipStreamBeginCapture(c->stream, hipStreamCaptureModeRelaxed));
        st = c->kernels.back()();
        hipGraph_t gr = nullptr;
        hipError_t ce = hipStreamEndCapture(c->stream, &gr);
        if (st) return fail(st);
        if (ce != hipSuccess) return fail(set_error(SQ_ERR_HIP, std::string("hipStreamEndCapture: ") + hipGetErrorString(ce)));
        c->graph_def = gr;
        ce = hipGraphInstantiate(&c->graph, gr, nullptr, nullptr, 0);
        if (ce != hipSuccess) return fail(set_error(SQ_ERR_HIP, std::string("hipGraphInstantiate: ") + hipGetErrorString(ce)));
    }
    if ((st = setup_persistent(c))) return fail(st);
    SQ_HIP_CHECK(hipDeviceSynchronize());
    *out = c;
    return 0;
}

void ctx_destroy(sq_ctx* c) {
    if (!c) return;
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    if (c->graph) (void)hipGraphExecDestroy(c->graph);
    if (c->graph_def) (void)hipGraphDestroy(c->graph_def);
    dfree(c->kcache); dfree(c->vcache); dfree(c->rope); dfree(c->d_pos); dfree(c->d_token); dfree(c->d_ids);
    dfree(c->d_hist); dfree(c->d_nhist); dfree(c->hidden); dfree(c->q); dfree(c->attn); dfree(c->tap_q);
    dfree(c->tap_d); dfree(c->ffn_act); dfree(c->ptap_q); dfree(c->ptap_d); dfree(c->logits); dfree(c->part_m);
    dfree(c->part_l); dfree(c->part_o); dfree(c->attn_counters); dfree(c->pv); dfree(c->pi); dfree(c->pn); dfree(c->dbg_normed);
    dfree(c->last_hidden); dfree(c->head_qs); dfree(c->head_d);
    dfree(c->p_hidden); dfree(c->p_normed); dfree(c->p_qkv); dfree(c->p_q); dfree(c->p_attn); dfree(c->p_gu);
    dfree(c->p_kvs); dfree(c->p_act); dfree(c->p_aq); dfree(c->p_ad); dfree(c->p_split);
    dfree(c->d_layers); dfree(c->s_stream); dfree(c->s_xchg); dfree(c->s_epoch); dfree(c->s_error); dfree(c->s_trace);
    dfree(c->d_sids); dfree(c->d_logp); dfree(c->d_id_error);
    if (c->h_pinned) (void)hipHostFree(c->h_pinned);
    if (c->stream) (void)hipStreamDestroy(c->stream);
    delete c;
}

int ctx_forward(sq_ctx* c, const uint32_t* ids, size_t n) {
    if (!c || (!ids && n)) return set_error(SQ_ERR_ARG, "forward: null argument");
    if (n == 0) return set_error(SQ_ERR_EMPTY, "forward: EmptyInput (model.rs:48-52)");
    if (c->seq_len + n > c->max_pos)
        return set_error(SQ_ERR_CACHE_FULL, "forward: " + std::to_string(c->seq_len + n) + " positions exceed the " +
                                                std::to_string(c->max_pos) + " the context holds");
    for (size_t i = 0; i < n; i++)
        if ((int64_t)ids[i] >= c->m->cfg.vocab) return set_error(SQ_ERR_ARG, "forward: token id out of range");
    // The staging buffer may still feed an earlier async copy.
    SQ_HIP_CHECK(hipStreamSynchronize(c->stream));
    memcpy(c->h_pinned, ids, n * 4);
    int st;
    if (n == 1) {
        SQ_HIP_CHECK(hipMemcpyAsync(c->d_token, c->h_pinned, 4, hipMemcpyHostToDevice, c->stream));
        st = run_decode_step(c);
    } else {
        st = run_prefill(c, n);
    }
    if (st) return st;
    c->seq_len += n;
    c->last_rows = n;
    c->last_tapped = c->a8 && (n > 1 ? c->taps : (c->taps || !c->persist));
    return 0;
}

int ctx_score(sq_ctx* c, const uint32_t* ids, size_t n, size_t burn, double* logp) {
    if (!c || !ids || !logp) return set_error(SQ_ERR_ARG, "score: null argument");
    if (burn == 0 || burn >= n) return set_error(SQ_ERR_ARG, "score: the burn-in must leave 1 to n - 1 scored tokens");
    if (n - 1 > c->max_pos)
        return set_error(SQ_ERR_CACHE_FULL, "score: a window of " + std::to_string(n) + " tokens needs " +
                                                std::to_string(n - 1) + " positions; the context holds " +
                                                std::to_string(c->max_pos));
    const int V = c->m->cfg.vocab;
    for (size_t i = 0; i < n; i++)
        if ((int64_t)ids[i] >= V) return set_error(SQ_ERR_ARG, "score: token id out of range");
    // A fresh cache per window (perplexity.rs:69-70).  The token history
    // restarts with the position: every head step appends to it, and it
    // holds max_pos + 1 entries.
    int st = ctx_reset(c);
    if (st) return st;
    st = ctx_forward(c, ids, burn);
    if (st) return st;
    // ctx_forward synchronized before staging the burn-in ids; the window
    // goes to the device behind the prefill on the same stream.
    SQ_HIP_CHECK(hipMemcpyAsync(c->d_sids, ids, n * 4, hipMemcpyHostToDevice, c->stream));
    // Every step stays on the device: the scored token's log-probability is
    // taken from the logits in place, and the same id is fed to the next
    // decode step from device memory.
    for (size_t i = burn; i < n; i++) {
        if ((st = launch_log_softmax_at(c->stream, c->logits, V, c->d_sids + i, c->d_logp + (i - burn),
                                        c->d_id_error)))
            return st;
        if (i + 1 < n) {
            if ((st = launch_copy_i32(c->stream, (const int*)(c->d_sids + i), (int*)c->d_token))) return st;
            if ((st = run_decode_step(c))) return st;
            c->seq_len++;
        }
    }
    SQ_HIP_CHECK(hipMemcpyAsync(logp, c->d_logp, (n - burn) * sizeof(double), hipMemcpyDeviceToHost, c->stream));
    SQ_HIP_CHECK(hipStreamSynchronize(c->stream));
    c->last_rows = 1;
    c->last_tapped = false;
    return ctx_check(c);
}

int ctx_prefill_phases(sq_ctx* c, const uint32_t* ids, size_t n, double* ms) {
    if (n < 2) return set_error(SQ_ERR_ARG, "prefill_phases: needs a prompt of at least 2 tokens");
    int st = ctx_reset(c);
    if (st) return st;
    c->prof = true;
    st = ctx_forward(c, ids, n);
    c->prof = false;
    hipError_t e = hipStreamSynchronize(c->stream);
    for (int k = 0; k < 4; k++) ms[k] = 0.0;
    for (size_t i = 0; !st && e == hipSuccess && i + 1 < c->prof_ev.size(); i++) {
        float t = 0.f;
        e = hipEventElapsedTime(&t, c->prof_ev[i], c->prof_ev[i + 1]);
        ms[c->prof_kind[i]] += t;
        ms[3] += t;
    }
    for (hipEvent_t ev : c->prof_ev) (void)hipEventDestroy(ev);
    c->prof_ev.clear();
    c->prof_kind.clear();
    if (st) return st;
    if (e != hipSuccess) return set_error(SQ_ERR_HIP, std::string("prefill_phases: ") + hipGetErrorString(e));
    return 0;
}

int ctx_set_taps(sq_ctx* c, bool on) {
    if (!c->a8) return set_error(SQ_ERR_UNSUPPORTED, "act_taps: the context has no quantized activations");
    SQ_HIP_CHECK(hipStreamSynchronize(c->stream));
    c->taps = on;
    c->step.taps = on ? 1 : 0;
    return 0;
}

int ctx_read_taps(sq_ctx* c, void* blocks, size_t n_blocks) {
    const Config& g = c->m->cfg;
    const size_t TW = tap_width(g), n = c->last_rows, D = g.dim;
    if (n == 0 || !c->last_tapped)
        return set_error(SQ_ERR_ARG, "act_tap_read: the most recent forward did not record its activations");
    const size_t body = n * g.n_layers * TW;  // elements before the LM-head row
    if (n_blocks < (body + D) / 32) return set_error(SQ_ERR_ARG, "act_tap_read: buffer too small");
    SQ_HIP_CHECK(hipStreamSynchronize(c->stream));
    std::vector<int8_t> qs(body + D);
    std::vector<uint16_t> d((body + D) / 32);
    const int8_t* sq = n > 1 ? c->ptap_q : c->tap_q;
    const uint16_t* sd = n > 1 ? c->ptap_d : c->tap_d;
    SQ_HIP_CHECK(hipMemcpy(qs.data(), sq, body, hipMemcpyDeviceToHost));
    SQ_HIP_CHECK(hipMemcpy(d.data(), sd, body / 16, hipMemcpyDeviceToHost));
    SQ_HIP_CHECK(hipMemcpy(qs.data() + body, c->head_qs, D, hipMemcpyDeviceToHost));
    SQ_HIP_CHECK(hipMemcpy(d.data() + body / 32, c->head_d, D / 16, hipMemcpyDeviceToHost));
    uint8_t* out = (uint8_t*)blocks;
    for (size_t b = 0; b < (body + D) / 32; b++) {
        memcpy(out + 34 * b, &d[b], 2);
        memcpy(out + 34 * b + 2, qs.data() + 32 * b, 32);
    }
    return 0;
}

int ctx_generate(sq_ctx* c, const uint32_t* prompt, size_t n_prompt, size_t max_tokens, uint32_t flags,
                 uint32_t* out, size_t* n_out, double* step_ms) {
    using clk = std::chrono::steady_clock;
    *n_out = 0;
    if (n_prompt == 0) return set_error(SQ_ERR_EMPTY, "generate: empty prompt");
    const uint32_t eos = c->m->cfg.eos;
    const bool ignore_eos = flags & SQ_GEN_IGNORE_EOS;
    // A fresh context per generation (text_generator.rs:58).
    if (int st = ctx_reset(c)) return st;
    if (max_tokens == 0) return 0;

    if (flags & SQ_GEN_NO_KV_CACHE) {
        // text_generator.rs:76-78: every step resets the cache and re-feeds
        // the prompt plus everything generated so far.
        std::vector<uint32_t> toks(prompt, prompt + n_prompt);
        for (size_t step = 0; step < max_tokens; step++) {
            auto t0 = clk::now();
            SQ_HIP_CHECK(hipStreamSynchronize(c->stream));
            c->seq_len = 0;
            SQ_HIP_CHECK(hipMemsetAsync(c->d_pos, 0, 4, c->stream));
            int st = ctx_forward(c, toks.data(), toks.size());
            if (st) return st;
            uint32_t tok;
            SQ_HIP_CHECK(hipMemcpyAsync(c->h_pinned, c->d_token, 4, hipMemcpyDeviceToHost, c->stream));
            SQ_HIP_CHECK(hipStreamSynchronize(c->stream));
            tok = c->h_pinned[0];
            if (step_ms) step_ms[step] = std::chrono::duration<double, std::milli>(clk::now() - t0).count();
            if (tok == eos && !ignore_eos) break;
            out[(*n_out)++] = tok;
            toks.push_back(tok);
        }
        return 0;
    }

    // Step 1: prefill + first token.
    auto t0 = clk::now();
    int st = ctx_forward(c, prompt, n_prompt);
    if (st) return st;
    SQ_HIP_CHECK(hipMemcpyAsync(c->h_pinned, c->d_token, 4, hipMemcpyDeviceToHost, c->stream));
    SQ_HIP_CHECK(hipStreamSynchronize(c->stream));
    uint32_t tok = c->h_pinned[0];
    if (step_ms) step_ms[0] = std::chrono::duration<double, std::milli>(clk::now() - t0).count();
    if (tok == eos && !ignore_eos) return 0;
    out[(*n_out)++] = tok;
    const size_t steps = std::min(max_tokens, c->max_pos - c->seq_len + 1);

    if (ignore_eos) {
        // Tokens never leave the GPU until the end: each replay reads the
        // previous step's token from device memory.
        std::vector<hipEvent_t> ev(steps);
        for (auto& e : ev) SQ_HIP_CHECK(hipEventCreate(&e));
        SQ_HIP_CHECK(hipEventRecord(ev[0], c->stream));
        for (size_t k = 1; k < steps; k++) {
            if ((st = run_decode_step(c))) return st;
            SQ_HIP_CHECK(hipEventRecord(ev[k], c->stream));
            c->seq_len++;
        }
        SQ_HIP_CHECK(hipStreamSynchronize(c->stream));
        for (size_t k = 1; k < steps; k++) {
            float ms = 0.f;
            SQ_HIP_CHECK(hipEventElapsedTime(&ms, ev[k - 1], ev[k]));
            if (step_ms) step_ms[k] = ms;
        }
        for (auto& e : ev) (void)hipEventDestroy(e);
        if (steps > 1)
            SQ_HIP_CHECK(hipMemcpy(out + 1, c->d_hist + 1, (steps - 1) * 4, hipMemcpyDeviceToHost));
        *n_out = steps;
        return 0;
    }

    for (size_t k = 1; k < steps; k++) {
        auto t1 = clk::now();
        if ((st = run_decode_step(c))) return st;
        c->seq_len++;
        SQ_HIP_CHECK(hipMemcpyAsync(c->h_pinned, c->d_token, 4, hipMemcpyDeviceToHost, c->stream));
        SQ_HIP_CHECK(hipStreamSynchronize(c->stream));
        tok = c->h_pinned[0];
        if (step_ms) step_ms[k] = std::chrono::duration<double, std::milli>(clk::now() - t1).count();
        if (tok == eos) break;
        out[(*n_out)++] = tok;
    }
    return 0;
}

int ctx_time_kernel(sq_ctx* c, int which, int iters, double* mean_us, uint64_t* bytes) {
    if (which < 0 || which >= K_COUNT || iters <= 0) return set_error(SQ_ERR_ARG, "time_kernel: bad kernel id");
    // Replays write the KV row at the current position and attend up to it.
    if (c->seq_len >= c->max_pos) return set_error(SQ_ERR_CACHE_FULL, "time_kernel: KV cache is full");
    const Config& g = c->m->cfg;
    hipEvent_t e0, e1;
    SQ_HIP_CHECK(hipEventCreate(&e0));
    SQ_HIP_CHECK(hipEventCreate(&e1));
    int st = c->kernels[which]();  // warm
    if (st) return st;
    SQ_HIP_CHECK(hipEventRecord(e0, c->stream));
    for (int i = 0; i < iters; i++)
        if ((st = c->kernels[which]())) return st;
    SQ_HIP_CHECK(hipEventRecord(e1, c->stream));
    SQ_HIP_CHECK(hipEventSynchronize(e1));
    float ms = 0.f;
    SQ_HIP_CHECK(hipEventElapsedTime(&ms, e0, e1));
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    *mean_us = 1000.0 * ms / iters;
    uint64_t b = c->kernel_bytes[which];
    if (which == K_ATTN) {
        const uint64_t P = c->seq_len + 1;  // positions attended by a replay at the current position
        b = 2ull * P * g.n_kv_heads * g.head_dim * 4 + (uint64_t)g.n_heads * g.head_dim * 4;
    }
    if (bytes) *bytes = b;
    return 0;
}

}  // namespace sq
