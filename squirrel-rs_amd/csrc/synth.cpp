// Seeded random-init Llama GGUF writer.
//
// Every weight element e of tensor t is a function of (seed, t, e) alone:
// a splitmix64 counter stream feeds Box-Muller in double precision, so the
// file is identical whatever the thread count.  Matrices are N(0, std) and
// quantized per 32-block:
//   Q8_0: the reference's own quantizer (src/kernels/dot_prod.rs:21-31);
//   Q4_0: ggml's reference quantizer: d = m / -8 with m the signed value of
//         largest magnitude, q = min(15, trunc(x/d + 8.5)); the reference pins
//         only the decode side, (q - 8) * d (src/kernels/tensor.rs:17-25);
//   BF16: round to nearest even.
// Norm gains are 1.0 (F32).  The LM head is tied (no output.weight).
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

#include "gguf.h"
#include "sq_common.h"

namespace sq {

namespace {

inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

struct Normal {
    uint64_t key;
    double sd;
    // Element e: pair p = e/2 -> (u1, u2) -> Box-Muller (cos for even, sin for odd).
    float operator()(uint64_t e) const {
        const uint64_t p = e >> 1;
        const uint64_t a = mix64(key + (2 * p + 0) * 0x9E3779B97F4A7C15ull);
        const uint64_t b = mix64(key + (2 * p + 1) * 0x9E3779B97F4A7C15ull);
        const double u1 = ((double)(a >> 11) + 1.0) * 0x1.0p-53;  // (0, 1]
        const double u2 = (double)(b >> 11) * 0x1.0p-53;          // [0, 1)
        const double r = std::sqrt(-2.0 * std::log(u1));
        const double th = 6.283185307179586476925 * u2;
        const double z = (e & 1) ? r * std::sin(th) : r * std::cos(th);
        return (float)(sd * z);
    }
};

uint16_t f32_to_f16_rne(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t exp = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (exp == 0xffu) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u | (man >> 13) : 0));
    const int e = (int)exp - 127 + 15;
    if (e >= 0x1f) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        man |= 0x800000u;
        const int shift = 14 - e;
        uint32_t hm = man >> shift;
        const uint32_t rem = man & ((1u << shift) - 1u), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (hm & 1u))) hm++;
        return (uint16_t)(sign | hm);
    }
    uint32_t h = sign | ((uint32_t)e << 10) | (man >> 13);
    const uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)h;
}

uint16_t f32_to_bf16_rne(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
    return (uint16_t)((x + 0x7fffu + ((x >> 16) & 1u)) >> 16);
}

#pragma STDC FP_CONTRACT OFF
void quant_q8_0(const float* x, uint8_t* out) {
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(x[i]));
    const float scale = amax / 127.0f;
    const float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
    const uint16_t d = f32_to_f16_rne(scale);
    memcpy(out, &d, 2);
    for (int i = 0; i < 32; i++) {
        float v = roundf(x[i] * inv);
        if (v < -127.0f) v = -127.0f;
        if (v > 127.0f) v = 127.0f;
        out[2 + i] = (uint8_t)(int8_t)(std::isnan(v) ? 0 : (int)v);
    }
}

void quant_q4_0(const float* x, uint8_t* out) {
    float amax = 0.0f, mx = 0.0f;
    for (int i = 0; i < 32; i++)
        if (amax < fabsf(x[i])) {
            amax = fabsf(x[i]);
            mx = x[i];
        }
    const float d = mx / -8.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const uint16_t dh = f32_to_f16_rne(d);
    memcpy(out, &dh, 2);
    for (int j = 0; j < 16; j++) {
        const float x0 = x[j] * id, x1 = x[16 + j] * id;
        int q0 = (int)(int8_t)(x0 + 8.5f), q1 = (int)(int8_t)(x1 + 8.5f);
        q0 = q0 < 15 ? q0 : 15;
        q1 = q1 < 15 ? q1 : 15;
        out[2 + j] = (uint8_t)(q0 | (q1 << 4));
    }
}

size_t row_bytes(int wtype, size_t k) {
    if (wtype == WT_Q8_0) return k / 32 * 34;
    if (wtype == WT_Q4_0) return k / 32 * 18;
    return k * 2;
}

// rows x k matrix of tensor index t, quantized row by row in parallel.
std::vector<uint8_t> gen_matrix(uint64_t seed, uint64_t t, size_t rows, size_t k, int wtype, double sd) {
    const size_t rb = row_bytes(wtype, k);
    std::vector<uint8_t> out(rows * rb);
    const Normal nrm{mix64(seed ^ (0xA24BAED4963EE407ull * (t + 1))), sd};
    unsigned nt = std::thread::hardware_concurrency();
    if (nt == 0) nt = 1;
    if (nt > 32) nt = 32;
    std::vector<std::thread> th;
    for (unsigned w = 0; w < nt; w++) {
        th.emplace_back([&, w]() {
            std::vector<float> row(k);
            for (size_t r = w; r < rows; r += nt) {
                for (size_t i = 0; i < k; i++) row[i] = nrm((uint64_t)r * k + i);
                uint8_t* o = out.data() + r * rb;
                for (size_t b = 0; b < k / 32; b++) {
                    if (wtype == WT_Q8_0) quant_q8_0(&row[b * 32], o + b * 34);
                    else if (wtype == WT_Q4_0) quant_q4_0(&row[b * 32], o + b * 18);
                    else
                        for (int i = 0; i < 32; i++) {
                            const uint16_t v = f32_to_bf16_rne(row[b * 32 + i]);
                            memcpy(o + (b * 32 + i) * 2, &v, 2);
                        }
                }
            }
        });
    }
    for (auto& x : th) x.join();
    return out;
}

}  // namespace

int synth_write(const std::string& path, const sq_synth_spec& s) {
    if (s.wtype != WT_Q8_0 && s.wtype != WT_Q4_0 && s.wtype != WT_BF16)
        return set_error(SQ_ERR_INVALID_TYPE, "synth: wtype must be Q8_0, Q4_0 or BF16");
    if (s.n_heads == 0 || s.n_kv_heads == 0 || s.dim % 32 || s.ffn_dim % 32 || s.dim % s.n_heads)
        return set_error(SQ_ERR_SHAPE, "synth: inconsistent dims");
    const uint64_t D = s.dim, F = s.ffn_dim, hd = s.dim / s.n_heads, QD = s.n_heads * hd, KVD = s.n_kv_heads * hd;
    const uint64_t V = s.vocab;
    const double sd = s.std_dev;
    GGUFWriter w;
    w.add_string("general.architecture", "llama");
    w.add_string("general.name", "synthetic-llama");
    w.add_u32("general.alignment", 32);
    w.add_u32("llama.block_count", s.n_layers);
    w.add_u32("llama.context_length", s.context_length);
    w.add_u32("llama.embedding_length", s.dim);
    w.add_u32("llama.feed_forward_length", s.ffn_dim);
    w.add_u32("llama.attention.head_count", s.n_heads);
    w.add_u32("llama.attention.head_count_kv", s.n_kv_heads);
    w.add_u32("llama.rope.dimension_count", (uint32_t)hd);
    w.add_f32("llama.rope.freq_base", s.rope_base);
    w.add_f32("llama.attention.layer_norm_rms_epsilon", s.rms_eps);
    w.add_u32("llama.vocab_size", s.vocab);
    w.add_u32("tokenizer.ggml.bos_token_id", s.bos);
    w.add_u32("tokenizer.ggml.eos_token_id", s.eos);

    std::vector<std::vector<uint8_t>> keep;
    std::vector<float> ones(D, 1.0f);
    uint64_t t = 0;
    auto add_mat = [&](const std::string& name, uint64_t k, uint64_t n) {
        keep.push_back(gen_matrix(s.seed, t++, n, k, (int)s.wtype, sd));
        w.add_tensor(name, {k, n}, s.wtype, keep.back().data(), keep.back().size());
    };
    add_mat("token_embd.weight", D, V);
    for (uint32_t i = 0; i < s.n_layers; i++) {
        const std::string p = "blk." + std::to_string(i) + ".";
        w.add_tensor(p + "attn_norm.weight", {D}, WT_F32, ones.data(), D * 4);
        add_mat(p + "attn_q.weight", D, QD);
        add_mat(p + "attn_k.weight", D, KVD);
        add_mat(p + "attn_v.weight", D, KVD);
        add_mat(p + "attn_output.weight", QD, D);
        w.add_tensor(p + "ffn_norm.weight", {D}, WT_F32, ones.data(), D * 4);
        add_mat(p + "ffn_gate.weight", D, F);
        add_mat(p + "ffn_up.weight", D, F);
        add_mat(p + "ffn_down.weight", F, D);
    }
    w.add_tensor("output_norm.weight", {D}, WT_F32, ones.data(), D * 4);
    return w.write(path);
}

}  // namespace sq
