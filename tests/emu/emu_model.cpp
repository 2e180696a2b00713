// Teacher-forced model run through the C ABI of the CPU emulation build,
// compared step by step with the oracle on the same GGUF file.
// TEST INFRASTRUCTURE ONLY.
//
//   emu_model <gguf> <oracle mode 0|1|2> <ctx flags> <n_prompt> <n_decode> <seed> <max_pos> [generate]
//   emu_model --write <gguf> <wtype> <seed> <n_layers> <dim> <ffn> <heads> <kv_heads> <vocab>
//
// Prints one line per step: "step <i> rel_l2 <e> max_abs <m> argmax <device> <oracle>".
// With a trailing "generate", also runs sq_generate over the prompt (greedy,
// EOS ignored) and prints the generated ids.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "../../include/squirrel_hip.h"
#include "../../oracle/oracle.h"
#include "gguf.h"

namespace sqemu {
extern uint64_t g_malloc_calls;  // hipMalloc calls so far (tests/emu/emu.cpp)
}

static void die(const char* what, int st) {
    fprintf(stderr, "%s failed: %d %s\n", what, st, sq_last_error());
    exit(2);
}

int main(int argc, char** argv) {
    if (argc == 11 && std::string(argv[1]) == "--write") {
        sq_synth_spec sp;
        memset(&sp, 0, sizeof(sp));
        sp.wtype = (uint32_t)atoi(argv[3]);
        sp.seed = (uint64_t)atoll(argv[4]);
        sp.n_layers = (uint32_t)atoi(argv[5]);
        sp.dim = (uint32_t)atoi(argv[6]);
        sp.ffn_dim = (uint32_t)atoi(argv[7]);
        sp.n_heads = (uint32_t)atoi(argv[8]);
        sp.n_kv_heads = (uint32_t)atoi(argv[9]);
        sp.vocab = (uint32_t)atoi(argv[10]);
        sp.context_length = 4096;
        sp.std_dev = 0.02f;
        sp.rope_base = 500000.0f;
        sp.rms_eps = 1e-5f;
        sp.bos = 1;
        sp.eos = 2;
        const int st = sq_synth_write_gguf(argv[2], &sp);
        if (st) die("sq_synth_write_gguf", st);
        return 0;
    }
    if (argc == 7 && std::string(argv[1]) == "--linear") {
        // sq_linear against the oracle's linear on random blocks:
        // --linear <wtype> <m> <k> <n> <mode>
        const int wt = atoi(argv[2]), m = atoi(argv[3]), k = atoi(argv[4]), n = atoi(argv[5]), md = atoi(argv[6]);
        std::mt19937 rng(7);
        std::normal_distribution<float> nd(0.0f, 1.0f);
        const size_t bb = wt == SQ_Q8_0 ? 34 : (wt == SQ_Q4_0 ? 18 : 64);
        std::vector<uint8_t> w((size_t)n * (k / 32) * bb);
        for (size_t b = 0; b < (size_t)n * (k / 32); b++) {
            uint8_t* p = w.data() + b * bb;
            if (wt == SQ_BF16) {
                for (int i = 0; i < 32; i++) {
                    const float v = nd(rng) * 0.02f;
                    uint32_t u;
                    memcpy(&u, &v, 4);
                    const uint16_t h = (uint16_t)(u >> 16);
                    memcpy(p + 2 * i, &h, 2);
                }
                continue;
            }
            const uint16_t d = or_f32_to_f16(0.001f + 0.002f * (float)(rng() % 1000) / 1000.0f);
            memcpy(p, &d, 2);
            for (size_t i = 2; i < bb; i++) p[i] = (uint8_t)(rng() & 0xFF);
        }
        std::vector<float> x((size_t)m * k);
        for (auto& v : x) v = nd(rng);
        sq_weight* W = nullptr;
        int st = sq_weight_upload(wt, w.data(), n, k, &W);
        if (st) die("sq_weight_upload", st);
        float *dx = nullptr, *dy = nullptr;
        sq_malloc((void**)&dx, x.size() * 4);
        sq_malloc((void**)&dy, (size_t)m * n * 4);
        sq_memcpy_h2d(dx, x.data(), x.size() * 4);
        if ((st = sq_linear(dx, m, k, W, dy, md == 0 ? SQ_CTX_F32_ACTS : 0))) die("sq_linear", st);
        std::vector<float> got((size_t)m * n), want((size_t)m * n);
        sq_memcpy_d2h(got.data(), dy, got.size() * 4);
        or_linear(x.data(), m, k, wt, w.data(), n, want.data(), md);
        double worst = 0;
        int shown = 0;
        for (size_t i = 0; i < got.size(); i++) {
            const double rel = std::fabs((double)got[i] - want[i]) / (std::fabs((double)want[i]) + 1e-3);
            worst = std::fmax(worst, rel);
            if (rel > 1e-2 && shown++ < 8)
                printf("bad row %zu col %zu got %.6g want %.6g\n", i / n, i % n, got[i], want[i]);
        }
        printf("linear wtype %d m %d k %d n %d mode %d worst_rel %.3e got0 %.6g want0 %.6g\n", wt, m, k, n, md, worst,
               got[0], want[0]);
        return 0;
    }
    if (argc == 2 && std::string(argv[1]) == "--noalloc-count") {
        // hipMalloc calls made by warm calls of sq_linear_noalloc on its two
        // paths (m = 1: the matvec; m = 67: the K-split matmul), next to
        // sq_linear's for the same calls
        const int k = 2048, n = 256;
        std::vector<uint8_t> w((size_t)n * (k / 32) * 34);
        for (size_t i = 0; i < w.size(); i++) w[i] = (uint8_t)(i * 131 + 7);
        for (size_t b = 0; b < (size_t)n * (k / 32); b++) {
            const uint16_t d = or_f32_to_f16(0.001f);
            memcpy(w.data() + b * 34, &d, 2);
        }
        sq_weight* W = nullptr;
        int st = sq_weight_upload(SQ_Q8_0, w.data(), n, k, &W);
        if (st) die("sq_weight_upload", st);
        float *dx = nullptr, *dy = nullptr;
        sq_malloc((void**)&dx, (size_t)67 * k * 4);
        sq_malloc((void**)&dy, (size_t)67 * n * 4);
        std::vector<float> x((size_t)67 * k, 0.5f);
        sq_memcpy_h2d(dx, x.data(), x.size() * 4);
        for (int m : {1, 67}) {
            if ((st = sq_linear_noalloc(dx, m, k, W, dy, 0))) die("sq_linear_noalloc", st);  // warm
            const uint64_t a0 = sqemu::g_malloc_calls;
            if ((st = sq_linear_noalloc(dx, m, k, W, dy, 0))) die("sq_linear_noalloc", st);
            const uint64_t a1 = sqemu::g_malloc_calls;
            if ((st = sq_linear(dx, m, k, W, dy, 0))) die("sq_linear", st);
            const uint64_t a2 = sqemu::g_malloc_calls;
            printf("m %d noalloc_mallocs %llu linear_mallocs %llu\n", m, (unsigned long long)(a1 - a0),
                   (unsigned long long)(a2 - a1));
        }
        return 0;
    }
    if (argc == 2 && std::string(argv[1]) == "--embed-guard") {
        // sq_embed with device ids in and past a 64-row Q8_0 table: the
        // in-range call succeeds; an id of 64 or of 2^32 - 1 is SQ_ERR_ARG
        // (the reference panics on the slice index, embedding.rs:43-44),
        // with every read in bounds
        const int rows = 64, k = 64;
        std::vector<uint8_t> w((size_t)rows * (k / 32) * 34, 1);
        sq_weight* W = nullptr;
        int st = sq_weight_upload(SQ_Q8_0, w.data(), rows, k, &W);
        if (st) die("sq_weight_upload", st);
        uint32_t* d_ids = nullptr;
        float* d_out = nullptr;
        sq_malloc((void**)&d_ids, 3 * 4);
        sq_malloc((void**)&d_out, 3 * k * 4);
        const uint32_t cases[3][3] = {{3, 63, 0}, {3, 64, 0}, {0xFFFFFFFFu, 1, 2}};
        for (auto& ids : cases) {
            sq_memcpy_h2d(d_ids, ids, sizeof(ids));
            printf("embed ids %u %u %u status %d\n", ids[0], ids[1], ids[2], sq_embed(d_ids, 3, W, d_out));
        }
        return 0;
    }
    if (argc < 8) {
        fprintf(stderr, "usage: emu_model gguf mode flags n_prompt n_decode seed max_pos [generate]\n");
        return 2;
    }
    const char* path = argv[1];
    const int mode = atoi(argv[2]);
    const uint32_t flags = (uint32_t)strtoul(argv[3], nullptr, 0);
    const int n_prompt = atoi(argv[4]), n_decode = atoi(argv[5]);
    const unsigned seed = (unsigned)atoi(argv[6]);
    const size_t max_pos = (size_t)atoi(argv[7]);
    bool gen = false;
    // corrupt=<step>,<layer>,<site>,<element>,<kind>: before the lock check of
    // that step, change one element of the device's blocks by 2 (kind 0) or
    // one block scale by 1% (kind 1) -- a planted mistake the lock must report
    int cs = -1, cl = 0, csite = 0, ce = 0, ck = 0;
    // plant=<step>,<layer>,<site>,<quanta>: the oracle's planted systematic
    // error (or_lock plant_*): that site's blocks as an implementation whose
    // scaled values are all off by <quanta> would produce them
    int ps = -1, pl = 0, psite = 0;
    float pq = 0.0f;
    float tol = 0.02f;  // tol=<quanta>: the lock's midpoint tolerance
    for (int i = 8; i < argc; i++) {
        const std::string a = argv[i];
        if (a == "generate") gen = true;
        if (a.rfind("corrupt=", 0) == 0) sscanf(a.c_str() + 8, "%d,%d,%d,%d,%d", &cs, &cl, &csite, &ce, &ck);
        if (a.rfind("plant=", 0) == 0) sscanf(a.c_str() + 6, "%d,%d,%d,%f", &ps, &pl, &psite, &pq);
        if (a.rfind("tol=", 0) == 0) tol = strtof(a.c_str() + 4, nullptr);
    }

    sq_model* m = nullptr;
    int st = sq_model_load_gguf(path, &m);
    if (st) die("sq_model_load_gguf", st);
    sq_model_info info;
    sq_model_info_get(m, &info);
    sq_ctx* c = nullptr;
    if ((st = sq_ctx_new(m, max_pos, flags, &c))) die("sq_ctx_new", st);
    printf("decode_kernel %d\n", sq_ctx_decode_kernel(c));

    std::mt19937 rng(seed);
    std::vector<uint32_t> ids(n_prompt + n_decode);
    for (auto& t : ids) t = rng() % info.vocab;

    // oracle model over the same file
    sq::GGUFFile f;
    if ((st = f.open(path))) die("GGUFFile::open", st);
    auto T = [&](const std::string& n) -> const void* {
        int s2 = 0;
        const uint8_t* p = f.tensor_data(n, &s2);
        if (!p) {
            fprintf(stderr, "tensor %s missing\n", n.c_str());
            exit(2);
        }
        return p;
    };
    std::vector<const void*> layer;
    for (uint32_t l = 0; l < info.n_layers; l++) {
        const std::string p = "blk." + std::to_string(l) + ".";
        for (const char* n : {"attn_norm", "attn_q", "attn_k", "attn_v", "attn_output", "ffn_norm", "ffn_gate",
                              "ffn_up", "ffn_down"})
            layer.push_back(T(p + n + ".weight"));
    }
    std::vector<float> inv_freq(info.head_dim / 2);
    sq_model_rope_inv_freq(m, inv_freq.data(), inv_freq.size());
    or_llama om;
    om.n_layers = info.n_layers;
    om.dim = info.dim;
    om.ffn_dim = info.ffn_dim;
    om.n_heads = info.n_heads;
    om.n_kv_heads = info.n_kv_heads;
    om.head_dim = info.head_dim;
    om.vocab = info.vocab;
    om.eps = info.rms_eps;
    om.wtype = info.wtype;
    om.tok_embd = T("token_embd.weight");
    om.output = f.tensors.count("output.weight") ? T("output.weight") : om.tok_embd;
    om.output_norm = (const float*)T("output_norm.weight");
    om.layer = layer.data();
    om.inv_freq = inv_freq.data();
    or_ctx* oc = or_ctx_new(&om, max_pos, mode);
    // the integer path is compared phase-locked: the oracle checks the
    // device's Q8_0 blocks at every quantization site and continues with them
    const bool locked = mode != 0 && info.wtype != SQ_BF16 && !(flags & SQ_CTX_F32_ACTS);
    if (locked && (st = sq_ctx_act_taps(c, 1))) die("sq_ctx_act_taps", st);
    const size_t TW = 2 * (size_t)info.dim + (size_t)info.n_heads * info.head_dim + info.ffn_dim;

    std::vector<float> got(info.vocab);
    for (int step = 0; step <= n_decode; step++) {
        const uint32_t* p = step == 0 ? ids.data() : ids.data() + n_prompt + step - 1;
        const size_t n = step == 0 ? (size_t)n_prompt : 1;
        if (step == 0) sq_gemm_counters(1, nullptr);
        if ((st = sq_forward(m, c, p, n))) die("sq_forward", st);
        if (step == 0) {
            // the prefill's matmul launches: all, K-split, 128 x 128 tiles,
            // most splits, 128 x 64 tiles, few-rows kernel
            uint64_t gc[6];
            sq_gemm_counters(0, gc);
            printf("gemm launches %llu split %llu tile128 %llu max_splits %llu tile128x64 %llu rows %llu\n",
                   (unsigned long long)gc[0], (unsigned long long)gc[1], (unsigned long long)gc[2],
                   (unsigned long long)gc[3], (unsigned long long)gc[4], (unsigned long long)gc[5]);
        }
        if ((st = sq_logits(c, got.data(), got.size()))) die("sq_logits", st);
        uint32_t tok = 0;
        if ((st = sq_argmax(c, &tok))) die("sq_argmax", st);
        or_lock lk;
        memset(&lk, 0, sizeof(lk));
        std::vector<or_block_q8_0> taps;
        if (locked) {
            taps.resize((n * info.n_layers * TW + info.dim) / 32);
            if ((st = sq_ctx_act_tap_read(c, taps.data(), taps.size()))) die("sq_ctx_act_tap_read", st);
            if (step == cs) {
                const size_t site_off[4] = {0, (size_t)info.dim, (size_t)info.dim + info.n_heads * info.head_dim,
                                            2 * (size_t)info.dim + info.n_heads * info.head_dim};
                const size_t el = n * (cl * TW + site_off[csite]) + ce;
                or_block_q8_0& b = taps[el / 32];
                if (ck == 0) b.qs[el % 32] = (int8_t)(b.qs[el % 32] > 0 ? b.qs[el % 32] - 2 : b.qs[el % 32] + 2);
                else b.d = or_f32_to_f16(or_f16_to_f32(b.d) * 1.01f);
            }
            lk.blocks = taps.data();
            lk.tol = tol;
            if (step == ps) {
                lk.plant_layer = pl;
                lk.plant_site = psite;
                lk.plant_quanta = pq;
            }
        }
        if ((st = or_forward_locked(&om, oc, p, n, locked ? &lk : nullptr))) die("or_forward", st);
        if (locked)
            printf("lock step %d values %llu flips %llu scale_flips %llu bad %llu first_bad %d/%d/%zu/%.3g "
                   "max_flip_dist %.3g max_scale_rel %.3g\n",
                   step, (unsigned long long)lk.values, (unsigned long long)lk.flips,
                   (unsigned long long)lk.scale_flips, (unsigned long long)lk.bad, lk.first_bad_layer,
                   lk.first_bad_site, lk.first_bad_index, lk.first_bad_dist, lk.max_flip_dist, lk.max_scale_rel);
        const float* want = or_ctx_logits(oc);
        double num = 0, den = 0, mx = 0;
        for (uint32_t i = 0; i < info.vocab; i++) {
            const double d = (double)got[i] - want[i];
            num += d * d;
            den += (double)want[i] * want[i];
            mx = std::fmax(mx, std::fabs(d));
        }
        std::vector<float> lh(info.dim);
        double hn = 0, hd = 0;
        if (sq_ctx_last_hidden(c, lh.data(), lh.size()) == 0) {
            const float* oh = or_ctx_last_hidden(oc);
            for (uint32_t i = 0; i < info.dim; i++) {
                hn += ((double)lh[i] - oh[i]) * ((double)lh[i] - oh[i]);
                hd += (double)oh[i] * oh[i];
            }
        }
        printf("step %d rel_l2 %.3e max_abs %.3e argmax %u %lld hidden_rel_l2 %.3e\n", step, std::sqrt(num / den), mx,
               tok, (long long)or_greedy(want, info.vocab), hd > 0 ? std::sqrt(hn / hd) : -1.0);
        fflush(stdout);
    }
    if (gen) {
        std::vector<uint32_t> out(n_decode + 1);
        size_t n_out = 0;
        if ((st = sq_generate(m, c, ids.data(), n_prompt, n_decode + 1, SQ_GEN_IGNORE_EOS, out.data(), &n_out,
                              nullptr)))
            die("sq_generate", st);
        printf("generated");
        for (size_t i = 0; i < n_out; i++) printf(" %u", out[i]);
        printf("\n");
        // the oracle's greedy loop over the same prompt (text_generator.rs:58-101)
        or_ctx_reset(oc);
        std::vector<uint32_t> cur(ids.begin(), ids.begin() + n_prompt);
        printf("oracle_generated");
        for (int k = 0; k <= n_decode; k++) {
            if ((st = or_forward(&om, oc, cur.data(), cur.size()))) die("or_forward", st);
            const uint32_t t = (uint32_t)or_greedy(or_ctx_logits(oc), info.vocab);
            printf(" %u", t);
            cur.assign(1, t);
        }
        printf("\n");
    }
    or_ctx_free(oc);
    sq_ctx_free(c);
    sq_model_free(m);
    printf("done\n");
    return 0;
}
