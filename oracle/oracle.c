/*
 * Oracle: CPU restatement of squirrel-rs's Llama token loop.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP implementation and the
 * timed CPU baseline.  Never linked into, loaded by, or called from the
 * product library.
 *
 * Reference citations are file:line in the squirrel-rs repository.
 * Compile with -O2 -ffp-contract=off (no -ffast-math): Rust neither contracts
 * a*b+c into an FMA nor reassociates float folds, and neither may this file.
 */
#define _GNU_SOURCE
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* half 2.7.1: f16::from_f32 / to_f32, bf16::to_f32 (IEEE-754, RNE)          */
/* ------------------------------------------------------------------------ */

uint16_t or_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (exp == 0xffu) {
        if (man == 0) return (uint16_t)(sign | 0x7c00u);
        return (uint16_t)(sign | 0x7e00u | (man >> 13));
    }
    int e = (int)exp - 127 + 15;
    if (e >= 0x1f) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        man |= 0x800000u;
        int shift = 14 - e;
        uint32_t hm = man >> shift;
        uint32_t rem = man & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (hm & 1u))) hm++;
        return (uint16_t)(sign | hm);
    }
    uint32_t h = sign | ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)h;
}

void or_f32_to_f16_array(const float* x, size_t n, uint16_t* out) {
    for (size_t i = 0; i < n; i++) out[i] = or_f32_to_f16(x[i]);
}

float or_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t x;
    if (exp == 0) {
        if (man == 0) {
            x = sign;
        } else {
            int e = -1;
            do { man <<= 1; e++; } while (!(man & 0x400u));
            man &= 0x3ffu;
            x = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 0x1f) {
        x = sign | 0x7f800000u | (man << 13);
    } else {
        x = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

float or_bf16_to_f32(uint16_t b) {
    uint32_t x = (uint32_t)b << 16;
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* ------------------------------------------------------------------------ */
/* Thread pool: stands in for rayon's global pool (src/cli.rs:37-47).        */
/* Parallelism never changes arithmetic: each output element is computed by */
/* exactly one call, as in the reference's par_iter closures.                */
/* ------------------------------------------------------------------------ */

typedef void (*or_task_fn)(void* ctx, size_t begin, size_t end);

static struct {
    pthread_mutex_t mu;
    pthread_cond_t cv_work, cv_done;
    int nthreads;          /* including the caller */
    pthread_t* tids;
    unsigned long gen;
    or_task_fn fn;
    void* ctx;
    size_t n, grain;
    atomic_size_t next;
    int active;            /* workers still running the current job */
    int shutdown;
    int started;
} g_pool = {.mu = PTHREAD_MUTEX_INITIALIZER,
             .cv_work = PTHREAD_COND_INITIALIZER,
             .cv_done = PTHREAD_COND_INITIALIZER,
             .nthreads = 1};

static void pool_run_chunks(void) {
    for (;;) {
        size_t b = atomic_fetch_add(&g_pool.next, g_pool.grain);
        if (b >= g_pool.n) break;
        size_t e = b + g_pool.grain;
        if (e > g_pool.n) e = g_pool.n;
        g_pool.fn(g_pool.ctx, b, e);
    }
}

static void* pool_worker(void* arg) {
    (void)arg;
    unsigned long seen = 0;
    pthread_mutex_lock(&g_pool.mu);
    for (;;) {
        while (g_pool.gen == seen && !g_pool.shutdown) pthread_cond_wait(&g_pool.cv_work, &g_pool.mu);
        if (g_pool.shutdown) break;
        seen = g_pool.gen;
        pthread_mutex_unlock(&g_pool.mu);
        pool_run_chunks();
        pthread_mutex_lock(&g_pool.mu);
        if (--g_pool.active == 0) pthread_cond_signal(&g_pool.cv_done);
    }
    pthread_mutex_unlock(&g_pool.mu);
    return NULL;
}

static void pool_stop(void) {
    if (!g_pool.started) return;
    pthread_mutex_lock(&g_pool.mu);
    g_pool.shutdown = 1;
    pthread_cond_broadcast(&g_pool.cv_work);
    pthread_mutex_unlock(&g_pool.mu);
    for (int i = 0; i < g_pool.nthreads - 1; i++) pthread_join(g_pool.tids[i], NULL);
    free(g_pool.tids);
    g_pool.tids = NULL;
    g_pool.shutdown = 0;
    g_pool.started = 0;
}

int or_set_threads(int n) {
    if (n < 1) n = 1;
    pool_stop();
    g_pool.nthreads = n;
    if (n > 1) {
        g_pool.tids = (pthread_t*)calloc((size_t)n - 1, sizeof(pthread_t));
        for (int i = 0; i < n - 1; i++) pthread_create(&g_pool.tids[i], NULL, pool_worker, NULL);
        g_pool.started = 1;
    }
    return n;
}

int or_get_threads(void) { return g_pool.nthreads; }

static void parallel_for(size_t n, size_t grain, or_task_fn fn, void* ctx) {
    if (n == 0) return;
    if (grain == 0) grain = 1;
    if (g_pool.nthreads <= 1 || n <= grain) {
        fn(ctx, 0, n);
        return;
    }
    pthread_mutex_lock(&g_pool.mu);
    g_pool.fn = fn;
    g_pool.ctx = ctx;
    g_pool.n = n;
    g_pool.grain = grain;
    atomic_store(&g_pool.next, 0);
    g_pool.active = g_pool.nthreads - 1;
    g_pool.gen++;
    pthread_cond_broadcast(&g_pool.cv_work);
    pthread_mutex_unlock(&g_pool.mu);
    pool_run_chunks();
    pthread_mutex_lock(&g_pool.mu);
    while (g_pool.active > 0) pthread_cond_wait(&g_pool.cv_done, &g_pool.mu);
    pthread_mutex_unlock(&g_pool.mu);
}

/* ------------------------------------------------------------------------ */
/* dot_prod.rs                                                              */
/* ------------------------------------------------------------------------ */

/* quantize_row_q8_0_scalar, src/kernels/dot_prod.rs:21-31.
 * amax folds from 0 with f32::max (NaN ignored); scale = amax/127;
 * inv = scale > 0 ? 1/scale : 0; d = f16(scale) (RNE);
 * q = (x*inv).round().clamp(-127,127) as i8, where round is half away from
 * zero, clamp keeps NaN, and `NaN as i8` is 0. */
void or_quantize_row_q8_0(const float* src, size_t n, or_block_q8_0* out) {
    size_t nb = n / 32;
    for (size_t b = 0; b < nb; b++) {
        const float* x = src + b * 32;
        float amax = 0.0f;
        for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(x[i]));
        float scale = amax / 127.0f;
        float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
        out[b].d = or_f32_to_f16(scale);
        for (int i = 0; i < 32; i++) {
            float v = roundf(x[i] * inv);
            if (v < -127.0f) v = -127.0f;
            if (v > 127.0f) v = 127.0f;
            out[b].qs[i] = isnan(v) ? (int8_t)0 : (int8_t)v;
        }
    }
}

/* dot_f32_q8_0_fallback, src/kernels/dot_prod.rs:86-96. */
float or_dot_f32_q8_0(const float* a, const or_block_q8_0* b, size_t nblocks) {
    float acc = 0.0f;
    for (size_t blk = 0; blk < nblocks; blk++) {
        const float* chunk = a + blk * 32;
        float block_acc = 0.0f;
        for (int i = 0; i < 32; i++) block_acc += chunk[i] * (float)b[blk].qs[i];
        acc += block_acc * or_f16_to_f32(b[blk].d);
    }
    return acc;
}

/* dot_f32_q4_0_fallback, src/kernels/dot_prod.rs:255-270.  The two products
 * are summed first, then added to block_acc. */
float or_dot_f32_q4_0(const float* a, const or_block_q4_0* b, size_t nblocks) {
    float acc = 0.0f;
    for (size_t blk = 0; blk < nblocks; blk++) {
        const float* chunk = a + blk * 32;
        float block_acc = 0.0f;
        for (int j = 0; j < 16; j++) {
            uint8_t byte = b[blk].qs[j];
            int lo = (int)(byte & 0x0F) - 8;
            int hi = (int)(byte >> 4) - 8;
            float t = chunk[j] * (float)lo + chunk[j + 16] * (float)hi;
            block_acc += t;
        }
        acc += block_acc * or_f16_to_f32(b[blk].d);
    }
    return acc;
}

/* dot_f32_bf16_fallback, src/kernels/dot_prod.rs:464-472: one running sum. */
float or_dot_f32_bf16(const float* a, const uint16_t* b, size_t n) {
    float acc = 0.0f;
    for (size_t i = 0; i < n; i++) acc += a[i] * or_bf16_to_f32(b[i]);
    return acc;
}

int32_t or_isum_q8_0_q8_0(const or_block_q8_0* a, const or_block_q8_0* b) {
    int32_t isum = 0;
    for (int i = 0; i < 32; i++) isum += (int32_t)a->qs[i] * (int32_t)b->qs[i];
    return isum;
}

int32_t or_isum_q8_0_q4_0(const or_block_q8_0* a, const or_block_q4_0* b) {
    int32_t isum = 0;
    for (int j = 0; j < 16; j++) {
        uint8_t byte = b->qs[j];
        int32_t lo = (int32_t)(byte & 0x0F) - 8;
        int32_t hi = (int32_t)(byte >> 4) - 8;
        isum += (int32_t)a->qs[j] * lo + (int32_t)a->qs[j + 16] * hi;
    }
    return isum;
}

/* dot_q8_0_q8_0_scalar, src/kernels/dot_prod.rs:378-388:
 * total += (isum as f32 * sa) * sb, with sa the activation scale. */
float or_dot_q8_0_q8_0(const or_block_q8_0* a, const or_block_q8_0* b, size_t nblocks) {
    float total = 0.0f;
    for (size_t blk = 0; blk < nblocks; blk++) {
        int32_t isum = or_isum_q8_0_q8_0(&a[blk], &b[blk]);
        float t = (float)isum * or_f16_to_f32(a[blk].d);
        t = t * or_f16_to_f32(b[blk].d);
        total += t;
    }
    return total;
}

/* dot_q8_0_q4_0_scalar, src/kernels/dot_prod.rs:391-403. */
float or_dot_q8_0_q4_0(const or_block_q8_0* a, const or_block_q4_0* b, size_t nblocks) {
    float total = 0.0f;
    for (size_t blk = 0; blk < nblocks; blk++) {
        int32_t isum = or_isum_q8_0_q4_0(&a[blk], &b[blk]);
        float t = (float)isum * or_f16_to_f32(a[blk].d);
        t = t * or_f16_to_f32(b[blk].d);
        total += t;
    }
    return total;
}

/* The combine order of the aarch64 NEON kernels (dot_prod.rs:189-252 and
 * 306-374, with the `dotprod` feature).  Each block yields four i32 lanes;
 * lane l sums elements {4l..4l+3} and {16+4l..16+4l+3} (two SDOTs,
 * :174-175, :291-292).  Block i+j of each group of four feeds accumulator j;
 * leftover blocks feed accumulator 0.  acc = fma(acc, f32(lane), sa*sb).
 * The end is vaddvq_f32((g0+g1)+(g2+g3)) = (v0+v1)+(v2+v3). */
static void neon_lanes_q8(const or_block_q8_0* a, const int8_t* w, int32_t lanes[4]) {
    for (int l = 0; l < 4; l++) {
        int32_t s = 0;
        for (int i = 0; i < 4; i++) s += (int32_t)a->qs[4 * l + i] * (int32_t)w[4 * l + i];
        for (int i = 0; i < 4; i++) s += (int32_t)a->qs[16 + 4 * l + i] * (int32_t)w[16 + 4 * l + i];
        lanes[l] = s;
    }
}

static float neon_combine(const or_block_q8_0* a, size_t nblocks, const void* w, int q4) {
    float g[4][4];
    memset(g, 0, sizeof g);
    for (size_t i = 0; i < nblocks; i++) {
        int8_t wq[32];
        uint16_t wd;
        if (q4) {
            const or_block_q4_0* b = (const or_block_q4_0*)w + i;
            for (int j = 0; j < 16; j++) {
                wq[j] = (int8_t)((b->qs[j] & 0x0F) - 8);
                wq[j + 16] = (int8_t)((b->qs[j] >> 4) - 8);
            }
            wd = b->d;
        } else {
            const or_block_q8_0* b = (const or_block_q8_0*)w + i;
            memcpy(wq, b->qs, 32);
            wd = b->d;
        }
        int32_t lanes[4];
        neon_lanes_q8(&a[i], wq, lanes);
        float s = or_f16_to_f32(a[i].d) * or_f16_to_f32(wd);
        size_t acc = (i < (nblocks / 4) * 4) ? (i % 4) : 0;
        for (int l = 0; l < 4; l++) g[acc][l] = fmaf((float)lanes[l], s, g[acc][l]);
    }
    float v[4];
    for (int l = 0; l < 4; l++) v[l] = (g[0][l] + g[1][l]) + (g[2][l] + g[3][l]);
    return (v[0] + v[1]) + (v[2] + v[3]);
}

float or_dot_q8_0_q8_0_neon(const or_block_q8_0* a, const or_block_q8_0* b, size_t nblocks) {
    return neon_combine(a, nblocks, b, 0);
}

float or_dot_q8_0_q4_0_neon(const or_block_q8_0* a, const or_block_q4_0* b, size_t nblocks) {
    return neon_combine(a, nblocks, b, 1);
}

/* dot_f32_f32, src/kernels/dot_prod.rs:540-549. */
int or_dot_f32_f32(const float* a, size_t na, const float* b, size_t nb, float* out) {
    if (na != nb) return OR_SHAPE;
    float acc = 0.0f;
    for (size_t i = 0; i < na; i++) acc += a[i] * b[i];
    *out = acc;
    return OR_OK;
}

/* WeightBlock::dequantize_into for each block type
 * (src/kernels/dot_prod.rs:409-414, 440-446, 524-528). */
void or_dequantize_row(int wtype, const void* blocks, size_t n, float* out) {
    size_t nb = n / 32;
    for (size_t b = 0; b < nb; b++) {
        float* o = out + b * 32;
        if (wtype == OR_Q8_0) {
            const or_block_q8_0* blk = (const or_block_q8_0*)blocks + b;
            float s = or_f16_to_f32(blk->d);
            for (int i = 0; i < 32; i++) o[i] = s * (float)blk->qs[i];
        } else if (wtype == OR_Q4_0) {
            const or_block_q4_0* blk = (const or_block_q4_0*)blocks + b;
            float s = or_f16_to_f32(blk->d);
            for (int j = 0; j < 16; j++) {
                o[j] = s * (float)((int)(blk->qs[j] & 0x0F) - 8);
                o[j + 16] = s * (float)((int)(blk->qs[j] >> 4) - 8);
            }
        } else {
            const uint16_t* v = (const uint16_t*)blocks + b * 32;
            for (int i = 0; i < 32; i++) o[i] = or_bf16_to_f32(v[i]);
        }
    }
}

/* ------------------------------------------------------------------------ */
/* matmul.rs + ops/linear.rs                                                */
/* ------------------------------------------------------------------------ */

static size_t row_bytes(int wtype, size_t k) {
    if (wtype == OR_Q8_0) return (k / 32) * 34;
    if (wtype == OR_Q4_0) return (k / 32) * 18;
    return k * 2;
}

/* One job covers m rows x n_out columns; task index i is output (i / n_out,
 * i % n_out).  The reference walks rows serially and columns in parallel
 * (src/kernels/matmul.rs:28-64); every output element is one independent dot
 * product either way, so spreading rows over the pool too changes no bit. */
typedef struct {
    const float* in;               /* f32 activations [m][k] (W8A32 / BF16) */
    const or_block_q8_0* aq;       /* quantized activations [m][k/32] (W8A8) */
    const uint8_t* w;
    size_t k, rb, n_out;
    int wtype, mode;
    float* out;
} linear_job;

static void linear_task(void* p, size_t begin, size_t end) {
    const linear_job* j = (const linear_job*)p;
    size_t nb = j->k / 32;
    for (size_t i = begin; i < end; i++) {
        const size_t r = i / j->n_out, c = i % j->n_out;
        const float* a_row = j->in ? j->in + r * j->k : NULL;
        const or_block_q8_0* aq_row = j->aq ? j->aq + r * nb : NULL;
        const uint8_t* wr = j->w + c * j->rb;
        float v;
        if (j->wtype == OR_BF16) {
            v = or_dot_f32_bf16(a_row, (const uint16_t*)wr, j->k);
        } else if (j->mode == OR_W8A32) {
            v = (j->wtype == OR_Q8_0) ? or_dot_f32_q8_0(a_row, (const or_block_q8_0*)wr, nb)
                                      : or_dot_f32_q4_0(a_row, (const or_block_q4_0*)wr, nb);
        } else if (j->mode == OR_W8A8) {
            v = (j->wtype == OR_Q8_0) ? or_dot_q8_0_q8_0(aq_row, (const or_block_q8_0*)wr, nb)
                                      : or_dot_q8_0_q4_0(aq_row, (const or_block_q4_0*)wr, nb);
        } else {
            v = (j->wtype == OR_Q8_0) ? or_dot_q8_0_q8_0_neon(aq_row, (const or_block_q8_0*)wr, nb)
                                      : or_dot_q8_0_q4_0_neon(aq_row, (const or_block_q4_0*)wr, nb);
        }
        j->out[r * j->n_out + c] = v;
    }
}

/* linear -> linear_blocks -> matmul_f32_q / matmul_prequant_q
 * (src/ops/linear.rs:26-70, src/kernels/matmul.rs:7-24,68-171).
 * Quantized activations are formed for all rows first (matmul.rs:91-98). */
static int linear_rows(const float* in, const or_block_q8_0* aq, size_t m, size_t k, int wtype,
                       const void* w, size_t n_out, float* out, int mode) {
    linear_job j;
    j.in = in;
    j.aq = aq;
    j.n_out = n_out;
    j.out = out;
    j.w = (const uint8_t*)w;
    j.k = k;
    j.rb = row_bytes(wtype, k);
    j.wtype = wtype;
    j.mode = mode;
    parallel_for(m * n_out, 64, linear_task, &j);
    return OR_OK;
}

int or_linear(const float* in, size_t m, size_t k, int wtype, const void* w, size_t n_out,
              float* out, int mode) {
    if (wtype != OR_Q8_0 && wtype != OR_Q4_0 && wtype != OR_BF16) return OR_INVALID_TYPE;
    if (k % 32 != 0) return OR_SHAPE;
    int int_acts = (wtype != OR_BF16) && mode != OR_W8A32;
    or_block_q8_0* aq = NULL;
    if (int_acts) {
        aq = (or_block_q8_0*)malloc(sizeof(or_block_q8_0) * (m * k / 32 + 1));
        or_quantize_row_q8_0(in, m * k, aq);
    }
    int st = linear_rows(in, aq, m, k, wtype, w, n_out, out, mode);
    free(aq);
    return st;
}

/* matmul_prequant_q (src/kernels/matmul.rs:133-171): activations already
 * quantized (linear_shared quantizes once per projection group,
 * src/ops/linear.rs:117-127). */
int or_linear_prequant(const or_block_q8_0* aq, size_t m, size_t k, int wtype, const void* w,
                       size_t n_out, float* out, int mode) {
    if (wtype != OR_Q8_0 && wtype != OR_Q4_0) return OR_INVALID_TYPE;
    if (k % 32 != 0 || mode == OR_W8A32) return OR_SHAPE;
    return linear_rows(NULL, aq, m, k, wtype, w, n_out, out, mode);
}

int or_block_isums(const or_block_q8_0* a, int wtype, const void* w_row, size_t nblocks,
                   int32_t* isums) {
    if (wtype == OR_Q8_0) {
        for (size_t b = 0; b < nblocks; b++)
            isums[b] = or_isum_q8_0_q8_0(&a[b], (const or_block_q8_0*)w_row + b);
        return OR_OK;
    }
    if (wtype == OR_Q4_0) {
        for (size_t b = 0; b < nblocks; b++)
            isums[b] = or_isum_q8_0_q4_0(&a[b], (const or_block_q4_0*)w_row + b);
        return OR_OK;
    }
    return OR_INVALID_TYPE;
}

/* ------------------------------------------------------------------------ */
/* softmax.rs, rms_norm.rs, rope.rs, sigmoid.rs, silu.rs                    */
/* ------------------------------------------------------------------------ */

/* softmax_f32, src/kernels/softmax.rs:4-27. */
int or_softmax(const float* a, float* out, size_t n) {
    if (n == 0) return OR_EMPTY;
    float max = -INFINITY;
    for (size_t i = 0; i < n; i++) max = fmaxf(max, a[i]);
    float sum = 0.0f;
    for (size_t i = 0; i < n; i++) {
        out[i] = expf(a[i] - max);
        sum += out[i];
    }
    float inv = 1.0f / sum;
    for (size_t i = 0; i < n; i++) out[i] *= inv;
    return OR_OK;
}

/* rms_norm over rows -> rms_norm_f32_into, src/ops/rms_norm.rs:13-43,
 * src/kernels/rms_norm.rs:40-56: sequential sum of squares, then
 * y = (x*w)/sqrt(ss/n + eps) (a division, not a reciprocal multiply). */
int or_rms_norm_rows(const float* in, const float* w, float* out, size_t rows, size_t dim,
                     float eps) {
    if (dim == 0) return OR_SHAPE;
    for (size_t r = 0; r < rows; r++) {
        const float* x = in + r * dim;
        float* y = out + r * dim;
        float ss = 0.0f;
        for (size_t i = 0; i < dim; i++) ss += x[i] * x[i];
        float mean = ss / (float)dim;
        float rms = sqrtf(mean + eps);
        for (size_t i = 0; i < dim; i++) y[i] = (x[i] * w[i]) / rms;
    }
    return OR_OK;
}

/* rope_rows -> rope_f32_interleaved, src/ops/rope.rs:6-32,
 * src/kernels/rope.rs:7-36.  Row i uses position base_pos + i; each head
 * rotates adjacent pairs (x[2j], x[2j+1]) by theta = f32(pos) * inv_freq[j]. */
int or_rope_rows(float* t, size_t rows, size_t row_dim, size_t base_pos, const float* inv_freq,
                 size_t half) {
    size_t head_dim = 2 * half;
    if (head_dim == 0 || row_dim % head_dim != 0) return OR_SHAPE;
    if (row_dim == 0) return OR_EMPTY;
    for (size_t r = 0; r < rows; r++) {
        float pos = (float)(base_pos + r);
        float* row = t + r * row_dim;
        for (size_t h = 0; h < row_dim / head_dim; h++) {
            float* head = row + h * head_dim;
            for (size_t j = 0; j < half; j++) {
                float theta = pos * inv_freq[j];
                float s = sinf(theta), c = cosf(theta);
                float a = head[2 * j], b = head[2 * j + 1];
                head[2 * j] = a * c - b * s;
                head[2 * j + 1] = a * s + b * c;
            }
        }
    }
    return OR_OK;
}

/* sigmoid_f32, src/kernels/sigmoid.rs:2-9. */
float or_sigmoid(float x) {
    if (x >= 0.0f) return 1.0f / (1.0f + expf(-x));
    float z = expf(x);
    return z / (1.0f + z);
}

/* silu_f32, src/kernels/silu.rs:4-8. */
void or_silu(float* x, size_t n) {
    for (size_t i = 0; i < n; i++) x[i] = x[i] * or_sigmoid(x[i]);
}

/* compute_rope_inv_freq, src/models/llama/config.rs:83-127. */
void or_rope_inv_freq(size_t head_dim, float base, float factor, float low, float high,
                      float orig_ctx, float* out) {
    size_t half = head_dim / 2;
    float inv_head_dim = 1.0f / (float)head_dim;
    for (size_t j = 0; j < half; j++) {
        float e = -2.0f * (float)j;
        e = e * inv_head_dim;
        out[j] = powf(base, e);
    }
    const float two_pi = 6.28318530717958647692f;
    float low_wl = orig_ctx / low;
    float high_wl = orig_ctx / high;
    for (size_t j = 0; j < half; j++) {
        float f = out[j];
        float wavelen = two_pi / f;
        if (wavelen > low_wl) {
            out[j] = f / factor;
        } else if (wavelen >= high_wl) {
            float smooth = (orig_ctx / wavelen - low) / (high - low);
            float a = (1.0f - smooth) * (f / factor);
            float b = smooth * f;
            out[j] = a + b;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* attention.rs                                                             */
/* ------------------------------------------------------------------------ */

typedef struct {
    const float *q, *k, *v;
    float* out;
    size_t seq_q, seq_k, n_heads, n_kv_heads, head_dim, offset, group;
    float scale;
} sdpa_job;

static void sdpa_task(void* p, size_t begin, size_t end) {
    const sdpa_job* j = (const sdpa_job*)p;
    size_t live_max = j->seq_k;
    float* scores = (float*)malloc(sizeof(float) * (live_max ? live_max : 1));
    float* probs = (float*)malloc(sizeof(float) * (live_max ? live_max : 1));
    for (size_t idx = begin; idx < end; idx++) {
        size_t t = idx / j->n_heads, h = idx % j->n_heads;
        size_t kv_h = h / j->group;
        size_t live = j->offset + t + 1;
        const float* q_row = j->q + (t * j->n_heads + h) * j->head_dim;
        for (size_t s = 0; s < live; s++) {
            const float* k_row = j->k + (s * j->n_kv_heads + kv_h) * j->head_dim;
            float d;
            or_dot_f32_f32(q_row, j->head_dim, k_row, j->head_dim, &d);
            scores[s] = d * j->scale;
        }
        or_softmax(scores, probs, live);
        float* o = j->out + idx * j->head_dim;
        for (size_t d = 0; d < j->head_dim; d++) o[d] = 0.0f;
        for (size_t s = 0; s < live; s++) {
            const float* v_row = j->v + (s * j->n_kv_heads + kv_h) * j->head_dim;
            float pr = probs[s];
            for (size_t d = 0; d < j->head_dim; d++) o[d] += pr * v_row[d];
        }
    }
    free(scores);
    free(probs);
}

/* sdpa_f32, src/kernels/attention.rs:11-70: causal GQA; query t attends to
 * keys 0..=offset+t with offset = seq_k - seq_q; kv head = h / (n_heads /
 * n_kv_heads); scale = 1/sqrt(head_dim). */
int or_sdpa(const float* q, const float* k, const float* v, float* out, size_t seq_q,
            size_t seq_k, size_t n_heads, size_t n_kv_heads, size_t head_dim) {
    if (n_kv_heads == 0 || n_heads % n_kv_heads != 0) return OR_SHAPE;
    if (seq_k < seq_q) return OR_SHAPE;
    sdpa_job j = {q, k, v, out, seq_q, seq_k, n_heads, n_kv_heads, head_dim, seq_k - seq_q,
                  n_heads / n_kv_heads, 1.0f / sqrtf((float)head_dim)};
    parallel_for(seq_q * n_heads, 1, sdpa_task, &j);
    return OR_OK;
}

/* ------------------------------------------------------------------------ */
/* samplers/greedy.rs                                                       */
/* ------------------------------------------------------------------------ */

/* GreedySampler::sample, src/samplers/greedy.rs:6-15: Iterator::max_by with
 * partial_cmp and NaN treated as Equal.  max_by keeps the later element
 * unless the running best compares Greater, so ties go to the last index and
 * any NaN comparison hands the lead to the later element. */
int64_t or_greedy(const float* logits, size_t n) {
    if (n == 0) return -1;
    size_t best = 0;
    for (size_t i = 1; i < n; i++) {
        float a = logits[best], b = logits[i];
        int greater = (!isnan(a) && !isnan(b) && a > b);
        if (!greater) best = i;
    }
    return (int64_t)best;
}

/* ------------------------------------------------------------------------ */
/* embedding.rs                                                             */
/* ------------------------------------------------------------------------ */

/* embed / embed_blocks, src/ops/embedding.rs:10-52. */
int or_embed(const uint32_t* tokens, size_t n_tokens, int wtype, const void* table,
             size_t embed_dim, size_t vocab, float* out) {
    if (wtype != OR_Q8_0 && wtype != OR_Q4_0 && wtype != OR_BF16) return OR_INVALID_TYPE;
    if (embed_dim % 32 != 0) return OR_SHAPE;
    size_t rb = row_bytes(wtype, embed_dim);
    for (size_t t = 0; t < n_tokens; t++) {
        if (tokens[t] >= vocab) return OR_SHAPE;
        const uint8_t* row = (const uint8_t*)table + (size_t)tokens[t] * rb;
        or_dequantize_row(wtype, row, embed_dim, out + t * embed_dim);
    }
    return OR_OK;
}

/* ------------------------------------------------------------------------ */
/* models/llama: Llama3_2::forward (src/models/llama/model.rs:45-97),       */
/* layers::{attention, ffn, block} (src/models/llama/layers.rs:24-109),     */
/* KvCache (src/models/common/kv_cache.rs:8-79).                            */
/* ------------------------------------------------------------------------ */

struct or_ctx {
    size_t max_pos, seq_len, cap_rows;
    int mode;
    float** k;  /* per layer [max_pos, kv_dim] */
    float** v;
    int n_layers;
    /* workspace (src/models/common/workspace.rs:10-50) */
    float *hidden, *normed, *q, *kk, *vv, *attn, *attn_out, *gate, *up, *ffn_act, *ffn_out;
    float *last_hidden, *logits;
    or_block_q8_0* aq; /* quantized activations of one site (rows x widest k / 32) */
};

or_ctx* or_ctx_new(const or_llama* m, size_t max_positions, int mode) {
    or_ctx* c = (or_ctx*)calloc(1, sizeof(or_ctx));
    size_t kv_dim = (size_t)m->n_kv_heads * m->head_dim;
    c->max_pos = max_positions;
    c->mode = mode;
    c->n_layers = m->n_layers;
    c->k = (float**)calloc((size_t)m->n_layers, sizeof(float*));
    c->v = (float**)calloc((size_t)m->n_layers, sizeof(float*));
    for (int l = 0; l < m->n_layers; l++) {
        c->k[l] = (float*)malloc(sizeof(float) * max_positions * kv_dim);
        c->v[l] = (float*)malloc(sizeof(float) * max_positions * kv_dim);
    }
    c->last_hidden = (float*)calloc((size_t)m->dim, sizeof(float));
    c->logits = (float*)calloc((size_t)m->vocab, sizeof(float));
    return c;
}

static void ctx_prepare(or_ctx* c, const or_llama* m, size_t seq) {
    if (seq <= c->cap_rows) return;
    size_t q_dim = (size_t)m->n_heads * m->head_dim, kv_dim = (size_t)m->n_kv_heads * m->head_dim;
    float** bufs[] = {&c->hidden, &c->normed, &c->q, &c->kk, &c->vv, &c->attn,
                      &c->attn_out, &c->gate, &c->up, &c->ffn_act, &c->ffn_out};
    size_t widths[] = {(size_t)m->dim, (size_t)m->dim, q_dim, kv_dim, kv_dim, q_dim,
                       (size_t)m->dim, (size_t)m->ffn_dim, (size_t)m->ffn_dim,
                       (size_t)m->ffn_dim, (size_t)m->dim};
    for (int i = 0; i < 11; i++) {
        free(*bufs[i]);
        *bufs[i] = (float*)calloc(seq * widths[i], sizeof(float));
    }
    size_t kmax = (size_t)m->ffn_dim > q_dim ? (size_t)m->ffn_dim : q_dim;
    if ((size_t)m->dim > kmax) kmax = (size_t)m->dim;
    free(c->aq);
    c->aq = (or_block_q8_0*)calloc(seq * kmax / 32 + 1, sizeof(or_block_q8_0));
    c->cap_rows = seq;
}

void or_ctx_free(or_ctx* c) {
    if (!c) return;
    for (int l = 0; l < c->n_layers; l++) {
        free(c->k[l]);
        free(c->v[l]);
    }
    free(c->k);
    free(c->v);
    float* bufs[] = {c->hidden, c->normed, c->q, c->kk, c->vv, c->attn, c->attn_out,
                     c->gate, c->up, c->ffn_act, c->ffn_out, c->last_hidden, c->logits};
    for (int i = 0; i < 13; i++) free(bufs[i]);
    free(c->aq);
    free(c);
}

void or_ctx_reset(or_ctx* c) { c->seq_len = 0; }
size_t or_ctx_seq_len(const or_ctx* c) { return c->seq_len; }
const float* or_ctx_logits(const or_ctx* c) { return c->logits; }
const float* or_ctx_last_hidden(const or_ctx* c) { return c->last_hidden; }

/* Phase lock (see oracle.h): compare the device's blocks of one site with
 * the oracle's own, count, and continue with the device's. */
static void lock_site(or_lock* lk, const float* x, size_t rows, size_t k, or_block_q8_0* own,
                      const or_block_q8_0* dev_in, int layer, int site) {
    size_t nb = rows * k / 32;
    or_block_q8_0* planted = NULL;
    const or_block_q8_0* dev = dev_in;
    if (lk->plant_quanta != 0.0f && layer == lk->plant_layer && site == lk->plant_site) {
        /* the planted error: this site's blocks as an implementation whose
         * scaled values are all off by plant_quanta would produce them */
        planted = (or_block_q8_0*)malloc(nb * sizeof(or_block_q8_0));
        for (size_t b = 0; b < nb; b++) {
            const float* xb = x + b * 32;
            float amax = 0.0f;
            for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(xb[i]));
            float scale = amax / 127.0f;
            float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
            planted[b].d = own[b].d;
            for (int i = 0; i < 32; i++) {
                float v = roundf(xb[i] * inv + lk->plant_quanta);
                v = fminf(127.0f, fmaxf(-127.0f, v));
                planted[b].qs[i] = isnan(v) ? (int8_t)0 : (int8_t)v;
            }
        }
        dev = planted;
    }
    const int kind = site < 5 ? site : 4;
    lk->site_values[kind] += nb * 32;
    for (size_t b = 0; b < nb; b++) {
        const float* xb = x + b * 32;
        lk->values += 32;
        if (own[b].d == dev[b].d && memcmp(own[b].qs, dev[b].qs, 32) == 0) continue;
        float amax = 0.0f;
        for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(xb[i]));
        float scale = amax / 127.0f;
        float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
        int ok = 1;
        size_t bad_i = 0;
        float bad_dist = 0.0f;
        if (own[b].d != dev[b].d) {
            /* adjacent binary16 values of one sign, and the oracle's f32 scale
             * at their rounding midpoint */
            int adjacent = ((own[b].d ^ dev[b].d) & 0x8000) == 0 &&
                           (own[b].d > dev[b].d ? own[b].d - dev[b].d : dev[b].d - own[b].d) == 1;
            float mid = 0.5f * (or_f16_to_f32(own[b].d) + or_f16_to_f32(dev[b].d));
            float rel = fabsf(scale - mid) / fabsf(mid);
            if (!adjacent || !(rel <= 1e-5f)) {
                ok = 0;
                bad_i = b * 32;
                bad_dist = -1.0f;
            } else {
                lk->scale_flips++;
                if (rel > lk->max_scale_rel) lk->max_scale_rel = rel;
            }
        }
        uint64_t flips = 0;
        float maxd = 0.0f;
        for (int i = 0; i < 32 && ok; i++) {
            int qo = own[b].qs[i], qd = dev[b].qs[i];
            if (qo == qd) continue;
            float v = fabsf(xb[i] * inv);
            float dist = fabsf((v - floorf(v)) - 0.5f);
            if ((qo - qd == 1 || qd - qo == 1) && dist <= lk->tol) {
                flips++;
                if (dist > maxd) maxd = dist;
            } else {
                ok = 0;
                bad_i = b * 32 + (size_t)i;
                bad_dist = dist;
            }
        }
        if (!ok) {
            if (lk->bad == 0) {
                lk->first_bad_layer = layer;
                lk->first_bad_site = site;
                lk->first_bad_index = bad_i;
                lk->first_bad_dist = bad_dist;
            }
            lk->bad++;
        } else {
            lk->flips += flips;
            lk->site_flips[kind] += flips;
            if (maxd > lk->max_flip_dist) lk->max_flip_dist = maxd;
        }
        own[b] = dev[b];
    }
    free(planted);
}

/* The quantized activations of one site: the oracle's own, or under a lock
 * the device's after the check; dev advances past the site's blocks. */
static const or_block_q8_0* site_blocks(or_ctx* c, const float* x, size_t rows, size_t k, or_lock* lk,
                                        const or_block_q8_0** dev, int layer, int site) {
    or_quantize_row_q8_0(x, rows * k, c->aq);
    if (lk) {
        lock_site(lk, x, rows, k, c->aq, *dev, layer, site);
        *dev += rows * k / 32;
    }
    return c->aq;
}

int or_forward(const or_llama* m, or_ctx* c, const uint32_t* ids, size_t n) {
    return or_forward_locked(m, c, ids, n, NULL);
}

int or_forward_locked(const or_llama* m, or_ctx* c, const uint32_t* ids, size_t n, or_lock* lock) {
    if (n == 0) return OR_EMPTY;
    if (c->seq_len + n > c->max_pos) return 5;
    size_t D = (size_t)m->dim, F = (size_t)m->ffn_dim, hd = (size_t)m->head_dim;
    size_t q_dim = (size_t)m->n_heads * hd, kv_dim = (size_t)m->n_kv_heads * hd;
    int mode = c->mode, wt = m->wtype;
    int int_acts = wt != OR_BF16 && mode != OR_W8A32;
    int st;
    if (lock && !int_acts) return OR_INVALID_TYPE;
    const or_block_q8_0* dev = lock ? lock->blocks : NULL;
    ctx_prepare(c, m, n);
    st = or_embed(ids, n, wt, m->tok_embd, D, (size_t)m->vocab, c->hidden);
    if (st) return st;
    size_t position = c->seq_len;
    for (int l = 0; l < m->n_layers; l++) {
        const void* const* L = m->layer + 9 * l;
        /* attention half (layers.rs:89-96) */
        or_rms_norm_rows(c->hidden, (const float*)L[0], c->normed, n, D, m->eps);
        /* linear_shared over q,k,v: the input is quantized once
         * (linear.rs:117-127) */
        if (int_acts) {
            const or_block_q8_0* a = site_blocks(c, c->normed, n, D, lock, &dev, l, 0);
            if ((st = or_linear_prequant(a, n, D, wt, L[1], q_dim, c->q, mode))) return st;
            if ((st = or_linear_prequant(a, n, D, wt, L[2], kv_dim, c->kk, mode))) return st;
            if ((st = or_linear_prequant(a, n, D, wt, L[3], kv_dim, c->vv, mode))) return st;
        } else {
            if ((st = or_linear(c->normed, n, D, wt, L[1], q_dim, c->q, mode))) return st;
            if ((st = or_linear(c->normed, n, D, wt, L[2], kv_dim, c->kk, mode))) return st;
            if ((st = or_linear(c->normed, n, D, wt, L[3], kv_dim, c->vv, mode))) return st;
        }
        or_rope_rows(c->q, n, q_dim, position, m->inv_freq, hd / 2);
        or_rope_rows(c->kk, n, kv_dim, position, m->inv_freq, hd / 2);
        memcpy(c->k[l] + position * kv_dim, c->kk, sizeof(float) * n * kv_dim);
        memcpy(c->v[l] + position * kv_dim, c->vv, sizeof(float) * n * kv_dim);
        st = or_sdpa(c->q, c->k[l], c->v[l], c->attn, n, position + n, (size_t)m->n_heads,
                     (size_t)m->n_kv_heads, hd);
        if (st) return st;
        if (int_acts) {
            const or_block_q8_0* a = site_blocks(c, c->attn, n, q_dim, lock, &dev, l, 1);
            if ((st = or_linear_prequant(a, n, q_dim, wt, L[4], D, c->attn_out, mode))) return st;
        } else if ((st = or_linear(c->attn, n, q_dim, wt, L[4], D, c->attn_out, mode))) {
            return st;
        }
        for (size_t i = 0; i < n * D; i++) c->hidden[i] += c->attn_out[i];
        /* FFN half (layers.rs:98-106, 64-77) */
        or_rms_norm_rows(c->hidden, (const float*)L[5], c->normed, n, D, m->eps);
        if (int_acts) {
            const or_block_q8_0* a = site_blocks(c, c->normed, n, D, lock, &dev, l, 2);
            if ((st = or_linear_prequant(a, n, D, wt, L[6], F, c->gate, mode))) return st;
            if ((st = or_linear_prequant(a, n, D, wt, L[7], F, c->up, mode))) return st;
        } else {
            if ((st = or_linear(c->normed, n, D, wt, L[6], F, c->gate, mode))) return st;
            if ((st = or_linear(c->normed, n, D, wt, L[7], F, c->up, mode))) return st;
        }
        or_silu(c->gate, n * F);
        for (size_t i = 0; i < n * F; i++) c->ffn_act[i] = c->gate[i] * c->up[i];
        if (int_acts) {
            const or_block_q8_0* a = site_blocks(c, c->ffn_act, n, F, lock, &dev, l, 3);
            if ((st = or_linear_prequant(a, n, F, wt, L[8], D, c->ffn_out, mode))) return st;
        } else if ((st = or_linear(c->ffn_act, n, F, wt, L[8], D, c->ffn_out, mode))) {
            return st;
        }
        for (size_t i = 0; i < n * D; i++) c->hidden[i] += c->ffn_out[i];
    }
    c->seq_len += n;
    /* Final norm over every row, then only the last row feeds the head
     * (model.rs:72-95). */
    or_rms_norm_rows(c->hidden + (n - 1) * D, m->output_norm, c->last_hidden, 1, D, m->eps);
    if (int_acts) {
        const or_block_q8_0* a = site_blocks(c, c->last_hidden, 1, D, lock, &dev, m->n_layers, 4);
        return or_linear_prequant(a, 1, D, wt, m->output, (size_t)m->vocab, c->logits, mode);
    }
    return or_linear(c->last_hidden, 1, D, wt, m->output, (size_t)m->vocab, c->logits, mode);
}
