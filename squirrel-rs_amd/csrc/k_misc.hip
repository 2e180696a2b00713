// Row-wise kernels: embedding, RMSNorm(+quantize), quantize, RoPE + KV cache
// append for prefill rows, SiLU * up (+quantize), elementwise ops, softmax,
// argmax, and debug taps.  All are HBM-trivial next to the matvecs; they exist
// for the batched prefill and for the operator-level entry points.
#include "launch.h"

namespace sq {
namespace {

constexpr int kBlock = 256;

inline int grid_for(size_t n, int per) { return (int)((n + per - 1) / per); }

inline int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(SQ_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
    return 0;
}

// embed_blocks (src/ops/embedding.rs:23-52) with dequantize_into
// (src/kernels/dot_prod.rs:409-414, 440-446, 524-528): exact.
__global__ __launch_bounds__(kBlock) void embed_kernel(MatView table, const uint32_t* tokens,
                                                        int dim, float* out, uint32_t* id_error) {
    const int t = blockIdx.x;
    uint32_t tok = tokens[t];
    // The reference indexes the table with the id and panics past its end
    // (embedding.rs:43-44).  Here the row read stays in bounds (an unsigned
    // compare, so ids of 2^31 and more are caught too) and the error word
    // tells the host, which turns it into a status.
    if (tok >= (uint32_t)table.rows) {
        if (threadIdx.x == 0) *id_error = 1u;
        tok = table.rows - 1;
    }
    const int KB = dim >> 5;
    float* o = out + (size_t)t * dim;
    for (int e = threadIdx.x; e < dim; e += kBlock) {
        const int blk = e >> 5, i = e & 31;
        float v;
        if (table.wtype == WT_Q8_0) {
            const int8_t* qs = (const int8_t*)table.qs + (size_t)tok * dim;
            const float sc = sq_f16_to_f32(table.scale[(size_t)tok * KB + blk]);
            v = sc * (float)qs[e];
        } else if (table.wtype == WT_Q4_0) {
            const uint8_t* qs = (const uint8_t*)table.qs + (size_t)tok * (dim / 2) + blk * 16;
            const float sc = sq_f16_to_f32(table.scale[(size_t)tok * KB + blk]);
            const int q = i < 16 ? (qs[i] & 0x0F) : (qs[i - 16] >> 4);
            v = sc * (float)(q - 8);
        } else {
            const uint16_t* w = (const uint16_t*)table.qs + (size_t)tok * dim;
            v = sq_bf16_to_f32(w[e]);
        }
        o[e] = v;
    }
}

// rms_norm over rows (src/ops/rms_norm.rs:13-43); when act_q is non-null the
// normed row is also quantized to Q8_0 (quantize_row_q8_0, dot_prod.rs:21-31).
// Defined below the Q8_0 emitter it uses.
__global__ __launch_bounds__(kBlock) void rmsnorm_rows_kernel(const float* x, const float* w, int dim,
                                                               float eps, float* out, int8_t* act_q,
                                                               uint16_t* act_d);

// quantize_row_q8_0 over n values (n a multiple of 32): one block per 32 lanes.
__global__ __launch_bounds__(kBlock) void quantize_kernel(const float* x, size_t n, int8_t* qs,
                                                           uint16_t* d) {
    const size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x;
    const bool vi = i < n;
    const float v = vi ? x[i] : 0.0f;
    float amax = fmaxf(sq_half_max(fabsf(v)), 0.0f);
    float scale = sq_q8_scale(amax);
    float inv = sq_q8_inv(scale);
    if (vi) {
        qs[i] = sq_q8_quant(v, inv);
        if ((i & 31) == 0) d[i >> 5] = sq_f32_to_f16(scale);
    }
}

// Q8_0 blocks of 8 consecutive values per thread (a lane quad holds a
// block): the quantizer above with 16-byte loads and 8-byte stores.  All
// values of one 32-element block are quantized with the same scale, so the
// result is that of quantize_kernel.
__device__ __forceinline__ void q8_emit8(const float* v, size_t g, bool valid, int8_t* qs, uint16_t* d) {
    float m = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; e++) m = fmaxf(m, fabsf(v[e]));
    const float amax = fmaxf(sq_quad_max(m), 0.0f);
    const float scale = sq_q8_scale(amax), inv = sq_q8_inv(scale);
    if (valid) {
        unsigned lo = 0, hi = 0;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            lo |= (unsigned)(uint8_t)sq_q8_quant(v[e], inv) << (8 * e);
            hi |= (unsigned)(uint8_t)sq_q8_quant(v[e + 4], inv) << (8 * e);
        }
        *(uint2*)(qs + 8 * g) = make_uint2(lo, hi);
        if ((g & 3) == 0) d[g >> 2] = sq_f32_to_f16(scale);
    }
}

__global__ __launch_bounds__(kBlock) void quantize8_kernel(const float* __restrict__ x, size_t n8,
                                                            int8_t* __restrict__ qs, uint16_t* __restrict__ d) {
    const size_t g = (size_t)blockIdx.x * kBlock + threadIdx.x;
    const bool vg = g < n8;
    float v[8] = {};
    if (vg) {
        const float4 a = ((const float4*)x)[2 * g], b = ((const float4*)x)[2 * g + 1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    }
    q8_emit8(v, g, vg, qs, d);
}

// Rows whose width is a multiple of 8 (of 32 when quantized) and at most
// 8 * kBlock take the vector path: thread t holds elements 8t..8t+7 (16-byte
// loads; the lane quad of a 32-element block shares its maximum).  Other
// widths keep one element per thread, read once when the row fits.
__global__ __launch_bounds__(kBlock) void rmsnorm_rows_kernel(const float* x, const float* w, int dim,
                                                               float eps, float* out, int8_t* act_q,
                                                               uint16_t* act_d) {
    // rows up to 8 * kBlock wide are read once, every load issued before any
    // arithmetic; wider rows are read twice
    constexpr int NC = 8;
    __shared__ float s_red[kBlock / 64];
    const int r = blockIdx.x;
    const float* xr = x + (size_t)r * dim;
    auto row_rms = [&](float ss) {
        ss = sq_wave_sum(ss);
        if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = ss;
        __syncthreads();
        float tot = 0.0f;
        for (int i = 0; i < kBlock / 64; i++) tot += s_red[i];
        return sqrtf(tot / (float)dim + eps);
    };
    if (dim % 8 == 0 && dim <= NC * kBlock && (act_q == nullptr || dim % 32 == 0) &&
        (((uintptr_t)x | (uintptr_t)w | (uintptr_t)out) & 15) == 0) {
        const int t8 = 8 * threadIdx.x;
        const bool vt = t8 < dim;
        float xv[8] = {}, wv[8] = {};
        if (vt) {
            const float4 a = *(const float4*)(xr + t8), b = *(const float4*)(xr + t8 + 4);
            const float4 c = *(const float4*)(w + t8), d = *(const float4*)(w + t8 + 4);
            xv[0] = a.x; xv[1] = a.y; xv[2] = a.z; xv[3] = a.w; xv[4] = b.x; xv[5] = b.y; xv[6] = b.z; xv[7] = b.w;
            wv[0] = c.x; wv[1] = c.y; wv[2] = c.z; wv[3] = c.w; wv[4] = d.x; wv[5] = d.y; wv[6] = d.z; wv[7] = d.w;
        }
        float ss = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) ss += xv[e] * xv[e];
        const float rms = row_rms(ss);
        float y[8];
#pragma unroll
        for (int e = 0; e < 8; e++) y[e] = vt ? (xv[e] * wv[e]) / rms : 0.0f;
        if (vt && out) {
            *(float4*)(out + (size_t)r * dim + t8) = make_float4(y[0], y[1], y[2], y[3]);
            *(float4*)(out + (size_t)r * dim + t8 + 4) = make_float4(y[4], y[5], y[6], y[7]);
        }
        if (act_q) q8_emit8(y, ((size_t)r * dim + t8) / 8, vt, act_q, act_d);
        return;
    }
    const bool cached = dim <= NC * kBlock;
    float xv[NC], wv[NC];
    float ss = 0.0f;
    if (cached) {
#pragma unroll
        for (int j = 0; j < NC; j++) {
            const int i = threadIdx.x + j * kBlock;
            xv[j] = i < dim ? xr[i] : 0.0f;
            wv[j] = i < dim ? w[i] : 0.0f;
        }
        // the same order as the loop below (elements past dim add 0)
#pragma unroll
        for (int j = 0; j < NC; j++) ss += xv[j] * xv[j];
    } else {
        for (int i = threadIdx.x; i < dim; i += kBlock) ss += xr[i] * xr[i];
    }
    const float rms = row_rms(ss);
    // dim is a multiple of 32 and the stride is a multiple of 64, so every
    // aligned 32-lane group holds one whole block.
    auto emit = [&](int i, float xi, float wi) {
        const bool vi = i < dim;
        const float y = vi ? (xi * wi) / rms : 0.0f;
        if (vi && out) out[(size_t)r * dim + i] = y;
        if (act_q) {
            float amax = fmaxf(sq_half_max(fabsf(y)), 0.0f);
            float scale = sq_q8_scale(amax);
            float inv = sq_q8_inv(scale);
            if (vi) {
                act_q[(size_t)r * dim + i] = sq_q8_quant(y, inv);
                if ((i & 31) == 0) act_d[((size_t)r * dim + i) >> 5] = sq_f32_to_f16(scale);
            }
        }
    };
    if (cached) {
#pragma unroll
        for (int j = 0; j < NC; j++) {
            if (j * kBlock >= dim) break;
            emit(threadIdx.x + j * kBlock, xv[j], wv[j]);
        }
    } else {
        for (int base = 0; base < dim; base += kBlock) {
            const int i = base + threadIdx.x;
            emit(i, i < dim ? xr[i] : 0.0f, i < dim ? w[i] : 0.0f);
        }
    }
}

// silu_mul_kernel with 8 consecutive FFN outputs per thread (ffn is a
// multiple of 32, so a group never crosses a row).
__global__ __launch_bounds__(kBlock) void silu_mul8_kernel(const float* __restrict__ gu, int ffn, size_t n8,
                                                            float* __restrict__ out, int8_t* __restrict__ act_q,
                                                            uint16_t* __restrict__ act_d) {
    const size_t g = (size_t)blockIdx.x * kBlock + threadIdx.x;
    const bool vg = g < n8;
    float v[8] = {};
    if (vg) {
        const size_t i = 8 * g, m = i / ffn, j = i % ffn;
        const float4* G = (const float4*)(gu + m * 2 * ffn + j);
        const float4* U = (const float4*)(gu + m * 2 * ffn + ffn + j);
        const float4 g0 = G[0], g1 = G[1], u0 = U[0], u1 = U[1];
        const float gv[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
        const float uv[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float sg = gv[e] * sq_sigmoid(gv[e]);
            v[e] = sg * uv[e];
        }
        if (out) {
            ((float4*)out)[2 * g] = make_float4(v[0], v[1], v[2], v[3]);
            ((float4*)out)[2 * g + 1] = make_float4(v[4], v[5], v[6], v[7]);
        }
    }
    if (act_q) q8_emit8(v, g, vg, act_q, act_d);
}

// Split payload/scale <-> GGUF 34-byte Q8_0 blocks (tensor.rs:10-15).
__global__ void pack_q8_kernel(const int8_t* qs, const uint16_t* d, size_t nblocks, uint8_t* out) {
    const size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    uint8_t* o = out + b * 34;
    const uint16_t s = d[b];
    o[0] = (uint8_t)(s & 0xFF);
    o[1] = (uint8_t)(s >> 8);
    for (int i = 0; i < 32; i++) o[2 + i] = (uint8_t)qs[b * 32 + i];
}

__global__ void unpack_q8_kernel(const uint8_t* in, size_t nblocks, int8_t* qs, uint16_t* d) {
    const size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const uint8_t* p = in + b * 34;
    d[b] = (uint16_t)(p[0] | (p[1] << 8));
    for (int i = 0; i < 32; i++) qs[b * 32 + i] = (int8_t)p[2 + i];
}

// Prefill RoPE + KV append: row m of the fused qkv output is at position
// pos0+m (rope_rows, src/ops/rope.rs:28-30); q is rotated into q_out, k is
// rotated into the cache row, v is copied (KvCache::append, kv_cache.rs:38-53).
__global__ __launch_bounds__(kBlock) void rope_kv_kernel(const float* qkv, int ld, int q_dim,
                                                          int kv_dim, int head_dim, int pos0,
                                                          const float2* rope, float* q_out,
                                                          float* kcache, float* vcache) {
    const int m = blockIdx.x;
    const int p = pos0 + m;
    const int half = head_dim >> 1;
    const float* row = qkv + (size_t)m * ld;
    const int n_pairs = (q_dim + kv_dim) >> 1;
    for (int pi = threadIdx.x; pi < n_pairs; pi += kBlock) {
        const int e = 2 * pi;
        const bool is_q = e < q_dim;
        const int li = is_q ? e : e - q_dim;
        const int j = (li % head_dim) >> 1;
        const float2 cs = rope[(size_t)p * half + j];
        float o0, o1;
        sq_rotate(row[e], row[e + 1], cs.x, cs.y, o0, o1);
        if (is_q) {
            q_out[(size_t)m * q_dim + li] = o0;
            q_out[(size_t)m * q_dim + li + 1] = o1;
        } else {
            kcache[(size_t)p * kv_dim + li] = o0;
            kcache[(size_t)p * kv_dim + li + 1] = o1;
        }
    }
    for (int i = threadIdx.x; i < kv_dim; i += kBlock)
        vcache[(size_t)p * kv_dim + i] = row[q_dim + kv_dim + i];
}

// rope_f32_interleaved over rows with a per-row (cos, sin) table.
__global__ __launch_bounds__(kBlock) void rope_rows_kernel(float* t, int row_dim, int head_dim,
                                                            const float2* cs_rows) {
    const int r = blockIdx.x;
    const int half = head_dim >> 1;
    float* row = t + (size_t)r * row_dim;
    for (int pi = threadIdx.x; pi < row_dim / 2; pi += kBlock) {
        const int e = 2 * pi;
        const int j = (e % head_dim) >> 1;
        const float2 cs = cs_rows[(size_t)r * half + j];
        float o0, o1;
        sq_rotate(row[e], row[e + 1], cs.x, cs.y, o0, o1);
        row[e] = o0;
        row[e + 1] = o1;
    }
}

// ffn: gate = silu(gate); act = gate * up (layers.rs:73-74), then Q8_0
// blocks of act when act_q is non-null; the f32 act goes to out when that is
// non-null (the integer path only reads the blocks).  gu holds [gate | up]
// per row.
__global__ __launch_bounds__(kBlock) void silu_mul_kernel(const float* gu, int ffn, size_t n,
                                                           float* out, int8_t* act_q,
                                                           uint16_t* act_d) {
    const size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x;
    const bool vi = i < n;
    float f = 0.0f;
    if (vi) {
        const size_t m = i / ffn, j = i % ffn;
        const float g = gu[m * 2 * ffn + j];
        const float u = gu[m * 2 * ffn + ffn + j];
        const float sg = g * sq_sigmoid(g);
        f = sg * u;
        if (out) out[i] = f;
    }
    if (act_q) {
        float amax = fmaxf(sq_half_max(fabsf(f)), 0.0f);
        float scale = sq_q8_scale(amax);
        float inv = sq_q8_inv(scale);
        if (vi) {
            act_q[i] = sq_q8_quant(f, inv);
            if ((i & 31) == 0) act_d[i >> 5] = sq_f32_to_f16(scale);
        }
    }
}

__global__ void silu_kernel(float* x, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) x[i] = x[i] * sq_sigmoid(x[i]);
}

__global__ void mul_kernel(const float* a, const float* b, float* out, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = a[i] * b[i];
}

__global__ void add_kernel(float* a, const float* b, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) a[i] = a[i] + b[i];
}

// softmax_f32 (src/kernels/softmax.rs:4-27) over one row: max, exp(v - max),
// sum, multiply by 1/sum.  The sum is a tree, not a sequential fold.
__global__ __launch_bounds__(1024) void softmax_kernel(const float* in, float* out, int n) {
    __shared__ float s_red[16];
    const int tid = threadIdx.x;
    float m = -INFINITY;
    for (int i = tid; i < n; i += 1024) m = fmaxf(m, in[i]);
    m = sq_wave_max(m);
    if ((tid & 63) == 0) s_red[tid >> 6] = m;
    __syncthreads();
    float mx = -INFINITY;
    for (int w = 0; w < 16; w++) mx = fmaxf(mx, s_red[w]);
    __syncthreads();
    float s = 0.0f;
    for (int i = tid; i < n; i += 1024) {
        const float e = expf(in[i] - mx);
        out[i] = e;
        s += e;
    }
    s = sq_wave_sum(s);
    if ((tid & 63) == 0) s_red[tid >> 6] = s;
    __syncthreads();
    float tot = 0.0f;
    for (int w = 0; w < 16; w++) tot += s_red[w];
    const float inv = 1.0f / tot;
    for (int i = tid; i < n; i += 1024) out[i] = out[i] * inv;
}

// (value, index) reduction with the reference's tie rule (greedy.rs:8-13):
// the larger value wins; equal values go to the larger index.  NaN entries
// never win here; their largest index is tracked separately.
struct ArgBest {
    float v;
    int i;
    int nan;
};

__device__ __forceinline__ void arg_merge(ArgBest& a, float v, int i, int nan) {
    if (i >= 0 && (a.i < 0 || v > a.v || (v == a.v && i > a.i))) {
        a.v = v;
        a.i = i;
    }
    a.nan = nan > a.nan ? nan : a.nan;
}

__device__ ArgBest block_arg_reduce(ArgBest a) {
    __shared__ float s_v[16];
    __shared__ int s_i[16], s_n[16];
    for (int o = 32; o >= 1; o >>= 1) {
        float ov = __shfl_xor(a.v, o, 64);
        int oi = __shfl_xor(a.i, o, 64);
        int on = __shfl_xor(a.nan, o, 64);
        arg_merge(a, ov, oi, on);
    }
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        s_v[w] = a.v;
        s_i[w] = a.i;
        s_n[w] = a.nan;
    }
    __syncthreads();
    ArgBest r{-INFINITY, -1, -1};
    const int nw = blockDim.x >> 6;
    for (int k = 0; k < nw; k++) arg_merge(r, s_v[k], s_i[k], s_n[k]);
    __syncthreads();
    return r;
}

// Partials over contiguous chunks of an arbitrary logits row.
__global__ __launch_bounds__(256) void argmax_partials_kernel(const float* logits, int n,
                                                               float* pv, int* pi, int* pn) {
    const int chunk = (n + gridDim.x - 1) / gridDim.x;
    const int b0 = blockIdx.x * chunk;
    const int b1 = min(n, b0 + chunk);
    ArgBest a{-INFINITY, -1, -1};
    for (int i = b0 + threadIdx.x; i < b1; i += blockDim.x) {
        const float v = logits[i];
        if (v != v) arg_merge(a, 0.0f, -1, i);
        else arg_merge(a, v, i, -1);
    }
    ArgBest r = block_arg_reduce(a);
    if (threadIdx.x == 0) {
        pv[blockIdx.x] = r.v;
        pi[blockIdx.x] = r.i;
        pn[blockIdx.x] = r.nan;
    }
}

// GreedySampler::sample resolved from partials.  Iterator::max_by hands the
// lead to the later element whenever a comparison involves NaN, so the
// result is the last-maximum over the elements after the last NaN (or that
// NaN's index when it is the final element).
__global__ __launch_bounds__(1024) void argmax_final_kernel(const float* logits, int n,
                                                             const float* pv, const int* pi,
                                                             const int* pn, int n_parts,
                                                             uint32_t* token, int* pos, int advance,
                                                             uint32_t* history, int* n_hist) {
    ArgBest a{-INFINITY, -1, -1};
    for (int k = threadIdx.x; k < n_parts; k += blockDim.x) arg_merge(a, pv[k], pi[k], pn[k]);
    ArgBest r = block_arg_reduce(a);
    int result = r.i;
    if (r.nan >= 0) {
        ArgBest b{-INFINITY, -1, -1};
        for (int i = r.nan + 1 + threadIdx.x; i < n; i += blockDim.x) arg_merge(b, logits[i], i, -1);
        ArgBest rb = block_arg_reduce(b);
        result = rb.i >= 0 ? rb.i : r.nan;
    }
    if (threadIdx.x == 0) {
        *token = (uint32_t)result;
        if (history) {
            const int h = *n_hist;
            history[h] = (uint32_t)result;
            *n_hist = h + 1;
        }
        if (pos) *pos += advance;
    }
}

// log p(idx) under softmax(logits), in f64 (src/bin/perplexity.rs:112-117):
// the maximum folded in f32 with NaN entries skipped (f32::max), the sum of
// exp(f64(l) - max) in f64, then f64(l[idx]) - max - ln(sum).  The sum is a
// fixed-order tree over the workgroup, not the reference's sequential fold,
// so the two agree to f64 rounding.
__global__ __launch_bounds__(1024) void log_softmax_at_kernel(const float* __restrict__ logits, int n,
                                                              const uint32_t* __restrict__ idx,
                                                              double* __restrict__ out,
                                                              uint32_t* __restrict__ id_error) {
    __shared__ float s_m[16];
    __shared__ double s_s[16];
    const int tid = threadIdx.x;
    float m = -INFINITY;
    for (int i = tid; i < n; i += 1024) m = fmaxf(m, logits[i]);
    m = sq_wave_max(m);
    if ((tid & 63) == 0) s_m[tid >> 6] = m;
    __syncthreads();
    float mx = -INFINITY;
    for (int w = 0; w < 16; w++) mx = fmaxf(mx, s_m[w]);
    const double md = (double)mx;
    double s = 0.0;
    for (int i = tid; i < n; i += 1024) s += exp((double)logits[i] - md);
    for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
    if ((tid & 63) == 0) s_s[tid >> 6] = s;
    __syncthreads();
    if (tid == 0) {
        double tot = 0.0;
        for (int w = 0; w < 16; w++) tot += s_s[w];
        // an index past the row is the reference's panic (perplexity.rs:112-117)
        const uint32_t i = *idx;
        if (i >= (uint32_t)n) *id_error = 1u;
        *out = i < (uint32_t)n ? (double)logits[i] - md - log(tot) : (double)NAN;
    }
}

// Per-block exact integer sums of one quantized activation row against one
// weight row, in the same lane layout as the decode matvec.
__global__ __launch_bounds__(64) void block_isums_kernel(const int8_t* aq, MatView w, int row,
                                                          int32_t* out) {
    const int KB = w.k >> 5;
    for (int blk = threadIdx.x; blk < KB; blk += 64) {
        const int* a = (const int*)(aq + blk * 32);
        int isum = 0;
        if (w.wtype == WT_Q8_0) {
            const int* q = (const int*)((const int8_t*)w.qs + (size_t)row * w.k + blk * 32);
            for (int v = 0; v < 8; v++) isum = __builtin_amdgcn_sdot4(a[v], q[v], isum, false);
        } else {
            const int* q = (const int*)((const uint8_t*)w.qs + (size_t)row * (w.k / 2) + blk * 16);
            int asum = 0;
            for (int v = 0; v < 8; v++) asum = __builtin_amdgcn_sdot4(a[v], 0x01010101, asum, false);
            for (int v = 0; v < 4; v++) {
                isum = __builtin_amdgcn_sdot4(a[v], q[v] & 0x0F0F0F0F, isum, false);
                isum = __builtin_amdgcn_sdot4(a[4 + v], (q[v] >> 4) & 0x0F0F0F0F, isum, false);
            }
            isum -= 8 * asum;
        }
        out[blk] = isum;
    }
}

__global__ void copy_i32_kernel(const int* src, int* dst) { *dst = *src; }

}  // namespace

int launch_embed(hipStream_t s, const MatView& table, int wtype, const uint32_t* tokens, int n_tokens,
                 int dim, float* out, uint32_t* id_error) {
    if (!id_error) return set_error(SQ_ERR_ARG, "embed: no error word");
    MatView t = table;
    t.wtype = wtype;
    hipLaunchKernelGGL(embed_kernel, dim3(n_tokens), dim3(kBlock), 0, s, t, tokens, dim, out, id_error);
    return check_launch("embed");
}

int launch_rmsnorm_rows(hipStream_t s, const float* x, const float* w, int rows, int dim, float eps,
                        float* out, int8_t* act_q, uint16_t* act_d) {
    hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3(rows), dim3(kBlock), 0, s, x, w, dim, eps, out, act_q,
                       act_d);
    return check_launch("rmsnorm_rows");
}

int launch_quantize_rows(hipStream_t s, const float* x, size_t n, int8_t* qs, uint16_t* d) {
    if (n % 32 == 0 && ((uintptr_t)x & 15) == 0) {
        hipLaunchKernelGGL(quantize8_kernel, dim3(grid_for(n / 8, kBlock)), dim3(kBlock), 0, s, x, n / 8, qs, d);
        return check_launch("quantize");
    }
    hipLaunchKernelGGL(quantize_kernel, dim3(grid_for(n, kBlock)), dim3(kBlock), 0, s, x, n, qs, d);
    return check_launch("quantize");
}

int launch_pack_q8_blocks(hipStream_t s, const int8_t* qs, const uint16_t* d, size_t nblocks,
                          void* out) {
    hipLaunchKernelGGL(pack_q8_kernel, dim3(grid_for(nblocks, 256)), dim3(256), 0, s, qs, d, nblocks,
                       (uint8_t*)out);
    return check_launch("pack_q8");
}

int launch_unpack_q8_blocks(hipStream_t s, const void* in, size_t nblocks, int8_t* qs, uint16_t* d) {
    hipLaunchKernelGGL(unpack_q8_kernel, dim3(grid_for(nblocks, 256)), dim3(256), 0, s,
                       (const uint8_t*)in, nblocks, qs, d);
    return check_launch("unpack_q8");
}

int launch_rope_kv_rows(hipStream_t s, const float* qkv, int ld, int rows, int q_dim, int kv_dim,
                        int head_dim, int pos0, const float2* rope, float* q_out, float* kcache,
                        float* vcache) {
    hipLaunchKernelGGL(rope_kv_kernel, dim3(rows), dim3(kBlock), 0, s, qkv, ld, q_dim, kv_dim, head_dim,
                       pos0, rope, q_out, kcache, vcache);
    return check_launch("rope_kv");
}

int launch_rope_rows_table(hipStream_t s, float* t, int rows, int row_dim, int head_dim,
                           const float2* cs_rows) {
    hipLaunchKernelGGL(rope_rows_kernel, dim3(rows), dim3(kBlock), 0, s, t, row_dim, head_dim, cs_rows);
    return check_launch("rope_rows");
}

int launch_silu_mul_rows(hipStream_t s, const float* gu, int ffn, size_t n, float* out, int8_t* act_q,
                         uint16_t* act_d) {
    if (ffn % 32 == 0 && ((uintptr_t)gu & 15) == 0 && ((uintptr_t)out & 15) == 0) {
        hipLaunchKernelGGL(silu_mul8_kernel, dim3(grid_for(n / 8, kBlock)), dim3(kBlock), 0, s, gu, ffn, n / 8, out,
                           act_q, act_d);
        return check_launch("silu_mul");
    }
    hipLaunchKernelGGL(silu_mul_kernel, dim3(grid_for(n, kBlock)), dim3(kBlock), 0, s, gu, ffn, n, out,
                       act_q, act_d);
    return check_launch("silu_mul");
}

int launch_silu(hipStream_t s, float* x, size_t n) {
    hipLaunchKernelGGL(silu_kernel, dim3(grid_for(n, 256)), dim3(256), 0, s, x, n);
    return check_launch("silu");
}

int launch_mul(hipStream_t s, const float* a, const float* b, float* out, size_t n) {
    hipLaunchKernelGGL(mul_kernel, dim3(grid_for(n, 256)), dim3(256), 0, s, a, b, out, n);
    return check_launch("mul");
}

int launch_add_inplace(hipStream_t s, float* a, const float* b, size_t n) {
    hipLaunchKernelGGL(add_kernel, dim3(grid_for(n, 256)), dim3(256), 0, s, a, b, n);
    return check_launch("add");
}

int launch_softmax_row(hipStream_t s, const float* in, float* out, int n) {
    hipLaunchKernelGGL(softmax_kernel, dim3(1), dim3(1024), 0, s, in, out, n);
    return check_launch("softmax");
}

int launch_argmax_partials(hipStream_t s, const float* logits, int n, float* pv, int* pi, int* pn,
                           int n_parts) {
    hipLaunchKernelGGL(argmax_partials_kernel, dim3(n_parts), dim3(256), 0, s, logits, n, pv, pi, pn);
    return check_launch("argmax_partials");
}

int launch_argmax_final(hipStream_t s, const float* logits, int n, const float* pv, const int* pi,
                        const int* pn, int n_parts, uint32_t* token, int* pos, int advance,
                        uint32_t* history, int* n_hist) {
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(1024), 0, s, logits, n, pv, pi, pn, n_parts,
                       token, pos, advance, history, n_hist);
    return check_launch("argmax_final");
}

int launch_block_isums(hipStream_t s, const int8_t* aq, const MatView& w, int wtype, int row,
                       int32_t* out) {
    MatView v = w;
    v.wtype = wtype;
    hipLaunchKernelGGL(block_isums_kernel, dim3(1), dim3(64), 0, s, aq, v, row, out);
    return check_launch("block_isums");
}

int launch_log_softmax_at(hipStream_t s, const float* logits, int n, const uint32_t* idx, double* out,
                          uint32_t* id_error) {
    if (!id_error) return set_error(SQ_ERR_ARG, "log_softmax_at: no error word");
    hipLaunchKernelGGL(log_softmax_at_kernel, dim3(1), dim3(1024), 0, s, logits, n, idx, out, id_error);
    return check_launch("log_softmax_at");
}

int launch_copy_i32(hipStream_t s, const int* src, int* dst) {
    hipLaunchKernelGGL(copy_i32_kernel, dim3(1), dim3(1), 0, s, src, dst);
    return check_launch("copy_i32");
}

}  // namespace sq
