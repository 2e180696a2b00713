// Causal grouped-query attention over the device-resident f32 KV cache.
//
// Semantics: sdpa_f32 (src/kernels/attention.rs:11-70).  Query row t sees
// keys 0..=offset+t, kv head = h / (n_heads / n_kv_heads), scores are
// dot(q, k) * (1/sqrt(head_dim)), softmax subtracts the row max.  The kernels
// here compute the softmax online (running max / sum per split, merged with
// the log-sum-exp rule), so results agree to rounding, not bit for bit.
//
// Cache layout (KvCache, src/models/common/kv_cache.rs:1-16): per layer
// [position][n_kv_heads * head_dim] f32, row-major.
#include "launch.h"

namespace sq {
namespace {

constexpr int HD = 64;  // head_dim of the model kernels (Llama-3.2-1B)

inline int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(SQ_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
    return 0;
}

// Decode attention, flash-decoding split over positions.  One wavefront per
// (kv head, split); it owns the GQA group's G query heads, so each K/V row is
// read once for all of them.  Tile = 64 positions: lane = position for the
// scores, lane = dimension for P*V.
template <int G>
__global__ __launch_bounds__(64) void attn_decode_kernel(const float* __restrict__ q,
                                                          const float* __restrict__ kc,
                                                          const float* __restrict__ vc,
                                                          const int* __restrict__ pos_ptr,
                                                          int n_kv_heads, int nsplit, float* part_m,
                                                          float* part_l, float* part_o) {
    __shared__ float s_q[G][HD];
    __shared__ float s_p[G][64];
    const int g = blockIdx.x;
    const int sp = blockIdx.y;
    const int lane = threadIdx.x;
    const int P = *pos_ptr + 1;
    const int kv_dim = n_kv_heads * HD;
    const float scale = 1.0f / sqrtf((float)HD);

#pragma unroll
    for (int i = 0; i < G; i++) s_q[i][lane] = q[(g * G + i) * HD + lane];
    __syncthreads();

    float m[G], l[G], acc[G];
#pragma unroll
    for (int i = 0; i < G; i++) {
        m[i] = -INFINITY;
        l[i] = 0.0f;
        acc[i] = 0.0f;
    }

    for (int tile = sp; tile * 64 < P; tile += nsplit) {
        const int s = tile * 64 + lane;
        const bool valid = s < P;
        float sc[G];
        if (valid) {
            const float4* kr = (const float4*)(kc + (size_t)s * kv_dim + g * HD);
            float4 k4[HD / 4];
#pragma unroll
            for (int d = 0; d < HD / 4; d++) k4[d] = kr[d];
#pragma unroll
            for (int i = 0; i < G; i++) {
                float dot = 0.0f;
#pragma unroll
                for (int d = 0; d < HD / 4; d++) {
                    dot += s_q[i][4 * d + 0] * k4[d].x;
                    dot += s_q[i][4 * d + 1] * k4[d].y;
                    dot += s_q[i][4 * d + 2] * k4[d].z;
                    dot += s_q[i][4 * d + 3] * k4[d].w;
                }
                sc[i] = dot * scale;
            }
        } else {
#pragma unroll
            for (int i = 0; i < G; i++) sc[i] = -INFINITY;
        }
#pragma unroll
        for (int i = 0; i < G; i++) {
            const float tmax = sq_wave_max(sc[i]);
            const float mn = fmaxf(m[i], tmax);
            const float alpha = (m[i] == -INFINITY) ? 0.0f : expf(m[i] - mn);
            const float p = valid ? expf(sc[i] - mn) : 0.0f;
            l[i] = l[i] * alpha + sq_wave_sum(p);
            acc[i] *= alpha;
            m[i] = mn;
            s_p[i][lane] = p;
        }
        __syncthreads();
        const int nvalid = min(64, P - tile * 64);
        const float* vbase = vc + (size_t)tile * 64 * kv_dim + g * HD + lane;
        for (int j = 0; j < nvalid; j++) {
            const float v = vbase[(size_t)j * kv_dim];
#pragma unroll
            for (int i = 0; i < G; i++) acc[i] += s_p[i][j] * v;
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < G; i++) {
        const int idx = (g * G + i) * nsplit + sp;
        if (lane == 0) {
            part_m[idx] = m[i];
            part_l[idx] = l[i];
        }
        part_o[(size_t)idx * HD + lane] = acc[i];
    }
}

// Merge the splits of one head; lane = dimension.  Optionally quantizes the
// head's two 32-blocks for the o-projection (the reference quantizes the
// attention output row inside `linear`, src/kernels/matmul.rs:91-98).
__global__ __launch_bounds__(64) void attn_combine_kernel(const float* part_m, const float* part_l,
                                                           const float* part_o, int nsplit,
                                                           float* attn, int8_t* act_q,
                                                           uint16_t* act_d) {
    const int h = blockIdx.x;
    const int lane = threadIdx.x;
    float M = -INFINITY;
    for (int s = 0; s < nsplit; s++) M = fmaxf(M, part_m[h * nsplit + s]);
    float L = 0.0f, O = 0.0f;
    for (int s = 0; s < nsplit; s++) {
        const float ms = part_m[h * nsplit + s];
        if (ms == -INFINITY) continue;
        const float e = expf(ms - M);
        L += part_l[h * nsplit + s] * e;
        O += part_o[(size_t)(h * nsplit + s) * HD + lane] * e;
    }
    const float out = O / L;
    attn[h * HD + lane] = out;
    if (act_q) {
        float amax = fmaxf(sq_half_max(fabsf(out)), 0.0f);
        float scale = sq_q8_scale(amax);
        float inv = sq_q8_inv(scale);
        act_q[h * HD + lane] = sq_q8_quant(out, inv);
        if ((lane & 31) == 0) act_d[(h * HD + lane) >> 5] = sq_f32_to_f16(scale);
    }
}

// Prefill attention: 64 query rows of one head per workgroup, K/V tiles of
// 64 positions staged in LDS, online softmax.  Thread (ty, tx) owns query
// rows 4ty..4ty+3 and key columns / output dims 4tx..4tx+3.
constexpr int PT = 64;       // queries and keys per tile
constexpr int LDP = HD + 4;  // padded LDS row (floats)

__global__ __launch_bounds__(256) void attn_prefill_kernel(const float* __restrict__ q,
                                                            const float* __restrict__ kc,
                                                            const float* __restrict__ vc, int pos0,
                                                            int m_rows, int n_heads, int n_kv_heads,
                                                            float* __restrict__ out) {
    __shared__ __attribute__((aligned(16))) float s_q[PT][LDP];
    __shared__ __attribute__((aligned(16))) float s_k[PT][LDP];
    __shared__ __attribute__((aligned(16))) float s_v[PT][LDP];
    __shared__ __attribute__((aligned(16))) float s_p[PT][LDP];

    const int h = blockIdx.x;
    const int t0 = blockIdx.y * PT;
    const int group = n_heads / n_kv_heads;
    const int g = h / group;
    const int q_dim = n_heads * HD;
    const int kv_dim = n_kv_heads * HD;
    const int tid = threadIdx.x;
    const int ty = tid >> 4, tx = tid & 15;
    const float scale = 1.0f / sqrtf((float)HD);

    for (int e = tid; e < PT * HD / 4; e += 256) {
        const int r = e / (HD / 4), c4 = e % (HD / 4);
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (t0 + r < m_rows) v = *(const float4*)(q + (size_t)(t0 + r) * q_dim + h * HD + 4 * c4);
        *(float4*)&s_q[r][4 * c4] = v;
    }

    float mrow[4], lrow[4], o[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        mrow[i] = -INFINITY;
        lrow[i] = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++) o[i][j] = 0.0f;
    }

    const int last_q = min(t0 + PT, m_rows) - 1;
    const int n_keys = pos0 + last_q + 1;  // keys any row of this tile can see
    for (int k0 = 0; k0 < n_keys; k0 += PT) {
        __syncthreads();
        for (int e = tid; e < PT * HD / 4; e += 256) {
            const int r = e / (HD / 4), c4 = e % (HD / 4);
            float4 kv = make_float4(0.f, 0.f, 0.f, 0.f), vv = kv;
            if (k0 + r < n_keys) {
                kv = *(const float4*)(kc + (size_t)(k0 + r) * kv_dim + g * HD + 4 * c4);
                vv = *(const float4*)(vc + (size_t)(k0 + r) * kv_dim + g * HD + 4 * c4);
            }
            *(float4*)&s_k[r][4 * c4] = kv;
            *(float4*)&s_v[r][4 * c4] = vv;
        }
        __syncthreads();

        float sc[4][4];
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) sc[i][j] = 0.0f;
        for (int d = 0; d < HD; d += 4) {
            float4 qa[4], kb[4];
#pragma unroll
            for (int i = 0; i < 4; i++) qa[i] = *(const float4*)&s_q[4 * ty + i][d];
#pragma unroll
            for (int j = 0; j < 4; j++) kb[j] = *(const float4*)&s_k[4 * tx + j][d];
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++)
                    sc[i][j] += qa[i].x * kb[j].x + qa[i].y * kb[j].y + qa[i].z * kb[j].z +
                                qa[i].w * kb[j].w;
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int t = t0 + 4 * ty + i;
            const int limit = pos0 + t;  // inclusive key bound (causal)
            float rmax = -INFINITY;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int kk = k0 + 4 * tx + j;
                sc[i][j] = (kk <= limit && t < m_rows) ? sc[i][j] * scale : -INFINITY;
                rmax = fmaxf(rmax, sc[i][j]);
            }
#pragma unroll
            for (int o2 = 8; o2 >= 1; o2 >>= 1) rmax = fmaxf(rmax, __shfl_xor(rmax, o2, 64));
            const float mn = fmaxf(mrow[i], rmax);
            const float alpha = (mrow[i] == -INFINITY) ? 0.0f : expf(mrow[i] - mn);
            float rsum = 0.0f;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float p = (sc[i][j] == -INFINITY) ? 0.0f : expf(sc[i][j] - mn);
                s_p[4 * ty + i][4 * tx + j] = p;
                rsum += p;
            }
#pragma unroll
            for (int o2 = 8; o2 >= 1; o2 >>= 1) rsum += __shfl_xor(rsum, o2, 64);
            lrow[i] = lrow[i] * alpha + rsum;
            mrow[i] = mn;
#pragma unroll
            for (int j = 0; j < 4; j++) o[i][j] *= alpha;
        }
        __syncthreads();
        for (int c = 0; c < PT; c += 4) {
            float4 pa[4], vb[4];
#pragma unroll
            for (int i = 0; i < 4; i++) pa[i] = *(const float4*)&s_p[4 * ty + i][c];
#pragma unroll
            for (int cc = 0; cc < 4; cc++) vb[cc] = *(const float4*)&s_v[c + cc][4 * tx];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float pv[4] = {pa[i].x, pa[i].y, pa[i].z, pa[i].w};
#pragma unroll
                for (int cc = 0; cc < 4; cc++) {
                    o[i][0] += pv[cc] * vb[cc].x;
                    o[i][1] += pv[cc] * vb[cc].y;
                    o[i][2] += pv[cc] * vb[cc].z;
                    o[i][3] += pv[cc] * vb[cc].w;
                }
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int t = t0 + 4 * ty + i;
        if (t >= m_rows) continue;
        const float inv = 1.0f / lrow[i];
        float4 r = make_float4(o[i][0] * inv, o[i][1] * inv, o[i][2] * inv, o[i][3] * inv);
        *(float4*)(out + (size_t)t * q_dim + h * HD + 4 * tx) = r;
    }
}

// Any head_dim (operator-level entry): one wavefront per (query, head) row,
// scores in dynamic LDS.  Follows sdpa_f32 step by step: scores, softmax
// (max, exp, 1/sum), then out = sum_s p_s * v_s in position order.
__global__ __launch_bounds__(64) void sdpa_generic_kernel(const float* q, const float* k,
                                                           const float* v, float* out, int seq_q,
                                                           int seq_k, int n_heads, int n_kv_heads,
                                                           int head_dim) {
    extern __shared__ float s_sc[];
    const int idx = blockIdx.x;
    const int t = idx / n_heads, h = idx % n_heads;
    const int kv_h = h / (n_heads / n_kv_heads);
    const int live = (seq_k - seq_q) + t + 1;
    const int lane = threadIdx.x;
    const float scale = 1.0f / sqrtf((float)head_dim);
    const float* qr = q + (size_t)(t * n_heads + h) * head_dim;
    float mx = -INFINITY;
    for (int s = lane; s < live; s += 64) {
        const float* kr = k + (size_t)(s * n_kv_heads + kv_h) * head_dim;
        float dot = 0.0f;
        for (int d = 0; d < head_dim; d++) dot += qr[d] * kr[d];
        const float sc = dot * scale;
        s_sc[s] = sc;
        mx = fmaxf(mx, sc);
    }
    mx = sq_wave_max(mx);
    float sum = 0.0f;
    for (int s = lane; s < live; s += 64) {
        const float e = expf(s_sc[s] - mx);
        s_sc[s] = e;
        sum += e;
    }
    sum = sq_wave_sum(sum);
    const float inv = 1.0f / sum;
    __syncthreads();
    for (int d = lane; d < head_dim; d += 64) {
        float o = 0.0f;
        for (int s = 0; s < live; s++) o += (s_sc[s] * inv) * v[(size_t)(s * n_kv_heads + kv_h) * head_dim + d];
        out[(size_t)idx * head_dim + d] = o;
    }
}

}  // namespace

int launch_attn_decode(hipStream_t s, const float* q, const float* kcache, const float* vcache,
                       const int* pos, int n_heads, int n_kv_heads, int head_dim, int nsplit,
                       float* part_m, float* part_l, float* part_o) {
    if (head_dim != HD) return set_error(SQ_ERR_UNSUPPORTED, "attention kernels are built for head_dim 64");
    const int G = n_heads / n_kv_heads;
    dim3 grid(n_kv_heads, nsplit);
    switch (G) {
        case 1: hipLaunchKernelGGL(attn_decode_kernel<1>, grid, dim3(64), 0, s, q, kcache, vcache, pos, n_kv_heads, nsplit, part_m, part_l, part_o); break;
        case 2: hipLaunchKernelGGL(attn_decode_kernel<2>, grid, dim3(64), 0, s, q, kcache, vcache, pos, n_kv_heads, nsplit, part_m, part_l, part_o); break;
        case 4: hipLaunchKernelGGL(attn_decode_kernel<4>, grid, dim3(64), 0, s, q, kcache, vcache, pos, n_kv_heads, nsplit, part_m, part_l, part_o); break;
        case 8: hipLaunchKernelGGL(attn_decode_kernel<8>, grid, dim3(64), 0, s, q, kcache, vcache, pos, n_kv_heads, nsplit, part_m, part_l, part_o); break;
        default: return set_error(SQ_ERR_UNSUPPORTED, "GQA group size must be 1, 2, 4 or 8");
    }
    return check_launch("attn_decode");
}

int launch_attn_combine(hipStream_t s, const float* part_m, const float* part_l, const float* part_o,
                        int n_heads, int head_dim, int nsplit, float* attn, int8_t* act_q,
                        uint16_t* act_d) {
    if (head_dim != HD) return set_error(SQ_ERR_UNSUPPORTED, "attention kernels are built for head_dim 64");
    hipLaunchKernelGGL(attn_combine_kernel, dim3(n_heads), dim3(64), 0, s, part_m, part_l, part_o, nsplit,
                       attn, act_q, act_d);
    return check_launch("attn_combine");
}

int launch_attn_prefill(hipStream_t s, const float* q, const float* kcache, const float* vcache, int pos0,
                        int m, int n_heads, int n_kv_heads, int head_dim, float* out) {
    if (head_dim != HD) return set_error(SQ_ERR_UNSUPPORTED, "attention kernels are built for head_dim 64");
    dim3 grid(n_heads, (m + PT - 1) / PT);
    hipLaunchKernelGGL(attn_prefill_kernel, grid, dim3(256), 0, s, q, kcache, vcache, pos0, m, n_heads,
                       n_kv_heads, out);
    return check_launch("attn_prefill");
}

int launch_sdpa_generic(hipStream_t s, const float* q, const float* k, const float* v, float* out,
                        int seq_q, int seq_k, int n_heads, int n_kv_heads, int head_dim) {
    if (seq_k > 16384) return set_error(SQ_ERR_SHAPE, "sdpa: at most 16384 keys per call");
    hipLaunchKernelGGL(sdpa_generic_kernel, dim3(seq_q * n_heads), dim3(64), (size_t)seq_k * 4, s, q, k, v,
                       out, seq_q, seq_k, n_heads, n_kv_heads, head_dim);
    return check_launch("sdpa_generic");
}

}  // namespace sq
