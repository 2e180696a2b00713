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
#include <cstdlib>
#include <cstring>

#include "launch.h"

namespace sq {
namespace {

constexpr int HD = 64;  // head_dim of the model kernels (Llama-3.2-1B)

inline int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(SQ_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
    return 0;
}

// Decode attention.  One workgroup per (kv head, tile of 64 positions): the
// tile's K and V rows are staged in LDS with one coalesced load round, the G
// query heads sharing the kv head (GQA) score all 64 positions in parallel,
// and each head's tile partial (running max m, sum l, unnormalized P*V) goes
// to global memory.  The workgroup that finishes last for a kv head (device
// fence + atomic counter) merges the tiles with the log-sum-exp rule, writes
// the attention output and, for the integer path, its Q8_0 blocks (the
// reference quantizes this row inside the o-projection's `linear`,
// src/kernels/matmul.rs:91-98).  Tiles beyond the current length exit at
// once, so one launch shape serves every position of a captured graph.
constexpr int TP = 64;  // positions per tile

template <int G>
__global__ __launch_bounds__(256) void attn_decode_kernel(
    const float* __restrict__ q, const float* __restrict__ kc, const float* __restrict__ vc,
    const int* __restrict__ pos_ptr, int n_kv_heads, int max_tiles, float* part_m, float* part_l,
    float* part_o, unsigned* counters, float* attn, int8_t* act_q, uint16_t* act_d) {
    __shared__ float s_k[TP][HD + 1];
    __shared__ __attribute__((aligned(16))) float s_v[TP][HD];
    __shared__ float s_q[G][HD];
    __shared__ float s_p[G][TP];
    __shared__ float s_m[G], s_l[G];
    __shared__ int s_last;
    const int g = blockIdx.x;
    const int tile = blockIdx.y;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int P = *pos_ptr + 1;
    const int ntiles = (P + TP - 1) / TP;
    if (tile >= ntiles) return;
    const int kv_dim = n_kv_heads * HD;
    const int s0 = tile * TP;
    const float scale = 1.0f / sqrtf((float)HD);

    for (int e = tid; e < TP * HD / 4; e += 256) {
        const int r = e / (HD / 4), c4 = e % (HD / 4);
        float4 k4 = make_float4(0.f, 0.f, 0.f, 0.f), v4 = k4;
        if (s0 + r < P) {
            const size_t off = (size_t)(s0 + r) * kv_dim + g * HD + 4 * c4;
            k4 = *(const float4*)(kc + off);
            v4 = *(const float4*)(vc + off);
        }
        s_k[r][4 * c4 + 0] = k4.x;
        s_k[r][4 * c4 + 1] = k4.y;
        s_k[r][4 * c4 + 2] = k4.z;
        s_k[r][4 * c4 + 3] = k4.w;
        *(float4*)&s_v[r][4 * c4] = v4;
    }
    for (int e = tid; e < G * HD; e += 256) s_q[e / HD][e % HD] = q[(size_t)g * G * HD + e];
    __syncthreads();

    // scores = dot(q, k) * (1/sqrt(head_dim)) (attention.rs:52-55)
    for (int idx = tid; idx < G * TP; idx += 256) {
        const int i = idx / TP, sp = idx % TP;
        float dot = 0.0f;
#pragma unroll 16
        for (int d = 0; d < HD; d++) dot += s_q[i][d] * s_k[sp][d];
        s_p[i][sp] = (s0 + sp < P) ? dot * scale : -INFINITY;
    }
    __syncthreads();
    for (int i = wave; i < G; i += 4) {
        const float v = s_p[i][lane];
        const float m = sq_wave_max(v);
        const float p = (v == -INFINITY) ? 0.0f : expf(v - m);
        const float l = sq_wave_sum(p);
        s_p[i][lane] = p;
        if (lane == 0) {
            s_m[i] = m;
            s_l[i] = l;
        }
    }
    __syncthreads();
    for (int idx = tid; idx < G * HD; idx += 256) {
        const int i = idx / HD, d = idx % HD;
        float o = 0.0f;
#pragma unroll 16
        for (int sp = 0; sp < TP; sp++) o += s_p[i][sp] * s_v[sp][d];
        const int pidx = (g * G + i) * max_tiles + tile;
        part_o[(size_t)pidx * HD + d] = o;
        if (d == 0) {
            part_m[pidx] = s_m[i];
            part_l[pidx] = s_l[i];
        }
    }

    __syncthreads();
    if (tid == 0) {
        __threadfence();
        const unsigned prev = atomicAdd(&counters[g], 1u);
        s_last = prev == (unsigned)(ntiles - 1);
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    for (int idx = tid; idx < G * HD; idx += 256) {
        const int i = idx / HD, d = idx % HD, h = g * G + i;
        float M = -INFINITY;
        for (int t = 0; t < ntiles; t++) M = fmaxf(M, part_m[h * max_tiles + t]);
        float L = 0.0f, O = 0.0f;
        for (int t = 0; t < ntiles; t++) {
            const int pidx = h * max_tiles + t;
            const float mt = part_m[pidx];
            if (mt == -INFINITY) continue;
            const float e = expf(mt - M);
            L += part_l[pidx] * e;
            O += part_o[(size_t)pidx * HD + d] * e;
        }
        const float out = O / L;
        attn[h * HD + d] = out;
        if (act_q) {
            const float amax = fmaxf(sq_half_max(fabsf(out)), 0.0f);
            const float sc = sq_q8_scale(amax);
            const float inv = sq_q8_inv(sc);
            act_q[h * HD + d] = sq_q8_quant(out, inv);
            if ((d & 31) == 0) act_d[(h * HD + d) >> 5] = sq_f32_to_f16(sc);
        }
    }
    if (tid == 0) atomicExch(&counters[g], 0u);
}

// Prefill attention on the matrix cores, f32 in and out
// (v_mfma_f32_16x16x4_f32): 64 query rows of one head per workgroup, 16 per
// wavefront; K and V tiles of 64 positions staged in LDS (V transposed);
// online softmax per query.
// MFMA operand layout (checked on the device): lane l supplies A[l % 16][l / 16]
// and B[l / 16][l % 16]; result r of lane l is D[4 (l / 16) + r][l % 16].
// The scores are formed transposed, S^T = K Q^T: the key rows are the row
// operand and the queries the column operand, with contraction index
// 16 (l / 16) + s at step s, so each lane's 16 operands of the 64 dims are
// contiguous in LDS.  Lane l then holds keys 4 (l / 16) + 0..3 of each
// 16-key subtile for query l % 16, which is exactly the column operand of
// O^T = V^T P^T when step s of a subtile takes key 4 (l / 16) + s: the
// probabilities never leave the registers.  A query's scores sit in the four
// lanes l % 16 + 16 j, so its maximum and sum are an in-lane fold plus two
// lane exchanges.
constexpr int PT = 64;       // queries and keys per tile
constexpr int ALD = HD + 4;  // padded LDS row (floats)
typedef float am_v4f __attribute__((ext_vector_type(4)));

// Three workgroups per CU (152 registers; capped at 128 for four per CU,
// 11 of them spill, and it measured the same).
__global__ __launch_bounds__(256, 3) void attn_prefill_kernel(const float* __restrict__ q,
                                                            const float* __restrict__ kc,
                                                            const float* __restrict__ vc, int pos0,
                                                            int m_rows, int n_heads, int n_kv_heads,
                                                            float* __restrict__ out, int8_t* __restrict__ act_q,
                                                            uint16_t* __restrict__ act_d) {
    __shared__ __attribute__((aligned(16))) float s_k[PT][ALD];   // [key][dim]
    __shared__ __attribute__((aligned(16))) float s_vt[HD][ALD];  // [dim][key]

    const int h = blockIdx.x;
    // A query tile's work grows with its index (causal).  Workgroups are
    // dispatched in order; with quarters [0, B), [B, 2B), [2B, 3B), [3B, 4B)
    // of the tile indices taken as a, 4B-1-a, B+a, 3B-1-a, workgroups a
    // quarter of the grid apart carry equal work in sum, which balances the
    // CUs when the grid is resident at once (four workgroups per CU) and
    // interleaves cheap and costly tiles when it is dispatched in waves
    // (measured equal to heaviest-first order there).
    int ty = blockIdx.y;
    if ((gridDim.y & 3) == 0) {
        const int B = gridDim.y >> 2, k = ty / B, a = ty % B;
        ty = k == 0 ? a : k == 1 ? 4 * B - 1 - a : k == 2 ? B + a : 3 * B - 1 - a;
    }
    const int t0 = ty * PT;
    const int g = h / (n_heads / n_kv_heads);
    const int q_dim = n_heads * HD;
    const int kv_dim = n_kv_heads * HD;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int li = lane & 15, lk = lane >> 4;
    // Scores in base-2 units, s' = (q . k) * scale * log2(e), so that each
    // probability is one exp2 (v_exp_f32): exp(x - m) = exp2(x' - m').
    const float scale2 = (1.0f / sqrtf((float)HD)) * 1.44269504088896341f;

    // this lane's query (t0 + 16 wave + li) and its dims 16 lk .. 16 lk + 15
    const int tq = t0 + 16 * wave + li;
    float qa[16];
#pragma unroll
    for (int c = 0; c < 4; c++) {
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (tq < m_rows) v = *(const float4*)(q + (size_t)tq * q_dim + h * HD + 16 * lk + 4 * c);
        qa[4 * c] = v.x; qa[4 * c + 1] = v.y; qa[4 * c + 2] = v.z; qa[4 * c + 3] = v.w;
    }
    // online softmax state of query tq: the running maximum (the same in
    // its four lanes), this lane's part of the running sum, and
    // o[dt][r] = O^T[16 dt + 4 lk + r][tq]
    float mrow = -INFINITY, lpart = 0.0f;
    am_v4f o[4];
#pragma unroll
    for (int dt = 0; dt < 4; dt++) o[dt] = am_v4f{0.f, 0.f, 0.f, 0.f};

    const int last_q = min(t0 + PT, m_rows) - 1;
    const int n_keys = pos0 + last_q + 1;  // keys any row of this tile can see
    const int limit = pos0 + tq;           // query tq sees keys 0 ..= limit
    // Tiles below pos0 + t0 + 1 keys are visible to every query of the tile
    // and need no mask.  A tile that reaches past n_keys is always a masked
    // one, and key 0 is visible to every query, so each query's running
    // maximum is finite from the first tile on.
    const int unmasked_end = pos0 + t0 + 1;

    // This thread's four 16-byte units of a K tile (row e / 16, dims
    // 4 (e % 16) ..) and of a V tile (row e % 64, dims 4 (e / 64) ..) for
    // e = tid + 256 i.  Rows past the last key read the last key (finite
    // values): their scores are masked, and their probabilities are zero.
    // A tile's loads are issued half an iteration before it is staged (K
    // during the softmax and P.V, V during the next scores), so their
    // latency is spent on work.  The registers are vector-typed: with float4
    // (a struct) the copies global -> registers -> LDS were kept in scratch
    // memory (10% of the kernel's time).
    am_v4f kreg[4], vreg[4];
    auto load_k = [&](int kb) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int e = tid + 256 * i, r = e >> 4, c4 = e & 15;
            kreg[i] = *(const am_v4f*)(kc + (size_t)min(kb + r, n_keys - 1) * kv_dim + g * HD + 4 * c4);
        }
    };
    auto load_v = [&](int kb) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int e = tid + 256 * i, r = e & 63, c4 = e >> 6;
            vreg[i] = *(const am_v4f*)(vc + (size_t)min(kb + r, n_keys - 1) * kv_dim + g * HD + 4 * c4);
        }
    };
    auto store_k = [&]() {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int e = tid + 256 * i, r = e >> 4, c4 = e & 15;
            *(am_v4f*)&s_k[r][4 * c4] = kreg[i];
        }
    };
    auto store_v = [&]() {  // transposed
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int e = tid + 256 * i, r = e & 63, c4 = e >> 6;
            s_vt[4 * c4][r] = vreg[i][0];
            s_vt[4 * c4 + 1][r] = vreg[i][1];
            s_vt[4 * c4 + 2][r] = vreg[i][2];
            s_vt[4 * c4 + 3][r] = vreg[i][3];
        }
    };
    load_k(0);
    load_v(0);
    store_k();
    __syncthreads();
    for (int k0 = 0; k0 < n_keys; k0 += PT) {
        const bool more = k0 + PT < n_keys;
        // S^T for 4 subtiles of 16 keys: sc[t][r] = score of key k0 + 16 t + 4 lk + r
        am_v4f sc[4];
#pragma unroll
        for (int t = 0; t < 4; t++) {
            // one subtile's operand reads at a time (hoisted together they
            // would take 64 VGPRs)
            asm volatile("" ::: "memory");
            const float* kr = &s_k[16 * t + li][16 * lk];
            am_v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const am_v4f k4 = *(const am_v4f*)(kr + 4 * c);
#pragma unroll
                for (int j = 0; j < 4; j++) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(k4[j], qa[4 * c + j], acc, 0, 0, 0);
            }
            sc[t] = acc;
        }
        // this tile's V (s_vt was last read by the previous P.V, before the
        // barrier that ended it); then the next tile's K rows are requested
        store_v();
        if (more) load_k(k0 + PT);
        // scale, causal mask (the tile's last keys only), online softmax
        // (the four lanes of query tq hold its 64 scores)
        float tmax = -INFINITY;
        if (k0 + PT > unmasked_end) {
#pragma unroll
            for (int t = 0; t < 4; t++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int kk = k0 + 16 * t + 4 * lk + r;
                    sc[t][r] = kk <= limit ? sc[t][r] * scale2 : -INFINITY;
                    tmax = fmaxf(tmax, sc[t][r]);
                }
        } else {
#pragma unroll
            for (int t = 0; t < 4; t++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    sc[t][r] *= scale2;
                    tmax = fmaxf(tmax, sc[t][r]);
                }
        }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
        // finite (see unmasked_end); exp2(-inf) = 0 covers the first tile's
        // alpha and the masked scores
        const float mn = fmaxf(mrow, tmax);
        const float alpha = __builtin_amdgcn_exp2f(mrow - mn);
        float rsum = 0.0f;
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float p = __builtin_amdgcn_exp2f(sc[t][r] - mn);
                sc[t][r] = p;
                rsum += p;
            }
        // the row sum stays split over the four lanes until the end
        lpart = lpart * alpha + rsum;
        mrow = mn;
        __syncthreads();  // V staged; every wavefront is done with s_k
        // O^T[dt] = alpha O^T[dt] + V^T[16 dt + li][keys] P^T[keys][tq] over the 64 keys
#pragma unroll
        for (int dt = 0; dt < 4; dt++) {
            asm volatile("" ::: "memory");
            am_v4f acc = o[dt] * alpha;
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const am_v4f v4 = *(const am_v4f*)&s_vt[16 * dt + li][16 * t + 4 * lk];
#pragma unroll
                for (int s = 0; s < 4; s++) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(v4[s], sc[t][s], acc, 0, 0, 0);
            }
            o[dt] = acc;
        }
        if (more) {
            store_k();
            load_v(k0 + PT);
        }
        __syncthreads();  // the next K staged; every wavefront is done with s_vt
    }
    float lrow = lpart + __shfl_xor(lpart, 16, 64);
    lrow += __shfl_xor(lrow, 32, 64);
    const float inv = 1.0f / lrow;
    float y[4][4];
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
        for (int c = 0; c < 4; c++) y[dt][c] = o[dt][c] * inv;
    if (out != nullptr && tq < m_rows) {
#pragma unroll
        for (int dt = 0; dt < 4; dt++) {
            float* dst = out + (size_t)tq * q_dim + h * HD + 16 * dt + 4 * lk;
            *(float4*)dst = make_float4(y[dt][0], y[dt][1], y[dt][2], y[dt][3]);
        }
    }
    if (act_q != nullptr) {
        // The row's Q8_0 blocks (the o projection's input), as quantize8_kernel
        // forms them from the stored row: block b of this head is dims
        // 32 b .. 32 b + 31, eight on each of the lanes li + 16 lk (dt = 2 b,
        // 2 b + 1); their maximum over those four lanes.
#pragma unroll
        for (int b = 0; b < 2; b++) {
            float mx = 0.0f;
#pragma unroll
            for (int dt = 2 * b; dt < 2 * b + 2; dt++)
#pragma unroll
                for (int c = 0; c < 4; c++) mx = fmaxf(mx, fabsf(y[dt][c]));
            mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            const float scale = sq_q8_scale(fmaxf(mx, 0.0f)), qinv = sq_q8_inv(scale);
            if (tq < m_rows) {
#pragma unroll
                for (int dt = 2 * b; dt < 2 * b + 2; dt++) {
                    unsigned wq = 0;
#pragma unroll
                    for (int c = 0; c < 4; c++) wq |= (unsigned)(uint8_t)sq_q8_quant(y[dt][c], qinv) << (8 * c);
                    *(unsigned*)(act_q + (size_t)tq * q_dim + h * HD + 16 * dt + 4 * lk) = wq;
                }
                if (lk == 0) act_d[(size_t)tq * (q_dim / 32) + h * (HD / 32) + b] = sq_f32_to_f16(scale);
            }
        }
    }
}

// The same attention with its products on the f16 matrix instructions
// (v_mfma_f32_16x16x32_f16, 16 times the fp32 rate): every f32 operand x is
// split into hi = f16(x) (round to nearest even) and lo = f16((x - hi) 2^11),
// and a product a b is formed as hi_a hi_b + 2^-11 (hi_a lo_b + lo_a hi_b),
// accumulated in f32.  hi carries x's leading 11 bits and lo the next 11,
// so the dropped lo_a lo_b term and lo's rounding leave a relative error of
// about 2^-22 per product, against 2^-24 for one f32 rounding: the attention
// output stays within f32 rounding noise of the fp32 kernel.  Scaling lo by
// 2^11 keeps it a normal f16 whenever hi is one; q, k and v are scaled by
// 2^-8 before the split (power-of-two scalings, undone exactly in the
// scores and the output), so hi overflows only for |x| >= 2^23.
//
// The operands are split once per layer, before the attention, by
// kv_split_kernel into a workspace of 32-bit words (two halves each), with
// one 64-position tile of a kv head g as 16 KB in one piece:
//   K: word (g KP + pos) 64 + w: w < 32 the hi halves of dims 2w, 2w + 1,
//      w >= 32 the lo halves of dims 2 (w - 32), +1;
//   V: word ((g KT + tile) 64 + dim) 64 + w: hi (w < 32) or lo halves of
//      the tile's keys at slots 2 w', 2 w' + 1 (w' = w mod 32), in the slot
//      order of the P.V operands below;
// KP = 64 KT is the key capacity rounded up to a tile; positions past the
// last key of the last tile hold zeros.  The attention kernel then stages
// each tile with direct global -> LDS loads; every query tile of the same kv
// head reads the same split words.
//
// Layout: lane l supplies A[l % 16][8 (l / 16) .. +7] and
// B[8 (l / 16) .. +7][l % 16]; result r of lane l is D[4 (l / 16) + r][l % 16].
// Scores are formed transposed as in attn_prefill_kernel (S^T = K Q^T, key
// rows as the row operand): lane l holds keys 4 (l / 16) + 0..3 of each
// 16-key subtile for query l % 16.  For O^T = V^T P^T over a 32-key half u of
// the tile, lane l's eight contraction slots 8 (l / 16) + j take keys
// 32 u + 4 (l / 16) + j (j < 4) and 32 u + 16 + 4 (l / 16) + j - 4 (j >= 4),
// which are its own probabilities of subtiles 2 u and 2 u + 1; V^T is staged
// in LDS with its keys in that slot order, so the probabilities never leave
// the registers here either.
typedef _Float16 as_v8h __attribute__((ext_vector_type(8)));
typedef _Float16 as_v2h __attribute__((ext_vector_type(2)));
typedef float as_v2f __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) int8_t lds_i8;
// A direct global -> LDS load (global_load_lds_dwordx4 for 16 bytes per lane,
// global_load_lds_dword for 4): lane l reads `base + off` (base the same on
// every lane, in SGPRs) and its bytes land at lds + SIZE * l (lds the same on
// every lane: it goes to M0).  Issued from inline assembly, so the compiler's
// wait-count pass does not see it; the caller waits for its loads itself
// (s_waitcnt vmcnt) before a barrier.  M0 is named as clobbered; the compiler
// sets M0 itself before each instruction of its own that reads it.
template <int SIZE>
__device__ __forceinline__ void dma_to_lds(const void* base, uint32_t off, lds_i8* lds) {
    static_assert(SIZE == 4 || SIZE == 16, "dword or dwordx4");
    const unsigned m0 = __builtin_amdgcn_readfirstlane((unsigned)(size_t)lds);
    if constexpr (SIZE == 16)
        asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(m0)
                     : "memory", "m0");
    else
        asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(off), "s"(base), "s"(m0)
                     : "memory", "m0");
}
// s_waitcnt immediate: no vector-memory and no LDS operation outstanding
// (vmcnt 0, lgkmcnt 0; the export counter not waited on)
constexpr int att_wait_mem() { return 0x7 << 4; }

// 16-byte unit swizzle of LDS row r (only bits 0-3 of r count: an operand
// read starts at a row that is a multiple of 16): rows of one parity take eight distinct
// values over r / 2, and rows 0-7 (8-15) of one parity four values that
// differ from each other in bits 0 and 2, so lanes that read one unit of 16
// consecutive rows, or units two apart of 8 rows, hit distinct banks.
__device__ __forceinline__ int att_swz(int r) {
    return ((r >> 1) & 1) | (((r >> 2) & 1) << 2) | (((r >> 3) & 1) << 1);
}
constexpr float kLoUp = 2048.0f;            // 2^11
constexpr float kLoDown = 1.0f / 2048.0f;   // 2^-11
constexpr float kPre = 1.0f / 256.0f;       // 2^-8 on q, k and v

// hi and lo of two values scaled by `pre`, each pair packed into 32 bits
__device__ __forceinline__ void split2(float a, float b, float pre, uint32_t& hi, uint32_t& lo) {
    const as_v2f v = {a * pre, b * pre};
    const as_v2h h = __builtin_convertvector(v, as_v2h);
    const as_v2f back = __builtin_convertvector(h, as_v2f);
    const as_v2h l = __builtin_convertvector((v - back) * kLoUp, as_v2h);
    hi = __builtin_bit_cast(uint32_t, h);
    lo = __builtin_bit_cast(uint32_t, l);
}
__device__ __forceinline__ as_v8h pack8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    typedef uint32_t u4 __attribute__((ext_vector_type(4)));
    return __builtin_bit_cast(as_v8h, u4{a, b, c, d});
}
// slot of key kk (0..63) in the staged V^T rows
__device__ __forceinline__ int v_slot(int kk) {
    const int u = kk >> 5, k = kk & 31;
    return 32 * u + 8 * ((k & 15) >> 2) + 4 * (k >> 4) + (k & 3);
}

// One (64-position tile, kv head) of a layer's K and V rows into the split
// workspace (layout above); grid (tiles, kv heads), 256 threads.  Thread t
// splits K units e = t + 256 i (row e / 16, dims 4 (e % 16) ..) and V key
// pairs (keys 2 p, 2 p + 1, p = e % 32, dims 4 (e / 32) ..), e = t + 256 i.
__global__ __launch_bounds__(256) void kv_split_kernel(const float* __restrict__ kc, const float* __restrict__ vc,
                                                       int n_keys, int kv_dim, int key_cap,
                                                       uint32_t* __restrict__ kvs) {
    const int tile = blockIdx.x, g = blockIdx.y, tid = threadIdx.x;
    const int n_kv = gridDim.y;
    const int k0 = tile * PT;
    uint32_t* const ks = kvs + ((size_t)g * key_cap + k0) * 64;
    uint32_t* const vs = kvs + (size_t)n_kv * key_cap * 64 + ((size_t)g * (key_cap / PT) + tile) * 64 * 64;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int e = tid + 256 * i, r = e >> 4, c4 = e & 15;
        am_v4f x = {0.f, 0.f, 0.f, 0.f};
        if (k0 + r < n_keys) x = *(const am_v4f*)(kc + (size_t)(k0 + r) * kv_dim + g * HD + 4 * c4);
        uint32_t h0, l0, h1, l1;
        split2(x[0], x[1], kPre, h0, l0);
        split2(x[2], x[3], kPre, h1, l1);
        *(uint2*)(ks + r * 64 + 2 * c4) = make_uint2(h0, h1);
        *(uint2*)(ks + r * 64 + 32 + 2 * c4) = make_uint2(l0, l1);
    }
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int e = tid + 256 * i, p = e & 31, c4 = e >> 5;
        am_v4f x[2];
#pragma unroll
        for (int s = 0; s < 2; s++) {
            x[s] = am_v4f{0.f, 0.f, 0.f, 0.f};
            if (k0 + 2 * p + s < n_keys)
                x[s] = *(const am_v4f*)(vc + (size_t)(k0 + 2 * p + s) * kv_dim + g * HD + 4 * c4);
        }
        const int w = v_slot(2 * p) >> 1;
#pragma unroll
        for (int d = 0; d < 4; d++) {
            uint32_t hv, lv;
            split2(x[0][d], x[1][d], kPre, hv, lv);
            vs[(4 * c4 + d) * 64 + w] = hv;
            vs[(4 * c4 + d) * 64 + 32 + w] = lv;
        }
    }
}

__global__ __launch_bounds__(256, 4) void attn_prefill_split_kernel(const float* __restrict__ q,
                                                                  const uint32_t* __restrict__ kvs,
                                                                  int key_cap, int pos0,
                                                                  int m_rows, int n_heads, int n_kv_heads,
                                                                  float* __restrict__ out,
                                                                  int8_t* __restrict__ act_q,
                                                                  uint16_t* __restrict__ act_d) {
    // K [key][dim] and V^T [dim][key slot], hi and lo halves, 128-byte rows
    // of eight 16-byte units.  Row r keeps logical unit u at physical unit
    // u ^ att_swz(r): the operand reads (16 rows 16 t + l % 16, one unit per
    // lane group l / 16) then fall in distinct banks.  Each lo array starts
    // 128 bytes past a multiple of 256 from its hi array, so that the 16
    // lanes of a staging store (8 on a hi row, 8 on the same lo row) also do.
    typedef _Float16 Row[HD];
    constexpr int ARR = PT * HD, LO = ARR + 64;  // halves
    __shared__ __attribute__((aligned(16))) _Float16 s_buf[2 * (LO + ARR)];
    Row* const s_kh = (Row*)s_buf;
    Row* const s_kl = (Row*)(s_buf + LO);
    Row* const s_vh = (Row*)(s_buf + LO + ARR);
    Row* const s_vl = (Row*)(s_buf + 2 * LO + ARR);

    const int h = blockIdx.x;
    // query tiles in the order of attn_prefill_kernel (equal causal work per CU)
    int ty = blockIdx.y;
    if ((gridDim.y & 3) == 0) {
        const int B = gridDim.y >> 2, k = ty / B, a = ty % B;
        ty = k == 0 ? a : k == 1 ? 4 * B - 1 - a : k == 2 ? B + a : 3 * B - 1 - a;
    }
    const int t0 = ty * PT;
    const int g = h / (n_heads / n_kv_heads);
    const int q_dim = n_heads * HD;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int li = lane & 15, lk = lane >> 4;
    const uint32_t* const ks = kvs + (size_t)g * key_cap * 64;
    const uint32_t* const vs = kvs + (size_t)n_kv_heads * key_cap * 64 + (size_t)g * key_cap * 64;
    // base-2 scores of the 2^-8-scaled operands: s' = (q . k) 2^16 scale log2(e)
    const float scale2 = (1.0f / sqrtf((float)HD)) * 1.44269504088896341f * 65536.0f;

    // this lane's query (t0 + 16 wave + li), dims 32 c + 8 lk .. +7 as the
    // column operand of chunk c
    const int tq = t0 + 16 * wave + li;
    as_v8h qh[2], ql[2];
#pragma unroll
    for (int c = 0; c < 2; c++) {
        float x[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        if (tq < m_rows) {
            const float* src = q + (size_t)tq * q_dim + h * HD + 32 * c + 8 * lk;
            const float4 a = *(const float4*)src, b = *(const float4*)(src + 4);
            x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
            x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
        }
        uint32_t hi[4], lo[4];
#pragma unroll
        for (int j = 0; j < 4; j++) split2(x[2 * j], x[2 * j + 1], kPre, hi[j], lo[j]);
        qh[c] = pack8(hi[0], hi[1], hi[2], hi[3]);
        ql[c] = pack8(lo[0], lo[1], lo[2], lo[3]);
    }
    // online softmax state as in attn_prefill_kernel; the output accumulates
    // as oh + 2^-11 ox, oh[dt][r] / ox[dt][r] at O^T[16 dt + 4 lk + r][tq]
    float mrow = -INFINITY, lpart = 0.0f;
    am_v4f oh[4], ox[4];
#pragma unroll
    for (int dt = 0; dt < 4; dt++) oh[dt] = ox[dt] = am_v4f{0.f, 0.f, 0.f, 0.f};

    const int last_q = min(t0 + PT, m_rows) - 1;
    const int n_keys = pos0 + last_q + 1;
    const int limit = pos0 + tq;
    const int unmasked_end = pos0 + t0 + 1;

    // Staging: a tile's K (V) split words are 16 KB in one piece (64 rows of
    // 32 hi words, then 32 lo words: 256 bytes per row), copied with direct
    // global -> LDS loads (no registers held): each 64-lane load writes 1 KB,
    // eight 128-byte LDS rows, lane j physical unit j % 8 of row j / 8, so it
    // reads the logical unit (j % 8) ^ att_swz(row) of that row.  Wavefront w
    // loads rows 8 q .. 8 q + 7, q = w and w + 4, of each of the hi and lo
    // arrays (the same lane offsets serve K and V).  A tile's loads are
    // issued half an iteration before it is used (K during P.V, V during the
    // next scores).  Before each barrier a wavefront waits for its own loads
    // and for its own LDS reads: the compiler may place the matrix
    // instruction that consumes a read after the barrier, and the read must
    // have completed before any wavefront's next loads overwrite the tile.
    uint32_t off[2][2];  // [hi/lo][q = w, w + 4]: byte offsets within a tile
#pragma unroll
    for (int hl = 0; hl < 2; hl++)
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const int r = 8 * (wave + 4 * k) + (lane >> 3);
            const int u = (lane & 7) ^ att_swz(r);
            off[hl][k] = (uint32_t)(4 * (r * 64 + 32 * hl + 4 * u));
        }
    lds_i8* const lds_base = (lds_i8*)(int8_t*)s_buf;
    lds_i8* const lk_dst[2] = {lds_base, lds_base + 2 * LO};
    lds_i8* const lv_dst[2] = {lds_base + 2 * (LO + ARR), lds_base + 2 * (2 * LO + ARR)};
    auto issue = [&](const uint32_t* src, lds_i8* const (&dst)[2]) {
#pragma unroll
        for (int hl = 0; hl < 2; hl++)
#pragma unroll
            for (int k = 0; k < 2; k++) dma_to_lds<16>(src, off[hl][k], dst[hl] + 1024 * (wave + 4 * k));
    };
    auto wait_own = [] { __builtin_amdgcn_s_waitcnt(att_wait_mem()); };
    auto barrier = [] {
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    };
    issue(ks, lk_dst);
    issue(vs, lv_dst);
    wait_own();
    barrier();
    for (int k0 = 0; k0 < n_keys; k0 += PT) {
        const bool more = k0 + PT < n_keys;
        // S^T for 4 subtiles of 16 keys: sc[t][r] = score of key k0 + 16 t + 4 lk + r
        am_v4f sc[4];
#pragma unroll
        for (int t = 0; t < 4; t++) {
            asm volatile("" ::: "memory");
            am_v4f hh = {0.f, 0.f, 0.f, 0.f}, xx = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < 2; c++) {
                const int pu = 8 * ((4 * c + lk) ^ att_swz(li));
                const as_v8h kh = *(const as_v8h*)&s_kh[16 * t + li][pu];
                const as_v8h kl = *(const as_v8h*)&s_kl[16 * t + li][pu];
                hh = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, qh[c], hh, 0, 0, 0);
                xx = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, ql[c], xx, 0, 0, 0);
                xx = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl, qh[c], xx, 0, 0, 0);
            }
#pragma unroll
            for (int r = 0; r < 4; r++) sc[t][r] = fmaf(xx[r], kLoDown, hh[r]);
        }
        float tmax = -INFINITY;
        if (k0 + PT > unmasked_end) {
#pragma unroll
            for (int t = 0; t < 4; t++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int kk = k0 + 16 * t + 4 * lk + r;
                    sc[t][r] = kk <= limit ? sc[t][r] * scale2 : -INFINITY;
                    tmax = fmaxf(tmax, sc[t][r]);
                }
        } else {
#pragma unroll
            for (int t = 0; t < 4; t++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    sc[t][r] *= scale2;
                    tmax = fmaxf(tmax, sc[t][r]);
                }
        }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
        const float mn = fmaxf(mrow, tmax);
        const float alpha = __builtin_amdgcn_exp2f(mrow - mn);
        float rsum = 0.0f;
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float p = __builtin_amdgcn_exp2f(sc[t][r] - mn);
                sc[t][r] = p;
                rsum += p;
            }
        lpart = lpart * alpha + rsum;
        mrow = mn;
        // P^T operands of the two 32-key halves
        as_v8h ph[2], pl[2];
#pragma unroll
        for (int u = 0; u < 2; u++) {
            uint32_t hi[4], lo[4];
            split2(sc[2 * u][0], sc[2 * u][1], 1.0f, hi[0], lo[0]);
            split2(sc[2 * u][2], sc[2 * u][3], 1.0f, hi[1], lo[1]);
            split2(sc[2 * u + 1][0], sc[2 * u + 1][1], 1.0f, hi[2], lo[2]);
            split2(sc[2 * u + 1][2], sc[2 * u + 1][3], 1.0f, hi[3], lo[3]);
            ph[u] = pack8(hi[0], hi[1], hi[2], hi[3]);
            pl[u] = pack8(lo[0], lo[1], lo[2], lo[3]);
        }
        wait_own();  // this wavefront's V loads and K reads
        barrier();   // V staged; every wavefront is done with s_kh / s_kl
        if (more) issue(ks + (size_t)(k0 + PT) * 64, lk_dst);
#pragma unroll
        for (int dt = 0; dt < 4; dt++) {
            asm volatile("" ::: "memory");
            am_v4f ah = oh[dt] * alpha, ax = ox[dt] * alpha;
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const int pu = 8 * ((4 * u + lk) ^ att_swz(li));
                const as_v8h vh = *(const as_v8h*)&s_vh[16 * dt + li][pu];
                const as_v8h vl = *(const as_v8h*)&s_vl[16 * dt + li][pu];
                ah = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh, ph[u], ah, 0, 0, 0);
                ax = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh, pl[u], ax, 0, 0, 0);
                ax = __builtin_amdgcn_mfma_f32_16x16x32_f16(vl, ph[u], ax, 0, 0, 0);
            }
            oh[dt] = ah;
            ox[dt] = ax;
        }
        wait_own();  // this wavefront's loads of the next K and its V reads
        barrier();   // the next K staged; every wavefront is done with s_vh / s_vl
        if (more) issue(vs + (size_t)(k0 + PT) * 64, lv_dst);
    }
    float lrow = lpart + __shfl_xor(lpart, 16, 64);
    lrow += __shfl_xor(lrow, 32, 64);
    const float inv = 256.0f / lrow;  // undoes v's 2^-8
    float y[4][4];
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
        for (int c = 0; c < 4; c++) y[dt][c] = fmaf(ox[dt][c], kLoDown, oh[dt][c]) * inv;
    if (out != nullptr && tq < m_rows) {
#pragma unroll
        for (int dt = 0; dt < 4; dt++) {
            float* dst = out + (size_t)tq * q_dim + h * HD + 16 * dt + 4 * lk;
            *(float4*)dst = make_float4(y[dt][0], y[dt][1], y[dt][2], y[dt][3]);
        }
    }
    if (act_q != nullptr) {
        // the row's Q8_0 blocks, as attn_prefill_kernel forms them
#pragma unroll
        for (int b = 0; b < 2; b++) {
            float mx = 0.0f;
#pragma unroll
            for (int dt = 2 * b; dt < 2 * b + 2; dt++)
#pragma unroll
                for (int c = 0; c < 4; c++) mx = fmaxf(mx, fabsf(y[dt][c]));
            mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            const float scale = sq_q8_scale(fmaxf(mx, 0.0f)), qinv = sq_q8_inv(scale);
            if (tq < m_rows) {
#pragma unroll
                for (int dt = 2 * b; dt < 2 * b + 2; dt++) {
                    unsigned wq = 0;
#pragma unroll
                    for (int c = 0; c < 4; c++) wq |= (unsigned)(uint8_t)sq_q8_quant(y[dt][c], qinv) << (8 * c);
                    *(unsigned*)(act_q + (size_t)tq * q_dim + h * HD + 16 * dt + 4 * lk) = wq;
                }
                if (lk == 0) act_d[(size_t)tq * (q_dim / 32) + h * (HD / 32) + b] = sq_f32_to_f16(scale);
            }
        }
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

// Which prefill attention runs.  Prompts whose keys fit in kF32MaxKeys take
// attn_prefill_kernel (fp32 matrix instructions): its one small launch beats
// the K/V split pass plus the split-f16 kernel there (32 keys: 6.6 against
// 3.9 + 6.1 us; 128 keys: 10.8 against 4.5 + 7.6 us); longer ones take the
// split-f16 kernel (2048 keys: 176 against 5.5 + 74 us).
// SQUIRREL_ATTN_F32=1 pins the fp32 kernel and =0 the split one (test and
// measurement aids).
constexpr int kF32MaxKeys = 3 * PT;
bool attn_use_f32(int n_keys) {
    const char* e = getenv("SQUIRREL_ATTN_F32");
    if (e && !strcmp(e, "1")) return true;
    if (e && !strcmp(e, "0")) return false;
    return n_keys <= kF32MaxKeys;
}

}  // namespace

int launch_attn_decode(hipStream_t s, const float* q, const float* kcache, const float* vcache, const int* pos,
                       int n_heads, int n_kv_heads, int head_dim, int max_tiles, float* part_m, float* part_l,
                       float* part_o, unsigned* counters, float* attn, int8_t* act_q, uint16_t* act_d) {
    if (head_dim != HD) return set_error(SQ_ERR_UNSUPPORTED, "attention kernels are built for head_dim 64");
    const int G = n_heads / n_kv_heads;
    dim3 grid(n_kv_heads, max_tiles);
#define SQ_ATTN_LAUNCH(GG)                                                                                      \
    hipLaunchKernelGGL(attn_decode_kernel<GG>, grid, dim3(256), 0, s, q, kcache, vcache, pos, n_kv_heads,      \
                       max_tiles, part_m, part_l, part_o, counters, attn, act_q, act_d)
    switch (G) {
        case 1: SQ_ATTN_LAUNCH(1); break;
        case 2: SQ_ATTN_LAUNCH(2); break;
        case 4: SQ_ATTN_LAUNCH(4); break;
        case 8: SQ_ATTN_LAUNCH(8); break;
        default: return set_error(SQ_ERR_UNSUPPORTED, "GQA group size must be 1, 2, 4 or 8");
    }
#undef SQ_ATTN_LAUNCH
    return check_launch("attn_decode");
}

size_t attn_split_words(int max_keys, int n_kv_heads) {
    const size_t cap = ((size_t)max_keys + PT - 1) / PT * PT;
    return 2 * (size_t)n_kv_heads * cap * 64;
}

int launch_attn_prefill(hipStream_t s, const float* q, const float* kcache, const float* vcache, int pos0,
                        int m, int n_heads, int n_kv_heads, int head_dim, uint32_t* kv_split, int max_keys,
                        float* out, int8_t* act_q, uint16_t* act_d) {
    if (head_dim != HD) return set_error(SQ_ERR_UNSUPPORTED, "attention kernels are built for head_dim 64");
    const int n_keys = pos0 + m;
    if (n_keys > max_keys) return set_error(SQ_ERR_SHAPE, "attn_prefill: keys beyond the split workspace");
    dim3 grid(n_heads, (m + PT - 1) / PT);
    if (attn_use_f32(n_keys)) {
        hipLaunchKernelGGL(attn_prefill_kernel, grid, dim3(256), 0, s, q, kcache, vcache, pos0, m, n_heads,
                           n_kv_heads, out, act_q, act_d);
        return check_launch("attn_prefill");
    }
    const int key_cap = (max_keys + PT - 1) / PT * PT;
    hipLaunchKernelGGL(kv_split_kernel, dim3((n_keys + PT - 1) / PT, n_kv_heads), dim3(256), 0, s, kcache, vcache,
                       n_keys, n_kv_heads * HD, key_cap, kv_split);
    int st = check_launch("kv_split");
    if (st) return st;
    hipLaunchKernelGGL(attn_prefill_split_kernel, grid, dim3(256), 0, s, q, kv_split, key_cap, pos0, m, n_heads,
                       n_kv_heads, out, act_q, act_d);
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
