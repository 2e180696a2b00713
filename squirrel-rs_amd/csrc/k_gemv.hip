// Batch-1 matvec kernels for the decode step.
//
// out[row] = <activation row, weight row>, one output row per (wavefront,
// slot).  Lane L of a wavefront owns weight blocks L, L+64, ... of every row
// it processes, so a wavefront reads each row as contiguous 2 KB segments
// (Q8_0 payload) with 16-byte loads, and the lane's activation blocks stay in
// registers for every row.  Each wavefront keeps R rows in flight.
//
// Load ordering matters on CDNA: a wavefront's loads complete in issue order,
// so the prologue's inputs (the hidden row, norm gains, the RoPE position)
// are requested first, the first tile's weights right after them, and the
// prologue arithmetic then runs while the weight stream is in flight.  With
// a grid smaller than the tile count, later tiles are prefetched one tile
// ahead into a second register buffer.
//
// Arithmetic per weight block follows the reference:
//   A8 (integer path, src/kernels/dot_prod.rs:378-403):
//       isum = sum(qa*qw) exactly in i32 (v_dot4_i32_i8);
//       term = (f32(isum) * sa) * sw, then summed over blocks.
//   A32 (f32 activations, dot_prod.rs:86-96, 255-270, 464-472):
//       block_acc = sum(a*w), term = block_acc * sw.
// The per-block terms are the reference's; only the order in which blocks
// are summed differs (lane partials, then a wavefront butterfly).
#include "launch.h"

namespace sq {

namespace {

constexpr int kPad = 36;  // f32 activation LDS stride per 32-block (bank spread)

template <int WT>
struct WBlk;
template <>
struct WBlk<WT_Q8_0> { static constexpr int DW = 8; };   // 32 B payload
template <>
struct WBlk<WT_Q4_0> { static constexpr int DW = 4; };   // 16 B payload
template <>
struct WBlk<WT_BF16> { static constexpr int DW = 16; };  // 64 B payload

template <int WT, bool A8, int NBL, int R, int WAVES, int PRO, int EPI, int NBUF>
struct Gemv {
    static constexpr int NT = WAVES * 64;
    static constexpr int TR = WAVES * R;  // rows per tile
    static constexpr int KMAX = NBL * 64 * 32;
    static constexpr int DW = WBlk<WT>::DW;
    static constexpr int EPT = (KMAX + NT - 1) / NT;  // prologue elements per thread
};

// Dequantized element i of embedding row `tok` (dequantize_into,
// src/kernels/dot_prod.rs:409-414, 440-446, 524-528): exact.
__device__ __forceinline__ float embed_elem(const MatView& t, uint32_t tok, int i) {
    const int K = t.k, KB = K >> 5;
    const int blk = i >> 5, j = i & 31;
    if (t.wtype == WT_Q8_0) {
        const float sc = sq_f16_to_f32(t.scale[(size_t)tok * KB + blk]);
        return sc * (float)((const int8_t*)t.qs)[(size_t)tok * K + i];
    }
    if (t.wtype == WT_Q4_0) {
        const uint8_t* qs = (const uint8_t*)t.qs + (size_t)tok * (K / 2) + blk * 16;
        const float sc = sq_f16_to_f32(t.scale[(size_t)tok * KB + blk]);
        const int q = j < 16 ? (qs[j] & 0x0F) : (qs[j - 16] >> 4);
        return sc * (float)(q - 8);
    }
    return sq_bf16_to_f32(((const uint16_t*)t.qs)[(size_t)tok * K + i]);
}

template <int WT, bool A8, int NBL, int R, int WAVES, int PRO, int EPI, int NBUF>
__global__ __launch_bounds__(WAVES * 64) void gemv_kernel(GemvArgs a) {
    using G = Gemv<WT, A8, NBL, R, WAVES, PRO, EPI, NBUF>;
    constexpr int DW = G::DW;
    constexpr int TR = G::TR;
    static_assert(EPI != EPI_GATEUP || TR == 64, "gate/up tiles pair 32 gate with 32 up rows");
    static_assert(EPI != EPI_QKV || (R % 2) == 0, "RoPE pairs stay inside one wavefront");

    __shared__ __attribute__((aligned(16))) int8_t s_qs[A8 ? G::KMAX : 16];
    __shared__ uint16_t s_d[A8 ? G::KMAX / 32 : 1];
    __shared__ int s_asum[(A8 && WT == WT_Q4_0) ? G::KMAX / 32 : 1];
    __shared__ __attribute__((aligned(16))) float s_x[A8 ? 4 : (G::KMAX / 32) * kPad];
    __shared__ float s_red[WAVES];
    __shared__ float s_gu[64];
    __shared__ float s_bv[WAVES];
    __shared__ int s_bi[WAVES];
    __shared__ int s_bn[WAVES];

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int K = a.w.k;
    const int KB = K >> 5;
    const int n_tiles = (EPI == EPI_GATEUP) ? (a.n_rows >> 5) : (a.n_rows + TR - 1) / TR;

    const uint8_t* wbase = (const uint8_t*)a.w.qs;
    const size_t row_bytes = (size_t)KB * (DW * 4);

    auto row_of = [&](int t, int slot) -> int {
        if constexpr (EPI == EPI_GATEUP) {
            return slot < 32 ? t * 32 + slot : a.n_rows + t * 32 + (slot - 32);
        } else {
            return t * TR + slot;
        }
    };
    auto row_valid = [&](int t, int slot) -> bool {
        if constexpr (EPI == EPI_GATEUP) {
            return t < n_tiles;
        } else {
            return t * TR + slot < a.n_rows;
        }
    };

    // Two statically named weight buffers: indexing a register array with a
    // run-time buffer index would move it to scratch memory.
    int W0[R][NBL][DW], W1[NBUF == 2 ? R : 1][NBL][DW];
    uint16_t D0[R][NBL], D1[NBUF == 2 ? R : 1][NBL];

    auto load_tile = [&](auto& Wb, auto& Db, int t) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int slot = wave * R + r;
            const bool vr = row_valid(t, slot);
            const int row = vr ? row_of(t, slot) : 0;
#pragma unroll
            for (int b = 0; b < NBL; b++) {
                const int blk = lane + 64 * b;
                if (vr && blk < KB) {
                    const sq_v4i* p = (const sq_v4i*)(wbase + (size_t)row * row_bytes + (size_t)blk * (DW * 4));
#pragma unroll
                    for (int v = 0; v < DW / 4; v++) {
                        sq_v4i x = __builtin_nontemporal_load(p + v);
                        Wb[r][b][4 * v + 0] = x.x;
                        Wb[r][b][4 * v + 1] = x.y;
                        Wb[r][b][4 * v + 2] = x.z;
                        Wb[r][b][4 * v + 3] = x.w;
                    }
                    if constexpr (WT != WT_BF16) Db[r][b] = a.w.scale[(size_t)row * KB + blk];
                    else Db[r][b] = 0;
                } else {
#pragma unroll
                    for (int v = 0; v < DW; v++) Wb[r][b][v] = 0;
                    Db[r][b] = 0;
                }
            }
        }
    };

    int t = blockIdx.x;

    // ------------------------------------------------- prologue loads first
    float xv[PRO == PRO_NORM ? G::EPT : 1];
    float nw[PRO == PRO_NORM ? G::EPT : 1];
    int AQ[NBL][8];
    float AS[NBL];
    int ASUM[NBL];
    if constexpr (PRO == PRO_NORM) {
        const bool from_embed = a.embd.qs != nullptr;
        // an id past the table is the reference's panic (embedding.rs:43-44):
        // the read is clamped in bounds and the error word tells the host
        const uint32_t tok_in = from_embed ? *a.token : 0u;
        const uint32_t tok = min(tok_in, (uint32_t)(a.embd.rows - 1));
        if (tok_in != tok && t == 0 && tid == 0) *a.id_error = 1u;
#pragma unroll
        for (int j = 0; j < G::EPT; j++) {
            const int i = tid + j * G::NT;
            const bool vi = i < K;
            xv[j] = vi ? (from_embed ? embed_elem(a.embd, tok, i) : a.x[i]) : 0.0f;
            nw[j] = vi ? a.norm_w[i] : 0.0f;
        }
    } else if constexpr (PRO == PRO_Q8) {
#pragma unroll
        for (int b = 0; b < NBL; b++) {
            const int blk = lane + 64 * b;
            if (blk < KB) {
                const int4* p = (const int4*)(a.aq + blk * 32);
                int4 x0 = p[0], x1 = p[1];
                AQ[b][0] = x0.x; AQ[b][1] = x0.y; AQ[b][2] = x0.z; AQ[b][3] = x0.w;
                AQ[b][4] = x1.x; AQ[b][5] = x1.y; AQ[b][6] = x1.z; AQ[b][7] = x1.w;
                AS[b] = sq_f16_to_f32(a.ad[blk]);
            } else {
#pragma unroll
                for (int v = 0; v < 8; v++) AQ[b][v] = 0;
                AS[b] = 0.0f;
            }
            ASUM[b] = 0;
        }
    }
    // The RoPE position, read before the weight stream is requested.
    int qkv_pos = 0;
    if constexpr (EPI == EPI_QKV) qkv_pos = *a.pos;

    if (t < n_tiles) load_tile(W0, D0, t);

    // ---------------------------------------------------- prologue compute
    if constexpr (PRO == PRO_NORM) {
        // rms_norm_f32_into (src/kernels/rms_norm.rs:40-56): ss = sum x^2,
        // rms = sqrt(ss/n + eps), y = (x*w)/rms.
        if (a.embd.qs != nullptr && blockIdx.x == 0) {
#pragma unroll
            for (int j = 0; j < G::EPT; j++) {
                const int i = tid + j * G::NT;
                if (i < K) a.hidden_out[i] = xv[j];
            }
        }
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < G::EPT; j++) ss += xv[j] * xv[j];
        ss = sq_wave_sum(ss);
        if (lane == 0) s_red[wave] = ss;
        __syncthreads();
        float tot = 0.0f;
#pragma unroll
        for (int w = 0; w < WAVES; w++) tot += s_red[w];
        const float mean = tot / (float)K;
        const float rms = sqrtf(mean + a.eps);
        const bool tap_y = a.dbg_normed != nullptr && blockIdx.x == 0;
        const bool tap_q = a.dbg_qs != nullptr && blockIdx.x == 0;
#pragma unroll
        for (int j = 0; j < G::EPT; j++) {
            const int i = tid + j * G::NT;
            const bool vi = i < K;
            float y = vi ? (xv[j] * nw[j]) / rms : 0.0f;
            if constexpr (A8) {
                float amax = fmaxf(sq_half_max(fabsf(y)), 0.0f);
                float scale = sq_q8_scale(amax);
                float inv = sq_q8_inv(scale);
                int8_t q = sq_q8_quant(y, inv);
                if (vi) {
                    s_qs[i] = q;
                    if ((i & 31) == 0) s_d[i >> 5] = sq_f32_to_f16(scale);
                }
                if constexpr (WT == WT_Q4_0) {
                    int qi = q;
#pragma unroll
                    for (int o = 16; o >= 1; o >>= 1) qi += __shfl_xor(qi, o, 64);
                    if (vi && (i & 31) == 0) s_asum[i >> 5] = qi;
                }
                if (tap_y && vi) a.dbg_normed[i] = y;
                if (tap_q && vi) {
                    a.dbg_qs[i] = q;
                    if ((i & 31) == 0) a.dbg_d[i >> 5] = sq_f32_to_f16(scale);
                }
            } else {
                if (vi) s_x[(i >> 5) * kPad + (i & 31)] = y;
                if (tap_y && vi) a.dbg_normed[i] = y;
            }
        }
        __syncthreads();
        if constexpr (A8) {
#pragma unroll
            for (int b = 0; b < NBL; b++) {
                const int blk = lane + 64 * b;
                if (blk < KB) {
                    const int4* p = (const int4*)(s_qs + blk * 32);
                    int4 x0 = p[0], x1 = p[1];
                    AQ[b][0] = x0.x; AQ[b][1] = x0.y; AQ[b][2] = x0.z; AQ[b][3] = x0.w;
                    AQ[b][4] = x1.x; AQ[b][5] = x1.y; AQ[b][6] = x1.z; AQ[b][7] = x1.w;
                    AS[b] = sq_f16_to_f32(s_d[blk]);
                    if constexpr (WT == WT_Q4_0) ASUM[b] = s_asum[blk];
                } else {
#pragma unroll
                    for (int v = 0; v < 8; v++) AQ[b][v] = 0;
                    AS[b] = 0.0f;
                    ASUM[b] = 0;
                }
            }
        }
    } else if constexpr (PRO == PRO_Q8) {
        if constexpr (WT == WT_Q4_0) {
#pragma unroll
            for (int b = 0; b < NBL; b++) {
                int sacc = 0;
#pragma unroll
                for (int v = 0; v < 8; v++) sacc = __builtin_amdgcn_sdot4(AQ[b][v], 0x01010101, sacc, false);
                ASUM[b] = sacc;
            }
        }
    } else {  // PRO_F32
        for (int i = tid; i < K; i += G::NT) s_x[(i >> 5) * kPad + (i & 31)] = a.x[i];
        __syncthreads();
    }

    // ------------------------------------------------------------ main loop
    float best_v = -INFINITY;
    int best_i = -1;
    int nan_i = -1;
    auto compute_tile = [&](const auto& Wb, const auto& Db, int t) {
        float res[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            float acc = 0.0f;
#pragma unroll
            for (int b = 0; b < NBL; b++) {
                const int blk = lane + 64 * b;
                if (blk >= KB) continue;
                if constexpr (A8 && WT == WT_Q8_0) {
                    int isum = 0;
#pragma unroll
                    for (int v = 0; v < 8; v++) isum = __builtin_amdgcn_sdot4(AQ[b][v], Wb[r][b][v], isum, false);
                    acc += sq_q_term(isum, AS[b], sq_f16_to_f32(Db[r][b]));
                } else if constexpr (A8 && WT == WT_Q4_0) {
                    int isum = 0;
#pragma unroll
                    for (int v = 0; v < 4; v++) {
                        const int dw = Wb[r][b][v];
                        const int lo = dw & 0x0F0F0F0F;
                        const int hi = (dw >> 4) & 0x0F0F0F0F;
                        isum = __builtin_amdgcn_sdot4(AQ[b][v], lo, isum, false);
                        isum = __builtin_amdgcn_sdot4(AQ[b][4 + v], hi, isum, false);
                    }
                    isum -= 8 * ASUM[b];
                    acc += sq_q_term(isum, AS[b], sq_f16_to_f32(Db[r][b]));
                } else {
                    const float* xb = s_x + blk * kPad;
                    float bacc = 0.0f;
                    if constexpr (WT == WT_Q8_0) {
#pragma unroll
                        for (int v = 0; v < 8; v++) {
                            const int dw = Wb[r][b][v];
                            float4 x4 = *(const float4*)(xb + 4 * v);
                            bacc += x4.x * sq_sbyte_f(dw, 0);
                            bacc += x4.y * sq_sbyte_f(dw, 1);
                            bacc += x4.z * sq_sbyte_f(dw, 2);
                            bacc += x4.w * sq_sbyte_f(dw, 3);
                        }
                        acc += bacc * sq_f16_to_f32(Db[r][b]);
                    } else if constexpr (WT == WT_Q4_0) {
#pragma unroll
                        for (int v = 0; v < 4; v++) {
                            const unsigned dw = (unsigned)Wb[r][b][v];
                            float4 xl = *(const float4*)(xb + 4 * v);
                            float4 xh = *(const float4*)(xb + 16 + 4 * v);
                            bacc += xl.x * (float)((int)(dw & 15u) - 8) + xh.x * (float)((int)((dw >> 4) & 15u) - 8);
                            bacc += xl.y * (float)((int)((dw >> 8) & 15u) - 8) + xh.y * (float)((int)((dw >> 12) & 15u) - 8);
                            bacc += xl.z * (float)((int)((dw >> 16) & 15u) - 8) + xh.z * (float)((int)((dw >> 20) & 15u) - 8);
                            bacc += xl.w * (float)((int)((dw >> 24) & 15u) - 8) + xh.w * (float)((int)((dw >> 28) & 15u) - 8);
                        }
                        acc += bacc * sq_f16_to_f32(Db[r][b]);
                    } else {  // BF16
#pragma unroll
                        for (int v = 0; v < 16; v++) {
                            const unsigned dw = (unsigned)Wb[r][b][v];
                            float2 x2 = *(const float2*)(xb + 2 * v);
                            bacc += x2.x * __builtin_bit_cast(float, dw << 16);
                            bacc += x2.y * __builtin_bit_cast(float, dw & 0xFFFF0000u);
                        }
                        acc += bacc;
                    }
                }
            }
            res[r] = sq_wave_sum(acc);
        }

        // ------------------------------------------------------- epilogue
        if constexpr (EPI == EPI_STORE || EPI == EPI_RESID || EPI == EPI_LOGITS) {
#pragma unroll
            for (int r = 0; r < R; r++) {
                const int slot = wave * R + r;
                const int row = t * TR + slot;
                if (row < a.n_rows) {
                    if (lane == r) {
                        if constexpr (EPI == EPI_RESID) a.out[row] += res[r];
                        else a.out[row] = res[r];
                    }
                    if constexpr (EPI == EPI_LOGITS) {
                        const float v = res[r];
                        if (v != v) {
                            nan_i = row > nan_i ? row : nan_i;
                        } else if (v > best_v || (v == best_v && row > best_i)) {
                            best_v = v;
                            best_i = row;
                        }
                    }
                }
            }
        } else if constexpr (EPI == EPI_QKV) {
            const int p = qkv_pos;
#pragma unroll
            for (int r = 0; r < R; r += 2) {
                const int row = t * TR + wave * R + r;
                if (row >= a.n_rows || lane != r) continue;
                float v0 = res[r], v1 = res[r + 1];
                if (row < a.q_rows + a.kv_rows) {
                    const bool is_q = row < a.q_rows;
                    const int li = is_q ? row : row - a.q_rows;
                    const int hd = 2 * a.half;
                    const int j = (li % hd) >> 1;
                    const float2 cs = a.rope[(size_t)p * a.half + j];
                    float o0, o1;
                    sq_rotate(v0, v1, cs.x, cs.y, o0, o1);
                    if (is_q) {
                        a.q_out[li] = o0;
                        a.q_out[li + 1] = o1;
                    } else {
                        a.kcache[(size_t)p * a.kv_rows + li] = o0;
                        a.kcache[(size_t)p * a.kv_rows + li + 1] = o1;
                    }
                } else {
                    const int li = row - a.q_rows - a.kv_rows;
                    a.vcache[(size_t)p * a.kv_rows + li] = v0;
                    a.vcache[(size_t)p * a.kv_rows + li + 1] = v1;
                }
            }
        } else if constexpr (EPI == EPI_GATEUP) {
#pragma unroll
            for (int r = 0; r < R; r++)
                if (lane == r) s_gu[wave * R + r] = res[r];
            __syncthreads();
            if (wave == 0) {
                // layers::ffn (src/models/llama/layers.rs:64-77):
                // gate = silu(gate); ffn_act = gate * up; then the down
                // projection quantizes ffn_act per 32-block.
                const int l = lane & 31;
                const float g = s_gu[l];
                const float u = s_gu[32 + l];
                const float sg = g * sq_sigmoid(g);
                const float f = sg * u;
                const int o = t * 32 + l;
                if (lane < 32) a.ffn_act[o] = f;
                if (a.act_q != nullptr) {
                    float amax = fmaxf(sq_half_max(fabsf(f)), 0.0f);
                    float scale = sq_q8_scale(amax);
                    float inv = sq_q8_inv(scale);
                    if (lane < 32) a.act_q[o] = sq_q8_quant(f, inv);
                    if (lane == 0) a.act_d[t] = sq_f32_to_f16(scale);
                }
            }
            __syncthreads();
        }
    };

    if constexpr (NBUF == 2) {
        // Grid-stride over tiles with the next tile's weights in flight.
        while (t < n_tiles) {
            if (t + (int)gridDim.x < n_tiles) load_tile(W1, D1, t + gridDim.x);
            compute_tile(W0, D0, t);
            t += gridDim.x;
            if (t >= n_tiles) break;
            if (t + (int)gridDim.x < n_tiles) load_tile(W0, D0, t + gridDim.x);
            compute_tile(W1, D1, t);
            t += gridDim.x;
        }
    } else {
        for (; t < n_tiles; t += gridDim.x) {
            compute_tile(W0, D0, t);
            if (t + (int)gridDim.x < n_tiles) load_tile(W0, D0, t + gridDim.x);
        }
    }

    if constexpr (EPI == EPI_LOGITS) {
        // (value, index) with the reference's rule: the larger value wins,
        // equal values go to the larger index (Iterator::max_by keeps the
        // last maximum, src/samplers/greedy.rs:8-13).  NaN rows are tracked
        // separately and resolved by the last workgroup.
        auto merge = [](float& bv, int& bi, int& bn, float v, int i, int n) {
            if (i >= 0 && (bi < 0 || v > bv || (v == bv && i > bi))) {
                bv = v;
                bi = i;
            }
            bn = n > bn ? n : bn;
        };
        auto block_merge = [&](float& bv, int& bi, int& bn) {
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) {
                const float ov = __shfl_xor(bv, o, 64);
                const int oi = __shfl_xor(bi, o, 64);
                const int on = __shfl_xor(bn, o, 64);
                merge(bv, bi, bn, ov, oi, on);
            }
            __syncthreads();
            if (lane == 0) {
                s_bv[wave] = bv;
                s_bi[wave] = bi;
                s_bn[wave] = bn;
            }
            __syncthreads();
            bv = s_bv[0];
            bi = s_bi[0];
            bn = s_bn[0];
            for (int w = 1; w < WAVES; w++) merge(bv, bi, bn, s_bv[w], s_bi[w], s_bn[w]);
        };
        block_merge(best_v, best_i, nan_i);
        if (tid == 0) {
            a.part_val[blockIdx.x] = best_v;
            a.part_idx[blockIdx.x] = best_i;
            a.part_nan[blockIdx.x] = nan_i;
        }
    }
}

template <int WT, bool A8, int NBL, int R, int WAVES, int PRO, int EPI, int NBUF = 1>
int run(hipStream_t s, const GemvArgs& a, int max_grid, int* grid_out) {
    using G = Gemv<WT, A8, NBL, R, WAVES, PRO, EPI, NBUF>;
    const int n_tiles = (EPI == EPI_GATEUP) ? (a.n_rows / 32) : (a.n_rows + G::TR - 1) / G::TR;
    int grid = n_tiles < max_grid ? n_tiles : max_grid;
    if (grid < 1) grid = 1;
    hipLaunchKernelGGL((gemv_kernel<WT, A8, NBL, R, WAVES, PRO, EPI, NBUF>), dim3(grid),
                       dim3(G::NT), 0, s, a);
    if (grid_out) *grid_out = grid;
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return set_error(SQ_ERR_HIP, std::string("gemv launch: ") + hipGetErrorString(e));
    return 0;
}

// One instantiation family per weight type and activation kind.
template <int WT, bool A8>
int dispatch(hipStream_t s, int pro, int epi, const GemvArgs& a, int* grid_out) {
    const int K = a.w.k;
    const int KB = K / 32;
    constexpr int PRO_A = A8 ? PRO_Q8 : PRO_F32;
    switch (epi) {
        case EPI_QKV:
            if (pro != PRO_NORM || KB > 64) break;
            return run<WT, A8, 1, 2, 4, PRO_NORM, EPI_QKV>(s, a, 1 << 30, grid_out);
        case EPI_GATEUP:
            if (pro != PRO_NORM || KB > 64) break;
            if constexpr (WT == WT_BF16)
                return run<WT, A8, 1, 4, 16, PRO_NORM, EPI_GATEUP>(s, a, 1 << 30, grid_out);
            else
                return run<WT, A8, 1, 8, 8, PRO_NORM, EPI_GATEUP>(s, a, 1 << 30, grid_out);
        case EPI_LOGITS:
            if (pro != PRO_NORM || KB > 64) break;
            return run<WT, A8, 1, 4, 4, PRO_NORM, EPI_LOGITS, 2>(s, a, kLogitsGrid, grid_out);
        case EPI_RESID:
            if (pro != PRO_A) break;
            if (KB <= 64) return run<WT, A8, 1, 2, 4, PRO_A, EPI_RESID>(s, a, 1 << 30, grid_out);
            if (KB <= 256) return run<WT, A8, 4, 1, 4, PRO_A, EPI_RESID>(s, a, 1 << 30, grid_out);
            break;
        case EPI_STORE:
            if (pro != PRO_A) break;
            if (KB <= 64) return run<WT, A8, 1, 2, 4, PRO_A, EPI_STORE>(s, a, 1 << 30, grid_out);
            if (KB <= 256) return run<WT, A8, 4, 1, 4, PRO_A, EPI_STORE>(s, a, 1 << 30, grid_out);
            break;
        default:
            break;
    }
    return set_error(SQ_ERR_SHAPE,
                     "gemv: unsupported (prologue, epilogue, k) combination, k=" + std::to_string(K));
}

}  // namespace

int launch_gemv(hipStream_t s, int pro, int epi, bool a8, const GemvArgs& a, int* grid_out) {
    if (a.w.k <= 0 || a.w.k % 32 != 0)
        return set_error(SQ_ERR_SHAPE, "gemv: k must be a positive multiple of 32");
    if (epi == EPI_GATEUP && a.n_rows % 32 != 0)
        return set_error(SQ_ERR_SHAPE, "gemv: gate/up width must be a multiple of 32");
    if (a.embd.qs != nullptr &&
        (a.token == nullptr || a.id_error == nullptr || a.hidden_out == nullptr || a.embd.k != a.w.k))
        return set_error(SQ_ERR_ARG, "gemv: embedding prologue needs a token, an error word, a hidden output and k = dim");
    switch (a.w.wtype) {
        case WT_Q8_0:
            return a8 ? dispatch<WT_Q8_0, true>(s, pro, epi, a, grid_out)
                      : dispatch<WT_Q8_0, false>(s, pro, epi, a, grid_out);
        case WT_Q4_0:
            return a8 ? dispatch<WT_Q4_0, true>(s, pro, epi, a, grid_out)
                      : dispatch<WT_Q4_0, false>(s, pro, epi, a, grid_out);
        case WT_BF16:
            if (a8) return set_error(SQ_ERR_INVALID_TYPE, "gemv: BF16 weights take f32 activations");
            return dispatch<WT_BF16, false>(s, pro, epi, a, grid_out);
        default:
            return set_error(SQ_ERR_INVALID_TYPE, "gemv: unsupported weight type");
    }
}

}  // namespace sq
