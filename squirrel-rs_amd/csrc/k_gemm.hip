// Multi-row matmul for the batched prefill: out[m, n] (+)= in[m, :] . W[n, :].
// The integer path (Q8_0 activations) runs on MFMA (gemm_mfma_kernel below)
// from one 64-row tile of activations up; the kernel described next serves
// shorter inputs and f32 activations.
//
// A tile of MT activation rows is staged in LDS once; each wavefront then
// streams weight rows (lane = 32-block, as in the decode matvec) and dots
// every row of the tile against them, so weights are read ceil(M/MT) times
// instead of M times (the reference re-streams them per row,
// src/kernels/matmul.rs:34).  Per-block arithmetic is the decode matvec's:
// exact i32 block sums, term = (f32(isum) * sa) * sw.
#include <atomic>
#include <cstring>

#include "launch.h"

namespace sq {
namespace {

constexpr int kPad = 36;
constexpr int WAVES = 4;
constexpr int RPW = 4;               // weight rows per wavefront
constexpr int TN = WAVES * RPW;      // weight rows per workgroup

template <int WT>
struct Dw;
template <> struct Dw<WT_Q8_0> { static constexpr int v = 8; };
template <> struct Dw<WT_Q4_0> { static constexpr int v = 4; };
template <> struct Dw<WT_BF16> { static constexpr int v = 16; };

template <int WT, bool A8, int NBL, int MT>
__global__ __launch_bounds__(WAVES * 64) void gemm_kernel(MatView w, const int8_t* __restrict__ aq,
                                                           const uint16_t* __restrict__ ad,
                                                           const float* __restrict__ x, int m_rows,
                                                           float* __restrict__ out, int ldo,
                                                           int accumulate) {
    constexpr int KMAX = NBL * 64 * 32;
    constexpr int DW = Dw<WT>::v;
    __shared__ __attribute__((aligned(16))) int8_t s_qs[A8 ? MT * KMAX : 16];
    __shared__ float s_sa[A8 ? MT * KMAX / 32 : 1];
    __shared__ int s_asum[(A8 && WT == WT_Q4_0) ? MT * KMAX / 32 : 1];
    __shared__ __attribute__((aligned(16))) float s_x[A8 ? 4 : MT * (KMAX / 32) * kPad];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int K = w.k, KB = K >> 5;
    const int m0 = blockIdx.y * MT;
    const int mt = min(MT, m_rows - m0);

    if constexpr (A8) {
        for (int e = tid; e < MT * KB * 8; e += WAVES * 64) {
            const int m = e / (KB * 8), r = e % (KB * 8);
            int v = 0;
            if (m < mt) v = ((const int*)(aq + (size_t)(m0 + m) * K))[r];
            ((int*)(s_qs + m * KMAX))[r] = v;
        }
        for (int e = tid; e < MT * KB; e += WAVES * 64) {
            const int m = e / KB, b = e % KB;
            s_sa[m * (KMAX / 32) + b] = (m < mt) ? sq_f16_to_f32(ad[(size_t)(m0 + m) * KB + b]) : 0.0f;
        }
        __syncthreads();
        if constexpr (WT == WT_Q4_0) {
            for (int e = tid; e < MT * KB; e += WAVES * 64) {
                const int m = e / KB, b = e % KB;
                const int* p = (const int*)(s_qs + m * KMAX + b * 32);
                int sacc = 0;
                for (int v = 0; v < 8; v++) sacc = __builtin_amdgcn_sdot4(p[v], 0x01010101, sacc, false);
                s_asum[m * (KMAX / 32) + b] = sacc;
            }
        }
    } else {
        for (int e = tid; e < MT * K; e += WAVES * 64) {
            const int m = e / K, i = e % K;
            s_x[m * (KMAX / 32) * kPad + (i >> 5) * kPad + (i & 31)] =
                (m < mt) ? x[(size_t)(m0 + m) * K + i] : 0.0f;
        }
    }
    __syncthreads();

    const uint8_t* wbase = (const uint8_t*)w.qs;
    const size_t row_bytes = (size_t)KB * DW * 4;
    for (int r = 0; r < RPW; r++) {
        const int n = blockIdx.x * TN + wave * RPW + r;
        if (n >= w.rows) break;
        int W[NBL][DW];
        float sw[NBL];
#pragma unroll
        for (int b = 0; b < NBL; b++) {
            const int blk = lane + 64 * b;
            if (blk < KB) {
                const sq_v4i* p = (const sq_v4i*)(wbase + (size_t)n * row_bytes + (size_t)blk * DW * 4);
#pragma unroll
                for (int v = 0; v < DW / 4; v++) {
                    sq_v4i t = p[v];
                    W[b][4 * v] = t.x; W[b][4 * v + 1] = t.y; W[b][4 * v + 2] = t.z; W[b][4 * v + 3] = t.w;
                }
                sw[b] = (WT == WT_BF16) ? 1.0f : sq_f16_to_f32(w.scale[(size_t)n * KB + blk]);
            } else {
#pragma unroll
                for (int v = 0; v < DW; v++) W[b][v] = 0;
                sw[b] = 0.0f;
            }
        }
        float acc[MT];
#pragma unroll
        for (int m = 0; m < MT; m++) acc[m] = 0.0f;
#pragma unroll
        for (int b = 0; b < NBL; b++) {
            const int blk = lane + 64 * b;
            if (blk >= KB) continue;
#pragma unroll
            for (int m = 0; m < MT; m++) {
                if constexpr (A8) {
                    const sq_v4i* ap = (const sq_v4i*)(s_qs + m * KMAX + blk * 32);
                    const sq_v4i a0 = ap[0], a1 = ap[1];
                    const int A[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
                    int isum = 0;
                    if constexpr (WT == WT_Q8_0) {
#pragma unroll
                        for (int v = 0; v < 8; v++) isum = __builtin_amdgcn_sdot4(A[v], W[b][v], isum, false);
                    } else {
#pragma unroll
                        for (int v = 0; v < 4; v++) {
                            isum = __builtin_amdgcn_sdot4(A[v], W[b][v] & 0x0F0F0F0F, isum, false);
                            isum = __builtin_amdgcn_sdot4(A[4 + v], (W[b][v] >> 4) & 0x0F0F0F0F, isum, false);
                        }
                        isum -= 8 * s_asum[m * (KMAX / 32) + blk];
                    }
                    acc[m] += sq_q_term(isum, s_sa[m * (KMAX / 32) + blk], sw[b]);
                } else {
                    const float* xb = s_x + m * (KMAX / 32) * kPad + blk * kPad;
                    float bacc = 0.0f;
                    if constexpr (WT == WT_Q8_0) {
#pragma unroll
                        for (int v = 0; v < 8; v++) {
                            float4 x4 = *(const float4*)(xb + 4 * v);
                            bacc += x4.x * sq_sbyte_f(W[b][v], 0);
                            bacc += x4.y * sq_sbyte_f(W[b][v], 1);
                            bacc += x4.z * sq_sbyte_f(W[b][v], 2);
                            bacc += x4.w * sq_sbyte_f(W[b][v], 3);
                        }
                        acc[m] += bacc * sw[b];
                    } else if constexpr (WT == WT_Q4_0) {
#pragma unroll
                        for (int v = 0; v < 4; v++) {
                            const unsigned dw = (unsigned)W[b][v];
                            float4 xl = *(const float4*)(xb + 4 * v);
                            float4 xh = *(const float4*)(xb + 16 + 4 * v);
                            bacc += xl.x * (float)((int)(dw & 15u) - 8) + xh.x * (float)((int)((dw >> 4) & 15u) - 8);
                            bacc += xl.y * (float)((int)((dw >> 8) & 15u) - 8) + xh.y * (float)((int)((dw >> 12) & 15u) - 8);
                            bacc += xl.z * (float)((int)((dw >> 16) & 15u) - 8) + xh.z * (float)((int)((dw >> 20) & 15u) - 8);
                            bacc += xl.w * (float)((int)((dw >> 24) & 15u) - 8) + xh.w * (float)((int)((dw >> 28) & 15u) - 8);
                        }
                        acc[m] += bacc * sw[b];
                    } else {
#pragma unroll
                        for (int v = 0; v < 16; v++) {
                            const unsigned dw = (unsigned)W[b][v];
                            float2 x2 = *(const float2*)(xb + 2 * v);
                            bacc += x2.x * __builtin_bit_cast(float, dw << 16);
                            bacc += x2.y * __builtin_bit_cast(float, dw & 0xFFFF0000u);
                        }
                        acc[m] += bacc;
                    }
                }
            }
        }
#pragma unroll
        for (int m = 0; m < MT; m++) {
            const float v = sq_wave_sum(acc[m]);
            if (lane == m && m < mt) {
                float* o = out + (size_t)(m0 + m) * ldo + n;
                if (accumulate) *o += v;
                else *o = v;
            }
        }
    }
}

// ---- integer path on the matrix cores ------------------------------------------
// out[m, n] (+)= sum over blocks b of f32(isum_b[m, n]) * (sa[m, b] * sw[n, b]),
// each term fused into the running sum as the reference's aarch64 kernels
// combine blocks (dot_prod.rs:189-252; the scalar twin, dot_prod.rs:376-403,
// rounds (f32(isum) * sa) * sw instead): isum_b is the exact i32 dot of one
// 32-element block, which is one v_mfma_i32_16x16x32_i8 (K = 32) for a
// 16 x 16 tile of outputs.
//
// The kernel is bound by VALU issue: each output element and block costs
// the conversion of isum and the fused add.  The scale product sa * sw of
// two f16 values has at most 22 significant bits, so it is exact in f32
// however it is formed; it comes from one v_mfma_f32_16x16x16_f16 per tile
// and block, already in the result layout: lanes 0-15 hold the row's four
// block scales in k-slots 0-3 (the other lanes zeros), and the column
// operand of block b holds sw_b in k-slot b and zeros elsewhere.
//
// A workgroup computes a 64 x 64 tile of (activation rows) x (weight rows)
// with four wavefronts of 32 x 32 (2 x 2 MFMA tiles).  K advances in chunks
// of four blocks: the chunk's activation and weight bytes (64 rows x 128 B
// each, Q4_0 nibbles expanded to q - 8 as int8) and block scales are staged
// in LDS, rows MQ_LD bytes apart so that the 16 rows a wavefront's fragment
// loads touch spread over the banks.  MFMA operand layout (checked on the
// device): lane l supplies row l % 16, bytes 8 (l / 16) .. +7 of the block;
// result element r of lane l is row 4 (l / 16) + r, column l % 16.
constexpr int MQ_T = 64;           // tile rows (activations) and columns (weights)
constexpr int MQ_KB = 4;           // blocks per K chunk
constexpr int MQ_KC = MQ_KB * 32;  // bytes per row per K chunk
constexpr int MQ_LD = MQ_KC + 8;   // LDS row stride in bytes

typedef int mq_v4i __attribute__((ext_vector_type(4)));
typedef float sq_v4f __attribute__((ext_vector_type(4)));
typedef _Float16 mq_v4h __attribute__((ext_vector_type(4)));

template <int WT>
__global__ __launch_bounds__(256) void gemm_mfma_kernel(MatView w, const int8_t* __restrict__ aq,
                                                        const uint16_t* __restrict__ ad, int m_rows,
                                                        float* __restrict__ out, int ldo, int accumulate,
                                                        int kbs, size_t split_stride) {
    __shared__ __attribute__((aligned(16))) int8_t sA[MQ_T * MQ_LD];
    __shared__ __attribute__((aligned(16))) int8_t sW[MQ_T * MQ_LD];
    // f16 block scales: sSa[row][b]; row MQ_T is zeros (the k-slots of
    // lanes 16-63).  sSw[b][col] holds sw_b in slot b, zeros elsewhere
    // (16 lanes read 16 consecutive columns of one block).
    __shared__ __attribute__((aligned(16))) uint16_t sSa[MQ_T + 1][MQ_KB];
    __shared__ __attribute__((aligned(16))) uint16_t sSw[MQ_KB][MQ_T][MQ_KB];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int K = w.k, KB = K >> 5;
    const int m0 = blockIdx.y * MQ_T, n0 = blockIdx.x * MQ_T;
    // blocks [kb_begin, kb_end) of K: all of them, or split z of a K split
    // (its tile goes to a partial buffer, split_stride floats per split)
    const int kb_begin = blockIdx.z * kbs, kb_end = min(KB, kb_begin + kbs);
    out += blockIdx.z * split_stride;
    const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
    const int fr = lane & 15, fk = 8 * (lane >> 4);  // fragment row, byte offset in the block

    float acc[2][2][4];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 4; r++) acc[i][j][r] = 0.0f;

    // This thread's share of a chunk: activation (and Q8_0 weight) pieces
    // tid and tid + 256 of 64 rows x 8 sixteen-byte pieces, or one packed
    // Q4_0 block (row tid / 4, block tid % 4); the scales of row tid % 64,
    // block tid / 64.  The next chunk's share is loaded into registers while
    // the current one is multiplied.
    sq_v4i ra[2], rw[2];
    uint16_t rsa, rsw;
    auto fetch = [&](int kb0) {
#pragma unroll
        for (int q = 0; q < 2; q++) {
            const int p = tid + 256 * q, r = p >> 3, s = p & 7;
            const int k = kb0 * 32 + 16 * s;
            ra[q] = sq_v4i{0, 0, 0, 0};
            if (m0 + r < m_rows && k < kb_end * 32) ra[q] = *(const sq_v4i*)(aq + (size_t)(m0 + r) * K + k);
            if constexpr (WT == WT_Q8_0) {
                rw[q] = sq_v4i{0, 0, 0, 0};
                if (n0 + r < w.rows && k < kb_end * 32) rw[q] = *(const sq_v4i*)((const int8_t*)w.qs + (size_t)(n0 + r) * K + k);
            }
        }
        if constexpr (WT == WT_Q4_0) {
            const int r = tid >> 2, kb = kb0 + (tid & 3);
            rw[0] = sq_v4i{(int)0x88888888, (int)0x88888888, (int)0x88888888, (int)0x88888888};  // q = 8: zero weights
            if (n0 + r < w.rows && kb < kb_end) rw[0] = *(const sq_v4i*)((const uint8_t*)w.qs + (size_t)(n0 + r) * (K / 2) + kb * 16);
        }
        const int r = tid & 63, kb = kb0 + (tid >> 6);
        rsa = (m0 + r < m_rows && kb < kb_end) ? ad[(size_t)(m0 + r) * KB + kb] : (uint16_t)0;
        rsw = (n0 + r < w.rows && kb < kb_end) ? w.scale[(size_t)(n0 + r) * KB + kb] : (uint16_t)0;
    };
    auto stage = [&]() {
#pragma unroll
        for (int q = 0; q < 2; q++) {
            const int p = tid + 256 * q, r = p >> 3, s = p & 7;
            // LDS rows are MQ_LD bytes apart (8-byte aligned): two 8-byte stores
            int2* da = (int2*)(sA + r * MQ_LD + 16 * s);
            da[0] = make_int2(ra[q].x, ra[q].y);
            da[1] = make_int2(ra[q].z, ra[q].w);
            if constexpr (WT == WT_Q8_0) {
                int2* dw = (int2*)(sW + r * MQ_LD + 16 * s);
                dw[0] = make_int2(rw[q].x, rw[q].y);
                dw[1] = make_int2(rw[q].z, rw[q].w);
            }
        }
        if constexpr (WT == WT_Q4_0) {
            const int r = tid >> 2, b = tid & 3;
            // byte j holds element j (low nibble) and element j + 16 (high
            // nibble); per byte, nibble - 8 as a signed byte: (q | 0x80) - 8
            // stays within the byte, and xor 0x80 restores the sign
            const unsigned wd[4] = {(unsigned)rw[0].x, (unsigned)rw[0].y, (unsigned)rw[0].z, (unsigned)rw[0].w};
            int lo[4], hi[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                lo[i] = (int)((((wd[i] & 0x0F0F0F0Fu) | 0x80808080u) - 0x08080808u) ^ 0x80808080u);
                hi[i] = (int)(((((wd[i] >> 4) & 0x0F0F0F0Fu) | 0x80808080u) - 0x08080808u) ^ 0x80808080u);
            }
            int2* dw = (int2*)(sW + r * MQ_LD + 32 * b);
            dw[0] = make_int2(lo[0], lo[1]);
            dw[1] = make_int2(lo[2], lo[3]);
            dw[2] = make_int2(hi[0], hi[1]);
            dw[3] = make_int2(hi[2], hi[3]);
        }
        const int r = tid & 63, b = tid >> 6;
        sSa[r][b] = rsa;
        const unsigned sw = (unsigned)rsw << (16 * (b & 1));
        *(uint2*)&sSw[b][r][0] = (b < 2) ? make_uint2(sw, 0u) : make_uint2(0u, sw);
    };

    if (tid < MQ_KB) sSa[MQ_T][tid] = 0;
    fetch(kb_begin);
    for (int kb0 = kb_begin; kb0 < kb_end; kb0 += MQ_KB) {
        stage();
        __syncthreads();
        if (kb0 + MQ_KB < kb_end) fetch(kb0 + MQ_KB);
        // the row operands of the scale products: this row's four block
        // scales on lanes 0-15, zeros on the others
        mq_v4h sa[2];
#pragma unroll
        for (int i = 0; i < 2; i++) sa[i] = *(const mq_v4h*)&sSa[lane < 16 ? wm + 16 * i + fr : MQ_T][0];
        // Software pipeline over the chunk's blocks: the products of block
        // b + 1 for tile t are issued as soon as tile t of block b has been
        // folded in, so the matrix cores run while the VALU converts.  Blocks
        // past kb_end were staged as zeros (payload and scales), and
        // fma(0, 0, acc) leaves acc unchanged.
        long af[2], bf[2];
        mq_v4h sw[2];
        auto operands = [&](int b) {
#pragma unroll
            for (int i = 0; i < 2; i++) af[i] = *(const long*)(sA + (wm + 16 * i + fr) * MQ_LD + 32 * b + fk);
#pragma unroll
            for (int j = 0; j < 2; j++) {
                bf[j] = *(const long*)(sW + (wn + 16 * j + fr) * MQ_LD + 32 * b + fk);
                sw[j] = *(const mq_v4h*)&sSw[b][wn + 16 * j + fr][0];
            }
        };
        const mq_v4i zero = {0, 0, 0, 0};
        const sq_v4f fzero = {0.0f, 0.0f, 0.0f, 0.0f};
        mq_v4i d[4];
        sq_v4f sc[4];
        operands(0);
#pragma unroll
        for (int t = 0; t < 4; t++) {
            d[t] = __builtin_amdgcn_mfma_i32_16x16x32_i8(af[t >> 1], bf[t & 1], zero, 0, 0, 0);
            sc[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(sa[t >> 1], sw[t & 1], fzero, 0, 0, 0);
        }
#pragma unroll
        for (int b = 0; b < MQ_KB; b++) {
            if (b + 1 < MQ_KB) operands(b + 1);
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const int i = t >> 1, j = t & 1;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    // the combine of the reference's aarch64 kernels (dot_prod.rs:189-252):
                    // acc = fma(f32(isum), sa * sw, acc)
                    acc[i][j][r] = fmaf((float)d[t][r], sc[t][r], acc[i][j][r]);
                }
                if (b + 1 < MQ_KB) {
                    d[t] = __builtin_amdgcn_mfma_i32_16x16x32_i8(af[i], bf[j], zero, 0, 0, 0);
                    sc[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(sa[i], sw[j], fzero, 0, 0, 0);
                }
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = m0 + wm + 16 * i + (fk >> 1) + r, n = n0 + wn + 16 * j + fr;
                if (m < m_rows && n < w.rows) {
                    float* o = out + (size_t)m * ldo + n;
                    *o = accumulate ? *o + acc[i][j][r] : acc[i][j][r];
                }
            }
}

// ---- 128 x 128 tiles on the 32 x 32 matrix instructions ----------------------
// The same contraction on v_mfma_i32_32x32x32_i8 (the full int8 rate of
// gfx950; the 16 x 16 x 32 form runs at half of it), which gives the exact
// i32 isum of a 32 x 32 tile for one block: lane l supplies 16 bytes of row
// l % 32, half l / 32 of the block, and the other operand alike.  The scale
// products come from one v_mfma_f32_32x32x8_f16 per tile and block (lanes
// 0-31 hold the row's block scales in k-slots 0-1, the others zeros; the
// column operand of block b holds sw_b in slot b).  Result element r of lane
// l is row 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32.  A workgroup
// computes BM x BN (128 x 128 or 128 x 64) as four wavefronts of
// BM / 2 x BN / 2, that is (BM / 64) x (BN / 64) tiles of 32 x 32 each.  K
// advances two blocks per chunk through two LDS buffers with one barrier per
// chunk; every thread keeps two chunks' global loads in registers, issued two
// chunks ahead of their use.
constexpr int M8_KB = 2;           // blocks per chunk
constexpr int M8_KC = M8_KB * 32;  // bytes per row per chunk
constexpr int M8_LD = M8_KC + 16;  // LDS row stride: 16-byte reads of 8 consecutive rows cover all banks

typedef int m8_v16i __attribute__((ext_vector_type(16)));
typedef float m8_v16f __attribute__((ext_vector_type(16)));

template <int BM, int BN>
struct M8Loads {
    sq_v4i a[BM / 64];  // activation pieces (row p / 4, 16-byte unit p % 4 for p = tid + 256 q)
    sq_v4i w[BN / 64];  // Q8_0: weight pieces as a[]; Q4_0: w[0] is one packed block
    uint16_t sa, sw;
    bool va, vw;  // the scales are in range (applied when staged)
};

// Wavefronts per SIMD: two (174 registers on 128 x 128 tiles, 192 on
// 128 x 64; at three the 128 x 64 tiles spill).
template <int BM, int BN>
constexpr int m8_occupancy() { return 2; }

template <int WT, int BM, int BN>
__global__ __launch_bounds__(256, (m8_occupancy<BM, BN>())) void gemm_mfma32_kernel(
    MatView w, const int8_t* __restrict__ aq, const uint16_t* __restrict__ ad, int m_rows,
    float* __restrict__ out, int ldo, int accumulate, int kbs, size_t split_stride) {
    static_assert(BM == 128 && (BN == 64 || BN == 128), "tiles of 128 x 128 or 128 x 64");
    constexpr int SM = BM / 64, SN = BN / 64;  // 32 x 32 tiles per wavefront in M and N
    constexpr int NT = SM * SN;
    __shared__ __attribute__((aligned(16))) int8_t sA[2][BM * M8_LD];
    __shared__ __attribute__((aligned(16))) int8_t sW[2][BN * M8_LD];
    // sSa[buf][row][slot]: the chunk's two block scales in slots 0-1; slots
    // 2-3 and row BM stay zero.  sSw[buf][b][col]: sw_b in slot b.
    __shared__ __attribute__((aligned(16))) uint16_t sSa[2][BM + 1][4];
    __shared__ __attribute__((aligned(16))) uint16_t sSw[2][M8_KB][BN][4];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int K = w.k, KB = K >> 5;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int kb_begin = blockIdx.z * kbs, kb_end = min(KB, kb_begin + kbs);
    out += blockIdx.z * split_stride;
    const int wm = (wave >> 1) * (BM / 2), wn = (wave & 1) * (BN / 2);
    const int fr = lane & 31, fh = lane >> 5;
    // the scale each thread fetches and stages: row tid % T of block
    // (tid / T) % 2 (with 64 columns threads 128-255 repeat threads 0-127)
    const int ra_s = tid & (BM - 1), ba_s = (tid / BM) & 1;
    const int rw_s = tid & (BN - 1), bw_s = (tid / BN) & 1;

    // Clear what staging never writes (slots 2-3, row BM), so no clear can
    // land on a scale another thread has already staged; the first chunk's
    // barrier publishes both.
    for (int i = tid; i < 2 * (BM + 1); i += 256) {
        uint32_t* z = (uint32_t*)&sSa[i / (BM + 1)][i % (BM + 1)][0];
        z[1] = 0;
        if (i % (BM + 1) == BM) z[0] = 0;
    }

    // Every thread issues the same loads for every chunk, without branches:
    // rows and blocks past the end read the last valid row and block, and
    // their scales are set to zero, so their terms are fma(isum, 0, acc) =
    // acc and rows past the end are never stored.  With a fixed count of
    // loads per chunk the wait before staging one register set can leave the
    // other set's loads in flight.
    auto fetch = [&](M8Loads<BM, BN>& L, int kb0) {
#pragma unroll
        for (int q = 0; q < SM; q++) {
            const int p = tid + 256 * q, r = p >> 2, u = p & 3;
            const int kb = min(kb0 + (u >> 1), KB - 1);
            const size_t ra = (size_t)min(m0 + r, m_rows - 1);
            L.a[q] = *(const sq_v4i*)(aq + ra * K + kb * 32 + 16 * (u & 1));
        }
        if constexpr (WT == WT_Q8_0) {
#pragma unroll
            for (int q = 0; q < SN; q++) {
                const int p = tid + 256 * q, r = p >> 2, u = p & 3;
                const int kb = min(kb0 + (u >> 1), KB - 1);
                const size_t rw = (size_t)min(n0 + r, w.rows - 1);
                L.w[q] = *(const sq_v4i*)((const int8_t*)w.qs + rw * K + kb * 32 + 16 * (u & 1));
            }
        } else {
            const int r = (tid >> 1) & (BN - 1), kb = min(kb0 + (tid & 1), KB - 1);
            L.w[0] = *(const sq_v4i*)((const uint8_t*)w.qs + (size_t)min(n0 + r, w.rows - 1) * (K / 2) + kb * 16);
        }
        const int kba = kb0 + ba_s, kbw = kb0 + bw_s;
        L.sa = ad[(size_t)min(m0 + ra_s, m_rows - 1) * KB + min(kba, KB - 1)];
        L.sw = w.scale[(size_t)min(n0 + rw_s, w.rows - 1) * KB + min(kbw, KB - 1)];
        L.va = m0 + ra_s < m_rows && kba < kb_end;
        L.vw = n0 + rw_s < w.rows && kbw < kb_end;
    };
    auto stage = [&](const M8Loads<BM, BN>& L, int buf) {
#pragma unroll
        for (int q = 0; q < SM; q++) {
            const int p = tid + 256 * q, r = p >> 2, u = p & 3;
            *(sq_v4i*)(sA[buf] + r * M8_LD + 16 * u) = L.a[q];
        }
        if constexpr (WT == WT_Q8_0) {
#pragma unroll
            for (int q = 0; q < SN; q++) {
                const int p = tid + 256 * q, r = p >> 2, u = p & 3;
                *(sq_v4i*)(sW[buf] + r * M8_LD + 16 * u) = L.w[q];
            }
        } else {
            // byte j holds element j (low nibble) and j + 16 (high nibble);
            // per byte, nibble - 8 as a signed byte (see gemm_mfma_kernel)
            const int r = (tid >> 1) & (BN - 1), b = tid & 1;
            const unsigned wd[4] = {(unsigned)L.w[0].x, (unsigned)L.w[0].y, (unsigned)L.w[0].z, (unsigned)L.w[0].w};
            int lo[4], hi[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                lo[i] = (int)((((wd[i] & 0x0F0F0F0Fu) | 0x80808080u) - 0x08080808u) ^ 0x80808080u);
                hi[i] = (int)(((((wd[i] >> 4) & 0x0F0F0F0Fu) | 0x80808080u) - 0x08080808u) ^ 0x80808080u);
            }
            *(sq_v4i*)(sW[buf] + r * M8_LD + 32 * b) = sq_v4i{lo[0], lo[1], lo[2], lo[3]};
            *(sq_v4i*)(sW[buf] + r * M8_LD + 32 * b + 16) = sq_v4i{hi[0], hi[1], hi[2], hi[3]};
        }
        // (with 64 columns threads 128-255 store what threads 0-127 store:
        // the same values, fetched from the same places)
        sSa[buf][ra_s][ba_s] = L.va ? L.sa : (uint16_t)0;
        *(uint2*)&sSw[buf][bw_s][rw_s][0] = make_uint2(L.vw ? (unsigned)L.sw << (16 * bw_s) : 0u, 0u);
    };

    m8_v16f acc[NT];
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[t][r] = 0.0f;

    auto compute = [&](int buf) {
        const int8_t* A = sA[buf];
        const int8_t* W = sW[buf];
        mq_v4h sa[SM];
#pragma unroll
        for (int i = 0; i < SM; i++) sa[i] = *(const mq_v4h*)&sSa[buf][fh == 0 ? wm + 32 * i + fr : BM][0];
        // one block's operands at a time: the row and column fragments and
        // the column scale operands of the SM x SN tiles
        sq_v4i af[SM], bf[SN];
        mq_v4h sw[SN];
        auto operands = [&](int b) {
#pragma unroll
            for (int i = 0; i < SM; i++) af[i] = *(const sq_v4i*)(A + (wm + 32 * i + fr) * M8_LD + 32 * b + 16 * fh);
#pragma unroll
            for (int j = 0; j < SN; j++) {
                bf[j] = *(const sq_v4i*)(W + (wn + 32 * j + fr) * M8_LD + 32 * b + 16 * fh);
                sw[j] = *(const mq_v4h*)&sSw[buf][b][wn + 32 * j + fr][0];
            }
        };
        // Products for (block, tile) pairs k = NT b + t, issued one pair ahead
        // of the pair being folded in.
        const m8_v16i izero = {};
        const m8_v16f fzero = {};
        m8_v16i d[2];
        m8_v16f sc[2];
        operands(0);
        d[0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[0], bf[0], izero, 0, 0, 0);
        sc[0] = __builtin_amdgcn_mfma_f32_32x32x8f16(sa[0], sw[0], fzero, 0, 0, 0);
#pragma unroll
        for (int k = 0; k < NT * M8_KB; k++) {
            if (k + 1 < NT * M8_KB) {
                const int t1 = (k + 1) % NT, i = t1 / SN, j = t1 % SN;
                if (t1 == 0) operands((k + 1) / NT);
                d[(k + 1) & 1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], izero, 0, 0, 0);
                sc[(k + 1) & 1] = __builtin_amdgcn_mfma_f32_32x32x8f16(sa[i], sw[j], fzero, 0, 0, 0);
            }
            // On 128 x 128 tiles the next pair's matrix instructions are kept
            // issued ahead of this pair's VALU work: left to itself the
            // scheduler moves them after it and waits for each result (224 vs
            // 229 us for the gate/up projection of a 2048-token prompt; on
            // 128 x 64 tiles the same barriers cost 11%).
            if constexpr (BN == 128) __builtin_amdgcn_sched_barrier(0);
            const int t = k % NT;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                // the combine of the reference's aarch64 kernels (dot_prod.rs:189-252):
                // acc = fma(f32(isum), sa * sw, acc)
                acc[t][r] = fmaf((float)d[k & 1][r], sc[k & 1][r], acc[t][r]);
            }
            if constexpr (BN == 128) __builtin_amdgcn_sched_barrier(0);
        }
    };

    // Chunk c's loads are in set c % 2 and its tiles in buffer c % 2.  Once a
    // set is staged it takes chunk c + 2; buffer c % 2 was last read in chunk
    // c - 2, before the previous chunk's barrier.
    // The loop body is straight-line code over two chunks (an odd count gets
    // one chunk past kb_end, whose zero scales fold nothing), so the wait
    // before staging a set leaves the other set's loads in flight.
    M8Loads<BM, BN> L0, L1;
    const int n_chunks = (kb_end - kb_begin + M8_KB - 1) / M8_KB;
    fetch(L0, kb_begin);
    fetch(L1, kb_begin + M8_KB);
    for (int c = 0; c < n_chunks; c += 2) {
        stage(L0, 0);
        __syncthreads();
        fetch(L0, kb_begin + (c + 2) * M8_KB);
        compute(0);
        stage(L1, 1);
        __syncthreads();
        fetch(L1, kb_begin + (c + 3) * M8_KB);
        compute(1);
    }
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int m = m0 + wm + 32 * (t / SN) + 8 * (r >> 2) + 4 * fh + (r & 3);
            const int n = n0 + wn + 32 * (t % SN) + fr;
            if (m < m_rows && n < w.rows) {
                float* o = out + (size_t)m * ldo + n;
                *o = accumulate ? *o + acc[t][r] : acc[t][r];
            }
        }
}

// Matmul epilogues: RW_STORE writes (or adds) the tile; RW_GATEUP and RW_QKV
// are described with the kernels that take them.
enum : int { RW_STORE = 0, RW_GATEUP = 1, RW_QKV = 2 };
struct RowsEpi {
    int8_t* act_q;       // RW_GATEUP: FFN activation blocks [m][ffn], scales [m][ffn / 32]
    uint16_t* act_d;
    const float2* rope;  // RW_QKV: (cos, sin) per position and pair
    float* q_out;        // [m][q_dim]
    float* kcache;       // [position][kv_dim]
    float* vcache;
    int q_dim, kv_dim, head_dim, pos0;
};
// ---- the same contraction with direct global -> LDS loads ---------------------
// gemm_dma_kernel computes what gemm_mfma32_kernel computes, with the same
// matrix instructions folding the same per-block terms in the same order
// (so both give the same bits), but its tiles never pass through registers:
// global_load_lds_dwordx4 writes each 64-lane load (1 KB) straight into one
// of ST LDS stages, and the loads run ST - 1 stages ahead of the one being
// multiplied.  A stage holds, for SKB blocks of K (32 SKB bytes per row), the
// BM activation rows and BN weight rows (Q8_0 payload) and the blocks' fp16
// scales, two per 32-bit word: word d of row r at sa[d][r] (sw[d][r]).  Row
// r's 16-byte units are stored with unit u at position u ^ dma_swz(r): the
// 16-byte operand reads of 8 (16) consecutive rows at one unit then fall in
// distinct banks of a 32 (64) bank LDS.  The loads are issued from inline
// assembly (dma_to_lds), and each wavefront waits for its own loads of a
// stage before a bare s_barrier (no fence: a fence would wait for every load
// in flight).  Needs a block count per K range that is a multiple of SKB.
//
// Epilogues: RW_GATEUP (128 x 128 tiles) takes the stacked [gate; up]
// matrix with column tile x holding gate rows 64 x + 32 h .. + 31 and the
// same up rows in its tiles 2 h and 2 h + 1 (h the wavefront's column half),
// so every output element of a wavefront's gate tile has its up value at the
// same register of the next tile; the 32 lanes of a half-wavefront then hold
// one prompt row's FFN block, and SiLU(gate) * up and its Q8_0 block are
// formed as silu_mul8_kernel forms them.  RW_QKV applies RoPE to the q and
// k columns (the pair partner of column n is column n ^ 1, lane l ^ 1) and
// appends the K and V rows to the cache, as rope_kv_kernel does.  The same
// operations on the same values as the separate kernels, so the same bits.
typedef __attribute__((address_space(3))) int8_t lds_i8;

template <int BM, int BN, int SKB>
struct DmaStage {
    int8_t a[BM * 32 * SKB];
    int8_t w[BN * 32 * SKB];
    uint32_t sa[SKB / 2][BM];  // sa_{2d} | sa_{2d+1} << 16
    uint32_t sw[SKB / 2][BN];
};

template <int SKB>
__device__ __forceinline__ int dma_swz(int r) {
    // (bits 0-3 of r only: the operand reads' row bases are multiples of 32)
    if constexpr (SKB == 2) return ((r >> 1) ^ (r >> 2)) & 3;  // four units per row
    else return (r ^ ((r >> 3) & 1)) & 7;                      // eight units per row
}

// A direct global -> LDS load (global_load_lds_dwordx4 for 16 bytes per lane,
// global_load_lds_dword for 4): lane l reads `base + off` (base the same on
// every lane, in SGPRs) and its bytes land at lds + SIZE * l (lds the same on
// every lane: it goes to M0).  Issued from inline assembly, so the compiler's
// wait-count pass does not see it: that pass cannot tell which stage such a
// load writes once a loop merges its state, and would make every read of any
// stage wait for every load in flight.  The caller waits for the loads itself
// (s_waitcnt vmcnt) before a barrier.  M0 is named as clobbered; the
// compiler sets M0 itself before each instruction of its own that reads it.
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

// s_waitcnt immediate: at most n vector-memory operations outstanding (the
// LDS and export counters not waited on).
constexpr int dma_vmcnt(int n) { return (n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8); }

// SQUIRREL_GEMM_DMA=0 keeps the full-rate tilings on the register-staged
// kernel (a test and measurement aid: both give the same bits).
bool gemm_dma_enabled() {
    const char* e = getenv("SQUIRREL_GEMM_DMA");
    return !(e && !strcmp(e, "0"));
}

constexpr int DMA_KB = 2;      // blocks per stage
constexpr int DMA_STAGES = 3;  // LDS stages
// Wavefronts per SIMD: three on both tilings.  The 128 x 128 tiles get there
// (at most 168 registers) by issuing each tile's matrix instructions right
// before their combine instead of one tile ahead: the third wavefront hides
// the matrix latency (193 against 210 us for the gate/up projection of a
// 2048-token prompt, where two wavefronts with the one-ahead issue fit).
// The 128 x 64 tiles keep the one-ahead issue (132 registers; four
// wavefronts would spill).
template <int BM, int BN>
constexpr int dma_occupancy() { return 3; }
// the loads' 32-bit byte offsets (row * k) stay below 2^31
bool dma_offsets_fit(const MatView& w, int m) {
    return (int64_t)max(w.rows, m) * w.k < ((int64_t)1 << 31);
}

template <int BM, int BN, int ST, int SKB, int EPI>
__global__ __launch_bounds__(256, (dma_occupancy<BM, BN>())) void gemm_dma_kernel(
    MatView w, const int8_t* __restrict__ aq, const uint16_t* __restrict__ ad, int m_rows,
    float* __restrict__ out, int ldo, int accumulate, int kbs, size_t split_stride, RowsEpi ep) {
    static_assert(BM == 128 && (BN == 64 || BN == 128), "tiles of 128 x 128 or 128 x 64");
    static_assert(EPI != RW_GATEUP || BN == 128, "the gate/up epilogue takes 128 x 128 tiles");
    static_assert(ST >= 2 && ST <= 4, "two to four stages");
    static_assert(SKB == 2 || SKB == 4, "two or four blocks per stage");
    constexpr int SM = BM / 64, SN = BN / 64;
    constexpr int NT = SM * SN;
    constexpr int SKC = 32 * SKB, UPR = 2 * SKB;  // bytes and 16-byte units per row and stage
    constexpr int LA = BM * UPR / 256, LW = BN * UPR / 256;  // 1 KB payload loads per wavefront and stage
    constexpr int LS = SKB / 2;  // scale loads per wavefront and stage
    constexpr int LPW = LA + LW + LS;
    typedef DmaStage<BM, BN, SKB> Stage;
    __shared__ __attribute__((aligned(16))) Stage stg[ST];
    Stage &st0 = stg[0], &st1 = stg[1 % ST], &st2 = stg[2 % ST], &st3 = stg[3 % ST];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int K = w.k, KB = K >> 5;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int kb_begin = blockIdx.z * kbs, kb_end = min(KB, kb_begin + kbs);
    out += blockIdx.z * split_stride;
    const int wm = (wave >> 1) * (BM / 2), wn = (wave & 1) * (BN / 2);
    const int fr = lane & 31, fh = lane >> 5;

    // Per-lane byte offsets of this wavefront's loads from the stage's first
    // block.  Payload load q covers 1 KB of the stage: rows 1024 q / SKC ..,
    // lane j writing physical unit j % UPR of row 1024 q / SKC + j / UPR,
    // which holds logical unit (j % UPR) ^ swz(row).
    const int ffn = w.rows / 2;  // RW_GATEUP: FFN width
    auto wrow_of = [&](int r) {  // weight row of tile row r
        if constexpr (EPI == RW_GATEUP)
            return ((r >> 5) & 1) * ffn + min(64 * (int)blockIdx.x + 32 * (r >> 6) + (r & 31), ffn - 1);
        else
            return min(n0 + r, w.rows - 1);
    };
    uint32_t offa[LA], offw[LW];
#pragma unroll
    for (int i = 0; i < LA; i++) {
        const int q = wave + 4 * i, r = q * (1024 / SKC) + lane / UPR, u = (lane % UPR) ^ dma_swz<SKB>(r);
        offa[i] = (uint32_t)(min(m0 + r, m_rows - 1) * K + 16 * u);
    }
#pragma unroll
    for (int i = 0; i < LW; i++) {
        const int q = wave + 4 * i, r = q * (1024 / SKC) + lane / UPR, u = (lane % UPR) ^ dma_swz<SKB>(r);
        offw[i] = (uint32_t)(wrow_of(r) * K + 16 * u);
    }
    // The scale words: wavefronts 0 and 1 take the activation rows 64 v ..
    // 64 v + 63, wavefronts 2 and 3 the weight rows (with 64 columns, 32 rows
    // each, on lanes 0-31); load d of a stage is word d of every row.
    const bool sc_act = wave < 2;
    const int sc_row = sc_act ? 64 * wave + lane : (BN == 128 ? 64 * (wave - 2) + lane : 32 * (wave - 2) + lane);
    const bool sc_on = sc_act || BN == 128 || lane < 32;
    const uint32_t offs = 2 * (uint32_t)((sc_act ? min(m0 + sc_row, m_rows - 1) : wrow_of(sc_row)) * KB);
    const uint16_t* sc_src = sc_act ? ad : w.scale;
    const int sc_dst = sc_act ? 64 * wave : (BN == 128 ? 64 * (wave - 2) : 32 * (wave - 2));

    auto lds = [](Stage& S) { return (lds_i8*)(int8_t*)&S; };
    auto issue = [&](Stage& S, int kb0) {
        lds_i8* const base = lds(S);
        const int8_t* ga = aq + (size_t)kb0 * 32;
        const int8_t* gw = (const int8_t*)w.qs + (size_t)kb0 * 32;
#pragma unroll
        for (int i = 0; i < LA; i++) dma_to_lds<16>(ga, offa[i], base + 1024 * (wave + 4 * i));
#pragma unroll
        for (int i = 0; i < LW; i++) dma_to_lds<16>(gw, offw[i], base + BM * SKC + 1024 * (wave + 4 * i));
        if (sc_on) {
            const uint16_t* gs = sc_src + kb0;
            lds_i8* const sb = base + BM * SKC + BN * SKC + (sc_act ? 0 : 4 * LS * BM);
#pragma unroll
            for (int d = 0; d < LS; d++)
                dma_to_lds<4>(gs + 2 * d, offs, sb + 4 * (d * (sc_act ? BM : BN) + sc_dst));
        }
    };

    m8_v16f acc[NT];
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[t][r] = 0.0f;

    // Operand addresses within a stage (bytes): row tile i / column tile j
    // at block b is logical unit 2 b + fh (wm, wn and 32 i, 32 j are
    // multiples of 32, so swz depends on fr alone).
    int ra[SM], rw[SN], ua[SKB];
#pragma unroll
    for (int i = 0; i < SM; i++) ra[i] = (wm + 32 * i + fr) * SKC;
#pragma unroll
    for (int j = 0; j < SN; j++) rw[j] = (wn + 32 * j + fr) * SKC;
#pragma unroll
    for (int b = 0; b < SKB; b++) ua[b] = 16 * ((2 * b + fh) ^ dma_swz<SKB>(fr));
    const uint32_t lo_mask = fh ? 0u : 0xFFFFFFFFu;  // k-slots 4-7 (lanes 32-63) are zero

    auto compute = [&](const Stage& S) {
        // scale operands: lanes 0-31 hold k-slots 0-3 of row (column) fr, the
        // others slots 4-7 (zero).  Block 2 d pairs (sa_{2d}, 0) with (sw_{2d},
        // sw_{2d+1}); block 2 d + 1 pairs (0, sa_{2d+1}) with the same.
        uint32_t sar[LS][SM], swr[LS][SN];
#pragma unroll
        for (int d = 0; d < LS; d++) {
#pragma unroll
            for (int i = 0; i < SM; i++) sar[d][i] = S.sa[d][wm + 32 * i + fr] & lo_mask;
#pragma unroll
            for (int j = 0; j < SN; j++) swr[d][j] = S.sw[d][wn + 32 * j + fr] & lo_mask;
        }
        sq_v4i af[SM], bf[SN];
        auto operands = [&](int b) {
#pragma unroll
            for (int i = 0; i < SM; i++) af[i] = *(const sq_v4i*)(S.a + ra[i] + ua[b]);
#pragma unroll
            for (int j = 0; j < SN; j++) bf[j] = *(const sq_v4i*)(S.w + rw[j] + ua[b]);
        };
        auto sa_op = [&](int b, int i) {
            const uint32_t v = (b & 1) ? (sar[b >> 1][i] & 0xFFFF0000u) : (sar[b >> 1][i] & 0xFFFFu);
            return __builtin_bit_cast(mq_v4h, make_uint2(v, 0u));
        };
        auto sw_op = [&](int b, int j) { return __builtin_bit_cast(mq_v4h, make_uint2(swr[b >> 1][j], 0u)); };
        const m8_v16i izero = {};
        const m8_v16f fzero = {};
        if constexpr (BN == 128) {
            // (block, tile) pairs k = NT b + t in order, each pair's matrix
            // instructions right before its combine
#pragma unroll
            for (int k = 0; k < NT * SKB; k++) {
                const int t = k % NT, i = t / SN, j = t % SN, b = k / NT;
                if (t == 0) operands(b);
                const m8_v16i d = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], izero, 0, 0, 0);
                const m8_v16f sc = __builtin_amdgcn_mfma_f32_32x32x8f16(sa_op(b, i), sw_op(b, j), fzero, 0, 0, 0);
                // the combine of the reference's aarch64 kernels (dot_prod.rs:189-252):
                // acc = fma(f32(isum), sa * sw, acc)
#pragma unroll
                for (int r = 0; r < 16; r++) acc[t][r] = fmaf((float)d[r], sc[r], acc[t][r]);
            }
        } else {
            // the same pairs, each one's matrix instructions issued one pair
            // ahead of its combine
            m8_v16i d[2];
            m8_v16f sc[2];
            operands(0);
            d[0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[0], bf[0], izero, 0, 0, 0);
            sc[0] = __builtin_amdgcn_mfma_f32_32x32x8f16(sa_op(0, 0), sw_op(0, 0), fzero, 0, 0, 0);
#pragma unroll
            for (int k = 0; k < NT * SKB; k++) {
                if (k + 1 < NT * SKB) {
                    const int t1 = (k + 1) % NT, i = t1 / SN, j = t1 % SN, b1 = (k + 1) / NT;
                    if (t1 == 0) operands(b1);
                    d[(k + 1) & 1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], izero, 0, 0, 0);
                    sc[(k + 1) & 1] = __builtin_amdgcn_mfma_f32_32x32x8f16(sa_op(b1, i), sw_op(b1, j), fzero, 0, 0, 0);
                }
                const int t = k % NT;
#pragma unroll
                for (int r = 0; r < 16; r++) acc[t][r] = fmaf((float)d[k & 1][r], sc[k & 1][r], acc[t][r]);
            }
        }
    };

    // Wait until this wavefront's loads of the stage about to be multiplied
    // have landed: `ahead` later stages' loads may stay in flight.
    auto wait_stage = [&](int ahead) {
        if (ahead >= 2) __builtin_amdgcn_s_waitcnt(dma_vmcnt(2 * LPW));
        else if (ahead == 1) __builtin_amdgcn_s_waitcnt(dma_vmcnt(LPW));
        else __builtin_amdgcn_s_waitcnt(dma_vmcnt(0));
    };
    // (every LDS read of a stage is consumed by a matrix instruction before
    // the wavefront reaches the next barrier, so no read is still in flight
    // when another wavefront's loads overwrite the stage; the bare barrier
    // does not wait for LDS writes, so it serves the main loop only, which
    // writes LDS through the loads alone)
    auto barrier = [] {
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    };
    // One stage: wait for its loads, then refill the stage the previous one
    // used and multiply this one.
    const int n = (kb_end - kb_begin) / SKB;
    auto chunk = [&](int cc, Stage& cur, Stage& refill) {
        if (cc < n) {
            wait_stage(min(ST - 2, n - 1 - cc));
            barrier();
            if (cc + ST - 1 < n) issue(refill, kb_begin + SKB * (cc + ST - 1));
            compute(cur);
        }
    };
    // the first ST - 1 stages' loads
    if (0 < n) issue(st0, kb_begin);
    if constexpr (ST >= 3)
        if (1 < n) issue(st1, kb_begin + SKB);
    if constexpr (ST >= 4)
        if (2 < n) issue(st2, kb_begin + 2 * SKB);
    for (int c = 0; c < n; c += ST) {
        if constexpr (ST == 2) {
            chunk(c, st0, st1);
            chunk(c + 1, st1, st0);
        } else if constexpr (ST == 3) {
            chunk(c, st0, st2);
            chunk(c + 1, st1, st0);
            chunk(c + 2, st2, st1);
        } else {
            chunk(c, st0, st3);
            chunk(c + 1, st1, st0);
            chunk(c + 2, st2, st1);
            chunk(c + 3, st3, st2);
        }
    }
    // element r of tile t is row 8 (r / 4) + 4 fh + r % 4 of row tile t / SN,
    // column fr of column tile t % SN
    if constexpr (EPI == RW_GATEUP) {
        // SiLU(gate) * up of the workgroup's 128 rows x 64 FFN columns goes
        // to LDS (the stages are free once every wavefront is past its last
        // chunk); then thread t takes row t / 2, block t % 2: the block's
        // maximum, Q8_0 scale and quants as silu_mul8_kernel forms them,
        // stored as 32 bytes.  Row r's 16-byte chunk c (of 16) sits at
        // position c of its half rotated by 2 r + c / 8, so a row's writes and
        // the readers' 16-byte reads of 8 consecutive threads fall in distinct
        // banks (of 32).
        // The two barriers here are __syncthreads: each wavefront's LDS
        // writes must have landed before another reads them (the main loop's
        // bare barrier waits for nothing, and no load is in flight by now).
        static_assert(BM * 64 * sizeof(float) <= sizeof(stg), "the SiLU tile fits the stages");
        float* const tileb = (float*)&stg[0];
        auto at = [](int row, int col) {
            const int c = col >> 2;
            return row * 64 + 4 * ((c & 8) | (((c & 7) + 2 * row + (c >> 3)) & 7)) + (col & 3);
        };
        __syncthreads();
        const int fc = 32 * (wave & 1) + fr;  // the workgroup's FFN column
#pragma unroll
        for (int i = 0; i < SM; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const float g = acc[SN * i][r], u = acc[SN * i + 1][r];
                const int row = wm + 32 * i + 8 * (r >> 2) + 4 * fh + (r & 3);
                tileb[at(row, fc)] = (g * sq_sigmoid(g)) * u;  // silu(gate) * up (silu_mul8_kernel)
            }
        __syncthreads();
        const int row = tid >> 1, blk = tid & 1, m = m0 + row, f0 = 64 * blockIdx.x + 32 * blk;
        float v[32];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const sq_v4f x = *(const sq_v4f*)(tileb + at(row, 32 * blk + 4 * k));
            v[4 * k] = x.x;
            v[4 * k + 1] = x.y;
            v[4 * k + 2] = x.z;
            v[4 * k + 3] = x.w;
        }
        float mx = fabsf(v[0]);
#pragma unroll
        for (int k = 1; k < 32; k++) mx = fmaxf(mx, fabsf(v[k]));
        const float scale = sq_q8_scale(fmaxf(mx, 0.0f)), inv = sq_q8_inv(scale);
        if (m < m_rows && f0 < ffn) {
            unsigned q[8];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                q[k] = 0;
#pragma unroll
                for (int c = 0; c < 4; c++) q[k] |= (unsigned)(uint8_t)sq_q8_quant(v[4 * k + c], inv) << (8 * c);
            }
            sq_v4i* const dst = (sq_v4i*)(ep.act_q + (size_t)m * ffn + f0);
            dst[0] = sq_v4i{(int)q[0], (int)q[1], (int)q[2], (int)q[3]};
            dst[1] = sq_v4i{(int)q[4], (int)q[5], (int)q[6], (int)q[7]};
            ep.act_d[(size_t)m * (ffn / 32) + f0 / 32] = sq_f32_to_f16(scale);
        }
        return;
    }
    if constexpr (EPI == RW_QKV) {
        const int QD = ep.q_dim, KVD = ep.kv_dim;
#pragma unroll
        for (int t = 0; t < NT; t++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const float v = acc[t][r];
                const float pv = __shfl_xor(v, 1, 64);  // column n ^ 1 of the same prompt row
                const int m = m0 + wm + 32 * (t / SN) + 8 * (r >> 2) + 4 * fh + (r & 3);
                const int n = n0 + wn + 32 * (t % SN) + fr;
                if (m >= m_rows || n >= w.rows) continue;
                const int p = ep.pos0 + m;
                if (n < QD + KVD) {
                    const bool is_q = n < QD;
                    const int li = is_q ? n : n - QD;
                    const float2 cs = ep.rope[(size_t)p * (ep.head_dim >> 1) + ((li % ep.head_dim) >> 1)];
                    float o0, o1;
                    if (n & 1) sq_rotate(pv, v, cs.x, cs.y, o0, o1);
                    else sq_rotate(v, pv, cs.x, cs.y, o0, o1);
                    const float o = (n & 1) ? o1 : o0;
                    if (is_q) ep.q_out[(size_t)m * QD + li] = o;
                    else ep.kcache[(size_t)p * KVD + li] = o;
                } else {
                    ep.vcache[(size_t)p * KVD + (n - QD - KVD)] = v;
                }
            }
        return;
    }
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int m = m0 + wm + 32 * (t / SN) + 8 * (r >> 2) + 4 * fh + (r & 3);
            const int n2 = n0 + wn + 32 * (t % SN) + fr;
            if (m < m_rows && n2 < w.rows) {
                float* o = out + (size_t)m * ldo + n2;
                *o = accumulate ? *o + acc[t][r] : acc[t][r];
            }
        }
}

// out[r, c] (+)= the sum of the K-split partial tiles, in split order.
__global__ __launch_bounds__(256) void split_sum_kernel(const float* __restrict__ ws, int splits, size_t stride,
                                                        int m, int n, float* __restrict__ out, int ldo,
                                                        int accumulate) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)m * n) return;
    float v = 0.0f;
    for (int z = 0; z < splits; z++) v += ws[z * stride + i];
    float* o = out + (i / n) * (size_t)ldo + i % n;
    *o = accumulate ? *o + v : v;
}

// The same sums four elements per thread (16-byte loads and stores) where
// n, ldo and stride are multiples of 4 and the buffers 16-byte aligned.
__global__ __launch_bounds__(256) void split_sum4_kernel(const float* __restrict__ ws, int splits, size_t stride,
                                                         int m, int n, float* __restrict__ out, int ldo,
                                                         int accumulate) {
    const size_t i = 4 * ((size_t)blockIdx.x * 256 + threadIdx.x);
    if (i >= (size_t)m * n) return;
    float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int z = 0; z < splits; z++) {
        const float4 p = *(const float4*)(ws + z * stride + i);
        v.x += p.x;
        v.y += p.y;
        v.z += p.z;
        v.w += p.w;
    }
    float4* o = (float4*)(out + (i / n) * (size_t)ldo + i % n);
    if (accumulate) {
        const float4 a = *o;
        v = make_float4(a.x + v.x, a.y + v.y, a.z + v.z, a.w + v.w);
    }
    *o = v;
}

// The stacked q|k|v projection's K-split partials ([m][ncols] each, stride
// apart) summed in split order as split_sum_kernel sums them, then RoPE on the
// q and k columns and the KV-cache append as rope_kv_kernel applies them: one
// workgroup per prompt row, the same operations on the same values.
__global__ __launch_bounds__(256) void split_sum_rope_kernel(const float* __restrict__ ws, int splits, size_t stride,
                                                             int ncols, RowsEpi ep) {
    const int m = blockIdx.x, p = ep.pos0 + m;
    const int QD = ep.q_dim, KVD = ep.kv_dim, half = ep.head_dim >> 1;
    const float* row = ws + (size_t)m * ncols;
    auto sum = [&](int e) {
        float v = 0.0f;
        for (int z = 0; z < splits; z++) v += row[z * stride + e];
        return v;
    };
    for (int pi = threadIdx.x; pi < (QD + KVD) >> 1; pi += 256) {
        const int e = 2 * pi;
        const bool is_q = e < QD;
        const int li = is_q ? e : e - QD;
        const float2 cs = ep.rope[(size_t)p * half + ((li % ep.head_dim) >> 1)];
        float o0, o1;
        sq_rotate(sum(e), sum(e + 1), cs.x, cs.y, o0, o1);
        if (is_q) {
            ep.q_out[(size_t)m * QD + li] = o0;
            ep.q_out[(size_t)m * QD + li + 1] = o1;
        } else {
            ep.kcache[(size_t)p * KVD + li] = o0;
            ep.kcache[(size_t)p * KVD + li + 1] = o1;
        }
    }
    for (int i = threadIdx.x; i < KVD; i += 256) ep.vcache[(size_t)p * KVD + i] = sum(QD + KVD + i);
}

// out (+)= the split partials in split order, on the vector kernel where the
// shapes and buffers allow it.
int launch_split_sum(hipStream_t s, const float* ws, int splits, size_t stride, int m, int n, float* out, int ldo,
                     bool acc) {
    const size_t total = (size_t)m * n;
    if (n % 4 == 0 && ldo % 4 == 0 && stride % 4 == 0 && (((uintptr_t)ws | (uintptr_t)out) & 15) == 0)
        hipLaunchKernelGGL(split_sum4_kernel, dim3((unsigned)((total / 4 + 255) / 256)), dim3(256), 0, s, ws, splits,
                           stride, m, n, out, ldo, acc ? 1 : 0);
    else
        hipLaunchKernelGGL(split_sum_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, ws, splits,
                           stride, m, n, out, ldo, acc ? 1 : 0);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(SQ_ERR_HIP, std::string("split sum launch: ") + hipGetErrorString(e));
    return 0;
}

// ---- few activation rows: the weights streamed once --------------------------
// A prompt of a few dozen rows (the short prompts of a generation) makes the
// matmul a weight stream with little arithmetic per byte.  The 64 x 64
// kernel leaves most of its tile empty there, and on narrow matrices splits
// K over workgroups and sums the partials in a second launch.  Here a
// workgroup takes 32 activation rows and NT tiles of 32 weight rows: one
// v_mfma_i32_32x32x32_i8 per block and tile (lane l supplies 16 bytes of row
// l % 32, half l / 32 of the block; activations as operand A, weights as
// operand B) and one v_mfma_f32_32x32x8f16 for the scale products sa * sw
// (lanes 0-31 hold the row's and the column's scale in k-slot 0, the others
// zeros).  Its RW_NW wavefronts take consecutive ranges of the workgroup's
// K, each with two batches of RW_NB blocks of loads in flight (branch-free:
// blocks past a range read a clamped address and get zero scales), and sum
// their partial tiles through LDS in wavefront order.  A long K on a narrow
// matrix is also split over workgroups (blockIdx.z), whose partial tiles
// split_sum_kernel adds in split order.  The per-block combine is that of
// the other kernels: fma(f32(isum), sa * sw, acc) (dot_prod.rs:189-252).
//
// Epilogues (EPI): RW_STORE writes (or adds) the tile.  RW_GATEUP: the FFN
// gate/up projection with SiLU(gate) * up and its Q8_0 blocks (two tiles:
// gate rows 32 j.. and the up rows ffn + 32 j..); a 32-lane half of a
// wavefront then holds one prompt row's 32 values of FFN block j and forms
// the block as silu_mul8_kernel does.  RW_QKV: the stacked q|k|v projection
// with RoPE on q and k and the KV-cache append, as rope_kv_kernel does (the
// pair partner of column n is column n ^ 1, lane l ^ 1).  The same
// operations on the same values, so the same bits as the separate kernels.
constexpr int RW_NW = 8;  // wavefronts per workgroup
constexpr int RW_NB = 4;  // blocks per load batch with one column tile (two with two)

template <int NT, int NB>
struct RwBatch {
    typedef unsigned short scales __attribute__((ext_vector_type(NB)));
    sq_v4i w[NT][NB];  // Q8_0: 16 bytes of the block; Q4_0: the packed block
    sq_v4i a[NB];
    scales sw[NT], sa;  // the batch's f16 block scales of this lane's weight rows and activation row
};

template <int WT, int NT, int NB, int EPI>
__global__ __launch_bounds__(RW_NW * 64) void gemm_rows_kernel(MatView w, const int8_t* __restrict__ aq,
                                                               const uint16_t* __restrict__ ad, int m_rows,
                                                               float* __restrict__ out, int ldo, int accumulate,
                                                               int per, int kbs, size_t split_stride, RowsEpi ep) {
    constexpr bool GU = EPI == RW_GATEUP;
    static_assert(!GU || NT == 2, "the gate/up epilogue pairs two tiles");
    static_assert(EPI != RW_QKV || NT == 1, "the q|k|v epilogue takes one tile");
    __shared__ float red[RW_NW][NT * 16][64];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int K = w.k, KB = K >> 5;
    const int n0 = blockIdx.x * 32 * NT, m0 = blockIdx.y * 32;
    const int fr = lane & 31, fh = lane >> 5;
    // the workgroup's blocks [kb_begin, kb_end) (split blockIdx.z), and this
    // wavefront's [kbw, kend): per (a multiple of 2 NB) per wavefront
    const int kb_begin = blockIdx.z * kbs, kb_end = min(KB, kb_begin + kbs);
    out += blockIdx.z * split_stride;
    const int kbw = kb_begin + wave * per, kend = min(kb_end, kbw + per);
    const int nb = per / NB;
    typedef RwBatch<NT, NB> Batch;
    size_t wrow[NT];
    bool wvalid[NT];
    const int ffn = w.rows / 2, j0 = blockIdx.x * 32;  // GU: the FFN block's first column
#pragma unroll
    for (int t = 0; t < NT; t++) {
        if constexpr (GU) {
            wvalid[t] = j0 + fr < ffn;
            wrow[t] = (size_t)(t * ffn + min(j0 + fr, ffn - 1));
        } else {
            wrow[t] = (size_t)min(n0 + 32 * t + fr, w.rows - 1);
            wvalid[t] = n0 + 32 * t + fr < w.rows;
        }
    }
    const size_t arow = (size_t)min(m0 + fr, m_rows - 1);

    auto load = [&](Batch& B, int kb) {
        const int kc = min(kb, KB - NB);  // KB is a multiple of NB
#pragma unroll
        for (int j = 0; j < NB; j++) {
#pragma unroll
            for (int t = 0; t < NT; t++) {
                if constexpr (WT == WT_Q8_0)
                    B.w[t][j] = *(const sq_v4i*)((const int8_t*)w.qs + wrow[t] * K + (kc + j) * 32 + 16 * fh);
                else
                    B.w[t][j] = *(const sq_v4i*)((const uint8_t*)w.qs + wrow[t] * (K / 2) + (kc + j) * 16);
            }
            B.a[j] = *(const sq_v4i*)(aq + arow * K + (kc + j) * 32 + 16 * fh);
        }
#pragma unroll
        for (int t = 0; t < NT; t++) B.sw[t] = *(const typename Batch::scales*)(w.scale + wrow[t] * KB + kc);
        B.sa = *(const typename Batch::scales*)(ad + arow * KB + kc);
    };
    m8_v16f acc[NT];
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[t][r] = 0.0f;
    const m8_v16i izero = {};
    const m8_v16f fzero = {};
    auto compute = [&](const Batch& B, int kb) {
#pragma unroll
        for (int j = 0; j < NB; j++) {
            // blocks past the range fold nothing: both scales zero (an
            // activation scale may be inf, and inf * 0 would not be).  Lane
            // l % 32 carries activation row l % 32 in sa and weight row
            // l % 32 in sw, so a weight row past the matrix zeroes only sw.
            // (selects, not branches: a branch here lets the compiler move
            // every block's combine after all the matrix instructions)
            const bool inb = kb + j < kend && fh == 0;
            const _Float16 h0 = 0;
            const mq_v4h sa = {__builtin_bit_cast(_Float16, inb ? (uint16_t)B.sa[j] : (uint16_t)0), h0, h0, h0};
#pragma unroll
            for (int t = 0; t < NT; t++) {
                sq_v4i wf = B.w[t][j];
                if constexpr (WT == WT_Q4_0) {
                    // byte i holds element i (low nibble) and i + 16 (high
                    // nibble): half fh of the block is one nibble of every
                    // byte, as q - 8 in a signed byte ((q | 0x80) - 8 stays
                    // within the byte, and xor 0x80 restores the sign)
                    const int sh = 4 * fh;
                    wf.x = (int)(((((unsigned)wf.x >> sh) & 0x0F0F0F0Fu) | 0x80808080u) - 0x08080808u) ^ (int)0x80808080u;
                    wf.y = (int)(((((unsigned)wf.y >> sh) & 0x0F0F0F0Fu) | 0x80808080u) - 0x08080808u) ^ (int)0x80808080u;
                    wf.z = (int)(((((unsigned)wf.z >> sh) & 0x0F0F0F0Fu) | 0x80808080u) - 0x08080808u) ^ (int)0x80808080u;
                    wf.w = (int)(((((unsigned)wf.w >> sh) & 0x0F0F0F0Fu) | 0x80808080u) - 0x08080808u) ^ (int)0x80808080u;
                }
                const uint16_t swv = inb && wvalid[t] ? (uint16_t)B.sw[t][j] : (uint16_t)0;
                const mq_v4h sw = {__builtin_bit_cast(_Float16, swv), h0, h0, h0};
                const m8_v16i d = __builtin_amdgcn_mfma_i32_32x32x32_i8(B.a[j], wf, izero, 0, 0, 0);
                const m8_v16f sc = __builtin_amdgcn_mfma_f32_32x32x8f16(sa, sw, fzero, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 16; r++) acc[t][r] = fmaf((float)d[r], sc[r], acc[t][r]);
                // one tile's products live at a time: left to itself the
                // scheduler issues every block's matrix instructions first and
                // spills their results
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };
    Batch B0, B1;
    load(B0, kbw);
    load(B1, kbw + NB);
    for (int b = 0; b + 2 < nb; b += 2) {
        compute(B0, kbw + b * NB);
        load(B0, kbw + (b + 2) * NB);
        compute(B1, kbw + (b + 1) * NB);
        load(B1, kbw + (b + 3) * NB);
    }
    compute(B0, kbw + (nb - 2) * NB);
    compute(B1, kbw + (nb - 1) * NB);

    // partial tiles summed in wavefront order; element r of lane l of tile t
    // is row 8 (r / 4) + 4 (l / 32) + r % 4, column 32 t + l % 32
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
        for (int r = 0; r < 16; r++) red[wave][16 * t + r][lane] = acc[t][r];
    __syncthreads();
    if constexpr (GU) {
        // e = 64 r + l: lanes l < 32 and l >= 32 of a wavefront are two
        // prompt rows' FFN block j (column l % 32)
        for (int e = tid; e < 16 * 64; e += RW_NW * 64) {
            const int r = e >> 6, l = e & 63;
            float g = 0.0f, u = 0.0f;
#pragma unroll
            for (int q = 0; q < RW_NW; q++) {
                g += red[q][r][l];
                u += red[q][16 + r][l];
            }
            const float v = (g * sq_sigmoid(g)) * u;  // silu(gate) * up (silu_mul8_kernel)
            float mx = fabsf(v);
#pragma unroll
            for (int o = 16; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
            const float scale = sq_q8_scale(fmaxf(mx, 0.0f)), inv = sq_q8_inv(scale);
            const int mm = m0 + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3), jj = l & 31;
            if (mm < m_rows && j0 + jj < ffn) {
                ep.act_q[(size_t)mm * ffn + j0 + jj] = sq_q8_quant(v, inv);
                if (jj == 0) ep.act_d[(size_t)mm * (ffn / 32) + blockIdx.x] = sq_f32_to_f16(scale);
            }
        }
        return;
    }
    if constexpr (EPI == RW_QKV) {
        for (int e = tid; e < 16 * 64; e += RW_NW * 64) {
            const int r = e >> 6, l = e & 63;
            float v = 0.0f;
#pragma unroll
            for (int q = 0; q < RW_NW; q++) v += red[q][r][l];
            const float pv = __shfl_xor(v, 1, 64);  // column n ^ 1 of the same prompt row
            const int mm = m0 + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3), n = n0 + (l & 31);
            if (mm >= m_rows || n >= w.rows) continue;
            const int QD = ep.q_dim, KVD = ep.kv_dim, p = ep.pos0 + mm;
            if (n < QD + KVD) {
                const bool is_q = n < QD;
                const int li = is_q ? n : n - QD;
                const float2 cs = ep.rope[(size_t)p * (ep.head_dim >> 1) + ((li % ep.head_dim) >> 1)];
                float o0, o1;
                if (n & 1) sq_rotate(pv, v, cs.x, cs.y, o0, o1);
                else sq_rotate(v, pv, cs.x, cs.y, o0, o1);
                const float o = (n & 1) ? o1 : o0;
                if (is_q) ep.q_out[(size_t)mm * QD + li] = o;
                else ep.kcache[(size_t)p * KVD + li] = o;
            } else {
                ep.vcache[(size_t)p * KVD + (n - QD - KVD)] = v;
            }
        }
        return;
    }
    for (int e = tid; e < NT * 16 * 64; e += RW_NW * 64) {
        const int tr = e >> 6, l = e & 63, t = tr >> 4, r = tr & 15;
        float v = 0.0f;
#pragma unroll
        for (int q = 0; q < RW_NW; q++) v += red[q][tr][l];
        const int mm = m0 + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3), nn = n0 + 32 * t + (l & 31);
        if (mm < m_rows && nn < w.rows) {
            float* o = out + (size_t)mm * ldo + nn;
            *o = accumulate ? *o + v : v;
        }
    }
}

// Compute units of the current device (the grid-size rules below are in
// workgroups per CU).
int device_cus() {
    static int cus[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cus[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}

// Matmul launches since the last reset (measurement aid): all, K-split,
// full-rate 128 x 128 tiles, the largest split count, full-rate 128 x 64
// tiles.
std::atomic<uint64_t> g_launches{0}, g_split_launches{0}, g_tile128_launches{0}, g_max_splits{0},
    g_tile128x64_launches{0}, g_rows_launches{0};
// bn: 0 for the 64 x 64 kernel, 32 for the few-rows kernel, else the
// full-rate kernel's tile columns (64 or 128)
void count_launch(int splits, int bn) {
    g_launches++;
    if (bn == 32) g_rows_launches++;
    if (splits > 1) g_split_launches++;
    if (bn == 128) g_tile128_launches++;
    if (bn == 64) g_tile128x64_launches++;
    uint64_t prev = g_max_splits.load();
    while ((uint64_t)splits > prev && !g_max_splits.compare_exchange_weak(prev, (uint64_t)splits)) {
    }
}

// A grid of fewer tiles than the device has CUs (short inputs, narrow
// matrices) splits K over about two workgroups per CU when the workspace
// holds the partial tiles; the partials are then summed in a fixed order, so
// results do not depend on scheduling.
template <int WT>
int run_mfma(hipStream_t s, const MatView& w, const int8_t* aq, const uint16_t* ad, int m, float* out, int ldo,
             bool acc, float* ws, size_t ws_floats) {
    const int gx = (w.rows + MQ_T - 1) / MQ_T, gy = (m + MQ_T - 1) / MQ_T;
    const int KB = w.k / 32, chunks = (KB + MQ_KB - 1) / MQ_KB;
    const int cus = device_cus();
    int splits = 1;
    if (ws != nullptr && gx * gy < cus) {
        splits = min(chunks, (2 * cus + gx * gy - 1) / (gx * gy));
        while (splits > 1 && (size_t)splits * m * w.rows > ws_floats) splits--;
    }
    const int kbs = ((chunks + splits - 1) / splits) * MQ_KB;  // blocks per split
    splits = (KB + kbs - 1) / kbs;
    count_launch(splits, 0);
    hipError_t e;
    if (splits == 1) {
        hipLaunchKernelGGL(gemm_mfma_kernel<WT>, dim3(gx, gy), dim3(256), 0, s, w, aq, ad, m, out, ldo, acc ? 1 : 0,
                           KB, (size_t)0);
    } else {
        const size_t stride = (size_t)m * w.rows;
        hipLaunchKernelGGL(gemm_mfma_kernel<WT>, dim3(gx, gy, splits), dim3(256), 0, s, w, aq, ad, m, ws, w.rows, 0,
                           kbs, stride);
        e = hipGetLastError();
        if (e != hipSuccess) return set_error(SQ_ERR_HIP, std::string("gemm launch: ") + hipGetErrorString(e));
        if (const int st = launch_split_sum(s, ws, splits, stride, m, w.rows, out, ldo, acc)) return st;
    }
    e = hipGetLastError();
    if (e != hipSuccess) return set_error(SQ_ERR_HIP, std::string("gemm launch: ") + hipGetErrorString(e));
    return 0;
}

// The full-rate kernel.  Its tiles pay where the output alone gives at
// least two workgroups per CU (512 on MI355X): 128 x 128 tiles for the
// gate/up projection of a 2048-token prompt (2048 tiles), 128 x 64 tiles
// where 128 x 128 ones are too few (its QKV, o and down projections: 768,
// 512 and 512 tiles; 7.8 against 8.0 ms for all the prompt's matmuls with
// those on the 64 x 64 kernel, whose 64 x 64 tiles on the full-rate
// instruction measured 9.5 ms).  A smaller grid returns 1 (nothing launched)
// and takes gemm_mfma_kernel with its K split.  When pinned to a tiling, a
// grid of fewer than two workgroups per CU splits K while the workspace
// holds the partial tiles.
template <int WT, int BM, int BN>
int run_mfma32(hipStream_t s, const MatView& w, const int8_t* aq, const uint16_t* ad, int m, float* out, int ldo,
               bool acc, float* ws, size_t ws_floats, bool force, int target = 0) {
    const int gx = (w.rows + BN - 1) / BN, gy = (m + BM - 1) / BM;
    const int KB = w.k / 32, chunks = (KB + M8_KB - 1) / M8_KB;
    const int full = target > 0 ? target : 2 * device_cus();
    if (!force && gx * gy < full) return 1;
    int splits = 1;
    if (ws != nullptr && gx * gy < full) {
        splits = min(chunks, (full + gx * gy - 1) / (gx * gy));
        while (splits > 1 && (size_t)splits * m * w.rows > ws_floats) splits--;
    }
    const int kbs = ((chunks + splits - 1) / splits) * M8_KB;
    splits = (KB + kbs - 1) / kbs;
    count_launch(splits, BN);
    // Q8_0 weights with an even block count take the direct-to-LDS kernel
    // (the same results); Q4_0 nibbles are expanded while staging.
    const bool dma = WT == WT_Q8_0 && kbs % DMA_KB == 0 && KB % DMA_KB == 0 && dma_offsets_fit(w, m) &&
                     gemm_dma_enabled();
    constexpr int ST = DMA_STAGES;
    hipError_t e;
    if (splits == 1) {
        if (dma)
            hipLaunchKernelGGL((gemm_dma_kernel<BM, BN, ST, DMA_KB, RW_STORE>), dim3(gx, gy), dim3(256), 0, s, w, aq, ad, m,
                               out, ldo, acc ? 1 : 0, KB, (size_t)0, RowsEpi{});
        else
            hipLaunchKernelGGL((gemm_mfma32_kernel<WT, BM, BN>), dim3(gx, gy), dim3(256), 0, s, w, aq, ad, m, out, ldo,
                               acc ? 1 : 0, KB, (size_t)0);
    } else {
        const size_t stride = (size_t)m * w.rows;
        if (dma)
            hipLaunchKernelGGL((gemm_dma_kernel<BM, BN, ST, DMA_KB, RW_STORE>), dim3(gx, gy, splits), dim3(256), 0, s, w, aq,
                               ad, m, ws, w.rows, 0, kbs, stride, RowsEpi{});
        else
            hipLaunchKernelGGL((gemm_mfma32_kernel<WT, BM, BN>), dim3(gx, gy, splits), dim3(256), 0, s, w, aq, ad, m,
                               ws, w.rows, 0, kbs, stride);
        e = hipGetLastError();
        if (e != hipSuccess) return set_error(SQ_ERR_HIP, std::string("gemm launch: ") + hipGetErrorString(e));
        if (const int st = launch_split_sum(s, ws, splits, stride, m, w.rows, out, ldo, acc)) return st;
    }
    e = hipGetLastError();
    if (e != hipSuccess) return set_error(SQ_ERR_HIP, std::string("gemm launch: ") + hipGetErrorString(e));
    return 0;
}

// The few-rows kernel: grid (column tiles of 32 NT, row tiles of 32, K
// splits), K in blocks of 32 with KB a multiple of RW_NB.  Two column tiles
// per workgroup where that still gives every CU a workgroup (the FFN gate/up
// projection: twice the weights in flight per CU, one round of the grid); a
// K split where the grid has fewer workgroups than CUs and each split keeps
// two full batches per wavefront (the FFN down projection, K = 8192: four
// splits).
template <int WT, int NT, int EPI = RW_STORE>
int launch_rows(hipStream_t s, const MatView& w, const int8_t* aq, const uint16_t* ad, int m, float* out, int ldo,
                bool acc, int gx, int gy, int splits, int kbs, float* ws, const RowsEpi& ep = RowsEpi{}) {
    constexpr int NB = NT == 1 ? RW_NB : RW_NB / 2;
    const int per = ((kbs + RW_NW - 1) / RW_NW + 2 * NB - 1) / (2 * NB) * (2 * NB);
    if (splits == 1) {
        hipLaunchKernelGGL((gemm_rows_kernel<WT, NT, NB, EPI>), dim3(gx, gy), dim3(RW_NW * 64), 0, s, w, aq, ad, m, out,
                           ldo, acc ? 1 : 0, per, kbs, (size_t)0, ep);
    } else {
        const size_t stride = (size_t)m * w.rows;
        hipLaunchKernelGGL((gemm_rows_kernel<WT, NT, NB, RW_STORE>), dim3(gx, gy, splits), dim3(RW_NW * 64), 0, s, w, aq,
                           ad, m, ws, w.rows, 0, per, kbs, stride, RowsEpi{});
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return set_error(SQ_ERR_HIP, std::string("gemm launch: ") + hipGetErrorString(e));
        if (const int st = launch_split_sum(s, ws, splits, stride, m, w.rows, out, ldo, acc)) return st;
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(SQ_ERR_HIP, std::string("gemm launch: ") + hipGetErrorString(e));
    return 0;
}

template <int WT>
int run_rows(hipStream_t s, const MatView& w, const int8_t* aq, const uint16_t* ad, int m, float* out, int ldo,
             bool acc, float* ws, size_t ws_floats) {
    const int KB = w.k / 32, cus = device_cus();
    const int gy = (m + 31) / 32, tiles = (w.rows + 31) / 32;
    const bool two = (tiles + 1) / 2 * gy >= cus;
    const int gx = two ? (tiles + 1) / 2 : tiles;
    int splits = 1;
    if (ws != nullptr && gx * gy < cus) {
        splits = min((cus + gx * gy - 1) / (gx * gy), KB / (RW_NW * 2 * RW_NB));
        while (splits > 1 && ((size_t)splits * m * w.rows > ws_floats || KB % splits || (KB / splits) % RW_NB))
            splits--;
        splits = max(splits, 1);
    }
    const int kbs = KB / splits;
    count_launch(splits, 32);
    return two ? launch_rows<WT, 2>(s, w, aq, ad, m, out, ldo, acc, gx, gy, splits, kbs, ws)
               : launch_rows<WT, 1>(s, w, aq, ad, m, out, ldo, acc, gx, gy, splits, kbs, ws);
}

// SQUIRREL_GEMM_TILE pins the prefill matmul's kernel (a test and
// measurement aid): "64" the 64 x 64 kernel, "128x64" and "128" the
// full-rate kernel on 128 x 64 or 128 x 128 tiles, "rows" the few-rows
// kernel.  Unset, inputs of at most 32 rows take the few-rows kernel, and
// larger ones the largest full-rate tiling whose grid fills the device.
enum : int { TILE_AUTO = 0, TILE_64 = 1, TILE_128X64 = 2, TILE_128 = 3, TILE_ROWS = 4 };
int gemm_tile_override() {
    const char* e = getenv("SQUIRREL_GEMM_TILE");
    if (!e) return TILE_AUTO;
    if (!strcmp(e, "64")) return TILE_64;
    if (!strcmp(e, "128x64")) return TILE_128X64;
    if (!strcmp(e, "128")) return TILE_128;
    if (!strcmp(e, "rows")) return TILE_ROWS;
    return TILE_AUTO;
}

// Inputs the few-rows kernel takes unless a tiling is pinned: up to 32 rows.
bool rows_kernel_fits(int m, int k) { return m <= 32 && (k / 32) % RW_NB == 0 && gemm_tile_override() == TILE_AUTO; }

// The full-rate tiling an input of m >= 128 rows takes with no tiling
// pinned (bn 0: neither; then the 64 x 64 kernel), shared by the plain path
// and the fused epilogues so that both fold the same terms:
//  - 128 x 128 tiles where they give every CU two workgroups;
//  - for Q8_0 weights, where 128 x 128 tiles cover a third to a half of the
//    device's three-per-CU slots, the same tiles with K split two or three
//    ways (one round; the partials summed in split order): the o and FFN
//    down projections of a 2048-token prompt (256 tiles) split three ways,
//    its q|k|v projection (384 tiles) two -- about half the time of the
//    unsplit 128 x 64 tiles for the down projection, whose 512 workgroups
//    leave a third of the direct-to-LDS kernel's slots empty;
//  - 128 x 64 tiles where those give every CU two workgroups.
struct Tiling {
    int bn, splits;
};
Tiling auto_tiling(const MatView& w, int wt, int m, bool have_ws, size_t ws_floats) {
    if (m < 128) return {0, 1};
    const int cus = device_cus(), gy = (m + 127) / 128, g = (w.rows + 127) / 128 * gy;
    if (g >= 2 * cus) return {128, 1};
    if (wt == WT_Q8_0 && w.k / 32 >= 64 && have_ws) {
        const int splits = (3 * cus + g - 1) / g;
        if (splits <= 3 && (size_t)splits * m * w.rows <= ws_floats) return {128, splits};
    }
    if ((w.rows + 63) / 64 * gy >= 2 * cus) return {64, 1};
    return {0, 1};
}

template <int WT>
int run_integer(hipStream_t s, const MatView& w, const int8_t* aq, const uint16_t* ad, int m, float* out, int ldo,
                bool acc, float* ws, size_t ws_floats) {
    const int tile = gemm_tile_override();
    if ((tile == TILE_ROWS && (w.k / 32) % RW_NB == 0) || rows_kernel_fits(m, w.k))
        return run_rows<WT>(s, w, aq, ad, m, out, ldo, acc, ws, ws_floats);
    if (tile == TILE_128)
        return run_mfma32<WT, 128, 128>(s, w, aq, ad, m, out, ldo, acc, ws, ws_floats, true);
    if (tile == TILE_128X64)
        return run_mfma32<WT, 128, 64>(s, w, aq, ad, m, out, ldo, acc, ws, ws_floats, true);
    if (tile == TILE_AUTO) {
        const Tiling t = auto_tiling(w, WT, m, ws != nullptr, ws_floats);
        const int g = (w.rows + 127) / 128 * ((m + 127) / 128);
        if (t.bn == 128)
            return run_mfma32<WT, 128, 128>(s, w, aq, ad, m, out, ldo, acc, ws, ws_floats, true,
                                            t.splits > 1 ? t.splits * g : 0);
        if (t.bn == 64) return run_mfma32<WT, 128, 64>(s, w, aq, ad, m, out, ldo, acc, ws, ws_floats, true);
    }
    return run_mfma<WT>(s, w, aq, ad, m, out, ldo, acc, ws, ws_floats);
}

// SQUIRREL_PREFILL_UNFUSED=1 turns the fused gate/up and q|k|v epilogues
// off (a test aid: the separate kernels give the same bits).
bool prefill_fusion_enabled() {
    const char* e = getenv("SQUIRREL_PREFILL_UNFUSED");
    return !(e && !strcmp(e, "1"));
}

// The direct-to-LDS kernel with a fused epilogue, where the unfused path
// would run that kernel on the same tiles with no K split (Q8_0, an even
// block count, a grid of at least two workgroups per CU and no pinned
// tiling); -1 when it does not apply.
template <int BN, int EPI>
int run_dma_fused(hipStream_t s, const MatView& w, const int8_t* aq, const uint16_t* ad, int m, int gx,
                  const RowsEpi& ep, size_t ws_floats) {
    const int KB = w.k / 32, gy = (m + 127) / 128;
    if (w.wtype != WT_Q8_0 || KB % DMA_KB || !dma_offsets_fit(w, m) || !gemm_dma_enabled() ||
        gemm_tile_override() != TILE_AUTO)
        return -1;
    const Tiling t = auto_tiling(w, WT_Q8_0, m, ws_floats > 0, ws_floats);  // the unfused path's choice
    if (t.bn != BN || t.splits != 1) return -1;
    count_launch(1, BN);
    hipLaunchKernelGGL((gemm_dma_kernel<128, BN, DMA_STAGES, DMA_KB, EPI>), dim3(gx, gy), dim3(256), 0, s, w, aq, ad, m,
                       nullptr, 0, 0, KB, (size_t)0, ep);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(SQ_ERR_HIP, std::string("gemm launch: ") + hipGetErrorString(e));
    return 0;
}

// The FFN gate/up projection with SiLU * up and its Q8_0 blocks fused (one
// launch instead of two): up to 32 prompt rows on the few-rows kernel, long
// prompts on the direct-to-LDS kernel; -1 when it does not apply.
template <int WT>
int run_gateup_silu(hipStream_t s, const MatView& w, const int8_t* aq, const uint16_t* ad, int m, int8_t* act_q,
                    uint16_t* act_d, size_t ws_floats) {
    const int ffn = w.rows / 2, KB = w.k / 32;
    if (w.rows % 2 || ffn % 32 || !prefill_fusion_enabled()) return -1;
    if (!rows_kernel_fits(m, w.k)) {
        if (ffn % 64) return -1;
        RowsEpi ep{};
        ep.act_q = act_q;
        ep.act_d = act_d;
        return run_dma_fused<128, RW_GATEUP>(s, w, aq, ad, m, ffn / 64, ep, ws_floats);
    }
    const int gx = ffn / 32, gy = (m + 31) / 32;
    if (gx * gy < device_cus()) return -1;  // the split-free two-tile form only
    count_launch(1, 32);
    RowsEpi ep{};
    ep.act_q = act_q;
    ep.act_d = act_d;
    return launch_rows<WT, 2, RW_GATEUP>(s, w, aq, ad, m, nullptr, 0, false, gx, gy, 1, KB, nullptr, ep);
}

// The stacked q|k|v projection of up to 32 prompt rows with RoPE and the
// KV-cache append fused (one launch instead of two); -1 when it does not
// apply.
template <int WT>
int run_qkv_rope(hipStream_t s, const MatView& w, const int8_t* aq, const uint16_t* ad, int m, const RowsEpi& ep,
                 float* ws, size_t ws_floats) {
    const int KB = w.k / 32, gx = (w.rows + 31) / 32, gy = (m + 31) / 32;
    if (ep.head_dim % 2 || (ep.q_dim + ep.kv_dim) % 2 || w.rows != ep.q_dim + 2 * ep.kv_dim ||
        !prefill_fusion_enabled())
        return -1;
    if (!rows_kernel_fits(m, w.k)) {
        if (ws == nullptr) ws_floats = 0;
        const Tiling t = auto_tiling(w, WT, m, ws_floats > 0, ws_floats);
        if (t.bn == 64) return run_dma_fused<64, RW_QKV>(s, w, aq, ad, m, (w.rows + 63) / 64, ep, ws_floats);
        if (t.bn == 128 && t.splits == 1)
            return run_dma_fused<128, RW_QKV>(s, w, aq, ad, m, (w.rows + 127) / 128, ep, ws_floats);
        // K split over 128 x 128 tiles: the partials, then their sum with
        // RoPE and the KV append (the plain path's split sum, then RoPE)
        if (WT != WT_Q8_0 || t.bn != 128 || KB % DMA_KB || !dma_offsets_fit(w, m) || !gemm_dma_enabled() ||
            gemm_tile_override() != TILE_AUTO)
            return -1;
        // the plain path's K partition (run_mfma32)
        const int chunks = (KB + M8_KB - 1) / M8_KB, kbs = (chunks + t.splits - 1) / t.splits * M8_KB;
        if ((KB + kbs - 1) / kbs != t.splits || kbs % DMA_KB) return -1;
        count_launch(t.splits, 128);
        const size_t stride = (size_t)m * w.rows;
        hipLaunchKernelGGL((gemm_dma_kernel<128, 128, DMA_STAGES, DMA_KB, RW_STORE>),
                           dim3((w.rows + 127) / 128, (m + 127) / 128, t.splits), dim3(256), 0, s, w, aq, ad, m, ws,
                           w.rows, 0, kbs, stride, RowsEpi{});
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return set_error(SQ_ERR_HIP, std::string("gemm launch: ") + hipGetErrorString(e));
        hipLaunchKernelGGL(split_sum_rope_kernel, dim3(m), dim3(256), 0, s, ws, t.splits, stride, w.rows, ep);
        e = hipGetLastError();
        if (e != hipSuccess) return set_error(SQ_ERR_HIP, std::string("split sum launch: ") + hipGetErrorString(e));
        return 0;
    }
    // where run_rows would pair tiles or split K (other sums than the plain path's)
    if ((gx + 1) / 2 * gy >= device_cus() || (gx * gy < device_cus() && KB / (RW_NW * 2 * RW_NB) >= 2)) return -1;
    count_launch(1, 32);
    return launch_rows<WT, 1, RW_QKV>(s, w, aq, ad, m, nullptr, 0, false, gx, gy, 1, KB, nullptr, ep);
}

template <int WT, bool A8, int NBL, int MT>
int run(hipStream_t s, const MatView& w, const int8_t* aq, const uint16_t* ad, const float* x, int m,
        float* out, int ldo, bool acc) {
    dim3 grid((w.rows + TN - 1) / TN, (m + MT - 1) / MT);
    hipLaunchKernelGGL((gemm_kernel<WT, A8, NBL, MT>), grid, dim3(WAVES * 64), 0, s, w, aq, ad, x, m, out,
                       ldo, acc ? 1 : 0);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(SQ_ERR_HIP, std::string("gemm launch: ") + hipGetErrorString(e));
    return 0;
}

template <int WT, bool A8>
int dispatch(hipStream_t s, const MatView& w, const int8_t* aq, const uint16_t* ad, const float* x, int m,
             float* out, int ldo, bool acc) {
    const int KB = w.k / 32;
    if constexpr (A8) {
        if (KB <= 64) return run<WT, true, 1, 16>(s, w, aq, ad, x, m, out, ldo, acc);
        if (KB <= 256) return run<WT, true, 4, 8>(s, w, aq, ad, x, m, out, ldo, acc);
    } else {
        if (KB <= 64) return run<WT, false, 1, 8>(s, w, aq, ad, x, m, out, ldo, acc);
        if (KB <= 256) return run<WT, false, 4, 2>(s, w, aq, ad, x, m, out, ldo, acc);
    }
    return set_error(SQ_ERR_SHAPE, "gemm: k above 8192 is not supported");
}

}  // namespace

void gemm_counters(bool reset, uint64_t* out) {
    if (out) {
        out[0] = g_launches.load();
        out[1] = g_split_launches.load();
        out[2] = g_tile128_launches.load();
        out[3] = g_max_splits.load();
        out[4] = g_tile128x64_launches.load();
        out[5] = g_rows_launches.load();
    }
    if (reset) {
        g_launches = 0;
        g_split_launches = 0;
        g_tile128_launches = 0;
        g_max_splits = 0;
        g_tile128x64_launches = 0;
        g_rows_launches = 0;
    }
}

int launch_gateup_silu(hipStream_t s, const MatView& w, int wtype, const int8_t* aq, const uint16_t* ad, int m,
                       int8_t* act_q, uint16_t* act_d, size_t ws_floats) {
    if (w.k <= 0 || w.k % 32 != 0 || m <= 0) return -1;
    MatView v = w;
    v.wtype = wtype;
    if (wtype == WT_Q8_0) return run_gateup_silu<WT_Q8_0>(s, v, aq, ad, m, act_q, act_d, ws_floats);
    if (wtype == WT_Q4_0) return run_gateup_silu<WT_Q4_0>(s, v, aq, ad, m, act_q, act_d, ws_floats);
    return -1;
}

int launch_qkv_rope(hipStream_t s, const MatView& w, int wtype, const int8_t* aq, const uint16_t* ad, int m,
                    int q_dim, int kv_dim, int head_dim, int pos0, const float2* rope, float* q_out, float* kcache,
                    float* vcache, float* ws, size_t ws_floats) {
    if (w.k <= 0 || w.k % 32 != 0 || m <= 0) return -1;
    MatView v = w;
    v.wtype = wtype;
    RowsEpi ep{};
    ep.rope = rope;
    ep.q_out = q_out;
    ep.kcache = kcache;
    ep.vcache = vcache;
    ep.q_dim = q_dim;
    ep.kv_dim = kv_dim;
    ep.head_dim = head_dim;
    ep.pos0 = pos0;
    if (wtype == WT_Q8_0) return run_qkv_rope<WT_Q8_0>(s, v, aq, ad, m, ep, ws, ws_floats);
    if (wtype == WT_Q4_0) return run_qkv_rope<WT_Q4_0>(s, v, aq, ad, m, ep, ws, ws_floats);
    return -1;
}

int launch_gemm(hipStream_t s, const MatView& w, int wtype, bool a8, const int8_t* aq, const uint16_t* ad,
                const float* x, int m, float* out, int ldo, bool accumulate, float* ws, size_t ws_floats) {
    if (w.k <= 0 || w.k % 32 != 0) return set_error(SQ_ERR_SHAPE, "gemm: k must be a positive multiple of 32");
    if (m <= 0) return set_error(SQ_ERR_EMPTY, "gemm: no rows");
    MatView v = w;
    v.wtype = wtype;
    switch (wtype) {
        // the integer path runs on the matrix cores
        // (without a workspace for a K split, inputs below one 64-row tile
        // stay on the VALU kernel, which spreads the weights over more workgroups)
        case WT_Q8_0:
            if (a8 && (m >= MQ_T || ws != nullptr || rows_kernel_fits(m, w.k)))
                return run_integer<WT_Q8_0>(s, v, aq, ad, m, out, ldo, accumulate, ws, ws_floats);
            return a8 ? dispatch<WT_Q8_0, true>(s, v, aq, ad, x, m, out, ldo, accumulate)
                      : dispatch<WT_Q8_0, false>(s, v, aq, ad, x, m, out, ldo, accumulate);
        case WT_Q4_0:
            if (a8 && (m >= MQ_T || ws != nullptr || rows_kernel_fits(m, w.k)))
                return run_integer<WT_Q4_0>(s, v, aq, ad, m, out, ldo, accumulate, ws, ws_floats);
            return a8 ? dispatch<WT_Q4_0, true>(s, v, aq, ad, x, m, out, ldo, accumulate)
                      : dispatch<WT_Q4_0, false>(s, v, aq, ad, x, m, out, ldo, accumulate);
        case WT_BF16:
            if (a8) return set_error(SQ_ERR_INVALID_TYPE, "gemm: BF16 weights take f32 activations");
            return dispatch<WT_BF16, false>(s, v, aq, ad, x, m, out, ldo, accumulate);
        default:
            return set_error(SQ_ERR_INVALID_TYPE, "gemm: unsupported weight type");
    }
}

}  // namespace sq
