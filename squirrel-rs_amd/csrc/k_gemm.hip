// Multi-row matmul for the batched prefill: out[m, n] (+)= in[m, :] . W[n, :].
//
// A tile of MT activation rows is staged in LDS once; each wavefront then
// streams weight rows (lane = 32-block, as in the decode matvec) and dots
// every row of the tile against them, so weights are read ceil(M/MT) times
// instead of M times (the reference re-streams them per row,
// src/kernels/matmul.rs:34).  Per-block arithmetic is the decode matvec's:
// exact i32 block sums, term = (f32(isum) * sa) * sw.
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

int launch_gemm(hipStream_t s, const MatView& w, int wtype, bool a8, const int8_t* aq, const uint16_t* ad,
                const float* x, int m, float* out, int ldo, bool accumulate) {
    if (w.k <= 0 || w.k % 32 != 0) return set_error(SQ_ERR_SHAPE, "gemm: k must be a positive multiple of 32");
    if (m <= 0) return set_error(SQ_ERR_EMPTY, "gemm: no rows");
    MatView v = w;
    v.wtype = wtype;
    switch (wtype) {
        case WT_Q8_0:
            return a8 ? dispatch<WT_Q8_0, true>(s, v, aq, ad, x, m, out, ldo, accumulate)
                      : dispatch<WT_Q8_0, false>(s, v, aq, ad, x, m, out, ldo, accumulate);
        case WT_Q4_0:
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
