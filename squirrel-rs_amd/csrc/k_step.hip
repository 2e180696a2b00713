// Persistent decode step: one launch computes a whole token.
//
// The decode step is a chain of dependent matvecs (per layer: QKV, attention,
// o-projection, gate/up, down; then the LM head).  As separate kernels every
// link pays a launch, a ramp-up and a tail.  Here one workgroup per CU stays
// resident for the whole token and the links are data dependencies between
// workgroups, resolved through memory:
//
// * Exchange words.  Every value handed from one phase to the next (hidden
//   row, q row, the new K/V row, quantized activations, argmax partials) is
//   stored as a 64-bit word: payload in the low half, the producing phase's
//   tag in the high half, with an agent-scope atomic store (coherent across
//   the XCDs' L2s, single-copy atomic).  A consumer polls the words it needs
//   with agent-scope loads until each carries the expected tag.  There are no
//   grid barriers, no flags and no store-completion waits: a consumer starts
//   as soon as its own inputs exist.
// * Tags are `epoch + phase` and grow across launches (the epoch word is
//   advanced by every launch), so a word from an earlier phase or launch never
//   matches.  A workgroup reads a phase's inputs only when it has work in that
//   phase; the dependency chain then guarantees no input is overwritten before
//   every workgroup that needs it has read it.
// * The residual stream stays in registers: wavefront w owns hidden row w and
//   adds the o-projection and down outputs of that row to it.
// * Weights of the next phase are requested as soon as the current phase's
//   inputs have arrived, so the HBM stream runs ahead of the dependency chain.
// * Every wait is bounded by a wall-clock limit and a poll count: on expiry
//   the workgroup raises the launch's error word; every waiting workgroup sees
//   it and leaves, so the grid always drains.
//
// Arithmetic per phase is that of the multi-kernel path (k_gemv.hip,
// k_attn.hip): the reference's integer block dot (dot_prod.rs:378-403), its
// RMSNorm (rms_norm.rs:40-56), Q8_0 activation quantizer (dot_prod.rs:21-31),
// interleaved RoPE (rope.rs:7-36), SDPA (attention.rs:11-70), SiLU
// (silu.rs, sigmoid.rs) and greedy tie rule (greedy.rs:6-15).
#include "launch.h"

namespace sq {

namespace {

constexpr int SW = 8;          // wavefronts per workgroup
constexpr int SNT = SW * 64;   // threads per workgroup
constexpr int HDIM = 64;       // head_dim
constexpr int TPOS = 64;       // attention positions per tile
constexpr int CHUNK = 1;       // tiles per attention work item
constexpr int DMAX = 2048;     // model width supported
constexpr int FMAX = 8192;     // FFN width supported
constexpr int MAXG = 8;        // GQA group size supported
constexpr int XMAX = FMAX / 4 + FMAX / 32;  // exchange words gathered at once
constexpr int WPT = (XMAX + SNT - 1) / SNT; // ... per thread

typedef float sq_v4f __attribute__((ext_vector_type(4)));
typedef unsigned long long u64;

// ---- global address space ----------------------------------------------------
// Pointers read from memory (the per-layer views) are generic to the
// compiler, which would access them with flat instructions.  A flat load also
// counts against lgkmcnt, so every LDS or scalar wait would stall behind the
// weight stream.  All device-memory accesses here go through these casts.
template <typename T>
using gptr = __attribute__((address_space(1))) T*;
template <typename T>
__device__ __forceinline__ gptr<T> gl(T* p) {
    return (gptr<T>)p;
}
template <typename T>
__device__ __forceinline__ gptr<const T> gl(const T* p) {
    return (gptr<const T>)p;
}

// Read-only for the whole launch (per-layer views): constant address space,
// so the compiler reads it with scalar loads instead of vector loads that
// would queue behind the weight stream.
template <typename T>
using cptr = const __attribute__((address_space(4))) T*;

__device__ __forceinline__ MatView view_of(const __attribute__((address_space(4))) MatView& v) {
    MatView m;
    m.qs = v.qs;
    m.scale = v.scale;
    m.rows = v.rows;
    m.k = v.k;
    m.wtype = v.wtype;
    return m;
}

template <typename T>
__device__ __forceinline__ T ld_c(const T* p) {
    return __hip_atomic_load((gptr<T>)const_cast<T*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ void st_c(T* p, T v) {
    __hip_atomic_store(gl(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void put(u64* p, unsigned payload, unsigned tag) {
    st_c(p, ((u64)tag << 32) | payload);
}
__device__ __forceinline__ void putf(u64* p, float v, unsigned tag) { put(p, __builtin_bit_cast(unsigned, v), tag); }

// ---- waiting ---------------------------------------------------------------
struct Ctl {
    int* error;
    long long limit;  // wall-clock ticks one wait may take
};

// Poll one word until it carries `tag`.  False on timeout or a raised error.
__device__ __forceinline__ bool await_word(const u64* p, u64& w, unsigned tag, const Ctl& C) {
    if ((unsigned)(w >> 32) == tag) return true;
    const long long t0 = wall_clock64();
    for (int polls = 1;; polls++) {
        __builtin_amdgcn_s_sleep(4);
        w = ld_c(p);
        if ((unsigned)(w >> 32) == tag) return true;
        if ((polls & 15) == 0) {
            if (ld_c(C.error) != 0) return false;
            if (wall_clock64() - t0 > C.limit || polls > (1 << 20)) {
                st_c(C.error, 1);
                return false;
            }
        }
    }
}

struct StepShared {
    alignas(16) unsigned xw[XMAX];  // gathered exchange payloads
    alignas(16) int8_t qs[DMAX];
    uint16_t d[DMAX / 32];
    int asum[DMAX / 32];
    float red[SW];
    float gu[64];
    float bv[SW];
    int bi[SW];
    int bn[SW];
    int abort;
    // attention
    float k[TPOS][HDIM + 1];
    alignas(16) float v[TPOS][HDIM];
    float qh[MAXG][HDIM];
    float p[MAXG][TPOS];
    float m[MAXG], l[MAXG];
};

// The whole workgroup gathers words src[0..n) once they carry `tag`; their
// payloads land in S.xw.  False: the launch is being abandoned.
__device__ __forceinline__ bool gather(StepShared& S, const u64* src, int n, unsigned tag, const Ctl& C) {
    const int tid = threadIdx.x;
    u64 w[WPT];
#pragma unroll
    for (int j = 0; j < WPT; j++) {
        const int i = tid + j * SNT;
        w[j] = i < n ? ld_c(src + i) : 0;
    }
    bool ok = true;
#pragma unroll
    for (int j = 0; j < WPT; j++) {
        const int i = tid + j * SNT;
        if (i < n && ok) {
            ok = await_word(src + i, w[j], tag, C);
            S.xw[i] = (unsigned)w[j];
        }
    }
    if (!ok) S.abort = 1;
    __syncthreads();
    return S.abort == 0;
}

// ---- weight rows held in registers ------------------------------------------
template <int WT>
struct Blk;
template <>
struct Blk<WT_Q8_0> { static constexpr int DW = 8; };
template <>
struct Blk<WT_Q4_0> { static constexpr int DW = 4; };

template <int WT, int NBL, int R>
struct Rows {
    int w[R][NBL][Blk<WT>::DW];
    uint16_t d[R][NBL];
};

// A zero fp16 scale: rows and blocks a lane does not own read it, so their
// terms vanish without a branch around the loads.
__device__ const uint16_t kZeroScale = 0;

// Rows `row[r]` (negative: none) of m, the lane's blocks lane, lane+64, ...
// Branch-free: every lane issues all its loads back to back (a missing row or
// block reads row 0 / block 0 with a zero scale).  A branch per row would let
// the compiler place each row's scale conversion inside the branch, making
// every row wait for the previous row's scale load.
template <int WT, int NBL, int R>
__device__ __forceinline__ void load_rows(Rows<WT, NBL, R>& B, const MatView& m, const int (&row)[R], int lane) {
    constexpr int DW = Blk<WT>::DW;
    const int KB = m.k >> 5;
    const size_t row_bytes = (size_t)KB * (DW * 4);
    const gptr<const uint8_t> base = gl((const uint8_t*)m.qs);
    const gptr<const uint16_t> scale = gl(m.scale);
#pragma unroll
    for (int r = 0; r < R; r++) {
#pragma unroll
        for (int b = 0; b < NBL; b++) {
            const int blk = lane + 64 * b;
            const bool valid = row[r] >= 0 && blk < KB;
            const size_t rr = valid ? (size_t)row[r] : 0;
            const int bb = valid ? blk : 0;
            const gptr<const sq_v4i> p = (gptr<const sq_v4i>)(base + rr * row_bytes + (size_t)bb * (DW * 4));
#pragma unroll
            for (int v = 0; v < DW / 4; v++) {
                const sq_v4i x = __builtin_nontemporal_load(p + v);
                B.w[r][b][4 * v + 0] = x.x;
                B.w[r][b][4 * v + 1] = x.y;
                B.w[r][b][4 * v + 2] = x.z;
                B.w[r][b][4 * v + 3] = x.w;
            }
            B.d[r][b] = *(valid ? scale + rr * KB + bb : gl(&kZeroScale));
        }
    }
}

// Quantized activation blocks of one lane (lane, lane+64, ...).
template <int NBL>
struct Act {
    int q[NBL][8];
    float s[NBL];
    int sum[NBL];  // sum of the block's q (Q4_0 offset term)
};

// res[r] = sum over blocks of (f32(isum) * sa) * sw, wavefront-reduced.
template <int WT, int NBL, int R>
__device__ __forceinline__ void dot_rows(const Rows<WT, NBL, R>& B, const Act<NBL>& A, int KB, int lane,
                                         float (&res)[R]) {
#pragma unroll
    for (int r = 0; r < R; r++) {
        float acc = 0.0f;
#pragma unroll
        for (int b = 0; b < NBL; b++) {
            const int blk = lane + 64 * b;
            if (blk >= KB) continue;
            int isum = 0;
            if constexpr (WT == WT_Q8_0) {
#pragma unroll
                for (int v = 0; v < 8; v++) isum = __builtin_amdgcn_sdot4(A.q[b][v], B.w[r][b][v], isum, false);
            } else {
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const int dw = B.w[r][b][v];
                    isum = __builtin_amdgcn_sdot4(A.q[b][v], dw & 0x0F0F0F0F, isum, false);
                    isum = __builtin_amdgcn_sdot4(A.q[b][4 + v], (dw >> 4) & 0x0F0F0F0F, isum, false);
                }
                isum -= 8 * A.sum[b];
            }
            acc += sq_q_term(isum, A.s[b], sq_f16_to_f32(B.d[r][b]));
        }
        res[r] = sq_wave_sum(acc);
    }
}

// Activation blocks from gathered exchange payloads: nblk blocks of 8 payload
// words (32 int8) at S.xw[0..), then nblk scale words (f32 of the fp16 scale).
template <int WT, int NBL>
__device__ __forceinline__ void act_from_xw(Act<NBL>& A, const StepShared& S, int nblk, int lane) {
#pragma unroll
    for (int b = 0; b < NBL; b++) {
        const int blk = lane + 64 * b;
        if (blk < nblk) {
#pragma unroll
            for (int v = 0; v < 8; v++) A.q[b][v] = (int)S.xw[blk * 8 + v];
            A.s[b] = __builtin_bit_cast(float, S.xw[nblk * 8 + blk]);
        } else {
#pragma unroll
            for (int v = 0; v < 8; v++) A.q[b][v] = 0;
            A.s[b] = 0.0f;
        }
        int s = 0;
        if constexpr (WT == WT_Q4_0) {
#pragma unroll
            for (int v = 0; v < 8; v++) s = __builtin_amdgcn_sdot4(A.q[b][v], 0x01010101, s, false);
        }
        A.sum[b] = s;
    }
}

// One row against activation blocks gathered in S.xw (nblk blocks of 8
// payload words, then nblk scale words), read from LDS as they are used.
template <int WT, int NBL>
__device__ __forceinline__ float dot_row_xw(const Rows<WT, NBL, 1>& B, const StepShared& S, int nblk, int lane) {
    float acc = 0.0f;
#pragma unroll
    for (int b = 0; b < NBL; b++) {
        const int blk = lane + 64 * b;
        if (blk >= nblk) continue;
        const uint4* pq = (const uint4*)(S.xw + blk * 8);
        const uint4 a0 = pq[0], a1 = pq[1];
        const int aq[8] = {(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w, (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
        const float sa = __builtin_bit_cast(float, S.xw[nblk * 8 + blk]);
        int isum = 0;
        if constexpr (WT == WT_Q8_0) {
#pragma unroll
            for (int v = 0; v < 8; v++) isum = __builtin_amdgcn_sdot4(aq[v], B.w[0][b][v], isum, false);
        } else {
            int asum = 0;
#pragma unroll
            for (int v = 0; v < 8; v++) asum = __builtin_amdgcn_sdot4(aq[v], 0x01010101, asum, false);
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int dw = B.w[0][b][v];
                isum = __builtin_amdgcn_sdot4(aq[v], dw & 0x0F0F0F0F, isum, false);
                isum = __builtin_amdgcn_sdot4(aq[4 + v], (dw >> 4) & 0x0F0F0F0F, isum, false);
            }
            isum -= 8 * asum;
        }
        acc += sq_q_term(isum, sa, sq_f16_to_f32(B.d[0][b]));
    }
    return sq_wave_sum(acc);
}

// Quantize 32-element blocks held one element per lane (lanes 0..31 and
// 32..63 are two blocks) and publish them: payload words q[blk*8 + j] and
// scale words s[blk] (f32 of the fp16 scale), blk = block0 + (lane >> 5).
// Lanes with `valid` false hold no element (their half is not published).
__device__ __forceinline__ void quant_put(float v, int lane, int block0, u64* q, u64* s, unsigned tag, bool valid) {
    const float amax = fmaxf(sq_half_max(fabsf(valid ? v : 0.0f)), 0.0f);
    const float sc = sq_q8_scale(amax);
    const int qv = valid ? ((int)sq_q8_quant(v, sq_q8_inv(sc)) & 0xFF) : 0;
    const int b1 = __shfl_down(qv, 1, 64), b2 = __shfl_down(qv, 2, 64), b3 = __shfl_down(qv, 3, 64);
    const int blk = block0 + (lane >> 5);
    if ((lane & 3) == 0 && valid)
        put(q + (size_t)blk * 8 + ((lane & 31) >> 2), (unsigned)(qv | (b1 << 8) | (b2 << 16) | (b3 << 24)), tag);
    if ((lane & 31) == 0 && valid) putf(s + blk, sq_f16_to_f32(sq_f32_to_f16(sc)), tag);
}

// RMSNorm of a D-wide row (x: EPT elements per thread, indexes tid + j*SNT)
// and Q8_0 quantization into S.qs / S.d (rms_norm.rs:40-56, dot_prod.rs:21-31).
constexpr int EPT = DMAX / SNT;
// Norm gains of the row elements a thread owns, requested ahead of the
// phase's input gather so both arrive together.
__device__ __forceinline__ void load_gains(float (&nw)[EPT], const float* w, int D) {
#pragma unroll
    for (int j = 0; j < EPT; j++) {
        const int i = threadIdx.x + j * SNT;
        nw[j] = i < D ? gl(w)[i] : 0.0f;
    }
}

template <int WT>
__device__ __forceinline__ void norm_quant(StepShared& S, const float (&x)[EPT], const float (&nw)[EPT], int D,
                                           float eps, float* dbg_y, int8_t* dbg_q, uint16_t* dbg_d) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < EPT; j++) ss += x[j] * x[j];
    ss = sq_wave_sum(ss);
    if (lane == 0) S.red[wave] = ss;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int k = 0; k < SW; k++) tot += S.red[k];
    const float rms = sqrtf(tot / (float)D + eps);
#pragma unroll
    for (int j = 0; j < EPT; j++) {
        const int i = tid + j * SNT;
        const bool vi = i < D;
        const float y = vi ? (x[j] * nw[j]) / rms : 0.0f;
        const float amax = fmaxf(sq_half_max(fabsf(y)), 0.0f);
        const float sc = sq_q8_scale(amax);
        const int8_t q = sq_q8_quant(y, sq_q8_inv(sc));
        if (vi) {
            S.qs[i] = q;
            if ((i & 31) == 0) S.d[i >> 5] = sq_f32_to_f16(sc);
            if (dbg_y) {
                dbg_y[i] = y;
                dbg_q[i] = q;
                if ((i & 31) == 0) dbg_d[i >> 5] = sq_f32_to_f16(sc);
            }
        }
        if constexpr (WT == WT_Q4_0) {
            int qi = q;
#pragma unroll
            for (int o = 16; o >= 1; o >>= 1) qi += __shfl_xor(qi, o, 64);
            if (vi && (i & 31) == 0) S.asum[i >> 5] = qi;
        }
    }
    __syncthreads();
}

template <int WT>
__device__ __forceinline__ void act_from_lds(Act<1>& A, const StepShared& S, int KB, int lane) {
    if (lane < KB) {
        const int4* p = (const int4*)(S.qs + lane * 32);
        const int4 x0 = p[0], x1 = p[1];
        A.q[0][0] = x0.x; A.q[0][1] = x0.y; A.q[0][2] = x0.z; A.q[0][3] = x0.w;
        A.q[0][4] = x1.x; A.q[0][5] = x1.y; A.q[0][6] = x1.z; A.q[0][7] = x1.w;
        A.s[0] = sq_f16_to_f32(S.d[lane]);
        A.sum[0] = (WT == WT_Q4_0) ? S.asum[lane] : 0;
    } else {
#pragma unroll
        for (int v = 0; v < 8; v++) A.q[0][v] = 0;
        A.s[0] = 0.0f;
        A.sum[0] = 0;
    }
}

// Gathered hidden row -> x[] (element tid + j*SNT).
__device__ __forceinline__ void x_from_xw(float (&x)[EPT], const StepShared& S, int D) {
#pragma unroll
    for (int j = 0; j < EPT; j++) {
        const int i = threadIdx.x + j * SNT;
        x[j] = i < D ? __builtin_bit_cast(float, S.xw[i]) : 0.0f;
    }
}

__device__ __forceinline__ void arg_merge(float& bv, int& bi, int& bn, float v, int i, int n) {
    if (i >= 0 && (bi < 0 || v > bv || (v == bv && i > bi))) {
        bv = v;
        bi = i;
    }
    bn = n > bn ? n : bn;
}

__device__ __forceinline__ void block_arg(StepShared& S, float& bv, int& bi, int& bn) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        const int on = __shfl_xor(bn, o, 64);
        arg_merge(bv, bi, bn, ov, oi, on);
    }
    __syncthreads();
    if (lane == 0) {
        S.bv[wave] = bv;
        S.bi[wave] = bi;
        S.bn[wave] = bn;
    }
    __syncthreads();
    bv = S.bv[0];
    bi = S.bi[0];
    bn = S.bn[0];
    for (int w = 1; w < SW; w++) arg_merge(bv, bi, bn, S.bv[w], S.bi[w], S.bn[w]);
}

// Phase tags: layer l, phase j in [0, 6): QKV, attention, tile merge, o, gate/up, down.
enum : int { PH_QKV = 0, PH_ATTN = 1, PH_MERGE = 2, PH_O = 3, PH_GU = 4, PH_DOWN = 5, PH_PER_LAYER = 6 };
// Timeline slots of one layer (optional measurement).
enum TraceSlot : int {
    TS_QKV_IN = 0, TS_QKV = 1, TS_ATTN = 2, TS_MERGE = 3, TS_O_IN = 4, TS_O = 5, TS_GU_IN = 6, TS_GU_DOT = 7,
    TS_GU = 8, TS_DOWN_IN = 9, TS_DOWN = 10, TS_PER_LAYER = 16
};

template <int WT>
__global__ __launch_bounds__(SNT, 1) void decode_step_kernel(StepArgs a) {
    __shared__ StepShared S;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int G = gridDim.x, wg = blockIdx.x;
    const int NW = G * SW;             // wavefronts in the launch
    const int gw = wg * SW + wave;     // this wavefront's global index
    const int D = a.dim, F = a.ffn;
    const int QD = a.n_heads * HDIM, KVD = a.n_kv_heads * HDIM;
    const int KB = D >> 5;
    const int GQ = a.n_heads / a.n_kv_heads;
    const Ctl C{a.error, a.spin_limit};
    const unsigned epoch = *a.epoch;
    auto tag = [&](int l, int ph) -> unsigned { return epoch + 1u + (unsigned)(l * PH_PER_LAYER + ph); };
    const unsigned head_tag = epoch + 1u + (unsigned)(a.n_layers * PH_PER_LAYER);
    const int pos = *a.pos;
    const uint32_t tok = *a.token;
    const int P = pos + 1;
    const int ntiles = (P + TPOS - 1) / TPOS;
    const int nchunks = (ntiles + CHUNK - 1) / CHUNK;
    const Xchg X = a.x;
    if (tid == 0) S.abort = 0;
    if (a.trace && tid == 0) a.trace[(size_t)wg * a.trace_stride] = wall_clock64();
    __syncthreads();
    // timeline slots per layer (measurement): see TraceSlot
    auto stamp = [&](int l, int slot) {
        if (a.trace && tid == 0) {
            const int k = 1 + l * TS_PER_LAYER + slot;
            if (k < a.trace_stride) a.trace[(size_t)wg * a.trace_stride + k] = wall_clock64();
        }
    };

    const int q_units = (QD + 2 * KVD) / 2;   // RoPE pairs of the stacked QKV rows
    const int gu_tiles = F / 32;

    // The residual row this wavefront owns (hidden[gw]), from the embedding
    // of the token (embed, model.rs:57-62; dequantize_into is exact).
    auto embed_at = [&](int i) -> float {
        const float sc = sq_f16_to_f32(gl(a.embd.scale)[(size_t)tok * KB + (i >> 5)]);
        if constexpr (WT == WT_Q8_0) {
            return sc * (float)gl((const int8_t*)a.embd.qs)[(size_t)tok * D + i];
        } else {
            const gptr<const uint8_t> qs = gl((const uint8_t*)a.embd.qs) + (size_t)tok * (D / 2) + (i >> 5) * 16;
            const int jj = i & 31;
            const int q = jj < 16 ? (qs[jj] & 0x0F) : (qs[jj - 16] >> 4);
            return sc * (float)(q - 8);
        }
    };
    float h_own = gw < D ? embed_at(gw) : 0.0f;

    float x[EPT];
    Rows<WT, 1, 2> Wq;
    Rows<WT, 1, 1> Wo;
    Rows<WT, 1, 8> Wg;
    Rows<WT, 4, 1> Wd;
    Rows<WT, 1, 4> Wh0, Wh1;

    auto qkv_rows = [&](int u, int (&rr)[2]) {
        rr[0] = u < q_units ? 2 * u : -1;
        rr[1] = u < q_units ? 2 * u + 1 : -1;
    };
    auto gu_rows = [&](int t, int (&rr)[8]) {
#pragma unroll
        for (int r = 0; r < 8; r++) {
            const int slot = wave * 8 + r;
            rr[r] = t < gu_tiles ? (slot < 32 ? t * 32 + slot : F + t * 32 + (slot - 32)) : -1;
        }
    };
    auto head_rows = [&](int u, int (&rr)[4]) {
#pragma unroll
        for (int r = 0; r < 4; r++) rr[r] = (4 * u + r < a.vocab) ? 4 * u + r : -1;
    };
    const cptr<StepLayer> LY = (cptr<StepLayer>)a.layers;
    float nw[EPT];
    {
        int rr[2];
        qkv_rows(gw, rr);
        const MatView m0 = view_of(LY[0].qkv);
        load_rows(Wq, m0, rr, lane);
    }

    for (int l = 0; l < a.n_layers; l++) {

        const gptr<float> kc = gl(a.kcache + (size_t)l * a.kv_layer);
        const gptr<float> vc = gl(a.vcache + (size_t)l * a.kv_layer);

        // ------------------------------------------------ QKV + RoPE + KV append
        {
            const unsigned T = tag(l, PH_QKV);
            const bool work = wg * SW < q_units;
            // RoPE (cos, sin) of this wavefront's row pair, requested early
            float rc = 1.0f, rs = 0.0f;
            if (gw < q_units && 2 * gw < QD + KVD) {
                const int li = 2 * gw < QD ? 2 * gw : 2 * gw - QD;
                const gptr<const float> cs =
                    gl((const float*)a.rope) + 2 * ((size_t)pos * (HDIM / 2) + ((li % HDIM) >> 1));
                rc = cs[0];
                rs = cs[1];
            }
            if (work) {
                load_gains(nw, LY[l].attn_norm, D);
                if (l == 0) {
#pragma unroll
                    for (int j = 0; j < EPT; j++) {
                        const int i = tid + j * SNT;
                        x[j] = i < D ? embed_at(i) : 0.0f;
                    }
                } else {
                    if (!gather(S, X.h, D, tag(l - 1, PH_DOWN), C)) return;
                    x_from_xw(x, S, D);
                }
            }
            stamp(l, TS_QKV_IN);
            if (work) {
                const bool dbg = l == 0 && wg == 0 && a.dbg_normed != nullptr;
                norm_quant<WT>(S, x, nw, D, a.eps, dbg ? a.dbg_normed : nullptr, a.dbg_qs, a.dbg_d);
                Act<1> A;
                act_from_lds<WT>(A, S, KB, lane);
                if (gw < q_units) {
                    const int u = gw;
                    float res[2];
                    dot_rows<WT, 1, 2>(Wq, A, KB, lane, res);
                    if (lane == 0) {
                        const int row = 2 * u;
                        if (row < QD + KVD) {
                            const bool is_q = row < QD;
                            const int li = is_q ? row : row - QD;
                            float o0, o1;
                            sq_rotate(res[0], res[1], rc, rs, o0, o1);
                            if (is_q) {
                                putf(X.q + li, o0, T);
                                putf(X.q + li + 1, o1, T);
                            } else {
                                kc[(size_t)pos * KVD + li] = o0;
                                kc[(size_t)pos * KVD + li + 1] = o1;
                                putf(X.k + li, o0, T);
                                putf(X.k + li + 1, o1, T);
                            }
                        } else {
                            const int li = row - QD - KVD;
                            vc[(size_t)pos * KVD + li] = res[0];
                            vc[(size_t)pos * KVD + li + 1] = res[1];
                            putf(X.v + li, res[0], T);
                            putf(X.v + li + 1, res[1], T);
                        }
                    }
                }
            }
            // the o-projection row of this wavefront, requested after the
            // outputs are out (registers of pending loads would hold them up)
            {
                const int rr[1] = {gw < D ? gw : -1};
                const MatView mv = view_of(LY[l].o);
                load_rows(Wo, mv, rr, lane);
            }
            stamp(l, TS_QKV);
        }

        // ------------------------------------------------ attention (GQA)
        // Work item = (kv head, chunk of tiles): one 64-position tile per item
        // (CHUNK = 1); the partials of a head merge across workgroups.
        {
            const unsigned Tin = tag(l, PH_QKV), T = tag(l, PH_ATTN);
            const int items = a.n_kv_heads * nchunks;
            const float scale = 1.0f / sqrtf((float)HDIM);
            for (int it = wg; it < items; it += G) {
                const int g = it / nchunks, tile = it % nchunks;
                const int s0 = tile * TPOS;
                const bool cur = s0 + TPOS > pos;  // this tile holds the new position
                // q of the group's heads and, in the last tile, the new K/V row
                {
                    const int nq = GQ * HDIM;
                    const int n = nq + (cur ? 2 * HDIM : 0);
                    bool ok = true;
                    for (int e = tid; e < n; e += SNT) {
                        const u64* src = e < nq ? X.q + (size_t)g * nq + e
                                                : (e < nq + HDIM ? X.k + g * HDIM + (e - nq) : X.v + g * HDIM + (e - nq - HDIM));
                        u64 w = ld_c(src);
                        if (!await_word(src, w, Tin, C)) {
                            ok = false;
                            break;
                        }
                        const float f = __builtin_bit_cast(float, (unsigned)w);
                        if (e < nq) S.qh[e / HDIM][e % HDIM] = f;
                        else if (e < nq + HDIM) S.k[pos - s0][e - nq] = f;
                        else S.v[pos - s0][e - nq - HDIM] = f;
                    }
                    if (!ok) S.abort = 1;
                }
                for (int e = tid; e < TPOS * HDIM / 4; e += SNT) {
                    const int r = e / (HDIM / 4), c4 = e % (HDIM / 4);
                    const int sp = s0 + r;
                    if (sp == pos) continue;  // gathered above
                    float4 k4 = make_float4(0.f, 0.f, 0.f, 0.f), v4 = k4;
                    if (sp < pos) {
                        const size_t off = (size_t)sp * KVD + g * HDIM + 4 * c4;
                        const sq_v4f kk = *(gptr<const sq_v4f>)(kc + off);
                        const sq_v4f vv = *(gptr<const sq_v4f>)(vc + off);
                        k4 = make_float4(kk.x, kk.y, kk.z, kk.w);
                        v4 = make_float4(vv.x, vv.y, vv.z, vv.w);
                    }
                    S.k[r][4 * c4 + 0] = k4.x;
                    S.k[r][4 * c4 + 1] = k4.y;
                    S.k[r][4 * c4 + 2] = k4.z;
                    S.k[r][4 * c4 + 3] = k4.w;
                    *(float4*)&S.v[r][4 * c4] = v4;
                }
                __syncthreads();
                if (S.abort) return;
                // scores = dot(q, k) * (1/sqrt(head_dim)) (attention.rs:52-55)
                for (int idx = tid; idx < GQ * TPOS; idx += SNT) {
                    const int i = idx / TPOS, sp = idx % TPOS;
                    float dot = 0.0f;
#pragma unroll 16
                    for (int d = 0; d < HDIM; d++) dot += S.qh[i][d] * S.k[sp][d];
                    S.p[i][sp] = (s0 + sp < P) ? dot * scale : -INFINITY;
                }
                __syncthreads();
                if (wave < GQ) {
                    const float v = S.p[wave][lane];
                    const float m = sq_wave_max(v);
                    const float p = (v == -INFINITY) ? 0.0f : expf(v - m);
                    const float sum = sq_wave_sum(p);
                    S.p[wave][lane] = p;
                    if (lane == 0) {
                        S.m[wave] = m;
                        S.l[wave] = sum;
                    }
                }
                __syncthreads();
                if (wave < GQ) {
                    const int h = g * GQ + wave, d = lane;
                    float o = 0.0f;
#pragma unroll 16
                    for (int sp = 0; sp < TPOS; sp++) o += S.p[wave][sp] * S.v[sp][d];
                    if (nchunks == 1) {
                        quant_put(o / S.l[wave], lane, h * 2, X.a, X.a + QD / 4, T, true);
                    } else {
                        // partial (o[64], m, l) of head h, tile `tile`
                        u64* pt = X.t + ((size_t)h * a.max_tiles + tile) * (HDIM + 2);
                        putf(pt + d, o, T);
                        if (lane == 0) {
                            putf(pt + HDIM, S.m[wave], T);
                            putf(pt + HDIM + 1, S.l[wave], T);
                        }
                    }
                }
                __syncthreads();
            }
            stamp(l, TS_ATTN);
            if (nchunks > 1) {
                // merge the tiles of each head, then quantize the row
                const unsigned Tm = tag(l, PH_MERGE);
                bool ok = true;
                for (int h = gw; h < a.n_heads && ok; h += NW) {
                    const int d = lane;
                    float M = -INFINITY, Lsum = 0.0f, O = 0.0f;
                    for (int t0 = 0; t0 < nchunks && ok; t0 += 2) {
                        u64 wo[2], wm[2], wl[2];
#pragma unroll
                        for (int j = 0; j < 2; j++) {
                            const u64* pt = X.t + ((size_t)h * a.max_tiles + t0 + j) * (HDIM + 2);
                            if (t0 + j < nchunks) {
                                wo[j] = ld_c(pt + d);
                                wm[j] = ld_c(pt + HDIM);
                                wl[j] = ld_c(pt + HDIM + 1);
                            }
                        }
#pragma unroll
                        for (int j = 0; j < 2; j++) {
                            if (t0 + j >= nchunks || !ok) continue;
                            const u64* pt = X.t + ((size_t)h * a.max_tiles + t0 + j) * (HDIM + 2);
                            ok = await_word(pt + d, wo[j], T, C) && await_word(pt + HDIM, wm[j], T, C) &&
                                 await_word(pt + HDIM + 1, wl[j], T, C);
                            if (!ok) continue;
                            const float mt = __builtin_bit_cast(float, (unsigned)wm[j]);
                            if (mt == -INFINITY) continue;
                            const float Mn = fmaxf(M, mt);
                            const float es = (M == -INFINITY) ? 0.0f : expf(M - Mn);
                            const float et = expf(mt - Mn);
                            Lsum = Lsum * es + __builtin_bit_cast(float, (unsigned)wl[j]) * et;
                            O = O * es + __builtin_bit_cast(float, (unsigned)wo[j]) * et;
                            M = Mn;
                        }
                    }
                    // lanes of one wavefront agree on ok (each waits on its own
                    // word; any failure aborts the launch)
                    if (__all(ok)) quant_put(O / Lsum, lane, h * 2, X.a, X.a + QD / 4, Tm, true);
                    else ok = false;
                }
                if (!ok) S.abort = 1;
                __syncthreads();
                if (S.abort) return;
                stamp(l, TS_MERGE);
            }
        }

        // ------------------------------------------------ o-projection + residual
        {
            const unsigned Tin = tag(l, nchunks > 1 ? PH_MERGE : PH_ATTN), T = tag(l, PH_O);
            const bool work = wg * SW < D;
            const int QB = QD >> 5;
            if (work && !gather(S, X.a, QD / 4 + QB, Tin, C)) return;
            stamp(l, TS_O_IN);
            if (work && gw < D) {
                h_own += dot_row_xw<WT, 1>(Wo, S, QB, lane);  // elementwise_add (layers.rs:81-109)
                if (lane == 0) putf(X.h + gw, h_own, T);
            }
            {
                int rr[8];
                gu_rows(wg, rr);
                const MatView mv = view_of(LY[l].gateup);
                load_rows(Wg, mv, rr, lane);
            }
            stamp(l, TS_O);
        }

        // ------------------------------------------------ gate/up + SiLU*up + quant
        {
            const unsigned T = tag(l, PH_GU);
            const bool work = wg < gu_tiles;
            if (work) {
                load_gains(nw, LY[l].ffn_norm, D);
                if (!gather(S, X.h, D, tag(l, PH_O), C)) return;
                x_from_xw(x, S, D);
            }
            stamp(l, TS_GU_IN);
            if (work) {
                norm_quant<WT>(S, x, nw, D, a.eps, nullptr, nullptr, nullptr);
                Act<1> A;
                act_from_lds<WT>(A, S, KB, lane);
                float res[8];
                dot_rows<WT, 1, 8>(Wg, A, KB, lane, res);
                if (lane == 0) {
#pragma unroll
                    for (int r = 0; r < 8; r++) S.gu[wave * 8 + r] = res[r];
                }
            }
            stamp(l, TS_GU_DOT);
            if (work) {
                __syncthreads();
                if (wave == 0) {
                    // layers::ffn (layers.rs:64-77): silu(gate) * up, then the
                    // down projection's Q8_0 quantization per 32-block.
                    const int j = lane & 31;
                    const float gt = S.gu[j];
                    const float up = S.gu[32 + j];
                    const float f = (gt * sq_sigmoid(gt)) * up;
                    quant_put(f, lane, wg, X.f, X.f + F / 4, T, lane < 32);
                }
            }
            {
                const int rr[1] = {gw < D ? gw : -1};
                const MatView mv = view_of(LY[l].down);
                load_rows(Wd, mv, rr, lane);
            }
            stamp(l, TS_GU);
        }

        // ------------------------------------------------ down + residual
        {
            const unsigned T = tag(l, PH_DOWN);
            const bool work = wg * SW < D;
            const int FB = F >> 5;
            if (work && !gather(S, X.f, F / 4 + FB, tag(l, PH_GU), C)) return;
            stamp(l, TS_DOWN_IN);
            if (work && gw < D) {
                h_own += dot_row_xw<WT, 4>(Wd, S, FB, lane);
                if (lane == 0) putf(X.h + gw, h_own, T);
            }
            if (l + 1 < a.n_layers) {
                int rr[2];
                qkv_rows(gw, rr);
                const MatView mn = view_of(LY[l + 1].qkv);
                load_rows(Wq, mn, rr, lane);
            }
            stamp(l, TS_DOWN);
        }
    }

    // ---------------------------------------------------- final norm + LM head
    {
        const int units = (a.vocab + 3) / 4;
        {
            int rr[4];
            head_rows(gw, rr);
            load_rows(Wh0, a.head, rr, lane);
        }
        load_gains(nw, a.out_norm, D);
        if (!gather(S, X.h, D, tag(a.n_layers - 1, PH_DOWN), C)) return;
        x_from_xw(x, S, D);
        stamp(a.n_layers, 0);
        const bool dbg = wg == 0 && a.last_hidden != nullptr;
        norm_quant<WT>(S, x, nw, D, a.eps, dbg ? a.last_hidden : nullptr, a.head_qs, a.head_d);
        Act<1> A;
        act_from_lds<WT>(A, S, KB, lane);
        float best_v = -INFINITY;
        int best_i = -1, nan_i = -1;
        auto compute = [&](const Rows<WT, 1, 4>& Wb, int uu) {
            float res[4];
            dot_rows<WT, 1, 4>(Wb, A, KB, lane, res);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int row = 4 * uu + r;
                if (row >= a.vocab) continue;
                if (lane == r) st_c(&a.logits[row], res[r]);
                const float v = res[r];
                if (v != v) {
                    nan_i = row > nan_i ? row : nan_i;
                } else if (v > best_v || (v == best_v && row > best_i)) {
                    best_v = v;
                    best_i = row;
                }
            }
        };
        int u = gw;
        while (u < units) {
            if (u + NW < units) {
                int rr[4];
                head_rows(u + NW, rr);
                load_rows(Wh1, a.head, rr, lane);
            }
            compute(Wh0, u);
            u += NW;
            if (u >= units) break;
            if (u + NW < units) {
                int rr[4];
                head_rows(u + NW, rr);
                load_rows(Wh0, a.head, rr, lane);
            }
            compute(Wh1, u);
            u += NW;
        }
        block_arg(S, best_v, best_i, nan_i);
        // The logits must be visible before the partial is (the NaN rule may
        // rescan them): wait for this workgroup's stores, then publish.
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (tid == 0) {
            putf(X.p + 3 * wg, best_v, head_tag);
            put(X.p + 3 * wg + 1, (unsigned)best_i, head_tag);
            put(X.p + 3 * wg + 2, (unsigned)nan_i, head_tag);
        }
        stamp(a.n_layers, 1);
    }

    // ---------------------------------------------------- greedy (workgroup 0)
    if (wg != 0) return;
    if (!gather(S, X.p, 3 * G, head_tag, C)) return;
    {
        float bv = -INFINITY;
        int bi = -1, bn = -1;
        for (int k = tid; k < G; k += SNT)
            arg_merge(bv, bi, bn, __builtin_bit_cast(float, S.xw[3 * k]), (int)S.xw[3 * k + 1], (int)S.xw[3 * k + 2]);
        block_arg(S, bv, bi, bn);
        int result = bi;
        if (bn >= 0) {
            // Iterator::max_by hands the lead to the later element whenever a
            // comparison involves NaN: the last maximum after the last NaN, or
            // that NaN when nothing follows it.
            float cv = -INFINITY;
            int ci = -1, cn = -1;
            for (int i = bn + 1 + tid; i < a.vocab; i += SNT) {
                const float v = ld_c(&a.logits[i]);
                if (v == v) arg_merge(cv, ci, cn, v, i, -1);
            }
            block_arg(S, cv, ci, cn);
            result = ci >= 0 ? ci : bn;
        }
        if (tid == 0) {
            *a.token = (uint32_t)result;
            const int h = *a.n_hist;
            a.history[h] = (uint32_t)result;
            *a.n_hist = h + 1;
            *a.pos = pos + 1;
            *a.epoch = head_tag + 1u;
            if (a.trace) {
                const int k = 1 + a.n_layers * TS_PER_LAYER + 2;
                if (k < a.trace_stride) a.trace[k] = wall_clock64();
            }
        }
    }
}

}  // namespace

bool decode_step_fits(int dim, int ffn, int n_heads, int n_kv_heads, int grid) {
    // every phase but the LM head gives each wavefront at most one unit:
    // QKV row pairs and o/down rows per wavefront, gate/up tiles per workgroup
    const int nw = grid * SW;
    const int q_units = (n_heads + n_kv_heads * 2) * HDIM / 2;
    return dim <= DMAX && ffn <= FMAX && dim % 32 == 0 && ffn % 32 == 0 && n_heads * HDIM <= DMAX &&
           n_kv_heads > 0 && n_heads % n_kv_heads == 0 && n_heads / n_kv_heads <= MAXG && q_units <= nw &&
           dim <= nw && ffn / 32 <= grid && 3 * grid <= XMAX;
}

int launch_decode_step(hipStream_t s, int wtype, const StepArgs& a, int grid) {
    if (a.dim > DMAX || a.dim % 32 != 0 || a.ffn % 32 != 0 || a.ffn > FMAX)
        return set_error(SQ_ERR_UNSUPPORTED, "persistent decode step: dim <= 2048, ffn <= 8192, multiples of 32");
    if (a.n_kv_heads <= 0 || a.n_heads % a.n_kv_heads != 0 || a.n_heads / a.n_kv_heads > MAXG)
        return set_error(SQ_ERR_UNSUPPORTED, "persistent decode step: GQA group size must be at most 8");
    if (a.n_heads * HDIM > DMAX)
        return set_error(SQ_ERR_UNSUPPORTED, "persistent decode step: q width must be at most 2048");
    if (!decode_step_fits(a.dim, a.ffn, a.n_heads, a.n_kv_heads, grid))
        return set_error(SQ_ERR_UNSUPPORTED, "persistent decode step: the grid is too small for one unit per "
                                             "wavefront in every phase");
    // One workgroup per CU (the grid is the CU count and a CU holds one of
    // these workgroups), so every workgroup is resident at once; were one
    // not, the bounded waits would end the step with an error, not a hang.
    if (wtype == WT_Q8_0)
        hipLaunchKernelGGL(decode_step_kernel<WT_Q8_0>, dim3(grid), dim3(SNT), 0, s, a);
    else if (wtype == WT_Q4_0)
        hipLaunchKernelGGL(decode_step_kernel<WT_Q4_0>, dim3(grid), dim3(SNT), 0, s, a);
    else
        return set_error(SQ_ERR_UNSUPPORTED, "persistent decode step: Q8_0 and Q4_0 weights only");
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(SQ_ERR_HIP, std::string("decode step launch: ") + hipGetErrorString(e));
    return 0;
}

int decode_step_max_grid(int wtype, int* grid) {
    int dev = 0, cus = 0, per_cu = 0;
    SQ_HIP_CHECK(hipGetDevice(&dev));
    SQ_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    const void* f = wtype == WT_Q4_0 ? (const void*)decode_step_kernel<WT_Q4_0> : (const void*)decode_step_kernel<WT_Q8_0>;
    SQ_HIP_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, f, SNT, 0));
    if (per_cu < 1) return set_error(SQ_ERR_UNSUPPORTED, "persistent decode step does not fit on a CU");
    *grid = cus;
    return 0;
}

size_t exchange_words(int dim, int ffn, int n_heads, int n_kv_heads, int max_tiles, int grid) {
    const size_t QD = (size_t)n_heads * HDIM, KVD = (size_t)n_kv_heads * HDIM;
    return dim + QD + 2 * KVD + (QD / 4 + QD / 32) + ((size_t)ffn / 4 + ffn / 32) + 3 * (size_t)grid +
           (size_t)n_heads * max_tiles * (HDIM + 2);
}

}  // namespace sq
