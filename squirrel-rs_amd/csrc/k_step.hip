// Persistent decode step: one launch computes a whole token.
//
// The decode step is a chain of dependent matvecs (per layer: QKV, attention,
// o-projection, gate/up, down; then the LM head).  One workgroup per CU stays
// resident for the whole token; the chain's links are data dependencies
// between workgroups, resolved through memory.
//
// Weight stream.  At context set-up every weight row is copied, once, into a
// per-CU stream: CU `wg` finds the rows it will multiply, in the order it
// will multiply them (per layer: QKV rows, o rows, gate/up rows, down rows;
// then its LM-head rows), as one contiguous range of HBM.  A row of k
// elements is its block payloads (k bytes Q8_0, k/2 bytes Q4_0) followed by
// its fp16 block scales (k/16 bytes), counted in 16-byte units.  A Q8_0 row
// holds the first 16 bytes of every block, then the second 16 bytes of every
// block, so that the lanes of a wavefront (lane = block) read consecutive
// units.
//
// Roles inside a workgroup (6 wavefronts):
// * Two loader wavefronts copy the CU's stream into a 96 KB LDS ring with
//   direct global->LDS loads (global_load_lds_dwordx4: 1 KB per instruction,
//   no registers held), as far ahead of the computation as the ring allows.
//   The HBM stream so runs continuously, independent of the dependency chain.
// * Four compute wavefronts never load weights from HBM.  A wavefront's loads
//   complete in issue order, so a poll queued behind a weight load would wait
//   for it; keeping the weights off the compute wavefronts keeps every poll
//   short.  They poll the phase inputs, normalize/quantize, read their rows
//   from the ring and publish the outputs.
// The groups synchronize through LDS counters (units filled by the loaders,
// units consumed by each compute wavefront); the compute group synchronizes
// among itself through an LDS arrival counter, so no loader ever waits on a
// workgroup barrier.
//
// Exchange words.  Every value handed from one phase to the next (hidden
// row, q row, the new K/V row, quantized activations, argmax partials) is a
// 64-bit word: payload in the low half, the producing phase's tag in the high
// half, written with an agent-scope atomic store (coherent across the XCDs'
// L2s, single-copy atomic).  A consumer polls the words it needs with
// agent-scope loads until each carries the expected tag.  Tags are
// `epoch + phase` and grow across launches (the epoch word advances with every
// launch), so a word from an earlier phase or launch never matches.  A
// workgroup reads a phase's inputs only when it has work in that phase; the
// dependency chain then guarantees no input is overwritten before every
// workgroup that needs it has read it.  The residual stream stays in
// registers: the compute wavefront that owns a hidden row adds the o and down
// outputs of that row to it.
//
// Every wait is bounded by a wall-clock limit and a poll count: on expiry the
// workgroup raises the launch's error word; every waiting wavefront sees it
// (or its workgroup's abort flag) and leaves, so the grid always drains.
//
// Arithmetic per phase is that of the multi-kernel path (k_gemv.hip,
// k_attn.hip): the reference's integer block dot (dot_prod.rs:378-403), its
// RMSNorm (rms_norm.rs:40-56), Q8_0 activation quantizer (dot_prod.rs:21-31),
// interleaved RoPE (rope.rs:7-36), SDPA (attention.rs:11-70), SiLU
// (silu.rs, sigmoid.rs) and greedy tie rule (greedy.rs:6-15).
#include <type_traits>

#include "launch.h"

namespace sq {

namespace {

constexpr int NCW = 4;             // compute wavefronts
constexpr int NLW = 2;             // loader wavefronts
constexpr int SW = NCW + NLW;      // wavefronts per workgroup
constexpr int SNT = SW * 64;       // threads per workgroup
constexpr int CNT = NCW * 64;      // compute threads
constexpr int RU = 9216;           // ring size in 16-byte units (144 KB), a multiple of 64
constexpr int LBATCH = 16;         // 1 KB direct-to-LDS instructions per loader batch (two in flight)
constexpr int HDIM = 64;           // head_dim
constexpr int TPOS = 64;           // attention positions per tile
constexpr int DMAX = 2048;         // model width supported (one 32-block per lane)
constexpr int FMAX = 8192;         // FFN width supported
constexpr int MAXG = 4;            // GQA group size supported (one compute wavefront per head)
constexpr int RMAX = 2;            // residual rows a compute wavefront owns
// eighths of a wavefront's LM-head rows that come through the ring (the
// rest the compute wavefronts load themselves; Q4_0 rows, half the bytes,
// measured slower that way and all come through the ring)
constexpr int head_ring_8ths(int wt) { return wt == WT_Q8_0 ? 4 : 8; }
constexpr int XMAX = FMAX / 4 + FMAX / 32;  // exchange words gathered at once
constexpr int WPT = (XMAX + CNT - 1) / CNT;  // ... per compute thread
// during attention xw holds each wavefront's new K row and the tile slots' partials
static_assert(NCW * HDIM + NCW * MAXG * (HDIM + 2) <= XMAX, "attention scratch exceeds xw");

typedef float sq_v4f __attribute__((ext_vector_type(4)));
typedef unsigned long long u64;

// ---- the per-CU weight stream ---------------------------------------------------
struct StreamGeo {
    int nq, no, ng, nd, nh;    // rows per phase: QKV, o, gate/up, down, LM head
    int ua, uo, ud;            // units per row at k = dim, q_dim, ffn
    int offo, offg, offd, LU;  // unit offsets of o, gate/up, down in a layer; units per layer
    int total;                 // units in this CU's stream
    int row0q, row0o, row0h;   // first row of this CU in QKV, o/down, LM head
    int tile;                  // gate/up tile: gate rows tile*32.., up rows ffn + tile*32..
};

__host__ __device__ inline int stream_row_units(int wt, int k) { return (wt == WT_Q8_0 ? k / 16 : k / 32) + k / 256; }

// QKV: nq consecutive rows of the stacked q|k|v matrix (whole RoPE pairs).
// o and down: the same no rows (the hidden rows this CU owns).  Gate/up: the
// 32 gate and 32 up rows of one 32-wide FFN tile (CUs below ffn/32).  Head:
// nh consecutive vocabulary rows.  Rows past a matrix's end repeat row 0.
__host__ __device__ inline StreamGeo stream_geo(int wt, int L, int D, int F, int QD, int KVD, int vocab, int G,
                                                int wg) {
    StreamGeo g;
    const int q_units = (QD + 2 * KVD) / 2;
    g.nq = 2 * ((q_units + G - 1) / G);
    g.no = (D + G - 1) / G;
    g.ng = wg < F / 32 ? 64 : 0;
    g.nd = g.no;
    g.nh = (vocab + G - 1) / G;
    g.ua = stream_row_units(wt, D);
    g.uo = stream_row_units(wt, QD);
    g.ud = stream_row_units(wt, F);
    g.offo = g.nq * g.ua;
    g.offg = g.offo + g.no * g.uo;
    g.offd = g.offg + g.ng * g.ua;
    g.LU = g.offd + g.nd * g.ud;
    g.total = L * g.LU + g.nh * g.ua;
    g.row0q = wg * g.nq;
    g.row0o = wg * g.no;
    g.row0h = wg * g.nh;
    g.tile = wg;
    return g;
}

// ---- address spaces ------------------------------------------------------------
// Pointers read from memory (the per-layer views) are generic to the
// compiler, which would access them with flat instructions (flat loads also
// count against lgkmcnt).  All device-memory accesses go through these casts.
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
// read with scalar loads.
template <typename T>
using cptr = const __attribute__((address_space(4))) T*;

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

// ---- wavefront sum without LDS ------------------------------------------------
// DPP butterfly: quad swaps, half-row and row mirrors leave every lane of a
// 16-lane row with the row's sum; two row broadcasts accumulate the rows into
// lane 63, which is read back as a wave-uniform value.  (The shuffle-based
// sum would go through the LDS crossbar, which the ring keeps busy.)
template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp_mov(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROWS, 0xF, false));
}
__device__ __forceinline__ float wave_total(float v) {
    v += dpp_mov<0xB1, 0xF>(v);   // quad_perm [1,0,3,2]
    v += dpp_mov<0x4E, 0xF>(v);   // quad_perm [2,3,0,1]
    v += dpp_mov<0x141, 0xF>(v);  // row_half_mirror
    v += dpp_mov<0x140, 0xF>(v);  // row_mirror
    v += dpp_mov<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
    v += dpp_mov<0x143, 0xC>(v);  // row_bcast:31 into rows 2 and 3
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
// The same butterfly with fmaxf.
__device__ __forceinline__ float wave_maximum(float v) {
    v = fmaxf(v, dpp_mov<0xB1, 0xF>(v));
    v = fmaxf(v, dpp_mov<0x4E, 0xF>(v));
    v = fmaxf(v, dpp_mov<0x141, 0xF>(v));
    v = fmaxf(v, dpp_mov<0x140, 0xF>(v));
    const float b15 = __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, v), __builtin_bit_cast(int, v), 0x142, 0xA, 0xF, false));
    v = fmaxf(v, b15);
    const float b31 = __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, v), __builtin_bit_cast(int, v), 0x143, 0xC, 0xF, false));
    v = fmaxf(v, b31);
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
__device__ __forceinline__ float lane_value(float v, int lane_index) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane_index));
}

// ---- shared state ---------------------------------------------------------------
struct StepShared {
    alignas(16) uint8_t ring[RU * 16];   // weight ring (loaders write, compute reads)
    alignas(16) unsigned xw[XMAX];       // gathered exchange payloads
    alignas(16) int aq[DMAX / 4];        // normalized activation as Q8_0: payload (32 int8 per block)
    float as[DMAX / 32];                 // ... block scales (f32 of the fp16 scale)
    int asum[DMAX / 32];                 // ... sums of each block's payload (Q4_0 offset term)
    float ssum[NCW];                     // per-wavefront partial sums of squares
    float gu[64];                        // gate/up outputs of the workgroup's tile
    float bv[NCW];
    int bi[NCW];
    int bn[NCW];
    int done[NLW];  // per loader: its next instruction (all its earlier ones are in LDS)
    int cons[NCW];  // per compute wavefront: stream units consumed (its entries ending at or below)
    int csync;      // compute-group arrival counter
    int abort;
};

template <typename T>
__device__ __forceinline__ T lds_ld(const T* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
template <typename T>
__device__ __forceinline__ void lds_st(T* p, T v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
template <typename T>
__device__ __forceinline__ void lds_release(T* p, T v) {
    __hip_atomic_store(p, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// ---- bounded waiting ------------------------------------------------------------
struct Ctl {
    int* error;
    long long limit;  // wall-clock ticks one wait may take
};

// Poll exchange words p[0..N) (null: no word) until each carries `tag`.
// Every round re-requests all words still stale at once, so a round costs one
// memory round trip however many words are pending.  False on timeout, a
// raised error or the workgroup's abort flag.
template <int N>
__device__ __forceinline__ bool await_words(const u64* const (&p)[N], u64 (&w)[N], unsigned tag, const Ctl& C,
                                            const int* abort) {
    auto pending = [&]() {
        bool any = false;
#pragma unroll
        for (int j = 0; j < N; j++) any |= p[j] != nullptr && (unsigned)(w[j] >> 32) != tag;
        return any;
    };
    if (!pending()) return true;
    // The wall clock is first read at the first periodic check: reading it
    // is a scalar-memory access whose latency would delay the first polls.
    long long t0 = 0;
    for (int polls = 1;; polls++) {
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int j = 0; j < N; j++)
            if (p[j] != nullptr && (unsigned)(w[j] >> 32) != tag) w[j] = ld_c(p[j]);
        if (!pending()) return true;
        if ((polls & 15) == 0) {
            if (ld_c(C.error) != 0 || lds_ld(abort)) return false;
            const long long now = wall_clock64();
            if (polls == 16) t0 = now;
            if (now - t0 > C.limit || polls > (1 << 20)) {
                st_c(C.error, 1);
                return false;
            }
        }
    }
}

// await_words with the addresses formed by addr(j) (null: no word) at each
// use instead of held in registers.
template <int N, typename A>
__device__ __forceinline__ bool await_words_at(A&& addr, u64 (&w)[N], unsigned tag, const Ctl& C, const int* abort) {
    auto pending = [&]() {
        bool any = false;
#pragma unroll
        for (int j = 0; j < N; j++) any |= addr(j) != nullptr && (unsigned)(w[j] >> 32) != tag;
        return any;
    };
    if (!pending()) return true;
    long long t0 = 0;  // read at the first periodic check (see await_words)
    for (int polls = 1;; polls++) {
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int j = 0; j < N; j++) {
            const u64* p = addr(j);
            if (p != nullptr && (unsigned)(w[j] >> 32) != tag) w[j] = ld_c(p);
        }
        if (!pending()) return true;
        if ((polls & 15) == 0) {
            if (ld_c(C.error) != 0 || lds_ld(abort)) return false;
            const long long now = wall_clock64();
            if (polls == 16) t0 = now;
            if (now - t0 > C.limit || polls > (1 << 20)) {
                st_c(C.error, 1);
                return false;
            }
        }
    }
}

// Spin until an LDS condition holds (bounded), then acquire.  False: abandon
// the launch.
template <typename F>
__device__ __forceinline__ bool spin_lds(F&& ready, StepShared& S, const Ctl& C) {
    bool ok = true;
    if (!ready()) {
        long long t0 = 0;  // read at the first periodic check (see await_words)
        for (int polls = 1;; polls++) {
            __builtin_amdgcn_s_sleep(1);
            if (ready()) break;
            if ((polls & 63) == 0) {
                if (lds_ld(&S.abort) || ld_c(C.error) != 0) {
                    ok = false;
                    break;
                }
                const long long now = wall_clock64();
                if (polls == 64) t0 = now;
                if (now - t0 > C.limit || polls > (1 << 24)) {
                    st_c(C.error, 1);
                    ok = false;
                    break;
                }
            }
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    return ok;
}

// Compute-group barrier (the loaders take no part).  gen counts this
// wavefront's arrivals.
__device__ __forceinline__ bool csync(StepShared& S, int& gen, const Ctl& C) {
    gen++;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    if ((threadIdx.x & 63) == 0) __hip_atomic_fetch_add(&S.csync, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    const int target = NCW * gen;
    const bool ok = spin_lds([&] { return lds_ld(&S.csync) >= target; }, S, C);
    if (!ok) lds_st(&S.abort, 1);
    return ok && !lds_ld(&S.abort);
}

// The compute group gathers words src[0..n) once they carry `tag`; payloads
// land in xw.  False: abandon.
__device__ __forceinline__ bool gather(StepShared& S, unsigned* xw, const u64* src, int n, unsigned tag, const Ctl& C,
                                       int& gen) {
    // t is made opaque here so that the addresses below are formed in place:
    // hoisted out of the layer loop they would stay live (and spill)
    int t = threadIdx.x;  // < CNT
    asm volatile("" : "+v"(t));
    const u64* p[WPT];
    u64 w[WPT];
#pragma unroll
    for (int j = 0; j < WPT; j++) {
        const int i = t + j * CNT;
        p[j] = i < n ? src + i : nullptr;
        w[j] = i < n ? ld_c(src + i) : 0;
    }
    if (!await_words(p, w, tag, C, &S.abort)) lds_st(&S.abort, 1);
#pragma unroll
    for (int j = 0; j < WPT; j++) {
        const int i = t + j * CNT;
        if (i < n) xw[i] = (unsigned)w[j];
    }
    return csync(S, gen, C);
}

// ---- reading rows from the ring ----------------------------------------------------
// Ring position of the unit k units past ring position rb (rb < RU, k < RU):
// one subtraction and an unsigned min wrap it.
__device__ __forceinline__ unsigned ring_wrap(unsigned o) { return min(o, o - (unsigned)RU); }

// Q8_0 activation block of one lane: payload q[8] (32 int8), scale s, and the
// sum of the payload (Q4_0 offset term).
struct ActQ {
    int q[8];
    float s;
    int sum;
};

// One lane's block of one row, as read from the ring: payload (two 16-byte
// units Q8_0, one Q4_0) and the fp16 scale.
struct RowData {
    uint4 w0, w1;
    uint16_t d;
};

// Reads block `blk` of the row whose first unit sits at ring position rb (P
// payload units).  Reads only: the batch's reads are all issued before any of
// its arithmetic.
template <int WT>
__device__ __forceinline__ RowData row_fetch(const StepShared& S, unsigned rb, int P, int blk) {
    RowData r;
    if constexpr (WT == WT_Q8_0) {
        // first halves of the row's blocks, then second halves: lanes read
        // consecutive units, conflict-free across the LDS banks
        r.w0 = *(const uint4*)(S.ring + ring_wrap(rb + blk) * 16);
        r.w1 = *(const uint4*)(S.ring + ring_wrap(rb + (P >> 1) + blk) * 16);
    } else {
        r.w0 = *(const uint4*)(S.ring + ring_wrap(rb + blk) * 16);
        r.w1 = r.w0;
    }
    r.d = *(const uint16_t*)(S.ring + ring_wrap(rb + P + (blk >> 3)) * 16 + (blk & 7) * 2);
    return r;
}

// The block's term (f32(isum) * sa) * sw (dot_prod.rs:378-403); zero where
// `valid` is false (a lane past the row's blocks reads unrelated ring bytes).
template <int WT>
__device__ __forceinline__ float row_math(const RowData& r, const ActQ& A, bool valid) {
    int isum = 0;
    if constexpr (WT == WT_Q8_0) {
        isum = __builtin_amdgcn_sdot4(A.q[0], (int)r.w0.x, isum, false);
        isum = __builtin_amdgcn_sdot4(A.q[1], (int)r.w0.y, isum, false);
        isum = __builtin_amdgcn_sdot4(A.q[2], (int)r.w0.z, isum, false);
        isum = __builtin_amdgcn_sdot4(A.q[3], (int)r.w0.w, isum, false);
        isum = __builtin_amdgcn_sdot4(A.q[4], (int)r.w1.x, isum, false);
        isum = __builtin_amdgcn_sdot4(A.q[5], (int)r.w1.y, isum, false);
        isum = __builtin_amdgcn_sdot4(A.q[6], (int)r.w1.z, isum, false);
        isum = __builtin_amdgcn_sdot4(A.q[7], (int)r.w1.w, isum, false);
    } else {
        const int dw[4] = {(int)r.w0.x, (int)r.w0.y, (int)r.w0.z, (int)r.w0.w};
#pragma unroll
        for (int v = 0; v < 4; v++) {
            isum = __builtin_amdgcn_sdot4(A.q[v], dw[v] & 0x0F0F0F0F, isum, false);
            isum = __builtin_amdgcn_sdot4(A.q[4 + v], (dw[v] >> 4) & 0x0F0F0F0F, isum, false);
        }
        isum -= 8 * A.sum;
    }
    const float t = sq_q_term(isum, A.s, sq_f16_to_f32(r.d));
    return valid ? t : 0.0f;
}

// wave_total of R values, stage by stage, so the DPP latencies overlap.
template <int R>
__device__ __forceinline__ void wave_totals(float (&v)[R]) {
#pragma unroll
    for (int r = 0; r < R; r++) v[r] += dpp_mov<0xB1, 0xF>(v[r]);
#pragma unroll
    for (int r = 0; r < R; r++) v[r] += dpp_mov<0x4E, 0xF>(v[r]);
#pragma unroll
    for (int r = 0; r < R; r++) v[r] += dpp_mov<0x141, 0xF>(v[r]);
#pragma unroll
    for (int r = 0; r < R; r++) v[r] += dpp_mov<0x140, 0xF>(v[r]);
#pragma unroll
    for (int r = 0; r < R; r++) v[r] += dpp_mov<0x142, 0xA>(v[r]);
#pragma unroll
    for (int r = 0; r < R; r++) v[r] += dpp_mov<0x143, 0xC>(v[r]);
#pragma unroll
    for (int r = 0; r < R; r++) v[r] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v[r]), 63));
}

// ---- the loaders ----------------------------------------------------------------
// Loader k issues the 64-unit instructions j = k, k + NLW, ... of the stream
// [0, total): instruction j fills ring units (64 j mod RU) .. +63 (RU is a
// multiple of 64, so an instruction never wraps).  An instruction may be
// issued once every unit it overwrites is consumed: its last unit lies within
// RU units of the consumed boundary (the least of the compute wavefronts'
// counters).  A batch is LBATCH of the loader's next instructions; while the
// ring has room, a loader keeps two batches in flight and publishes S.done[k]
// as each lands; when it has not, the loader issues as many instructions as
// fit and waits for them.
//
// Progress: a compute wavefront waits for a batch of up to R of its rows
// (rows are dealt round-robin, stride NCW).  When every wavefront waits on
// the ring, the wavefront with the lowest next row has a batch ending at most
// NCW * R rows (or all the phase's rows) past the consumed boundary, so its
// last instruction is issuable
// whenever those rows plus one instruction fit in the ring (R = 4 rows of
// width dim, 2 rows of width q_dim or ffn, 2 QKV row pairs); ring_fits checks
// that.
// The least of the compute wavefronts' consumed counters, read by a loader.
// The reads are one inline-assembly block (reads, then the wait for them):
// for an ordinary LDS read the compiler would first wait for every
// direct-to-LDS load still in flight (they write LDS), which would serialize
// the loader's batches.  The outputs are early-clobber and only used after the
// block, so no result is read before its load has returned.
static_assert(NCW == 4, "min_consumed reads four counters");
__device__ __forceinline__ int min_consumed(const StepShared& S) {
    unsigned addr[NCW];
#pragma unroll
    for (int w = 0; w < NCW; w++) addr[w] = (unsigned)(size_t)(const __attribute__((address_space(3))) int*)&S.cons[w];
    int c0, c1, c2, c3;
    asm volatile(
        "ds_read_b32 %0, %4\n\t"
        "ds_read_b32 %1, %5\n\t"
        "ds_read_b32 %2, %6\n\t"
        "ds_read_b32 %3, %7\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(c0), "=&v"(c1), "=&v"(c2), "=&v"(c3)
        : "v"(addr[0]), "v"(addr[1]), "v"(addr[2]), "v"(addr[3])
        : "memory");
    return __builtin_amdgcn_readfirstlane(min(min(c0, c1), min(c2, c3)));
}

// A loader's store of its done counter, as inline assembly: as an atomic
// release store the compiler would first wait for every direct-to-LDS load in
// flight, including the batch just issued.  The caller waits (s_waitcnt) for
// the loads the counter covers.
__device__ __forceinline__ void publish_done(StepShared& S, int k, int v) {
    const unsigned addr = (unsigned)(size_t)(__attribute__((address_space(3))) int*)&S.done[k];
    asm volatile("ds_write_b32 %0, %1" ::"v"(addr), "v"(v) : "memory");
}

// s_waitcnt immediate that waits until at most n vector-memory operations
// are outstanding (lgkm and exp counters untouched).
constexpr int vmcnt_imm(int n) { return (n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8); }

__device__ __forceinline__ void run_loader(StepShared& S, gptr<const uint8_t> stream, int total, int k, const Ctl& C) {
    const int lane = threadIdx.x & 63;
    const int n_instr = (total + 63) / 64;
    auto issue = [&](int j0, int j1) {
        for (int jj = j0; jj <= j1; jj += NLW) {
            const int u = jj * 64 + lane;
            if (u < total)
                __builtin_amdgcn_global_load_lds((__attribute__((address_space(1))) void*)(stream + (size_t)u * 16),
                                                 (__attribute__((address_space(3))) void*)(S.ring + ((jj * 64) % RU) * 16),
                                                 16, 0, 0);
        }
    };
    if (k < n_instr) {
        const int last = n_instr - 1 - ((n_instr - 1 - k) % NLW);  // this loader's last instruction
        int j = k;
        int pend = -1;  // done value of the batch in flight (-1: none)
        while (j <= last) {
            // A full batch (LBATCH instructions) that fits behind the consumed
            // boundary is issued while the previous one is still in flight;
            // once it is issued, at most LBATCH instructions are outstanding
            // when the previous batch has landed.
            const int j_full = j + NLW * (LBATCH - 1);
            if (j_full <= last && (j_full + 1) * 64 <= min_consumed(S) + RU) {
                issue(j, j_full);
                if (pend >= 0) {
                    __builtin_amdgcn_s_waitcnt(vmcnt_imm(LBATCH));
                    publish_done(S, k, pend);
                }
                pend = j = j_full + NLW;
                continue;
            }
            if (pend >= 0) {  // land what is in flight first
                __builtin_amdgcn_s_waitcnt(0);
                lds_release(&S.done[k], pend);
                pend = -1;
                continue;
            }
            // a partial batch: at least instruction j must be issuable; mc is
            // the counter value that allowed it, so allowed >= j below
            int mc = 0;
            const bool ok = spin_lds(
                [&] {
                    mc = min_consumed(S);
                    return (j + 1) * 64 <= mc + RU;
                },
                S, C);
            if (!ok) {
                lds_st(&S.abort, 1);
                return;
            }
            const int allowed = (mc + RU) / 64 - 1;  // last issuable instruction
            int j_last = min(j_full, last);
            if (j_last > allowed) j_last = allowed - (allowed - j) % NLW;
            j_last = max(j_last, j);  // j itself is issuable: every pass advances j
            // a batch that is full after all goes through the pipelined path
            if (j_last == j_full) continue;
            issue(j, j_last);
            __builtin_amdgcn_s_waitcnt(0);
            j = j_last + NLW;
            lds_release(&S.done[k], j);
        }
        if (pend >= 0) {
            __builtin_amdgcn_s_waitcnt(0);
            lds_release(&S.done[k], pend);
        }
    }
    lds_release(&S.done[k], n_instr + NLW);
}

// Units of the stream in the ring from the start (all instructions below the
// least of the loaders' next instructions).
__device__ __forceinline__ int filled_units(const StepShared& S) {
    int d = lds_ld(&S.done[0]);
#pragma unroll
    for (int k = 1; k < NLW; k++) d = min(d, lds_ld(&S.done[k]));
    return d * 64;
}

// ---- activations --------------------------------------------------------------
// Norm gains of the 8 row elements a compute thread normalizes (elements
// 8t .. 8t+7), requested before the phase's input gather so that both arrive
// together.
struct Gains {
    sq_v4f v[2];
};
__device__ __forceinline__ Gains load_gains(const float* w, int D) {
    const int t = threadIdx.x;  // < CNT
    const gptr<const sq_v4f> wp = (gptr<const sq_v4f>)(gl(w) + (t < D / 8 ? t * 8 : 0));
    Gains G;
    G.v[0] = wp[0];
    G.v[1] = wp[1];
    return G;
}

template <int CTRL>
__device__ __forceinline__ int dpp_int(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}

// RMSNorm (rms_norm.rs:40-56) of the hidden row and its Q8_0 quantization
// (dot_prod.rs:21-31), spread over the compute group: thread t owns elements
// 8t .. 8t+7 of the row.  They come from the exchange words src[hslot(8t + e)]
// once these carry `tag` (or, with src null, from the token's embedding row).  The
// sum of squares is reduced per wavefront, then across the wavefronts in a
// fixed order after a compute-group barrier; the four threads of a 32-block
// (a lane quad) agree on its scale through DPP and the blocks land in
// S.aq / S.as / S.asum (and, when non-null, the f32 row in dbg_y and the
// blocks in dbg_q / dbg_d).  Ends with a compute-group barrier; false:
// abandon.
template <typename Embed>
__device__ __forceinline__ bool norm_quant(StepShared& S, const u64* src, unsigned tag, Embed&& embed, const Gains& G,
                                           int D, float eps, float* dbg_y, int8_t* dbg_q, uint16_t* dbg_d, int& gen,
                                           const Ctl& C) {
    int t = threadIdx.x;
    asm volatile("" : "+v"(t));  // addresses formed in place (see gather)
    const int lane = t & 63, cw = t >> 6;
    const int KB = D >> 5;
    const bool mine = t < 4 * KB;
    float xs[8];
    if (src != nullptr) {
            const u64* p[8];
        u64 w[8];
#pragma unroll
        for (int e = 0; e < 8; e++) {
            p[e] = mine ? src + e * (D >> 3) + t : nullptr;  // element 8t + e (hslot)
            w[e] = mine ? ld_c(src + e * (D >> 3) + t) : 0;
        }
        if (!await_words(p, w, tag, C, &S.abort)) lds_st(&S.abort, 1);
#pragma unroll
        for (int e = 0; e < 8; e++) xs[e] = __builtin_bit_cast(float, (unsigned)w[e]);
    } else {
#pragma unroll
        for (int e = 0; e < 8; e++) xs[e] = mine ? embed(8 * t + e) : 0.0f;
    }
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; e++) ss += mine ? xs[e] * xs[e] : 0.0f;
    ss = wave_total(ss);
    if (lane == 0) S.ssum[cw] = ss;
    if (!csync(S, gen, C)) return false;
    float tot = 0.0f;
#pragma unroll
    for (int w = 0; w < NCW; w++) tot += S.ssum[w];
    const float rms = sqrtf(tot / (float)D + eps);
    if (mine) {
        const float gs[8] = {G.v[0].x, G.v[0].y, G.v[0].z, G.v[0].w, G.v[1].x, G.v[1].y, G.v[1].z, G.v[1].w};
        float y[8];
        float amax = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            y[e] = (xs[e] * gs[e]) / rms;
            amax = fmaxf(amax, fabsf(y[e]));
        }
        // the block's amax over its lane quad
        amax = fmaxf(amax, __builtin_bit_cast(float, dpp_int<0xB1>(__builtin_bit_cast(int, amax))));
        amax = fmaxf(amax, __builtin_bit_cast(float, dpp_int<0x4E>(__builtin_bit_cast(int, amax))));
        const float sc = sq_q8_scale(amax);
        const float inv = sq_q8_inv(sc);
        int packed[2] = {0, 0};
        int qsum = 0;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const int qv = sq_q8_quant(y[e], inv);
            qsum += qv;
            packed[e >> 2] |= (qv & 0xFF) << (8 * (e & 3));
        }
        qsum += dpp_int<0xB1>(qsum);
        qsum += dpp_int<0x4E>(qsum);
        const int blk = t >> 2;
        *(int2*)&S.aq[2 * t] = make_int2(packed[0], packed[1]);
        const uint16_t d16 = sq_f32_to_f16(sc);
        if ((t & 3) == 0) {
            S.as[blk] = sq_f16_to_f32(d16);
            S.asum[blk] = qsum;
        }
        if (dbg_y) {
#pragma unroll
            for (int e = 0; e < 8; e++) dbg_y[8 * t + e] = y[e];
        }
        if (dbg_q) {
            *(int2*)(dbg_q + 8 * t) = make_int2(packed[0], packed[1]);
            if ((t & 3) == 0) dbg_d[blk] = d16;
        }
    }
    return csync(S, gen, C);
}

// Word of the hidden-row exchange X.h that holds element `row`: element
// 8t + e sits at e * (D / 8) + t, so that compute thread t's eight words
// (norm_quant) are e * (D / 8) + t for e < 8 -- one coalesced 512-byte run
// per wavefront and load instead of eight scattered 64-byte pieces.
__device__ __forceinline__ int hslot(int row, int D) { return (row & 7) * (D >> 3) + (row >> 3); }

// The lane's activation block (block = lane) after norm_quant.
__device__ __forceinline__ ActQ act_lane(const StepShared& S, int D) {
    const int lane = threadIdx.x & 63;
    const bool v = lane < (D >> 5);
    const int b = v ? lane : 0;
    const uint4* p = (const uint4*)&S.aq[8 * b];
    const uint4 a0 = p[0], a1 = p[1];
    ActQ A;
    A.q[0] = v ? (int)a0.x : 0;
    A.q[1] = v ? (int)a0.y : 0;
    A.q[2] = v ? (int)a0.z : 0;
    A.q[3] = v ? (int)a0.w : 0;
    A.q[4] = v ? (int)a1.x : 0;
    A.q[5] = v ? (int)a1.y : 0;
    A.q[6] = v ? (int)a1.z : 0;
    A.q[7] = v ? (int)a1.w : 0;
    A.s = v ? S.as[b] : 0.0f;
    A.sum = v ? S.asum[b] : 0;
    return A;
}

// Activation block `blk` of gathered exchange payloads (nblk blocks of 8
// payload words, then nblk scale words); zero past nblk.
template <int WT>
__device__ __forceinline__ ActQ xw_block(const unsigned* xw, int nblk, int blk) {
    const bool v = blk < nblk;
    const int b = v ? blk : 0;
    const uint4* pq = (const uint4*)(xw + b * 8);
    const uint4 a0 = pq[0], a1 = pq[1];
    ActQ A;
    A.q[0] = v ? (int)a0.x : 0;
    A.q[1] = v ? (int)a0.y : 0;
    A.q[2] = v ? (int)a0.z : 0;
    A.q[3] = v ? (int)a0.w : 0;
    A.q[4] = v ? (int)a1.x : 0;
    A.q[5] = v ? (int)a1.y : 0;
    A.q[6] = v ? (int)a1.z : 0;
    A.q[7] = v ? (int)a1.w : 0;
    A.s = v ? __builtin_bit_cast(float, xw[nblk * 8 + b]) : 0.0f;
    A.sum = 0;
    if constexpr (WT == WT_Q4_0) {
#pragma unroll
        for (int k = 0; k < 8; k++) A.sum = __builtin_amdgcn_sdot4(A.q[k], 0x01010101, A.sum, false);
    }
    return A;
}

// Quantize 32-element blocks held one element per lane (lanes 0..31 and
// 32..63 are two blocks) and publish them: payload words q[blk*8 + j] and
// scale words s[blk] (f32 of the fp16 scale), blk = block0 + (lane >> 5).
// Lanes with `valid` false hold no element (their half is not published).
// The block maxima and the byte packing move values between lanes with DPP
// and lane reads only: LDS permutes would queue behind the ring traffic.
// When tq is non-null the blocks also go to the activation taps: payload
// word i to tq[i], the fp16 scale of block b to td[b].
__device__ __forceinline__ void quant_put(float v, int lane, int block0, u64* q, u64* s, unsigned tag, bool valid,
                                          int* tq = nullptr, uint16_t* td = nullptr) {
    float m = fabsf(valid ? v : 0.0f);
    m = fmaxf(m, dpp_mov<0xB1, 0xF>(m));   // quad_perm [1,0,3,2]
    m = fmaxf(m, dpp_mov<0x4E, 0xF>(m));   // quad_perm [2,3,0,1]
    m = fmaxf(m, dpp_mov<0x141, 0xF>(m));  // row_half_mirror
    m = fmaxf(m, dpp_mov<0x140, 0xF>(m));  // row_mirror: every lane holds its row's maximum
    // row_bcast:15 into rows 1 and 3 (rows 0 and 2 keep theirs): lanes 31
    // and 63 hold the maxima of lanes 0..31 and 32..63
    m = fmaxf(m, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, m),
                                                                      __builtin_bit_cast(int, m), 0x142, 0xA, 0xF,
                                                                      false)));
    const float lo = lane_value(m, 31), hi = lane_value(m, 63);
    const float amax = fmaxf(lane < 32 ? lo : hi, 0.0f);
    const float sc = sq_q8_scale(amax);
    const int qv = valid ? ((int)sq_q8_quant(v, sq_q8_inv(sc)) & 0xFF) : 0;
    // bytes of lanes 4k+1, 4k+2, 4k+3 to lane 4k: quad_perm [1,1,1,1], [2,2,2,2], [3,3,3,3]
    const int b1 = dpp_int<0x55>(qv), b2 = dpp_int<0xAA>(qv), b3 = dpp_int<0xFF>(qv);
    const int blk = block0 + (lane >> 5);
    const unsigned word = (unsigned)(qv | (b1 << 8) | (b2 << 16) | (b3 << 24));
    const uint16_t d16 = sq_f32_to_f16(sc);
    if ((lane & 3) == 0 && valid) {
        put(q + (size_t)blk * 8 + ((lane & 31) >> 2), word, tag);
        if (tq) gl(tq)[(size_t)blk * 8 + ((lane & 31) >> 2)] = (int)word;
    }
    if ((lane & 31) == 0 && valid) {
        putf(s + blk, sq_f16_to_f32(d16), tag);
        if (tq) gl(td)[blk] = d16;
    }
}

__device__ __forceinline__ void arg_merge(float& bv, int& bi, int& bn, float v, int i, int n) {
    if (i >= 0 && (bi < 0 || v > bv || (v == bv && i > bi))) {
        bv = v;
        bi = i;
    }
    bn = n > bn ? n : bn;
}

// (value, index, NaN index) over the wavefront, in every lane.  arg_merge is
// the maximum under a total order, so the merge order is free: the DPP
// butterfly of wave_total, where lanes a step does not write keep their own
// triple (merging a triple with itself leaves it unchanged).
template <int CTRL, int ROWS>
__device__ __forceinline__ int dpp_keep(int v) {
    return __builtin_amdgcn_update_dpp(v, v, CTRL, ROWS, 0xF, false);
}
template <int CTRL, int ROWS>
__device__ __forceinline__ void arg_step(float& bv, int& bi, int& bn) {
    const float ov = __builtin_bit_cast(float, dpp_keep<CTRL, ROWS>(__builtin_bit_cast(int, bv)));
    const int oi = dpp_keep<CTRL, ROWS>(bi);
    const int on = dpp_keep<CTRL, ROWS>(bn);
    arg_merge(bv, bi, bn, ov, oi, on);
}
__device__ __forceinline__ void wave_arg(float& bv, int& bi, int& bn) {
    arg_step<0xB1, 0xF>(bv, bi, bn);   // quad_perm [1,0,3,2]
    arg_step<0x4E, 0xF>(bv, bi, bn);   // quad_perm [2,3,0,1]
    arg_step<0x141, 0xF>(bv, bi, bn);  // row_half_mirror
    arg_step<0x140, 0xF>(bv, bi, bn);  // row_mirror
    arg_step<0x142, 0xA>(bv, bi, bn);  // row_bcast:15 into rows 1 and 3
    arg_step<0x143, 0xC>(bv, bi, bn);  // row_bcast:31 into rows 2 and 3: lane 63 holds the result
    bv = lane_value(bv, 63);
    bi = __builtin_amdgcn_readlane(bi, 63);
    bn = __builtin_amdgcn_readlane(bn, 63);
}

// Phase tags: layer l, phase j in [0, 6): QKV, attention, tile merge, o, gate/up, down.
enum : int { PH_QKV = 0, PH_ATTN = 1, PH_MERGE = 2, PH_O = 3, PH_GU = 4, PH_DOWN = 5, PH_PER_LAYER = 6 };
// Timeline slots of one layer (optional measurement).
enum TraceSlot : int {
    TS_QKV_IN = 0,  // QKV input row gathered, normalized and quantized
    TS_QKV = 1, TS_ATTN = 2, TS_MERGE = 3, TS_O_IN = 4, TS_O = 5, TS_GU_IN = 6, TS_GU_DOT = 7,
    TS_GU = 8, TS_DOWN_IN = 9, TS_DOWN = 10,
    TS_ATT_Q = 11,     // attention: q and the new K/V row gathered (first item)
    TS_ATT_S = 12,     // attention: scores done (first item)
    TS_ATT_PV = 13,    // attention: outputs published (first item)
    TS_RING_GU = 14,   // ticks wavefront 0 waited on the ring in the gate/up phase (a duration)
    TS_RING_ALL = 15,  // ticks wavefront 0 waited on the ring in the layer (a duration)
    TS_QKV_POLL = 16,  // QKV: the input row's polls begin
    TS_PER_LAYER = 20
};

// INSTR: the optional measurement and test outputs (the per-workgroup
// timeline, the activation taps) are compiled in.  A launch that asks for
// neither runs the instance without them, whose code the compiler lays out
// better (measured about 3.5% faster per token).
//
// WIDE: the attention paths of long contexts (items of several tiles spread
// over the compute wavefronts, and a one-round merge of more than eight
// chunks) are compiled in.  Either instance computes every position; the
// host launches the wide one where those paths run, since the added code
// makes the compiler's choices elsewhere cost 1-2% per token.
//
// Each instance starts on a 4 KB boundary.  The same machine code runs at
// different speeds depending on where it starts modulo 4 KB (the Q4_0
// instance between 1991 and 2087 tokens/s for start offsets 0x000-0xf00,
// Q8_0 within 1%); aligned, an edit to one instance no longer moves the
// others.
template <int WT, bool INSTR, bool WIDE>
__global__ __launch_bounds__(SNT, 1) __attribute__((aligned(4096))) void decode_step_kernel(StepArgs a) {
    __shared__ StepShared S;
    // the wavefront index is uniform; readfirstlane lets the compiler keep
    // everything derived from it (roles, row loops) in scalar registers
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int G = gridDim.x, wg = blockIdx.x;
    const int D = a.dim, F = a.ffn;
    const int QD = a.n_heads * HDIM, KVD = a.n_kv_heads * HDIM;
    const int KB = D >> 5;
    const int GQ = a.n_heads / a.n_kv_heads;
    const Ctl C{a.error, a.spin_limit};
    StreamGeo g0 = stream_geo(WT, a.n_layers, D, F, QD, KVD, a.vocab, G, wg);
    // The LM head: row i = cw + NCW r of the CU's block is wavefront cw's
    // r-th row.  Rows r < head_nr come through the ring (the block's first
    // NCW head_nr rows, so the loaders stop there); the compute wavefronts
    // load the others themselves, which adds their requests to the loaders'.
    int head_nr = (g0.nh + NCW - 1) / NCW;
    if constexpr (head_ring_8ths(WT) < 8) {
        head_nr = (head_nr * head_ring_8ths(WT) + 7) / 8;
        g0.total = a.n_layers * g0.LU + min(g0.nh, NCW * head_nr) * g0.ua;
    }
    const StreamGeo g = g0;

    if (tid == 0) {
        S.abort = 0;
        S.csync = 0;
    }
    if (tid < NLW) S.done[tid] = 0;
    if (tid < NCW) S.cons[tid] = 0;
    if (INSTR && a.trace && tid == 0) a.trace[(size_t)wg * a.trace_stride] = wall_clock64();
    __syncthreads();  // the workgroup's only full barrier

    if (wave >= NCW) {
        run_loader(S, gl((const uint8_t*)a.stream) + (size_t)wg * a.stream_stride * 16, g.total, wave - NCW, C);
        return;
    }

    // ------------------------------------------------------------ compute group
    const int cw = wave;  // 0..NCW-1
    const unsigned epoch = *a.epoch;
    auto tag = [&](int l, int ph) -> unsigned { return epoch + 1u + (unsigned)(l * PH_PER_LAYER + ph); };
    const unsigned head_tag = epoch + 1u + (unsigned)(a.n_layers * PH_PER_LAYER);
    const int pos = *a.pos;
    // an id past the table is the reference's panic (embedding.rs:43-44):
    // the read is clamped in bounds and the error word tells the host
    const uint32_t tok_in = *a.token;
    const uint32_t tok = min(tok_in, (uint32_t)(a.embd.rows - 1));
    if (tok_in != tok && blockIdx.x == 0 && threadIdx.x == 0) *a.id_error = 1u;
    const int P = pos + 1;
    const int ntiles = (P + TPOS - 1) / TPOS;
    // Attention work: chunks of tpc consecutive 64-position tiles per KV
    // head, as few tiles per chunk as lets one round of the grid take every
    // (KV head, chunk) item; more than one chunk per head adds a merge phase.
    const int tpc = (ntiles * a.n_kv_heads + G - 1) / G;
    const int nchunks = (ntiles + tpc - 1) / tpc;
    const Xchg X = a.x;
    const cptr<StepLayer> LY = (cptr<StepLayer>)a.layers;
    // quantized-activation taps (sq_ctx::tap_q layout): per layer, sites of
    // width D, QD, D, F
    const size_t TW = 2 * (size_t)D + QD + F;
    const bool tap_a = INSTR && a.taps != 0;      // producers write their blocks' taps
    const bool tapping = tap_a && wg == 0;        // workgroup 0 writes the norm sites' taps
    // Tap addresses of site offset `so` of layer l, formed where they are used:
    // the opaque offset keeps the compiler from holding one address per site
    // live across the layer loop (register pressure).
    auto tap_q = [&](int l, size_t so) -> int8_t* {
        size_t o = (size_t)l * TW + so;
        asm volatile("" : "+s"(o));
        return a.dbg_qs + o;
    };
    auto tap_d = [&](int l, size_t so) -> uint16_t* {
        size_t o = ((size_t)l * TW + so) / 32;
        asm volatile("" : "+s"(o));
        return a.dbg_d + o;
    };
    int gen = 0;  // compute-group barrier count
    auto next_xw = [&]() -> unsigned* { return S.xw; };

    auto stamp = [&](int l, int slot) {
        if (INSTR && a.trace && tid == 0) {
            const int k = 1 + l * TS_PER_LAYER + slot;
            if (k < a.trace_stride) a.trace[(size_t)wg * a.trace_stride + k] = wall_clock64();
        }
    };
    auto put_duration = [&](int l, int slot, long long v) {
        if (INSTR && a.trace && tid == 0) {
            const int k = 1 + l * TS_PER_LAYER + slot;
            if (k < a.trace_stride) a.trace[(size_t)wg * a.trace_stride + k] = (unsigned long long)v;
        }
    };
    auto fail = [&]() { lds_st(&S.abort, 1); };
    // Ring fill level as last read (wave-uniform).  ensure(end) returns once
    // the ring holds stream units below `end`, reading the loaders' counters
    // only when the cached level falls short (when tracing, the time waited
    // is added to ring_wait).
    int filled_c = 0;
    long long ring_wait = 0;
    auto ensure = [&](int end) -> bool {
        if (filled_c >= end) return true;
        const long long t = INSTR && a.trace ? wall_clock64() : 0;
        const bool ok = spin_lds(
            [&] {
                filled_c = __builtin_amdgcn_readfirstlane(filled_units(S));
                return filled_c >= end;
            },
            S, C);
        if (INSTR && a.trace) ring_wait += wall_clock64() - t;
        return ok;
    };
    // this wavefront is done with every own row ending at or below `end`
    auto consumed = [&](int end) {
        if (lane == 0) lds_release(&S.cons[cw], end);
    };
    // ring position of stream unit u (u is wave-uniform)
    auto ring_pos = [&](int u) -> unsigned { return (unsigned)__builtin_amdgcn_readfirstlane(u % RU); };

    // Dot products of this wavefront's rows i = cw + NCW * (r0 + r), r < n
    // (n <= R), of a phase whose row i occupies stream units base + i*ru ..,
    // against activation A (one 32-block per lane, lanes below kb).  All rows'
    // reads are issued before any reduction.  False: abandon.
    auto dot_batch = [&](auto Rc, int base, int ru, int pu, int r0, int n, int kb, const ActQ& A, float* res) -> bool {
        constexpr int R = decltype(Rc)::value;
        if (!ensure(base + (cw + NCW * (r0 + n - 1) + 1) * ru)) return false;
        // rows past n re-read the batch's first row (in the ring; discarded)
        RowData rd[R];
#pragma unroll
        for (int r = 0; r < R; r++)
            rd[r] = row_fetch<WT>(S, ring_pos(base + (cw + NCW * (r0 + (r < n ? r : 0))) * ru), pu, lane);
        float t[R];
#pragma unroll
        for (int r = 0; r < R; r++) t[r] = row_math<WT>(rd[r], A, lane < kb);
        wave_totals(t);
#pragma unroll
        for (int r = 0; r < R; r++) res[r] = t[r];
        return true;
    };

    // Residual rows owned: o/down rows i = cw + NCW r of this CU, from the
    // embedding of the token (embed, model.rs:57-62; dequantize_into is exact).
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
    float h_own[RMAX];
#pragma unroll
    for (int r = 0; r < RMAX; r++) {
        const int i = cw + NCW * r;
        const int row = g.row0o + i;
        h_own[r] = (i < g.no && row < D) ? embed_at(row) : 0.0f;
    }
    // rows of o/down this wavefront owns (i = cw, cw + NCW)
    const int n_own = g.no > cw + NCW ? 2 : (g.no > cw ? 1 : 0);

    for (int l = 0; l < a.n_layers; l++) {
        const int lb = l * g.LU;  // first unit of the layer
        const gptr<float> kc = gl(a.kcache + (size_t)l * a.kv_layer);
        const gptr<float> vc = gl(a.vcache + (size_t)l * a.kv_layer);

        // ------------------------------------------------ QKV + RoPE + KV append
        {
            const unsigned T = tag(l, PH_QKV);
            if (g.row0q < QD + 2 * KVD) {
                // this wavefront's row pairs p = cw + NCW r (r < 2) and their
                // RoPE (cos, sin), requested before the input gather
                const int np = g.nq / 2 > cw + NCW ? 2 : (g.nq / 2 > cw ? 1 : 0);
                float rc[2] = {1.0f, 1.0f}, rs[2] = {0.0f, 0.0f};
#pragma unroll
                for (int r = 0; r < 2; r++) {
                    const int row = g.row0q + 2 * (cw + NCW * r);
                    if (r < np && row < QD + KVD) {
                        const int li = row < QD ? row : row - QD;
                        const cptr<float> cs =
                            (cptr<float>)a.rope + 2 * ((size_t)pos * (HDIM / 2) + ((li % HDIM) >> 1));
                        rc[r] = cs[0];
                        rs[r] = cs[1];
                    }
                }
                const Gains gn = load_gains(LY[l].attn_norm, D);
                const bool tap0 = wg == 0 && (l == 0 || tapping);
                stamp(l, TS_QKV_POLL);
                if (!norm_quant(S, l == 0 ? nullptr : X.h, l == 0 ? 0u : tag(l - 1, PH_DOWN), embed_at, gn, D, a.eps,
                                (l == 0 && wg == 0) ? a.dbg_normed : nullptr, tap0 ? tap_q(l, 0) : nullptr,
                                tap0 ? tap_d(l, 0) : nullptr, gen, C))
                    return;
                stamp(l, TS_QKV_IN);
                const ActQ A = act_lane(S, D);
                const int pu = stream_row_units(WT, D) - D / 256;
                if (np > 0) {
                    // a pair is two consecutive rows: 2 * ua units
                    if (!ensure(lb + (cw + NCW * (np - 1) + 1) * 2 * g.ua)) return fail();
                    RowData rd[4];
#pragma unroll
                    for (int r = 0; r < 2; r++) {
                        const unsigned rb = ring_pos(lb + 2 * (cw + NCW * (r < np ? r : 0)) * g.ua);
                        rd[2 * r] = row_fetch<WT>(S, rb, pu, lane);
                        rd[2 * r + 1] = row_fetch<WT>(S, ring_wrap(rb + g.ua), pu, lane);
                    }
                    float tt[4];
#pragma unroll
                    for (int k = 0; k < 4; k++) tt[k] = row_math<WT>(rd[k], A, lane < KB);
                    wave_totals(tt);
#pragma unroll
                    for (int r = 0; r < 2; r++) {
                        if (r >= np) continue;
                        const float r0 = tt[2 * r], r1 = tt[2 * r + 1];
                        const int row = g.row0q + 2 * (cw + NCW * r);
                        if (lane == 0 && row < QD + 2 * KVD) {
                            if (row < QD + KVD) {
                                const bool is_q = row < QD;
                                const int li = is_q ? row : row - QD;
                                float o0, o1;
                                sq_rotate(r0, r1, rc[r], rs[r], o0, o1);
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
                                vc[(size_t)pos * KVD + li] = r0;
                                vc[(size_t)pos * KVD + li + 1] = r1;
                                putf(X.v + li, r0, T);
                                putf(X.v + li + 1, r1, T);
                            }
                        }
                    }
                }
            }
            consumed(lb + g.offo);
            stamp(l, TS_QKV);
        }

        // ------------------------------------------------ attention (GQA)
        // Work item = (kv head, chunk of tpc 64-position tiles).  Wavefront
        // cw < GQ takes query head gh*GQ + cw on its own and walks the
        // chunk's tiles with an online softmax (the tile-merge arithmetic of
        // the merge phase): lane = position for the scores (its K row in
        // registers, q[d] read from lane d), lane = dimension for the output
        // (its V column in registers, p read from lane `position`).  Cached
        // rows (positions < pos) come from the KV cache, the new rows from this
        // launch's exchange words; the new K row reaches its lane through a
        // 64-word scratch of the wavefront in xw.
        {
            const unsigned Tin = tag(l, PH_QKV), T = tag(l, PH_ATTN);
            const int items = a.n_kv_heads * nchunks;
            const float scale = 1.0f / sqrtf((float)HDIM);
            for (int it = wg; it < items; it += G) {
                const int gh = it / nchunks, chunk = it % nchunks;
                const int t_begin = chunk * tpc, t_end = min(ntiles, t_begin + tpc);
                const bool cur = t_end == ntiles;  // this chunk holds the new position
                const int nt = t_end - t_begin;
                if (WIDE && nt > 1 && nt <= NCW) {
                    // Tile slots: slot s takes tile t_begin + s for its share of
                    // the group's query heads (NCW/NS wavefronts per slot), so the
                    // chunk's tiles are in flight at once and each wavefront reads
                    // one tile's K and V.  The slots' (o, m, l) meet in LDS and
                    // wavefront j folds head j's in tile order: the same terms in
                    // the same order as one wavefront walking the tiles.
                    const int NS = nt == 2 ? 2 : NCW, WPS = NCW / NS, HPW = (GQ + WPS - 1) / WPS;
                    const int slot = cw / WPS, j0 = (cw % WPS) * HPW, nh = min(HPW, GQ - j0);
                    const int tile = t_begin + slot;
                    float* part = (float*)(S.xw + NCW * HDIM);  // [NS][MAXG][HDIM + 2]
                    if (nh > 0 && tile < t_end) {
                        const int s0 = tile * TPOS;
                        const bool last = tile == ntiles - 1;  // holds the new position
                        sq_v4f kr[HDIM / 4];
                        {
                            const bool cached = s0 + lane < pos;
                            const gptr<const sq_v4f> kp =
                                (gptr<const sq_v4f>)(kc + (size_t)(cached ? s0 + lane : 0) * KVD + gh * HDIM);
#pragma unroll
                            for (int i = 0; i < HDIM / 4; i++) kr[i] = kp[i];
                        }
                        asm volatile("" ::: "memory");
                        int t = tid;
                        asm volatile("" : "+v"(t));
                        const int d = t & 63;
                        // q[lane] of this wavefront's heads, then the new K/V rows' element lane
                        const u64* pw[MAXG + 2];
                        u64 w[MAXG + 2];
#pragma unroll
                        for (int j = 0; j < MAXG; j++) pw[j] = j < nh ? X.q + (size_t)(gh * GQ + j0 + j) * HDIM + d : nullptr;
                        pw[MAXG] = last ? X.k + gh * HDIM + d : nullptr;
                        pw[MAXG + 1] = last ? X.v + gh * HDIM + d : nullptr;
#pragma unroll
                        for (int j = 0; j < MAXG + 2; j++) w[j] = pw[j] ? ld_c(pw[j]) : 0;
                        if (!await_words(pw, w, Tin, C, &S.abort)) return fail();
                        if (last) {
                            unsigned* scr = S.xw + cw * HDIM;  // the new K row
                            scr[lane] = (unsigned)w[MAXG];
                            __builtin_amdgcn_wave_barrier();
                            if (s0 + lane == pos) {
#pragma unroll
                                for (int i = 0; i < HDIM / 4; i++) kr[i] = *(const sq_v4f*)(scr + 4 * i);
                            }
                        }
                        const float vn = __builtin_bit_cast(float, (unsigned)w[MAXG + 1]);
                        if (it == wg) stamp(l, TS_ATT_Q);
                        // scores = dot(q, k) * (1/sqrt(head_dim)) (attention.rs:52-55)
                        float sc[MAXG];
#pragma unroll
                        for (int j = 0; j < MAXG; j++) {
                            if (j >= nh) continue;
                            const float qv = __builtin_bit_cast(float, (unsigned)w[j]);
                            float dot = 0.0f;
#pragma unroll
                            for (int i = 0; i < HDIM / 4; i++) {
                                dot += lane_value(qv, 4 * i + 0) * kr[i].x;
                                dot += lane_value(qv, 4 * i + 1) * kr[i].y;
                                dot += lane_value(qv, 4 * i + 2) * kr[i].z;
                                dot += lane_value(qv, 4 * i + 3) * kr[i].w;
                            }
                            sc[j] = (s0 + lane < P) ? dot * scale : -INFINITY;
                        }
                        if (it == wg) stamp(l, TS_ATT_S);
                        // V[s0 + sp][lane], row 0 standing in for positions
                        // without a cached row (weight 0 below)
                        float vv[TPOS];
#pragma unroll
                        for (int sp = 0; sp < TPOS; sp++) {
                            const gptr<const float> vrow =
                                vc + (size_t)(s0 + sp < pos ? s0 + sp : 0) * KVD + gh * HDIM;
                            vv[sp] = vrow[lane];
                        }
#pragma unroll
                        for (int j = 0; j < MAXG; j++) {
                            if (j >= nh) continue;
                            const float mt = wave_maximum(sc[j]);
                            const float pr = (sc[j] == -INFINITY) ? 0.0f : expf(sc[j] - mt);
                            const float lt = wave_total(pr);
                            const float pm = s0 + lane == pos ? 0.0f : pr;
                            float ot = 0.0f;
#pragma unroll
                            for (int k = 0; k < TPOS; k++) ot += lane_value(pm, k) * vv[k];
                            if (s0 + TPOS > pos) ot += lane_value(pr, pos - s0) * vn;
                            float* pp = part + (slot * MAXG + j0 + j) * (HDIM + 2);
                            pp[lane] = ot;
                            if (lane == 0) {
                                pp[HDIM] = mt;
                                pp[HDIM + 1] = lt;
                            }
                        }
                    }
                    if (!csync(S, gen, C)) return;
                    if (cw < GQ) {
                        const int h = gh * GQ + cw;
                        float M = -INFINITY, Lsum = 0.0f, O = 0.0f;
                        for (int s = 0; s < nt; s++) {
                            const float* pp = part + (s * MAXG + cw) * (HDIM + 2);
                            const float mt = pp[HDIM], lt = pp[HDIM + 1], ot = pp[lane];
                            // fold the tile into the chunk (the merge phase's arithmetic)
                            if (mt != -INFINITY) {
                                const float Mn = fmaxf(M, mt);
                                const float es = (M == -INFINITY) ? 0.0f : expf(M - Mn);
                                const float et = expf(mt - Mn);
                                Lsum = Lsum * es + lt * et;
                                O = O * es + ot * et;
                                M = Mn;
                            }
                        }
                        if (nchunks == 1) {
                            quant_put(O / Lsum, lane, h * 2, X.a, X.a + QD / 4, T, true,
                                      tap_a ? (int*)tap_q(l, D) : nullptr, tap_a ? tap_d(l, D) : nullptr);
                        } else {
                            u64* pt = X.t + ((size_t)h * a.max_tiles + chunk) * (HDIM + 2);
                            putf(pt + lane, O, T);
                            if (lane == 0) {
                                putf(pt + HDIM, M, T);
                                putf(pt + HDIM + 1, Lsum, T);
                            }
                        }
                    }
                    if (it == wg) stamp(l, TS_ATT_PV);
                    // the partials are read before a next item writes them
                    if (it + G < items && !csync(S, gen, C)) return;
                    continue;
                }
                if (cw >= GQ) continue;
                const int h = gh * GQ + cw;
                // the first tile's K rows are requested before the q words are
                // polled (and stay ahead of the polling loop)
                auto load_k = [&](int s0, sq_v4f (&kr)[HDIM / 4]) {
                    const bool cached = s0 + lane < pos;
                    const gptr<const sq_v4f> kp =
                        (gptr<const sq_v4f>)(kc + (size_t)(cached ? s0 + lane : 0) * KVD + gh * HDIM);
#pragma unroll
                    for (int i = 0; i < HDIM / 4; i++) kr[i] = kp[i];
                };
                sq_v4f kr[HDIM / 4];
                load_k(t_begin * TPOS, kr);
                asm volatile("" ::: "memory");
                // q[lane] of head h and, in the last chunk, the new K/V rows' element lane
                int t = tid;
                asm volatile("" : "+v"(t));
                const int d = t & 63;
                const u64* pw[3] = {X.q + (size_t)h * HDIM + d, cur ? X.k + gh * HDIM + d : nullptr,
                                    cur ? X.v + gh * HDIM + d : nullptr};
                u64 w[3];
#pragma unroll
                for (int j = 0; j < 3; j++) w[j] = pw[j] ? ld_c(pw[j]) : 0;
                if (!await_words(pw, w, Tin, C, &S.abort)) return fail();
                const float qv = __builtin_bit_cast(float, (unsigned)w[0]);
                const float vn = __builtin_bit_cast(float, (unsigned)w[2]);
                unsigned* scr = S.xw + cw * HDIM;  // the new K row
                scr[lane] = (unsigned)w[1];
                __builtin_amdgcn_wave_barrier();
                if (it == wg) stamp(l, TS_ATT_Q);
                float M = -INFINITY, Lsum = 0.0f, O = 0.0f;
                // One tile: scores with lane = position, then the output with
                // lane = dimension.  A tile that is not the chunk's last holds
                // its V column in two halves of registers (the first requested
                // before the softmax, the second once the first is used) and
                // requests the next tile's K rows meanwhile; the last tile
                // requests its whole V column once the scores are done.
                auto do_tile = [&](int tile, auto last_c) {
                    constexpr bool LAST = decltype(last_c)::value;
                    const int s0 = tile * TPOS;
                    if (s0 + lane == pos) {
#pragma unroll
                        for (int i = 0; i < HDIM / 4; i++) kr[i] = *(const sq_v4f*)(scr + 4 * i);
                    }
                    // scores = dot(q, k) * (1/sqrt(head_dim)) (attention.rs:52-55)
                    float dot = 0.0f;
#pragma unroll
                    for (int i = 0; i < HDIM / 4; i++) {
                        dot += lane_value(qv, 4 * i + 0) * kr[i].x;
                        dot += lane_value(qv, 4 * i + 1) * kr[i].y;
                        dot += lane_value(qv, 4 * i + 2) * kr[i].z;
                        dot += lane_value(qv, 4 * i + 3) * kr[i].w;
                    }
                    const float v = (s0 + lane < P) ? dot * scale : -INFINITY;
                    if (it == wg && tile == t_begin) stamp(l, TS_ATT_S);
                    // V[s0 + sp][lane] for sp in [k0, k0 + n); row 0 stands in
                    // for positions without a cached row (weight 0 below)
                    auto load_v = [&](int k0, float* vv, auto n_c) {
#pragma unroll
                        for (int k = 0; k < decltype(n_c)::value; k++) {
                            const int sp = k0 + k;
                            // row pointer uniform, lane offset in a register: scalar-base loads
                            const gptr<const float> vrow =
                                vc + (size_t)(s0 + sp < pos ? s0 + sp : 0) * KVD + gh * HDIM;
                            vv[k] = vrow[lane];
                        }
                    };
                    constexpr int NV = LAST ? TPOS : TPOS / 2;
                    float vv[NV];
                    load_v(0, vv, std::integral_constant<int, NV>{});
                    const float mt = wave_maximum(v);
                    const float pr = (v == -INFINITY) ? 0.0f : expf(v - mt);
                    const float lt = wave_total(pr);
                    if (!LAST) load_k(s0 + TPOS, kr);
                    // o[lane] = sum over positions of p * v (lane = dimension), in
                    // position order.  Positions past pos weigh 0 (their V value
                    // is a finite stand-in); the new row, the last position, is
                    // added last from its exchange word.
                    const float pm = s0 + lane == pos ? 0.0f : pr;
                    float ot = 0.0f;
#pragma unroll
                    for (int k = 0; k < NV; k++) ot += lane_value(pm, k) * vv[k];
                    if (!LAST) {
                        asm volatile("" ::: "memory");  // the second half's loads stay after the first's use
                        load_v(TPOS / 2, vv, std::integral_constant<int, NV>{});
#pragma unroll
                        for (int k = 0; k < NV; k++) ot += lane_value(pm, TPOS / 2 + k) * vv[k];
                    }
                    if (s0 + TPOS > pos) ot += lane_value(pr, pos - s0) * vn;
                    // fold the tile into the chunk (the merge phase's arithmetic)
                    if (mt != -INFINITY) {
                        const float Mn = fmaxf(M, mt);
                        const float es = (M == -INFINITY) ? 0.0f : expf(M - Mn);
                        const float et = expf(mt - Mn);
                        Lsum = Lsum * es + lt * et;
                        O = O * es + ot * et;
                        M = Mn;
                    }
                };
#pragma unroll 1
                for (int tile = t_begin; tile + 1 < t_end; tile++) do_tile(tile, std::false_type{});
                do_tile(t_end - 1, std::true_type{});
                if (nchunks == 1) {
                    quant_put(O / Lsum, lane, h * 2, X.a, X.a + QD / 4, T, true, tap_a ? (int*)tap_q(l, D) : nullptr,
                              tap_a ? tap_d(l, D) : nullptr);
                } else {
                    // partial (o[64], m, l) of head h, chunk `chunk`
                    u64* pt = X.t + ((size_t)h * a.max_tiles + chunk) * (HDIM + 2);
                    putf(pt + lane, O, T);
                    if (lane == 0) {
                        putf(pt + HDIM, M, T);
                        putf(pt + HDIM + 1, Lsum, T);
                    }
                }
                if (it == wg) stamp(l, TS_ATT_PV);
            }
            // the scratch in xw is free again before the o gather writes xw
            if (wg < items && !csync(S, gen, C)) return;
            stamp(l, TS_ATTN);
            if (nchunks > 1) {
                // merge the chunks of each head, then quantize the row
                const unsigned Tm = tag(l, PH_MERGE);
                bool ok = true;
                if (WIDE && nchunks > 8) {
                    // Many chunks: one workgroup per head (from the last one
                    // down, as below).  Its wavefronts poll a round of up to
                    // CPR chunks at once, wavefront cw chunks c0 + cw + NCW k,
                    // into xw; wavefront 0 then folds them in chunk order.
                    constexpr int CPR = 8 * NCW;
                    static_assert(CPR * (HDIM + 2) <= XMAX, "merge round exceeds xw");
                    float* part = (float*)S.xw;  // [chunk - c0][HDIM + 2]
                    for (int h = G - 1 - wg; h < a.n_heads; h += G) {
                        const u64* ph = X.t + (size_t)h * a.max_tiles * (HDIM + 2);
                        float M = -INFINITY, Lsum = 0.0f, O = 0.0f;
                        for (int c0 = 0; c0 < nchunks; c0 += CPR) {
                            auto addr = [&](int j) -> const u64* {
                                const int c = c0 + cw + NCW * (j / 3);
                                if (c >= nchunks) return nullptr;
                                const u64* pt = ph + (size_t)c * (HDIM + 2);
                                return j % 3 == 0 ? pt + lane : pt + HDIM + (j % 3 - 1);
                            };
                            u64 w[24];
#pragma unroll
                            for (int j = 0; j < 24; j++) w[j] = addr(j) ? ld_c(addr(j)) : 0;
                            const bool okw = await_words_at(addr, w, T, C, &S.abort);
                            if (!__all(okw)) return fail();
#pragma unroll
                            for (int k = 0; k < 8; k++) {
                                const int c = c0 + cw + NCW * k;
                                if (c >= nchunks) continue;
                                float* pp = part + (c - c0) * (HDIM + 2);
                                pp[lane] = __builtin_bit_cast(float, (unsigned)w[3 * k]);
                                if (lane == 0) {
                                    pp[HDIM] = __builtin_bit_cast(float, (unsigned)w[3 * k + 1]);
                                    pp[HDIM + 1] = __builtin_bit_cast(float, (unsigned)w[3 * k + 2]);
                                }
                            }
                            if (!csync(S, gen, C)) return;
                            if (cw == 0) {
                                const int n = min(CPR, nchunks - c0);
                                for (int c = 0; c < n; c++) {
                                    const float* pp = part + c * (HDIM + 2);
                                    const float mt = pp[HDIM];
                                    if (mt == -INFINITY) continue;
                                    const float Mn = fmaxf(M, mt);
                                    const float es = (M == -INFINITY) ? 0.0f : expf(M - Mn);
                                    const float et = expf(mt - Mn);
                                    Lsum = Lsum * es + pp[HDIM + 1] * et;
                                    O = O * es + pp[lane] * et;
                                    M = Mn;
                                }
                            }
                            // the round's partials are folded before xw is written again
                            if (!csync(S, gen, C)) return;
                        }
                        if (cw == 0)
                            quant_put(O / Lsum, lane, h * 2, X.a, X.a + QD / 4, Tm, true,
                                      tap_a ? (int*)tap_q(l, D) : nullptr, tap_a ? tap_d(l, D) : nullptr);
                    }
                } else {
                    // from the last workgroup down: those are the last to get attention items
                    for (int h = (G - 1 - wg) * NCW + cw; h < a.n_heads && ok; h += G * NCW) {
                        const int d = lane;
                        float M = -INFINITY, Lsum = 0.0f, O = 0.0f;
                        const u64* ph = X.t + (size_t)h * a.max_tiles * (HDIM + 2);
                        // (o[d], m, l) of the chunks t0 .. t0 + MT - 1, polled as one
                        // batch and merged in chunk order
                        auto merge_batch = [&](int t0, auto mt_c) -> bool {
                            constexpr int MT = decltype(mt_c)::value;
                            auto addr = [&](int j) -> const u64* {
                                const int tt = t0 + j / 3;
                                if (tt >= nchunks) return nullptr;
                                const u64* pt = ph + (size_t)tt * (HDIM + 2);
                                return j % 3 == 0 ? pt + d : pt + HDIM + (j % 3 - 1);
                            };
                            u64 w[3 * MT];
#pragma unroll
                            for (int j = 0; j < 3 * MT; j++) w[j] = addr(j) ? ld_c(addr(j)) : 0;
                            if (!await_words_at(addr, w, T, C, &S.abort)) return false;
#pragma unroll
                            for (int j2 = 0; j2 < MT; j2++) {
                                if (t0 + j2 >= nchunks) continue;
                                const float mt = __builtin_bit_cast(float, (unsigned)w[3 * j2 + 1]);
                                if (mt == -INFINITY) continue;
                                const float Mn = fmaxf(M, mt);
                                const float es = (M == -INFINITY) ? 0.0f : expf(M - Mn);
                                const float et = expf(mt - Mn);
                                Lsum = Lsum * es + __builtin_bit_cast(float, (unsigned)w[3 * j2 + 2]) * et;
                                O = O * es + __builtin_bit_cast(float, (unsigned)w[3 * j2]) * et;
                                M = Mn;
                            }
                            return true;
                        };
                        // two chunks: one small batch; more: batches of eight
                        if (nchunks <= 2) {
                            ok = merge_batch(0, std::integral_constant<int, 2>{});
                        } else {
                            for (int t0 = 0; t0 < nchunks && ok; t0 += 8)
                                ok = merge_batch(t0, std::integral_constant<int, 8>{});
                        }
                        // lanes of one wavefront agree on ok (any failure aborts)
                        if (__all(ok))
                            quant_put(O / Lsum, lane, h * 2, X.a, X.a + QD / 4, Tm, true,
                                      tap_a ? (int*)tap_q(l, D) : nullptr, tap_a ? tap_d(l, D) : nullptr);
                        else ok = false;
                    }
                    if (!ok) return fail();
                }
                stamp(l, TS_MERGE);
            }
        }

        // ------------------------------------------------ o-projection + residual
        {
            const unsigned Tin = tag(l, nchunks > 1 ? PH_MERGE : PH_ATTN), T = tag(l, PH_O);
            const int QB = QD >> 5;
            if (g.row0o < D) {
                unsigned* xw = next_xw();
                if (!gather(S, xw, X.a, QD / 4 + QB, Tin, C, gen)) return;
                stamp(l, TS_O_IN);
                if (n_own > 0) {
                    const ActQ A = xw_block<WT>(xw, QB, lane);
                    float res[RMAX];
                    if (!dot_batch(std::integral_constant<int, RMAX>{}, lb + g.offo, g.uo,
                                   stream_row_units(WT, QD) - QD / 256, 0, n_own, QB, A, res))
                        return fail();
#pragma unroll
                    for (int r = 0; r < RMAX; r++) {
                        const int row = g.row0o + cw + NCW * r;
                        if (r < n_own && row < D) {
                            h_own[r] += res[r];  // elementwise_add (layers.rs:81-109)
                            if (lane == 0) putf(X.h + hslot(row, D), h_own[r], T);
                        }
                    }
                }
            }
            consumed(lb + g.offg);
            stamp(l, TS_O);
        }

        // ------------------------------------------------ gate/up + SiLU*up + quant
        {
            const unsigned T = tag(l, PH_GU);
            if (g.ng > 0) {
                const Gains gn = load_gains(LY[l].ffn_norm, D);
                const long long rw0 = ring_wait;
                if (!norm_quant(S, X.h, tag(l, PH_O), embed_at, gn, D, a.eps, nullptr,
                                tapping ? tap_q(l, D + QD) : nullptr, tapping ? tap_d(l, D + QD) : nullptr, gen, C))
                    return;
                stamp(l, TS_GU_IN);
                const ActQ A = act_lane(S, D);
                const int pu = stream_row_units(WT, D) - D / 256;
                // rows i = cw + NCW r < 64, eight per batch
                const int ng_w = (64 - cw + NCW - 1) / NCW;
#pragma unroll 1
                for (int r0 = 0; r0 < ng_w; r0 += 8) {
                    const int n = min(8, ng_w - r0);
                    float res[8];
                    if (!dot_batch(std::integral_constant<int, 8>{}, lb + g.offg, g.ua, pu, r0, n, KB, A, res))
                        return fail();
                    consumed(lb + g.offg + (cw + NCW * (r0 + n - 1) + 1) * g.ua);
                    if (lane == 0) {
#pragma unroll
                        for (int r = 0; r < 8; r++)
                            if (r < n) S.gu[cw + NCW * (r0 + r)] = res[r];
                    }
                }
                stamp(l, TS_GU_DOT);
                put_duration(l, TS_RING_GU, ring_wait - rw0);
                if (!csync(S, gen, C)) return;
                if (cw == 0) {
                    // layers::ffn (layers.rs:64-77): silu(gate) * up, then the
                    // down projection's Q8_0 quantization per 32-block.
                    const int j = lane & 31;
                    const float gt = S.gu[j];
                    const float up = S.gu[32 + j];
                    const float f = (gt * sq_sigmoid(gt)) * up;
                    quant_put(f, lane, g.tile, X.f, X.f + F / 4, T, lane < 32,
                              tap_a ? (int*)tap_q(l, 2 * D + QD) : nullptr, tap_a ? tap_d(l, 2 * D + QD) : nullptr);
                }
            }
            consumed(lb + g.offd);
            stamp(l, TS_GU);
        }

        // ------------------------------------------------ down + residual
        {
            const unsigned T = tag(l, PH_DOWN);
            const int FB = F >> 5;
            if (g.row0o < D) {
                // A workgroup without a gate/up tile passed no barrier since
                // its o rows read xw: one here keeps the gather from
                // overwriting it early.
                if (g.ng == 0 && !csync(S, gen, C)) return;
                unsigned* xw = next_xw();
                if (!gather(S, xw, X.f, F / 4 + FB, tag(l, PH_GU), C, gen)) return;
                stamp(l, TS_DOWN_IN);
                if (n_own > 0) {
                    const int pu = stream_row_units(WT, F) - F / 256;
                    if (!ensure(lb + g.offd + (cw + NCW * (n_own - 1) + 1) * g.ud)) return fail();
                    // lane blocks b = lane + 64 k (k < FMAX / 2048), activations
                    // read once for both rows
                    // lane blocks b = lane + 64 k (k < nk), both rows' reads
                    // issued before any arithmetic
                    constexpr int KD = FMAX / 2048;
                    const int nk = (FB + 63) / 64;
                    unsigned rb[RMAX];
#pragma unroll
                    for (int r = 0; r < RMAX; r++) rb[r] = ring_pos(lb + g.offd + (cw + NCW * (r < n_own ? r : 0)) * g.ud);
                    ActQ Ak[KD];
#pragma unroll
                    for (int k = 0; k < KD; k++) {
                        if (k >= nk) break;
                        const int b = lane + 64 * k;
                        Ak[k] = xw_block<WT>(xw, FB, b < FB ? b : 0);
                    }
                    float t[RMAX] = {0.0f, 0.0f};
#pragma unroll
                    for (int r = 0; r < RMAX; r++) {
                        if (r >= n_own) break;
                        RowData rd[KD];
#pragma unroll
                        for (int k = 0; k < KD; k++) {
                            if (k >= nk) break;
                            const int b = lane + 64 * k;
                            rd[k] = row_fetch<WT>(S, rb[r], pu, b < FB ? b : 0);
                        }
#pragma unroll
                        for (int k = 0; k < KD; k++) {
                            if (k >= nk) break;
                            t[r] += row_math<WT>(rd[k], Ak[k], lane + 64 * k < FB);
                        }
                    }
                    wave_totals(t);
#pragma unroll
                    for (int r = 0; r < RMAX; r++) {
                        if (r >= n_own) continue;
                        const float res = t[r];
                        const int row = g.row0o + cw + NCW * r;
                        if (row < D) {
                            h_own[r] += res;
                            if (lane == 0) putf(X.h + hslot(row, D), h_own[r], T);
                        }
                    }
                }
            }
            consumed(lb + g.LU);
            stamp(l, TS_DOWN);
            put_duration(l, TS_RING_ALL, ring_wait);
            ring_wait = 0;
        }
    }

    // ---------------------------------------------------- final norm + LM head
    {
        const Gains gn = load_gains(a.out_norm, D);
        const bool dbg = wg == 0 && a.last_hidden != nullptr;
        if (!norm_quant(S, X.h, tag(a.n_layers - 1, PH_DOWN), embed_at, gn, D, a.eps, dbg ? a.last_hidden : nullptr,
                        dbg ? a.head_qs : nullptr, dbg ? a.head_d : nullptr, gen, C))
            return;
        stamp(a.n_layers, 0);
        const ActQ A = act_lane(S, D);
        const int pu = stream_row_units(WT, D) - D / 256;
        const int hb = a.n_layers * g.LU;
        const int nh_w = g.nh > cw ? (g.nh - cw + NCW - 1) / NCW : 0;  // rows of this wavefront
        // Lane r (< 4) of each batch takes the batch's row r: it stores that
        // logit and keeps a running (value, index, last NaN) over its rows;
        // the lanes merge once after the loop.
        float best_v = -INFINITY;
        int best_i = -1, nan_i = -1;
        if constexpr (WT == WT_Q8_0) {
            const int nrw = min(head_nr, nh_w);                            // ... through the ring
            const int nrb = (nrw + 3) / 4, ndb = (nh_w - nrw + 3) / 4;    // ring and direct batches
            auto take = [&](const float (&res)[4], int r0, int n) {
                const float v = lane == 0 ? res[0] : (lane == 1 ? res[1] : (lane == 2 ? res[2] : res[3]));
                const int row = g.row0h + cw + NCW * (r0 + lane);
                if (lane < n && row < a.vocab) {
                    st_c(&a.logits[row], v);
                    if (v != v) nan_i = max(nan_i, row);
                    else if (v > best_v || (v == best_v && row > best_i)) {
                        best_v = v;
                        best_i = row;
                    }
                }
            };
            // direct rows: batch b is rows r = nrw + 4b + q, read from the head
            // matrix itself (rows past the wavefront's or the vocabulary's end
            // read row 0; their results are dropped)
            RowData dr[4];
            auto issue_direct = [&](int b) {
                const int blk = lane < KB ? lane : 0;
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const int r = nrw + 4 * b + q;
                    int row = g.row0h + cw + NCW * r;
                    row = (r < nh_w && row < a.vocab) ? row : 0;
                    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
                    auto as_u4 = [](u32x4 v) { return make_uint4(v.x, v.y, v.z, v.w); };
                    const gptr<const u32x4> p = (gptr<const u32x4>)(gl((const int8_t*)a.head.qs) + (size_t)row * D + 32 * blk);
                    dr[q].w0 = as_u4(p[0]);
                    dr[q].w1 = as_u4(p[1]);
                    dr[q].d = gl(a.head.scale)[(size_t)row * KB + blk];
                }
            };
            auto direct_batch = [&](int b) {
                float t[4];
#pragma unroll
                for (int q = 0; q < 4; q++) t[q] = row_math<WT>(dr[q], A, lane < KB);
                wave_totals(t);
                take(t, nrw + 4 * b, min(4, nh_w - nrw - 4 * b));
            };
            int db = 0;
            if (ndb > 0) issue_direct(0);
#pragma unroll 1
            for (int rb = 0; rb < nrb; rb++) {
                const int r0 = 4 * rb;
                const int n = min(4, nrw - r0);
                float res[4];
                if (!dot_batch(std::integral_constant<int, 4>{}, hb, g.ua, pu, r0, n, KB, A, res)) return fail();
                consumed(hb + (cw + NCW * (r0 + n - 1) + 1) * g.ua);
                take(res, r0, n);
                // direct batches spread evenly over the ring batches, the next
                // one's loads in flight meanwhile
                if (db < ndb && db * nrb <= rb * ndb) {
                    direct_batch(db);
                    if (++db < ndb) issue_direct(db);
                }
            }
#pragma unroll 1
            while (db < ndb) {
                direct_batch(db);
                if (++db < ndb) issue_direct(db);
            }
        } else {
#pragma unroll 1
            for (int r0 = 0; r0 < nh_w; r0 += 4) {
                const int n = min(4, nh_w - r0);
                float res[4];
                if (!dot_batch(std::integral_constant<int, 4>{}, hb, g.ua, pu, r0, n, KB, A, res)) return fail();
                consumed(hb + (cw + NCW * (r0 + n - 1) + 1) * g.ua);
                const float v = lane == 0 ? res[0] : (lane == 1 ? res[1] : (lane == 2 ? res[2] : res[3]));
                const int row = g.row0h + cw + NCW * (r0 + lane);
                if (lane < n && row < a.vocab) {
                    st_c(&a.logits[row], v);
                    if (v != v) nan_i = row;  // rows grow along the loop
                    else if (v > best_v || (v == best_v && row > best_i)) {
                        best_v = v;
                        best_i = row;
                    }
                }
            }
        }
        wave_arg(best_v, best_i, nan_i);
        consumed(g.total);
        // The logits must be visible before the partial is (the NaN rule may
        // rescan them): wait for this wavefront's stores, then publish.
        __builtin_amdgcn_s_waitcnt(0);
        if (lane == 0) {
            S.bv[cw] = best_v;
            S.bi[cw] = best_i;
            S.bn[cw] = nan_i;
        }
        if (!csync(S, gen, C)) return;
        if (tid == 0) {
            float bv = S.bv[0];
            int bi = S.bi[0], bn = S.bn[0];
            for (int w = 1; w < NCW; w++) arg_merge(bv, bi, bn, S.bv[w], S.bi[w], S.bn[w]);
            putf(X.p + 3 * wg, bv, head_tag);
            put(X.p + 3 * wg + 1, (unsigned)bi, head_tag);
            put(X.p + 3 * wg + 2, (unsigned)bn, head_tag);
        }
        stamp(a.n_layers, 1);
    }

    // ---------------------------------------------------- greedy (workgroup 0)
    if (wg != 0) return;
    {
        unsigned* xw = next_xw();
        if (!gather(S, xw, X.p, 3 * G, head_tag, C, gen)) return;
        float bv = -INFINITY;
        int bi = -1, bn = -1;
        for (int k = tid; k < G; k += CNT)
            arg_merge(bv, bi, bn, __builtin_bit_cast(float, xw[3 * k]), (int)xw[3 * k + 1], (int)xw[3 * k + 2]);
        wave_arg(bv, bi, bn);
        if (lane == 0) {
            S.bv[cw] = bv;
            S.bi[cw] = bi;
            S.bn[cw] = bn;
        }
        if (!csync(S, gen, C)) return;
        bv = S.bv[0];
        bi = S.bi[0];
        bn = S.bn[0];
        for (int w = 1; w < NCW; w++) arg_merge(bv, bi, bn, S.bv[w], S.bi[w], S.bn[w]);
        int result = bi;
        if (bn >= 0) {
            // Iterator::max_by hands the lead to the later element whenever a
            // comparison involves NaN: the last maximum after the last NaN, or
            // that NaN when nothing follows it.
            float cv = -INFINITY;
            int ci = -1, cn = -1;
            for (int i = bn + 1 + tid; i < a.vocab; i += CNT) {
                const float v = ld_c(&a.logits[i]);
                if (v == v) arg_merge(cv, ci, cn, v, i, -1);
            }
            wave_arg(cv, ci, cn);
            if (!csync(S, gen, C)) return;  // every wavefront has read S.bv
            if (lane == 0) {
                S.bv[cw] = cv;
                S.bi[cw] = ci;
                S.bn[cw] = cn;
            }
            if (!csync(S, gen, C)) return;
            cv = S.bv[0];
            ci = S.bi[0];
            cn = S.bn[0];
            for (int w = 1; w < NCW; w++) arg_merge(cv, ci, cn, S.bv[w], S.bi[w], S.bn[w]);
            result = ci >= 0 ? ci : bn;
        }
        if (tid == 0) {
            *a.token = (uint32_t)result;
            const int h = *a.n_hist;
            a.history[h] = (uint32_t)result;
            *a.n_hist = h + 1;
            *a.pos = pos + 1;
            *a.epoch = head_tag + 1u;
            if (INSTR && a.trace) {
                const int k = 1 + a.n_layers * TS_PER_LAYER + 2;
                if (k < a.trace_stride) a.trace[k] = wall_clock64();
            }
        }
    }
}

// Copies the weight rows into the per-CU streams: blockIdx.y is the CU,
// unit u = blockIdx.x * 256 + threadIdx.x of its stream.
template <int WT>
__global__ __launch_bounds__(256) void build_stream_kernel(StepArgs a, uint8_t* dst) {
    const int G = gridDim.y, wg = blockIdx.y;
    const int D = a.dim, F = a.ffn;
    const int QD = a.n_heads * HDIM, KVD = a.n_kv_heads * HDIM;
    const StreamGeo g = stream_geo(WT, a.n_layers, D, F, QD, KVD, a.vocab, G, wg);
    const int u = blockIdx.x * 256 + threadIdx.x;
    if (u >= g.total) return;
    MatView m;
    int row, ur;
    if (u >= a.n_layers * g.LU) {
        const int r = u - a.n_layers * g.LU;
        m = a.head;
        row = g.row0h + r / g.ua;
        ur = r % g.ua;
        if (row >= a.vocab) row = 0;
    } else {
        const int l = u / g.LU, r = u % g.LU;
        const StepLayer& Ly = a.layers[l];
        if (r < g.offo) {
            m = Ly.qkv;
            row = g.row0q + r / g.ua;
            ur = r % g.ua;
            if (row >= QD + 2 * KVD) row = 0;
        } else if (r < g.offg) {
            m = Ly.o;
            row = g.row0o + (r - g.offo) / g.uo;
            ur = (r - g.offo) % g.uo;
            if (row >= D) row = 0;
        } else if (r < g.offd) {
            const int i = (r - g.offg) / g.ua;
            m = Ly.gateup;
            row = i < 32 ? g.tile * 32 + i : F + g.tile * 32 + (i - 32);
            ur = (r - g.offg) % g.ua;
        } else {
            m = Ly.down;
            row = g.row0o + (r - g.offd) / g.ud;
            ur = (r - g.offd) % g.ud;
            if (row >= D) row = 0;
        }
    }
    const int pu = stream_row_units(WT, m.k) - m.k / 256;  // payload units of a row
    // Q8_0: stream unit j < pu/2 is the first half of block j, unit pu/2 + j
    // its second half
    const int us = WT == WT_Q8_0 && ur < pu ? (ur < pu / 2 ? 2 * ur : 2 * (ur - pu / 2) + 1) : ur;
    const uint8_t* src = ur < pu ? (const uint8_t*)m.qs + (size_t)row * pu * 16 + (size_t)us * 16
                                 : (const uint8_t*)m.scale + (size_t)row * (m.k / 16) + (size_t)(ur - pu) * 16;
    *(uint4*)(dst + ((size_t)wg * a.stream_stride + u) * 16) = *(const uint4*)src;
}

}  // namespace

// A batch of R rows per wavefront, rows dealt round-robin over NCW
// wavefronts: the batch awaited by the wavefront with the lowest next row ends
// at most min(NCW * R, rows of the phase) rows past the consumed boundary.
static bool ring_fits(int dim, int ffn, int n_heads, int n_kv_heads, int grid) {
    const int QD = n_heads * HDIM, KVD = n_kv_heads * HDIM;
    const int pairs = ((QD + 2 * KVD) / 2 + grid - 1) / grid;  // QKV row pairs per CU
    const int no = (dim + grid - 1) / grid;                     // o / down rows per CU
    auto span = [](int rows, int R, int units) { return (int64_t)std::min(NCW * R, rows) * units + 64 <= RU; };
    const int ua = stream_row_units(WT_Q8_0, dim);
    return span(pairs, 2, 2 * ua) && span(64, 4, ua) && span(1 << 30, 4, ua) &&
           span(no, RMAX, stream_row_units(WT_Q8_0, QD)) && span(no, RMAX, stream_row_units(WT_Q8_0, ffn));
}

bool decode_step_fits(int dim, int ffn, int n_heads, int n_kv_heads, int grid) {
    // Each CU owns at most NCW * RMAX o/down rows (its residual rows) and one
    // gate/up tile; the K widths are multiples of 256, so every row is a whole
    // number of 16-byte units (payload and scales).
    const int QD = n_heads * HDIM;
    return grid > 0 && dim <= DMAX && ffn <= FMAX && dim % 256 == 0 && ffn % 256 == 0 && QD % 256 == 0 &&
           QD <= DMAX && n_kv_heads > 0 && n_heads % n_kv_heads == 0 && n_heads / n_kv_heads <= MAXG &&
           (dim + grid - 1) / grid <= NCW * RMAX && ffn / 32 <= grid && 3 * grid <= XMAX &&
           (n_heads + 2 * n_kv_heads) * HDIM / 2 <= 2 * NCW * grid && ring_fits(dim, ffn, n_heads, n_kv_heads, grid);
}

size_t decode_stream_stride(int wtype, int n_layers, int dim, int ffn, int n_heads, int n_kv_heads, int vocab,
                            int grid) {
    const StreamGeo g = stream_geo(wtype, n_layers, dim, ffn, n_heads * HDIM, n_kv_heads * HDIM, vocab, grid, 0);
    return ((size_t)g.total + 63) / 64 * 64;
}

int launch_build_stream(hipStream_t s, int wtype, const StepArgs& a, int grid, void* dst) {
    if (wtype != WT_Q8_0 && wtype != WT_Q4_0)
        return set_error(SQ_ERR_UNSUPPORTED, "persistent decode step: Q8_0 and Q4_0 weights only");
    if (!decode_step_fits(a.dim, a.ffn, a.n_heads, a.n_kv_heads, grid))
        return set_error(SQ_ERR_UNSUPPORTED, "persistent decode step: shape not supported");
    const size_t stride = decode_stream_stride(wtype, a.n_layers, a.dim, a.ffn, a.n_heads, a.n_kv_heads, a.vocab, grid);
    if (a.stream_stride != stride) return set_error(SQ_ERR_ARG, "weight stream: stride does not match the model");
    const dim3 bl((unsigned)((stride + 255) / 256), (unsigned)grid);
    if (wtype == WT_Q8_0)
        hipLaunchKernelGGL(build_stream_kernel<WT_Q8_0>, bl, dim3(256), 0, s, a, (uint8_t*)dst);
    else
        hipLaunchKernelGGL(build_stream_kernel<WT_Q4_0>, bl, dim3(256), 0, s, a, (uint8_t*)dst);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(SQ_ERR_HIP, std::string("weight stream build: ") + hipGetErrorString(e));
    return 0;
}

static int decode_step_resident(int wtype, bool instr, bool wide, int* out);

// The step kernel instance for a weight type, with or without the
// measurement and test outputs and the long-context attention paths (null:
// not a step weight type).
template <int WT>
static const void* decode_step_function_t(bool instr, bool wide) {
    if (instr)
        return wide ? (const void*)decode_step_kernel<WT, true, true> : (const void*)decode_step_kernel<WT, true, false>;
    return wide ? (const void*)decode_step_kernel<WT, false, true> : (const void*)decode_step_kernel<WT, false, false>;
}
static const void* decode_step_function(int wtype, bool instr, bool wide) {
    if (wtype == WT_Q8_0) return decode_step_function_t<WT_Q8_0>(instr, wide);
    if (wtype == WT_Q4_0) return decode_step_function_t<WT_Q4_0>(instr, wide);
    return nullptr;
}

// True when a step at position pos has attention items of several tiles or
// more than eight chunks per head (the kernel's own item geometry).
static bool decode_step_wide(int pos, int n_kv_heads, int grid) {
    const int ntiles = (pos + TPOS) / TPOS;
    const int tpc = (ntiles * n_kv_heads + grid - 1) / grid;
    const int nchunks = (ntiles + tpc - 1) / tpc;
    return tpc > 1 || nchunks > 8;
}

int launch_decode_step(hipStream_t s, int wtype, const StepArgs& a, int grid, int pos) {
    if (!decode_step_fits(a.dim, a.ffn, a.n_heads, a.n_kv_heads, grid))
        return set_error(SQ_ERR_UNSUPPORTED, "persistent decode step: shape not supported (dim <= 2048, ffn <= 8192, "
                                             "multiples of 256, GQA group <= 4)");
    if (a.stream == nullptr ||
        a.stream_stride != decode_stream_stride(wtype, a.n_layers, a.dim, a.ffn, a.n_heads, a.n_kv_heads, a.vocab, grid))
        return set_error(SQ_ERR_ARG, "persistent decode step: the weight stream was not built for this grid");
    // The workgroups wait on each other, so all of them must be resident at
    // once.  A grid above what the device holds (workgroups per CU times the
    // CU count) is refused here; within it, the launch places one workgroup
    // per CU.  (A cooperative launch would also guarantee residency against
    // other work on the device, at about 15 us per token; the bounded waits
    // end such a step with an error instead of a hang.)
    if (wtype != WT_Q8_0 && wtype != WT_Q4_0)
        return set_error(SQ_ERR_UNSUPPORTED, "persistent decode step: Q8_0 and Q4_0 weights only");
    const bool instr = a.taps != 0 || a.trace != nullptr;
    // SQUIRREL_STEP_WIDE=1 / =0 pins the instance (a test and measurement
    // aid: both compute every position, bit for bit alike)
    const char* pin = getenv("SQUIRREL_STEP_WIDE");
    const bool wide = pin && (pin[0] == '0' || pin[0] == '1') ? pin[0] == '1' : decode_step_wide(pos, a.n_kv_heads, grid);
    int resident = 0;
    if (int st = decode_step_resident(wtype, instr, wide, &resident)) return st;
    if (grid > resident)
        return set_error(SQ_ERR_HIP, "decode step launch: a grid of " + std::to_string(grid) +
                                         " workgroups cannot be resident at once on this device (at most " +
                                         std::to_string(resident) + ")");
    const void* f = decode_step_function(wtype, instr, wide);
    void* args[] = {(void*)&a};
    const hipError_t e = hipLaunchKernel(f, dim3(grid), dim3(SNT), args, 0, s);
    if (e != hipSuccess) return set_error(SQ_ERR_HIP, std::string("decode step launch: ") + hipGetErrorString(e));
    return 0;
}

// Workgroups of a step kernel instance the current device holds at once (per
// CU times CUs), looked up once per device.
static int decode_step_resident(int wtype, bool instr, bool wide, int* out) {
    static int cached[2][2][2][64] = {};
    int dev = 0;
    SQ_HIP_CHECK(hipGetDevice(&dev));
    int& slot = cached[wtype == WT_Q4_0 ? 1 : 0][instr ? 1 : 0][wide ? 1 : 0][dev & 63];
    if (slot == 0) {
        int cus = 0, per_cu = 0;
        SQ_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
        const void* f = decode_step_function(wtype, instr, wide);
        if (!f) return set_error(SQ_ERR_UNSUPPORTED, "persistent decode step: Q8_0 and Q4_0 weights only");
        SQ_HIP_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, f, SNT, 0));
        slot = per_cu * cus;
    }
    *out = slot;
    return 0;
}

int decode_step_max_grid(int wtype, int* grid) {
    int dev = 0, cus = 0, resident = 0;
    SQ_HIP_CHECK(hipGetDevice(&dev));
    SQ_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    // every instance (with and without the measurement outputs and the
    // long-context paths) must fit
    for (int v = 0; v < 4; v++) {
        if (int st = decode_step_resident(wtype, (v & 1) != 0, (v & 2) != 0, &resident)) return st;
        if (resident < cus) return set_error(SQ_ERR_UNSUPPORTED, "persistent decode step does not fit on a CU");
    }
    *grid = cus;
    return 0;
}

size_t exchange_words(int dim, int ffn, int n_heads, int n_kv_heads, int max_tiles, int grid) {
    const size_t QD = (size_t)n_heads * HDIM, KVD = (size_t)n_kv_heads * HDIM;
    return dim + QD + 2 * KVD + (QD / 4 + QD / 32) + ((size_t)ffn / 4 + ffn / 32) + 3 * (size_t)grid +
           (size_t)n_heads * max_tiles * (HDIM + 2);
}

}  // namespace sq
