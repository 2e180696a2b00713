// CPU emulation of the HIP device and runtime subset used by the squirrel-hip
// kernels outside the persistent decode step.  TEST INFRASTRUCTURE ONLY: it
// lets the kernels' own source run on the host, one fiber per work-item,
// under AddressSanitizer, so that an out-of-bounds index in any kernel or
// launch shows up as a sanitizer report on the CPU.
//
// Execution model.
//   * A launch runs its workgroups one after another.  Inside a workgroup
//     every work-item is a fiber; fibers run until they reach a
//     synchronization point (__syncthreads, a cross-lane operation, a
//     wavefront barrier) and are resumed round-robin.
//   * Cross-lane operations (DPP moves, readlane, shuffles, MFMA) are
//     wavefront collectives: every live lane of the 64-wide wavefront must
//     reach the same operation before any lane gets its result, which is what
//     lockstep execution guarantees on the device.  A wavefront whose lanes
//     reach different collectives, or a workgroup that cannot make progress,
//     aborts with a message (divergent cross-lane code or a barrier that not
//     every work-item reaches).
//   * __shared__ variables are static storage (workgroups never run
//     concurrently); device memory is host heap memory.
//   * Streams are synchronous; graph capture records the launches and
//     copies and a graph launch replays them in order.
#pragma once

#include <cmath>
#include <cstddef>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <tuple>
#include <type_traits>
#include <utility>

// ------------------------------------------------------------------ qualifiers
#define __global__
#define __device__
#define __host__
#define __forceinline__ inline
#define __shared__ static
#define __launch_bounds__(...)
#define __constant__ static
#define __align__(n) alignas(n)

// ------------------------------------------------------------------ vector types
struct alignas(8) float2 { float x, y; };
struct alignas(16) float4 { float x, y, z, w; };
struct alignas(8) int2 { int x, y; };
struct alignas(16) int4 { int x, y, z, w; };
struct alignas(8) uint2 { unsigned x, y; };
inline float2 make_float2(float a, float b) { return float2{a, b}; }
inline float4 make_float4(float a, float b, float c, float d) { return float4{a, b, c, d}; }
inline int2 make_int2(int a, int b) { return int2{a, b}; }
inline int4 make_int4(int a, int b, int c, int d) { return int4{a, b, c, d}; }
inline uint2 make_uint2(unsigned a, unsigned b) { return uint2{a, b}; }

struct dim3 {
    unsigned x, y, z;
    constexpr dim3(unsigned a = 1, unsigned b = 1, unsigned c = 1) : x(a), y(b), z(c) {}
};

// ------------------------------------------------------------------ runtime types
typedef int hipError_t;
enum : int {
    hipSuccess = 0,
    hipErrorInvalidValue = 1,
    hipErrorOutOfMemory = 2,
    hipErrorInvalidConfiguration = 9,
    hipErrorNotReady = 600,
    hipErrorLaunchFailure = 719,
};
struct sqemu_stream;
struct sqemu_event;
struct sqemu_graph;
typedef sqemu_stream* hipStream_t;
typedef sqemu_event* hipEvent_t;
typedef sqemu_graph* hipGraph_t;
typedef sqemu_graph* hipGraphExec_t;
typedef void* hipGraphNode_t;
enum hipMemcpyKind { hipMemcpyHostToHost = 0, hipMemcpyHostToDevice = 1, hipMemcpyDeviceToHost = 2,
                     hipMemcpyDeviceToDevice = 3, hipMemcpyDefault = 4 };
enum hipStreamCaptureMode { hipStreamCaptureModeGlobal = 0, hipStreamCaptureModeThreadLocal = 1,
                            hipStreamCaptureModeRelaxed = 2 };
enum hipDeviceAttribute_t { hipDeviceAttributeWallClockRate = 1, hipDeviceAttributeMultiprocessorCount = 2,
                            hipDeviceAttributeMaxSharedMemoryPerBlock = 3,
                            hipDeviceAttributeCooperativeLaunch = 4 };
#define hipStreamNonBlocking 1u
#define hipStreamDefault 0u
#define hipHostMallocDefault 0u
// a device symbol: its address and size (the device copy is the host object)
struct sqemu_symbol {
    const void* p;
    size_t bytes;
};
#define HIP_SYMBOL(x) (sqemu_symbol{(const void*)&(x), sizeof(x)})

// ------------------------------------------------------------------ emulator core
namespace sqemu {

// Current work-item and workgroup coordinates.
extern dim3 g_tid;
extern dim3 g_block;
extern dim3 g_blockdim;
extern dim3 g_griddim;
extern int g_lane;  // lane of the current work-item in its wavefront

// Synchronization points.
void syncthreads();
void wave_barrier();
// Deposits v (bit pattern) for the current lane, waits for every live lane
// of the wavefront, and returns a pointer to the 64 deposited values.
const uint64_t* wave_exchange(uint64_t v, int site);
// Wider deposit for MFMA operands: n 64-bit words per lane.
const uint64_t* wave_exchange_n(const uint64_t* v, int n, int site);
void* dyn_lds();

[[noreturn]] void fatal(const char* fmt, ...);

using Task = std::function<void()>;
// Queues one operation on a stream (the null stream when s is null), or
// records it while that stream is capturing.  Queued operations run at the
// next synchronization point that covers their stream, in stream order.
void submit(hipStream_t s, Task t);
void run_grid(dim3 grid, dim3 block, size_t dyn_lds_bytes, const std::function<void()>& body);
bool capturing();
// Runs what is queued on a stream (with the null stream's ordering) / on all.
void drain(hipStream_t s);
void drain_all();

template <typename T>
inline uint64_t to_bits(T v) {
    static_assert(sizeof(T) <= 8, "collective payload is at most 8 bytes");
    uint64_t b = 0;
    std::memcpy(&b, &v, sizeof(T));
    return b;
}
template <typename T>
inline T from_bits(uint64_t b) {
    T v;
    std::memcpy(&v, &b, sizeof(T));
    return v;
}

// DPP source lane for `ctrl` (GFX9 encodings used by the kernels), or -1.
int dpp_source(int lane, int ctrl);

template <typename T>
inline T update_dpp(T old, T src, int ctrl, int row_mask, int bank_mask, bool bound_ctrl) {
    const uint64_t* all = wave_exchange(to_bits(src), 0x1000 + ctrl);
    const int lane = g_lane;
    const int row = lane >> 4, bank = (lane >> 2) & 3;
    if (!((row_mask >> row) & 1) || !((bank_mask >> bank) & 1)) return old;
    const int s = dpp_source(lane, ctrl);
    if (s < 0) return bound_ctrl ? T(0) : old;
    return from_bits<T>(all[s]);
}

template <typename T>
inline T readlane(T v, int l) {
    const uint64_t* all = wave_exchange(to_bits(v), 0x2000);
    if (l < 0 || l > 63) fatal("readlane: lane %d out of range", l);
    return from_bits<T>(all[l]);
}

template <typename T>
inline T shfl_xor(T v, int mask, int width) {
    const uint64_t* all = wave_exchange(to_bits(v), 0x3000 + mask);
    const int lane = g_lane;
    int src = lane ^ mask;
    if (width < 64 && (src / width) != (lane / width)) src = lane;
    return from_bits<T>(all[src]);
}

// global_load_lds_dword / _dwordx4 (a direct global -> LDS load): each lane
// copies `size` bytes from its global address to the wavefront's LDS base +
// offset + lane * size.  The copy happens at once; the device's wait for it
// (s_waitcnt vmcnt) has nothing to wait for here.
inline void global_load_lds(const void* src, void* lds, unsigned size, int offset) {
    memcpy((char*)lds + offset + (size_t)g_lane * size, src, size);
}

inline int sdot4(int a, int b, int c, bool clamp) {
    (void)clamp;
    int s = c;
    for (int k = 0; k < 4; k++) {
        const int x = (int8_t)((unsigned)a >> (8 * k));
        const int y = (int8_t)((unsigned)b >> (8 * k));
        s += x * y;
    }
    return s;
}

}  // namespace sqemu

typedef int sqemu_v4i __attribute__((ext_vector_type(4)));
typedef float sqemu_v4f __attribute__((ext_vector_type(4)));

namespace sqemu {
// v_mfma_i32_16x16x32_i8: lane l supplies A[l%16][8(l/16) .. +7] and
// B[8(l/16) .. +7][l%16]; element r of lane l's result is D[4(l/16)+r][l%16].
inline sqemu_v4i mfma_i32_16x16x32_i8(long a, long b, sqemu_v4i c) {
    const uint64_t mine[2] = {(uint64_t)a, (uint64_t)b};
    const uint64_t* all = wave_exchange_n(mine, 2, 0x4000);
    const int lane = g_lane;
    const int col = lane & 15;
    sqemu_v4i d = c;
    for (int r = 0; r < 4; r++) {
        const int row = 4 * (lane >> 4) + r;
        int s = 0;
        for (int k = 0; k < 32; k++) {
            const int la = row + 16 * (k >> 3), lb = col + 16 * (k >> 3);
            const int8_t av = (int8_t)(all[2 * la] >> (8 * (k & 7)));
            const int8_t bv = (int8_t)(all[2 * lb + 1] >> (8 * (k & 7)));
            s += (int)av * (int)bv;
        }
        d[r] += s;
    }
    return d;
}
// v_mfma_f32_16x16x4_f32: lane l supplies A[l%16][l/16] and B[l/16][l%16].
inline sqemu_v4f mfma_f32_16x16x4f32(float a, float b, sqemu_v4f c) {
    uint64_t mine[2];
    mine[0] = to_bits(a);
    mine[1] = to_bits(b);
    const uint64_t* all = wave_exchange_n(mine, 2, 0x4001);
    const int lane = g_lane;
    const int col = lane & 15;
    sqemu_v4f d = c;
    for (int r = 0; r < 4; r++) {
        const int row = 4 * (lane >> 4) + r;
        float s = d[r];
        for (int k = 0; k < 4; k++) {
            const float av = from_bits<float>(all[2 * (row + 16 * k)]);
            const float bv = from_bits<float>(all[2 * (col + 16 * k) + 1]);
            s += av * bv;
        }
        d[r] = s;
    }
    return d;
}
// v_mfma_f32_16x16x16_f16: lane l supplies A[l%16][4(l/16) .. +3] and
// B[4(l/16) .. +3][l%16] as four halves.  The sum is formed in double and
// rounded once, which is the device result whenever that sum is exact in
// f32 (the only way the kernels use it).
typedef _Float16 sqemu_v4h __attribute__((ext_vector_type(4)));
inline sqemu_v4f mfma_f32_16x16x16f16(sqemu_v4h a, sqemu_v4h b, sqemu_v4f c) {
    uint64_t mine[2];
    memcpy(&mine[0], &a, 8);
    memcpy(&mine[1], &b, 8);
    const uint64_t* all = wave_exchange_n(mine, 2, 0x4002);
    const int lane = g_lane;
    const int col = lane & 15;
    sqemu_v4f d = c;
    for (int r = 0; r < 4; r++) {
        const int row = 4 * (lane >> 4) + r;
        double s = d[r];
        for (int k = 0; k < 16; k++) {
            _Float16 av, bv;
            memcpy(&av, (const char*)&all[2 * (row + 16 * (k >> 2))] + 2 * (k & 3), 2);
            memcpy(&bv, (const char*)&all[2 * (col + 16 * (k >> 2)) + 1] + 2 * (k & 3), 2);
            s += (double)av * (double)bv;
        }
        d[r] = (float)s;
    }
    return d;
}
// v_mfma_f32_16x16x32_f16: lane l supplies A[l%16][8(l/16) .. +7] and
// B[8(l/16) .. +7][l%16] as eight halves; the sum is formed in double and
// rounded once (every product of two halves is exact in f32).
typedef _Float16 sqemu_v8h __attribute__((ext_vector_type(8)));
inline sqemu_v4f mfma_f32_16x16x32f16(sqemu_v8h a, sqemu_v8h b, sqemu_v4f c) {
    uint64_t mine[4];
    memcpy(&mine[0], &a, 16);
    memcpy(&mine[2], &b, 16);
    const uint64_t* all = wave_exchange_n(mine, 4, 0x4005);
    const int lane = g_lane;
    const int col = lane & 15;
    sqemu_v4f d = c;
    for (int r = 0; r < 4; r++) {
        const int row = 4 * (lane >> 4) + r;
        double s = d[r];
        for (int k = 0; k < 32; k++) {
            _Float16 av, bv;
            memcpy(&av, (const char*)&all[4 * (row + 16 * (k >> 3))] + 2 * (k & 7), 2);
            memcpy(&bv, (const char*)&all[4 * (col + 16 * (k >> 3)) + 2] + 2 * (k & 7), 2);
            s += (double)av * (double)bv;
        }
        d[r] = (float)s;
    }
    return d;
}
// 32 x 32 results: element r of lane l is D[8(r/4) + 4(l/32) + r%4][l%32].
typedef int sqemu_v16i __attribute__((ext_vector_type(16)));
typedef float sqemu_v16f __attribute__((ext_vector_type(16)));
inline int mfma32_row(int lane, int r) { return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); }
// v_mfma_i32_32x32x32_i8: lane l supplies A[l%32][16(l/32) .. +15] and
// B[16(l/32) .. +15][l%32].
inline sqemu_v16i mfma_i32_32x32x32_i8(sqemu_v4i a, sqemu_v4i b, sqemu_v16i c) {
    uint64_t mine[4];
    memcpy(&mine[0], &a, 16);
    memcpy(&mine[2], &b, 16);
    const uint64_t* all = wave_exchange_n(mine, 4, 0x4003);
    const int lane = g_lane;
    const int col = lane & 31;
    sqemu_v16i d = c;
    for (int r = 0; r < 16; r++) {
        const int row = mfma32_row(lane, r);
        int s = 0;
        for (int k = 0; k < 32; k++) {
            const int8_t* pa = (const int8_t*)&all[4 * (row + 32 * (k >> 4))];
            const int8_t* pb = (const int8_t*)&all[4 * (col + 32 * (k >> 4)) + 2];
            s += (int)pa[k & 15] * (int)pb[k & 15];
        }
        d[r] += s;
    }
    return d;
}
// v_mfma_f32_32x32x8_f16: lane l supplies A[l%32][4(l/32) .. +3] and
// B[4(l/32) .. +3][l%32]; the sum is formed in double and rounded once (exact
// in the kernels' use).
inline sqemu_v16f mfma_f32_32x32x8f16(sqemu_v4h a, sqemu_v4h b, sqemu_v16f c) {
    uint64_t mine[2];
    memcpy(&mine[0], &a, 8);
    memcpy(&mine[1], &b, 8);
    const uint64_t* all = wave_exchange_n(mine, 2, 0x4004);
    const int lane = g_lane;
    const int col = lane & 31;
    sqemu_v16f d = c;
    for (int r = 0; r < 16; r++) {
        const int row = mfma32_row(lane, r);
        double s = d[r];
        for (int k = 0; k < 8; k++) {
            _Float16 av, bv;
            memcpy(&av, (const char*)&all[2 * (row + 32 * (k >> 2))] + 2 * (k & 3), 2);
            memcpy(&bv, (const char*)&all[2 * (col + 32 * (k >> 2)) + 1] + 2 * (k & 3), 2);
            s += (double)av * (double)bv;
        }
        d[r] = (float)s;
    }
    return d;
}
// v_mfma_f32_16x16x8_bf16-style operands are not emulated.
}  // namespace sqemu

#define threadIdx (::sqemu::g_tid)
#define blockIdx (::sqemu::g_block)
#define blockDim (::sqemu::g_blockdim)
#define gridDim (::sqemu::g_griddim)
#define __syncthreads() ::sqemu::syncthreads()
#define __threadfence() ((void)0)
#define __builtin_amdgcn_wave_barrier() ::sqemu::wave_barrier()
#define __builtin_amdgcn_update_dpp(o, s, c, r, b, bc) ::sqemu::update_dpp((o), (s), (c), (r), (b), (bc))
#define __builtin_amdgcn_readlane(v, l) ::sqemu::readlane((v), (l))
#define __builtin_amdgcn_s_barrier() ::sqemu::syncthreads()
// the kernels take v_readfirstlane of wavefront-uniform values only
#define __builtin_amdgcn_readfirstlane(v) (v)
// wait counts have nothing to wait for: memory operations complete at once
#define __builtin_amdgcn_s_waitcnt(n) ((void)(n))
#define __builtin_amdgcn_global_load_lds(src, lds, size, off, aux) \
    ::sqemu::global_load_lds((const void*)(src), (void*)(lds), (size), (off))
// scheduling hints have no effect on the emulated execution
#define __builtin_amdgcn_sched_barrier(m) ((void)(m))
// v_exp_f32 (2^x): the host exp2f stands in for the device instruction
#define __builtin_amdgcn_exp2f(x) ::exp2f((float)(x))
#define __builtin_amdgcn_sdot4(a, b, c, cl) ::sqemu::sdot4((a), (b), (c), (cl))
#define __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, c, x, y, z) ::sqemu::mfma_i32_16x16x32_i8((a), (b), (c))
#define __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, x, y, z) ::sqemu::mfma_f32_16x16x4f32((a), (b), (c))
#define __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, x, y, z) ::sqemu::mfma_f32_16x16x16f16((a), (b), (c))
#define __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, x, y, z) ::sqemu::mfma_f32_16x16x32f16((a), (b), (c))
#define __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, x, y, z) ::sqemu::mfma_i32_32x32x32_i8((a), (b), (c))
#define __builtin_amdgcn_mfma_f32_32x32x8f16(a, b, c, x, y, z) ::sqemu::mfma_f32_32x32x8f16((a), (b), (c))
#define __shfl_xor(v, m, w) ::sqemu::shfl_xor((v), (m), (w))

template <typename T>
inline T atomicAdd(T* p, T v) {
    T o = *p;
    *p = o + v;
    return o;
}
template <typename T>
inline T atomicExch(T* p, T v) {
    T o = *p;
    *p = v;
    return o;
}
template <typename T>
inline T atomicMax(T* p, T v) {
    T o = *p;
    if (v > o) *p = v;
    return o;
}

// Device min / max overloads of the HIP headers.
template <typename T>
inline T min(T a, T b) { return b < a ? b : a; }
template <typename T>
inline T max(T a, T b) { return a < b ? b : a; }

// ------------------------------------------------------------------ kernel launch
namespace sqemu {
// Device memory on the GPU is its own address range; here it is host memory.
// Every 8-byte word of every kernel argument is checked when the launch runs
// (also on each graph replay): a word that points into host memory (heap,
// stack, globals, file mappings) outside every live device allocation is a
// host or freed pointer handed to a kernel, which the device could not
// dereference, and stops the run.
void check_kernel_arg(const void* kernel, int index, const void* arg, size_t bytes);
template <typename... P, typename... A>
void launch(void (*k)(P...), dim3 grid, dim3 block, size_t shm, hipStream_t stream, A&&... args) {
    auto tup = std::make_tuple(static_cast<std::decay_t<P>>(args)...);
    submit(stream, [=]() {
        std::apply(
            [&](const auto&... a) {
                int i = 0;
                (check_kernel_arg(reinterpret_cast<const void*>(k), i++, &a, sizeof(a)), ...);
            },
            tup);
        run_grid(grid, block, shm, [&]() { std::apply(k, tup); });
    });
}
}  // namespace sqemu
#define hipLaunchKernelGGL(kernel, grid, block, shm, stream, ...) \
    ::sqemu::launch(kernel, dim3(grid), dim3(block), (size_t)(shm), (stream), ##__VA_ARGS__)

// ------------------------------------------------------------------ runtime API
hipError_t hipGetLastError();
hipError_t hipPeekAtLastError();
const char* hipGetErrorString(hipError_t e);
hipError_t hipGetDeviceCount(int* n);
hipError_t hipGetDevice(int* d);
hipError_t hipSetDevice(int d);
hipError_t hipDeviceGetAttribute(int* v, hipDeviceAttribute_t a, int dev);
hipError_t hipDeviceSynchronize();
hipError_t hipMalloc(void** p, size_t n);
template <typename T>
inline hipError_t hipMalloc(T** p, size_t n) { return hipMalloc((void**)p, n); }
hipError_t hipFree(void* p);
hipError_t hipHostMalloc(void** p, size_t n, unsigned flags);
template <typename T>
inline hipError_t hipHostMalloc(T** p, size_t n, unsigned flags) { return hipHostMalloc((void**)p, n, flags); }
hipError_t hipHostFree(void* p);
hipError_t hipMemcpy(void* d, const void* s, size_t n, hipMemcpyKind k);
hipError_t hipMemcpyAsync(void* d, const void* s, size_t n, hipMemcpyKind k, hipStream_t st);
hipError_t hipMemset(void* d, int v, size_t n);
hipError_t hipMemsetAsync(void* d, int v, size_t n, hipStream_t st);
hipError_t hipStreamCreate(hipStream_t* s);
hipError_t hipStreamCreateWithFlags(hipStream_t* s, unsigned flags);
hipError_t hipStreamDestroy(hipStream_t s);
hipError_t hipStreamSynchronize(hipStream_t s);
hipError_t hipEventCreate(hipEvent_t* e);
hipError_t hipEventDestroy(hipEvent_t e);
hipError_t hipEventRecord(hipEvent_t e, hipStream_t s);
hipError_t hipEventSynchronize(hipEvent_t e);
hipError_t hipEventElapsedTime(float* ms, hipEvent_t a, hipEvent_t b);
hipError_t hipStreamBeginCapture(hipStream_t s, hipStreamCaptureMode m);
hipError_t hipStreamEndCapture(hipStream_t s, hipGraph_t* g);
hipError_t hipGraphInstantiate(hipGraphExec_t* e, hipGraph_t g, hipGraphNode_t* n, char* log, size_t len);
hipError_t hipGraphLaunch(hipGraphExec_t e, hipStream_t s);
hipError_t hipGraphExecDestroy(hipGraphExec_t e);
hipError_t hipGraphDestroy(hipGraph_t g);
hipError_t hipGetSymbolAddress(void** p, sqemu_symbol sym);
