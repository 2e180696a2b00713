// CPU emulation core for the HIP kernels: fiber scheduler, wavefront
// collectives and the runtime API subset.  TEST INFRASTRUCTURE ONLY (see
// include/hip/hip_runtime.h for the execution model).
#include <hip/hip_runtime.h>

#include <sys/mman.h>

#include <chrono>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <deque>
#include <map>
#include <memory>
#include <set>
#include <vector>

#if defined(__has_feature)
#if __has_feature(address_sanitizer)
#define SQEMU_ASAN 1
#endif
#endif
#ifdef SQEMU_ASAN
#include <sanitizer/asan_interface.h>
#endif
// The sanitizer's fiber-switch annotations cost a system call per switch;
// without them the sanitizer still checks every access (shadow memory is
// per address, not per stack), and kernels never unwind across a switch.
#define SQEMU_FIBER_ANNOTATIONS 0

// Fiber switch for x86-64 System V: saves the callee-saved registers and the
// stack pointer of the current context in *from and resumes `to`.
extern "C" void sqemu_swap(void** from, void* to);
asm(R"(
    .text
    .globl sqemu_swap
    .type sqemu_swap,@function
sqemu_swap:
    pushq %rbp
    pushq %rbx
    pushq %r12
    pushq %r13
    pushq %r14
    pushq %r15
    movq %rsp, (%rdi)
    movq %rsi, %rsp
    popq %r15
    popq %r14
    popq %r13
    popq %r12
    popq %rbx
    popq %rbp
    ret
    .size sqemu_swap, .-sqemu_swap
)");

namespace sqemu {

dim3 g_tid, g_block, g_blockdim, g_griddim;
int g_lane = 0;

namespace {

constexpr size_t kStack = 512 * 1024;
constexpr int kMaxN = 4;  // 64-bit words per lane in one collective

struct Wave {
    int size = 0;  // work-items the wavefront started with
    int live = 0;
    int count = 0;
    unsigned gen = 0;
    int site = -1;
    uint64_t slot[2][64 * kMaxN];
};

struct Block {
    int live = 0;
    int count = 0;
    unsigned gen = 0;
};

struct FiberRec {
    void* sp = nullptr;
    char* stack = nullptr;
    bool done = false;
    dim3 tid;
    int lane = 0;
    int wave = 0;
};

std::vector<FiberRec> g_fibers;
std::vector<Wave> g_waves;
Block g_blk;
void* g_sched_sp = nullptr;
int g_cur = -1;
const std::function<void()>* g_body = nullptr;
uint64_t g_progress = 0;
std::vector<char> g_dyn;
size_t g_dyn_bytes = 0;

#if SQEMU_FIBER_ANNOTATIONS
const void* g_sched_stack_bottom = nullptr;
size_t g_sched_stack_size = 0;
#endif

void switch_to_sched() {
    FiberRec& f = g_fibers[g_cur];
#if SQEMU_FIBER_ANNOTATIONS
    void* fake = nullptr;
    __sanitizer_start_switch_fiber(f.done ? nullptr : &fake, g_sched_stack_bottom, g_sched_stack_size);
    sqemu_swap(&f.sp, g_sched_sp);
    __sanitizer_finish_switch_fiber(fake, nullptr, nullptr);
#else
    sqemu_swap(&f.sp, g_sched_sp);
#endif
}

void yield() { switch_to_sched(); }

void fiber_entry() {
#if SQEMU_FIBER_ANNOTATIONS
    __sanitizer_finish_switch_fiber(nullptr, &g_sched_stack_bottom, &g_sched_stack_size);
#endif
    (*g_body)();
    FiberRec& f = g_fibers[g_cur];
    f.done = true;
    g_blk.live--;
    g_waves[f.wave].live--;
    g_progress++;
    switch_to_sched();
    fatal("a finished fiber was resumed");
}

void set_current(int i) {
    g_cur = i;
    FiberRec& f = g_fibers[i];
    g_tid = f.tid;
    g_lane = f.lane;
}

}  // namespace

void fatal(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    fprintf(stderr, "sqemu: ");
    vfprintf(stderr, fmt, ap);
    fprintf(stderr, " (block %u,%u,%u thread %u)\n", g_block.x, g_block.y, g_block.z, g_tid.x);
    va_end(ap);
    fflush(stderr);
    abort();
}

void syncthreads() {
    if (g_cur < 0) fatal("__syncthreads outside a kernel");
    g_blk.count++;
    g_progress++;
    const unsigned gen = g_blk.gen;
    while (g_blk.gen == gen) {
        if (g_blk.count >= g_blk.live) {
            g_blk.gen++;
            g_blk.count = 0;
            g_progress++;
            break;
        }
        yield();
    }
}

static const uint64_t* collective(const uint64_t* v, int n, int site) {
    if (g_cur < 0) fatal("cross-lane operation outside a kernel");
    FiberRec& f = g_fibers[g_cur];
    Wave& w = g_waves[f.wave];
    if (w.live != w.size)
        fatal("wavefront %d: cross-lane operation 0x%x after %d of its lanes returned", f.wave, site, w.size - w.live);
    if (w.count == 0) {
        w.site = site;
    } else if (w.site != site) {
        fatal("wavefront %d: lanes reached different cross-lane operations (0x%x vs 0x%x)", f.wave, w.site, site);
    }
    const unsigned gen = w.gen;
    uint64_t* s = w.slot[gen & 1];
    for (int i = 0; i < n; i++) s[n * f.lane + i] = v[i];
    w.count++;
    g_progress++;
    while (w.gen == gen) {
        if (w.live != w.size)
            fatal("wavefront %d: %d lanes returned while others wait at cross-lane operation 0x%x", f.wave,
                  w.size - w.live, site);
        if (w.count >= w.live) {
            w.gen++;
            w.count = 0;
            g_progress++;
            break;
        }
        yield();
    }
    return s;
}

const uint64_t* wave_exchange(uint64_t v, int site) { return collective(&v, 1, site); }
const uint64_t* wave_exchange_n(const uint64_t* v, int n, int site) {
    if (n > kMaxN) fatal("collective payload too wide");
    return collective(v, n, site);
}
void wave_barrier() {
    uint64_t z = 0;
    collective(&z, 1, 0x7000);
}

void* dyn_lds() {
    if (g_dyn_bytes == 0) fatal("dynamic LDS used by a launch that reserved none");
    return g_dyn.data();
}

int dpp_source(int lane, int ctrl) {
    const int row = lane >> 4, in_row = lane & 15;
    if (ctrl >= 0 && ctrl <= 0xFF) return (lane & ~3) | ((ctrl >> (2 * (lane & 3))) & 3);
    if (ctrl >= 0x101 && ctrl <= 0x10F) {  // row_shl
        const int n = ctrl - 0x100;
        return in_row + n <= 15 ? lane + n : -1;
    }
    if (ctrl >= 0x111 && ctrl <= 0x11F) {  // row_shr
        const int n = ctrl - 0x110;
        return in_row >= n ? lane - n : -1;
    }
    if (ctrl >= 0x121 && ctrl <= 0x12F) {  // row_ror
        const int n = ctrl - 0x120;
        return (lane & ~15) | ((in_row - n) & 15);
    }
    switch (ctrl) {
        case 0x140: return (lane & ~15) | (15 - in_row);   // row_mirror
        case 0x141: return (lane & ~7) | (7 - (lane & 7));  // row_half_mirror
        case 0x142: return row >= 1 ? 16 * row - 1 : -1;    // row_bcast:15
        case 0x143: return row >= 2 ? 31 : -1;              // row_bcast:31
        default: fatal("DPP control 0x%x is not emulated", ctrl);
    }
}

void run_grid(dim3 grid, dim3 block, size_t dyn_bytes, const std::function<void()>& body) {
    const unsigned nt = block.x * block.y * block.z;
    if (nt == 0 || nt > 1024) fatal("launch: %u work-items per workgroup", nt);
    if (grid.x == 0 || grid.y == 0 || grid.z == 0) fatal("launch: empty grid");
    if (grid.y > 65535 || grid.z > 65535) fatal("launch: grid (%u, %u, %u) exceeds the y/z limits", grid.x, grid.y, grid.z);
    if (block.y != 1 || block.z != 1) fatal("launch: only one-dimensional workgroups are emulated");
    const int nwaves = (int)((nt + 63) / 64);
    static std::vector<char*> stacks;
    while (stacks.size() < nt) {
        void* p = mmap(nullptr, kStack, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS | MAP_NORESERVE, -1, 0);
        if (p == MAP_FAILED) fatal("mmap of a fiber stack failed");
        stacks.push_back((char*)p);
    }
    g_body = &body;
    g_griddim = grid;
    g_blockdim = block;
    g_dyn_bytes = dyn_bytes;
    g_dyn.assign(dyn_bytes ? dyn_bytes : 1, 0);
    for (unsigned bz = 0; bz < grid.z; bz++)
        for (unsigned by = 0; by < grid.y; by++)
            for (unsigned bx = 0; bx < grid.x; bx++) {
                g_block = dim3(bx, by, bz);
                g_fibers.assign(nt, FiberRec{});
                g_waves.assign(nwaves, Wave{});
                g_blk = Block{};
                g_blk.live = (int)nt;
                for (unsigned t = 0; t < nt; t++) {
                    FiberRec& f = g_fibers[t];
                    f.tid = dim3(t, 0, 0);
                    f.lane = (int)(t & 63);
                    f.wave = (int)(t >> 6);
                    g_waves[f.wave].live++;
                    g_waves[f.wave].size++;
                    f.stack = stacks[t];
#ifdef SQEMU_ASAN
                    __asan_unpoison_memory_region(f.stack, kStack);
#endif
                    // initial frame: six callee-saved registers, then the entry
                    // address that sqemu_swap returns to; 16-byte alignment at entry
                    uintptr_t top = ((uintptr_t)(f.stack + kStack) & ~(uintptr_t)15) - 8;
                    void** sp = (void**)top;
                    *--sp = (void*)&fiber_entry;
                    for (int r = 0; r < 6; r++) *--sp = nullptr;
                    f.sp = sp;
                }
                int alive = (int)nt;
                uint64_t idle_rounds = 0;
                while (alive > 0) {
                    const uint64_t before = g_progress;
                    for (unsigned t = 0; t < nt; t++) {
                        if (g_fibers[t].done) continue;
                        set_current((int)t);
#if SQEMU_FIBER_ANNOTATIONS
                        void* fake = nullptr;
                        __sanitizer_start_switch_fiber(&fake, g_fibers[t].stack, kStack);
                        sqemu_swap(&g_sched_sp, g_fibers[t].sp);
                        __sanitizer_finish_switch_fiber(fake, nullptr, nullptr);
#else
                        sqemu_swap(&g_sched_sp, g_fibers[t].sp);
#endif
                        if (g_fibers[t].done) alive--;
                    }
                    g_cur = -1;
                    if (g_progress == before) {
                        if (++idle_rounds > 2) {
                            int at_bar = 0;
                            for (auto& w : g_waves) at_bar += w.count;
                            fatal("workgroup cannot progress: %d of %d live work-items at __syncthreads, %d at "
                                  "cross-lane operations",
                                  g_blk.count, g_blk.live, at_bar);
                        }
                    } else {
                        idle_rounds = 0;
                    }
                }
            }
    g_cur = -1;
}

}  // namespace sqemu

// ------------------------------------------------------------------ streams
// Streams are asynchronous as on the device: every copy, fill, launch and
// event record is queued on its stream and runs only at a synchronization
// point that covers that stream (hipStreamSynchronize, hipDeviceSynchronize,
// hipEventSynchronize, and the implicit ones below), in stream order.  So a
// host buffer rewritten before the copy that reads it has run, a result read
// before its producer has run, or work ordered only by the legacy null
// stream against a non-blocking stream shows up here as wrong data.
//  * The null stream synchronizes with blocking streams (work queued on one
//    first drains the other) but not with streams created with
//    hipStreamNonBlocking.
//  * hipMemcpy runs on the null stream.  It returns when it is done, except
//    from pageable host memory to the device, where it returns once the
//    source is staged and the transfer stays queued on the null stream.
//    hipMemset is queued on the null stream (asynchronous for device memory).
//  * hipFree and hipHostFree synchronize the device first.
//  * hipMemcpyAsync from pinned host memory (hipHostMalloc) reads the source
//    when the copy runs; from pageable memory it is staged when called.  Into
//    pinned memory the destination keeps its old contents until the copy
//    runs; into pageable memory the call drains the stream and copies at once.
struct sqemu_stream {
    bool nonblocking = false;
    bool capturing = false;
    std::deque<sqemu::Task> q;
    std::vector<sqemu::Task>* capture = nullptr;
};

namespace sqemu {
namespace {
sqemu_stream g_null_stream;
std::set<sqemu_stream*> g_streams;
bool g_draining = false;

sqemu_stream* S(hipStream_t s) { return s ? s : &g_null_stream; }

void drain_one(sqemu_stream* st) {
    if (g_draining) fatal("a queued operation synchronized a stream");
    g_draining = true;
    while (!st->q.empty()) {
        Task t = std::move(st->q.front());
        st->q.pop_front();
        t();
    }
    g_draining = false;
}

void drain_blocking() {
    for (sqemu_stream* st : g_streams)
        if (!st->nonblocking) drain_one(st);
}
}  // namespace

void drain(hipStream_t s) {
    sqemu_stream* st = S(s);
    if (st == &g_null_stream) drain_blocking();
    drain_one(st);
}

void drain_all() {
    drain_one(&g_null_stream);
    for (sqemu_stream* st : g_streams) drain_one(st);
}

bool capturing() {
    if (g_null_stream.capturing) return true;
    for (sqemu_stream* st : g_streams)
        if (st->capturing) return true;
    return false;
}

void submit(hipStream_t s, Task t) {
    sqemu_stream* st = S(s);
    if (st->capturing) {
        st->capture->push_back(std::move(t));
        return;
    }
    // legacy null-stream ordering against the blocking streams
    if (st == &g_null_stream) drain_blocking();
    else if (!st->nonblocking) drain_one(&g_null_stream);
    st->q.push_back(std::move(t));
}

// Live device allocations (hipMalloc, hipHostMalloc, device symbols): base -> bytes.
std::map<uintptr_t, size_t> g_dev;

namespace {
// The allocation that holds address a (one past the end counts), or none.
const std::pair<const uintptr_t, size_t>* dev_block(uintptr_t a, size_t n = 0) {
    auto it = g_dev.upper_bound(a);
    if (it == g_dev.begin()) return nullptr;
    --it;
    return a + n <= it->first + it->second ? &*it : nullptr;
}

// Where a host address lies, or nullptr when it is no host memory: the
// sanitizer's heap, stack and globals, else a mapping of /proc/self/maps
// (file mappings such as the model file; the sanitizer's shadow regions,
// which span terabytes, excluded).
const char* host_region(uintptr_t a) {
#ifdef SQEMU_ASAN
    char name[64];
    void* base = nullptr;
    size_t size = 0;
    const char* kind = __asan_locate_address((void*)a, name, sizeof name, &base, &size);
    if (!strcmp(kind, "heap") || !strcmp(kind, "stack") || !strcmp(kind, "stack-fake") || !strcmp(kind, "global"))
        return kind;
#endif
    FILE* f = fopen("/proc/self/maps", "r");
    if (!f) return nullptr;
    unsigned long lo, hi;
    char line[512];
    const char* found = nullptr;
    while (!found && fgets(line, sizeof line, f)) {
        if (sscanf(line, "%lx-%lx", &lo, &hi) == 2 && a >= lo && a < hi && hi - lo < (1ull << 40)) found = "mapping";
    }
    fclose(f);
    return found;
}
}  // namespace

void check_kernel_arg(const void* kernel, int index, const void* arg, size_t bytes) {
    for (size_t off = 0; off + 8 <= bytes; off += 8) {
        uint64_t w;
        memcpy(&w, (const char*)arg + off, 8);
        if (w < 4096 || w >= (1ull << 47) || dev_block(w)) continue;
        if (const char* where = host_region(w)) {
            char fn[256] = "?";
#ifdef SQEMU_ASAN
            // (the symbolizer takes return addresses: one byte into the entry)
            __sanitizer_symbolize_pc((char*)const_cast<void*>(kernel) + 1, "%f", fn, sizeof fn);
#endif
            fatal("kernel %s (%p) argument %d (bytes %zu-%zu) holds 0x%lx, in host memory (%s) outside every live "
                  "device allocation",
                  fn, kernel, index, off, off + 7, (unsigned long)w, where);
        }
    }
}

void check_copy(const char* what, const void* d, const void* s, size_t n, hipMemcpyKind k) {
    if (!n) return;
    const bool dd = k == hipMemcpyDeviceToDevice || k == hipMemcpyHostToDevice;
    const bool sd = k == hipMemcpyDeviceToDevice || k == hipMemcpyDeviceToHost;
    if (dd && !dev_block((uintptr_t)d, n)) fatal("%s: destination %p (+%zu) is no device allocation", what, d, n);
    if (sd && s && !dev_block((uintptr_t)s, n)) fatal("%s: source %p (+%zu) is no device allocation", what, s, n);
}
}  // namespace sqemu

// ------------------------------------------------------------------ runtime API
struct sqemu_event {
    std::chrono::steady_clock::time_point t;
    sqemu_stream* stream = nullptr;
    bool done = true;
};
struct sqemu_graph {
    std::vector<sqemu::Task> tasks;
};

namespace sqemu {
// Pinned host allocations (hipHostMalloc): base -> bytes.
std::map<uintptr_t, size_t> g_pinned;
namespace {
bool pinned(const void* p, size_t n) {
    auto it = g_pinned.upper_bound((uintptr_t)p);
    if (it == g_pinned.begin()) return false;
    --it;
    return (uintptr_t)p + n <= it->first + it->second;
}
}  // namespace
}  // namespace sqemu

hipError_t hipGetLastError() { return hipSuccess; }
hipError_t hipPeekAtLastError() { return hipSuccess; }
const char* hipGetErrorString(hipError_t e) { return e == hipSuccess ? "no error" : "emulated error"; }
hipError_t hipGetDeviceCount(int* n) {
    *n = 1;
    return hipSuccess;
}
hipError_t hipGetDevice(int* d) {
    *d = 0;
    return hipSuccess;
}
hipError_t hipSetDevice(int) { return hipSuccess; }
hipError_t hipDeviceGetAttribute(int* v, hipDeviceAttribute_t a, int) {
    switch (a) {
        case hipDeviceAttributeWallClockRate: *v = 100000; break;
        // SQEMU_CUS: a smaller emulated device, so that the grid-size rules
        // (workgroups per CU) pick the large-grid kernels for small inputs
        case hipDeviceAttributeMultiprocessorCount: {
            const char* e = getenv("SQEMU_CUS");
            *v = e ? atoi(e) : 256;
            if (*v <= 0) *v = 256;
            break;
        }
        case hipDeviceAttributeMaxSharedMemoryPerBlock: *v = 160 * 1024; break;
        case hipDeviceAttributeCooperativeLaunch: *v = 1; break;
        default: return hipErrorInvalidValue;
    }
    return hipSuccess;
}
hipError_t hipDeviceSynchronize() {
    sqemu::drain_all();
    return hipSuccess;
}
namespace sqemu {
uint64_t g_malloc_calls = 0;
}
hipError_t hipMalloc(void** p, size_t n) {
    sqemu::g_malloc_calls++;
    // exact-size heap blocks: the sanitizer poisons everything past n
    void* q = nullptr;
    if (posix_memalign(&q, 256, n ? n : 1)) return hipErrorOutOfMemory;
    // device memory starts with arbitrary contents
    memset(q, 0xA5, n ? n : 1);
    *p = q;
    sqemu::g_dev[(uintptr_t)q] = n;
    return hipSuccess;
}
hipError_t hipFree(void* p) {
    // an implicit device synchronization, as on the device
    sqemu::drain_all();
    if (p && !sqemu::g_dev.erase((uintptr_t)p)) sqemu::fatal("hipFree of %p, not a device allocation", p);
    sqemu::g_pinned.erase((uintptr_t)p);
    free(p);
    return hipSuccess;
}
hipError_t hipHostMalloc(void** p, size_t n, unsigned) {
    hipError_t e = hipMalloc(p, n);
    if (e == hipSuccess) sqemu::g_pinned[(uintptr_t)*p] = n;
    return e;
}
hipError_t hipHostFree(void* p) { return hipFree(p); }
hipError_t hipMemcpy(void* d, const void* s, size_t n, hipMemcpyKind k) {
    if (sqemu::capturing()) sqemu::fatal("hipMemcpy during a stream capture");
    if (k == hipMemcpyHostToDevice && !sqemu::pinned(s, n)) {
        // from pageable memory the call returns once the source is staged;
        // the transfer itself is null-stream work, so a non-blocking stream
        // is not ordered after it
        auto staged = std::make_shared<std::vector<char>>((const char*)s, (const char*)s + n);
        sqemu::submit(nullptr, [=]() {
            sqemu::check_copy("hipMemcpy", d, s, n, k);
            if (n) memcpy(d, staged->data(), n);
        });
        return hipSuccess;
    }
    // on the null stream: ordered after its own work and the blocking
    // streams', not after non-blocking streams
    sqemu::drain(nullptr);
    sqemu::check_copy("hipMemcpy", d, s, n, k);
    if (n) memcpy(d, s, n);
    return hipSuccess;
}
hipError_t hipMemcpyAsync(void* d, const void* s, size_t n, hipMemcpyKind k, hipStream_t st) {
    if (k == hipMemcpyHostToDevice && !sqemu::pinned(s, n) && !(st ? st->capturing : false)) {
        // pageable source: staged at the call
        auto staged = std::make_shared<std::vector<char>>((const char*)s, (const char*)s + n);
        sqemu::submit(st, [=]() {
            sqemu::check_copy("hipMemcpyAsync", d, s, n, k);
            if (n) memcpy(d, staged->data(), n);
        });
        return hipSuccess;
    }
    if (k == hipMemcpyDeviceToHost && !sqemu::pinned(d, n) && !(st ? st->capturing : false)) {
        // pageable destination: the call returns once the copy is done
        sqemu::submit(st, [=]() {
            sqemu::check_copy("hipMemcpyAsync", d, s, n, k);
            if (n) memmove(d, s, n);
        });
        sqemu::drain(st);
        return hipSuccess;
    }
    sqemu::submit(st, [=]() {
        sqemu::check_copy("hipMemcpyAsync", d, s, n, k);
        if (n) memmove(d, s, n);
    });
    return hipSuccess;
}
hipError_t hipMemset(void* d, int v, size_t n) {
    if (sqemu::capturing()) sqemu::fatal("hipMemset during a stream capture");
    sqemu::submit(nullptr, [=]() {
        sqemu::check_copy("hipMemset", d, nullptr, n, hipMemcpyHostToDevice);
        if (n) memset(d, v, n);
    });
    return hipSuccess;
}
hipError_t hipMemsetAsync(void* d, int v, size_t n, hipStream_t st) {
    sqemu::submit(st, [=]() {
        sqemu::check_copy("hipMemsetAsync", d, nullptr, n, hipMemcpyHostToDevice);
        if (n) memset(d, v, n);
    });
    return hipSuccess;
}
hipError_t hipStreamCreate(hipStream_t* s) { return hipStreamCreateWithFlags(s, hipStreamDefault); }
hipError_t hipStreamCreateWithFlags(hipStream_t* s, unsigned flags) {
    *s = new sqemu_stream();
    (*s)->nonblocking = (flags & hipStreamNonBlocking) != 0;
    sqemu::g_streams.insert(*s);
    return hipSuccess;
}
hipError_t hipStreamDestroy(hipStream_t s) {
    // queued work still completes
    sqemu::drain(s);
    sqemu::g_streams.erase(s);
    delete s;
    return hipSuccess;
}
hipError_t hipStreamSynchronize(hipStream_t s) {
    sqemu::drain(s);
    return hipSuccess;
}
hipError_t hipEventCreate(hipEvent_t* e) {
    *e = new sqemu_event{std::chrono::steady_clock::now(), nullptr, true};
    return hipSuccess;
}
hipError_t hipEventDestroy(hipEvent_t e) {
    delete e;
    return hipSuccess;
}
hipError_t hipEventRecord(hipEvent_t e, hipStream_t s) {
    e->stream = s ? s : nullptr;
    e->done = false;
    sqemu::submit(s, [e]() {
        e->t = std::chrono::steady_clock::now();
        e->done = true;
    });
    return hipSuccess;
}
hipError_t hipEventSynchronize(hipEvent_t e) {
    sqemu::drain(e->stream);
    return hipSuccess;
}
hipError_t hipEventElapsedTime(float* ms, hipEvent_t a, hipEvent_t b) {
    if (!a->done || !b->done) return hipErrorNotReady;
    *ms = std::chrono::duration<float, std::milli>(b->t - a->t).count();
    return hipSuccess;
}
hipError_t hipStreamBeginCapture(hipStream_t s, hipStreamCaptureMode) {
    sqemu_stream* st = s ? s : nullptr;
    if (!st || st->capturing) return hipErrorInvalidValue;
    st->capturing = true;
    st->capture = new std::vector<sqemu::Task>();
    return hipSuccess;
}
hipError_t hipStreamEndCapture(hipStream_t s, hipGraph_t* g) {
    if (!s || !s->capturing) return hipErrorInvalidValue;
    s->capturing = false;
    *g = new sqemu_graph{std::move(*s->capture)};
    delete s->capture;
    s->capture = nullptr;
    return hipSuccess;
}
hipError_t hipGraphInstantiate(hipGraphExec_t* e, hipGraph_t g, hipGraphNode_t*, char*, size_t) {
    *e = new sqemu_graph{g->tasks};
    return hipSuccess;
}
hipError_t hipGraphLaunch(hipGraphExec_t e, hipStream_t s) {
    for (auto& t : e->tasks) sqemu::submit(s, t);
    return hipSuccess;
}
hipError_t hipGraphExecDestroy(hipGraphExec_t e) {
    delete e;
    return hipSuccess;
}
hipError_t hipGraphDestroy(hipGraph_t g) {
    delete g;
    return hipSuccess;
}
hipError_t hipGetSymbolAddress(void** p, sqemu_symbol sym) {
    *p = const_cast<void*>(sym.p);
    sqemu::g_dev[(uintptr_t)*p] = sym.bytes;
    return hipSuccess;
}
