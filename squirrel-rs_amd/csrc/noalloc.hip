// sq_linear_noalloc: the linear operator with no device allocation.
//
// sq_linear allocates its scratch (the Q8_0 activation payload and block
// scales, and the partial tiles of a K split) with hipMalloc on every call.
// Callers that cannot allocate -- tight serving loops, harnesses that forbid
// it -- use this variant: its scratch is one
// file-scope device array, `scratch`, held by each GPU the library runs on
// until the process ends.  The kernels and their launch shapes are
// sq_linear's, with the same K-split workspace size, so both entry points
// give identical results.
//
// The array's host-side name is not a device address: the first call on a
// device (with that device current) looks up the device copy's address with
// hipGetSymbolAddress and keeps it per device; every kernel argument uses
// that address.  Every call on a GPU shares that GPU's array, so calls that
// overlap on one GPU race.  Each call launches on the null stream and
// synchronizes it, so it cannot be recorded under a stream capture.  No part of the scratch
// needs to start at zero: the quantizer writes every activation block it
// produces and a K split writes every partial tile it sums.
#include <mutex>

#include "model.h"

namespace sq {
namespace {

constexpr size_t kActsMax = (size_t)4 << 20;  // m * k activation elements at most (e.g. 2048 x 2048)
constexpr size_t kOffD = kActsMax;             // fp16 block scales after the payload
constexpr size_t kOffWs = kOffD + kActsMax / 16;
constexpr size_t kScratchBytes = kOffWs + kGemmSplitFloats * sizeof(float);  // 20.25 MiB

__device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
uint8_t* g_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device (looked up once per
// device), or null with the error recorded.
uint8_t* scratch_ptr(int* status) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        *status = set_error(SQ_ERR_HIP, std::string("linear_noalloc: hipGetDevice: ") + hipGetErrorString(e));
        return nullptr;
    }
    if (dev < 0 || dev >= kMaxDevices) {
        *status = set_error(SQ_ERR_UNSUPPORTED, "linear_noalloc: device index beyond the supported 64");
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) {
            *status = set_error(SQ_ERR_HIP, std::string("linear_noalloc: hipGetSymbolAddress: ") + hipGetErrorString(e));
            return nullptr;
        }
        g_ptr[dev] = (uint8_t*)p;
    }
    return g_ptr[dev];
}

}  // namespace
}  // namespace sq

using namespace sq;

extern "C" int sq_linear_noalloc(const float* d_in, size_t m, size_t k, const sq_weight* w, float* d_out,
                                 uint32_t flags) {
    if (!w || !d_in || !d_out) return set_error(SQ_ERR_ARG, "linear_noalloc: null argument");
    if (k != (size_t)w->m.k) return set_error(SQ_ERR_SHAPE, "linear_noalloc: ShapeMismatch (in_dim != weight k)");
    if (m == 0) return 0;
    if (w->m.wtype == WT_BF16 || (flags & SQ_CTX_F32_ACTS)) return set_error(SQ_ERR_UNSUPPORTED, kA32Disabled);
    if (m > kActsMax / k)
        return set_error(SQ_ERR_SHAPE, "linear_noalloc: m * k = " + std::to_string(m * k) +
                                           " exceeds the static scratch's " + std::to_string(kActsMax) +
                                           " activation elements; use sq_linear");
    int st = 0;
    uint8_t* base = scratch_ptr(&st);
    if (!base) return st;
    int8_t* aq = (int8_t*)base;
    uint16_t* ad = (uint16_t*)(base + kOffD);
    float* ws = (float*)(base + kOffWs);
    if ((st = launch_quantize_rows(nullptr, d_in, m * k, aq, ad))) return st;
    if (m == 1 && k / 32 <= 256) {
        GemvArgs a{};
        a.w = view(w->m);
        a.n_rows = w->m.rows;
        a.aq = aq;
        a.ad = ad;
        a.x = d_in;
        a.out = d_out;
        st = launch_gemv(nullptr, PRO_Q8, EPI_STORE, true, a, nullptr);
    } else {
        st = launch_gemm(nullptr, view(w->m), w->m.wtype, true, aq, ad, d_in, (int)m, d_out, w->m.rows, false, ws,
                         kGemmSplitFloats);
    }
    if (st) return st;
    const hipError_t e = hipStreamSynchronize(nullptr);
    if (e != hipSuccess) return set_error(SQ_ERR_HIP, std::string("linear_noalloc: ") + hipGetErrorString(e));
    return 0;
}
