// Checks that the CPU emulation catches what it is meant to catch.
// TEST INFRASTRUCTURE ONLY.  `selftest oob` launches a kernel that reads one
// element past a device buffer (the sanitizer must stop it); `selftest
// diverge` calls a cross-lane operation from half a wavefront (the emulator
// must abort); `selftest host` hands the kernel a host array, `selftest
// hoststruct` a struct holding one, and `selftest freed` replays a captured
// launch whose buffer was freed after the capture (each must be refused);
// `selftest ok` runs the in-bounds twin and prints the sum.
// Stream timing: `selftest pinned` rewrites a pinned source after queuing its
// copy and before synchronizing (the copy must see the rewrite: sum 512);
// `selftest nullstream` reads a non-blocking stream's result with hipMemcpy
// without synchronizing that stream (the read must miss it: sum 256, not 64);
// `selftest synced` is the correct twin of the latter (sum 64).
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>

__global__ void read_kernel(const float* x, int n, int extra, float* out) {
    float v = 0.0f;
    for (int i = threadIdx.x; i < n + extra; i += 64) v += x[i];
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    if (threadIdx.x == 0) *out = v;
}

struct View {
    const float* x;
    int n;
};

__global__ void view_kernel(View v, float* out) {
    if (threadIdx.x == 0) *out = v.x[0] + (float)v.n;
}

__global__ void set_kernel(float* out, float v) {
    if (threadIdx.x == 0) *out = v;
}

__global__ void diverge_kernel(float* out) {
    float v = (float)threadIdx.x;
    if (threadIdx.x < 32) v += __shfl_xor(v, 1, 64);
    out[threadIdx.x] = v;
}

int main(int argc, char** argv) {
    const char* what = argc > 1 ? argv[1] : "ok";
    const int n = 256;
    float *x = nullptr, *out = nullptr;
    hipMalloc(&x, n * sizeof(float));
    hipMalloc(&out, 64 * sizeof(float));
    float h[n];
    for (int i = 0; i < n; i++) h[i] = 1.0f;
    hipMemcpy(x, h, sizeof(h), hipMemcpyHostToDevice);
    if (!strcmp(what, "pinned")) {
        float* hp = nullptr;
        hipHostMalloc(&hp, n * sizeof(float), hipHostMallocDefault);
        for (int i = 0; i < n; i++) hp[i] = 1.0f;
        hipStream_t s;
        hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
        hipMemcpyAsync(x, hp, n * sizeof(float), hipMemcpyHostToDevice, s);
        for (int i = 0; i < n; i++) hp[i] = 2.0f;  // before the copy has run
        hipLaunchKernelGGL(read_kernel, dim3(1), dim3(64), 0, s, x, n, 0, out);
        hipStreamSynchronize(s);
    } else if (!strcmp(what, "nullstream") || !strcmp(what, "synced")) {
        hipLaunchKernelGGL(read_kernel, dim3(1), dim3(64), 0, nullptr, x, n, 0, out);
        hipDeviceSynchronize();
        hipStream_t s;
        hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
        hipLaunchKernelGGL(set_kernel, dim3(1), dim3(64), 0, s, out, 64.0f);
        if (!strcmp(what, "synced")) hipStreamSynchronize(s);
    } else if (!strcmp(what, "diverge")) {
        hipLaunchKernelGGL(diverge_kernel, dim3(1), dim3(64), 0, nullptr, out);
    } else if (!strcmp(what, "host")) {
        hipLaunchKernelGGL(read_kernel, dim3(1), dim3(64), 0, nullptr, (const float*)h, n, 0, out);
    } else if (!strcmp(what, "hoststruct")) {
        hipLaunchKernelGGL(view_kernel, dim3(1), dim3(64), 0, nullptr, View{h, n}, out);
    } else if (!strcmp(what, "freed")) {
        float* tmp = nullptr;
        hipMalloc(&tmp, n * sizeof(float));
        hipMemcpy(tmp, h, sizeof(h), hipMemcpyHostToDevice);
        hipStream_t s;
        hipStreamCreate(&s);
        hipGraph_t g;
        hipGraphExec_t ge;
        hipStreamBeginCapture(s, hipStreamCaptureModeGlobal);
        hipLaunchKernelGGL(read_kernel, dim3(1), dim3(64), 0, s, (const float*)tmp, n, 0, out);
        hipStreamEndCapture(s, &g);
        hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
        hipGraphLaunch(ge, s);  // in bounds: tmp is live
        hipFree(tmp);
        hipGraphLaunch(ge, s);  // tmp was freed
    } else {
        hipLaunchKernelGGL(read_kernel, dim3(1), dim3(64), 0, nullptr, x, n, strcmp(what, "oob") ? 0 : 1, out);
    }
    float r = 0;
    hipMemcpy(&r, out, 4, hipMemcpyDeviceToHost);
    printf("sum %g\n", r);
    return 0;
}
