// Checks that the CPU emulation catches what it is meant to catch.
// TEST INFRASTRUCTURE ONLY.  `selftest oob` launches a kernel that reads one
// element past a device buffer (the sanitizer must stop it); `selftest
// diverge` calls a cross-lane operation from half a wavefront (the emulator
// must abort); `selftest ok` runs the in-bounds twin and prints the sum.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>

__global__ void read_kernel(const float* x, int n, int extra, float* out) {
    float v = 0.0f;
    for (int i = threadIdx.x; i < n + extra; i += 64) v += x[i];
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
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
    if (!strcmp(what, "diverge")) {
        hipLaunchKernelGGL(diverge_kernel, dim3(1), dim3(64), 0, nullptr, out);
    } else {
        hipLaunchKernelGGL(read_kernel, dim3(1), dim3(64), 0, nullptr, x, n, strcmp(what, "oob") ? 0 : 1, out);
    }
    float r = 0;
    hipMemcpy(&r, out, 4, hipMemcpyDeviceToHost);
    printf("sum %g\n", r);
    return 0;
}
