// Sustained int8 matrix-core throughput of the device: the ceiling the engine's GEMMs are measured
// against besides the published peak. Every wave runs independent v_mfma_i32_16x16x64_i8 chains on
// register operands (no memory traffic but one checksum store per lane), enough waves to fill every
// SIMD several times over.
//
//     hipcc --offload-arch=gfx950 -O3 -std=c++17 -Xclang -target-feature -Xclang -packed-fp32-ops \
//         calib_mfma.hip -o gpurun_out/calib_mfma && gpurun_out/calib_mfma [iterations]
//
// Prints the achieved TOP/s (2 ops per multiply-accumulate) of three timed launches.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

typedef int v4i __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void mfma_chains(int iters, int seed, int* out) {
    const int t = (int)threadIdx.x;
    const v4i a = {seed, seed + 1, seed + 2, t};
    const v4i b = {seed ^ 3, seed + 5, 7, t ^ 9};
    v4i acc[16];
#pragma unroll
    for (int i = 0; i < 16; i++) acc[i] = v4i{0, 0, 0, 0};
    for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int i = 0; i < 16; i++) acc[i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, acc[i], 0, 0, 0);
    }
    int x = 0;
#pragma unroll
    for (int i = 0; i < 16; i++) x ^= acc[i][0] ^ acc[i][1] ^ acc[i][2] ^ acc[i][3];
    out[blockIdx.x * blockDim.x + threadIdx.x] = x;
}

static void check(hipError_t e, const char* what) {
    if (e != hipSuccess) {
        std::fprintf(stderr, "%s: %s\n", what, hipGetErrorString(e));
        std::exit(1);
    }
}

int main(int argc, char** argv) {
    const int iters = argc > 1 ? std::atoi(argv[1]) : 2000;
    if (iters < 1 || iters > 100000) {
        std::fprintf(stderr, "iterations must be in [1, 100000]\n");
        return 1;
    }
    int dev = 0, cus = 0;
    check(hipGetDevice(&dev), "hipGetDevice");
    check(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev), "hipDeviceGetAttribute");
    const int blocks = cus * 8, threads = 256;  // 8 waves per SIMD
    int* out = nullptr;
    check(hipMalloc(&out, (size_t)blocks * threads * sizeof(int)), "hipMalloc");
    hipEvent_t e0, e1;
    check(hipEventCreate(&e0), "hipEventCreate");
    check(hipEventCreate(&e1), "hipEventCreate");
    hipLaunchKernelGGL(mfma_chains, dim3(blocks), dim3(threads), 0, 0, 16, 1, out);
    check(hipGetLastError(), "launch");
    check(hipDeviceSynchronize(), "warm-up");
    const double ops = (double)blocks * (threads / 64) * iters * 16 * (16.0 * 16 * 64 * 2);
    for (int rep = 0; rep < 3; rep++) {
        check(hipEventRecord(e0), "hipEventRecord");
        hipLaunchKernelGGL(mfma_chains, dim3(blocks), dim3(threads), 0, 0, iters, rep, out);
        check(hipGetLastError(), "launch");
        check(hipEventRecord(e1), "hipEventRecord");
        check(hipEventSynchronize(e1), "hipEventSynchronize");
        float ms = 0.0f;
        check(hipEventElapsedTime(&ms, e0, e1), "hipEventElapsedTime");
        std::printf("int8 MFMA (v_mfma_i32_16x16x64_i8), %d CUs: %.3f ms, %.1f TOP/s\n", cus, ms, ops / ms / 1e9);
    }
    check(hipFree(out), "hipFree");
    return 0;
}
