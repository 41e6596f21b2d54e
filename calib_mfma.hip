// Sustained int8 matrix-core throughput of the device: the ceiling the engine's GEMMs are measured
// against besides the published peak. Each workgroup is shaped like the weight-stationary GEMM's: 8 waves
// (2 per SIMD), a 144 KiB weight slab in LDS, and per K step each wave reads its eight 1 KiB weight
// fragments from LDS and issues 24 independent v_mfma_i32_16x16x64_i8 against three activation fragments
// in registers (one memory-free K step of the engine's GEMMs), over 18 K steps, in launches of ~15 ms.
// The rate depends on the operand bits (switching activity and with it the clock the part sustains), so
// it is measured twice: weights and activations random (what the engine's GEMMs multiply) and all zero.
//
//     hipcc --offload-arch=gfx950 -O3 -std=c++17 -Xclang -target-feature -Xclang -packed-fp32-ops \
//         calib_mfma.hip -o gpurun_out/calib_mfma && gpurun_out/calib_mfma [iterations]
//
// A third run issues the same work as v_mfma_i32_32x32x32_i8 (each wave 32 tokens x 64 channels x 3
// planes per K step: half the LDS weight bytes and register operand reads per operation), random operands.
//
// Prints the achieved TOP/s (2 ops per multiply-accumulate) of the best of three timed launches per
// operand set.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int KS = 18;  // K steps held in LDS: 144 KiB, one workgroup per CU as in the slab GEMM

__device__ __forceinline__ int mix(unsigned i, unsigned seed) {
    unsigned h = (i + 1u) * 2654435761u ^ seed * 40503u;
    h ^= h >> 13;
    h *= 0x5bd1e995u;
    h ^= h >> 15;
    return (int)h;
}

__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void mfma_steps(int iters, int random,
                                                                                             int* out) {
    extern __shared__ __align__(16) int8_t slab[];
    const int t = (int)threadIdx.x, lane = t & 63;
    for (int i = t; i < KS * 8192 / 4; i += 512) ((int*)slab)[i] = random ? mix(i, 7u) : 0;
    __syncthreads();
    v4i a[3];
#pragma unroll
    for (int l = 0; l < 3; l++)
        a[l] = random ? v4i{mix(4 * t + l, 11u), mix(4 * t + l, 13u), mix(4 * t + l, 17u), mix(4 * t + l, 19u)}
                      : v4i{0, 0, 0, 0};
    v4i acc[3][8];
#pragma unroll
    for (int l = 0; l < 3; l++)
#pragma unroll
        for (int i = 0; i < 8; i++) acc[l][i] = v4i{0, 0, 0, 0};
    for (int it = 0; it < iters; it++) {
        for (int ks = 0; ks < KS; ks++) {
            const int8_t* wp = slab + ks * 8192 + lane * 16;
            v4i wf[8];
#pragma unroll
            for (int i = 0; i < 8; i++) wf[i] = *(const v4i*)(wp + i * 1024);
#pragma unroll
            for (int i = 0; i < 8; i++)
#pragma unroll
                for (int l = 0; l < 3; l++) acc[l][i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf[i], a[l], acc[l][i], 0, 0, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 24, 0);
        }
    }
    int x = 0;
#pragma unroll
    for (int l = 0; l < 3; l++)
#pragma unroll
        for (int i = 0; i < 8; i++) x ^= acc[l][i][0] ^ acc[l][i][1] ^ acc[l][i][2] ^ acc[l][i][3];
    out[blockIdx.x * blockDim.x + threadIdx.x] = x;
}

// The same K steps on the 32x32x32 form: per K step of 64, two 32-deep halves, each two LDS fragment reads
// (64 channels) against three activation fragments: 12 MFMAs of 65536 ops, the work of the 24 above.
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void mfma_steps32(int iters, int* out) {
    extern __shared__ __align__(16) int8_t slab[];
    const int t = (int)threadIdx.x, lane = t & 63;
    for (int i = t; i < KS * 8192 / 4; i += 512) ((int*)slab)[i] = mix(i, 7u);
    __syncthreads();
    v4i a[2][3];
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int l = 0; l < 3; l++) {
            const int k = 8 * t + 3 * h + l;
            a[h][l] = v4i{mix(k, 11u), mix(k, 13u), mix(k, 17u), mix(k, 19u)};
        }
    v16i acc[3][2];
#pragma unroll
    for (int l = 0; l < 3; l++)
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[l][i][r] = 0;
    for (int it = 0; it < iters; it++) {
        for (int ks = 0; ks < KS; ks++) {
            const int8_t* wp = slab + ks * 8192 + lane * 16;
            v4i wf[2][2];
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int i = 0; i < 2; i++) wf[h][i] = *(const v4i*)(wp + (h * 2 + i) * 1024);
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int i = 0; i < 2; i++)
#pragma unroll
                    for (int l = 0; l < 3; l++)
                        acc[l][i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(wf[h][i], a[h][l], acc[l][i], 0, 0, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 12, 0);
        }
    }
    int x = 0;
#pragma unroll
    for (int l = 0; l < 3; l++)
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) x ^= acc[l][i][r];
    out[blockIdx.x * blockDim.x + threadIdx.x] = x;
}

static void check(hipError_t e, const char* what) {
    if (e != hipSuccess) {
        std::fprintf(stderr, "%s: %s\n", what, hipGetErrorString(e));
        std::exit(1);
    }
}

int main(int argc, char** argv) {
    const int iters = argc > 1 ? std::atoi(argv[1]) : 512;
    if (iters < 1 || iters > 100000) {
        std::fprintf(stderr, "iterations must be in [1, 100000]\n");
        return 1;
    }
    int dev = 0, cus = 0;
    check(hipGetDevice(&dev), "hipGetDevice");
    check(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev), "hipDeviceGetAttribute");
    const int blocks = cus * 4, threads = 512;  // four rounds of one workgroup per CU
    const size_t lds = (size_t)KS * 8192;
    check(hipFuncSetAttribute((const void*)mfma_steps, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
          "hipFuncSetAttribute");
    int* out = nullptr;
    check(hipMalloc(&out, (size_t)blocks * threads * sizeof(int)), "hipMalloc");
    hipEvent_t e0, e1;
    check(hipEventCreate(&e0), "hipEventCreate");
    check(hipEventCreate(&e1), "hipEventCreate");
    const double ops = (double)blocks * (threads / 64) * iters * KS * 24 * (16.0 * 16 * 64 * 2);
    for (int random = 1; random >= 0; random--) {
        hipLaunchKernelGGL(mfma_steps, dim3(blocks), dim3(threads), lds, 0, 4, random, out);
        check(hipGetLastError(), "launch");
        check(hipDeviceSynchronize(), "warm-up");
        float best = 1e30f;
        for (int rep = 0; rep < 3; rep++) {
            check(hipEventRecord(e0), "hipEventRecord");
            hipLaunchKernelGGL(mfma_steps, dim3(blocks), dim3(threads), lds, 0, iters, random, out);
            check(hipGetLastError(), "launch");
            check(hipEventRecord(e1), "hipEventRecord");
            check(hipEventSynchronize(e1), "hipEventSynchronize");
            float ms = 0.0f;
            check(hipEventElapsedTime(&ms, e0, e1), "hipEventElapsedTime");
            if (ms < best) best = ms;
        }
        std::printf("int8 MFMA (v_mfma_i32_16x16x64_i8), %d CUs, %s operands: %.3f ms, %.1f TOP/s\n", cus,
                    random ? "random" : "zero", best, ops / best / 1e9);
    }
    check(hipFuncSetAttribute((const void*)mfma_steps32, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
          "hipFuncSetAttribute");
    hipLaunchKernelGGL(mfma_steps32, dim3(blocks), dim3(threads), lds, 0, 4, out);
    check(hipGetLastError(), "launch");
    check(hipDeviceSynchronize(), "warm-up");
    float best = 1e30f;
    for (int rep = 0; rep < 3; rep++) {
        check(hipEventRecord(e0), "hipEventRecord");
        hipLaunchKernelGGL(mfma_steps32, dim3(blocks), dim3(threads), lds, 0, iters, out);
        check(hipGetLastError(), "launch");
        check(hipEventRecord(e1), "hipEventRecord");
        check(hipEventSynchronize(e1), "hipEventSynchronize");
        float ms = 0.0f;
        check(hipEventElapsedTime(&ms, e0, e1), "hipEventElapsedTime");
        if (ms < best) best = ms;
    }
    std::printf("int8 MFMA (v_mfma_i32_32x32x32_i8), %d CUs, random operands: %.3f ms, %.1f TOP/s\n", cus, best,
                ops / best / 1e9);
    check(hipFree(out), "hipFree");
    return 0;
}
