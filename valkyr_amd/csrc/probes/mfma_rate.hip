// MFMA issue-rate probe: a register-only loop of independent bf16 MFMA
// accumulator chains, one block per CU, 4 or 8 waves per block (one or two
// waves per SIMD), timed with HIP events.  It measures what the matrix cores
// sustain when nothing but MFMAs issue, the ceiling the attention and GEMM
// kernels are compared against.
//   make -C valkyr_amd/csrc probes && ./valkyr_amd/csrc/probes/mfma_rate
#include <hip/hip_runtime.h>
#include <stdio.h>

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

template <int CH, bool BIG>
__global__ void mfma_loop(float *out, int iters) {
    bf16x8 a, b;
    for (int i = 0; i < 8; ++i) {
        a[i] = (__bf16)(threadIdx.x * 0.001f + i);
        b[i] = (__bf16)(i * 0.5f);
    }
    float s = 0;
    if constexpr (!BIG) {
        f32x4 acc[CH];
        for (int c = 0; c < CH; ++c) acc[c] = f32x4{0, 0, 0, 0};
        for (int it = 0; it < iters; ++it)
#pragma unroll
            for (int c = 0; c < CH; ++c) acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[c], 0, 0, 0);
        for (int c = 0; c < CH; ++c) s += acc[c][0] + acc[c][1] + acc[c][2] + acc[c][3];
    } else {
        f32x16 acc[CH];
        for (int c = 0; c < CH; ++c)
            for (int r = 0; r < 16; ++r) acc[c][r] = 0;
        for (int it = 0; it < iters; ++it)
#pragma unroll
            for (int c = 0; c < CH; ++c) acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[c], 0, 0, 0);
        for (int c = 0; c < CH; ++c)
            for (int r = 0; r < 16; ++r) s += acc[c][r];
    }
    out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

#define CHECK(x)                                                                       \
    do {                                                                               \
        hipError_t e_ = (x);                                                           \
        if (e_ != hipSuccess) {                                                        \
            fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));                    \
            return 1;                                                                  \
        }                                                                              \
    } while (0)

template <int CH, bool BIG>
int run(int waves, float *out) {
    const int iters = 4000, reps = 5;
    const dim3 grid(256), block(64 * waves);  // one block per CU
    hipLaunchKernelGGL((mfma_loop<CH, BIG>), grid, block, 0, 0, out, 100);
    CHECK(hipDeviceSynchronize());
    hipEvent_t e0, e1;
    CHECK(hipEventCreate(&e0));
    CHECK(hipEventCreate(&e1));
    CHECK(hipEventRecord(e0));
    for (int r = 0; r < reps; ++r) hipLaunchKernelGGL((mfma_loop<CH, BIG>), grid, block, 0, 0, out, iters);
    CHECK(hipEventRecord(e1));
    CHECK(hipEventSynchronize(e1));
    float ms = 0;
    CHECK(hipEventElapsedTime(&ms, e0, e1));
    const double per = BIG ? 2.0 * 32 * 32 * 16 : 2.0 * 16 * 16 * 32;
    const double flops = (double)reps * 256 * waves * iters * CH * per;
    printf("%s  %2d chains  %d wave(s)/SIMD: %6.0f TFLOP/s\n", BIG ? "32x32x16" : "16x16x32", CH,
           waves / 4, flops / (ms * 1e-3) / 1e12);
    CHECK(hipEventDestroy(e0));
    CHECK(hipEventDestroy(e1));
    return 0;
}

int main() {
    float *out = nullptr;
    CHECK(hipMalloc(&out, 256 * 512 * sizeof(float)));
    for (int w : {4, 8}) {
        if (run<4, false>(w, out) || run<8, false>(w, out) || run<16, false>(w, out) ||
            run<2, true>(w, out) || run<4, true>(w, out))
            return 1;
    }
    CHECK(hipFree(out));
    return 0;
}
