// Shared definitions for the gfx950 (CDNA4) kernels of libvkhip.
//
// Everything here is written for one target: wave64, MFMA matrix cores,
// 160 KB LDS per CU.  No portability layers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

typedef __bf16 bf16;
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

#define VKH_DEV __device__ __forceinline__

namespace vkh {

constexpr int kWave = 64;

// fp32 -> bf16, round-to-nearest-even (v_cvt_pk_bf16_f32 on gfx950).
VKH_DEV bf16 to_bf16(float x) { return (bf16)x; }
VKH_DEV float to_f32(bf16 x) { return (float)x; }
VKH_DEV float to_f32(float x) { return x; }

// SwiGLU of one element (swiglu_forward.comp / train_transformer.zig:839-851):
// z sigmoid(z) u with sigmoid(z) = 1 / (1 + e^-z), every operation rounded on
// its own, shared by the standalone kernel and the gate/up GEMM's epilogue so
// both give the same bits.
VKH_DEV float swiglu1(float z, float u) {
#pragma clang fp contract(off)
    const float sig = 1.0f / (1.0f + expf(-z));
    return z * sig * u;
}

VKH_DEV bf16x8 cvt8(float a0, float a1, float a2, float a3, float a4, float a5, float a6,
                    float a7) {
    bf16x8 r;
    r[0] = (bf16)a0; r[1] = (bf16)a1; r[2] = (bf16)a2; r[3] = (bf16)a3;
    r[4] = (bf16)a4; r[5] = (bf16)a5; r[6] = (bf16)a6; r[7] = (bf16)a7;
    return r;
}

VKH_DEV f32x4 mfma16x16x32(const bf16x8 &a, const bf16x8 &b, const f32x4 &c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
VKH_DEV f32x4 mfma16x16x4(float a, float b, const f32x4 &c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Wave-wide reductions (64 lanes) via DPP-friendly shuffles.
VKH_DEV float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
VKH_DEV double wave_sum(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
VKH_DEV float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// Reductions over the 16 lanes of a DPP row (lanes 16 g .. 16 g + 15), the
// lanes that hold one row of an MFMA 16x16 accumulator: quad swaps, then
// the half-row and row mirrors.  Every lane ends with the row's result.
template <int CTRL>
VKH_DEV float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                                 0xf, 0xf, false));
}
VKH_DEV float row16_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));   // quad_perm [1,0,3,2]
    v = fmaxf(v, dpp_f<0x4E>(v));   // quad_perm [2,3,0,1]
    v = fmaxf(v, dpp_f<0x141>(v));  // row_half_mirror
    return fmaxf(v, dpp_f<0x140>(v));  // row_mirror
}
VKH_DEV float row16_sum(float v) {
    v += dpp_f<0xB1>(v);
    v += dpp_f<0x4E>(v);
    v += dpp_f<0x141>(v);
    return v + dpp_f<0x140>(v);
}

// Block-wide sum for blockDim.x == NT (multiple of 64). `sh` needs NT/64 floats.
template <int NT>
VKH_DEV float block_sum(float v, float *sh) {
    v = wave_sum(v);
    const int w = threadIdx.x / kWave, l = threadIdx.x % kWave;
    __syncthreads();
    if (l == 0) sh[w] = v;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < NT / kWave; ++i) t += sh[i];
    return t;
}

inline unsigned ceil_div(size_t a, size_t b) { return (unsigned)((a + b - 1) / b); }

// Causal grids with row 0 the heaviest: the block row of grid row y (of n)
// when the whole grid is resident at once with two blocks per CU.  The first
// half of the rows goes heaviest first and the second half lightest first, so
// blocks y and y + n / 2, which the in-order dispatch places on one CU, carry
// about equal work together.  (A grid larger than the resident slots keeps
// heaviest-first order: blocks then start as CUs free up.)
VKH_DEV int zigzag(int y, int n) {
    const int h = n / 2;
    return y < h ? y : n - 1 - (y - h);
}
// Compute units of the current device (cached per device).
int cu_count();
// Whether a grid of `blocks` fits the device's CUs at two blocks each.
inline bool fits_two_per_cu(long blocks) { return blocks <= 2L * cu_count(); }

}  // namespace vkh
