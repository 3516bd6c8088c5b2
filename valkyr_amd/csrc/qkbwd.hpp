// The attention backward's fused q/k gradient epilogue, shared by the bf16
// recompute kernels (k_attn.hip) and the fp32 matrix-core kernels
// (k_attn_f32.hip): dQ / dK rows in the MFMA accumulator layout taken back
// through RoPE and the Q/K-RMSNorm, and the block's gain-gradient partial.
#pragma once

#include "ops.hpp"

namespace vkh {
namespace {

// ── fused q/k gradient epilogue (recompute kernels) ───────────────────
// The recompute kernels end with dQ / dK rows in the accumulator layout: the
// four lanes g = 0..3 of one c16 hold a head row (head_dim 128), lane g its
// elements d = 16 i + 4 g + r in v[i][r].  qk_row_bwd takes such a row back
// through RoPE (rotary_dim = head_dim: pairs d, d + 64 sit in tiles i, i + 4
// of the same lane, both rotated by table column d) and the Q/K-RMSNorm
// (fp64 row sums as in qkv_bwd8_k, combined over the four lanes), and adds
// the row's gain-gradient terms v_rot * ri * x to dw.  Every lane of the
// wave calls it (lane shuffles); `ok` masks rows past the sequence.
VKH_DEV void qk_row_bwd(float (&v)[8][4], float (&dw)[8][4], bool ok, const QkEpi &e,
                        const float *xrow, const float *gain, int pos, int g) {
    if (e.rot) {
        const float2 *tr = e.rope + (long)pos * 64 + 4 * g;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float4 c01 = make_float4(1.f, 0.f, 1.f, 0.f), c23 = c01;
            if (ok) {
                c01 = *reinterpret_cast<const float4 *>(tr + 16 * i);
                c23 = *reinterpret_cast<const float4 *>(tr + 16 * i + 2);
            }
            const float cs[4][2] = {{c01.x, c01.y}, {c01.z, c01.w}, {c23.x, c23.y}, {c23.z, c23.w}};
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float lo = v[i][r], hi = v[i + 4][r];
                v[i][r] = cs[r][0] * lo + cs[r][1] * hi;
                v[i + 4][r] = -cs[r][1] * lo + cs[r][0] * hi;
            }
        }
    }
    if (!gain) return;
    float x[8][4], gw[8][4];
    double ss = 0, A = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float4 xv = ok ? *reinterpret_cast<const float4 *>(xrow + 16 * i + 4 * g)
                             : make_float4(0.f, 0.f, 0.f, 0.f);
        const float4 gv = *reinterpret_cast<const float4 *>(gain + 16 * i + 4 * g);
        x[i][0] = xv.x; x[i][1] = xv.y; x[i][2] = xv.z; x[i][3] = xv.w;
        gw[i][0] = gv.x; gw[i][1] = gv.y; gw[i][2] = gv.z; gw[i][3] = gv.w;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            ss += (double)x[i][r] * (double)x[i][r];
            A += (double)v[i][r] * (double)gw[i][r] * (double)x[i][r];
        }
    }
    ss += __shfl_xor(ss, 16, 64);
    ss += __shfl_xor(ss, 32, 64);
    A += __shfl_xor(A, 16, 64);
    A += __shfl_xor(A, 32, 64);
    const float ri = 1.0f / sqrtf((float)(ss / 128.0) + e.eps);
    const float ri3 = ri * ri * ri / 128.0f;
    const float Af = (float)A;
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            if (ok) dw[i][r] += v[i][r] * ri * x[i][r];
            v[i][r] = ri * gw[i][r] * v[i][r] - ri3 * x[i][r] * Af;
        }
}

// Gain-gradient partial of a block: dw summed over the 16 rows of each lane
// group (a fixed xor tree), then over waves 0..nw-1 in order through `red`
// ([nw][128] floats of LDS); the sum goes to part[0..127].  Every thread of
// the block calls it (barriers); waves with `mine` false only take part in
// the barriers.
VKH_DEV void qk_dw_block(float (&dw)[8][4], float *red, int wave, int nw, bool mine, int lane,
                         float *part) {
    if (mine) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float a = dw[i][r];
                a += __shfl_xor(a, 1, 64);
                a += __shfl_xor(a, 2, 64);
                a += __shfl_xor(a, 4, 64);
                a += __shfl_xor(a, 8, 64);
                dw[i][r] = a;
            }
        if (lane % 16 == 0) {
            const int g = lane / 16;
#pragma unroll
            for (int i = 0; i < 8; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) red[wave * 128 + 16 * i + 4 * g + r] = dw[i][r];
        }
    }
    __syncthreads();
    const int tid = threadIdx.x;
    if (tid < 128) {
        float a = red[tid];
        for (int w = 1; w < nw; ++w) a += red[w * 128 + tid];
        part[tid] = a;
    }
}

}  // namespace
}  // namespace vkh
