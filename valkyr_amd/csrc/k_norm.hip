// RMSNorm forward/backward and the Q/K-norm + RoPE kernels.
//
// rmsnorm.comp / rmsnorm_backward.comp restated with two changes:
//   * the gain gradient is reduced on the GPU (per-block partial sums, then a
//     fixed-order column sum) instead of per-row partials read back and summed
//     on the host (transformer.zig:2151-2191);
//   * the residual add that follows each backward norm in the layer
//     (add_in_place.comp at transformer.zig:1992, :2069) is fused into dx.
// Row reductions accumulate in fp64 like the CPU oracle
// (train_transformer.zig:88-99), and fp contraction is off so the per-element
// fp32 formulas round exactly as written.
//
// Layout on the GPU: one wave owns one row (RMSNorm) or one (row, head)
// (Q/K norm + RoPE).  Each lane holds contiguous vector chunks of the row, the
// row reductions are wave shuffles (no block barriers in the row loop), and
// the RoPE partner element (i <-> i +- rotary_dim/2) comes from a lane
// shuffle.  Gain gradients stay in registers across a wave's rows and are
// combined per block in a fixed order.
#include <algorithm>
#include <type_traits>

#include "ops.hpp"
#include "qkv8.hpp"

#pragma clang fp contract(off)

namespace vkh {

namespace {

constexpr int NT = 256;
constexpr int NW = NT / 64;

template <typename TO>
VKH_DEV void store4(TO *p, float a, float b, float c, float d);
template <>
VKH_DEV void store4<float>(float *p, float a, float b, float c, float d) {
    *reinterpret_cast<float4 *>(p) = make_float4(a, b, c, d);
}
template <>
VKH_DEV void store4<bf16>(bf16 *p, float a, float b, float c, float d) {
    bf16x4 v;
    v[0] = (bf16)a; v[1] = (bf16)b; v[2] = (bf16)c; v[3] = (bf16)d;
    *reinterpret_cast<bf16x4 *>(p) = v;
}

// ── RMSNorm: one wave per row, lane l holds columns 4 l + 256 j ─────────

// C4 = float4 chunks per lane (dim <= 256 * C4)
// Sum over the 64 lanes of a wave: DPP row sums, then the four row results
// combined in a fixed order (no LDS round trips, unlike shuffles).
VKH_DEV double wave_sum_dpp(double v) {
    v = grp_sum<16>(v);
    const long long b = __builtin_bit_cast(long long, v);
    double r[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)b, 16 * k);
        const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(b >> 32), 16 * k);
        r[k] = __builtin_bit_cast(double, ((long long)hi << 32) | (long long)lo);
    }
    return (r[0] + r[1]) + (r[2] + r[3]);
}

template <typename TO, int C4>
__global__ __launch_bounds__(NT) void rmsnorm_fwd_k(const float *x, const float *w, TO *y, int rows,
                                                     int dim, float eps, int gq) {
    const int lane = threadIdx.x % 64;
    const int nw = gridDim.x * NW;
    for (int row = blockIdx.x * NW + threadIdx.x / 64; row < rows; row += nw) {
        const float *xr = x + (long)row * dim;
        float4 xv[C4];
        double ss = 0;
#pragma unroll
        for (int j = 0; j < C4; ++j) {
            const int c = 4 * lane + 256 * j;
            xv[j] = c < dim ? *reinterpret_cast<const float4 *>(xr + c) : make_float4(0.f, 0.f, 0.f, 0.f);
            ss += (double)xv[j].x * (double)xv[j].x;
            ss += (double)xv[j].y * (double)xv[j].y;
            ss += (double)xv[j].z * (double)xv[j].z;
            ss += (double)xv[j].w * (double)xv[j].w;
        }
        ss = wave_sum_dpp(ss);
        const double m = ss / (double)dim;
        const float ri = 1.0f / sqrtf((float)m + eps);
#pragma unroll
        for (int j = 0; j < C4; ++j) {
            const int c = 4 * lane + 256 * j;
            if (c >= dim) continue;
            float4 g = *reinterpret_cast<const float4 *>(w + c);
            if (gq) g = make_float4(g.x + 1.0f, g.y + 1.0f, g.z + 1.0f, g.w + 1.0f);
            store4<TO>(y + (long)row * dim + c, g.x * ri * xv[j].x, g.y * ri * xv[j].y,
                       g.z * ri * xv[j].z, g.w * ri * xv[j].w);
        }
    }
}

// dxb (optional): bf16 copy of dx, the operand of the next GEMMs.
// partial[blockIdx.x][dim]: this block's gain-gradient sum over its rows.
template <int C4>
__global__ __launch_bounds__(NT) void rmsnorm_bwd_k(const float *dy, const float *x,
                                                     const float *w, float *dx, bf16 *dxb,
                                                     const float *res, float *partial, int rows,
                                                     int dim, float eps, int gq) {
    __shared__ float4 red[NW][64 * C4];
    const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
    const int nw = gridDim.x * NW;
    float4 gain[C4], dwa[C4];
#pragma unroll
    for (int j = 0; j < C4; ++j) {
        const int c = 4 * lane + 256 * j;
        gain[j] = c < dim ? *reinterpret_cast<const float4 *>(w + c) : make_float4(0.f, 0.f, 0.f, 0.f);
        if (gq) gain[j] = make_float4(gain[j].x + 1.0f, gain[j].y + 1.0f, gain[j].z + 1.0f, gain[j].w + 1.0f);
        dwa[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    const float ri3_div = (float)dim;
    for (int row = blockIdx.x * NW + wave; row < rows; row += nw) {
        const long ro = (long)row * dim;
        float4 xv[C4], dv[C4], rv[C4];
        double ss = 0, A = 0;
#pragma unroll
        for (int j = 0; j < C4; ++j) {
            const int c = 4 * lane + 256 * j;
            const bool ok = c < dim;
            xv[j] = ok ? *reinterpret_cast<const float4 *>(x + ro + c) : make_float4(0.f, 0.f, 0.f, 0.f);
            dv[j] = ok ? *reinterpret_cast<const float4 *>(dy + ro + c) : make_float4(0.f, 0.f, 0.f, 0.f);
            rv[j] = (ok && res) ? *reinterpret_cast<const float4 *>(res + ro + c) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int j = 0; j < C4; ++j) {
            const float xs[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
            const float ds[4] = {dv[j].x, dv[j].y, dv[j].z, dv[j].w};
            const float gs[4] = {gain[j].x, gain[j].y, gain[j].z, gain[j].w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const double xd = xs[q];
                ss += xd * xd;
                A += (double)ds[q] * (double)gs[q] * xd;
            }
        }
        ss = wave_sum_dpp(ss);
        A = wave_sum_dpp(A);
        const double m = ss / (double)dim;
        const float ri = 1.0f / sqrtf((float)m + eps);
        const float ri3_over_D = ri * ri * ri / ri3_div;
        const float A_f = (float)A;
#pragma unroll
        for (int j = 0; j < C4; ++j) {
            const int c = 4 * lane + 256 * j;
            if (c >= dim) continue;
            const float xs[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
            const float ds[4] = {dv[j].x, dv[j].y, dv[j].z, dv[j].w};
            const float gs[4] = {gain[j].x, gain[j].y, gain[j].z, gain[j].w};
            float o[4], dw[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                o[q] = ri * gs[q] * ds[q] - ri3_over_D * xs[q] * A_f;
                dw[q] = ds[q] * ri * xs[q];
            }
            if (res) {
                const float4 r = rv[j];
                o[0] = o[0] + r.x; o[1] = o[1] + r.y; o[2] = o[2] + r.z; o[3] = o[3] + r.w;
            }
            store4<float>(dx + ro + c, o[0], o[1], o[2], o[3]);
            if (dxb) store4<bf16>(dxb + ro + c, o[0], o[1], o[2], o[3]);
            dwa[j].x += dw[0]; dwa[j].y += dw[1]; dwa[j].z += dw[2]; dwa[j].w += dw[3];
        }
    }
    // combine the waves' gain partials in a fixed order, ((w0 + w1) + w2) + w3,
    // after one barrier: each wave leaves its sums in its own LDS slot
#pragma unroll
    for (int j = 0; j < C4; ++j) red[wave][64 * j + lane] = dwa[j];
    __syncthreads();
    for (int i = threadIdx.x; i < 64 * C4; i += NT) {
        const int c = 4 * (i % 64) + 256 * (i / 64);
        if (c >= dim) continue;
        const float4 a = red[0][i], b = red[1][i], e = red[2][i], d = red[3][i];
        *reinterpret_cast<float4 *>(partial + (long)blockIdx.x * dim + c) =
            make_float4(((a.x + b.x) + e.x) + d.x, ((a.y + b.y) + e.y) + d.y,
                        ((a.z + b.z) + e.z) + d.z, ((a.w + b.w) + e.w) + d.w);
    }
}

// Wide rows (dim > 2048): one row per block iteration instead of one per
// wave, so a thread holds 4 columns per 1024 (C4B <= 4 float4 of x, dy,
// residual, gain and gain-gradient sum) rather than 16 float4 of each, which
// left one wave per SIMD and spilled.  The row sums (fp64) are combined over
// the block's four waves in a fixed order through LDS (double-buffered by row
// parity, one barrier per row); each thread's columns' gain sums are its own,
// so the block's partial row needs no reduction.  Same grid as rmsnorm_bwd_k
// (the partial-row count the consumers use).
template <int C4B>
__global__ __launch_bounds__(NT) void rmsnorm_bwd_row_k(const float *dy, const float *x,
                                                         const float *w, float *dx, bf16 *dxb,
                                                         const float *res, float *partial,
                                                         int rows, int dim, float eps, int gq) {
    __shared__ double sred[2][2][NW];
    const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
    float4 gain[C4B], dwa[C4B];
#pragma unroll
    for (int j = 0; j < C4B; ++j) {
        const int c = 4 * threadIdx.x + 1024 * j;
        gain[j] = c < dim ? *reinterpret_cast<const float4 *>(w + c) : make_float4(0.f, 0.f, 0.f, 0.f);
        if (gq) gain[j] = make_float4(gain[j].x + 1.0f, gain[j].y + 1.0f, gain[j].z + 1.0f, gain[j].w + 1.0f);
        dwa[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    const float ri3_div = (float)dim;
    int par = 0;
    for (int row = blockIdx.x; row < rows; row += gridDim.x, par ^= 1) {
        const long ro = (long)row * dim;
        float4 xv[C4B], dv[C4B], rv[C4B];
        double ss = 0, A = 0;
#pragma unroll
        for (int j = 0; j < C4B; ++j) {
            const int c = 4 * threadIdx.x + 1024 * j;
            const bool ok = c < dim;
            xv[j] = ok ? *reinterpret_cast<const float4 *>(x + ro + c) : make_float4(0.f, 0.f, 0.f, 0.f);
            dv[j] = ok ? *reinterpret_cast<const float4 *>(dy + ro + c) : make_float4(0.f, 0.f, 0.f, 0.f);
            rv[j] = (ok && res) ? *reinterpret_cast<const float4 *>(res + ro + c) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int j = 0; j < C4B; ++j) {
            const float xs[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
            const float ds[4] = {dv[j].x, dv[j].y, dv[j].z, dv[j].w};
            const float gs[4] = {gain[j].x, gain[j].y, gain[j].z, gain[j].w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const double xd = xs[q];
                ss += xd * xd;
                A += (double)ds[q] * (double)gs[q] * xd;
            }
        }
        ss = wave_sum_dpp(ss);
        A = wave_sum_dpp(A);
        if (lane == 0) {
            sred[par][0][wave] = ss;
            sred[par][1][wave] = A;
        }
        __syncthreads();
        ss = ((sred[par][0][0] + sred[par][0][1]) + sred[par][0][2]) + sred[par][0][3];
        A = ((sred[par][1][0] + sred[par][1][1]) + sred[par][1][2]) + sred[par][1][3];
        const double m = ss / (double)dim;
        const float ri = 1.0f / sqrtf((float)m + eps);
        const float ri3_over_D = ri * ri * ri / ri3_div;
        const float A_f = (float)A;
#pragma unroll
        for (int j = 0; j < C4B; ++j) {
            const int c = 4 * threadIdx.x + 1024 * j;
            if (c >= dim) continue;
            const float xs[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
            const float ds[4] = {dv[j].x, dv[j].y, dv[j].z, dv[j].w};
            const float gs[4] = {gain[j].x, gain[j].y, gain[j].z, gain[j].w};
            float o[4], dw[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                o[q] = ri * gs[q] * ds[q] - ri3_over_D * xs[q] * A_f;
                dw[q] = ds[q] * ri * xs[q];
            }
            if (res) {
                const float4 r = rv[j];
                o[0] = o[0] + r.x; o[1] = o[1] + r.y; o[2] = o[2] + r.z; o[3] = o[3] + r.w;
            }
            store4<float>(dx + ro + c, o[0], o[1], o[2], o[3]);
            if (dxb) store4<bf16>(dxb + ro + c, o[0], o[1], o[2], o[3]);
            dwa[j].x += dw[0]; dwa[j].y += dw[1]; dwa[j].z += dw[2]; dwa[j].w += dw[3];
        }
    }
#pragma unroll
    for (int j = 0; j < C4B; ++j) {
        const int c = 4 * threadIdx.x + 1024 * j;
        if (c < dim) *reinterpret_cast<float4 *>(partial + (long)blockIdx.x * dim + c) = dwa[j];
    }
}

// out[c] = sum_b partial[b * stride + c].  A block owns 16 columns; its 16
// row groups each sum a strided subset of the partial rows with four
// independent accumulators, then the groups are combined in LDS in a fixed
// order, so the result does not depend on scheduling.
constexpr int CS_COLS = 16, CS_GROUPS = 16;
__global__ __launch_bounds__(CS_COLS *CS_GROUPS) void colsum_k(const float *partial, int nparts,
                                                              long stride, int dim, float *out) {
    __shared__ float sh[CS_GROUPS][CS_COLS + 1];
    const int cl = threadIdx.x % CS_COLS, g = threadIdx.x / CS_COLS;
    const int c = blockIdx.x * CS_COLS + cl;
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
    if (c < dim) {
        int b = g;
        for (; b + 3 * CS_GROUPS < nparts; b += 4 * CS_GROUPS) {
            a0 += partial[(long)b * stride + c];
            a1 += partial[(long)(b + CS_GROUPS) * stride + c];
            a2 += partial[(long)(b + 2 * CS_GROUPS) * stride + c];
            a3 += partial[(long)(b + 3 * CS_GROUPS) * stride + c];
        }
        for (; b < nparts; b += CS_GROUPS) a0 += partial[(long)b * stride + c];
    }
    sh[g][cl] = (a0 + a1) + (a2 + a3);
    __syncthreads();
    if (g == 0 && c < dim) {
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < CS_GROUPS; ++i) s += sh[i][cl];
        out[c] = s;
    }
}

// ── RoPE ─────────────────────────────────────────────────────────────

// qk_rope_partial_batched.comp / qk_rope_backward_batched.comp with the
// cos/sin of (position, pair) taken from a table built by the same fp32
// formula (position p = row % seq_len).
// Scalar form for rows or rotary widths that are not multiples of 4.
// One thread per (row, head, 4-element group of the rotary half) and per
// 4-element group of the non-rotary tail: the pair (i, i + half) is loaded
// once (two float4) and both rotated outputs are written, so every element
// is read from memory once; the cos / sin of the row's position come from
// the table (L2).  32-bit index arithmetic over the flattened work.
__global__ __launch_bounds__(NT) void qk_rope_pair_k(const float *q_in, long ldq_in, float *q_out,
                                                     long ldq_out, const float *k_in, long ldk_in,
                                                     float *k_out, long ldk_out, int n_rows, int hq,
                                                     int hkv, int hd, int rot, int seq_len,
                                                     const float2 *tab, int backward) {
    const int half = rot / 2, npair = half / 4, per_head = npair + (hd - rot) / 4;
    const int heads = hq + hkv, total = n_rows * heads * per_head;
    for (int u = blockIdx.x * NT + threadIdx.x; u < total; u += gridDim.x * NT) {
        const int k = u % per_head, rh = u / per_head, h = rh % heads, p = rh / heads;
        const bool is_q = h < hq;
        const float *in = (is_q ? q_in + (long)p * ldq_in : k_in + (long)p * ldk_in) +
                          (is_q ? h : h - hq) * hd;
        float *out = (is_q ? q_out + (long)p * ldq_out : k_out + (long)p * ldk_out) +
                     (is_q ? h : h - hq) * hd;
        if (k >= npair) {  // beyond the rotary span: copied
            const int i = rot + 4 * (k - npair);
            __builtin_nontemporal_store(__builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(in + i)),
                                        reinterpret_cast<f32x4 *>(out + i));
            continue;
        }
        const int i = 4 * k;
        // streamed once: non-temporal, so the table keeps its place in the caches
        const f32x4 lo = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(in + i));
        const f32x4 hi = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(in + i + half));
        const float2 *tr = tab + (long)(p % seq_len) * half + i;
        const float4 c01 = *reinterpret_cast<const float4 *>(tr);
        const float4 c23 = *reinterpret_cast<const float4 *>(tr + 2);
        const float xl[4] = {lo[0], lo[1], lo[2], lo[3]}, xh[4] = {hi[0], hi[1], hi[2], hi[3]};
        const float cs[4] = {c01.x, c01.z, c23.x, c23.z}, sn[4] = {c01.y, c01.w, c23.y, c23.w};
        float ol[4], oh[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            if (!backward) {
                ol[e] = xl[e] * cs[e] - xh[e] * sn[e];
                oh[e] = xl[e] * sn[e] + xh[e] * cs[e];
            } else {
                ol[e] = cs[e] * xl[e] + sn[e] * xh[e];
                oh[e] = -sn[e] * xl[e] + cs[e] * xh[e];
            }
        }
        __builtin_nontemporal_store(f32x4{ol[0], ol[1], ol[2], ol[3]}, reinterpret_cast<f32x4 *>(out + i));
        __builtin_nontemporal_store(f32x4{oh[0], oh[1], oh[2], oh[3]},
                                    reinterpret_cast<f32x4 *>(out + i + half));
    }
}

__global__ void qk_rope_k(const float *q_in, long ldq_in, float *q_out, long ldq_out,
                          const float *k_in, long ldk_in, float *k_out, long ldk_out, int n_rows,
                          int hq, int hkv, int hd, int rot, int seq_len, const float2 *tab,
                          int backward) {
    const long total = (long)n_rows * (hq + hkv) * hd;
    const long stride = (long)gridDim.x * blockDim.x;
    const int half = rot / 2;
    for (long g = blockIdx.x * (long)blockDim.x + threadIdx.x; g < total; g += stride) {
        const int ht = (hq + hkv) * hd;
        const int p = (int)(g / ht);
        const int within = (int)(g % ht);
        const int h = within / hd, i = within % hd;
        const bool is_q = h < hq;
        const int hl = is_q ? h : h - hq;
        const float *in = is_q ? q_in + p * ldq_in : k_in + p * ldk_in;
        float *out = is_q ? q_out + p * ldq_out : k_out + p * ldk_out;
        const int off = hl * hd;
        if (i >= rot) {
            out[off + i] = in[off + i];
            continue;
        }
        const int j = i < half ? i : i - half;
        const float2 cs = tab[(long)(p % seq_len) * half + j];
        const float a = in[off + j], b = in[off + j + half];
        float o;
        if (!backward) o = (i < half) ? a * cs.x - b * cs.y : a * cs.y + b * cs.x;
        else o = (i < half) ? cs.x * a + cs.y * b : -cs.y * a + cs.x * b;
        out[off + i] = o;
    }
}

// ── fused per-head Q/K RMSNorm + RoPE (+ operand cast) ───────────────

// One wave per (row, head); lane l holds elements EPL l .. EPL l + EPL - 1
// of the head (EPL = 1, 2, 4 for head_dim <= 64, 128, 256).
template <int EPL>
VKH_DEV void ld_epl(const float *p, float (&v)[EPL], bool ok) {
    if (!ok) {
#pragma unroll
        for (int i = 0; i < EPL; ++i) v[i] = 0.f;
        return;
    }
    if constexpr (EPL == 4) {
        const float4 t = *reinterpret_cast<const float4 *>(p);
        v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
    } else if constexpr (EPL == 2) {
        const float2 t = *reinterpret_cast<const float2 *>(p);
        v[0] = t.x; v[1] = t.y;
    } else {
        v[0] = *p;
    }
}

template <typename TO, int EPL>
VKH_DEV void st_epl(TO *p, const float (&v)[EPL]) {
    if constexpr (EPL == 4) {
        store4<TO>(p, v[0], v[1], v[2], v[3]);
    } else {
#pragma unroll
        for (int i = 0; i < EPL; ++i) p[i] = (TO)v[i];
    }
}

// pv[i] = the head's element j(e) = e < half ? e + half : e - half, e = EPL lane + i
template <int EPL>
VKH_DEV void rope_partner(const float (&v)[EPL], float (&pv)[EPL], int lane, int half) {
    if (half % EPL == 0) {
        const int e0 = EPL * lane;
        int src = (e0 < half ? e0 + half : e0 - half) / EPL;
        src = src < 0 ? 0 : (src > 63 ? 63 : src);
#pragma unroll
        for (int i = 0; i < EPL; ++i) pv[i] = __shfl(v[i], src, 64);
    } else {
#pragma unroll
        for (int i = 0; i < EPL; ++i) {
            const int e = EPL * lane + i;
            const int j = e < half ? e + half : e - half;
            int src = j / EPL;
            src = src < 0 ? 0 : (src > 63 ? 63 : src);
            const int si = j - src * EPL;
            float r = 0.f;
#pragma unroll
            for (int i2 = 0; i2 < EPL; ++i2) {
                const float t = __shfl(v[i2], src, 64);
                if (si == i2) r = t;
            }
            pv[i] = r;
        }
    }
}

// The per-item inputs of a wave: the head's values, the pre-norm q/k (for
// the backward's norm) and the RoPE (cos, sin) of each lane's elements.
template <int EPL>
struct HeadItem {
    float v[EPL], x[EPL];
    float2 cs[EPL];
};

template <int EPL>
VKH_DEV void load_item(HeadItem<EPL> &it, const float *vp, const float *xp, const float2 *tr,
                       int e0, int rot, int half, bool on, bool qk) {
    ld_epl<EPL>(vp, it.v, on);
    ld_epl<EPL>(xp, it.x, on && xp != nullptr);
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
        const int e = e0 + i;
        it.cs[i] = (qk && e < rot) ? tr[e < half ? e : e - half] : make_float2(1.f, 0.f);
    }
}

// Forward: normalised and rotated q, k plus v, written as attention operands
// of type TO.  Items are (row, head) over the q, k and v heads; each wave
// prefetches its next item while it finishes the current one.
template <typename TO, int EPL>
__global__ __launch_bounds__(NT) void qkv_fwd_k(QkvLayout L, const float *qkv, long ld_qkv,
                                                 const float *wq, const float *wk, TO *out,
                                                 long ld_out, const float2 *tab) {
    const int lane = threadIdx.x % 64;
    const int hd = L.head_dim, Hqk = L.n_q_heads + L.n_kv_heads, Htot = Hqk + L.n_kv_heads;
    const int half = L.rotary_dim / 2, rot = L.rotary_dim;
    const long items = (long)L.n_rows * Htot;
    const long nw = (long)gridDim.x * NW;
    const int e0 = EPL * lane;
    const bool on = e0 < hd;
    float gq[EPL], gk[EPL];
    ld_epl<EPL>(wq + e0, gq, on && L.qk_norm);
    ld_epl<EPL>(wk + e0, gk, on && L.qk_norm);
    auto fetch = [&](long it, HeadItem<EPL> &d) {
        const int t = (int)(it / Htot), h = (int)(it % Htot);
        load_item<EPL>(d, qkv + (long)t * ld_qkv + h * hd + e0, nullptr,
                       tab + (long)(t % L.seq_len) * half, e0, rot, half, on, h < Hqk);
    };
    long it = (long)blockIdx.x * NW + threadIdx.x / 64;
    HeadItem<EPL> cur;
    if (it < items) fetch(it, cur);
    for (; it < items; it += nw) {
        HeadItem<EPL> nxt;
        if (it + nw < items) fetch(it + nw, nxt);
        const int t = (int)(it / Htot), h = (int)(it % Htot);
        float y[EPL];
#pragma unroll
        for (int i = 0; i < EPL; ++i) y[i] = cur.v[i];
        if (h < Hqk) {
            if (L.qk_norm) {
                const bool is_q = h < L.n_q_heads;
                double ss = 0;
#pragma unroll
                for (int i = 0; i < EPL; ++i) ss += (double)y[i] * (double)y[i];
                ss = wave_sum(ss);
                const float ri = 1.0f / sqrtf((float)(ss / (double)hd) + L.eps);
#pragma unroll
                for (int i = 0; i < EPL; ++i) y[i] = (is_q ? gq[i] : gk[i]) * ri * y[i];
            }
            if (rot > 0) {
                float pv[EPL];
                rope_partner<EPL>(y, pv, lane, half);
#pragma unroll
                for (int i = 0; i < EPL; ++i) {
                    const int e = e0 + i;
                    if (e >= rot) continue;
                    const float2 cs = cur.cs[i];
                    y[i] = e < half ? y[i] * cs.x - pv[i] * cs.y : pv[i] * cs.y + y[i] * cs.x;
                }
            }
        }
        if (on) st_epl<TO, EPL>(out + (long)t * ld_out + h * hd + e0, y);
        cur = nxt;
    }
}

// Backward on the fused d_qkv buffer:
//   dn = rope^T(g);  d_pre = rmsnorm_bw(dn; x = pre-norm q/k);  dw += dn*ri*x
// outb (optional): the results go to this bf16 copy of the whole row (q, k
// and the untouched v columns) instead of back into dqkv.
template <int EPL>
__global__ __launch_bounds__(NT) void qkv_bwd_k(QkvLayout L, float *dqkv, long ld,
                                                 const float *qkv, long ld_qkv, const float *wq,
                                                 const float *wk, float *partial,
                                                 const float2 *tab, bf16 *outb, long ldb) {
    __shared__ float red[2][256];
    const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
    const int hd = L.head_dim, Hqk = L.n_q_heads + L.n_kv_heads;
    const int Htot = outb ? Hqk + L.n_kv_heads : Hqk;
    const int half = L.rotary_dim / 2, rot = L.rotary_dim;
    const long items = (long)L.n_rows * Htot;
    const long nw = (long)gridDim.x * NW;
    const int e0 = EPL * lane;
    const bool on = e0 < hd;
    float gq[EPL], gk[EPL], dwq[EPL], dwk[EPL];
    ld_epl<EPL>(wq + e0, gq, on && L.qk_norm);
    ld_epl<EPL>(wk + e0, gk, on && L.qk_norm);
#pragma unroll
    for (int i = 0; i < EPL; ++i) dwq[i] = dwk[i] = 0.f;
    auto fetch = [&](long it, HeadItem<EPL> &d) {
        const int t = (int)(it / Htot), h = (int)(it % Htot);
        const bool qk = h < Hqk;
        load_item<EPL>(d, dqkv + (long)t * ld + h * hd + e0,
                       (qk && L.qk_norm) ? qkv + (long)t * ld_qkv + h * hd + e0 : nullptr,
                       tab + (long)(t % L.seq_len) * half, e0, rot, half, on, qk);
    };
    long it = (long)blockIdx.x * NW + wave;
    HeadItem<EPL> cur;
    if (it < items) fetch(it, cur);
    for (; it < items; it += nw) {
        HeadItem<EPL> nxt;
        if (it + nw < items) fetch(it + nw, nxt);
        const int t = (int)(it / Htot), h = (int)(it % Htot);
        float gv[EPL];
#pragma unroll
        for (int i = 0; i < EPL; ++i) gv[i] = cur.v[i];
        if (h < Hqk) {
            const bool is_q = h < L.n_q_heads;
            if (rot > 0) {
                float pv[EPL];
                rope_partner<EPL>(gv, pv, lane, half);
#pragma unroll
                for (int i = 0; i < EPL; ++i) {
                    const int e = e0 + i;
                    if (e >= rot) continue;
                    const float2 cs = cur.cs[i];
                    gv[i] = e < half ? cs.x * gv[i] + cs.y * pv[i] : -cs.y * pv[i] + cs.x * gv[i];
                }
            }
            if (L.qk_norm) {
                double ss = 0, A = 0;
#pragma unroll
                for (int i = 0; i < EPL; ++i) {
                    const float gw = is_q ? gq[i] : gk[i];
                    ss += (double)cur.x[i] * (double)cur.x[i];
                    A += (double)gv[i] * (double)gw * (double)cur.x[i];
                }
                ss = wave_sum(ss);
                A = wave_sum(A);
                const float ri = 1.0f / sqrtf((float)(ss / (double)hd) + L.eps);
                const float ri3_over_D = ri * ri * ri / (float)hd;
                const float A_f = (float)A;
#pragma unroll
                for (int i = 0; i < EPL; ++i) {
                    const float gw = is_q ? gq[i] : gk[i];
                    const float o = ri * gw * gv[i] - ri3_over_D * cur.x[i] * A_f;
                    const float dwv = gv[i] * ri * cur.x[i];
                    if (is_q) dwq[i] += dwv; else dwk[i] += dwv;
                    gv[i] = o;
                }
            }
        }
        if (on) {
            if (outb) st_epl<bf16, EPL>(outb + (long)t * ldb + h * hd + e0, gv);
            else if (h < Hqk) st_epl<float, EPL>(dqkv + (long)t * ld + h * hd + e0, gv);
        }
        cur = nxt;
    }
    // combine the waves' gain partials in a fixed order
    for (int wv = 0; wv < NW; ++wv) {
        if (wave == wv && on) {
#pragma unroll
            for (int i = 0; i < EPL; ++i) {
                red[0][e0 + i] = wv ? red[0][e0 + i] + dwq[i] : dwq[i];
                red[1][e0 + i] = wv ? red[1][e0 + i] + dwk[i] : dwk[i];
            }
        }
        __syncthreads();
    }
    for (int c = threadIdx.x; c < 2 * hd; c += NT)
        partial[(long)blockIdx.x * 2 * hd + c] = red[c / hd][c % hd];
}

// ── Q/K norm + RoPE, several heads per wave ─────────────────────────────
// For head_dim 64 / 128 a head is LPH = 8 / 16 lanes holding 8 consecutive
// elements each, so one wave works on 64 / LPH (row, head) items at once.
// The per-head reductions stay inside a DPP row (quad swaps, half-row and row
// mirrors, fp64 like the wave-per-head kernels above) and, for full-width
// RoPE at LPH = 16, the partner element i +- 64 sits in lane j ^ 8 of the
// same row (row rotate by 8).  Requires rotary_dim % 16 == 0 so a lane's 8
// elements are all on one side of the rotation.

template <typename TO, int LPH>
__global__ __launch_bounds__(NT) void qkv_fwd8_k(QkvLayout L, const float *qkv, long ld_qkv,
                                                  const float *wq, const float *wk, TO *out,
                                                  long ld_out, const float2 *tab) {
    constexpr int G = 64 / LPH;
    const int lane = threadIdx.x % 64, j = lane % LPH, g = lane / LPH;
    const int hd = L.head_dim, Hqk = L.n_q_heads + L.n_kv_heads, Htot = Hqk + L.n_kv_heads;
    const int half = L.rotary_dim / 2;
    const long items = (long)L.n_rows * Htot;
    const long stride = (long)gridDim.x * NW * G;
    const Rope8 rp = rope8(j, half);
    float gq[8], gk[8];
    if (L.qk_norm) {
        ld8(wq + 8 * j, gq);
        ld8(wk + 8 * j, gk);
    }
    auto fetch = [&](long it, Item8 &d) {
        const int t = (int)(it / Htot), h = (int)(it % Htot);
        load8<LPH>(d, qkv + (long)t * ld_qkv + h * hd + 8 * j, nullptr,
                   tab + (long)(t % L.seq_len) * half, rp, it < items, h < Hqk);
    };
    long it = ((long)blockIdx.x * NW + threadIdx.x / 64) * G + g;
    const long wave_first = it - g;
    Item8 cur;
    fetch(it, cur);
    for (long wb = wave_first; wb < items; wb += stride, it += stride) {
        Item8 nxt;
        if (wb + stride < items) fetch(it + stride, nxt);
        const bool valid = it < items;
        const int t = (int)(it / Htot), h = (int)(it % Htot);
        const bool qk = valid && h < Hqk;
        float y[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) y[i] = cur.v[i];
        qkv_fwd_item8<LPH>(L, y, cur.cs, qk, h < L.n_q_heads, gq, gk, rp, lane, half);
        if (valid) st8(out + (long)t * ld_out + h * hd + 8 * j, y);
        if (wb + stride < items) cur = nxt;
    }
}

template <int LPH>
__global__ __launch_bounds__(NT) void qkv_bwd8_k(QkvLayout L, float *dqkv, long ld,
                                                  const float *qkv, long ld_qkv, const float *wq,
                                                  const float *wk, float *partial,
                                                  const float2 *tab, bf16 *outb, long ldb) {
    constexpr int G = 64 / LPH;
    __shared__ float red[2][128];
    const int lane = threadIdx.x % 64, wave = threadIdx.x / 64, j = lane % LPH, g = lane / LPH;
    const int hd = L.head_dim, Hqk = L.n_q_heads + L.n_kv_heads;
    const int Htot = outb ? Hqk + L.n_kv_heads : Hqk;
    const int half = L.rotary_dim / 2;
    const long items = (long)L.n_rows * Htot;
    const long stride = (long)gridDim.x * NW * G;
    const Rope8 rp = rope8(j, half);
    float gq[8], gk[8], dwq[8], dwk[8];
    if (L.qk_norm) {
        ld8(wq + 8 * j, gq);
        ld8(wk + 8 * j, gk);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) dwq[i] = dwk[i] = 0.f;
    auto fetch = [&](long it, Item8 &d) {
        const int t = (int)(it / Htot), h = (int)(it % Htot);
        const bool qk = h < Hqk;
        load8<LPH>(d, dqkv + (long)t * ld + h * hd + 8 * j,
                   (qk && L.qk_norm) ? qkv + (long)t * ld_qkv + h * hd + 8 * j : nullptr,
                   tab + (long)(t % L.seq_len) * half, rp, it < items, qk);
    };
    long it = ((long)blockIdx.x * NW + wave) * G + g;
    const long wave_first = it - g;
    Item8 cur;
    fetch(it, cur);
    for (long wb = wave_first; wb < items; wb += stride, it += stride) {
        Item8 nxt;
        if (wb + stride < items) fetch(it + stride, nxt);
        const bool valid = it < items;
        const int t = (int)(it / Htot), h = (int)(it % Htot);
        const bool qk = valid && h < Hqk;
        const bool is_q = h < L.n_q_heads;
        float gv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) gv[i] = cur.v[i];
        if (half > 0) {
            float pv[8];
            partner8<LPH>(gv, pv, lane, rp, half);
            if (qk && rp.rot_lane) {
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const float2 cs = cur.cs[i];
                    gv[i] = rp.lower ? cs.x * gv[i] + cs.y * pv[i] : -cs.y * pv[i] + cs.x * gv[i];
                }
            }
        }
        if (L.qk_norm) {
            double ss = 0, A = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float gw = is_q ? gq[i] : gk[i];
                ss += (double)cur.x[i] * (double)cur.x[i];
                A += (double)gv[i] * (double)gw * (double)cur.x[i];
            }
            ss = grp_sum<LPH>(ss);
            A = grp_sum<LPH>(A);
            if (qk) {
                const float ri = 1.0f / sqrtf((float)(ss / (double)hd) + L.eps);
                const float ri3_over_D = ri * ri * ri / (float)hd;
                const float A_f = (float)A;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const float gw = is_q ? gq[i] : gk[i];
                    const float o = ri * gw * gv[i] - ri3_over_D * cur.x[i] * A_f;
                    const float dwv = gv[i] * ri * cur.x[i];
                    if (is_q) dwq[i] += dwv; else dwk[i] += dwv;
                    gv[i] = o;
                }
            }
        }
        if (valid) {
            if (outb) st8(outb + (long)t * ldb + h * hd + 8 * j, gv);
            else if (h < Hqk) st8(dqkv + (long)t * ld + h * hd + 8 * j, gv);
        }
        if (wb + stride < items) cur = nxt;
    }
    // combine the lane groups' gain partials in a fixed (wave, group) order
    for (int s = 0; s < NW * G; ++s) {
        if (wave * G + g == s) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                red[0][8 * j + i] = s ? red[0][8 * j + i] + dwq[i] : dwq[i];
                red[1][8 * j + i] = s ? red[1][8 * j + i] + dwk[i] : dwk[i];
            }
        }
        __syncthreads();
    }
    for (int c = threadIdx.x; c < 2 * hd; c += NT)
        partial[(long)blockIdx.x * 2 * hd + c] = red[c / hd][c % hd];
}

// Grid caps (the gain partials are one row per block; in the training step
// a larger Q/K-norm backward grid made its column sums on the side stream
// slower than it made the kernel faster).
constexpr int kRmsMaxBlocks = 512, kQkvMaxBlocks = 512;

inline int rms_grid(int rows) { return std::max(1, std::min(kRmsMaxBlocks, (rows + NW - 1) / NW)); }

inline long qkv_items(const QkvLayout &L, bool with_v) {
    return (long)L.n_rows * (L.n_q_heads + L.n_kv_heads + (with_v ? L.n_kv_heads : 0));
}
inline int qkv_grid(long items, int cap) {
    return (int)std::max<long>(1, std::min<long>(cap, (items + 4 * NW - 1) / (4 * NW)));
}

template <class F>
hipError_t by_c4(int dim, F &&f) {
    if (dim <= 256) return f(std::integral_constant<int, 1>{});
    if (dim <= 512) return f(std::integral_constant<int, 2>{});
    if (dim <= 1024) return f(std::integral_constant<int, 4>{});
    if (dim <= 2048) return f(std::integral_constant<int, 8>{});
    return f(std::integral_constant<int, 16>{});
}

template <class F>
hipError_t by_epl(int hd, F &&f) {
    if (hd <= 64) return f(std::integral_constant<int, 1>{});
    if (hd <= 128) return f(std::integral_constant<int, 2>{});
    return f(std::integral_constant<int, 4>{});
}

inline bool al16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

// The several-heads-per-wave kernels: head_dim 64 or 128, rotary width a
// multiple of 16, 16-byte aligned rows (out_align = elements per 16 bytes).
inline bool qkv8_ok(const QkvLayout &L, const void *in, long ld_in, const void *out, long ld_out,
                    int out_align) {
    return (L.head_dim == 64 || L.head_dim == 128) && L.rotary_dim % 16 == 0 &&
           L.rotary_dim <= L.head_dim && L.seq_len > 0 && al16(in) && al16(out) &&
           ld_in % 4 == 0 && ld_out % out_align == 0;
}
inline int qkv8_grid(const QkvLayout &L, long items, int cap) {
    const long per_block = (long)NW * (64 / (L.head_dim / 8));
    return (int)std::max<long>(1, std::min<long>(cap, (items + 2 * per_block - 1) / (2 * per_block)));
}
template <class F>
hipError_t by_lph(int hd, F &&f) {
    if (hd == 64) return f(std::integral_constant<int, 8>{});
    return f(std::integral_constant<int, 16>{});
}

}  // namespace

size_t rmsnorm_partial_floats(int rows, int dim) { return (size_t)rms_grid(rows) * dim; }
int rmsnorm_partial_rows(int rows) { return rms_grid(rows); }

hipError_t column_sums(const float *partial, int nparts, long stride, int dim, float *out,
                       hipStream_t st) {
    if (dim <= 0) return hipSuccess;
    hipLaunchKernelGGL(colsum_k, dim3(ceil_div(dim, CS_COLS)), dim3(CS_COLS * CS_GROUPS), 0, st,
                       partial, nparts, stride, dim, out);
    return hipGetLastError();
}

hipError_t rmsnorm_forward(const float *x, const float *w, void *y, DType ydt, int rows, int dim,
                           float eps, int gemma_quirk, hipStream_t st) {
    if (rows <= 0) return hipSuccess;
    if (dim <= 0 || dim > 4096 || dim % 4 || !al16(x) || !al16(w) || ((uintptr_t)y & 7u))
        return hipErrorInvalidValue;
    const int grid = std::max(1, std::min(4096, (rows + NW - 1) / NW));
    return by_c4(dim, [&](auto c4) {
        constexpr int C4 = decltype(c4)::value;
        if (ydt == DType::BF16)
            hipLaunchKernelGGL((rmsnorm_fwd_k<bf16, C4>), dim3(grid), dim3(NT), 0, st, x, w,
                               (bf16 *)y, rows, dim, eps, gemma_quirk);
        else
            hipLaunchKernelGGL((rmsnorm_fwd_k<float, C4>), dim3(grid), dim3(NT), 0, st, x, w,
                               (float *)y, rows, dim, eps, gemma_quirk);
        return hipGetLastError();
    });
}

hipError_t rmsnorm_backward(const float *dy, const float *x, const float *w, float *dx,
                            bf16 *dxb, const float *residual, float *dw, float *partial, int rows,
                            int dim, float eps, int gemma_quirk, hipStream_t st) {
    if (rows <= 0) return hipSuccess;
    if (dim <= 0 || dim > 4096 || dim % 4 || !al16(dy) || !al16(x) || !al16(w) || !al16(dx) ||
        ((uintptr_t)dxb & 7u) || !al16(residual))
        return hipErrorInvalidValue;
    const int grid = rms_grid(rows);
    hipError_t e;
    if (dim > 2048) {  // wide rows: a block per row (dim <= 4096: 4 float4 per thread)
        hipLaunchKernelGGL((rmsnorm_bwd_row_k<4>), dim3(grid), dim3(NT), 0, st, dy, x, w, dx, dxb,
                           residual, partial, rows, dim, eps, gemma_quirk);
        e = hipGetLastError();
    } else {
        e = by_c4(dim, [&](auto c4) {
            constexpr int C4 = decltype(c4)::value;
            hipLaunchKernelGGL((rmsnorm_bwd_k<C4>), dim3(grid), dim3(NT), 0, st, dy, x, w, dx, dxb,
                               residual, partial, rows, dim, eps, gemma_quirk);
            return hipGetLastError();
        });
    }
    if (e != hipSuccess) return e;
    if (dw)
        hipLaunchKernelGGL(colsum_k, dim3(ceil_div(dim, CS_COLS)), dim3(CS_COLS * CS_GROUPS), 0, st,
                           (const float *)partial, grid, (long)dim, dim, dw);
    return hipGetLastError();
}

hipError_t qk_rope(const float *q_in, long ldq_in, float *q_out, long ldq_out, const float *k_in,
                   long ldk_in, float *k_out, long ldk_out, int n_rows, int n_q_heads,
                   int n_kv_heads, int head_dim, int rotary_dim, int seq_len, const float2 *tab,
                   bool backward, hipStream_t st) {
    if (n_rows <= 0) return hipSuccess;
    if (rotary_dim > head_dim || (rotary_dim & 1) || seq_len <= 0) return hipErrorInvalidValue;
    const bool v4 = head_dim % 4 == 0 && rotary_dim % 8 == 0 && al16(q_in) && al16(q_out) &&
                    al16(k_in) && al16(k_out) && al16(tab) && ldq_in % 4 == 0 &&
                    ldq_out % 4 == 0 && ldk_in % 4 == 0 && ldk_out % 4 == 0;
    const long units = (long)n_rows * (n_q_heads + n_kv_heads) * (rotary_dim / 8 + (head_dim - rotary_dim) / 4);
    if (v4 && units < (1L << 31)) {
        const long g = std::min<long>(16384, (units + NT - 1) / NT);
        hipLaunchKernelGGL(qk_rope_pair_k, dim3((unsigned)g), dim3(NT), 0, st, q_in, ldq_in, q_out,
                           ldq_out, k_in, ldk_in, k_out, ldk_out, n_rows, n_q_heads, n_kv_heads,
                           head_dim, rotary_dim, seq_len, tab, backward ? 1 : 0);
        return hipGetLastError();
    }
    const long total = (long)n_rows * (n_q_heads + n_kv_heads) * head_dim;
    long g = (total + NT - 1) / NT;
    if (g > 4096) g = 4096;
    hipLaunchKernelGGL(qk_rope_k, dim3((unsigned)g), dim3(NT), 0, st, q_in, ldq_in, q_out, ldq_out,
                       k_in, ldk_in, k_out, ldk_out, n_rows, n_q_heads, n_kv_heads, head_dim,
                       rotary_dim, seq_len, tab, backward ? 1 : 0);
    return hipGetLastError();
}

size_t qkv_partial_floats(const QkvLayout &L) { return (size_t)kQkvMaxBlocks * 2 * L.head_dim; }

static bool qkv_shape_ok(const QkvLayout &L, long ld_in, long ld_out) {
    return L.head_dim > 0 && L.head_dim <= 256 && L.head_dim % 4 == 0 && L.rotary_dim <= L.head_dim &&
           (L.rotary_dim & 1) == 0 && L.seq_len > 0 && ld_in % 4 == 0 && ld_out % 4 == 0;
}

hipError_t qkv_prepare_forward(const QkvLayout &L, const float *qkv, long ld_qkv,
                               const float *wq, const float *wk, void *out, long ld_out,
                               DType out_dt, const float2 *rope_tab, hipStream_t st) {
    if (L.n_rows <= 0) return hipSuccess;
    if (!qkv_shape_ok(L, ld_qkv, ld_out) || !al16(qkv) || ((uintptr_t)out & 7u) ||
        (L.qk_norm && (!al16(wq) || !al16(wk))))
        return hipErrorInvalidValue;
    if (qkv8_ok(L, qkv, ld_qkv, out, ld_out, out_dt == DType::BF16 ? 8 : 4)) {
        const int grid = qkv8_grid(L, qkv_items(L, true), 2048);
        return by_lph(L.head_dim, [&](auto lph) {
            constexpr int LPH = decltype(lph)::value;
            if (out_dt == DType::BF16)
                hipLaunchKernelGGL((qkv_fwd8_k<bf16, LPH>), dim3(grid), dim3(NT), 0, st, L, qkv,
                                   ld_qkv, wq, wk, (bf16 *)out, ld_out, rope_tab);
            else
                hipLaunchKernelGGL((qkv_fwd8_k<float, LPH>), dim3(grid), dim3(NT), 0, st, L, qkv,
                                   ld_qkv, wq, wk, (float *)out, ld_out, rope_tab);
            return hipGetLastError();
        });
    }
    const int grid = qkv_grid(qkv_items(L, true), 2048);
    return by_epl(L.head_dim, [&](auto epl) {
        constexpr int EPL = decltype(epl)::value;
        if (out_dt == DType::BF16)
            hipLaunchKernelGGL((qkv_fwd_k<bf16, EPL>), dim3(grid), dim3(NT), 0, st, L, qkv, ld_qkv,
                               wq, wk, (bf16 *)out, ld_out, rope_tab);
        else
            hipLaunchKernelGGL((qkv_fwd_k<float, EPL>), dim3(grid), dim3(NT), 0, st, L, qkv, ld_qkv,
                               wq, wk, (float *)out, ld_out, rope_tab);
        return hipGetLastError();
    });
}

hipError_t qkv_prepare_backward(const QkvLayout &L, float *dqkv, long ld, const float *qkv,
                                long ld_qkv, const float *wq, const float *wk, float *dwq,
                                float *dwk, float *partial, const float2 *rope_tab,
                                bf16 *outb, long ldb, hipStream_t st, int *nparts) {
    if (L.n_rows <= 0) return hipSuccess;
    if (!qkv_shape_ok(L, ld, ld_qkv) || (outb && ldb % 4) || !al16(dqkv) || !al16(qkv) ||
        ((uintptr_t)outb & 7u) || (L.qk_norm && (!al16(wq) || !al16(wk))))
        return hipErrorInvalidValue;
    const bool fast = qkv8_ok(L, qkv, ld_qkv, dqkv, ld, 4) &&
                      (!outb || (al16(outb) && ldb % 8 == 0));
    const int grid = fast ? qkv8_grid(L, qkv_items(L, outb != nullptr), kQkvMaxBlocks)
                          : qkv_grid(qkv_items(L, outb != nullptr), kQkvMaxBlocks);
    hipError_t e;
    if (fast)
        e = by_lph(L.head_dim, [&](auto lph) {
            constexpr int LPH = decltype(lph)::value;
            hipLaunchKernelGGL((qkv_bwd8_k<LPH>), dim3(grid), dim3(NT), 0, st, L, dqkv, ld, qkv,
                               ld_qkv, wq, wk, partial, rope_tab, outb, ldb);
            return hipGetLastError();
        });
    else
        e = by_epl(L.head_dim, [&](auto epl) {
            constexpr int EPL = decltype(epl)::value;
            hipLaunchKernelGGL((qkv_bwd_k<EPL>), dim3(grid), dim3(NT), 0, st, L, dqkv, ld, qkv,
                               ld_qkv, wq, wk, partial, rope_tab, outb, ldb);
            return hipGetLastError();
        });
    if (e != hipSuccess) return e;
    if (nparts) *nparts = grid;
    if (L.qk_norm && dwq && dwk) {
        hipLaunchKernelGGL(colsum_k, dim3(ceil_div(L.head_dim, CS_COLS)), dim3(CS_COLS * CS_GROUPS), 0, st,
                           (const float *)partial, grid, (long)2 * L.head_dim, L.head_dim, dwq);
        hipLaunchKernelGGL(colsum_k, dim3(ceil_div(L.head_dim, CS_COLS)), dim3(CS_COLS * CS_GROUPS), 0, st,
                           (const float *)partial + L.head_dim, grid, (long)2 * L.head_dim,
                           L.head_dim, dwk);
    }
    return hipGetLastError();
}

}  // namespace vkh

#include <math.h>

void vkh::rope_table_host(float2 *tab, int seq_len, int rotary_dim, float theta) {
    const int half = rotary_dim / 2;
    const float rdim_f = (float)rotary_dim;
    for (int j = 0; j < half; ++j) {
        const float freq = 1.0f / powf(theta, (2.0f * (float)j) / rdim_f);
        for (int p = 0; p < seq_len; ++p) {
            const float angle = (float)p * freq;
            tab[(long)p * half + j] = make_float2(cosf(angle), sinf(angle));
        }
    }
}
