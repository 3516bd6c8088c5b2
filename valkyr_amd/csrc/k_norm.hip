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
#include "ops.hpp"

#pragma clang fp contract(off)

namespace vkh {

namespace {

constexpr int NT = 256;
constexpr int MAX_CPT = 16;  // columns per thread => dim <= 4096

VKH_DEV double block_sum_d(double v, double *sh) {
    v = wave_sum(v);
    const int w = threadIdx.x / 64, l = threadIdx.x % 64;
    __syncthreads();
    if (l == 0) sh[w] = v;
    __syncthreads();
    double t = 0;
#pragma unroll
    for (int i = 0; i < NT / 64; ++i) t += sh[i];
    return t;
}

template <typename TO>
__global__ __launch_bounds__(NT) void rmsnorm_fwd_k(const float *x, const float *w, TO *y,
                                                     int dim, float eps, int gq) {
    __shared__ double sh[NT / 64];
    const long row = blockIdx.x;
    const float *xr = x + row * dim;
    TO *yr = y + row * dim;
    double ss = 0;
    for (int c = threadIdx.x; c < dim; c += NT) ss += (double)xr[c] * (double)xr[c];
    ss = block_sum_d(ss, sh);
    const double m = ss / (double)dim;
    const float ri = 1.0f / sqrtf((float)m + eps);
    for (int c = threadIdx.x; c < dim; c += NT) {
        const float gain = gq ? w[c] + 1.0f : w[c];
        yr[c] = (TO)(gain * ri * xr[c]);
    }
}

// Rows [blockIdx.x * rpb, ...) of one norm; per-thread gain-gradient partials.
// dxb (optional): bf16 copy of dx, the operand of the next GEMMs.
__global__ __launch_bounds__(NT) void rmsnorm_bwd_k(const float *dy, const float *x,
                                                     const float *w, float *dx, bf16 *dxb,
                                                     const float *res, float *partial,
                                                     int rows, int dim, float eps, int gq,
                                                     int rpb) {
    __shared__ double sh[NT / 64];
    float dwacc[MAX_CPT];
#pragma unroll
    for (int k = 0; k < MAX_CPT; ++k) dwacc[k] = 0.f;
    const int r0 = blockIdx.x * rpb;
    const int r1 = min(rows, r0 + rpb);
    const float ri3_div = (float)dim;
    for (int row = r0; row < r1; ++row) {
        const float *xr = x + (long)row * dim;
        const float *dyr = dy + (long)row * dim;
        double ss = 0, A = 0;
#pragma unroll
        for (int k = 0; k < MAX_CPT; ++k) {
            const int c = threadIdx.x + k * NT;
            if (c < dim) {
                const double xv = xr[c];
                const float gain = gq ? w[c] + 1.0f : w[c];
                ss += xv * xv;
                A += (double)dyr[c] * (double)gain * xv;
            }
        }
        ss = block_sum_d(ss, sh);
        A = block_sum_d(A, sh);
        const double m = ss / (double)dim;
        const float ri = 1.0f / sqrtf((float)m + eps);
        const float ri3_over_D = ri * ri * ri / ri3_div;
        const float A_f = (float)A;
#pragma unroll
        for (int k = 0; k < MAX_CPT; ++k) {
            const int c = threadIdx.x + k * NT;
            if (c < dim) {
                const float gain = gq ? w[c] + 1.0f : w[c];
                const float xv = xr[c], dv = dyr[c];
                float o = ri * gain * dv - ri3_over_D * xv * A_f;
                if (res) o = o + res[(long)row * dim + c];
                dx[(long)row * dim + c] = o;
                if (dxb) dxb[(long)row * dim + c] = (bf16)o;
                dwacc[k] += dv * ri * xv;
            }
        }
    }
#pragma unroll
    for (int k = 0; k < MAX_CPT; ++k) {
        const int c = threadIdx.x + k * NT;
        if (c < dim) partial[(long)blockIdx.x * dim + c] = dwacc[k];
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

inline int rms_blocks(int rows) { return rows < 512 ? rows : 512; }

// ── RoPE ─────────────────────────────────────────────────────────────

// qk_rope_partial_batched.comp / qk_rope_backward_batched.comp with the
// cos/sin of (position, pair) taken from a table built by the same fp32
// formula.  One thread per element of the combined [rows, Hq + Hkv, hd].
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

template <typename TO>
VKH_DEV void store_out(TO *p, float v);
template <>
VKH_DEV void store_out<float>(float *p, float v) { *p = v; }
template <>
VKH_DEV void store_out<bf16>(bf16 *p, float v) { *p = (bf16)v; }

constexpr int MAX_EPL = 4;  // elements per lane => head_dim <= 256

// One block per row; waves take heads round-robin.  Forward: normalised and
// rotated q, k plus v, written as attention operands of type TO.
template <typename TO>
__global__ __launch_bounds__(NT) void qkv_fwd_k(QkvLayout L, const float *qkv, long ld_qkv,
                                                 const float *wq, const float *wk, TO *out,
                                                 long ld_out, const float2 *tab) {
    __shared__ float stage[NT / 64][256];
    const int t = blockIdx.x;
    const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
    const int hd = L.head_dim, H = L.n_q_heads + L.n_kv_heads;
    const int half = L.rotary_dim / 2;
    const int p = t % L.seq_len;
    const float *row = qkv + (long)t * ld_qkv;
    TO *orow = out + (long)t * ld_out;
    const int iters = (H + 3) / 4;
    for (int it = 0; it < iters; ++it) {
        const int h = it * 4 + wave;
        const bool active = h < H;
        float y[MAX_EPL];
        if (active) {
            const bool is_q = h < L.n_q_heads;
            const int col0 = h * hd;  // q heads then k heads are contiguous
            const float *g = is_q ? wq : wk;
            double ss = 0;
#pragma unroll
            for (int k = 0; k < MAX_EPL; ++k) {
                const int e = lane + 64 * k;
                y[k] = e < hd ? row[col0 + e] : 0.f;
                ss += (double)y[k] * (double)y[k];
            }
            if (L.qk_norm) {
                ss = wave_sum(ss);
                const float ri = 1.0f / sqrtf((float)(ss / (double)hd) + L.eps);
#pragma unroll
                for (int k = 0; k < MAX_EPL; ++k) {
                    const int e = lane + 64 * k;
                    if (e < hd) y[k] = g[e] * ri * y[k];
                }
            }
#pragma unroll
            for (int k = 0; k < MAX_EPL; ++k) {
                const int e = lane + 64 * k;
                if (e < hd) stage[wave][e] = y[k];
            }
        }
        __syncthreads();
        if (active) {
#pragma unroll
            for (int k = 0; k < MAX_EPL; ++k) {
                const int e = lane + 64 * k;
                if (e >= hd) continue;
                float o = y[k];
                if (e < L.rotary_dim) {
                    const int j = e < half ? e : e - half;
                    const float2 cs = tab[(long)p * half + j];
                    const float a = stage[wave][j], b = stage[wave][j + half];
                    o = (e < half) ? a * cs.x - b * cs.y : a * cs.y + b * cs.x;
                }
                store_out<TO>(orow + h * hd + e, o);
            }
        }
        __syncthreads();
    }
    // v: copy / cast
    const int vcol0 = H * hd, vn = L.n_kv_heads * hd;
    for (int c = threadIdx.x; c < vn; c += NT) store_out<TO>(orow + vcol0 + c, row[vcol0 + c]);
}

// Backward on the fused d_qkv buffer (q/k columns in place):
//   dn = rope^T(g);  d_pre = rmsnorm_bw(dn; x = pre-norm q/k);  dw += dn*ri*x
// outb (optional): the results go to this bf16 copy of the whole row (q, k
// and the untouched v columns) instead of back into dqkv.
__global__ __launch_bounds__(NT) void qkv_bwd_k(QkvLayout L, float *dqkv, long ld,
                                                 const float *qkv, long ld_qkv, const float *wq,
                                                 const float *wk, float *partial,
                                                 const float2 *tab, int rpb, bf16 *outb,
                                                 long ldb) {
    __shared__ float stage[NT / 64][256];
    __shared__ float red[NT / 64][2][256];
    const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
    const int hd = L.head_dim, H = L.n_q_heads + L.n_kv_heads;
    const int half = L.rotary_dim / 2;
    float dwq[MAX_EPL], dwk[MAX_EPL];
#pragma unroll
    for (int k = 0; k < MAX_EPL; ++k) dwq[k] = dwk[k] = 0.f;
    const int r0 = blockIdx.x * rpb, r1 = min(L.n_rows, r0 + rpb);
    const int iters = (H + 3) / 4;
    for (int t = r0; t < r1; ++t) {
        const int p = t % L.seq_len;
        float *drow = dqkv + (long)t * ld;
        const float *xrow = qkv + (long)t * ld_qkv;
        for (int it = 0; it < iters; ++it) {
            const int h = it * 4 + wave;
            const bool active = h < H;
            float gv[MAX_EPL];
            if (active) {
#pragma unroll
                for (int k = 0; k < MAX_EPL; ++k) {
                    const int e = lane + 64 * k;
                    gv[k] = e < hd ? drow[h * hd + e] : 0.f;
                    if (e < hd) stage[wave][e] = gv[k];
                }
            }
            __syncthreads();
            if (active) {
                const bool is_q = h < L.n_q_heads;
                const float *g = is_q ? wq : wk;
                float dn[MAX_EPL], xv[MAX_EPL];
                double ss = 0, A = 0;
#pragma unroll
                for (int k = 0; k < MAX_EPL; ++k) {
                    const int e = lane + 64 * k;
                    dn[k] = gv[k];
                    xv[k] = 0.f;
                    if (e >= hd) continue;
                    if (e < L.rotary_dim) {
                        const int j = e < half ? e : e - half;
                        const float2 cs = tab[(long)p * half + j];
                        const float a = stage[wave][j], b = stage[wave][j + half];
                        dn[k] = (e < half) ? cs.x * a + cs.y * b : -cs.y * a + cs.x * b;
                    }
                    if (L.qk_norm) {
                        xv[k] = xrow[h * hd + e];
                        ss += (double)xv[k] * (double)xv[k];
                        A += (double)dn[k] * (double)g[e] * (double)xv[k];
                    }
                }
                if (L.qk_norm) {
                    ss = wave_sum(ss);
                    A = wave_sum(A);
                    const float ri = 1.0f / sqrtf((float)(ss / (double)hd) + L.eps);
                    const float ri3_over_D = ri * ri * ri / (float)hd;
                    const float A_f = (float)A;
#pragma unroll
                    for (int k = 0; k < MAX_EPL; ++k) {
                        const int e = lane + 64 * k;
                        if (e >= hd) continue;
                        const float o = ri * g[e] * dn[k] - ri3_over_D * xv[k] * A_f;
                        const float dwv = dn[k] * ri * xv[k];
                        if (is_q) dwq[k] += dwv; else dwk[k] += dwv;
                        if (outb) outb[(long)t * ldb + h * hd + e] = (bf16)o;
                        else drow[h * hd + e] = o;
                    }
                } else {
#pragma unroll
                    for (int k = 0; k < MAX_EPL; ++k) {
                        const int e = lane + 64 * k;
                        if (e >= hd) continue;
                        if (outb) outb[(long)t * ldb + h * hd + e] = (bf16)dn[k];
                        else drow[h * hd + e] = dn[k];
                    }
                }
            }
            __syncthreads();
        }
        if (outb) {
            const int vcol0 = H * hd, vn = L.n_kv_heads * hd;
            for (int c = threadIdx.x; c < vn; c += NT)
                outb[(long)t * ldb + vcol0 + c] = (bf16)drow[vcol0 + c];
        }
    }
    // combine the 4 waves' gain partials, fixed order
#pragma unroll
    for (int k = 0; k < MAX_EPL; ++k) {
        const int e = lane + 64 * k;
        if (e < hd) {
            red[wave][0][e] = dwq[k];
            red[wave][1][e] = dwk[k];
        }
    }
    __syncthreads();
    for (int c = threadIdx.x; c < 2 * hd; c += NT) {
        const int which = c / hd, e = c % hd;
        float s = 0.f;
#pragma unroll
        for (int wv = 0; wv < NT / 64; ++wv) s += red[wv][which][e];
        partial[(long)blockIdx.x * 2 * hd + c] = s;
    }
}

inline int qkv_blocks(int rows) { return rows < 512 ? rows : 512; }

}  // namespace

size_t rmsnorm_partial_floats(int rows, int dim) { return (size_t)rms_blocks(rows) * dim; }

hipError_t rmsnorm_forward(const float *x, const float *w, void *y, DType ydt, int rows, int dim,
                           float eps, int gemma_quirk, hipStream_t st) {
    if (rows <= 0) return hipSuccess;
    if (ydt == DType::BF16)
        hipLaunchKernelGGL(rmsnorm_fwd_k<bf16>, dim3(rows), dim3(NT), 0, st, x, w, (bf16 *)y, dim,
                           eps, gemma_quirk);
    else
        hipLaunchKernelGGL(rmsnorm_fwd_k<float>, dim3(rows), dim3(NT), 0, st, x, w, (float *)y, dim,
                           eps, gemma_quirk);
    return hipGetLastError();
}

hipError_t rmsnorm_backward(const float *dy, const float *x, const float *w, float *dx,
                            bf16 *dxb, const float *residual, float *dw, float *partial, int rows,
                            int dim, float eps, int gemma_quirk, hipStream_t st) {
    if (rows <= 0) return hipSuccess;
    if (dim > NT * MAX_CPT) return hipErrorInvalidValue;
    const int nb = rms_blocks(rows);
    const int rpb = (rows + nb - 1) / nb;
    const int nblocks = (rows + rpb - 1) / rpb;
    hipLaunchKernelGGL(rmsnorm_bwd_k, dim3(nblocks), dim3(NT), 0, st, dy, x, w, dx, dxb, residual,
                       partial, rows, dim, eps, gemma_quirk, rpb);
    if (dw)
        hipLaunchKernelGGL(colsum_k, dim3(ceil_div(dim, CS_COLS)), dim3(CS_COLS * CS_GROUPS), 0, st,
                           (const float *)partial, nblocks, (long)dim, dim, dw);
    return hipGetLastError();
}

hipError_t qk_rope(const float *q_in, long ldq_in, float *q_out, long ldq_out, const float *k_in,
                   long ldk_in, float *k_out, long ldk_out, int n_rows, int n_q_heads,
                   int n_kv_heads, int head_dim, int rotary_dim, int seq_len, const float2 *tab,
                   bool backward, hipStream_t st) {
    if (n_rows <= 0) return hipSuccess;
    if (rotary_dim > head_dim || (rotary_dim & 1) || seq_len <= 0) return hipErrorInvalidValue;
    const long total = (long)n_rows * (n_q_heads + n_kv_heads) * head_dim;
    long g = (total + NT - 1) / NT;
    if (g > 4096) g = 4096;
    hipLaunchKernelGGL(qk_rope_k, dim3((unsigned)g), dim3(NT), 0, st, q_in, ldq_in, q_out, ldq_out,
                       k_in, ldk_in, k_out, ldk_out, n_rows, n_q_heads, n_kv_heads, head_dim,
                       rotary_dim, seq_len, tab, backward ? 1 : 0);
    return hipGetLastError();
}

size_t qkv_partial_floats(const QkvLayout &L) { return (size_t)qkv_blocks(L.n_rows) * 2 * L.head_dim; }

hipError_t qkv_prepare_forward(const QkvLayout &L, const float *qkv, long ld_qkv,
                               const float *wq, const float *wk, void *out, long ld_out,
                               DType out_dt, const float2 *rope_tab, hipStream_t st) {
    if (L.n_rows <= 0) return hipSuccess;
    if (L.head_dim > 64 * MAX_EPL || L.rotary_dim > L.head_dim || (L.rotary_dim & 1))
        return hipErrorInvalidValue;
    if (out_dt == DType::BF16)
        hipLaunchKernelGGL(qkv_fwd_k<bf16>, dim3(L.n_rows), dim3(NT), 0, st, L, qkv, ld_qkv, wq, wk,
                           (bf16 *)out, ld_out, rope_tab);
    else
        hipLaunchKernelGGL(qkv_fwd_k<float>, dim3(L.n_rows), dim3(NT), 0, st, L, qkv, ld_qkv, wq,
                           wk, (float *)out, ld_out, rope_tab);
    return hipGetLastError();
}

hipError_t qkv_prepare_backward(const QkvLayout &L, float *dqkv, long ld, const float *qkv,
                                long ld_qkv, const float *wq, const float *wk, float *dwq,
                                float *dwk, float *partial, const float2 *rope_tab,
                                bf16 *outb, long ldb, hipStream_t st) {
    if (L.n_rows <= 0) return hipSuccess;
    if (L.head_dim > 64 * MAX_EPL || L.rotary_dim > L.head_dim || (L.rotary_dim & 1))
        return hipErrorInvalidValue;
    const int nb = qkv_blocks(L.n_rows);
    const int rpb = (L.n_rows + nb - 1) / nb;
    const int nblocks = (L.n_rows + rpb - 1) / rpb;
    hipLaunchKernelGGL(qkv_bwd_k, dim3(nblocks), dim3(NT), 0, st, L, dqkv, ld, qkv, ld_qkv, wq, wk,
                       partial, rope_tab, rpb, outb, ldb);
    if (L.qk_norm && dwq && dwk) {
        hipLaunchKernelGGL(colsum_k, dim3(ceil_div(L.head_dim, CS_COLS)), dim3(CS_COLS * CS_GROUPS), 0, st,
                           (const float *)partial, nblocks, (long)2 * L.head_dim, L.head_dim, dwq);
        hipLaunchKernelGGL(colsum_k, dim3(ceil_div(L.head_dim, CS_COLS)), dim3(CS_COLS * CS_GROUPS), 0, st,
                           (const float *)partial + L.head_dim, nblocks, (long)2 * L.head_dim,
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
