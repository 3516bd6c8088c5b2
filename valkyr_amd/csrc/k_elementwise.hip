// Bandwidth-bound elementwise kernels: fill, add, scale, cast, SwiGLU fwd/bwd,
// embedding lookup and Adam.  All are float4-vectorised grid-stride loops
// sized to fill the 256 CUs; fp contraction is disabled so each kernel
// rounds exactly like the scalar reference formula it restates.
#include <atomic>

#include "ops.hpp"
#include "adam.hpp"

#pragma clang fp contract(off)

namespace vkh {

namespace {

constexpr int NT = 256;

VKH_DEV void st4(float *p, float4 v) { *reinterpret_cast<float4 *>(p) = v; }
VKH_DEV void st4(bf16 *p, float4 v) {
    bf16x4 b;
    b[0] = (bf16)v.x; b[1] = (bf16)v.y; b[2] = (bf16)v.z; b[3] = (bf16)v.w;
    *reinterpret_cast<bf16x4 *>(p) = b;
}
VKH_DEV void st1(float *p, float v) { *p = v; }
VKH_DEV void st1(bf16 *p, float v) { *p = (bf16)v; }

inline unsigned grid_for(size_t n_vec) {
    size_t g = (n_vec + NT - 1) / NT;
    const size_t cap = 256 * 16;  // 16 blocks per CU is plenty for a streaming kernel
    if (g > cap) g = cap;
    return (unsigned)(g ? g : 1);
}

__global__ void fill_k(float *p, size_t n, float v, bool vec) {
    const size_t n4 = vec ? n / 4 : 0;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    float4 f = make_float4(v, v, v, v);
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n4; i += stride)
        reinterpret_cast<float4 *>(p)[i] = f;
    for (size_t i = n4 * 4 + blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += stride) p[i] = v;
}

__global__ void add_k(float *dst, const float *a, const float *b, size_t n, bool vec) {
    // dst = a + b  (dst may alias a)
    const size_t n4 = vec ? n / 4 : 0;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n4; i += stride) {
        float4 x = reinterpret_cast<const float4 *>(a)[i];
        float4 y = reinterpret_cast<const float4 *>(b)[i];
        reinterpret_cast<float4 *>(dst)[i] = make_float4(x.x + y.x, x.y + y.y, x.z + y.z, x.w + y.w);
    }
    for (size_t i = n4 * 4 + blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += stride)
        dst[i] = a[i] + b[i];
}

__global__ void scale_k(const float *in, float *out, size_t n, float s, bool vec) {
    const size_t n4 = vec ? n / 4 : 0;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n4; i += stride) {
        float4 x = reinterpret_cast<const float4 *>(in)[i];
        reinterpret_cast<float4 *>(out)[i] = make_float4(x.x * s, x.y * s, x.z * s, x.w * s);
    }
    for (size_t i = n4 * 4 + blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = in[i] * s;
}

// The aligned form: each block streams one contiguous chunk of NT * SC_U
// float4 (16 KB in, 16 KB out), all loads issued before the stores,
// non-temporal (the stream is not reused); the last n % 4 elements in block
// 0.  As a plain read-n / write-n stream it is also the copy ceiling the
// bandwidth kernels are measured against.
constexpr int SC_U = 4;
__global__ __launch_bounds__(NT) void scale_chunk_k(const float *in_, float *out_, size_t n, float s) {
    const size_t n4 = n / 4;
    const f32x4 *in = reinterpret_cast<const f32x4 *>(in_);
    f32x4 *out = reinterpret_cast<f32x4 *>(out_);
    const size_t base = (size_t)blockIdx.x * (NT * SC_U) + threadIdx.x;
    f32x4 x[SC_U];
#pragma unroll
    for (int u = 0; u < SC_U; ++u) {
        const size_t j = base + (size_t)u * NT;
        if (j < n4) x[u] = __builtin_nontemporal_load(&in[j]);
    }
#pragma unroll
    for (int u = 0; u < SC_U; ++u) {
        const size_t j = base + (size_t)u * NT;
        if (j < n4) __builtin_nontemporal_store(x[u] * s, &out[j]);
    }
    if (blockIdx.x == 0 && threadIdx.x < n - 4 * n4) out_[4 * n4 + threadIdx.x] = in_[4 * n4 + threadIdx.x] * s;
}

__global__ void cast_bf16_k(const float *in, bf16 *out, size_t n, bool vec) {
    const size_t n4 = vec ? n / 4 : 0;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n4; i += stride) {
        float4 x = reinterpret_cast<const float4 *>(in)[i];
        bf16x4 y;
        y[0] = (bf16)x.x; y[1] = (bf16)x.y; y[2] = (bf16)x.z; y[3] = (bf16)x.w;
        reinterpret_cast<bf16x4 *>(out)[i] = y;
    }
    for (size_t i = n4 * 4 + blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = (bf16)in[i];
}

// sigmoid(z) = 1 / (1 + exp(-z))  (train_transformer.zig:832-834)
__device__ __forceinline__ float sigmoidf_(float z) { return 1.0f / (1.0f + expf(-z)); }

// Streaming kernels give each block one contiguous chunk (SW_U float4 per
// thread, all loads issued before any store, non-temporal): on MI355X that
// pattern measured 6.2 TB/s for a 1 GB copy against 5.0-5.3 TB/s for a
// grid-stride loop.  The SwiGLU kernels take one row chunk per block
// (blockIdx.y = row), so rows with their own leading dimensions need no
// index division.
constexpr int SW_U = 4;

VKH_DEV float4 ldnt4(const float *p) {
    const f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}

// swiglu_forward.comp / train_transformer.zig:839-851
template <typename TO>
__global__ __launch_bounds__(NT) void swiglu_fwd_k(const float *pg, long ldpg, const float *up,
                                                    long ldup, TO *g, long ldg, int cols4) {
    const long r = blockIdx.y;
    const int c0 = (int)blockIdx.x * NT * SW_U + (int)threadIdx.x;
    float4 z[SW_U], u[SW_U];
#pragma unroll
    for (int k = 0; k < SW_U; ++k) {
        const int c = 4 * (c0 + k * NT);
        if (c0 + k * NT < cols4) {
            z[k] = ldnt4(pg + r * ldpg + c);
            u[k] = ldnt4(up + r * ldup + c);
        }
    }
#pragma unroll
    for (int k = 0; k < SW_U; ++k) {
        if (c0 + k * NT >= cols4) continue;
        float4 o;
        o.x = swiglu1(z[k].x, u[k].x);
        o.y = swiglu1(z[k].y, u[k].y);
        o.z = swiglu1(z[k].z, u[k].z);
        o.w = swiglu1(z[k].w, u[k].w);
        st4(g + r * ldg + 4 * (c0 + k * NT), o);
    }
}

__device__ __forceinline__ void swiglu_bw1(float dg, float z, float u, float &dz, float &du) {
    const float sig = sigmoidf_(z);
    const float silu_z = z * sig;
    const float silu_grad = sig + silu_z * (1.0f - sig);
    du = dg * silu_z;
    dz = dg * u * silu_grad;
}

// swiglu_backward.comp / train_transformer.zig:857-875
template <typename TO>
__global__ __launch_bounds__(NT) void swiglu_bwd_k(const float *dg, long lddg, const float *pg,
                                                    long ldpg, const float *up, long ldup, TO *dpg,
                                                    long lddpg, TO *dup, long lddup, int cols4) {
    const long r = blockIdx.y;
    const int c0 = (int)blockIdx.x * NT * SW_U + (int)threadIdx.x;
    float4 d[SW_U], z[SW_U], u[SW_U];
#pragma unroll
    for (int k = 0; k < SW_U; ++k) {
        const int c = 4 * (c0 + k * NT);
        if (c0 + k * NT < cols4) {
            d[k] = ldnt4(dg + r * lddg + c);
            z[k] = ldnt4(pg + r * ldpg + c);
            u[k] = ldnt4(up + r * ldup + c);
        }
    }
#pragma unroll
    for (int k = 0; k < SW_U; ++k) {
        if (c0 + k * NT >= cols4) continue;
        const int c = 4 * (c0 + k * NT);
        float4 oz, ou;
        swiglu_bw1(d[k].x, z[k].x, u[k].x, oz.x, ou.x);
        swiglu_bw1(d[k].y, z[k].y, u[k].y, oz.y, ou.y);
        swiglu_bw1(d[k].z, z[k].z, u[k].z, oz.z, ou.z);
        swiglu_bw1(d[k].w, z[k].w, u[k].w, oz.w, ou.w);
        st4(dpg + r * lddpg + c, oz);
        st4(dup + r * lddup + c, ou);
    }
}

// scalar fallbacks for shapes whose columns are not a multiple of 4
template <typename TO>
__global__ void swiglu_fwd_s(const float *pg, long ldpg, const float *up, long ldup, TO *g,
                             long ldg, int rows, int cols) {
    const size_t n = (size_t)rows * cols;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += stride) {
        const long r = (long)(i / cols);
        const int c = (int)(i % cols);
        const float z = pg[r * ldpg + c];
        st1(g + r * ldg + c, swiglu1(z, up[r * ldup + c]));
    }
}

template <typename TO>
__global__ void swiglu_bwd_s(const float *dg, long lddg, const float *pg, long ldpg,
                             const float *up, long ldup, TO *dpg, long lddpg, TO *dup,
                             long lddup, int rows, int cols) {
    const size_t n = (size_t)rows * cols;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += stride) {
        const long r = (long)(i / cols);
        const int c = (int)(i % cols);
        float dz, du;
        swiglu_bw1(dg[r * lddg + c], pg[r * ldpg + c], up[r * ldup + c], dz, du);
        st1(dpg + r * lddpg + c, dz);
        st1(dup + r * lddup + c, du);
    }
}

// embed_lookup_batched.comp
__global__ void embed_lookup_k(const float *embed, const uint32_t *ids, float *out, int n_pos,
                               int dim, float scale, bool vec) {
    const size_t n = (size_t)n_pos * dim;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    if (vec) {
        const int d4 = dim / 4;
        for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n / 4; i += stride) {
            const int p = (int)(i / d4), c = (int)(i % d4);
            float4 e = reinterpret_cast<const float4 *>(embed + (size_t)ids[p] * dim)[c];
            reinterpret_cast<float4 *>(out)[i] = make_float4(e.x * scale, e.y * scale, e.z * scale, e.w * scale);
        }
    } else {
        for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += stride) {
            const int p = (int)(i / dim), c = (int)(i % dim);
            out[i] = embed[(size_t)ids[p] * dim + c] * scale;
        }
    }
}

// The same lookup from a bf16 table (a frozen bf16 base), widened to fp32
// (dim % 4 == 0, 8-byte aligned rows).
__global__ void embed_lookup_bf16_k(const bf16 *embed, const uint32_t *ids, float *out, int n_pos,
                                    int dim, float scale) {
    const size_t n4 = (size_t)n_pos * dim / 4;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    const int d4 = dim / 4;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n4; i += stride) {
        const int p = (int)(i / d4), c = (int)(i % d4);
        const bf16x4 e = reinterpret_cast<const bf16x4 *>(embed + (size_t)ids[p] * dim)[c];
        reinterpret_cast<float4 *>(out)[i] =
            make_float4((float)e[0] * scale, (float)e[1] * scale, (float)e[2] * scale, (float)e[3] * scale);
    }
}

// Streaming update: every byte is touched once, so loads and stores are
// non-temporal.  Each block updates one contiguous chunk of NT * ADAM_U
// float4 (all loads issued before the first store), the pattern that
// measured fastest for large streams on MI355X.  pb (optional): bf16 copy of
// the updated parameters (the GEMM operand shadow).
constexpr int ADAM_U = 4;

__global__ __launch_bounds__(NT) void adam_chunk_k(float *p_, const float *g_, float *m_,
                                                    float *v_, bf16 *pb, size_t n, float lr,
                                                    float b1, float b2, float eps, float bc1,
                                                    float bc2, float wd) {
    const size_t n4 = n / 4;
    f32x4 *p = reinterpret_cast<f32x4 *>(p_), *m = reinterpret_cast<f32x4 *>(m_),
          *v = reinterpret_cast<f32x4 *>(v_);
    const f32x4 *g = reinterpret_cast<const f32x4 *>(g_);
    const size_t base = (size_t)blockIdx.x * (NT * ADAM_U) + threadIdx.x;
    f32x4 pp[ADAM_U], gg[ADAM_U], mm[ADAM_U], vv[ADAM_U];
#pragma unroll
    for (int u = 0; u < ADAM_U; ++u) {
        const size_t j = base + (size_t)u * NT;
        if (j < n4) {
            pp[u] = __builtin_nontemporal_load(&p[j]);
            gg[u] = __builtin_nontemporal_load(&g[j]);
            mm[u] = __builtin_nontemporal_load(&m[j]);
            vv[u] = __builtin_nontemporal_load(&v[j]);
        }
    }
#pragma unroll
    for (int u = 0; u < ADAM_U; ++u) {
        const size_t j = base + (size_t)u * NT;
        if (j >= n4) continue;
        adam4(pp[u], gg[u], mm[u], vv[u], lr, b1, b2, eps, bc1, bc2, wd);
        __builtin_nontemporal_store(pp[u], &p[j]);
        __builtin_nontemporal_store(mm[u], &m[j]);
        __builtin_nontemporal_store(vv[u], &v[j]);
        if (pb) {
            bf16x4 b;
            b[0] = (bf16)pp[u].x; b[1] = (bf16)pp[u].y; b[2] = (bf16)pp[u].z; b[3] = (bf16)pp[u].w;
            __builtin_nontemporal_store(b, reinterpret_cast<bf16x4 *>(pb) + j);
        }
    }
    // the last n % 4 elements
    if (blockIdx.x == 0 && threadIdx.x < n - 4 * n4) {
        const size_t k = 4 * n4 + threadIdx.x;
        adam1(p_[k], g_[k], m_[k], v_[k], lr, b1, b2, eps, bc1, bc2, wd);
        if (pb) pb[k] = (bf16)p_[k];
    }
}

// Adam over the rows of a [rows, dim] table (dim % 4 == 0) whose mark is not
// `stamp`: the rows a step's tokens touched carry the stamp and are updated
// by the embedding backward once their gradient is complete, the others as
// soon as the head's weight gradient is.  Same chunking as adam_chunk_k.
__global__ __launch_bounds__(NT) void adam_rows_k(float *p_, const float *g_, float *m_, float *v_,
                                                   bf16 *pb, size_t n, unsigned dim4,
                                                   const uint32_t *mark, uint32_t stamp,
                                                   AdamHyper h) {
    const size_t n4 = n / 4;
    f32x4 *p = reinterpret_cast<f32x4 *>(p_), *m = reinterpret_cast<f32x4 *>(m_),
          *v = reinterpret_cast<f32x4 *>(v_);
    const f32x4 *g = reinterpret_cast<const f32x4 *>(g_);
    const size_t base = (size_t)blockIdx.x * (NT * ADAM_U) + threadIdx.x;
    f32x4 pp[ADAM_U], gg[ADAM_U], mm[ADAM_U], vv[ADAM_U];
    bool on[ADAM_U];
#pragma unroll
    for (int u = 0; u < ADAM_U; ++u) {
        const size_t j = base + (size_t)u * NT;
        on[u] = j < n4 && mark[j / dim4] != stamp;
        if (on[u]) {
            pp[u] = __builtin_nontemporal_load(&p[j]);
            gg[u] = __builtin_nontemporal_load(&g[j]);
            mm[u] = __builtin_nontemporal_load(&m[j]);
            vv[u] = __builtin_nontemporal_load(&v[j]);
        }
    }
#pragma unroll
    for (int u = 0; u < ADAM_U; ++u) {
        if (!on[u]) continue;
        const size_t j = base + (size_t)u * NT;
        adam4(pp[u], gg[u], mm[u], vv[u], h);
        __builtin_nontemporal_store(pp[u], &p[j]);
        __builtin_nontemporal_store(mm[u], &m[j]);
        __builtin_nontemporal_store(vv[u], &v[j]);
        if (pb) {
            bf16x4 b;
            b[0] = (bf16)pp[u].x; b[1] = (bf16)pp[u].y; b[2] = (bf16)pp[u].z; b[3] = (bf16)pp[u].w;
            __builtin_nontemporal_store(b, reinterpret_cast<bf16x4 *>(pb) + j);
        }
    }
}

// mark[ids[i]] = stamp (duplicate ids write the same value)
__global__ void mark_rows_k(const uint32_t *ids, int n, uint32_t *mark, uint32_t rows,
                            uint32_t stamp) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n && ids[i] < rows) mark[ids[i]] = stamp;
}

// Adam over a span that holds norm gains whose gradients are still per-block
// partial sums (the RMSNorm backward kernels' [nparts][stride] partials):
// blocks [0, nchunk) run the chunked update on every other element; each
// following block takes GN_COLS columns of one gain, sums their partials in
// the column-sum kernel's order (GN_GROUPS strided groups, four accumulators,
// then the groups in order), stores the gradient and updates those elements.
constexpr int GN_COLS = 16, GN_GROUPS = 16;
static_assert(GN_COLS * GN_GROUPS == NT, "gain block shape");

__global__ __launch_bounds__(NT) void adam_gains_k(float *p_, float *g_, float *m_, float *v_,
                                                    bf16 *pb, size_t n, unsigned nchunk,
                                                    AdamGains gs, float lr, float b1, float b2,
                                                    float eps, float bc1, float bc2, float wd,
                                                    unsigned nblk) {
    // blocks [0, nblk) walk the nchunk chunks; the gain blocks follow
    if (blockIdx.x < nblk) {
      for (unsigned ch = blockIdx.x; ch < nchunk; ch += nblk) {
        const size_t n4 = n / 4;
        f32x4 *p = reinterpret_cast<f32x4 *>(p_), *m = reinterpret_cast<f32x4 *>(m_),
              *v = reinterpret_cast<f32x4 *>(v_);
        const f32x4 *g = reinterpret_cast<const f32x4 *>(g_);
        const size_t base = (size_t)ch * (NT * ADAM_U) + threadIdx.x;
        auto gain_elem = [&](size_t j) {
            bool in = false;
#pragma unroll
            for (int i = 0; i < kAdamMaxGains; ++i)
                in |= i < gs.n && 4 * j - gs.g[i].off < (size_t)gs.g[i].dim;
            return in;
        };
        f32x4 pp[ADAM_U], gg[ADAM_U], mm[ADAM_U], vv[ADAM_U];
#pragma unroll
        for (int u = 0; u < ADAM_U; ++u) {
            const size_t j = base + (size_t)u * NT;
            if (j < n4 && !gain_elem(j)) {
                pp[u] = __builtin_nontemporal_load(&p[j]);
                gg[u] = __builtin_nontemporal_load(&g[j]);
                mm[u] = __builtin_nontemporal_load(&m[j]);
                vv[u] = __builtin_nontemporal_load(&v[j]);
            }
        }
#pragma unroll
        for (int u = 0; u < ADAM_U; ++u) {
            const size_t j = base + (size_t)u * NT;
            if (j >= n4 || gain_elem(j)) continue;
            adam4(pp[u], gg[u], mm[u], vv[u], lr, b1, b2, eps, bc1, bc2, wd);
            __builtin_nontemporal_store(pp[u], &p[j]);
            __builtin_nontemporal_store(mm[u], &m[j]);
            __builtin_nontemporal_store(vv[u], &v[j]);
            if (pb) {
                bf16x4 b;
                b[0] = (bf16)pp[u].x; b[1] = (bf16)pp[u].y; b[2] = (bf16)pp[u].z; b[3] = (bf16)pp[u].w;
                __builtin_nontemporal_store(b, reinterpret_cast<bf16x4 *>(pb) + j);
            }
        }
      }
        return;
    }
    // a gain block: which gain, which columns
    unsigned blk = blockIdx.x - nblk;
    int gi = 0;
    for (; gi < gs.n; ++gi) {
        const unsigned nb = (gs.g[gi].dim + GN_COLS - 1) / GN_COLS;
        if (blk < nb) break;
        blk -= nb;
    }
    if (gi >= gs.n) return;
    const AdamGain G = gs.g[gi];
    __shared__ float sh[GN_GROUPS][GN_COLS + 1];
    const int cl = threadIdx.x % GN_COLS, grp = threadIdx.x / GN_COLS;
    const int c = (int)blk * GN_COLS + cl;
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
    if (c < (int)G.dim) {
        int b = grp;
        for (; b + 3 * GN_GROUPS < G.nparts; b += 4 * GN_GROUPS) {
            a0 += G.partial[(long)b * G.stride + c];
            a1 += G.partial[(long)(b + GN_GROUPS) * G.stride + c];
            a2 += G.partial[(long)(b + 2 * GN_GROUPS) * G.stride + c];
            a3 += G.partial[(long)(b + 3 * GN_GROUPS) * G.stride + c];
        }
        for (; b < G.nparts; b += GN_GROUPS) a0 += G.partial[(long)b * G.stride + c];
    }
    sh[grp][cl] = (a0 + a1) + (a2 + a3);
    __syncthreads();
    if (grp == 0 && c < (int)G.dim) {
        float sum = 0.f;
#pragma unroll
        for (int i = 0; i < GN_GROUPS; ++i) sum += sh[i][cl];
        const size_t k = G.off + c;
        g_[k] = sum;
        adam1(p_[k], sum, m_[k], v_[k], lr, b1, b2, eps, bc1, bc2, wd);
        if (pb) pb[k] = (bf16)p_[k];
    }
}

// Unaligned spans: a grid-stride loop over scalars and float4 where aligned.
constexpr int ADAM_GRID = 256 * 32;

__global__ __launch_bounds__(NT) void adam_k(float *p_, const float *g_, float *m_, float *v_,
                                              bf16 *pb, size_t n, float lr, float b1, float b2,
                                              float eps, float bc1, float bc2, float wd, bool vec) {
    const size_t n4 = vec ? n / 4 : 0;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    f32x4 *p = reinterpret_cast<f32x4 *>(p_), *m = reinterpret_cast<f32x4 *>(m_),
          *v = reinterpret_cast<f32x4 *>(v_);
    const f32x4 *g = reinterpret_cast<const f32x4 *>(g_);
    size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    for (; i + (ADAM_U - 1) * stride < n4; i += ADAM_U * stride) {
        f32x4 pp[ADAM_U], gg[ADAM_U], mm[ADAM_U], vv[ADAM_U];
#pragma unroll
        for (int u = 0; u < ADAM_U; ++u) {
            const size_t j = i + u * stride;
            pp[u] = __builtin_nontemporal_load(&p[j]);
            gg[u] = __builtin_nontemporal_load(&g[j]);
            mm[u] = __builtin_nontemporal_load(&m[j]);
            vv[u] = __builtin_nontemporal_load(&v[j]);
        }
#pragma unroll
        for (int u = 0; u < ADAM_U; ++u) {
            const size_t j = i + u * stride;
            adam4(pp[u], gg[u], mm[u], vv[u], lr, b1, b2, eps, bc1, bc2, wd);
            __builtin_nontemporal_store(pp[u], &p[j]);
            __builtin_nontemporal_store(mm[u], &m[j]);
            __builtin_nontemporal_store(vv[u], &v[j]);
            if (pb) {
                bf16x4 b;
                b[0] = (bf16)pp[u].x; b[1] = (bf16)pp[u].y; b[2] = (bf16)pp[u].z; b[3] = (bf16)pp[u].w;
                __builtin_nontemporal_store(b, reinterpret_cast<bf16x4 *>(pb) + j);
            }
        }
    }
    for (; i < n4; i += stride) {
        f32x4 pp = p[i], mm = m[i], vv = v[i];
        adam4(pp, g[i], mm, vv, lr, b1, b2, eps, bc1, bc2, wd);
        p[i] = pp;
        m[i] = mm;
        v[i] = vv;
        if (pb) st4(pb + 4 * i, make_float4(pp.x, pp.y, pp.z, pp.w));
    }
    for (size_t k = n4 * 4 + blockIdx.x * (size_t)blockDim.x + threadIdx.x; k < n; k += stride) {
        adam1(p_[k], g_[k], m_[k], v_[k], lr, b1, b2, eps, bc1, bc2, wd);
        if (pb) pb[k] = (bf16)p_[k];
    }
}

inline bool al16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace

int cu_count() {
    static std::atomic<int> cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    int n = cached[dev].load(std::memory_order_relaxed);
    if (n <= 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
        cached[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

hipError_t fill_f32(float *p, size_t n, float v, hipStream_t st) {
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(fill_k, dim3(grid_for(n / 4 + 1)), dim3(NT), 0, st, p, n, v, al16(p));
    return hipGetLastError();
}

hipError_t add_in_place(float *dst, const float *src, size_t n, hipStream_t st) {
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(add_k, dim3(grid_for(n / 4 + 1)), dim3(NT), 0, st, dst, (const float *)dst,
                       src, n, al16(dst) && al16(src));
    return hipGetLastError();
}

hipError_t vec_add(const float *a, const float *b, float *c, size_t n, hipStream_t st) {
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(add_k, dim3(grid_for(n / 4 + 1)), dim3(NT), 0, st, c, a, b, n,
                       al16(a) && al16(b) && al16(c));
    return hipGetLastError();
}

hipError_t scale(const float *in, float *out, size_t n, float s, hipStream_t st) {
    if (!n) return hipSuccess;
    const size_t blocks = (n / 4 + NT * SC_U - 1) / (NT * SC_U);
    if (al16(in) && al16(out) && blocks >= 1 && blocks < (1u << 31)) {
        hipLaunchKernelGGL(scale_chunk_k, dim3((unsigned)blocks), dim3(NT), 0, st, in, out, n, s);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(scale_k, dim3(grid_for(n / 4 + 1)), dim3(NT), 0, st, in, out, n, s,
                       al16(in) && al16(out));
    return hipGetLastError();
}

hipError_t cast_f32_to_bf16(const float *in, bf16 *out, size_t n, hipStream_t st) {
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(cast_bf16_k, dim3(grid_for(n / 4 + 1)), dim3(NT), 0, st, in, out, n,
                       al16(in) && ((uintptr_t)out & 7u) == 0);
    return hipGetLastError();
}

hipError_t swiglu_forward(const float *pg, long ldpg, const float *up, long ldup, void *g,
                          long ldg, DType gdt, int rows, int cols, hipStream_t st) {
    if (rows <= 0 || cols <= 0) return hipSuccess;
    const bool v4 = (cols % 4 == 0) && (ldpg % 4 == 0) && (ldup % 4 == 0) && (ldg % 4 == 0) &&
                    al16(pg) && al16(up) && ((uintptr_t)g & (gdt == DType::F32 ? 15u : 7u)) == 0 &&
                    rows <= 65535;
    const unsigned gs = grid_for((size_t)rows * cols);
    const dim3 gv((unsigned)ceil_div(cols / 4, NT * SW_U), (unsigned)rows);
    if (gdt == DType::F32) {
        if (v4)
            hipLaunchKernelGGL(swiglu_fwd_k<float>, gv, dim3(NT), 0, st, pg, ldpg, up, ldup,
                               (float *)g, ldg, cols / 4);
        else
            hipLaunchKernelGGL(swiglu_fwd_s<float>, dim3(gs), dim3(NT), 0, st, pg, ldpg, up, ldup,
                               (float *)g, ldg, rows, cols);
    } else {
        if (v4)
            hipLaunchKernelGGL(swiglu_fwd_k<bf16>, gv, dim3(NT), 0, st, pg, ldpg, up, ldup,
                               (bf16 *)g, ldg, cols / 4);
        else
            hipLaunchKernelGGL(swiglu_fwd_s<bf16>, dim3(gs), dim3(NT), 0, st, pg, ldpg, up, ldup,
                               (bf16 *)g, ldg, rows, cols);
    }
    return hipGetLastError();
}

hipError_t swiglu_backward(const float *dg, long lddg, const float *pg, long ldpg,
                           const float *up, long ldup, void *dpg, long lddpg, void *dup,
                           long lddup, DType odt, int rows, int cols, hipStream_t st) {
    if (rows <= 0 || cols <= 0) return hipSuccess;
    const uintptr_t om = odt == DType::F32 ? 15u : 7u;
    const bool v4 = (cols % 4 == 0) && (lddg % 4 == 0) && (ldpg % 4 == 0) && (ldup % 4 == 0) &&
                    (lddpg % 4 == 0) && (lddup % 4 == 0) && al16(dg) && al16(pg) && al16(up) &&
                    ((uintptr_t)dpg & om) == 0 && ((uintptr_t)dup & om) == 0 && rows <= 65535;
    const unsigned gs = grid_for((size_t)rows * cols);
    const dim3 gv((unsigned)ceil_div(cols / 4, NT * SW_U), (unsigned)rows);
    if (odt == DType::F32) {
        if (v4)
            hipLaunchKernelGGL(swiglu_bwd_k<float>, gv, dim3(NT), 0, st, dg, lddg, pg, ldpg,
                               up, ldup, (float *)dpg, lddpg, (float *)dup, lddup, cols / 4);
        else
            hipLaunchKernelGGL(swiglu_bwd_s<float>, dim3(gs), dim3(NT), 0, st, dg, lddg, pg, ldpg,
                               up, ldup, (float *)dpg, lddpg, (float *)dup, lddup, rows, cols);
    } else {
        if (v4)
            hipLaunchKernelGGL(swiglu_bwd_k<bf16>, gv, dim3(NT), 0, st, dg, lddg, pg, ldpg,
                               up, ldup, (bf16 *)dpg, lddpg, (bf16 *)dup, lddup, cols / 4);
        else
            hipLaunchKernelGGL(swiglu_bwd_s<bf16>, dim3(gs), dim3(NT), 0, st, dg, lddg, pg, ldpg,
                               up, ldup, (bf16 *)dpg, lddpg, (bf16 *)dup, lddup, rows, cols);
    }
    return hipGetLastError();
}

hipError_t embed_lookup(const float *embed, const uint32_t *ids, float *out, int n_pos, int dim,
                        float scale_, hipStream_t st) {
    if (n_pos <= 0 || dim <= 0) return hipSuccess;
    const bool v4 = (dim % 4 == 0) && al16(embed) && al16(out);
    hipLaunchKernelGGL(embed_lookup_k, dim3(grid_for((size_t)n_pos * dim / (v4 ? 4 : 1))), dim3(NT),
                       0, st, embed, ids, out, n_pos, dim, scale_, v4);
    return hipGetLastError();
}

hipError_t embed_lookup_bf16(const bf16 *embed, const uint32_t *ids, float *out, int n_pos,
                             int dim, float scale_, hipStream_t st) {
    if (n_pos <= 0 || dim <= 0) return hipSuccess;
    if (dim % 4 || ((uintptr_t)embed & 7u) || !al16(out)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(embed_lookup_bf16_k, dim3(grid_for((size_t)n_pos * dim / 4)), dim3(NT), 0, st,
                       embed, ids, out, n_pos, dim, scale_);
    return hipGetLastError();
}

hipError_t adam_step_gains(float *p, float *g, float *m, float *v, size_t n, float lr, float beta1,
                           float beta2, float eps, float bc1, float bc2, float wd, bf16 *pb,
                           const AdamGains &gs, hipStream_t st, unsigned max_blocks) {
    if (!n) return hipSuccess;
    const bool vec = al16(p) && al16(g) && al16(m) && al16(v) && ((uintptr_t)pb & 7u) == 0 &&
                     n % 4 == 0;
    unsigned gain_blocks = 0;
    for (int i = 0; i < gs.n; ++i) {
        // whole float4 vectors inside the span
        if (gs.g[i].off % 4 || gs.g[i].dim % 4 || gs.g[i].off + gs.g[i].dim > n) return hipErrorInvalidValue;
        gain_blocks += ceil_div(gs.g[i].dim, GN_COLS);
    }
    if (!vec || gs.n > kAdamMaxGains) return hipErrorInvalidValue;
    const size_t nchunk = std::max<size_t>(1, (n / 4 + NT * ADAM_U - 1) / (NT * ADAM_U));
    if (nchunk + gain_blocks >= (1u << 31)) return hipErrorInvalidValue;
    const unsigned nblk = (unsigned)(max_blocks ? std::min<size_t>(nchunk, max_blocks) : nchunk);
    hipLaunchKernelGGL(adam_gains_k, dim3(nblk + gain_blocks), dim3(NT), 0, st, p, g, m, v, pb, n,
                       (unsigned)nchunk, gs, lr, beta1, beta2, eps, bc1, bc2, wd, nblk);
    return hipGetLastError();
}

hipError_t adam_step(float *p, const float *g, float *m, float *v, size_t n, float lr,
                     float beta1, float beta2, float eps, float bc1, float bc2, float wd,
                     bf16 *pb, hipStream_t st) {
    if (!n) return hipSuccess;
    const bool vec = al16(p) && al16(g) && al16(m) && al16(v) && ((uintptr_t)pb & 7u) == 0;
    if (vec) {
        const size_t blocks = std::max<size_t>(1, (n / 4 + NT * ADAM_U - 1) / (NT * ADAM_U));
        if (blocks < (1u << 31)) {
            hipLaunchKernelGGL(adam_chunk_k, dim3((unsigned)blocks), dim3(NT), 0, st, p, g, m, v, pb,
                               n, lr, beta1, beta2, eps, bc1, bc2, wd);
            return hipGetLastError();
        }
    }
    size_t grid = (n / 4 + NT - 1) / NT;
    grid = grid < 1 ? 1 : (grid > ADAM_GRID ? ADAM_GRID : grid);
    hipLaunchKernelGGL(adam_k, dim3((unsigned)grid), dim3(NT), 0, st, p, g, m, v, pb, n, lr,
                       beta1, beta2, eps, bc1, bc2, wd, vec);
    return hipGetLastError();
}

hipError_t adam_rows_unmarked(float *p, const float *g, float *m, float *v, bf16 *pb, int rows,
                              int dim, const uint32_t *mark, uint32_t stamp, const AdamHyper &h,
                              hipStream_t st) {
    if (rows <= 0 || dim <= 0) return hipSuccess;
    const size_t n = (size_t)rows * dim;
    const bool vec = al16(p) && al16(g) && al16(m) && al16(v) && ((uintptr_t)pb & 7u) == 0;
    if (!vec || dim % 4 || !mark) return hipErrorInvalidValue;
    const size_t blocks = (n / 4 + NT * ADAM_U - 1) / (NT * ADAM_U);
    if (blocks >= (1u << 31)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(adam_rows_k, dim3((unsigned)blocks), dim3(NT), 0, st, p, g, m, v, pb, n,
                       (unsigned)(dim / 4), mark, stamp, h);
    return hipGetLastError();
}

hipError_t mark_rows(const uint32_t *ids, int n, uint32_t *mark, int rows, uint32_t stamp,
                     hipStream_t st) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(mark_rows_k, dim3(ceil_div(n, NT)), dim3(NT), 0, st, ids, n, mark,
                       (uint32_t)rows, stamp);
    return hipGetLastError();
}

}  // namespace vkh
