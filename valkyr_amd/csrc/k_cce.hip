// Cut cross-entropy over the vocabulary (reference: shaders/cce_forward.comp,
// cce_backward_dh.comp, cce_backward_dw.comp; oracle src/cpu/cce.zig:89-268).
//
// Forward: the logits z = h W^T are produced tile by tile by the MFMA GEMM
// and never stored; its epilogue reduces each wave's 64-column slice of a row
// to (max, sum exp(z - max), sum z) and captures the target logit.  A second
// kernel merges the slices per row (fp64) into lse and the per-row loss
// lse - (1 - eps) z_t - eps mean(z) + lambda_z lse^2, and a third averages.
//
// Backward: the logits are recomputed once by the GEMM whose epilogue writes
//   dz = ((1 + 2 lambda_z lse) exp(z - lse) - (1 - eps)[v == t] - eps / V) / N
// (bf16 in the bf16 precision, fp32 otherwise) to HBM, then two MFMA GEMMs
// form dh = dz W and dW = dz^T h.  The reference recomputes the logits twice
// with scalar dot products (per row for dh, per vocab row for dW,
// cce_backward_dh.comp:109-123, cce_backward_dw.comp:73-103); on a 288 GB
// part the [N, V] dz buffer (0.6 GB at N = 2048) is cheap and turns the
// backward into three dense GEMMs.
//
// With fp32 dz (the fp32 precision) the forward's epilogue can also store the
// fp32 logits into the dz buffer (z_out), and the backward then forms dz from
// them in place with one streaming pass (cce_dz_k, the dz epilogue's
// arithmetic element by element) instead of recomputing the logits GEMM: the
// same values bit for bit, 2.5 GB of traffic in place of a 0.64 TFLOP product.
#include "gemm16.hpp"
#include "ops.hpp"

namespace vkh {

namespace {

constexpr int WN = 64;  // columns per wave slice with the 128x128 tile
constexpr float LOG2E = 1.4426950408889634f;

struct CceWork {
    float *pm, *ps, *pz;  // [N][nparts]
    float *zt;            // [N]
    int nparts;
};

inline CceWork carve(float *work, const CceShape &s) {
    const int np = (s.V + WN - 1) / WN;
    const size_t part = (size_t)s.N * np;
    return CceWork{work, work + part, work + 2 * part, work + 3 * part, np};
}

struct EpiCceStats {
    CceWork w;
    const uint32_t *tgt;
    int V;
    float *zo = nullptr;  // when set: the logits themselves, [N, V] row-major

    template <int TM, int TN>
    VKH_DEV void apply(const f32x4 (&acc)[TM][TN], const FragPos &fp, const GemmShape &s) const {
        static_assert(TN * 16 == WN, "wave slice width");
        const int part = fp.col0 / WN;
        // the last tile's second slice can lie wholly past V: it owns no partial
        if (part >= w.nparts) return;
        // slices wholly inside the vocabulary (all but the last) skip the
        // per-column range checks
        if (fp.col0 + WN <= V) rows<TM, TN, true>(acc, fp, s, part);
        else rows<TM, TN, false>(acc, fp, s, part);
    }

    template <int TM, int TN, bool FULL>
    VKH_DEV void rows(const f32x4 (&acc)[TM][TN], const FragPos &fp, const GemmShape &s,
                      int part) const {
        const int c16 = fp.lane % 16, g = fp.lane / 16;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = fp.row0 + 16 * i + 4 * g + r;
                const bool rok = row < s.M;
                // the target column relative to this lane's first column: the
                // lane of fragment j holds it when tc == 16 j
                const int tc = rok ? (int)tgt[row] - fp.col0 - c16 : -1;
                float mx = -INFINITY, zs = 0.f;
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    if (FULL || fp.col0 + 16 * j + c16 < V) {
                        const float z = acc[i][j][r];
                        mx = fmaxf(mx, z);
                        zs += z;
                        if (tc == 16 * j) w.zt[row] = z;
                        if (zo && rok) zo[(size_t)row * V + fp.col0 + 16 * j + c16] = z;
                    }
                }
                mx = row16_max(mx);
                const float mxl = mx * LOG2E;
                float se = 0.f;
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    if (FULL || fp.col0 + 16 * j + c16 < V)
                        se += __builtin_amdgcn_exp2f(fmaf(acc[i][j][r], LOG2E, -mxl));
                se = row16_sum(se);
                zs = row16_sum(zs);
                if (rok && c16 == 0) {
                    const size_t idx = (size_t)row * w.nparts + part;
                    w.pm[idx] = mx;
                    w.ps[idx] = se;
                    w.pz[idx] = zs;
                }
            }
    }
};

// dz of one row: the coefficients of dz = sf exp(z - lse) - off - [v == t] tsc
// (the 1 / N folded in), and one element of it.  The dz epilogue and cce_dz_k
// both compute through these, so their results agree bit for bit.
struct DzRow {
    float lL2, sf;
};
VKH_DEV DzRow dz_row(float l, float zl2, float inv_n) { return DzRow{l * LOG2E, (1.0f + zl2 * l) * inv_n}; }
VKH_DEV float dz_elem(float z, const DzRow &r, float off, float tsc, bool is_t) {
    const float p = __builtin_amdgcn_exp2f(fmaf(z, LOG2E, -r.lL2));
    float d = fmaf(r.sf, p, -off);
    if (is_t) d -= tsc;
    return d;
}

template <typename TZ>
struct EpiCceDz {
    TZ *dz;
    const uint32_t *tgt;
    const float *lse;
    int V;
    float inv_n, t_scale, eps_over_v, zl2;

    template <int TM, int TN>
    VKH_DEV void apply(const f32x4 (&acc)[TM][TN], const FragPos &fp, const GemmShape &s) const {
        if (fp.col0 + 16 * TN <= V) rows<TM, TN, true>(acc, fp, s);
        else rows<TM, TN, false>(acc, fp, s);
    }

    // dz = (sf p - eps / V - [v == t] (1 - eps)) / N with p = exp(z - lse),
    // sf = 1 + 2 lambda_z lse; the 1 / N folded into the coefficients
    template <int TM, int TN, bool FULL>
    VKH_DEV void rows(const f32x4 (&acc)[TM][TN], const FragPos &fp, const GemmShape &s) const {
        const int c16 = fp.lane % 16, g = fp.lane / 16;
        const float off = eps_over_v * inv_n, tsc = t_scale * inv_n;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = fp.row0 + 16 * i + 4 * g + r;
                if (row >= s.M) continue;
                const DzRow dr = dz_row(lse[row], zl2, inv_n);
                const int tc = (int)tgt[row] - fp.col0 - c16;
                TZ *out = dz + (size_t)row * V + fp.col0 + c16;
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    if (!FULL && fp.col0 + 16 * j + c16 >= V) continue;
                    out[16 * j] = (TZ)dz_elem(acc[i][j][r], dr, off, tsc, tc == 16 * j);
                }
            }
    }
};

// dz from the stored fp32 logits z [N, V] (z and dz may be the same buffer: each
// element is read and then written by one thread).  Block (x, row): 4 columns
// per thread with 16-byte rows (V % 4 == 0 and 16-byte aligned), else 1.
template <typename TZ, int VEC>
__global__ __launch_bounds__(256) void cce_dz_k(const float *z, TZ *dz, const uint32_t *tgt,
                                                const float *lse, int V, float inv_n, float t_scale,
                                                float eps_over_v, float zl2) {
    const int row = blockIdx.y;
    const int c0 = (blockIdx.x * 256 + threadIdx.x) * VEC;
    if (c0 >= V) return;
    const DzRow dr = dz_row(lse[row], zl2, inv_n);
    const float off = eps_over_v * inv_n, tsc = t_scale * inv_n;
    const int t = (int)tgt[row];
    const size_t i = (size_t)row * V + c0;
    if constexpr (VEC == 4) {
        const float4 zv = *reinterpret_cast<const float4 *>(z + i);
        const float d0 = dz_elem(zv.x, dr, off, tsc, t == c0), d1 = dz_elem(zv.y, dr, off, tsc, t == c0 + 1),
                    d2 = dz_elem(zv.z, dr, off, tsc, t == c0 + 2), d3 = dz_elem(zv.w, dr, off, tsc, t == c0 + 3);
        if constexpr (sizeof(TZ) == 4) {
            *reinterpret_cast<float4 *>(dz + i) = make_float4(d0, d1, d2, d3);
        } else {
            dz[i] = (TZ)d0; dz[i + 1] = (TZ)d1; dz[i + 2] = (TZ)d2; dz[i + 3] = (TZ)d3;
        }
    } else {
        dz[i] = (TZ)dz_elem(z[i], dr, off, tsc, t == c0);
    }
}

__global__ void cce_merge_k(CceShape s, CceWork w, float *lse, float *loss_row) {
    const int lane = threadIdx.x % 64;
    const int row = blockIdx.x * (blockDim.x / 64) + threadIdx.x / 64;
    if (row >= s.N) return;
    const float *pm = w.pm + (size_t)row * w.nparts;
    const float *ps = w.ps + (size_t)row * w.nparts;
    const float *pz = w.pz + (size_t)row * w.nparts;
    float M = -INFINITY;
    for (int i = lane; i < w.nparts; i += 64) M = fmaxf(M, pm[i]);
    M = wave_max(M);
    double S = 0, Z = 0;
    for (int i = lane; i < w.nparts; i += 64) {
        S += (double)ps[i] * exp((double)pm[i] - (double)M);
        Z += (double)pz[i];
    }
    S = wave_sum(S);
    Z = wave_sum(Z);
    if (lane == 0) {
        const float l = (float)(log(S) + (double)M);
        lse[row] = l;
        const double eps = s.label_smoothing;
        const double ce = (double)l - (double)(1.0f - s.label_smoothing) * (double)w.zt[row] -
                          eps * (Z / (double)s.V);
        const double zp = (double)s.z_loss_scale * (double)l * (double)l;
        if (loss_row) loss_row[row] = (float)(ce + zp);
        w.pm[(size_t)row * w.nparts] = (float)(ce + zp);  // reuse slot 0 for the mean
    }
}

__global__ void cce_mean_k(CceShape s, CceWork w, float *loss_mean) {
    __shared__ double sh[4];
    double acc = 0;
    for (int r = threadIdx.x; r < s.N; r += blockDim.x) acc += (double)w.pm[(size_t)r * w.nparts];
    acc = wave_sum(acc);
    if (threadIdx.x % 64 == 0) sh[threadIdx.x / 64] = acc;
    __syncthreads();
    if (threadIdx.x == 0) loss_mean[0] = (float)((sh[0] + sh[1] + sh[2] + sh[3]) / (double)s.N);
}

template <class Epi>
hipError_t logits_gemm(Precision pr, const CceShape &s, const float *h, const float *w,
                       const Epi &epi, hipStream_t st) {
    GemmOperand a{h, s.D, vec_ok(h, s.D, 4, Lay::K)};
    GemmOperand b{w, s.D, vec_ok(w, s.D, 4, Lay::K)};
    GemmShape sh{s.N, s.V, s.D};
    if (pr == Precision::BF16)
        return launch_gemm<TileCfg<128, 128, 64>, true, float, Lay::K, float, Lay::K>(a, b, sh, epi, st);
    // fp32: the DMA-staged 256 x 256 tile on the fp32 matrix cores (64-column
    // wave slices, as the epilogues need) where the operands fit its rules
    const size_t hb = ((size_t)(s.N - 1) * s.D + s.D) * 4, wb = ((size_t)(s.V - 1) * s.D + s.D) * 4;
    if (s.D % 4 == 0 && ((uintptr_t)h & 15u) == 0 && ((uintptr_t)w & 15u) == 0 &&
        hb < (1ull << 31) && wb < (1ull << 31)) {
        const Op16 a16{(const bf16 *)h, s.D, (unsigned)hb}, b16{(const bf16 *)w, s.D, (unsigned)wb};
        const SplitK one{1, nullptr};
        return launch_gemm16<Tile16<256, 256, 2, 4>, Lay::K, Lay::K, Epi, true>(
            a16, b16, sh, epi, one, tile_group_rows<Lay::K, Lay::K>(), st);
    }
    return launch_gemm<TileCfg<128, 128, 32>, false, float, Lay::K, float, Lay::K>(a, b, sh, epi, st);
}

// bf16 operands: the gemm16 kernel with 64-column wave slices (8 waves in a
// 2 x 4 grid), falling back to the generic MFMA GEMM for unaligned shapes.
template <class Epi>
hipError_t logits16(const CceShape &s, const bf16 *h, const bf16 *w, const Epi &epi,
                    hipStream_t st) {
    GemmShape sh{s.N, s.V, s.D};
    const size_t hb = ((size_t)(s.N - 1) * s.D + s.D) * 2, wb = ((size_t)(s.V - 1) * s.D + s.D) * 2;
    const bool ok = s.D % 8 == 0 && ((uintptr_t)h & 15u) == 0 && ((uintptr_t)w & 15u) == 0 &&
                    hb < (1ull << 31) && wb < (1ull << 31);
    if (!ok) {
        GemmOperand a{h, s.D, vec_ok(h, s.D, 2, Lay::K)};
        GemmOperand b{w, s.D, vec_ok(w, s.D, 2, Lay::K)};
        return launch_gemm<TileCfg<128, 128, 64>, true, bf16, Lay::K, bf16, Lay::K>(a, b, sh, epi, st);
    }
    const Op16 a{h, s.D, (unsigned)hb}, b{w, s.D, (unsigned)wb};
    const SplitK one{1, nullptr};
    constexpr int g = tile_group_rows<Lay::K, Lay::K>();
    if ((long)ceil_div(s.N, 256) * ceil_div(s.V, 256) >= 256)
        return launch_gemm16<Tile16<256, 256, 2, 4>, Lay::K, Lay::K>(a, b, sh, epi, one, g, st);
    return launch_gemm16<Tile16<128, 256, 2, 4>, Lay::K, Lay::K>(a, b, sh, epi, one, g, st);
}

}  // namespace

size_t cce_work_floats(const CceShape &s) {
    const size_t np = (s.V + WN - 1) / WN;
    return 3 * (size_t)s.N * np + s.N;
}

hipError_t cce_forward(Precision pr, const CceShape &s, const float *h, const float *w,
                       const uint32_t *tgt, float *lse, float *loss_row, float *loss_mean,
                       float *work, hipStream_t st, float *z_out) {
    if (s.N <= 0) return hipSuccess;
    CceWork cw = carve(work, s);
    EpiCceStats e{cw, tgt, s.V, z_out};
    hipError_t err = logits_gemm(pr, s, h, w, e, st);
    if (err != hipSuccess) return err;
    hipLaunchKernelGGL(cce_merge_k, dim3(ceil_div(s.N, 4)), dim3(256), 0, st, s, cw, lse, loss_row);
    if (loss_mean) hipLaunchKernelGGL(cce_mean_k, dim3(1), dim3(256), 0, st, s, cw, loss_mean);
    return hipGetLastError();
}

hipError_t cce_backward(Precision pr, const CceShape &s, const float *h, const float *w,
                        const uint32_t *tgt, const float *lse, void *dz, float *dh, float *dw,
                        float dw_beta, hipStream_t st, const float *z) {
    if (s.N <= 0) return hipSuccess;
    const float inv_n = 1.0f / (float)s.N;
    const float t_scale = 1.0f - s.label_smoothing;
    const float eps_over_v = s.label_smoothing / (float)s.V;
    const float zl2 = 2.0f * s.z_loss_scale;
    hipError_t err;
    const DType zdt = pr == Precision::BF16 ? DType::BF16 : DType::F32;
    if (z) {  // the logits the forward stored: dz in one streaming pass
        const bool v4 = s.V % 4 == 0 && ((uintptr_t)z & 15u) == 0 && ((uintptr_t)dz & 15u) == 0;
        const dim3 grid((unsigned)ceil_div(s.V, 256 * (v4 ? 4 : 1)), (unsigned)s.N);
        if (zdt == DType::BF16) {
            if (v4) hipLaunchKernelGGL((cce_dz_k<bf16, 4>), grid, dim3(256), 0, st, z, (bf16 *)dz, tgt, lse, s.V, inv_n, t_scale, eps_over_v, zl2);
            else hipLaunchKernelGGL((cce_dz_k<bf16, 1>), grid, dim3(256), 0, st, z, (bf16 *)dz, tgt, lse, s.V, inv_n, t_scale, eps_over_v, zl2);
        } else {
            if (v4) hipLaunchKernelGGL((cce_dz_k<float, 4>), grid, dim3(256), 0, st, z, (float *)dz, tgt, lse, s.V, inv_n, t_scale, eps_over_v, zl2);
            else hipLaunchKernelGGL((cce_dz_k<float, 1>), grid, dim3(256), 0, st, z, (float *)dz, tgt, lse, s.V, inv_n, t_scale, eps_over_v, zl2);
        }
        err = hipGetLastError();
    } else if (zdt == DType::BF16) {
        EpiCceDz<bf16> e{(bf16 *)dz, tgt, lse, s.V, inv_n, t_scale, eps_over_v, zl2};
        err = logits_gemm(pr, s, h, w, e, st);
    } else {
        EpiCceDz<float> e{(float *)dz, tgt, lse, s.V, inv_n, t_scale, eps_over_v, zl2};
        err = logits_gemm(pr, s, h, w, e, st);
    }
    if (err != hipSuccess) return err;
    const Mat mz{dz, s.V, zdt};
    if (zdt == DType::F32) {  // fp32: the DMA-staged fp32 kernels (generic where they do not apply)
        const GemmWs none{nullptr, 0};
        if (dw) {
            err = g32_tn((const float *)dz, s.V, h, s.D, dw, s.D, s.N, s.V, s.D, 1.f, dw_beta, none, st);
            if (err != hipSuccess) return err;
        }
        if (dh) err = g32_nn((const float *)dz, s.V, w, s.D, dh, s.D, s.N, s.V, s.D, 1.f, 0.f, none, st);
        return err;
    }
    if (dw) {
        err = gemm_tn(pr, mz, matf(h, s.D), dw, s.D, s.N, s.V, s.D, 1.f, dw_beta, st);
        if (err != hipSuccess) return err;
    }
    if (dh) err = gemm_nn(pr, mz, matf(w, s.D), dh, s.D, s.N, s.V, s.D, 1.f, 0.f, st);
    return err;
}

}  // namespace vkh

namespace vkh {

hipError_t cce_forward16(const CceShape &s, const bf16 *h, const bf16 *w, const uint32_t *tgt,
                         float *lse, float *loss_row, float *loss_mean, float *work,
                         hipStream_t st, float *z_out) {
    if (s.N <= 0) return hipSuccess;
    CceWork cw = carve(work, s);
    EpiCceStats e{cw, tgt, s.V, z_out};
    hipError_t err = logits16(s, h, w, e, st);
    if (err != hipSuccess) return err;
    hipLaunchKernelGGL(cce_merge_k, dim3(ceil_div(s.N, 4)), dim3(256), 0, st, s, cw, lse, loss_row);
    if (loss_mean) hipLaunchKernelGGL(cce_mean_k, dim3(1), dim3(256), 0, st, s, cw, loss_mean);
    return hipGetLastError();
}

hipError_t cce_backward16(const CceShape &s, const bf16 *h, const bf16 *w, const uint32_t *tgt,
                          const float *lse, bf16 *dz, float *dh, float *dw, float dw_beta,
                          const GemmWs &ws, hipStream_t st, const float *z) {
    if (s.N <= 0) return hipSuccess;
    EpiCceDz<bf16> e{dz, tgt, lse, s.V, 1.0f / (float)s.N, 1.0f - s.label_smoothing,
                     s.label_smoothing / (float)s.V, 2.0f * s.z_loss_scale};
    hipError_t err;
    if (z) {
        const bool v4 = s.V % 4 == 0 && ((uintptr_t)z & 15u) == 0;
        const dim3 grid((unsigned)ceil_div(s.V, 256 * (v4 ? 4 : 1)), (unsigned)s.N);
        if (v4) hipLaunchKernelGGL((cce_dz_k<bf16, 4>), grid, dim3(256), 0, st, z, dz, tgt, lse, s.V, e.inv_n, e.t_scale, e.eps_over_v, e.zl2);
        else hipLaunchKernelGGL((cce_dz_k<bf16, 1>), grid, dim3(256), 0, st, z, dz, tgt, lse, s.V, e.inv_n, e.t_scale, e.eps_over_v, e.zl2);
        err = hipGetLastError();
    } else {
        err = logits16(s, h, w, e, st);
    }
    if (err != hipSuccess) return err;
    // dW[V, D] = dz^T h ;  dh[N, D] = dz W
    if (dw) {
        err = g16_tn(dz, s.V, h, s.D, dw, s.D, s.N, s.V, s.D, 1.f, dw_beta, ws, st);
        if (err != hipSuccess) return err;
    }
    if (dh) err = g16_nn(dz, s.V, w, s.D, dh, s.D, s.N, s.V, s.D, 1.f, 0.f, ws, st);
    return err;
}

}  // namespace vkh
