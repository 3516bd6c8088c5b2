// Tiny-MLP TrainingRunner: the per-frame trainer of src/train/runner.zig
// (Linear -> ReLU -> Linear, hidden <= 64) behind the vkh_mlp_* C ABI.
//
// The reference records 11 dispatches per batched step (forward, dy, dh_pre,
// four outer-product / bias accumulators, four optimizer steps,
// runner.zig:1048-1200) with a global barrier after each.  Here a step is
// ONE launch while the batch fits a workgroup's LDS: a 256-thread block
// stages the weights (hidden axis padded, W1 transposed) and the batch
// (feature-major) in LDS, runs every sample's forward + loss gradient +
// backward (one thread per sample, the hidden vector in registers), then,
// after a block barrier, reduces every parameter's gradient over the batch
// (one thread per parameter, four samples per 16-byte LDS read) and applies
// SGD / Adam.  Larger batches use a per-sample kernel (64 samples per block,
// weights in LDS) plus a reduction/update kernel, split over sample chunks
// and summed in chunk order so that results do not depend on scheduling.
// Weights too large for LDS are read from a packed copy in HBM.
//
// Layout in HBM: parameters, gradients and Adam m / v are each one blob
// [W1 (H x I) | b1 (H) | W2 (O x H) | b2 (O)], so one thread index addresses
// any parameter and the optimizer runs inside the reducing kernel.  Batch
// activations are sample-major [N, dim] as in the reference's batched
// shaders.  One-sample calls read x / target from pinned host memory and
// write the prediction there, so a blocking step is one launch and one
// synchronization.  All arithmetic is fp32, as in the reference.
//
// Work per step is a few thousand FLOPs per sample: nothing here is HBM- or
// MFMA-bound at the sizes this runner is for; what costs is launches, memory
// round trips and host synchronization, which is what the design removes.
#include <math.h>
#include <string.h>

#include <algorithm>
#include <chrono>
#include <vector>

#include "internal.hpp"

namespace vkh {
namespace mlp {

constexpr int kMaxHidden = VKH_MLP_MAX_HIDDEN;
static_assert(kMaxHidden == 64, "the hidden-width buckets of by_hb end at 64");
constexpr int kBlock = 256;       // threads of the fused / reduction kernels
constexpr int kFwdBlock = 64;     // threads (samples) per block of the per-sample kernel
constexpr int kChunk = 256;       // samples per partial sum when the batch is split
constexpr int kFusedMaxN = 1024;  // fused single-block step up to this batch ...
constexpr size_t kFusedMaxWork = size_t(1) << 18;  // ... and N * params
constexpr size_t kLdsFloats = 16384;                // 64 KB of dynamic LDS per block
constexpr int kRing = 32;  // pinned x / target slots of the one-sample record calls

enum { MSE = 0, CE = 1 };
enum { SGD = 0, ADAM = 1 };
enum { PREDICT = 0, TRAIN_MSE = 1, TRAIN_CE = 2 };

// Dimensions and blob offsets (floats).
struct Shape {
    int I, H, O;
    int w1, b1, w2, b2, n;
};

static Shape make_shape(int I, int H, int O) {
    Shape s;
    s.I = I; s.H = H; s.O = O;
    s.w1 = 0;
    s.b1 = H * I;
    s.w2 = s.b1 + H;
    s.b2 = s.w2 + O * H;
    s.n = s.b2 + O;
    return s;
}

struct Opt {
    float lr, wd, beta1, beta2, eps, bc1, bc2;
};

// Weights staged in LDS, hidden axis padded to the bucket HB (a multiple of
// 4, zero-filled) so every hidden-axis read is a 16-byte ds_read:
//   w1t [I][HB] = W1 transposed, b1 [HB], w2 [O][HB], b2 [O].
struct WOff {
    int w1t, b1, w2, b2, end;
};

__host__ __device__ inline WOff woff(const Shape &s, int HB) {
    WOff w;
    w.w1t = 0;
    w.b1 = s.I * HB;
    w.w2 = w.b1 + HB;
    w.b2 = w.w2 + s.O * HB;
    w.end = w.b2 + ((s.O + 3) & ~3);
    return w;
}

// Element f of the padded weight layout, gathered from the parameter blob.
template <int HB>
VKH_DEV float weight_at(const float *P, const Shape &s, const WOff &w, int f) {
    if (f < w.b1) {
        const int i = f / HB, j = f - i * HB;
        return j < s.H ? P[s.w1 + (size_t)j * s.I + i] : 0.f;
    }
    if (f < w.w2) {
        const int j = f - w.b1;
        return j < s.H ? P[s.b1 + j] : 0.f;
    }
    if (f < w.b2) {
        const int q = f - w.w2, o = q / HB, j = q - o * HB;
        return j < s.H ? P[s.w2 + (size_t)o * s.H + j] : 0.f;
    }
    const int o = f - w.b2;
    return o < s.O ? P[s.b2 + o] : 0.f;
}

// dst[f] = fetch(f) for f in [0, E), threads tid, tid + nt, ...: each round
// issues kStageU loads before any store, so the whole staging costs one or
// two memory round trips rather than one per element.
constexpr int kStageU = 8;
template <class F>
VKH_DEV void stage(float *dst, int E, int tid, int nt, F fetch) {
    for (int base = tid; base < E; base += kStageU * nt) {
        float v[kStageU];
#pragma unroll
        for (int u = 0; u < kStageU; ++u) {
            const int f = base + u * nt;
            v[u] = f < E ? fetch(f) : 0.f;
        }
#pragma unroll
        for (int u = 0; u < kStageU; ++u) {
            const int f = base + u * nt;
            if (f < E) dst[f] = v[u];
        }
    }
}

// The padded weight layout into dst (a block's LDS, or HBM when the weights
// do not fit LDS).
template <int HB>
VKH_DEV void stage_weights(const float *P, const Shape &s, float *dst, int tid, int nt) {
    const WOff w = woff(s, HB);
    stage(dst, w.end, tid, nt, [&](int f) { return weight_at<HB>(P, s, w, f); });
}

// h_pre = W1 x + b1 for one sample: b1 first, then i ascending
// (cpu/train.zig:154-162, mlp2_forward_train_batched.comp).  Padded hidden
// units stay exactly 0.
template <int HB>
VKH_DEV void layer1(const float *lw, const Shape &s, const float *x, int xs, float (&hp)[HB]) {
    const WOff w = woff(s, HB);
    const f32x4 *b1 = (const f32x4 *)(lw + w.b1);
#pragma unroll
    for (int j = 0; j < HB / 4; ++j) {
        const f32x4 b = b1[j];
        hp[4 * j] = b[0]; hp[4 * j + 1] = b[1]; hp[4 * j + 2] = b[2]; hp[4 * j + 3] = b[3];
    }
    for (int i = 0; i < s.I; ++i) {
        const float xi = x[i * xs];
        const f32x4 *wr = (const f32x4 *)(lw + w.w1t + i * HB);
#pragma unroll
        for (int j = 0; j < HB / 4; ++j) {
            const f32x4 v = wr[j];
            hp[4 * j] += v[0] * xi;
            hp[4 * j + 1] += v[1] * xi;
            hp[4 * j + 2] += v[2] * xi;
            hp[4 * j + 3] += v[3] * xi;
        }
    }
}

// y[o] = W2[o,:] h + b2[o] (cpu/train.zig:165-172).
template <int HB>
VKH_DEV float layer2_row(const float *lw, const Shape &s, int o, const float (&hv)[HB]) {
    const WOff w = woff(s, HB);
    const f32x4 *wr = (const f32x4 *)(lw + w.w2 + o * HB);
    float acc = lw[w.b2 + o];
#pragma unroll
    for (int j = 0; j < HB / 4; ++j) {
        const f32x4 v = wr[j];
        acc += v[0] * hv[4 * j];
        acc += v[1] * hv[4 * j + 1];
        acc += v[2] * hv[4 * j + 2];
        acc += v[3] * hv[4 * j + 3];
    }
    return acc;
}

template <int HB>
VKH_DEV void dh_accum(const float *lw, const Shape &s, int o, float d, float (&dh)[HB]) {
    const f32x4 *wr = (const f32x4 *)(lw + woff(s, HB).w2 + o * HB);
#pragma unroll
    for (int j = 0; j < HB / 4; ++j) {
        const f32x4 v = wr[j];
        dh[4 * j] += d * v[0];
        dh[4 * j + 1] += d * v[1];
        dh[4 * j + 2] += d * v[2];
        dh[4 * j + 3] += d * v[3];
    }
}

template <int HB>
VKH_DEV void relu(const float (&hp)[HB], float (&hv)[HB]) {
#pragma unroll
    for (int j = 0; j < HB; ++j) hv[j] = hp[j] > 0.f ? hp[j] : 0.f;
}

// Per-sample outputs: global (inspection buffers, and the input of the
// reduction kernels) and, in the fused kernel, feature-major LDS copies
// (element (n, j) at j * ls + n) for its second phase.  Any pointer may be
// null.
struct SampleOut {
    float *h_pre, *h, *y, *dy, *dhp;  // global [N, dim]
    float *y_host;                    // pinned host [N, O]
    float *l_h, *l_dy, *l_dhp;        // LDS [dim][ls]
    int ls;
};

// One sample of a training step: forward, dy = dL/dy / N (MSE:
// mlp2_dy_batched.comp; CE: softmax_ce_loss_grad_batched.comp), and
// dh_pre = (W2^T dy) * 1[h_pre > 0] (mlp2_dh_pre_batched.comp).
template <int HB, int LOSS>
VKH_DEV void train_sample(const float *lw, const Shape &s, int n, const float *xn, int xs,
                          const float *tn, int ts, float inv_n, const SampleOut &out) {
    float hp[HB], hv[HB], dh[HB];
    layer1<HB>(lw, s, xn, xs, hp);
    relu<HB>(hp, hv);
    const size_t nH = (size_t)n * s.H, nO = (size_t)n * s.O;
#pragma unroll
    for (int j = 0; j < HB; ++j) {
        dh[j] = 0.f;
        if (j < s.H) {
            if (out.h_pre) out.h_pre[nH + j] = hp[j];
            if (out.h) out.h[nH + j] = hv[j];
            if (out.l_h) out.l_h[j * out.ls + n] = hv[j];
        }
    }
    float m = -INFINITY, inv_sum = 0.f;
    if (LOSS == CE) {
        for (int o = 0; o < s.O; ++o) m = fmaxf(m, layer2_row<HB>(lw, s, o, hv));
        float sum_e = 0.f;
        for (int o = 0; o < s.O; ++o) sum_e += expf(layer2_row<HB>(lw, s, o, hv) - m);
        inv_sum = 1.f / sum_e;
    }
    for (int o = 0; o < s.O; ++o) {
        const float yo = layer2_row<HB>(lw, s, o, hv);
        if (out.y) out.y[nO + o] = yo;
        if (out.y_host) out.y_host[nO + o] = yo;
        const float g = LOSS == CE ? expf(yo - m) * inv_sum : yo;  // softmax or y
        const float d = (g - tn[o * ts]) * inv_n;
        if (out.dy) out.dy[nO + o] = d;
        if (out.l_dy) out.l_dy[o * out.ls + n] = d;
        dh_accum<HB>(lw, s, o, d, dh);
    }
#pragma unroll
    for (int j = 0; j < HB; ++j) {
        if (j < s.H) {
            const float v = dh[j] * (hp[j] > 0.f ? 1.f : 0.f);
            if (out.dhp) out.dhp[nH + j] = v;
            if (out.l_dhp) out.l_dhp[j * out.ls + n] = v;
        }
    }
}

// Gradient of parameter p summed over samples [n0, n1) in ascending order
// (mlp2_dw_accum.comp, mlp2_db_accum.comp): dW1 = dh_pre^T x, db1 = sum dh_pre,
// dW2 = dy^T h, db2 = sum dy.  The arrays are sample-major, in LDS or HBM.
// Four interleaved partial sums (samples n = 0, 1, 2, 3 mod 4 from n0) for
// instruction-level parallelism, combined as (a0 + a1) + (a2 + a3): a fixed
// order, so results do not depend on scheduling; one sample gives exactly
// its own term.
template <class F>
VKH_DEV float sum4(int n0, int n1, F term) {
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
    int n = n0;
    for (; n + 3 < n1; n += 4) {
        a0 += term(n);
        a1 += term(n + 1);
        a2 += term(n + 2);
        a3 += term(n + 3);
    }
    for (; n < n1; ++n) a0 += term(n);
    return (a0 + a1) + (a2 + a3);
}

VKH_DEV float grad_sum(const Shape &s, int p, const float *x, const float *h, const float *dy,
                       const float *dhp, int n0, int n1) {
    if (p < s.b1) {
        const int j = p / s.I, i = p - j * s.I;
        return sum4(n0, n1, [&](int n) { return dhp[(size_t)n * s.H + j] * x[(size_t)n * s.I + i]; });
    }
    if (p < s.w2) {
        const int j = p - s.b1;
        return sum4(n0, n1, [&](int n) { return dhp[(size_t)n * s.H + j]; });
    }
    if (p < s.b2) {
        const int q = p - s.w2, o = q / s.H, j = q - o * s.H;
        return sum4(n0, n1, [&](int n) { return dy[(size_t)n * s.O + o] * h[(size_t)n * s.H + j]; });
    }
    const int o = p - s.b2;
    return sum4(n0, n1, [&](int n) { return dy[(size_t)n * s.O + o]; });
}

// Store the gradient and update parameter p: sgd_step.comp / adam_step.comp,
// decoupled weight decay on the W1 and W2 spans only (runner.zig:1178-1219).
template <int OPT>
VKH_DEV void update(float *P, float *G, float *M, float *V, const Shape &s, int p, float g,
                    const Opt &o) {
    const bool is_w = p < s.b1 || (p >= s.w2 && p < s.b2);
    const float wd = is_w ? o.wd : 0.f;
    G[p] = g;
    float v = P[p];
    if (wd > 0.f) v = v * (1.f - o.lr * wd);
    if (OPT == SGD) {
        P[p] = v - o.lr * g;
    } else {
        const float nm = o.beta1 * M[p] + (1.f - o.beta1) * g;
        const float nv = o.beta2 * V[p] + (1.f - o.beta2) * g * g;
        M[p] = nm;
        V[p] = nv;
        const float m_hat = nm / o.bc1, v_hat = nv / o.bc2;
        P[p] = v - o.lr * m_hat / (sqrtf(v_hat) + o.eps);
    }
}

// Fused-kernel LDS: staged weights, then feature-major sample arrays with
// row stride ls = N rounded up to 4, plus 4 (16-byte rows, and consecutive
// rows start in different banks): x [I], t [O], h [H], dy [O], dh_pre [H] and
// a row of ones (the "input" of the bias gradients).
__host__ __device__ inline int fused_ls(int N) { return ((N + 3) & ~3) + 4; }
static inline size_t fused_lds_floats(const Shape &s, int HB, int N) {
    return (size_t)woff(s, HB).end + (size_t)fused_ls(N) * (s.I + 2 * s.O + 2 * s.H + 1);
}

// ── kernels ───────────────────────────────────────────────────────────────

// One whole step in one workgroup.  Phase 1: stage weights, x and t in LDS,
// then one thread per sample (forward, loss gradient, backward).  Phase 2:
// one thread per parameter reduces over the batch from LDS, four samples per
// 16-byte read, and applies the update.  x and t may live in pinned host
// memory (read once, while staging).
template <int HB, int LOSS, int OPT>
__global__ __launch_bounds__(kBlock) void step_fused_k(float *P, float *G, float *M, float *V,
                                                       Shape s, const float *x, const float *t,
                                                       int N, float inv_n, SampleOut out, Opt o) {
    extern __shared__ __align__(16) float lds[];
    const WOff w = woff(s, HB);
    const int ls = fused_ls(N), N4 = (N + 3) & ~3;
    float *sx = lds + w.end, *st = sx + (size_t)ls * s.I, *sh = st + (size_t)ls * s.O;
    float *sdy = sh + (size_t)ls * s.H, *sdhp = sdy + (size_t)ls * s.O;
    float *ones = sdhp + (size_t)ls * s.H;
    // weights, x and t (transposed, zero-padded to ls) and the ones row are
    // contiguous in LDS: one staging pass
    const int ex = ls * s.I, et = ls * s.O, E = w.end + ex + et;
    stage(lds, E, threadIdx.x, kBlock, [&](int f) {
        if (f < w.end) return weight_at<HB>(P, s, w, f);
        f -= w.end;
        const float *src = x;
        int d = s.I;
        if (f >= ex) { f -= ex; src = t; d = s.O; }
        const int r = f / ls, n = f - r * ls;  // feature r of sample n
        return n < N ? src[(size_t)n * d + r] : 0.f;
    });
    for (int q = threadIdx.x; q < ls; q += kBlock) ones[q] = 1.f;
    __syncthreads();
    SampleOut so = out;
    so.l_h = sh; so.l_dy = sdy; so.l_dhp = sdhp; so.ls = ls;
    for (int n = threadIdx.x; n < N4; n += kBlock) {
        if (n < N) {
            train_sample<HB, LOSS>(lds, s, n, sx + n, ls, st + n, ls, inv_n, so);
        } else {  // the padding samples contribute exact zeros
            for (int j = 0; j < s.H; ++j) sh[j * ls + n] = sdhp[j * ls + n] = 0.f;
            for (int k = 0; k < s.O; ++k) sdy[k * ls + n] = 0.f;
        }
    }
    __syncthreads();
    // dW1|db1 = dh_pre^T [x | 1] (rows j, columns i <= I) and
    // dW2|db2 = dy^T [h | 1] (rows o, columns j <= H); the second group starts
    // on a wave boundary so no wave mixes the two
    const int nA = s.H * (s.I + 1), nA_pad = (nA + kWave - 1) & ~(kWave - 1);
    const int nB = s.O * (s.H + 1);
    for (int q = threadIdx.x; q < nA_pad + nB; q += kBlock) {
        const float *ar, *br;
        int pb;
        if (q < nA_pad) {
            if (q >= nA) continue;
            const int j = q / (s.I + 1), c = q - j * (s.I + 1);
            ar = sdhp + j * ls;
            br = c < s.I ? sx + c * ls : ones;
            pb = c < s.I ? s.w1 + j * s.I + c : s.b1 + j;
        } else {
            const int r = q - nA_pad, oo = r / (s.H + 1), c = r - oo * (s.H + 1);
            ar = sdy + oo * ls;
            br = c < s.H ? sh + c * ls : ones;
            pb = c < s.H ? s.w2 + oo * s.H + c : s.b2 + oo;
        }
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        for (int n = 0; n < N4; n += 4) {
            const f32x4 av = *(const f32x4 *)(ar + n), bv = *(const f32x4 *)(br + n);
            acc[0] += av[0] * bv[0];
            acc[1] += av[1] * bv[1];
            acc[2] += av[2] * bv[2];
            acc[3] += av[3] * bv[3];
        }
        update<OPT>(P, G, M, V, s, pb, (acc[0] + acc[1]) + (acc[2] + acc[3]), o);
    }
}

// The padded weight layout in HBM, for shapes whose weights exceed LDS.
template <int HB>
__global__ __launch_bounds__(kBlock) void pack_weights_k(const float *P, Shape s, float *gw) {
    stage_weights<HB>(P, s, gw, blockIdx.x * kBlock + threadIdx.x, gridDim.x * kBlock);
}

// Per-sample pass, kFwdBlock samples per block, weights staged in LDS (or,
// with GW, read from the packed copy in HBM).  PREDICT writes y (and
// y_host); TRAIN_* the full training pass.
template <int HB, int MODE, bool GW>
__global__ __launch_bounds__(kFwdBlock) void sample_k(const float *P, const float *gw, Shape s,
                                                      const float *x, const float *t, int N,
                                                      float inv_n, SampleOut out) {
    extern __shared__ __align__(16) float lds[];
    const float *lw = lds;
    if (GW) {
        lw = gw;
    } else {
        stage_weights<HB>(P, s, lds, threadIdx.x, kFwdBlock);
        __syncthreads();
    }
    const int n = blockIdx.x * kFwdBlock + threadIdx.x;
    if (n >= N) return;
    const float *xn = x + (size_t)n * s.I;
    if (MODE == PREDICT) {
        float hp[HB], hv[HB];
        layer1<HB>(lw, s, xn, 1, hp);
        relu<HB>(hp, hv);
        const size_t nO = (size_t)n * s.O;
        for (int o = 0; o < s.O; ++o) {
            const float yo = layer2_row<HB>(lw, s, o, hv);
            if (out.y) out.y[nO + o] = yo;
            if (out.y_host) out.y_host[nO + o] = yo;
        }
    } else {
        train_sample<HB, MODE == TRAIN_CE ? CE : MSE>(lw, s, n, xn, 1, t + (size_t)n * s.O, 1,
                                                       inv_n, out);
    }
}

// Reduction over all samples + update, one thread per parameter.
template <int OPT>
__global__ __launch_bounds__(kBlock) void reduce_update_k(float *P, float *G, float *M, float *V,
                                                          Shape s, const float *x, const float *h,
                                                          const float *dy, const float *dhp,
                                                          int N, Opt o) {
    const int p = blockIdx.x * kBlock + threadIdx.x;
    if (p >= s.n) return;
    update<OPT>(P, G, M, V, s, p, grad_sum(s, p, x, h, dy, dhp, 0, N), o);
}

// Partial sums over chunk blockIdx.y of kChunk samples.
__global__ __launch_bounds__(kBlock) void partial_k(float *part, Shape s, const float *x,
                                                    const float *h, const float *dy,
                                                    const float *dhp, int N) {
    const int p = blockIdx.x * kBlock + threadIdx.x;
    if (p >= s.n) return;
    const int n0 = blockIdx.y * kChunk, n1 = min(N, n0 + kChunk);
    part[(size_t)blockIdx.y * s.n + p] = grad_sum(s, p, x, h, dy, dhp, n0, n1);
}

// Chunk partials summed in chunk order + update.
template <int OPT>
__global__ __launch_bounds__(kBlock) void combine_update_k(float *P, float *G, float *M, float *V,
                                                           Shape s, const float *part,
                                                           int n_chunks, Opt o) {
    const int p = blockIdx.x * kBlock + threadIdx.x;
    if (p >= s.n) return;
    update<OPT>(P, G, M, V, s, p, sum4(0, n_chunks, [&](int c) { return part[(size_t)c * s.n + p]; }),
                o);
}

// Batch loss of the loss-target gate (mlp2_mse_loss_batched.comp,
// mlp2_ce_loss_batched.comp) from the current weights: per-thread partial
// over a strided subset of samples, then a fixed-order block tree.
template <int HB, int LOSS, bool GW>
__global__ __launch_bounds__(kBlock) void loss_k(const float *P, const float *gw, Shape s,
                                                 const float *x, const float *tgt, int N,
                                                 float *loss_out) {
    extern __shared__ __align__(16) float lds[];
    __shared__ float red[kBlock];
    const float *lw = lds;
    if (GW) {
        lw = gw;
    } else {
        stage_weights<HB>(P, s, lds, threadIdx.x, kBlock);
        __syncthreads();
    }
    float acc = 0.f;
    for (int n = threadIdx.x; n < N; n += kBlock) {
        float hp[HB], hv[HB];
        layer1<HB>(lw, s, x + (size_t)n * s.I, 1, hp);
        relu<HB>(hp, hv);
        const float *tn = tgt + (size_t)n * s.O;
        if (LOSS == MSE) {
            for (int o = 0; o < s.O; ++o) {
                const float d = layer2_row<HB>(lw, s, o, hv) - tn[o];
                acc += d * d;
            }
        } else {
            float m = -INFINITY;
            for (int o = 0; o < s.O; ++o) m = fmaxf(m, layer2_row<HB>(lw, s, o, hv));
            float sum_e = 0.f;
            for (int o = 0; o < s.O; ++o) sum_e += expf(layer2_row<HB>(lw, s, o, hv) - m);
            const float log_z = m + logf(sum_e);
            for (int o = 0; o < s.O; ++o) acc -= tn[o] * (layer2_row<HB>(lw, s, o, hv) - log_z);
        }
    }
    red[threadIdx.x] = acc;
    __syncthreads();
    for (int k = kBlock / 2; k > 0; k >>= 1) {
        if ((int)threadIdx.x < k) red[threadIdx.x] += red[threadIdx.x + k];
        __syncthreads();
    }
    if (threadIdx.x == 0)
        loss_out[0] = LOSS == MSE ? (red[0] * 0.5f) / (float)N : red[0] / (float)N;
}

// ── launch helpers (hidden width rounded up to a compile-time bucket) ───────

static inline int hb_of(int H) { return H <= 8 ? 8 : H <= 16 ? 16 : H <= 32 ? 32 : 64; }

template <template <int> class F, typename... A>
static void by_hb(int H, A... a) {
    switch (hb_of(H)) {
    case 8: F<8>::run(a...); break;
    case 16: F<16>::run(a...); break;
    case 32: F<32>::run(a...); break;
    default: F<64>::run(a...); break;
    }
}

template <int HB>
struct LaunchFused {
    static void run(hipStream_t st, int loss, int opt, float *P, float *G, float *M, float *V,
                    Shape s, const float *x, const float *t, int N, float inv_n, SampleOut out,
                    Opt o) {
        const size_t lds = fused_lds_floats(s, HB, N) * sizeof(float);
        dim3 g(1), b(kBlock);
        if (loss == MSE && opt == SGD)
            step_fused_k<HB, MSE, SGD><<<g, b, lds, st>>>(P, G, M, V, s, x, t, N, inv_n, out, o);
        else if (loss == MSE)
            step_fused_k<HB, MSE, ADAM><<<g, b, lds, st>>>(P, G, M, V, s, x, t, N, inv_n, out, o);
        else if (opt == SGD)
            step_fused_k<HB, CE, SGD><<<g, b, lds, st>>>(P, G, M, V, s, x, t, N, inv_n, out, o);
        else
            step_fused_k<HB, CE, ADAM><<<g, b, lds, st>>>(P, G, M, V, s, x, t, N, inv_n, out, o);
    }
};

template <int HB>
struct LaunchPack {
    static void run(hipStream_t st, const float *P, Shape s, float *gw) {
        const size_t n = (size_t)woff(s, HB).end;
        pack_weights_k<HB><<<(unsigned)std::min<size_t>((n + kBlock - 1) / kBlock, 1024), kBlock, 0,
                             st>>>(P, s, gw);
    }
};

// gw non-null: weights from the packed HBM copy (no LDS).
template <int HB>
struct LaunchSample {
    template <int MODE>
    static void go(hipStream_t st, const float *P, const float *gw, Shape s, const float *x,
                   const float *t, int N, float inv_n, SampleOut out) {
        const dim3 g((N + kFwdBlock - 1) / kFwdBlock), b(kFwdBlock);
        if (gw)
            sample_k<HB, MODE, true><<<g, b, 0, st>>>(P, gw, s, x, t, N, inv_n, out);
        else
            sample_k<HB, MODE, false><<<g, b, (size_t)woff(s, HB).end * sizeof(float), st>>>(
                P, gw, s, x, t, N, inv_n, out);
    }
    static void run(hipStream_t st, int mode, const float *P, const float *gw, Shape s,
                    const float *x, const float *t, int N, float inv_n, SampleOut out) {
        if (mode == PREDICT) go<PREDICT>(st, P, gw, s, x, t, N, inv_n, out);
        else if (mode == TRAIN_MSE) go<TRAIN_MSE>(st, P, gw, s, x, t, N, inv_n, out);
        else go<TRAIN_CE>(st, P, gw, s, x, t, N, inv_n, out);
    }
};

template <int HB>
struct LaunchLoss {
    template <int LOSS>
    static void go(hipStream_t st, const float *P, const float *gw, Shape s, const float *x,
                   const float *t, int N, float *out) {
        if (gw)
            loss_k<HB, LOSS, true><<<1, kBlock, 0, st>>>(P, gw, s, x, t, N, out);
        else
            loss_k<HB, LOSS, false><<<1, kBlock, (size_t)woff(s, HB).end * sizeof(float), st>>>(
                P, gw, s, x, t, N, out);
    }
    static void run(hipStream_t st, int loss, const float *P, const float *gw, Shape s,
                    const float *x, const float *t, int N, float *out) {
        if (loss == MSE) go<MSE>(st, P, gw, s, x, t, N, out);
        else go<CE>(st, P, gw, s, x, t, N, out);
    }
};

}  // namespace mlp
}  // namespace vkh

using namespace vkh;
using namespace vkh::mlp;

// ── the runner ────────────────────────────────────────────────────────────

struct vkh_mlp {
    vkh_mlp_config cfg;
    float lr = 0.f, wd = 0.f;
    Shape s;
    int device = 0;
    hipStream_t own = nullptr;
    hipEvent_t loss_ev = nullptr;
    char *arena = nullptr;  // device memory, every buffer below
    float *P = nullptr, *G = nullptr, *M = nullptr, *V = nullptr;
    // single-sample path (tickStep / tickPredict)
    float *hp1 = nullptr, *h1 = nullptr, *y1 = nullptr,
          *dy1 = nullptr, *dhp1 = nullptr;
    // batched surface (max_batch_size > 0)
    float *xb = nullptr, *yb = nullptr;                                 // predict
    float *xt = nullptr, *tt = nullptr, *hpt = nullptr, *ht = nullptr,  // train
          *yt = nullptr, *dyt = nullptr, *dhpt = nullptr;
    float *part = nullptr, *loss_d = nullptr;
    float *gw = nullptr;  // packed weights in HBM, only when they exceed LDS
    // pinned host memory, read / written by the kernels directly: one
    // sample's x, target and prediction; the loss and the predict staging
    float *pin = nullptr;
    float *x1_h = nullptr, *t1_h = nullptr, *y1_h = nullptr, *loss_h = nullptr,
          *ystage_h = nullptr;
    // one-sample record calls: each gets its own pinned (x, target) slot, so
    // every enqueued step reads the values passed to its own call; a slot is
    // reused only after the step that read it has run
    float *ring_h = nullptr;
    hipEvent_t ring_ev[kRing] = {};
    bool ring_used[kRing] = {};
    int ring_pos = 0;
    size_t ystage_n = 0;
    bool loss_pending = false, has_last = false;
    float last_loss = 0.f;
    uint32_t adam_step = 0;

    bool batched() const { return cfg.max_batch_size > 0; }

    vkh_status set_device() {
        VKH_HIP(hipSetDevice(device));
        return VKH_OK;
    }

    Opt opt_args(bool adam) {
        Opt o{lr, wd, cfg.adam_beta1, cfg.adam_beta2, cfg.adam_eps, 1.f, 1.f};
        if (adam) {
            // runner.zig:1188-1190: the step counter is bumped before the update
            adam_step += 1;
            const float tf = (float)adam_step;
            o.bc1 = 1.f - powf(cfg.adam_beta1, tf);
            o.bc2 = 1.f - powf(cfg.adam_beta2, tf);
        }
        return o;
    }

    bool weights_fit_lds() const { return (size_t)woff(s, hb_of(s.H)).end <= kLdsFloats; }

    // The packed weight copy the kernels read when the weights exceed LDS.
    const float *packed_weights(hipStream_t st) {
        if (!gw) return nullptr;
        by_hb<LaunchPack>(s.H, st, (const float *)P, s, gw);
        return gw;
    }

    SampleOut single_out(float *y_host) const {
        return SampleOut{hp1, h1, y1, dy1, dhp1, y_host, nullptr, nullptr, nullptr, 0};
    }
    SampleOut batch_out() const {
        return SampleOut{hpt, ht, yt, dyt, dhpt, nullptr, nullptr, nullptr, nullptr, 0};
    }

    // One training step over N samples at x / t (HBM or pinned host memory).
    vkh_status enqueue_step(hipStream_t st, const float *x, const float *t, int N, int loss,
                            int opt, const SampleOut &out) {
        const Opt o = opt_args(opt == ADAM);
        const float inv_n = 1.f / (float)N;
        const float *h = out.h, *dy = out.dy, *dhp = out.dhp;
        if (weights_fit_lds() && N <= kFusedMaxN && (size_t)N * s.n <= kFusedMaxWork &&
            fused_lds_floats(s, hb_of(s.H), N) <= kLdsFloats) {
            by_hb<LaunchFused>(s.H, st, loss, opt, P, G, M, V, s, x, t, N, inv_n, out, o);
        } else {
            by_hb<LaunchSample>(s.H, st, loss == CE ? (int)TRAIN_CE : (int)TRAIN_MSE,
                                (const float *)P, packed_weights(st), s, x, t, N, inv_n, out);
            const dim3 gp((s.n + kBlock - 1) / kBlock);
            if (N <= kChunk) {
                if (opt == SGD)
                    reduce_update_k<SGD><<<gp, kBlock, 0, st>>>(P, G, M, V, s, x, h, dy, dhp, N, o);
                else
                    reduce_update_k<ADAM><<<gp, kBlock, 0, st>>>(P, G, M, V, s, x, h, dy, dhp, N, o);
            } else {
                const int nc = (N + kChunk - 1) / kChunk;
                partial_k<<<dim3(gp.x, nc), kBlock, 0, st>>>(part, s, x, h, dy, dhp, N);
                if (opt == SGD)
                    combine_update_k<SGD><<<gp, kBlock, 0, st>>>(P, G, M, V, s, part, nc, o);
                else
                    combine_update_k<ADAM><<<gp, kBlock, 0, st>>>(P, G, M, V, s, part, nc, o);
            }
        }
        VKH_HIP(hipGetLastError());
        return VKH_OK;
    }

    vkh_status enqueue_predict(hipStream_t st, const float *x, int N, float *y, float *y_host) {
        const SampleOut out{nullptr, nullptr, y, nullptr, nullptr, y_host, nullptr, nullptr, nullptr, 0};
        by_hb<LaunchSample>(s.H, st, (int)PREDICT, (const float *)P, packed_weights(st), s, x,
                            (const float *)nullptr, N, 1.f, out);
        VKH_HIP(hipGetLastError());
        return VKH_OK;
    }

    // recordLossEval (runner.zig:1226-1292): loss of the current weights on the
    // staged batch, copied to pinned staging; an event marks its arrival.
    vkh_status enqueue_loss_eval(hipStream_t st, int N) {
        by_hb<LaunchLoss>(s.H, st, (int)cfg.loss, (const float *)P, packed_weights(st), s,
                          (const float *)xt, (const float *)tt, N, loss_d);
        VKH_HIP(hipGetLastError());
        VKH_HIP(hipMemcpyAsync(loss_h, loss_d, sizeof(float), hipMemcpyDeviceToHost, st));
        VKH_HIP(hipEventRecord(loss_ev, st));
        loss_pending = true;
        return VKH_OK;
    }

    vkh_status ring_take(int *slot) {
        const int k = ring_pos;
        ring_pos = (ring_pos + 1) % kRing;
        if (ring_used[k]) VKH_HIP(hipEventSynchronize(ring_ev[k]));
        ring_used[k] = false;
        *slot = k;
        return VKH_OK;
    }
    float *ring_x(int k) const { return ring_h + (size_t)k * (s.I + s.O); }
    float *ring_t(int k) const { return ring_x(k) + s.I; }
    vkh_status ring_done(int k, hipStream_t st) {
        VKH_HIP(hipEventRecord(ring_ev[k], st));
        ring_used[k] = true;
        return VKH_OK;
    }

    void release() {
        if (device >= 0) (void)hipSetDevice(device);
        for (auto &e : ring_ev)
            if (e) (void)hipEventDestroy(e), e = nullptr;
        if (loss_ev) (void)hipEventDestroy(loss_ev);
        if (own) (void)hipStreamDestroy(own);
        if (arena) (void)hipFree(arena);
        if (pin) (void)hipHostFree(pin);
        loss_ev = nullptr; own = nullptr; arena = nullptr; pin = nullptr;
    }
};

static inline hipStream_t stream_of(vkh_mlp *m, vkh_stream s) {
    return s ? (hipStream_t)s : m->own;
}

#define MLP_ARG(cond, msg)                                                \
    do {                                                                  \
        if (!(cond)) return fail(VKH_ERR_INVALID_ARGUMENT, "%s", msg);    \
    } while (0)

extern "C" {

void vkh_mlp_config_default(vkh_mlp_config *c, uint32_t dim_in, uint32_t dim_hidden,
                            uint32_t dim_out, float lr) {
    if (!c) return;
    memset(c, 0, sizeof(*c));
    c->dim_in = dim_in;
    c->dim_hidden = dim_hidden;
    c->dim_out = dim_out;
    c->lr = lr;
    c->init_scale = 0.3f;
    c->init_seed = 0xCAFEull;
    c->max_batch_size = 0;
    c->optimizer = VKH_MLP_SGD;
    c->adam_beta1 = 0.9f;
    c->adam_beta2 = 0.999f;
    c->adam_eps = 1e-8f;
    c->loss = VKH_MLP_MSE;
    c->decay = VKH_MLP_DECAY_NONE;
    c->decay_target = 0.f;
    c->weight_decay = 0.f;
}

// Mlp.init (cpu/train.zig:47-81) with Zig's DefaultPrng: xoshiro256++ seeded
// by four SplitMix64 outputs; rng.float(f32) takes the low 23 bits of a draw
// as the mantissa and its leading-zero count as the binary exponent.
static uint64_t mlp_splitmix(uint64_t &st) {
    uint64_t z = (st += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

struct ZigPrng {
    uint64_t s[4];
    explicit ZigPrng(uint64_t seed) {
        uint64_t st = seed;
        for (auto &w : s) w = mlp_splitmix(st);
    }
    static uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }
    uint64_t next() {
        const uint64_t r = rotl(s[0] + s[3], 23) + s[0];
        const uint64_t t = s[1] << 17;
        s[2] ^= s[0]; s[3] ^= s[1]; s[1] ^= s[2]; s[0] ^= s[3]; s[2] ^= t;
        s[3] = rotl(s[3], 45);
        return r;
    }
    float uniform01() {
        const uint64_t r = next();
        unsigned lz = r ? (unsigned)__builtin_clzll(r) : 64u;
        if (lz >= 41) {
            const uint64_t r2 = next();
            lz = 41 + (r2 ? (unsigned)__builtin_clzll(r2) : 64u);
            if (lz == 41 + 64) lz += (unsigned)__builtin_clz((uint32_t)next() | 0x7FFu);
        }
        const uint32_t bits = ((uint32_t)(126 - lz) << 23) | (uint32_t)(r & 0x7FFFFFu);
        float f;
        memcpy(&f, &bits, 4);
        return f;
    }
};

vkh_status vkh_mlp_create(const vkh_mlp_config *cfg, vkh_mlp **out) {
    MLP_ARG(cfg && out, "null argument");
    *out = nullptr;
    // runner.zig:329
    if (cfg->dim_hidden > VKH_MLP_MAX_HIDDEN)
        return fail(VKH_ERR_HIDDEN_DIM_EXCEEDS_MAX, "dim_hidden %u > %d", cfg->dim_hidden,
                    VKH_MLP_MAX_HIDDEN);
    MLP_ARG(cfg->dim_in && cfg->dim_hidden && cfg->dim_out, "zero dimension");
    MLP_ARG(cfg->dim_in <= (1u << 20) && cfg->dim_out <= (1u << 20), "dimension too large");
    MLP_ARG(cfg->optimizer <= VKH_MLP_ADAM && cfg->loss <= VKH_MLP_CROSS_ENTROPY &&
                cfg->decay <= VKH_MLP_DECAY_LOSS_TARGET,
            "unknown optimizer / loss / decay kind");
    MLP_ARG((uint64_t)cfg->max_batch_size * (cfg->dim_in + cfg->dim_out + 2 * VKH_MLP_MAX_HIDDEN) <
                (1ull << 31),
            "max_batch_size too large");
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev == 0)
        return fail(VKH_ERR_NO_DEVICE, "no HIP device visible");

    vkh_mlp *m = new vkh_mlp();
    m->cfg = *cfg;
    m->lr = cfg->lr;
    m->wd = cfg->weight_decay;
    m->s = make_shape((int)cfg->dim_in, (int)cfg->dim_hidden, (int)cfg->dim_out);
    auto bail = [&](vkh_status st) {
        m->release();
        delete m;
        return st;
    };
    if (hipGetDevice(&m->device) != hipSuccess) return bail(fail(VKH_ERR_HIP, "hipGetDevice"));
    const Shape &s = m->s;
    const size_t I = s.I, H = s.H, O = s.O, NB = cfg->max_batch_size;
    const bool adam = cfg->optimizer == VKH_MLP_ADAM;
    // device arena: every buffer 256-byte aligned
    size_t off = 0;
    struct Slot { float **p; size_t n; };
    const size_t n_chunks = NB > (size_t)kChunk ? (NB + kChunk - 1) / kChunk : 0;
    Slot slots[] = {
        {&m->P, (size_t)s.n}, {&m->G, (size_t)s.n},
        {&m->M, adam ? (size_t)s.n : 0}, {&m->V, adam ? (size_t)s.n : 0},
        {&m->hp1, H}, {&m->h1, H}, {&m->y1, O}, {&m->dy1, O},
        {&m->dhp1, H},
        {&m->xb, NB * I}, {&m->yb, NB * O},
        {&m->xt, NB * I}, {&m->tt, NB * O}, {&m->hpt, NB * H}, {&m->ht, NB * H},
        {&m->yt, NB * O}, {&m->dyt, NB * O}, {&m->dhpt, NB * H},
        {&m->part, n_chunks * (size_t)s.n}, {&m->loss_d, NB ? (size_t)1 : (size_t)0},
        {&m->gw, m->weights_fit_lds() ? (size_t)0 : (size_t)woff(s, hb_of(s.H)).end},
    };
    size_t offs[sizeof(slots) / sizeof(slots[0])];
    for (size_t k = 0; k < sizeof(slots) / sizeof(slots[0]); ++k) {
        offs[k] = off;
        off += (slots[k].n * sizeof(float) + 255) & ~(size_t)255;
    }
    note_allocation();
    hipError_t e = hipMalloc((void **)&m->arena, off ? off : 256);
    if (e != hipSuccess) return bail(hip_fail(e, "hipMalloc (mlp arena)"));
    for (size_t k = 0; k < sizeof(slots) / sizeof(slots[0]); ++k)
        *slots[k].p = slots[k].n ? (float *)(m->arena + offs[k]) : nullptr;
    e = hipMemset(m->arena, 0, off ? off : 256);  // Adam m / v zero-initialized
    if (e != hipSuccess) return bail(hip_fail(e, "hipMemset (mlp arena)"));
    // pinned staging: x, target, loss, predictions
    m->ystage_n = NB * O;
    const size_t pin_n = I + O + O + 1 + m->ystage_n + (size_t)kRing * (I + O);
    note_allocation();
    e = hipHostMalloc((void **)&m->pin, pin_n * sizeof(float), hipHostMallocDefault);
    if (e != hipSuccess) return bail(hip_fail(e, "hipHostMalloc (mlp staging)"));
    memset(m->pin, 0, pin_n * sizeof(float));
    m->x1_h = m->pin;
    m->t1_h = m->x1_h + I;
    m->y1_h = m->t1_h + O;
    m->loss_h = m->y1_h + O;
    m->ystage_h = m->loss_h + 1;
    m->ring_h = m->ystage_h + m->ystage_n;
    e = hipStreamCreateWithFlags(&m->own, hipStreamNonBlocking);
    if (e != hipSuccess) return bail(hip_fail(e, "hipStreamCreate"));
    e = hipEventCreateWithFlags(&m->loss_ev, hipEventDisableTiming);
    if (e != hipSuccess) return bail(hip_fail(e, "hipEventCreate"));
    for (auto &ev : m->ring_ev) {
        e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
        if (e != hipSuccess) return bail(hip_fail(e, "hipEventCreate"));
    }
    // initial weights on the host, then one upload
    std::vector<float> p0((size_t)s.n, 0.f);
    ZigPrng rng(cfg->init_seed);
    for (size_t k = 0; k < H * I; ++k) p0[s.w1 + k] = (rng.uniform01() * 2.0f - 1.0f) * cfg->init_scale;
    for (size_t k = 0; k < O * H; ++k) p0[s.w2 + k] = (rng.uniform01() * 2.0f - 1.0f) * cfg->init_scale;
    e = hipMemcpy(m->P, p0.data(), p0.size() * sizeof(float), hipMemcpyHostToDevice);
    if (e != hipSuccess) return bail(hip_fail(e, "hipMemcpy (initial weights)"));
    *out = m;
    return VKH_OK;
}

void vkh_mlp_destroy(vkh_mlp *m) {
    if (!m) return;
    if (m->device >= 0) (void)hipSetDevice(m->device);
    (void)hipDeviceSynchronize();
    m->release();
    delete m;
}

vkh_status vkh_mlp_get_config(const vkh_mlp *m, vkh_mlp_config *out) {
    MLP_ARG(m && out, "null argument");
    *out = m->cfg;
    return VKH_OK;
}

vkh_status vkh_mlp_set_lr(vkh_mlp *m, float lr) {
    MLP_ARG(m, "null runner");
    m->lr = lr;
    return VKH_OK;
}

float vkh_mlp_get_lr(const vkh_mlp *m) { return m ? m->lr : 0.f; }

vkh_status vkh_mlp_set_weight_decay(vkh_mlp *m, float wd) {
    MLP_ARG(m, "null runner");
    m->wd = wd;
    return VKH_OK;
}

uint32_t vkh_mlp_adam_step(const vkh_mlp *m) { return m ? m->adam_step : 0; }

// ── standalone (blocking) surface ─────────────────────────────────────────

// tickStep (runner.zig:598-620): forward, MSE gradient, backward and an SGD
// step on one sample (recordStep always uses the MSE head and SGD), then the
// pre-update prediction into out_pred when given.
vkh_status vkh_mlp_tick_step(vkh_mlp *m, const float *x, size_t x_len, const float *target,
                             size_t target_len, float *out_pred, size_t out_len) {
    MLP_ARG(m && x && target, "null argument");
    if (x_len != m->cfg.dim_in) return fail(VKH_ERR_X_DIM_MISMATCH, "x.len %zu != dim_in %u", x_len, m->cfg.dim_in);
    if (target_len != m->cfg.dim_out)
        return fail(VKH_ERR_TARGET_DIM_MISMATCH, "target.len %zu != dim_out %u", target_len, m->cfg.dim_out);
    if (out_pred && out_len != m->cfg.dim_out)
        return fail(VKH_ERR_OUT_DIM_MISMATCH, "out.len %zu != dim_out %u", out_len, m->cfg.dim_out);
    VKH_TRY(m->set_device());
    hipStream_t st = m->own;
    // the kernel reads x / target from pinned memory and writes the
    // prediction there: one launch and one synchronization per step
    memcpy(m->x1_h, x, x_len * sizeof(float));
    memcpy(m->t1_h, target, target_len * sizeof(float));
    VKH_TRY(m->enqueue_step(st, m->x1_h, m->t1_h, 1, MSE, SGD,
                            m->single_out(out_pred ? m->y1_h : nullptr)));
    VKH_HIP(hipStreamSynchronize(st));
    if (out_pred) memcpy(out_pred, m->y1_h, out_len * sizeof(float));
    return VKH_OK;
}

// tickPredict (runner.zig:626-637).
vkh_status vkh_mlp_tick_predict(vkh_mlp *m, const float *x, size_t x_len, float *out_pred,
                                size_t out_len) {
    MLP_ARG(m && x && out_pred, "null argument");
    if (x_len != m->cfg.dim_in) return fail(VKH_ERR_X_DIM_MISMATCH, "x.len %zu != dim_in %u", x_len, m->cfg.dim_in);
    if (out_len != m->cfg.dim_out)
        return fail(VKH_ERR_OUT_DIM_MISMATCH, "out.len %zu != dim_out %u", out_len, m->cfg.dim_out);
    VKH_TRY(m->set_device());
    hipStream_t st = m->own;
    memcpy(m->x1_h, x, x_len * sizeof(float));
    VKH_TRY(m->enqueue_predict(st, m->x1_h, 1, m->y1, m->y1_h));
    VKH_HIP(hipStreamSynchronize(st));
    memcpy(out_pred, m->y1_h, out_len * sizeof(float));
    return VKH_OK;
}

// Batch length checks shared by the batched calls (runner.zig:707-712,
// :735-740, :775-781): returns the sample count through n.
static vkh_status batch_n(vkh_mlp *m, size_t x_len, uint32_t *n) {
    if (!m->batched()) return fail(VKH_ERR_BATCH_SIZE_NOT_CONFIGURED, "max_batch_size is 0");
    if (x_len % m->cfg.dim_in != 0)
        return fail(VKH_ERR_X_BATCH_DIM_MISMATCH, "x_batch.len %zu not a multiple of dim_in %u", x_len, m->cfg.dim_in);
    const size_t nn = x_len / m->cfg.dim_in;
    if (nn > m->cfg.max_batch_size)
        return fail(VKH_ERR_BATCH_SIZE_EXCEEDS_MAX, "%zu samples > max_batch_size %u", nn, m->cfg.max_batch_size);
    *n = (uint32_t)nn;
    return VKH_OK;
}

// tickPredictBatch (runner.zig:705-733).
vkh_status vkh_mlp_tick_predict_batch(vkh_mlp *m, const float *x_batch, size_t x_len,
                                      float *out_y, size_t out_len) {
    MLP_ARG(m, "null runner");
    uint32_t n = 0;
    VKH_TRY(batch_n(m, x_len, &n));
    if (n == 0) return VKH_OK;
    MLP_ARG(x_batch && out_y, "null argument");
    if (out_len != (size_t)n * m->cfg.dim_out)
        return fail(VKH_ERR_OUT_BATCH_DIM_MISMATCH, "out_y.len %zu != %u * dim_out", out_len, n);
    VKH_TRY(m->set_device());
    hipStream_t st = m->own;
    VKH_HIP(hipMemcpyAsync(m->xb, x_batch, x_len * sizeof(float), hipMemcpyHostToDevice, st));
    VKH_TRY(m->enqueue_predict(st, m->xb, (int)n, m->yb, nullptr));
    VKH_HIP(hipMemcpyAsync(out_y, m->yb, out_len * sizeof(float), hipMemcpyDeviceToHost, st));
    VKH_HIP(hipStreamSynchronize(st));
    return VKH_OK;
}

static vkh_status stage_train_batch(vkh_mlp *m, const float *x_batch, size_t x_len,
                                    const float *t_batch, size_t t_len, uint32_t *n_out) {
    uint32_t n = 0;
    VKH_TRY(batch_n(m, x_len, &n));
    if (t_len != (size_t)n * m->cfg.dim_out)
        return fail(VKH_ERR_TARGET_BATCH_DIM_MISMATCH, "target_batch.len %zu != %u * dim_out", t_len, n);
    *n_out = n;
    if (n == 0) return VKH_OK;
    MLP_ARG(x_batch && t_batch, "null argument");
    VKH_TRY(m->set_device());
    hipStream_t st = m->own;
    VKH_HIP(hipMemcpyAsync(m->xt, x_batch, x_len * sizeof(float), hipMemcpyHostToDevice, st));
    VKH_HIP(hipMemcpyAsync(m->tt, t_batch, t_len * sizeof(float), hipMemcpyHostToDevice, st));
    VKH_HIP(hipStreamSynchronize(st));
    return VKH_OK;
}

// tickStepBatch (runner.zig:746-763): one mean-gradient step over the batch.
vkh_status vkh_mlp_tick_step_batch(vkh_mlp *m, const float *x_batch, size_t x_len,
                                   const float *target_batch, size_t target_len) {
    MLP_ARG(m, "null runner");
    if (!m->batched()) return fail(VKH_ERR_BATCH_SIZE_NOT_CONFIGURED, "max_batch_size is 0");
    if (x_len % m->cfg.dim_in != 0)
        return fail(VKH_ERR_X_BATCH_DIM_MISMATCH, "x_batch.len %zu not a multiple of dim_in %u", x_len, m->cfg.dim_in);
    if (x_len == 0) return VKH_OK;  // n == 0 returns before the target check (:750)
    uint32_t n = 0;
    VKH_TRY(stage_train_batch(m, x_batch, x_len, target_batch, target_len, &n));
    hipStream_t st = m->own;
    VKH_TRY(m->enqueue_step(st, m->xt, m->tt, (int)n, (int)m->cfg.loss, (int)m->cfg.optimizer,
                            m->batch_out()));
    VKH_HIP(hipStreamSynchronize(st));
    return VKH_OK;
}

// uploadTrainBatch (runner.zig:784-792): the batch later ticks train on.
// Blocking copy; call it when no enqueued step still reads the previous batch
// (after the host's frame fence, as the reference requires of its mapped
// buffers).
vkh_status vkh_mlp_upload_train_batch(vkh_mlp *m, const float *x_batch, size_t x_len,
                                      const float *target_batch, size_t target_len) {
    MLP_ARG(m, "null runner");
    uint32_t n = 0;
    return stage_train_batch(m, x_batch, x_len, target_batch, target_len, &n);
}

// uploadPredictInputs (runner.zig:797-803).
vkh_status vkh_mlp_upload_predict_inputs(vkh_mlp *m, const float *x_batch, size_t x_len) {
    MLP_ARG(m, "null runner");
    uint32_t n = 0;
    VKH_TRY(batch_n(m, x_len, &n));
    if (n == 0) return VKH_OK;
    MLP_ARG(x_batch, "null argument");
    VKH_TRY(m->set_device());
    VKH_HIP(hipMemcpyAsync(m->xb, x_batch, x_len * sizeof(float), hipMemcpyHostToDevice, m->own));
    VKH_HIP(hipStreamSynchronize(m->own));
    return VKH_OK;
}

// ── attach mode: enqueue on the caller's stream, never wait ───────────────

// tickStepRecord (runner.zig:655-665): x / target go to a pinned slot that
// the enqueued step reads when the stream reaches it.  The reference writes
// one host-visible buffer, so two records before a submit both see the last
// values; here each record keeps its own.
vkh_status vkh_mlp_tick_step_record(vkh_mlp *m, vkh_stream stream, const float *x, size_t x_len,
                                    const float *target, size_t target_len) {
    MLP_ARG(m && x && target, "null argument");
    if (x_len != m->cfg.dim_in) return fail(VKH_ERR_X_DIM_MISMATCH, "x.len %zu != dim_in %u", x_len, m->cfg.dim_in);
    if (target_len != m->cfg.dim_out)
        return fail(VKH_ERR_TARGET_DIM_MISMATCH, "target.len %zu != dim_out %u", target_len, m->cfg.dim_out);
    VKH_TRY(m->set_device());
    hipStream_t st = stream_of(m, stream);
    int k = 0;
    VKH_TRY(m->ring_take(&k));
    memcpy(m->ring_x(k), x, x_len * sizeof(float));
    memcpy(m->ring_t(k), target, target_len * sizeof(float));
    VKH_TRY(m->enqueue_step(st, m->ring_x(k), m->ring_t(k), 1, MSE, SGD, m->single_out(nullptr)));
    return m->ring_done(k, st);
}

// tickPredictRecord (runner.zig:670-678): the prediction stays on the GPU
// (vkh_mlp_buffer VKH_MLP_BUF_Y).
vkh_status vkh_mlp_tick_predict_record(vkh_mlp *m, vkh_stream stream, const float *x, size_t x_len) {
    MLP_ARG(m && x, "null argument");
    if (x_len != m->cfg.dim_in) return fail(VKH_ERR_X_DIM_MISMATCH, "x.len %zu != dim_in %u", x_len, m->cfg.dim_in);
    VKH_TRY(m->set_device());
    hipStream_t st = stream_of(m, stream);
    int k = 0;
    VKH_TRY(m->ring_take(&k));
    memcpy(m->ring_x(k), x, x_len * sizeof(float));
    VKH_TRY(m->enqueue_predict(st, m->ring_x(k), 1, m->y1, nullptr));
    return m->ring_done(k, st);
}

// tickStepBatchRecord (runner.zig:768-773).
vkh_status vkh_mlp_tick_step_batch_record(vkh_mlp *m, vkh_stream stream, uint32_t n_samples) {
    MLP_ARG(m, "null runner");
    if (!m->batched()) return fail(VKH_ERR_BATCH_SIZE_NOT_CONFIGURED, "max_batch_size is 0");
    if (n_samples == 0) return VKH_OK;
    if (n_samples > m->cfg.max_batch_size)
        return fail(VKH_ERR_BATCH_SIZE_EXCEEDS_MAX, "%u samples > max_batch_size %u", n_samples, m->cfg.max_batch_size);
    VKH_TRY(m->set_device());
    return m->enqueue_step(stream_of(m, stream), m->xt, m->tt, (int)n_samples, (int)m->cfg.loss,
                           (int)m->cfg.optimizer, m->batch_out());
}

// tickPredictBatchRecord (runner.zig:1001-1021).
vkh_status vkh_mlp_tick_predict_batch_record(vkh_mlp *m, vkh_stream stream, uint32_t n_samples) {
    MLP_ARG(m, "null runner");
    if (!m->batched()) return fail(VKH_ERR_BATCH_SIZE_NOT_CONFIGURED, "max_batch_size is 0");
    if (n_samples == 0) return VKH_OK;
    if (n_samples > m->cfg.max_batch_size)
        return fail(VKH_ERR_BATCH_SIZE_EXCEEDS_MAX, "%u samples > max_batch_size %u", n_samples, m->cfg.max_batch_size);
    VKH_TRY(m->set_device());
    return m->enqueue_predict(stream_of(m, stream), m->xb, (int)n_samples, m->yb, nullptr);
}

// recordPredictReadback (runner.zig:815-851): y_batch -> pinned staging.
vkh_status vkh_mlp_record_predict_readback(vkh_mlp *m, vkh_stream stream, uint32_t n_samples) {
    MLP_ARG(m, "null runner");
    if (!m->batched()) return fail(VKH_ERR_BATCH_SIZE_NOT_CONFIGURED, "max_batch_size is 0");
    if (n_samples == 0) return VKH_OK;
    if (n_samples > m->cfg.max_batch_size)
        return fail(VKH_ERR_BATCH_SIZE_EXCEEDS_MAX, "%u samples > max_batch_size %u", n_samples, m->cfg.max_batch_size);
    VKH_TRY(m->set_device());
    VKH_HIP(hipMemcpyAsync(m->ystage_h, m->yb, (size_t)n_samples * m->cfg.dim_out * sizeof(float),
                           hipMemcpyDeviceToHost, stream_of(m, stream)));
    return VKH_OK;
}

// readPredictStaging (runner.zig:857-863): valid once the stream that ran the
// readback has been synchronized.
vkh_status vkh_mlp_read_predict_staging(vkh_mlp *m, float *out_y, size_t out_len) {
    MLP_ARG(m, "null runner");
    if (!m->batched()) return fail(VKH_ERR_BATCH_SIZE_NOT_CONFIGURED, "max_batch_size is 0");
    if (out_len > m->ystage_n)
        return fail(VKH_ERR_OUTPUT_TOO_LARGE, "out_y.len %zu > staging %zu", out_len, m->ystage_n);
    MLP_ARG(out_y || out_len == 0, "null argument");
    memcpy(out_y, m->ystage_h, out_len * sizeof(float));
    return VKH_OK;
}

// tickFrameTrain (runner.zig:904-986): up to the budget of batched steps on
// the staged batch, enqueued on the caller's stream; with the loss-target
// policy, last tick's loss gates training and a fresh loss evaluation is
// enqueued every tick.
vkh_status vkh_mlp_tick_frame_train(vkh_mlp *m, vkh_stream stream, vkh_train_budget budget,
                                    uint32_t n_samples, vkh_tick_result *out) {
    MLP_ARG(m && out, "null argument");
    memset(out, 0, sizeof(*out));
    if (!m->batched()) return fail(VKH_ERR_BATCH_SIZE_NOT_CONFIGURED, "max_batch_size is 0");
    auto report_last = [&]() {
        out->has_loss = m->has_last ? 1u : 0u;
        out->last_loss = m->has_last ? m->last_loss : 0.f;
    };
    if (n_samples == 0) {
        report_last();
        out->idle = 1;
        return VKH_OK;
    }
    if (n_samples > m->cfg.max_batch_size)
        return fail(VKH_ERR_BATCH_SIZE_EXCEEDS_MAX, "%u samples > max_batch_size %u", n_samples, m->cfg.max_batch_size);
    const uint32_t max_steps = budget.mode == VKH_BUDGET_MICROSECONDS ? UINT32_MAX : budget.steps;
    const uint64_t us_cap = budget.mode == VKH_BUDGET_STEPS ? UINT64_MAX : budget.microseconds;
    if (max_steps == 0 || us_cap == 0) {
        report_last();
        out->idle = 1;
        return VKH_OK;
    }
    MLP_ARG(budget.mode <= VKH_BUDGET_EITHER, "unknown budget mode");
    VKH_TRY(m->set_device());
    const bool decay = m->cfg.decay != VKH_MLP_DECAY_NONE;
    // last tick's loss, once its copy has landed (runner.zig:932-945: a zero
    // in the staging before any measurement does not count)
    if (decay && m->loss_pending && hipEventQuery(m->loss_ev) == hipSuccess) {
        const float v = m->loss_h[0];
        if (m->has_last || v != 0.f) {
            m->last_loss = v;
            m->has_last = true;
        }
    }
    const bool should_train = !decay || !m->has_last || m->last_loss > m->cfg.decay_target;
    hipStream_t st = stream_of(m, stream);
    const auto t0 = std::chrono::steady_clock::now();
    uint32_t done = 0;
    if (should_train) {
        while (done < max_steps) {
            VKH_TRY(m->enqueue_step(st, m->xt, m->tt, (int)n_samples, (int)m->cfg.loss,
                                    (int)m->cfg.optimizer, m->batch_out()));
            ++done;
            const uint64_t us = (uint64_t)std::chrono::duration_cast<std::chrono::microseconds>(
                                    std::chrono::steady_clock::now() - t0).count();
            if (us >= us_cap) break;
        }
    }
    if (decay) VKH_TRY(m->enqueue_loss_eval(st, (int)n_samples));
    out->steps_completed = done;
    out->elapsed_us = (uint64_t)std::chrono::duration_cast<std::chrono::microseconds>(
                          std::chrono::steady_clock::now() - t0).count();
    report_last();
    out->idle = should_train ? 0u : 1u;
    return VKH_OK;
}

// getLastLoss (runner.zig:991-993).
vkh_status vkh_mlp_get_last_loss(const vkh_mlp *m, float *loss, uint32_t *has_loss) {
    MLP_ARG(m && loss && has_loss, "null argument");
    *has_loss = m->has_last ? 1u : 0u;
    *loss = m->has_last ? m->last_loss : 0.f;
    return VKH_OK;
}

// ── buffers ───────────────────────────────────────────────────────────────

vkh_status vkh_mlp_buffer(vkh_mlp *m, uint32_t which, float **dptr, size_t *numel) {
    MLP_ARG(m && dptr && numel, "null argument");
    const Shape &s = m->s;
    const size_t NB = m->cfg.max_batch_size;
    float *p = nullptr;
    size_t n = 0;
    switch (which) {
    case VKH_MLP_BUF_PARAMS: p = m->P; n = s.n; break;
    case VKH_MLP_BUF_GRADS: p = m->G; n = s.n; break;
    case VKH_MLP_BUF_ADAM_M: p = m->M; n = m->M ? s.n : 0; break;
    case VKH_MLP_BUF_ADAM_V: p = m->V; n = m->V ? s.n : 0; break;
    case VKH_MLP_BUF_Y: p = m->y1; n = s.O; break;
    case VKH_MLP_BUF_X_BATCH: p = m->xb; n = NB * s.I; break;
    case VKH_MLP_BUF_Y_BATCH: p = m->yb; n = NB * s.O; break;
    case VKH_MLP_BUF_X_TRAIN: p = m->xt; n = NB * s.I; break;
    case VKH_MLP_BUF_TARGET: p = m->tt; n = NB * s.O; break;
    case VKH_MLP_BUF_H_PRE_TRAIN: p = m->hpt; n = NB * s.H; break;
    case VKH_MLP_BUF_H_TRAIN: p = m->ht; n = NB * s.H; break;
    case VKH_MLP_BUF_Y_TRAIN: p = m->yt; n = NB * s.O; break;
    case VKH_MLP_BUF_DY_TRAIN: p = m->dyt; n = NB * s.O; break;
    case VKH_MLP_BUF_DH_PRE_TRAIN: p = m->dhpt; n = NB * s.H; break;
    default: return fail(VKH_ERR_INVALID_ARGUMENT, "unknown buffer id %u", which);
    }
    *dptr = n ? p : nullptr;
    *numel = n;
    return VKH_OK;
}

// Blocking copy of the first `numel` floats of a buffer, after all queued
// work on the device has finished.
vkh_status vkh_mlp_read_buffer(vkh_mlp *m, uint32_t which, float *host, size_t numel) {
    float *p = nullptr;
    size_t n = 0;
    VKH_TRY(vkh_mlp_buffer(m, which, &p, &n));
    if (numel > n) return fail(VKH_ERR_INVALID_ARGUMENT, "buffer %u holds %zu floats, %zu asked", which, n, numel);
    if (numel == 0) return VKH_OK;
    MLP_ARG(host, "null argument");
    VKH_TRY(m->set_device());
    VKH_HIP(hipDeviceSynchronize());
    VKH_HIP(hipMemcpy(host, p, numel * sizeof(float), hipMemcpyDeviceToHost));
    return VKH_OK;
}

// readWeights (runner.zig:684-689) into caller arrays of exactly the
// parameter shapes.
vkh_status vkh_mlp_read_weights(vkh_mlp *m, float *w1, size_t w1_len, float *b1, size_t b1_len,
                                float *w2, size_t w2_len, float *b2, size_t b2_len) {
    MLP_ARG(m && w1 && b1 && w2 && b2, "null argument");
    const Shape &s = m->s;
    MLP_ARG(w1_len == (size_t)s.H * s.I && b1_len == (size_t)s.H && w2_len == (size_t)s.O * s.H &&
                b2_len == (size_t)s.O,
            "destination shapes differ from the runner's");
    VKH_TRY(m->set_device());
    VKH_HIP(hipDeviceSynchronize());
    VKH_HIP(hipMemcpy(w1, m->P + s.w1, w1_len * sizeof(float), hipMemcpyDeviceToHost));
    VKH_HIP(hipMemcpy(b1, m->P + s.b1, b1_len * sizeof(float), hipMemcpyDeviceToHost));
    VKH_HIP(hipMemcpy(w2, m->P + s.w2, w2_len * sizeof(float), hipMemcpyDeviceToHost));
    VKH_HIP(hipMemcpy(b2, m->P + s.b2, b2_len * sizeof(float), hipMemcpyDeviceToHost));
    return VKH_OK;
}

}  // extern "C"
