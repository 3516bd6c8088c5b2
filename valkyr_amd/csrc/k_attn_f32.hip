// fp32 attention on the matrix cores (v_mfma_f32_16x16x4_f32): the training
// step's reference-precision path (fa_forward.comp, fa_bw_dq.comp,
// fa_bw_dkv.comp computed in fp32, as the reference does throughout).
//
// Tiles of 32 keys (forward, dQ) or 32 queries (dK/dV) are staged in LDS,
// double-buffered, with a padded row pitch of HD + 4 floats so the fragment
// reads below are free of bank conflicts; each block is 4 waves of 16 query
// or key rows whose own operands stay in registers.
//
// Fragment layout of v_mfma_f32_16x16x4_f32: lane (g, c) = (lane / 16,
// lane % 16) supplies A[c][k] and B[k][c] for contraction index k = g, and
// holds C[4 g + r][c] for r = 0..3.  Over a contraction of length 4 n the
// lane's k at step (u, e) stands for index 16 u + 4 g + e (one 16-byte read
// covers four steps), and an accumulator tile feeds the next product as its
// B operand directly: at step e the lane passes its own element e, i.e.
// contraction index 4 g + e, and the A operand is read at that index.
// The score tile is therefore oriented per kernel so that P and dS are
// always B operands (no register transposes):
//   forward   S^T = K Q^T, O^T += V^T P^T             (queries on lanes c)
//   dK / dV   S = Q K^T, dP = dO V^T;  dV^T += dO^T P, dK^T += Q^T dS
//   dQ        S^T = K Q^T, dP^T = V dO^T;  dQ^T += K^T dS^T
// Softmax in log2 units: Q (forward, dQ) or K (dK/dV) is pre-scaled by
// log2(e) / sqrt(hd), lse read in natural units and converted.
#include <math.h>

#include "ops.hpp"
#include "qkbwd.hpp"

#pragma clang fp contract(off)

namespace vkh {
namespace {

constexpr float F_LOG2E = 1.4426950408889634f;
constexpr float F_LN2 = 0.6931471805599453f;
constexpr int FNT = 256;  // 4 waves
constexpr int FT = 32;    // rows per staged tile

VKH_DEV float4 f4(const float *p) { return *reinterpret_cast<const float4 *>(p); }
VKH_DEV float4 f4_scale(float4 a, float s) { return make_float4(a.x * s, a.y * s, a.z * s, a.w * s); }
VKH_DEV f32x4 mfma4(const float4 &a, const float4 &b, f32x4 c) {
    c = mfma16x16x4(a.x, b.x, c);
    c = mfma16x16x4(a.y, b.y, c);
    c = mfma16x16x4(a.z, b.z, c);
    return mfma16x16x4(a.w, b.w, c);
}
VKH_DEV float xmax(float v) {
    v = fmaxf(v, __shfl_xor(v, 16));
    return fmaxf(v, __shfl_xor(v, 32));
}
VKH_DEV float xsum(float v) {
    v += __shfl_xor(v, 16);
    return v + __shfl_xor(v, 32);
}

// A FT x HD fp32 tile moved global -> registers -> LDS (pitch HD + 4) by NT threads.
template <int HD, int NT = FNT>
struct Tile {
    static constexpr int P = HD + 4, N4 = FT * HD / 4 / NT;
    static_assert(N4 * NT * 4 == FT * HD, "tile / thread count");
    float4 v[N4];
    VKH_DEV void load(const float *base, long ld, int tid) {
#pragma unroll
        for (int i = 0; i < N4; ++i) {
            const int x = tid + NT * i, r = x / (HD / 4), c = x % (HD / 4);
            v[i] = f4(base + (long)r * ld + 4 * c);
        }
    }
    VKH_DEV void store(float *lds, int tid) const {
#pragma unroll
        for (int i = 0; i < N4; ++i) {
            const int x = tid + NT * i, r = x / (HD / 4), c = x % (HD / 4);
            *reinterpret_cast<float4 *>(lds + r * P + 4 * c) = v[i];
        }
    }
};

// ── forward: block = 64 queries of one (sequence, head) ─────────────────
template <int HD>
__global__ __launch_bounds__(FNT, 2) void fa_fwd_f32m_k(AttnShape s, const float *q, long ldq,
                                                       const float *k, long ldk, const float *v,
                                                       long ldv, float *o, long ldo, float *lse,
                                                       bool zz) {
    constexpr int P = HD + 4, NU = HD / 16;
    __shared__ __attribute__((aligned(16))) float Ks[2][FT * P], Vs[2][FT * P];
    const int h = blockIdx.x % s.n_heads, b = blockIdx.x / s.n_heads;
    const int nqb = s.n_q / 64;
    const int y = (int)blockIdx.y, qb = s.causal ? nqb - 1 - (zz ? zigzag(y, nqb) : y) : y;
    const int tid = threadIdx.x, lane = tid % 64, g = lane / 16, c = lane % 16;
    const int wave = __builtin_amdgcn_readfirstlane(tid / 64);
    const int q0 = qb * 64, qw = q0 + 16 * wave, qi = qw + c;
    const int kvh = h / (s.n_heads / s.n_kv_heads);
    const float c2 = s.inv_sqrt_dim * F_LOG2E;
    float4 qf[NU];  // B of S^T = K Q^T: Q[qi][16 u + 4 g + e], pre-scaled
    {
        const float *qr = q + ((long)b * s.n_q + qi) * ldq + h * HD + 4 * g;
#pragma unroll
        for (int u = 0; u < NU; ++u) qf[u] = f4_scale(f4(qr + 16 * u), c2);
    }
    const int nkt = s.causal ? (q0 + 64) / FT : s.n_kv / FT;
    const float *kb = k + (long)b * s.n_kv * ldk + kvh * HD;
    const float *vb = v + (long)b * s.n_kv * ldv + kvh * HD;
    Tile<HD> tk, tv;
    tk.load(kb, ldk, tid);
    tv.load(vb, ldv, tid);
    tk.store(Ks[0], tid);
    tv.store(Vs[0], tid);
    __syncthreads();
    f32x4 ot[NU];  // O^T[16 j + 4 g + r][qi]
#pragma unroll
    for (int j = 0; j < NU; ++j) ot[j] = f32x4{0, 0, 0, 0};
    float m = -INFINITY, l = 0.f;  // running max (log2 units) and this lane's share of the sum
    for (int it = 0; it < nkt; ++it) {
        const int buf = it & 1;
        if (it + 1 < nkt) {
            tk.load(kb + (long)(it + 1) * FT * ldk, ldk, tid);
            tv.load(vb + (long)(it + 1) * FT * ldv, ldv, tid);
        }
        const float *Kl = Ks[buf], *Vl = Vs[buf];
        const int kt0 = it * FT;
        f32x4 st[2];  // S^T[kt0 + 16 ks + 4 g + r][qi]
        bool live[2];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            st[ks] = f32x4{0, 0, 0, 0};
            live[ks] = !s.causal || kt0 + 16 * ks <= qw + 15;  // wave-uniform
            if (live[ks]) {
                const float *kr = Kl + (16 * ks + c) * P + 4 * g;
#pragma unroll
                for (int u = 0; u < NU; ++u) st[ks] = mfma4(f4(kr + 16 * u), qf[u], st[ks]);
            }
        }
        float tmax = -INFINITY;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if (s.causal && kt0 + 16 * ks + 4 * g + r > qi) st[ks][r] = -INFINITY;
                tmax = fmaxf(tmax, st[ks][r]);
            }
        const float mn = fmaxf(m, xmax(tmax));  // finite: tile 0 holds key 0 <= qi
        const float alpha = __builtin_amdgcn_exp2f(m - mn);
        l *= alpha;
#pragma unroll
        for (int j = 0; j < NU; ++j) ot[j] *= alpha;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float pv = __builtin_amdgcn_exp2f(st[ks][r] - mn);
                st[ks][r] = pv;
                l += pv;
            }
        m = mn;
        // O^T += V^T P^T: step (ks, e) is key kt0 + 16 ks + 4 g + e
#pragma unroll
        for (int j = 0; j < NU; ++j)
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                if (!live[ks]) continue;
                const float *vr = Vl + (16 * ks + 4 * g) * P + 16 * j + c;
#pragma unroll
                for (int e = 0; e < 4; ++e) ot[j] = mfma16x16x4(vr[e * P], st[ks][e], ot[j]);
            }
        // buffer buf ^ 1 was last read before the previous barrier
        if (it + 1 < nkt) {
            tk.store(Ks[buf ^ 1], tid);
            tv.store(Vs[buf ^ 1], tid);
        }
        __syncthreads();
    }
    l = xsum(l);
    const float inv = 1.0f / l;
    float *orow = o + ((long)b * s.n_q + qi) * ldo + h * HD + 4 * g;
#pragma unroll
    for (int j = 0; j < NU; ++j)
        *reinterpret_cast<float4 *>(orow + 16 * j) =
            make_float4(ot[j][0] * inv, ot[j][1] * inv, ot[j][2] * inv, ot[j][3] * inv);
    if (lse && g == 0) lse[((long)b * s.n_q + qi) * s.n_heads + h] = (m + log2f(l)) * F_LN2;
}

// ── dK / dV: block = 64 keys of one (sequence, KV head) ─────────────────
// (32-key blocks on 2 waves, twice the grid in zigzag order, measured 185.5
// against 173.1 us at config 3: each staged query tile then feeds half the
// keys.  Where the 64-key grid is one block per CU, the causal 8:1 spread of
// block work stays.  Two groups of 4 waves per 64-key block, each taking
// every other (head, query tile) step from its own staged tiles and adding
// its sums to the other group's through LDS at the end: 159.5 against 178 us
// alone, but the fp32 step 78.2 against 77.0 ms, since the 136 KB block and
// its 8 waves of 242 VGPRs leave no room on the CU for the second stream's
// GEMM blocks.  Splitting the heavier half of the key blocks in two, each
// half of the steps summed raw and the halves added by a combine kernel in a
// fixed order: dK/dV 305 -> 205 us in the step plus a 20.5 us combine, but dQ
// then meets more of the second stream's work (98 -> 153 us) and the step
// went 77.0 -> 77.2 ms: with both streams busy the step is set by their
// total work, not by this kernel's span.)
// QKE: dK leaves through RoPE^T and the K-RMSNorm backward (p.qk), each block
// writing its k-gain partial to p.qk.pk[block].
template <int HD, bool QKE>
__global__ __launch_bounds__(FNT, 2) void fa_bwd_dkv_f32m_k(AttnShape s, AttnPtrs p, bool zz) {
    static_assert(!QKE || HD == 128, "the fused q/k epilogue takes 128-wide head rows");
    constexpr int P = HD + 4, NU = HD / 16;
    __shared__ __attribute__((aligned(16))) float Qs[2][FT * P], Os[2][FT * P];
    __shared__ float Ls[2][FT], Dl[2][FT];
    const int kvh = blockIdx.x % s.n_kv_heads, b = blockIdx.x / s.n_kv_heads;
    const int tid = threadIdx.x, lane = tid % 64, g = lane / 16, c = lane % 16;
    const int wave = __builtin_amdgcn_readfirstlane(tid / 64);
    const int kb = s.causal && zz ? zigzag((int)blockIdx.y, s.n_kv / 64) : (int)blockIdx.y;
    const int k0 = kb * 64, kw = k0 + 16 * wave, ki = kw + c;
    const int hpk = s.n_heads / s.n_kv_heads;
    const float c2 = s.inv_sqrt_dim * F_LOG2E;
    const float *Q = (const float *)p.q, *K = (const float *)p.k, *V = (const float *)p.v,
                *dO = (const float *)p.dout;
    float4 kf[NU], vf[NU];  // B of S = Q K^T and dP = dO V^T: K / V[ki][16 u + 4 g + e]
    {
        const float *kr = K + ((long)b * s.n_kv + ki) * p.ldk + kvh * HD + 4 * g;
        const float *vr = V + ((long)b * s.n_kv + ki) * p.ldv + kvh * HD + 4 * g;
#pragma unroll
        for (int u = 0; u < NU; ++u) {
            kf[u] = f4_scale(f4(kr + 16 * u), c2);
            vf[u] = f4(vr + 16 * u);
        }
    }
    const int qstart = s.causal ? k0 : 0;  // causal needs n_q == n_kv
    const int nqt = (s.n_q - qstart) / FT;
    const int niter = hpk * nqt;
    auto tile_of = [&](int it, int &h, int &q0) {
        h = kvh * hpk + it / nqt;
        q0 = qstart + (it % nqt) * FT;
    };
    Tile<HD> tq, tdo;
    float stat = 0.f;  // lse (threads 0..31) or D (32..63) of one tile row
    auto load = [&](int it) {
        int h, q0;
        tile_of(it, h, q0);
        const long row0 = (long)b * s.n_q + q0;
        tq.load(Q + row0 * p.ldq + h * HD, p.ldq, tid);
        tdo.load(dO + row0 * p.lddo + h * HD, p.lddo, tid);
        if (tid < 2 * FT) stat = (tid < FT ? p.lse : p.d)[(row0 + tid % FT) * s.n_heads + h];
    };
    auto store = [&](int buf) {
        tq.store(Qs[buf], tid);
        tdo.store(Os[buf], tid);
        if (tid < FT) Ls[buf][tid] = stat * F_LOG2E;
        else if (tid < 2 * FT) Dl[buf][tid - FT] = stat;
    };
    f32x4 dvt[NU], dkt[NU];  // dV^T / dK^T[16 j + 4 g + r][ki]
#pragma unroll
    for (int j = 0; j < NU; ++j) dvt[j] = dkt[j] = f32x4{0, 0, 0, 0};
    if (niter > 0) {
        load(0);
        store(0);
    }
    __syncthreads();
    for (int it = 0; it < niter; ++it) {
        const int buf = it & 1;
        if (it + 1 < niter) load(it + 1);
        int h, q0;
        tile_of(it, h, q0);
        (void)h;
        const float *Ql = Qs[buf], *Ol = Os[buf];
        f32x4 sa[2], da[2];  // S / dP[q0 + 16 qs + 4 g + r][ki]
        bool live[2];
#pragma unroll
        for (int qs = 0; qs < 2; ++qs) {
            sa[qs] = da[qs] = f32x4{0, 0, 0, 0};
            live[qs] = !s.causal || kw <= q0 + 16 * qs + 15;  // wave-uniform
            if (live[qs]) {
                const float *qr = Ql + (16 * qs + c) * P + 4 * g;
                const float *orr = Ol + (16 * qs + c) * P + 4 * g;
#pragma unroll
                for (int u = 0; u < NU; ++u) {
                    sa[qs] = mfma4(f4(qr + 16 * u), kf[u], sa[qs]);
                    da[qs] = mfma4(f4(orr + 16 * u), vf[u], da[qs]);
                }
            }
        }
        // P = exp2(S c - lse), dS = P (dP - D); zero above the diagonal
#pragma unroll
        for (int qs = 0; qs < 2; ++qs)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int qr = 16 * qs + 4 * g + r;
                float pv = __builtin_amdgcn_exp2f(sa[qs][r] - Ls[buf][qr]);
                if (s.causal && ki > q0 + qr) pv = 0.f;
                sa[qs][r] = pv;
                da[qs][r] = pv * (da[qs][r] - Dl[buf][qr]);
            }
        // dV^T += dO^T P, dK^T += Q^T dS: step (qs, e) is query q0 + 16 qs + 4 g + e
#pragma unroll
        for (int j = 0; j < NU; ++j)
#pragma unroll
            for (int qs = 0; qs < 2; ++qs) {
                if (!live[qs]) continue;
                const float *orr = Ol + (16 * qs + 4 * g) * P + 16 * j + c;
                const float *qr = Ql + (16 * qs + 4 * g) * P + 16 * j + c;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    dvt[j] = mfma16x16x4(orr[e * P], sa[qs][e], dvt[j]);
                    dkt[j] = mfma16x16x4(qr[e * P], da[qs][e], dkt[j]);
                }
            }
        if (it + 1 < niter) store(buf ^ 1);
        __syncthreads();
    }
    float *dkr = p.dk + ((long)b * s.n_kv + ki) * p.lddk + kvh * HD + 4 * g;
    float *dvr = p.dv + ((long)b * s.n_kv + ki) * p.lddv + kvh * HD + 4 * g;
    const float sc = s.inv_sqrt_dim;
    if constexpr (QKE) {
        __shared__ float red[4 * 128];
        const QkEpi &e = p.qk;
        float v[8][4], dw[8][4] = {};
#pragma unroll
        for (int j = 0; j < NU; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) v[j][r] = dkt[j][r] * sc;
        qk_row_bwd(v, dw, true, e, e.x + ((long)b * s.n_kv + ki) * e.ldx + (s.n_heads + kvh) * HD, e.gk, ki, g);
#pragma unroll
        for (int j = 0; j < NU; ++j) {
            *reinterpret_cast<float4 *>(dkr + 16 * j) = make_float4(v[j][0], v[j][1], v[j][2], v[j][3]);
            *reinterpret_cast<float4 *>(dvr + 16 * j) = make_float4(dvt[j][0], dvt[j][1], dvt[j][2], dvt[j][3]);
        }
        if (e.gk)  // uniform
            qk_dw_block(dw, red, wave, FNT / 64, true, lane, e.pk + ((long)blockIdx.y * gridDim.x + blockIdx.x) * HD);
        return;
    }
#pragma unroll
    for (int j = 0; j < NU; ++j) {
        *reinterpret_cast<float4 *>(dkr + 16 * j) =
            make_float4(dkt[j][0] * sc, dkt[j][1] * sc, dkt[j][2] * sc, dkt[j][3] * sc);
        *reinterpret_cast<float4 *>(dvr + 16 * j) = make_float4(dvt[j][0], dvt[j][1], dvt[j][2], dvt[j][3]);
    }
}

// ── dQ: block = 64 queries of one (sequence, head) ──────────────────────
// QKE: dQ leaves through RoPE^T and the Q-RMSNorm backward (p.qk), each block
// writing its q-gain partial to p.qk.pq[block].
template <int HD, bool QKE>
__global__ __launch_bounds__(FNT, 2) void fa_bwd_dq_f32m_k(AttnShape s, AttnPtrs p, bool zz) {
    static_assert(!QKE || HD == 128, "the fused q/k epilogue takes 128-wide head rows");
    constexpr int P = HD + 4, NU = HD / 16;
    __shared__ __attribute__((aligned(16))) float Ks[2][FT * P], Vs[2][FT * P];
    const int h = blockIdx.x % s.n_heads, b = blockIdx.x / s.n_heads;
    const int nqb = s.n_q / 64;
    const int y = (int)blockIdx.y, qb = s.causal ? nqb - 1 - (zz ? zigzag(y, nqb) : y) : y;
    const int tid = threadIdx.x, lane = tid % 64, g = lane / 16, c = lane % 16;
    const int wave = __builtin_amdgcn_readfirstlane(tid / 64);
    const int q0 = qb * 64, qw = q0 + 16 * wave, qi = qw + c;
    const int kvh = h / (s.n_heads / s.n_kv_heads);
    const float c2 = s.inv_sqrt_dim * F_LOG2E;
    const float *Q = (const float *)p.q, *K = (const float *)p.k, *V = (const float *)p.v,
                *dO = (const float *)p.dout;
    float4 qf[NU], of[NU];  // B of S^T = K Q^T and dP^T = V dO^T
    {
        const float *qr = Q + ((long)b * s.n_q + qi) * p.ldq + h * HD + 4 * g;
        const float *orr = dO + ((long)b * s.n_q + qi) * p.lddo + h * HD + 4 * g;
#pragma unroll
        for (int u = 0; u < NU; ++u) {
            qf[u] = f4_scale(f4(qr + 16 * u), c2);
            of[u] = f4(orr + 16 * u);
        }
    }
    const float l2 = p.lse[((long)b * s.n_q + qi) * s.n_heads + h] * F_LOG2E;
    const float dd = p.d[((long)b * s.n_q + qi) * s.n_heads + h];
    const int nkt = s.causal ? (q0 + 64) / FT : s.n_kv / FT;
    const float *kb = K + (long)b * s.n_kv * p.ldk + kvh * HD;
    const float *vb = V + (long)b * s.n_kv * p.ldv + kvh * HD;
    Tile<HD> tk, tv;
    tk.load(kb, p.ldk, tid);
    tv.load(vb, p.ldv, tid);
    tk.store(Ks[0], tid);
    tv.store(Vs[0], tid);
    __syncthreads();
    f32x4 dqt[NU];  // dQ^T[16 j + 4 g + r][qi]
#pragma unroll
    for (int j = 0; j < NU; ++j) dqt[j] = f32x4{0, 0, 0, 0};
    for (int it = 0; it < nkt; ++it) {
        const int buf = it & 1;
        if (it + 1 < nkt) {
            tk.load(kb + (long)(it + 1) * FT * p.ldk, p.ldk, tid);
            tv.load(vb + (long)(it + 1) * FT * p.ldv, p.ldv, tid);
        }
        const float *Kl = Ks[buf], *Vl = Vs[buf];
        const int kt0 = it * FT;
        f32x4 sa[2], da[2];  // S^T / dP^T[kt0 + 16 ks + 4 g + r][qi]
        bool live[2];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            sa[ks] = da[ks] = f32x4{0, 0, 0, 0};
            live[ks] = !s.causal || kt0 + 16 * ks <= qw + 15;  // wave-uniform
            if (live[ks]) {
                const float *kr = Kl + (16 * ks + c) * P + 4 * g;
                const float *vr = Vl + (16 * ks + c) * P + 4 * g;
#pragma unroll
                for (int u = 0; u < NU; ++u) {
                    sa[ks] = mfma4(f4(kr + 16 * u), qf[u], sa[ks]);
                    da[ks] = mfma4(f4(vr + 16 * u), of[u], da[ks]);
                }
            }
        }
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float pv = __builtin_amdgcn_exp2f(sa[ks][r] - l2);
                if (s.causal && kt0 + 16 * ks + 4 * g + r > qi) pv = 0.f;
                da[ks][r] = pv * (da[ks][r] - dd);  // dS^T
            }
        // dQ^T += K^T dS^T: step (ks, e) is key kt0 + 16 ks + 4 g + e
#pragma unroll
        for (int j = 0; j < NU; ++j)
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                if (!live[ks]) continue;
                const float *kr = Kl + (16 * ks + 4 * g) * P + 16 * j + c;
#pragma unroll
                for (int e = 0; e < 4; ++e) dqt[j] = mfma16x16x4(kr[e * P], da[ks][e], dqt[j]);
            }
        if (it + 1 < nkt) {
            tk.store(Ks[buf ^ 1], tid);
            tv.store(Vs[buf ^ 1], tid);
        }
        __syncthreads();
    }
    float *dqr = p.dq + ((long)b * s.n_q + qi) * p.lddq + h * HD + 4 * g;
    const float sc = s.inv_sqrt_dim;
    if constexpr (QKE) {
        __shared__ float red[4 * 128];
        const QkEpi &e = p.qk;
        float v[8][4], dw[8][4] = {};
#pragma unroll
        for (int j = 0; j < NU; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) v[j][r] = dqt[j][r] * sc;
        qk_row_bwd(v, dw, true, e, e.x + ((long)b * s.n_q + qi) * e.ldx + h * HD, e.gq, qi, g);
#pragma unroll
        for (int j = 0; j < NU; ++j)
            *reinterpret_cast<float4 *>(dqr + 16 * j) = make_float4(v[j][0], v[j][1], v[j][2], v[j][3]);
        if (e.gq)  // uniform
            qk_dw_block(dw, red, wave, FNT / 64, true, lane, e.pq + ((long)blockIdx.y * gridDim.x + blockIdx.x) * HD);
        return;
    }
#pragma unroll
    for (int j = 0; j < NU; ++j)
        *reinterpret_cast<float4 *>(dqr + 16 * j) =
            make_float4(dqt[j][0] * sc, dqt[j][1] * sc, dqt[j][2] * sc, dqt[j][3] * sc);
}

bool al16(const void *x) { return ((uintptr_t)x & 15) == 0; }

}  // namespace

// Shapes the fp32 tile kernels take: head_dim 64 or 128, whole 64-row tiles,
// a causal mask only with n_q == n_kv, rows 16-byte aligned.
bool fa_f32m_ok(const AttnShape &s) {
    return (s.head_dim == 64 || s.head_dim == 128) && s.n_q > 0 && s.n_kv > 0 &&
           s.n_q % 64 == 0 && s.n_kv % 64 == 0 && (!s.causal || s.n_q == s.n_kv) &&
           s.n_kv_heads > 0 && s.n_heads % s.n_kv_heads == 0;
}

bool fa_f32m_fwd(const AttnShape &s, const float *q, long ldq, const float *k, long ldk,
                 const float *v, long ldv, float *o, long ldo, float *lse, hipStream_t st) {
    if (!fa_f32m_ok(s) || !al16(q) || !al16(k) || !al16(v) || !al16(o) || ldq % 4 || ldk % 4 ||
        ldv % 4 || ldo % 4)
        return false;
    const dim3 grid(s.n_heads * s.n_batch, s.n_q / 64);
    const bool zz = fits_two_per_cu((long)grid.x * grid.y);
    if (s.head_dim == 128)
        hipLaunchKernelGGL(fa_fwd_f32m_k<128>, grid, dim3(FNT), 0, st, s, q, ldq, k, ldk, v, ldv, o, ldo, lse, zz);
    else
        hipLaunchKernelGGL(fa_fwd_f32m_k<64>, grid, dim3(FNT), 0, st, s, q, ldq, k, ldk, v, ldv, o, ldo, lse, zz);
    return true;
}

static bool ptrs_ok(const AttnPtrs &p) {
    return al16(p.q) && al16(p.k) && al16(p.v) && al16(p.dout) && p.ldq % 4 == 0 &&
           p.ldk % 4 == 0 && p.ldv % 4 == 0 && p.lddo % 4 == 0;
}

bool fa_f32m_dkv(const AttnShape &s, const AttnPtrs &p, hipStream_t st) {
    if (!fa_f32m_ok(s) || !ptrs_ok(p) || !al16(p.dk) || !al16(p.dv) || p.lddk % 4 || p.lddv % 4)
        return false;
    if (p.qk_fp32 && !fa_f32m_qk_ok(s, p)) return false;
    const dim3 grid(s.n_kv_heads * s.n_batch, s.n_kv / 64);
    const bool zz = fits_two_per_cu((long)grid.x * grid.y);
    if (p.qk_fp32) hipLaunchKernelGGL((fa_bwd_dkv_f32m_k<128, true>), grid, dim3(FNT), 0, st, s, p, zz);
    else if (s.head_dim == 128) hipLaunchKernelGGL((fa_bwd_dkv_f32m_k<128, false>), grid, dim3(FNT), 0, st, s, p, zz);
    else hipLaunchKernelGGL((fa_bwd_dkv_f32m_k<64, false>), grid, dim3(FNT), 0, st, s, p, zz);
    return true;
}

bool fa_f32m_dq(const AttnShape &s, const AttnPtrs &p, hipStream_t st) {
    if (!fa_f32m_ok(s) || !ptrs_ok(p) || !al16(p.dq) || p.lddq % 4) return false;
    if (p.qk_fp32 && !fa_f32m_qk_ok(s, p)) return false;
    const dim3 grid(s.n_heads * s.n_batch, s.n_q / 64);
    const bool zz = fits_two_per_cu((long)grid.x * grid.y);
    if (p.qk_fp32) hipLaunchKernelGGL((fa_bwd_dq_f32m_k<128, true>), grid, dim3(FNT), 0, st, s, p, zz);
    else if (s.head_dim == 128) hipLaunchKernelGGL((fa_bwd_dq_f32m_k<128, false>), grid, dim3(FNT), 0, st, s, p, zz);
    else hipLaunchKernelGGL((fa_bwd_dq_f32m_k<64, false>), grid, dim3(FNT), 0, st, s, p, zz);
    return true;
}

// The fused q/k epilogue's conditions: the tile kernels' shapes with 128-wide
// heads, a rotary span of 0 or the whole head, 16-byte aligned q/k input rows
// and gains, and every output pointer the tile kernels need.
bool fa_f32m_qk_ok(const AttnShape &s, const AttnPtrs &p) {
    const QkEpi &e = p.qk;
    return fa_f32m_ok(s) && s.head_dim == 128 && ptrs_ok(p) && al16(p.dq) && al16(p.dk) &&
           al16(p.dv) && p.lddq % 4 == 0 && p.lddk % 4 == 0 && p.lddv % 4 == 0 && e.x && al16(e.x) &&
           e.ldx % 4 == 0 && (e.rot == 0 || (e.rot == 128 && e.rope && al16(e.rope))) &&
           (!e.gq || (al16(e.gq) && e.pq)) && (!e.gk || (al16(e.gk) && e.pk));
}
int fa_f32m_dq_blocks(const AttnShape &s) { return s.n_heads * s.n_batch * (s.n_q / 64); }
int fa_f32m_dkv_blocks(const AttnShape &s) { return s.n_kv_heads * s.n_batch * (s.n_kv / 64); }

}  // namespace vkh
