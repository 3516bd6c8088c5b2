// FlashAttention forward (with LSE) and the FA-2 backward for gfx950.
//
// Reference kernels: shaders/fa_forward.comp, fa_bw_d.comp, fa_bw_dq.comp,
// fa_bw_dkv.comp; CPU oracle src/cpu/flash_attn.zig:91-376.  Same math
// (online softmax; backward recomputes P = exp(S - LSE), D = rowsum(O * dO),
// dS = P (dP - D)); causal limit k <= q + (n_kv - n_q); GQA head h reads
// kv head h / (n_heads / n_kv_heads).  Batch extension: rows are
// [n_batch * n], attention is block-diagonal per sequence.
//
// bf16 path (the hot path): v_mfma_f32_16x16x32_bf16 with fp32 accumulate.
// Scores are formed transposed where that lets P / dS be used straight from
// the accumulator registers as the B operand of the next MFMA:
//
//   forward:  S^T = K Q^T  ->  O^T += V^T P^T      (per-lane q column)
//   dK/dV:    S   = Q K^T  ->  dV^T += dO^T P,  dK^T += Q^T dS   (K, V in regs)
//   dQ:       S^T = K Q^T  ->  dQ^T += K^T dS^T                  (Q, dO in regs)
//
// An MFMA accumulator holds rows 4*(lane/16)+r and column lane%16; used as a
// B operand its rows become the contraction index, so the A operand that
// pairs with it reads its k values in the matching order {4g..4g+3,
// 16+4g..16+4g+3} from a transposed ([d][row]) LDS copy.  The transposed
// copies are produced in registers (4x8 bf16 block transpose) while the tile
// is staged, so every LDS access is an 8- or 16-byte vector op.
//
// Causal tiles that are entirely masked are skipped (the reference dQ kernel
// visits every key tile, fa_bw_dq.comp:114).  dQ is produced by its own
// kernel, so no atomics and the result is deterministic.
//
// fp32 path (precision = fp32, parity mode): one wave per query (or key) row,
// scalar FMAs with wave reductions, structured like the reference shaders.
#include "gemm16.hpp"
#include "ops.hpp"
#include "qkbwd.hpp"

namespace vkh {

namespace {

constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.6931471805599453f;
constexpr int NT = 256;

// ── bf16 tile staging ────────────────────────────────────────────────

// Stage a ROWS x HD bf16 tile (global rows [row0, row0 + ROWS), zero past
// rmax) into LDS: `direct` [ROWS][HD + 8] and/or `trans` [HD][ROWS + 8].
template <int ROWS, int HD>
VKH_DEV void stage_tile(const bf16 *g, long ld, int row0, int rmax, bf16 (*direct)[HD + 8],
                        bf16 (*trans)[ROWS + 8], int tid) {
    constexpr int DC = HD / 8, UNITS = (ROWS / 4) * DC;
    for (int u = tid; u < UNITS; u += NT) {
        const int rg = u / DC, dc = u % DC;
        uint4 w[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int r = row0 + rg * 4 + j;
            w[j] = r < rmax ? *reinterpret_cast<const uint4 *>(g + (long)r * ld + dc * 8)
                            : make_uint4(0, 0, 0, 0);
        }
        if (direct) {
#pragma unroll
            for (int j = 0; j < 4; ++j) *reinterpret_cast<uint4 *>(&direct[rg * 4 + j][dc * 8]) = w[j];
        }
        if (trans) {
            const uint32_t *w0 = &w[0].x, *w1 = &w[1].x, *w2 = &w[2].x, *w3 = &w[3].x;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                uint2 lo, hi;
                lo.x = (w0[c] & 0xffffu) | (w1[c] << 16);
                lo.y = (w2[c] & 0xffffu) | (w3[c] << 16);
                hi.x = (w0[c] >> 16) | (w1[c] & 0xffff0000u);
                hi.y = (w2[c] >> 16) | (w3[c] & 0xffff0000u);
                *reinterpret_cast<uint2 *>(&trans[dc * 8 + 2 * c][rg * 4]) = lo;
                *reinterpret_cast<uint2 *>(&trans[dc * 8 + 2 * c + 1][rg * 4]) = hi;
            }
        }
    }
}

// A-operand fragment from a transposed LDS copy: row `d`, contraction
// block starting at `k0` (32 wide), lane group g -> k {4g..4g+3, 16+4g..}.
template <int W>
VKH_DEV bf16x8 frag_trans(const bf16 (*t)[W], int d, int k0, int g) {
    const bf16x4 lo = *reinterpret_cast<const bf16x4 *>(&t[d][k0 + 4 * g]);
    const bf16x4 hi = *reinterpret_cast<const bf16x4 *>(&t[d][k0 + 16 + 4 * g]);
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

// B-operand fragment from two accumulator tiles (contraction rows 0-15 of
// tile a, 16-31 of tile b).
VKH_DEV bf16x8 frag_acc(const f32x4 &a, const f32x4 &b) {
    return cvt8(a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]);
}

VKH_DEV bf16x8 ld_frag(const bf16 *p) { return *reinterpret_cast<const bf16x8 *>(p); }

// ── forward ──────────────────────────────────────────────────────────
// Block: one (q-tile of 128 rows, head, sequence); 4 waves x 32 queries.
template <int HD>
__global__ __launch_bounds__(NT, 2) void fa_fwd_bf16_k(AttnShape s, const bf16 *q, long ldq,
                                                        const bf16 *k, long ldk, const bf16 *v,
                                                        long ldv, float *o, long ldo,
                                                        float *lse, bf16 *ob, long ldob) {
    constexpr int BM = 128, BN = 64, DS = HD / 32, DSUB = HD / 16;
    __shared__ __attribute__((aligned(16))) bf16 Ks[BN][HD + 8];
    __shared__ __attribute__((aligned(16))) bf16 Vt[HD][BN + 8];

    const int nqt = (s.n_q + BM - 1) / BM;
    // blockIdx.x = (head, sequence), blockIdx.y = q tile, heaviest (last) first
    const int qt = s.causal ? nqt - 1 - (int)blockIdx.y : (int)blockIdx.y;
    const int h = blockIdx.x % s.n_heads, b = blockIdx.x / s.n_heads;
    const int kvh = h / (s.n_heads / s.n_kv_heads);
    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64, g = lane / 16, c16 = lane % 16;
    const int q0 = qt * BM, qw0 = q0 + wave * 32;
    const int off = s.n_kv - s.n_q;
    const bf16 *qb = q + (long)b * s.n_q * ldq + h * HD;
    const bf16 *kb = k + (long)b * s.n_kv * ldk + kvh * HD;
    const bf16 *vb = v + (long)b * s.n_kv * ldv + kvh * HD;
    const float c2 = s.inv_sqrt_dim * LOG2E;

    bf16x8 qf[2][DS];
#pragma unroll
    for (int qs = 0; qs < 2; ++qs) {
        const int qr = qw0 + 16 * qs + c16;
#pragma unroll
        for (int ds = 0; ds < DS; ++ds)
            qf[qs][ds] = qr < s.n_q ? ld_frag(qb + (long)qr * ldq + 32 * ds + 8 * g) : bf16x8{};
    }
    f32x4 oacc[DSUB][2];
#pragma unroll
    for (int i = 0; i < DSUB; ++i) oacc[i][0] = oacc[i][1] = f32x4{0, 0, 0, 0};
    float m[2] = {-INFINITY, -INFINITY}, l[2] = {0.f, 0.f};

    int kend = s.n_kv;
    if (s.causal) kend = min(s.n_kv, q0 + BM + off);
    const int nkt = (kend + BN - 1) / BN;
    for (int kt = 0; kt < nkt; ++kt) {
        const int k0 = kt * BN;
        __syncthreads();
        stage_tile<BN, HD>(kb, ldk, k0, s.n_kv, Ks, nullptr, tid);
        stage_tile<BN, HD>(vb, ldv, k0, s.n_kv, nullptr, Vt, tid);
        __syncthreads();
        // keys beyond this wave's last visible key are masked; skip if all are
        const int wave_last_q = min(qw0 + 31, s.n_q - 1);
        if (s.causal && k0 > wave_last_q + off) continue;

        f32x4 st[4][2];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) st[ks][0] = st[ks][1] = f32x4{0, 0, 0, 0};
#pragma unroll
        for (int ds = 0; ds < DS; ++ds)
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const bf16x8 kf = ld_frag(&Ks[16 * ks + c16][32 * ds + 8 * g]);
                st[ks][0] = mfma16x16x32(kf, qf[0][ds], st[ks][0]);
                st[ks][1] = mfma16x16x32(kf, qf[1][ds], st[ks][1]);
            }
        bf16x8 pf[2][2];
#pragma unroll
        for (int qs = 0; qs < 2; ++qs) {
            const int qa = qw0 + 16 * qs + c16;
            float mt = -INFINITY;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int ka = k0 + 16 * ks + 4 * g + r;
                    float x = st[ks][qs][r] * c2;
                    if (ka >= s.n_kv || (s.causal && ka > qa + off)) x = -INFINITY;
                    st[ks][qs][r] = x;
                    mt = fmaxf(mt, x);
                }
            mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
            mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
            const float mn = fmaxf(m[qs], mt);
            const float so = (m[qs] == -INFINITY) ? 0.f : exp2f(m[qs] - mn);
            float lt = 0.f;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float x = st[ks][qs][r];
                    const float p = (x == -INFINITY) ? 0.f : exp2f(x - mn);
                    st[ks][qs][r] = p;
                    lt += p;
                }
            lt += __shfl_xor(lt, 16, 64);
            lt += __shfl_xor(lt, 32, 64);
            l[qs] = l[qs] * so + lt;
            m[qs] = mn;
#pragma unroll
            for (int i = 0; i < DSUB; ++i) oacc[i][qs] *= so;
            pf[qs][0] = frag_acc(st[0][qs], st[1][qs]);
            pf[qs][1] = frag_acc(st[2][qs], st[3][qs]);
        }
#pragma unroll
        for (int kst = 0; kst < 2; ++kst)
#pragma unroll
            for (int i = 0; i < DSUB; ++i) {
                const bf16x8 vf = frag_trans<BN + 8>(Vt, 16 * i + c16, 32 * kst, g);
                oacc[i][0] = mfma16x16x32(vf, pf[0][kst], oacc[i][0]);
                oacc[i][1] = mfma16x16x32(vf, pf[1][kst], oacc[i][1]);
            }
    }
#pragma unroll
    for (int qs = 0; qs < 2; ++qs) {
        const int qa = qw0 + 16 * qs + c16;
        if (qa >= s.n_q) continue;
        const float inv = l[qs] > 0.f ? 1.0f / l[qs] : 0.f;
        float *orow = o + ((long)b * s.n_q + qa) * ldo + h * HD;
#pragma unroll
        for (int i = 0; i < DSUB; ++i) {
            const f32x4 a = oacc[i][qs];
            const float4 ov = make_float4(a[0] * inv, a[1] * inv, a[2] * inv, a[3] * inv);
            if (o) *reinterpret_cast<float4 *>(orow + 16 * i + 4 * g) = ov;
            if (ob) {
                bf16x4 bv;
                bv[0] = (bf16)ov.x; bv[1] = (bf16)ov.y; bv[2] = (bf16)ov.z; bv[3] = (bf16)ov.w;
                *reinterpret_cast<bf16x4 *>(ob + ((long)b * s.n_q + qa) * ldob + h * HD + 16 * i + 4 * g) = bv;
            }
        }
        if (lse && g == 0)
            lse[((long)b * s.n_q + qa) * s.n_heads + h] =
                l[qs] > 0.f ? (m[qs] + log2f(l[qs])) * LN2 : -INFINITY;
    }
}

// ── backward: D = rowsum(O * dO) (fa_bw_d.comp), optional bf16 dO ─────
__global__ void fa_bw_d_k(AttnShape s, const float *o, long ldo, const float *dout, long lddo,
                          float *d, bf16 *dout16, long lddo16) {
    const int lane = threadIdx.x % 64;
    const long rows = (long)s.n_batch * s.n_q * s.n_heads;
    const long row = (long)blockIdx.x * (NT / 64) + threadIdx.x / 64;
    if (row >= rows) return;
    const long t = row / s.n_heads;
    const int h = (int)(row % s.n_heads);
    const float *orow = o + t * ldo + h * s.head_dim;
    const float *drow = dout + t * lddo + h * s.head_dim;
    double acc = 0;
    for (int e = lane; e < s.head_dim; e += 64) {
        float dv = drow[e];
        if (dout16) {
            const bf16 r = (bf16)dv;
            dout16[t * lddo16 + h * s.head_dim + e] = r;
            dv = (float)r;  // D must pair with the dO the MFMA kernels see
        }
        acc += (double)orow[e] * (double)dv;
    }
    acc = wave_sum(acc);
    if (lane == 0) d[t * s.n_heads + h] = (float)acc;
}

// Several (row, head) items per wave for head_dim 64 / 128: LPH = head_dim / 8
// lanes per item, 8 elements (two float4 of O and of dO) per lane, the fp64
// dot product reduced inside a DPP row; the next item's loads are issued
// before the current one is reduced.
template <int CTRL>
VKH_DEV double dppd(double v) {
    const long long b = __builtin_bit_cast(long long, v);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)b, CTRL, 0xf, 0xf, false);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(b >> 32), CTRL, 0xf, 0xf, false);
    return __builtin_bit_cast(double, ((long long)hi << 32) | (long long)(unsigned)lo);
}

// Eight elements of an fp32 or bf16 row, widened to fp32.
VKH_DEV void load_row8(const float *p, float4 &a, float4 &b) {
    a = reinterpret_cast<const float4 *>(p)[0];
    b = reinterpret_cast<const float4 *>(p)[1];
}
VKH_DEV void load_row8(const bf16 *p, float4 &a, float4 &b) {
    const bf16x8 v = *reinterpret_cast<const bf16x8 *>(p);
    a = make_float4((float)v[0], (float)v[1], (float)v[2], (float)v[3]);
    b = make_float4((float)v[4], (float)v[5], (float)v[6], (float)v[7]);
}

// D = rowsum(O * dO), LPH lanes per (row, head) with 8 elements each.  TI is
// the storage type of O and dO: fp32 (the reference's FaBwDPush layout; with
// dout16 the bf16 copy of dO the MFMA kernels read is written here too) or
// bf16 (both already in the operand precision: half the bytes to read).
template <int LPH, class TI>
__global__ __launch_bounds__(NT) void fa_bw_d8_k(AttnShape s, const TI *o, long ldo,
                                                  const TI *dout, long lddo, float *d,
                                                  bf16 *dout16, long lddo16) {
    constexpr int G = 64 / LPH;
    const int lane = threadIdx.x % 64, j = lane % LPH, g = lane / LPH;
    const long rows = (long)s.n_batch * s.n_q * s.n_heads;
    const long stride = (long)gridDim.x * (NT / 64) * G;
    const int hd = s.head_dim;
    struct It { float4 o0, o1, d0, d1; };
    auto fetch = [&](long it, It &x) {
        if (it < rows) {
            const long t = it / s.n_heads;
            const int h = (int)(it % s.n_heads);
            load_row8(o + t * ldo + h * hd + 8 * j, x.o0, x.o1);
            load_row8(dout + t * lddo + h * hd + 8 * j, x.d0, x.d1);
        } else {
            x.o0 = x.o1 = x.d0 = x.d1 = make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    long it = ((long)blockIdx.x * (NT / 64) + threadIdx.x / 64) * G + g;
    const long wave_first = it - g;
    It cur;
    fetch(it, cur);
    for (long wb = wave_first; wb < rows; wb += stride, it += stride) {
        It nxt;
        if (wb + stride < rows) fetch(it + stride, nxt);
        float dv[8] = {cur.d0.x, cur.d0.y, cur.d0.z, cur.d0.w, cur.d1.x, cur.d1.y, cur.d1.z, cur.d1.w};
        const float ov[8] = {cur.o0.x, cur.o0.y, cur.o0.z, cur.o0.w, cur.o1.x, cur.o1.y, cur.o1.z, cur.o1.w};
        const long t = it / s.n_heads;
        const int h = (int)(it % s.n_heads);
        if (dout16) {
            // D must pair with the dO the MFMA kernels see
            const bf16x8 r = cvt8(dv[0], dv[1], dv[2], dv[3], dv[4], dv[5], dv[6], dv[7]);
#pragma unroll
            for (int i = 0; i < 8; ++i) dv[i] = (float)r[i];
            if (it < rows) *reinterpret_cast<bf16x8 *>(dout16 + t * lddo16 + h * hd + 8 * j) = r;
        }
        double acc = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc += (double)ov[i] * (double)dv[i];
        acc += dppd<0xB1>(acc);
        acc += dppd<0x4E>(acc);
        acc += dppd<0x141>(acc);
        if constexpr (LPH == 16) acc += dppd<0x140>(acc);
        if (j == 0 && it < rows) d[t * s.n_heads + h] = (float)acc;
        if (wb + stride < rows) cur = nxt;
    }
}

// ── backward: dK, dV (fa_bw_dkv.comp) ────────────────────────────────
// Block: 128 keys of one kv head and sequence; 4 waves x 32 keys, K and V
// fragments resident in registers; loops over the heads of the GQA group
// and the q tiles (64 rows) that can see these keys.
template <int HD>
__global__ __launch_bounds__(NT, 1) void fa_bwd_dkv_bf16_k(AttnShape s, AttnPtrs p) {
    constexpr int BN = 128, BM = 64, DS = HD / 32, DSUB = HD / 16;
    __shared__ __attribute__((aligned(16))) bf16 Qs[BM][HD + 8];
    __shared__ __attribute__((aligned(16))) bf16 dOs[BM][HD + 8];
    __shared__ __attribute__((aligned(16))) bf16 Qt[HD][BM + 8];
    __shared__ __attribute__((aligned(16))) bf16 dOt[HD][BM + 8];
    __shared__ float lse_s[BM], d_s[BM];

    // blockIdx.x = (kv head, sequence), blockIdx.y = key tile: under a causal
    // mask the first key tiles see the most queries, so they go first
    const int kt = (int)blockIdx.y;
    const int kvh = blockIdx.x % s.n_kv_heads, b = blockIdx.x / s.n_kv_heads;
    const int hpk = s.n_heads / s.n_kv_heads;
    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64, g = lane / 16, c16 = lane % 16;
    const int k0 = kt * BN, kw0 = k0 + wave * 32;
    const int off = s.n_kv - s.n_q;
    const float c2 = s.inv_sqrt_dim * LOG2E;
    const bf16 *kb = (const bf16 *)p.k + (long)b * s.n_kv * p.ldk + kvh * HD;
    const bf16 *vb = (const bf16 *)p.v + (long)b * s.n_kv * p.ldv + kvh * HD;

    bf16x8 kf[2][DS], vf[2][DS];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
        const int kr = kw0 + 16 * ks + c16;
#pragma unroll
        for (int ds = 0; ds < DS; ++ds) {
            kf[ks][ds] = kr < s.n_kv ? ld_frag(kb + (long)kr * p.ldk + 32 * ds + 8 * g) : bf16x8{};
            vf[ks][ds] = kr < s.n_kv ? ld_frag(vb + (long)kr * p.ldv + 32 * ds + 8 * g) : bf16x8{};
        }
    }
    f32x4 dvt[DSUB][2], dkt[DSUB][2];
#pragma unroll
    for (int i = 0; i < DSUB; ++i) dvt[i][0] = dvt[i][1] = dkt[i][0] = dkt[i][1] = f32x4{0, 0, 0, 0};

    int qstart = 0;
    if (s.causal) qstart = max(0, k0 - off) / BM * BM;
    const int wave_first_k = kw0;
    for (int hh = 0; hh < hpk; ++hh) {
        const int h = kvh * hpk + hh;
        const bf16 *qb = (const bf16 *)p.q + (long)b * s.n_q * p.ldq + h * HD;
        const bf16 *ob = (const bf16 *)p.dout + (long)b * s.n_q * p.lddo + h * HD;
        for (int q0 = qstart; q0 < s.n_q; q0 += BM) {
            __syncthreads();
            stage_tile<BM, HD>(qb, p.ldq, q0, s.n_q, Qs, Qt, tid);
            stage_tile<BM, HD>(ob, p.lddo, q0, s.n_q, dOs, dOt, tid);
            if (tid < BM) {
                const int qa = q0 + tid;
                const long t = (long)b * s.n_q + qa;
                lse_s[tid] = qa < s.n_q ? p.lse[t * s.n_heads + h] * LOG2E : INFINITY;
                d_s[tid] = qa < s.n_q ? p.d[t * s.n_heads + h] : 0.f;
            }
            __syncthreads();
            // this wave's keys are all masked for every query of the tile?
            if (s.causal && wave_first_k > q0 + BM - 1 + off) continue;

            f32x4 sc[4][2], dp[4][2];
#pragma unroll
            for (int qs = 0; qs < 4; ++qs) sc[qs][0] = sc[qs][1] = dp[qs][0] = dp[qs][1] = f32x4{0, 0, 0, 0};
#pragma unroll
            for (int ds = 0; ds < DS; ++ds)
#pragma unroll
                for (int qs = 0; qs < 4; ++qs) {
                    const bf16x8 qa = ld_frag(&Qs[16 * qs + c16][32 * ds + 8 * g]);
                    const bf16x8 oa = ld_frag(&dOs[16 * qs + c16][32 * ds + 8 * g]);
                    sc[qs][0] = mfma16x16x32(qa, kf[0][ds], sc[qs][0]);
                    sc[qs][1] = mfma16x16x32(qa, kf[1][ds], sc[qs][1]);
                    dp[qs][0] = mfma16x16x32(oa, vf[0][ds], dp[qs][0]);
                    dp[qs][1] = mfma16x16x32(oa, vf[1][ds], dp[qs][1]);
                }
#pragma unroll
            for (int qs = 0; qs < 4; ++qs)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int ql = 16 * qs + 4 * g + r;
                    const int qa = q0 + ql;
                    const float lq = lse_s[ql], dq = d_s[ql];
#pragma unroll
                    for (int ks = 0; ks < 2; ++ks) {
                        const int ka = kw0 + 16 * ks + c16;
                        float pv = (lq == -INFINITY) ? 0.f : exp2f(sc[qs][ks][r] * c2 - lq);
                        if (qa >= s.n_q || ka >= s.n_kv || (s.causal && ka > qa + off)) pv = 0.f;
                        sc[qs][ks][r] = pv;
                        dp[qs][ks][r] = pv * (dp[qs][ks][r] - dq);
                    }
                }
#pragma unroll
            for (int qst = 0; qst < 2; ++qst) {
                const bf16x8 pb0 = frag_acc(sc[2 * qst][0], sc[2 * qst + 1][0]);
                const bf16x8 pb1 = frag_acc(sc[2 * qst][1], sc[2 * qst + 1][1]);
                const bf16x8 sb0 = frag_acc(dp[2 * qst][0], dp[2 * qst + 1][0]);
                const bf16x8 sb1 = frag_acc(dp[2 * qst][1], dp[2 * qst + 1][1]);
#pragma unroll
                for (int i = 0; i < DSUB; ++i) {
                    const bf16x8 oa = frag_trans<BM + 8>(dOt, 16 * i + c16, 32 * qst, g);
                    const bf16x8 qa = frag_trans<BM + 8>(Qt, 16 * i + c16, 32 * qst, g);
                    dvt[i][0] = mfma16x16x32(oa, pb0, dvt[i][0]);
                    dvt[i][1] = mfma16x16x32(oa, pb1, dvt[i][1]);
                    dkt[i][0] = mfma16x16x32(qa, sb0, dkt[i][0]);
                    dkt[i][1] = mfma16x16x32(qa, sb1, dkt[i][1]);
                }
            }
        }
    }
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
        const int ka = kw0 + 16 * ks + c16;
        if (ka >= s.n_kv) continue;
        const long t = (long)b * s.n_kv + ka;
        float *dkr = p.dk + t * p.lddk + kvh * HD;
        float *dvr = p.dv + t * p.lddv + kvh * HD;
#pragma unroll
        for (int i = 0; i < DSUB; ++i) {
            const f32x4 a = dkt[i][ks], c = dvt[i][ks];
            const float sc_ = s.inv_sqrt_dim;
            *reinterpret_cast<float4 *>(dkr + 16 * i + 4 * g) = make_float4(a[0] * sc_, a[1] * sc_, a[2] * sc_, a[3] * sc_);
            *reinterpret_cast<float4 *>(dvr + 16 * i + 4 * g) = make_float4(c[0], c[1], c[2], c[3]);
        }
    }
}

// ── backward: dQ (fa_bw_dq.comp) ─────────────────────────────────────
// Block: 128 queries of one head and sequence; 4 waves x 32 queries with
// Q and dO fragments in registers; loops over the key tiles (64) visible
// under the causal mask.
template <int HD>
__global__ __launch_bounds__(NT, 1) void fa_bwd_dq_bf16_k(AttnShape s, AttnPtrs p) {
    constexpr int BM = 128, BN = 64, DS = HD / 32, DSUB = HD / 16;
    __shared__ __attribute__((aligned(16))) bf16 Ks[BN][HD + 8];
    __shared__ __attribute__((aligned(16))) bf16 Vs[BN][HD + 8];
    __shared__ __attribute__((aligned(16))) bf16 Kt[HD][BN + 8];

    const int nqt = (s.n_q + BM - 1) / BM;
    // blockIdx.x = (head, sequence), blockIdx.y = q tile, heaviest (last) first
    const int qt = s.causal ? nqt - 1 - (int)blockIdx.y : (int)blockIdx.y;
    const int h = blockIdx.x % s.n_heads, b = blockIdx.x / s.n_heads;
    const int kvh = h / (s.n_heads / s.n_kv_heads);
    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64, g = lane / 16, c16 = lane % 16;
    const int q0 = qt * BM, qw0 = q0 + wave * 32;
    const int off = s.n_kv - s.n_q;
    const float c2 = s.inv_sqrt_dim * LOG2E;
    const bf16 *qb = (const bf16 *)p.q + (long)b * s.n_q * p.ldq + h * HD;
    const bf16 *ob = (const bf16 *)p.dout + (long)b * s.n_q * p.lddo + h * HD;
    const bf16 *kb = (const bf16 *)p.k + (long)b * s.n_kv * p.ldk + kvh * HD;
    const bf16 *vb = (const bf16 *)p.v + (long)b * s.n_kv * p.ldv + kvh * HD;

    bf16x8 qf[2][DS], of[2][DS];
    float lq[2], dq[2];
#pragma unroll
    for (int qs = 0; qs < 2; ++qs) {
        const int qa = qw0 + 16 * qs + c16;
        const bool ok = qa < s.n_q;
#pragma unroll
        for (int ds = 0; ds < DS; ++ds) {
            qf[qs][ds] = ok ? ld_frag(qb + (long)qa * p.ldq + 32 * ds + 8 * g) : bf16x8{};
            of[qs][ds] = ok ? ld_frag(ob + (long)qa * p.lddo + 32 * ds + 8 * g) : bf16x8{};
        }
        const long t = (long)b * s.n_q + qa;
        lq[qs] = ok ? p.lse[t * s.n_heads + h] * LOG2E : INFINITY;
        dq[qs] = ok ? p.d[t * s.n_heads + h] : 0.f;
    }
    f32x4 acc[DSUB][2];
#pragma unroll
    for (int i = 0; i < DSUB; ++i) acc[i][0] = acc[i][1] = f32x4{0, 0, 0, 0};

    int kend = s.n_kv;
    if (s.causal) kend = min(s.n_kv, q0 + BM + off);
    const int nkt = (kend + BN - 1) / BN;
    for (int kt = 0; kt < nkt; ++kt) {
        const int k0 = kt * BN;
        __syncthreads();
        stage_tile<BN, HD>(kb, p.ldk, k0, s.n_kv, Ks, Kt, tid);
        stage_tile<BN, HD>(vb, p.ldv, k0, s.n_kv, Vs, nullptr, tid);
        __syncthreads();
        const int wave_last_q = min(qw0 + 31, s.n_q - 1);
        if (s.causal && k0 > wave_last_q + off) continue;

        f32x4 st[4][2], dpt[4][2];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) st[ks][0] = st[ks][1] = dpt[ks][0] = dpt[ks][1] = f32x4{0, 0, 0, 0};
#pragma unroll
        for (int ds = 0; ds < DS; ++ds)
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const bf16x8 ka = ld_frag(&Ks[16 * ks + c16][32 * ds + 8 * g]);
                const bf16x8 va = ld_frag(&Vs[16 * ks + c16][32 * ds + 8 * g]);
                st[ks][0] = mfma16x16x32(ka, qf[0][ds], st[ks][0]);
                st[ks][1] = mfma16x16x32(ka, qf[1][ds], st[ks][1]);
                dpt[ks][0] = mfma16x16x32(va, of[0][ds], dpt[ks][0]);
                dpt[ks][1] = mfma16x16x32(va, of[1][ds], dpt[ks][1]);
            }
#pragma unroll
        for (int qs = 0; qs < 2; ++qs) {
            const int qa = qw0 + 16 * qs + c16;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int ka = k0 + 16 * ks + 4 * g + r;
                    float pv = (lq[qs] == -INFINITY) ? 0.f : exp2f(st[ks][qs][r] * c2 - lq[qs]);
                    if (qa >= s.n_q || ka >= s.n_kv || (s.causal && ka > qa + off)) pv = 0.f;
                    dpt[ks][qs][r] = pv * (dpt[ks][qs][r] - dq[qs]);
                }
        }
#pragma unroll
        for (int kst = 0; kst < 2; ++kst) {
            const bf16x8 s0 = frag_acc(dpt[2 * kst][0], dpt[2 * kst + 1][0]);
            const bf16x8 s1 = frag_acc(dpt[2 * kst][1], dpt[2 * kst + 1][1]);
#pragma unroll
            for (int i = 0; i < DSUB; ++i) {
                const bf16x8 ka = frag_trans<BN + 8>(Kt, 16 * i + c16, 32 * kst, g);
                acc[i][0] = mfma16x16x32(ka, s0, acc[i][0]);
                acc[i][1] = mfma16x16x32(ka, s1, acc[i][1]);
            }
        }
    }
#pragma unroll
    for (int qs = 0; qs < 2; ++qs) {
        const int qa = qw0 + 16 * qs + c16;
        if (qa >= s.n_q) continue;
        float *dqr = p.dq + ((long)b * s.n_q + qa) * p.lddq + h * HD;
        const float sc_ = s.inv_sqrt_dim;
#pragma unroll
        for (int i = 0; i < DSUB; ++i) {
            const f32x4 a = acc[i][qs];
            *reinterpret_cast<float4 *>(dqr + 16 * i + 4 * g) = make_float4(a[0] * sc_, a[1] * sc_, a[2] * sc_, a[3] * sc_);
        }
    }
}

// ── backward v2: dK/dV + dS (bf16) then dQ = dS K as a GEMM ───────────
//
// The dK/dV kernel keeps K and V of its 32 keys per wave in registers and
// streams the 64-row Q / dO tiles of every query head of the GQA group
// through double-buffered LDS, the next tile's global loads in flight while
// the current one computes (one barrier per tile).  The transposed operands
// (dO^T for dV, Q^T for dK) are read from the same row-major tiles with the
// gfx950 transposing LDS load (ds_read_b64_tr_b16), so no transposed copies
// are staged.  dS = P (dP - D) is written once as bf16 (exactly the values
// the dK MFMAs consume) to a [batch, head, n_kv, n_q] workspace (dS^T: each
// lane's 4 consecutive queries of one key are one 8-byte store), and dQ is
// then the plain product dS K, computed by the shared GEMM tile routine with
// the causal K limit; S and dP are not recomputed for dQ.
//
// ds_read_b64_tr_b16 (measured on MI355X): within each 16-lane group, lane i
// receives element (i % 4) of the 8-byte chunks addressed by lanes
// 4 j + i / 4, j = 0..3.  So if lane l of the group addresses row r0 + l / 4,
// column c0 + 4 (l % 4) of a row-major tile X, lane i gets X[r0 + j][c0 + i].

typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;

// X[r0 + j][c0 + (lane % 16)], j = 0..3, from a row-major LDS tile of pitch P
template <int P>
VKH_DEV bf16x4 ld_tr4(const bf16 *tile, int r0, int c0, int l16) {
    const bf16 *src = tile + (r0 + l16 / 4) * P + c0 + 4 * (l16 % 4);
    return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4 *)src);
}

// A operand (rows = tile columns c0 + lane%16, contraction = tile rows
// k0 + {4g..4g+3, 16+4g..16+4g+3}) read transposed from a row-major tile:
// the k order matches an accumulator used as the B operand (frag_acc).
template <int P>
VKH_DEV bf16x8 frag_tr(const bf16 *tile, int c0, int k0, int g, int l16) {
    const bf16x4 lo = ld_tr4<P>(tile, k0 + 4 * g, c0, l16);
    const bf16x4 hi = ld_tr4<P>(tile, k0 + 16 + 4 * g, c0, l16);
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

template <int HD, int BM>
__global__ __launch_bounds__(NT, 1) void fa_bwd_dkv2_k(AttnShape s, AttnPtrs p, bf16 *dsw) {
    constexpr int BN = 128, DS = HD / 32, DSUB = HD / 16;
    constexpr int QS = BM / 16, QST = BM / 32;  // 16-row score tiles, 32-row contraction steps
    constexpr int P = HD + 16;      // LDS pitch (elements): conflict-free b128 and tr reads
    constexpr int CH = HD / 8;      // 16-byte chunks per row
    constexpr int PER = BM * CH / NT;
    static_assert(PER * NT == BM * CH, "tile / thread mismatch");
    __shared__ __attribute__((aligned(16))) bf16 Qs[2][BM][P];
    __shared__ __attribute__((aligned(16))) bf16 Os[2][BM][P];
    __shared__ __attribute__((aligned(16))) bf16 Ks[BN][P];
    __shared__ __attribute__((aligned(16))) bf16 Vs[BN][P];
    __shared__ float lse_s[2][BM], d_s[2][BM];

    // blockIdx.x = (kv head, sequence), blockIdx.y = key tile: under a causal
    // mask the first key tiles see the most queries, so they go first
    const int kt = (int)blockIdx.y;
    const int kvh = blockIdx.x % s.n_kv_heads, b = blockIdx.x / s.n_kv_heads;
    const int hpk = s.n_heads / s.n_kv_heads;
    const int tid = threadIdx.x, lane = tid % 64, g = lane / 16, c16 = lane % 16;
    const int wave = __builtin_amdgcn_readfirstlane(tid / 64);  // uniform: scalar branches
    const int k0 = kt * BN, kw0 = k0 + wave * 32;
    const int off = s.n_kv - s.n_q;
    const float c2 = s.inv_sqrt_dim * LOG2E;
    const bf16 *kb = (const bf16 *)p.k + (long)b * s.n_kv * p.ldk + kvh * HD;
    const bf16 *vb = (const bf16 *)p.v + (long)b * s.n_kv * p.ldv + kvh * HD;

    // K and V of the block's keys stay in LDS (read as B fragments per tile):
    // holding them in registers would leave too few VGPRs for the tile.
    for (int u = tid; u < BN * CH; u += NT) {
        const int r = u / CH, c = u % CH, kr = k0 + r;
        const uint4 zero = make_uint4(0, 0, 0, 0);
        *reinterpret_cast<uint4 *>(&Ks[r][c * 8]) =
            kr < s.n_kv ? *reinterpret_cast<const uint4 *>(kb + (long)kr * p.ldk + c * 8) : zero;
        *reinterpret_cast<uint4 *>(&Vs[r][c * 8]) =
            kr < s.n_kv ? *reinterpret_cast<const uint4 *>(vb + (long)kr * p.ldv + c * 8) : zero;
    }
    f32x4 dvt[DSUB][2], dkt[DSUB][2];
#pragma unroll
    for (int i = 0; i < DSUB; ++i) dvt[i][0] = dvt[i][1] = dkt[i][0] = dkt[i][1] = f32x4{0, 0, 0, 0};

    // (query head, q tile) iterations, flattened so prefetch crosses heads
    const int qstart = s.causal ? max(0, k0 - off) / BM * BM : 0;
    const int nqt = s.n_q > qstart ? (s.n_q - qstart + BM - 1) / BM : 0;
    const int niter = hpk * nqt;

    uint4 rq[PER], ro[PER];
    float rl = 0.f, rd = 0.f;
    auto gload = [&](int it) {
        const int h = kvh * hpk + it / nqt, q0 = qstart + (it % nqt) * BM;
        const bf16 *qb = (const bf16 *)p.q + (long)b * s.n_q * p.ldq + h * HD;
        const bf16 *ob = (const bf16 *)p.dout + (long)b * s.n_q * p.lddo + h * HD;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int u = tid + i * NT, r = u / CH, c = u % CH, qa = q0 + r;
            rq[i] = qa < s.n_q ? *reinterpret_cast<const uint4 *>(qb + (long)qa * p.ldq + c * 8) : make_uint4(0, 0, 0, 0);
            ro[i] = qa < s.n_q ? *reinterpret_cast<const uint4 *>(ob + (long)qa * p.lddo + c * 8) : make_uint4(0, 0, 0, 0);
        }
        if (tid < BM) {
            const int qa = q0 + tid;
            const long t = (long)b * s.n_q + qa;
            rl = qa < s.n_q ? p.lse[t * s.n_heads + h] * LOG2E : INFINITY;
            rd = qa < s.n_q ? p.d[t * s.n_heads + h] : 0.f;
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int u = tid + i * NT, r = u / CH, c = u % CH;
            *reinterpret_cast<uint4 *>(&Qs[buf][r][c * 8]) = rq[i];
            *reinterpret_cast<uint4 *>(&Os[buf][r][c * 8]) = ro[i];
        }
        if (tid < BM) {
            lse_s[buf][tid] = rl;
            d_s[buf][tid] = rd;
        }
    };

    if (niter > 0) {
        gload(0);
        lstore(0);
    }
    __syncthreads();
    for (int it = 0; it < niter; ++it) {
        const int buf = it & 1;
        if (it + 1 < niter) gload(it + 1);
        const int h = kvh * hpk + it / nqt, q0 = qstart + (it % nqt) * BM;
        // dS^T rows of this lane's two keys: dsr[k * n_q + q]; 4 consecutive q per store
        bf16 *dsr = dsw + ((long)b * s.n_heads + h) * s.n_q * s.n_kv + (long)(kw0 + c16) * s.n_q +
                    q0 + 4 * g;
        const long ds_ks = 16L * s.n_q;
        const bool keys_ok = kw0 + 32 <= s.n_kv;
        // Waves whose keys are all above the diagonal run the same code (their
        // P and dS come out zero): one path keeps the accumulators in place.
        {
            const bf16 *Qb = &Qs[buf][0][0], *Ob = &Os[buf][0][0];
            f32x4 sc[QS][2], dp[QS][2];
#pragma unroll
            for (int qs = 0; qs < QS; ++qs) sc[qs][0] = sc[qs][1] = dp[qs][0] = dp[qs][1] = f32x4{0, 0, 0, 0};
#pragma unroll
            for (int ds = 0; ds < DS; ++ds) {
                const bf16x8 k0f = ld_frag(&Ks[wave * 32 + c16][32 * ds + 8 * g]);
                const bf16x8 k1f = ld_frag(&Ks[wave * 32 + 16 + c16][32 * ds + 8 * g]);
                const bf16x8 v0f = ld_frag(&Vs[wave * 32 + c16][32 * ds + 8 * g]);
                const bf16x8 v1f = ld_frag(&Vs[wave * 32 + 16 + c16][32 * ds + 8 * g]);
#pragma unroll
                for (int qs = 0; qs < QS; ++qs) {
                    const bf16x8 qa = ld_frag(Qb + (16 * qs + c16) * P + 32 * ds + 8 * g);
                    const bf16x8 oa = ld_frag(Ob + (16 * qs + c16) * P + 32 * ds + 8 * g);
                    sc[qs][0] = mfma16x16x32(qa, k0f, sc[qs][0]);
                    sc[qs][1] = mfma16x16x32(qa, k1f, sc[qs][1]);
                    dp[qs][0] = mfma16x16x32(oa, v0f, dp[qs][0]);
                    dp[qs][1] = mfma16x16x32(oa, v1f, dp[qs][1]);
                }
            }
            // P = exp2(S c2 - lse2); a fully masked row (lse = -inf) gets +inf -> P = 0.
            // Only tiles that touch the causal diagonal or an edge need per-element masks.
            const bool edge = (s.causal && kw0 + 31 > q0 + off) || !keys_ok;
#pragma unroll
            for (int qs = 0; qs < QS; ++qs) {
                const float4 l4 = *reinterpret_cast<const float4 *>(&lse_s[buf][16 * qs + 4 * g]);
                const float lqs[4] = {l4.x, l4.y, l4.z, l4.w};
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float lq = lqs[r] == -INFINITY ? INFINITY : lqs[r];
#pragma unroll
                    for (int ks = 0; ks < 2; ++ks) {
                        sc[qs][ks][r] = __builtin_amdgcn_exp2f(sc[qs][ks][r] * c2 - lq);
                    }
                }
            }
            if (edge) {
#pragma unroll
                for (int qs = 0; qs < QS; ++qs)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
#pragma unroll
                        for (int ks = 0; ks < 2; ++ks) {
                            const int qa = q0 + 16 * qs + 4 * g + r, ka = kw0 + 16 * ks + c16;
                            if (ka >= s.n_kv || (s.causal && ka > qa + off)) sc[qs][ks][r] = 0.f;
                        }
            }
#pragma unroll
            for (int qs = 0; qs < QS; ++qs) {
                const float4 d4 = *reinterpret_cast<const float4 *>(&d_s[buf][16 * qs + 4 * g]);
                const float dqs[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
                for (int r = 0; r < 4; ++r)
#pragma unroll
                    for (int ks = 0; ks < 2; ++ks)
                        dp[qs][ks][r] = sc[qs][ks][r] * (dp[qs][ks][r] - dqs[r]);
            }
#pragma unroll
            for (int ks = 0; ks < 2; ++ks)
#pragma unroll
                for (int qs = 0; qs < QS; ++qs) {
                    bf16x4 v;
                    v[0] = (bf16)dp[qs][ks][0]; v[1] = (bf16)dp[qs][ks][1];
                    v[2] = (bf16)dp[qs][ks][2]; v[3] = (bf16)dp[qs][ks][3];
                    if (keys_ok || kw0 + 16 * ks + c16 < s.n_kv)
                        *reinterpret_cast<bf16x4 *>(dsr + ks * ds_ks + 16 * qs) = v;
                }
#pragma unroll
            for (int qst = 0; qst < QST; ++qst) {
                const bf16x8 pb0 = frag_acc(sc[2 * qst][0], sc[2 * qst + 1][0]);
                const bf16x8 pb1 = frag_acc(sc[2 * qst][1], sc[2 * qst + 1][1]);
                const bf16x8 sb0 = frag_acc(dp[2 * qst][0], dp[2 * qst + 1][0]);
                const bf16x8 sb1 = frag_acc(dp[2 * qst][1], dp[2 * qst + 1][1]);
#pragma unroll
                for (int i = 0; i < DSUB; ++i) {
                    const bf16x8 oa = frag_tr<P>(Ob, 16 * i, 32 * qst, g, c16);
                    const bf16x8 qa = frag_tr<P>(Qb, 16 * i, 32 * qst, g, c16);
                    dvt[i][0] = mfma16x16x32(oa, pb0, dvt[i][0]);
                    dvt[i][1] = mfma16x16x32(oa, pb1, dvt[i][1]);
                    dkt[i][0] = mfma16x16x32(qa, sb0, dkt[i][0]);
                    dkt[i][1] = mfma16x16x32(qa, sb1, dkt[i][1]);
                }
            }
        }
        if (it + 1 < niter) lstore(buf ^ 1);
        // Pin the loop-carried dK/dV accumulators to AGPRs (the register
        // file the MFMAs accumulate in); otherwise the compiler carries them
        // in VGPRs and copies all of them in and out on every tile.
#pragma unroll
        for (int i = 0; i < DSUB; ++i)
            asm volatile("" : "+a"(dvt[i][0]), "+a"(dvt[i][1]), "+a"(dkt[i][0]), "+a"(dkt[i][1]));
        __syncthreads();
    }
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
        const int ka = kw0 + 16 * ks + c16;
        if (ka >= s.n_kv) continue;
        const long t = (long)b * s.n_kv + ka;
        float *dkr = p.dk + t * p.lddk + kvh * HD;
        float *dvr = p.dv + t * p.lddv + kvh * HD;
        const float sc_ = s.inv_sqrt_dim;
#pragma unroll
        for (int i = 0; i < DSUB; ++i) {
            const f32x4 a = dkt[i][ks], c = dvt[i][ks];
            *reinterpret_cast<float4 *>(dkr + 16 * i + 4 * g) = make_float4(a[0] * sc_, a[1] * sc_, a[2] * sc_, a[3] * sc_);
            *reinterpret_cast<float4 *>(dvr + 16 * i + 4 * g) = make_float4(c[0], c[1], c[2], c[3]);
        }
    }
}

// ── backward v3 (head_dim 128): dK/dV with the work split over two wave groups
//
// 8 waves per block of 128 keys.  Waves 0-3 ("P waves") own 32 keys each and
// compute S^T = K Q^T, P = exp2(S c - lse) and dV += P^T dO; waves 4-7 ("dS
// waves") own the same 32-key slices and compute dP^T = V dO^T, dS = P (dP - D)
// and dK += dS^T Q, taking P from the matching P wave through LDS (fp32, so
// dS is bit-identical to the one-group kernel).  Each wave then holds one
// 32 x 128 accumulator (64 registers) and one operand slice (K or V), which
// keeps it within 256 registers: two waves per SIMD, so one group's softmax /
// dS arithmetic overlaps the other group's MFMAs.
//
// Q / dO tiles (64 x 128 bf16) arrive by DMA (buffer_load ... lds) into
// unpadded LDS rows with a 16-byte chunk swizzle: chunk c of row r sits at
// c ^ (r & 15).  Measured on MI355X with the two fragment read patterns of
// this kernel (b128 rows, transposing b64): both run at the speed of a
// padded-pitch layout (no bank conflicts), where an unswizzled 256-byte pitch
// is 4x (b128) and 2.3x (transposing) slower.
// The next two tiles' DMA is in flight during the current tile (three
// buffers); there are two barriers per tile (P ready, tile done).

namespace dkv3 {
constexpr int NT3 = 512, BN = 128, BM = 64, HD = 128, DS = HD / 32, DSUB = HD / 16;
constexpr int QS = BM / 16, QST = BM / 32;
constexpr int TILE = BM * HD * 2;  // bytes of one Q or dO tile
constexpr int NBUF = 3;            // tile buffers (two DMA batches in flight)

VKH_DEV int swz(int r) { return r & 15; }

// byte offset of (row r, element col) in a swizzled tile
VKH_DEV int toff(int r, int col) { return r * (HD * 2) + (((col >> 3) ^ swz(r)) << 4) + (col & 7) * 2; }

VKH_DEV bf16x8 frag_row(const char *tile, int r, int col) {
    return *reinterpret_cast<const bf16x8 *>(tile + toff(r, col));
}

// X[r0 + j][c0 + (lane % 16)], j = 0..3 (see ld_tr4), from a swizzled tile
VKH_DEV bf16x4 tr4(const char *tile, int r0, int c0, int l16) {
    const char *src = tile + toff(r0 + l16 / 4, c0 + 4 * (l16 % 4));
    return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4 *)src);
}

// A operand of the dV / dK products: rows = tile columns c0 + lane % 16,
// contraction = tile rows k0 + {4g..4g+3, 16+4g..16+4g+3} (frag_acc order)
VKH_DEV bf16x8 frag_t(const char *tile, int c0, int k0, int g, int l16) {
    const bf16x4 lo = tr4(tile, k0 + 4 * g, c0, l16);
    const bf16x4 hi = tr4(tile, k0 + 16 + 4 * g, c0, l16);
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}
}  // namespace dkv3

__global__ __launch_bounds__(dkv3::NT3, 1) void fa_bwd_dkv3_k(AttnShape s, AttnPtrs p, bf16 *dsw) {
    using namespace dkv3;
    __shared__ __attribute__((aligned(16))) char Qs[NBUF][TILE];
    __shared__ __attribute__((aligned(16))) char Os[NBUF][TILE];
    __shared__ float Ls[NBUF][BM], Dd[NBUF][BM];
    __shared__ __attribute__((aligned(16))) f32x4 Pex[4][8][64];  // [pair][word/4][lane]

    // blockIdx.x = (kv head, sequence), blockIdx.y = key tile: under a causal
    // mask the first key tiles see the most queries, so they go first
    const int kt = (int)blockIdx.y;
    const int kvh = blockIdx.x % s.n_kv_heads, b = blockIdx.x / s.n_kv_heads;
    const int hpk = s.n_heads / s.n_kv_heads;
    const int tid = threadIdx.x, lane = tid % 64, g = lane / 16, c16 = lane % 16;
    const int wave = __builtin_amdgcn_readfirstlane(tid / 64);
    const bool pw = wave < 4;              // P wave (else dS wave)
    const int pair = wave & 3;
    const int k0 = kt * BN, kw0 = k0 + pair * 32;
    const float c2 = s.inv_sqrt_dim * LOG2E;
    const bool keys_ok = kw0 + 32 <= s.n_kv;

    // this wave's operand slice: K (P waves) or V (dS waves), 32 keys x HD
    const bf16 *kvb = pw ? (const bf16 *)p.k + (long)b * s.n_kv * p.ldk + kvh * HD
                         : (const bf16 *)p.v + (long)b * s.n_kv * p.ldv + kvh * HD;
    const long kvld = pw ? p.ldk : p.ldv;
    bf16x8 kv[2][DS];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
        const int kr = kw0 + 16 * ks + c16;
#pragma unroll
        for (int ds = 0; ds < DS; ++ds)
            kv[ks][ds] = kr < s.n_kv ? ld_frag(kvb + (long)kr * kvld + 32 * ds + 8 * g) : bf16x8{};
    }
    wait_vm0();  // the K / V slice is in registers before any DMA is queued
    f32x4 acc[DSUB][2];
#pragma unroll
    for (int i = 0; i < DSUB; ++i) acc[i][0] = acc[i][1] = f32x4{0, 0, 0, 0};

    // (query head, q tile) iterations; the fused path has n_q % 64 == 0 and
    // n_q == n_kv when causal.  Every key block walks the q tiles from the
    // last one down, heads inner: the co-resident blocks of one (sequence,
    // KV head), which sit on one XCD, then read the same Q / dO tile at about
    // the same time, so a tile comes from HBM once and from that XCD's L2 for
    // the others (walking up from each block's own diagonal, they read
    // different tiles and miss L2).
    const int qstart = s.causal ? k0 / BM * BM : 0;
    const int nqt = s.n_q > qstart ? (s.n_q - qstart) / BM : 0;
    const int niter = hpk * nqt;

    const sgpr4 rq = rsrc4((const bf16 *)p.q + (long)b * s.n_q * p.ldq,
                           (unsigned)((long)s.n_q * p.ldq * 2));
    const sgpr4 ro = rsrc4((const bf16 *)p.dout + (long)b * s.n_q * p.lddo,
                           (unsigned)((long)s.n_q * p.lddo * 2));
    const sgpr4 rl = rsrc4(p.lse + (long)b * s.n_q * s.n_heads, (unsigned)((long)s.n_q * s.n_heads * 4));
    const sgpr4 rd = rsrc4(p.d + (long)b * s.n_q * s.n_heads, (unsigned)((long)s.n_q * s.n_heads * 4));
    // DMA of tile `it` into buffer `buf`, issued by the P waves only (the dS
    // waves' global stores then never sit in front of a wait for the tile):
    // P wave w moves rows 16 w .. 16 w + 15 of Q and dO (four 4-row
    // instructions each); waves 0 / 1 also move lse / D.
    // Instruction i of P wave w fills tile rows 16 w + 4 i + g; lane (g, c16)
    // fetches the logical chunk stored at physical chunk c16 of its row.
    auto dma = [&](int it, int buf) {
        const int h = kvh * hpk + it % hpk, q0 = qstart + (nqt - 1 - it / hpk) * BM;
        const int r = q0 + 16 * wave + g;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int col = h * HD + 8 * (c16 ^ swz(16 * wave + 4 * i + g));
            const unsigned oq = (unsigned)(((r + 4 * i) * (int)p.ldq + col) * 2);
            const unsigned oo = (unsigned)(((r + 4 * i) * (int)p.lddo + col) * 2);
            dma16_async(rq, Qs[buf] + (16 * wave + 4 * i) * HD * 2, oq);
            dma16_async(ro, Os[buf] + (16 * wave + 4 * i) * HD * 2, oo);
        }
        if (wave == 0) dma4_async(rl, Ls[buf], (unsigned)(((q0 + lane) * s.n_heads + h) * 4));
        if (wave == 1) dma4_async(rd, Dd[buf], (unsigned)(((q0 + lane) * s.n_heads + h) * 4));
    };

    // Three tile buffers, two tiles in flight: at the top of iteration `it` a
    // P wave waits until only the newest batch (tile it + 1) is outstanding.
    if (pw) {
        if (niter > 0) dma(0, 0);
        if (niter > 1) dma(1, 1);
    }
    for (int it = 0; it < niter; ++it) {
        const int buf = it % NBUF;
        if (pw) {
            if (it + 1 < niter) {
                if (wave < 2) __builtin_amdgcn_s_waitcnt(0x0f70 | 9);  // 8 tile + 1 lse/D load
                else __builtin_amdgcn_s_waitcnt(0x0f70 | 8);
            } else {
                wait_vm0();
            }
        }
        lds_barrier();  // tile `it` landed; everyone is done with buffer (it + 2) % 3 and Pex
        if (it + 2 < niter && pw) dma(it + 2, (it + 2) % NBUF);
        const int h = kvh * hpk + it % hpk, q0 = qstart + (nqt - 1 - it / hpk) * BM;
        const char *Qb = Qs[buf], *Ob = Os[buf];
        const bool edge = (s.causal && kw0 + 31 > q0) || !keys_ok;
        f32x4 sc[QS][2];
#pragma unroll
        for (int qs = 0; qs < QS; ++qs) sc[qs][0] = sc[qs][1] = f32x4{0, 0, 0, 0};
        // phase 1: S^T (P waves) or dP^T (dS waves)
        const char *A1 = pw ? Qb : Ob;
#pragma unroll
        for (int ds = 0; ds < DS; ++ds)
#pragma unroll
            for (int qs = 0; qs < QS; ++qs) {
                const bf16x8 a = frag_row(A1, 16 * qs + c16, 32 * ds + 8 * g);
                sc[qs][0] = mfma16x16x32(a, kv[0][ds], sc[qs][0]);
                sc[qs][1] = mfma16x16x32(a, kv[1][ds], sc[qs][1]);
            }
        if (pw) {
            // P = exp2(S c2 - lse2); a fully masked row (lse = -inf) gets P = 0
#pragma unroll
            for (int qs = 0; qs < QS; ++qs) {
                const float4 l4 = *reinterpret_cast<const float4 *>(&Ls[buf][16 * qs + 4 * g]);
                const float lqs[4] = {l4.x, l4.y, l4.z, l4.w};
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float lq = lqs[r] == -INFINITY ? INFINITY : lqs[r] * LOG2E;
#pragma unroll
                    for (int ks = 0; ks < 2; ++ks)
                        sc[qs][ks][r] = __builtin_amdgcn_exp2f(sc[qs][ks][r] * c2 - lq);
                }
            }
            if (edge) {
#pragma unroll
                for (int qs = 0; qs < QS; ++qs)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
#pragma unroll
                        for (int ks = 0; ks < 2; ++ks) {
                            const int qa = q0 + 16 * qs + 4 * g + r, ka = kw0 + 16 * ks + c16;
                            if (ka >= s.n_kv || (s.causal && ka > qa)) sc[qs][ks][r] = 0.f;
                        }
            }
#pragma unroll
            for (int qs = 0; qs < QS; ++qs)
#pragma unroll
                for (int ks = 0; ks < 2; ++ks) Pex[pair][2 * qs + ks][lane] = sc[qs][ks];
        }
        lds_barrier();  // P ready
        if (pw) {
            // dV^T += dO^T P
#pragma unroll
            for (int qst = 0; qst < QST; ++qst) {
                const bf16x8 pb0 = frag_acc(sc[2 * qst][0], sc[2 * qst + 1][0]);
                const bf16x8 pb1 = frag_acc(sc[2 * qst][1], sc[2 * qst + 1][1]);
#pragma unroll
                for (int i = 0; i < DSUB; ++i) {
                    const bf16x8 oa = frag_t(Ob, 16 * i, 32 * qst, g, c16);
                    acc[i][0] = mfma16x16x32(oa, pb0, acc[i][0]);
                    acc[i][1] = mfma16x16x32(oa, pb1, acc[i][1]);
                }
            }
        } else {
            // dS = P (dP - D), stored as bf16 dS^T; dK^T += Q^T dS
            // wave-uniform base plus a 32-bit lane offset (a 64-bit per-lane
            // pointer here does not fit the register budget: it was spilled)
            bf16 *dsr = dsw + ((long)b * s.n_heads + h) * s.n_q * s.n_kv + (long)kw0 * s.n_q + q0;
            dsr += c16 * s.n_q + 4 * g;
            const long ds_ks = 16L * s.n_q;
#pragma unroll
            for (int qs = 0; qs < QS; ++qs) {
                const float4 d4 = *reinterpret_cast<const float4 *>(&Dd[buf][16 * qs + 4 * g]);
                const float dqs[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
                for (int ks = 0; ks < 2; ++ks) {
                    const f32x4 pv = Pex[pair][2 * qs + ks][lane];
#pragma unroll
                    for (int r = 0; r < 4; ++r) sc[qs][ks][r] = pv[r] * (sc[qs][ks][r] - dqs[r]);
                }
            }
#pragma unroll
            for (int ks = 0; ks < 2; ++ks)
#pragma unroll
                for (int qs = 0; qs < QS; ++qs) {
                    bf16x4 v;
                    v[0] = (bf16)sc[qs][ks][0]; v[1] = (bf16)sc[qs][ks][1];
                    v[2] = (bf16)sc[qs][ks][2]; v[3] = (bf16)sc[qs][ks][3];
                    if (keys_ok || kw0 + 16 * ks + c16 < s.n_kv)
                        *reinterpret_cast<bf16x4 *>(dsr + ks * ds_ks + 16 * qs) = v;
                }
#pragma unroll
            for (int qst = 0; qst < QST; ++qst) {
                const bf16x8 sb0 = frag_acc(sc[2 * qst][0], sc[2 * qst + 1][0]);
                const bf16x8 sb1 = frag_acc(sc[2 * qst][1], sc[2 * qst + 1][1]);
#pragma unroll
                for (int i = 0; i < DSUB; ++i) {
                    const bf16x8 qa = frag_t(Qb, 16 * i, 32 * qst, g, c16);
                    acc[i][0] = mfma16x16x32(qa, sb0, acc[i][0]);
                    acc[i][1] = mfma16x16x32(qa, sb1, acc[i][1]);
                }
            }
        }
    }
    // dK (scaled) from the dS waves, dV from the P waves
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
        const int ka = kw0 + 16 * ks + c16;
        if (ka >= s.n_kv) continue;
        const long t = (long)b * s.n_kv + ka;
        float *out = pw ? p.dv + t * p.lddv + kvh * HD : p.dk + t * p.lddk + kvh * HD;
        const float sc_ = pw ? 1.0f : s.inv_sqrt_dim;
#pragma unroll
        for (int i = 0; i < DSUB; ++i) {
            const f32x4 a = acc[i][ks];
            *reinterpret_cast<float4 *>(out + 16 * i + 4 * g) =
                make_float4(a[0] * sc_, a[1] * sc_, a[2] * sc_, a[3] * sc_);
        }
    }
}

// ── backward v4 (head_dim 128, an even number of query heads per KV head) ──
//
// Two kernels that each form S and dP themselves (seven score-sized products
// per (query, key) pair instead of five), so nothing of size
// [heads, n_q, n_kv] goes through HBM and neither kernel issues a global
// store inside its tile loop: the tile DMA is then the only vector-memory
// traffic there, and the waits for it can be counted exactly.
//
// Both are templates on the wave count NWV of a block.  NWV = 4: one wave
// per SIMD with 64 keys (dK/dV) or 64 queries (dQ) per wave in registers, so
// every MFMA operand fragment read from LDS feeds four MFMAs (half the LDS
// bytes per flop of a 32-row wave tile), accumulators in AGPRs.  NWV = 8: two
// waves per SIMD with 32 each, so one wave's softmax / dS arithmetic overlaps
// the other wave's MFMAs; on MI355X the 8-wave forms are the faster ones and
// are the ones launched.
VKH_DEV void st_row_bf16(bf16 *row, const float (&v)[8][4], int g) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        bf16x4 o;
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] = (bf16)v[i][r];
        *reinterpret_cast<bf16x4 *>(row + 16 * i + 4 * g) = o;
    }
}

namespace dkv4 {
constexpr int HD = 128, BM = 32, BN = 128;
constexpr int DS = HD / 32, DSUB = HD / 16, QS = BM / 16;
constexpr int TILE = BM * HD * 2;           // 8 KB: one Q or dO tile
constexpr int NBUF = 3;                     // tile buffers (two DMA batches in flight)
constexpr int STREAM = NBUF * 2 * TILE;     // 48 KB: one head group's Q / dO tiles
constexpr int LDS = 128 * 1024;            // tile streams + V in the loop, the exchange after
static_assert(2 * STREAM + BN * HD * 2 <= LDS, "tile streams and V slices exceed the LDS arena");
}  // namespace dkv4

// dK / dV.  Block = 128 keys of one (sequence, KV head); NWV waves = NWV / 2
// key slices x 2 head groups.  Wave (slice, group) holds K of its slice in
// VGPRs (V of the block's keys sits in LDS) and, per 32-query tile of a head
// of its group (heads kvh * hpk + group, + 2, ...), computes
//   S = Q K^T, dP = dO V^T            (A = Q / dO rows from LDS, b128)
//   P = exp2(S c - lse), dS = P (dP - D)
//   dV^T += dO^T P, dK^T += Q^T dS    (A = transposing LDS reads)
// P and dS are used straight from the accumulators as the B operands of the
// last two products (contraction rows in frag_acc order).  The two waves of a
// slice then sum their partial dK / dV through LDS: group 0 keeps dV and adds
// group 1's, group 1 keeps dK and adds group 0's.
// Each head group streams its Q / dO tiles through three LDS buffers (two
// tiles in flight); the first half of the group's waves moves Q (and lse),
// the second half dO (and D).  Tiles are visited from the last query down, heads inner, so the blocks
// of one (sequence, KV head), which sit on one XCD, read a tile at about the
// same time and share it in L2.  Under a causal mask the heaviest key blocks
// (lowest keys) have the lowest block ids and start first.
// NH: query heads per head group (hpk / 2) when known at compile time (1 for
// GQA 2:1, 2 for 4:1), 0 to read it from the shape; a constant turns the
// per-tile (head, query tile) split of the iteration index into shifts.
// PARTS = 2: the block's query heads are split between two blocks (blockIdx.z),
// each summing half of every head group's heads and writing its raw dK / dV
// (fp32, dK scaled) into its own slice of p.split_ws; fa_dkv_combine_k adds the
// two slices in part order and runs the epilogue.  That doubles the grid where
// the (sequence, KV head, key block) grid alone leaves CUs idle.
template <int NWV, bool QKE, int NH = 0, int PARTS = 1>
__global__ __launch_bounds__(NWV * 64, 1) void fa_bwd_dkv4_k(AttnShape s, AttnPtrs p) {
    using namespace dkv4;
    constexpr int NS = NWV / 2;                 // key slices per head group
    constexpr int KW = BN / NS, KS = KW / 16;   // keys per wave, 16-key sub-tiles
    constexpr int XSLOT = DSUB * KS * 64 * 16;  // one wave's dK^T or dV^T
    static_assert(NWV * XSLOT <= LDS, "exchange exceeds the LDS arena");
    constexpr int RP = BM / (NS / 2);           // Q or dO tile rows each wave moves
    using dkv3::frag_row;
    using dkv3::frag_t;
    __shared__ __attribute__((aligned(16))) char smem[LDS];
    __shared__ __attribute__((aligned(16))) float Ls[2][NBUF][64], Dd[2][NBUF][64];

    const int kt = (int)blockIdx.y;
    static_assert(PARTS == 1 || !QKE, "a split launch leaves the epilogue to the combine kernel");
    const int kvh = blockIdx.x % s.n_kv_heads, b = blockIdx.x / s.n_kv_heads;
    const int hpk = s.n_heads / s.n_kv_heads;
    const int nh = (NH ? NH : hpk / 2) / PARTS;  // this block's heads per head group
    const int zp = PARTS > 1 ? (int)blockIdx.z : 0;  // this block's half of the heads
    const int tid = threadIdx.x, lane = tid % 64, g = lane / 16, c16 = lane % 16;
    const int wave = __builtin_amdgcn_readfirstlane(tid / 64);
    const int sl = wave % NS, hg = wave / NS;  // key slice, head group
    // DMA share: the first half of a group's waves moves Q (and lse), the
    // second half dO (and D), RP rows each
    const bool tdo = sl >= NS / 2;
    const int part = sl % (NS / 2);
    const int k0 = kt * BN, kw0 = k0 + sl * KW;
    const float c2 = s.inv_sqrt_dim * LOG2E;

    // K and V of the slice as B operands: lane (g, c16) holds key 16 ks + c16,
    // d = 32 ds + 8 g .. + 7 (n_kv is a multiple of 128: no edge)
    bf16x8 kr[KS][DS];
    {
        const bf16 *kb = (const bf16 *)p.k + ((long)b * s.n_kv + kw0 + c16) * p.ldk + kvh * HD + 8 * g;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
            for (int ds = 0; ds < DS; ++ds) kr[ks][ds] = ld_frag(kb + 16L * ks * p.ldk + 32 * ds);
    }
    // V of the slice (64 rows, swizzled like the tiles) by DMA from the group-0 wave
    char *vsl = smem + 2 * STREAM + sl * KW * HD * 2;
    if (hg == 0) {
        const sgpr4 rv = rsrc4((const bf16 *)p.v + (long)b * s.n_kv * p.ldv,
                               (unsigned)((long)s.n_kv * p.ldv * 2));
#pragma unroll
        for (int i = 0; i < KW / 4; ++i) {
            const int r = 4 * i + g;
            const int col = kvh * HD + 8 * (c16 ^ dkv3::swz(r));
            dma16_async(rv, vsl + 4 * i * HD * 2, (unsigned)(((kw0 + r) * (int)p.ldv + col) * 2));
        }
    }
    wait_vm0();  // K in registers and V in LDS before any tile DMA is queued
    __syncthreads();
    f32x4 dvt[DSUB][KS], dkt[DSUB][KS];
#pragma unroll
    for (int i = 0; i < DSUB; ++i)
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) dvt[i][ks] = dkt[i][ks] = f32x4{0, 0, 0, 0};

    // causal: n_q == n_kv, so queries below k0 see none of the block's keys
    const int qstart = s.causal ? k0 : 0;
    const int nqt = (s.n_q - qstart) / BM;
    const int niter = nh * nqt;
    char *strm = smem + hg * STREAM;

    // this wave's DMA share: slice 0 moves Q and lse, slice 1 dO and D
    const sgpr4 rt = tdo ? rsrc4((const bf16 *)p.dout + (long)b * s.n_q * p.lddo,
                                (unsigned)((long)s.n_q * p.lddo * 2))
                        : rsrc4((const bf16 *)p.q + (long)b * s.n_q * p.ldq,
                                (unsigned)((long)s.n_q * p.ldq * 2));
    const int ldt = (int)(tdo ? p.lddo : p.ldq);
    const sgpr4 rs = rsrc4((tdo ? p.d : p.lse) + (long)b * s.n_q * s.n_heads,
                           (unsigned)((long)s.n_q * s.n_heads * 4));
    auto tile_of = [&](int it, int &h, int &q0) {
        h = kvh * hpk + hg + 2 * (zp * nh + it % nh);
        q0 = qstart + (nqt - 1 - it / nh) * BM;
    };
    // 9 vector-memory operations per wave and tile: instruction i fills tile
    // rows 4 i .. 4 i + 3, lane (g, c16) row 4 i + g at physical chunk c16
    // (the lane id is laundered so the per-lane offsets are recomputed here,
    // a few VALU operations, instead of being held in registers across the
    // loop: spilled, their reloads would wait for the tile DMA in flight)
    auto dma = [&](int it, int buf) {
        int h, q0;
        tile_of(it, h, q0);
        int ln = lane;
        asm volatile("" : "+v"(ln));
        const int lg = ln >> 4, l16 = ln & 15;
        char *dst = strm + buf * 2 * TILE + (tdo ? TILE : 0);
#pragma unroll
        for (int i = 0; i < RP / 4; ++i) {
            const int r = part * RP + 4 * i + lg;
            const int col = h * HD + 8 * (l16 ^ dkv3::swz(r));
            dma16_async(rt, dst + (part * RP + 4 * i) * HD * 2, (unsigned)(((q0 + r) * ldt + col) * 2));
        }
        if (part == 0) {  // uniform; each branch names its LDS array (no generic pointer)
            const unsigned so = (unsigned)(((q0 + ln) * s.n_heads + h) * 4);
            if (tdo) dma4_async(rs, Dd[hg][buf], so);
            else dma4_async(rs, Ls[hg][buf], so);
        }
    };

    if (niter > 0) dma(0, 0);
    if (niter > 1) dma(1, 1);
    // The tile loop is unrolled over the three buffers, so every LDS address
    // is a per-lane base plus a compile-time offset (no per-tile VALU adds).
    auto step = [&](const int it, auto bufc) {
        constexpr int buf = decltype(bufc)::value;
        if (it + 1 < niter) {  // tile it+1 (RP / 4 rows + the stats wave's dword) may stay in flight
            if (part == 0) __builtin_amdgcn_s_waitcnt(0x0f70 | (RP / 4 + 1));
            else __builtin_amdgcn_s_waitcnt(0x0f70 | (RP / 4));
        } else {
            wait_vm0();
        }
        lds_barrier();  // tile `it` landed; everyone is done with buffer (it + 2) % 3
        if (it + 2 < niter) dma(it + 2, (buf + 2) % NBUF);
        int h, q0;
        tile_of(it, h, q0);
        (void)h;
        const char *Qb = strm + buf * 2 * TILE, *Ob = Qb + TILE;
        // P = 0 where key kw0 + 16 ks + c16 lies above query q0 + 16 qs + 4 g + r,
        // i.e. 16 ks - r > lim[qs] (branch-free compare against a per-lane limit)
        const bool diag = s.causal && kw0 + KW - 1 > q0;
        int lim[QS];
#pragma unroll
        for (int qs = 0; qs < QS; ++qs) lim[qs] = s.causal ? q0 + 16 * qs + 4 * g - kw0 - c16 : (1 << 30);
        // lse and D of this lane's query rows q0 + 16 qs + 4 g + r, read from LDS
        // where they are used (not held across the tile).  Every query row sees
        // at least one key on this path (causal needs n_q == n_kv, so row q sees
        // keys 0..q), so its LSE is finite and no empty-row case arises here.
        auto lse2 = [&](int qs, int r) { return Ls[hg][buf][16 * qs + 4 * g + r] * LOG2E; };
        auto dval = [&](int qs, int r) { return Dd[hg][buf][16 * qs + 4 * g + r]; };
        // the dP accumulators start at -D, so they end as dP - D
        f32x4 sc[QS][KS], dp[QS][KS];
#pragma unroll
        for (int qs = 0; qs < QS; ++qs) {
            const f32x4 nd{-dval(qs, 0), -dval(qs, 1), -dval(qs, 2), -dval(qs, 3)};
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                sc[qs][ks] = f32x4{0, 0, 0, 0};
                dp[qs][ks] = nd;
            }
        }
        // Each phase walks its 8 A fragments with the next fragment's LDS read
        // issued before this one's MFMAs; the softmax and dS arithmetic of one
        // (qs, ks) tile rides along with each step of the following phase.
        bf16x8 fr[2];
        fr[0] = frag_row(Qb, c16, 8 * g);
        // S = Q K^T; f = (ds, qs) = (f / 2, f % 2)
#pragma unroll
        for (int f = 0; f < 8; ++f) {
            const int ds = f / 2, qs = f % 2, n = f + 1;
            fr[n & 1] = n < 8 ? frag_row(Qb, 16 * (n % 2) + c16, 32 * (n / 2) + 8 * g)
                              : frag_row(Ob, c16, 8 * g);
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) sc[qs][ks] = mfma16x16x32(fr[f & 1], kr[ks][ds], sc[qs][ks]);
        }
        // dP = dO V^T (V from LDS, each fragment read once and used for both
        // query halves), with P = exp2(S c - lse) of tile (f / 4, f % 4)
        bf16x8 vf[KS];
#pragma unroll
        for (int f = 0; f < 8; ++f) {
            const int ds = f / 2, qs = f % 2, n = f + 1;
            if (qs == 0)
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) vf[ks] = frag_row(vsl, 16 * ks + c16, 32 * ds + 8 * g);
            fr[n & 1] = n < 8 ? frag_row(Ob, 16 * (n % 2) + c16, 32 * (n / 2) + 8 * g)
                              : frag_t(Ob, 0, 0, g, c16);
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) dp[qs][ks] = mfma16x16x32(fr[f & 1], vf[ks], dp[qs][ks]);
            // the QS * KS score tiles spread evenly over the 8 steps
            constexpr int EVERY = 8 / (QS * KS);
            static_assert(EVERY >= 1 && EVERY * QS * KS == 8, "exp schedule");
            if (f % EVERY == 0) {
                const int t2 = f / EVERY, qs2 = t2 / KS, ks2 = t2 % KS;
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    sc[qs2][ks2][r] = __builtin_amdgcn_exp2f(sc[qs2][ks2][r] * c2 - lse2(qs2, r));
            }
        }
        if (diag) {  // keys above a query of the tile (uniform; no MFMA inside)
#pragma unroll
            for (int qs = 0; qs < QS; ++qs)
#pragma unroll
                for (int ks = 0; ks < KS; ++ks)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (16 * ks - r > lim[qs]) sc[qs][ks][r] = 0.f;
        }
        // dV^T += dO^T P, with dS = P (dP - D) of tile (i / 4, i % 4) (dp holds dP - D)
        {
            bf16x8 pb[KS];
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) pb[ks] = frag_acc(sc[0][ks], sc[1][ks]);
#pragma unroll
            for (int i = 0; i < DSUB; ++i) {
                const int n = i + 1;
                fr[n & 1] = n < DSUB ? frag_t(Ob, 16 * n, 0, g, c16) : frag_t(Qb, 0, 0, g, c16);
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) dvt[i][ks] = mfma16x16x32(fr[i & 1], pb[ks], dvt[i][ks]);
                constexpr int EVERY = DSUB / (QS * KS);
                static_assert(EVERY >= 1 && EVERY * QS * KS == DSUB, "dS schedule");
                if (i % EVERY == 0) {
                    const int t2 = i / EVERY, qs2 = t2 / KS, ks2 = t2 % KS;
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        dp[qs2][ks2][r] = sc[qs2][ks2][r] * dp[qs2][ks2][r];
                }
            }
        }
        // dK^T += Q^T dS
        {
            bf16x8 sb[KS];
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) sb[ks] = frag_acc(dp[0][ks], dp[1][ks]);
#pragma unroll
            for (int i = 0; i < DSUB; ++i) {
                if (i + 1 < DSUB) fr[(i + 1) & 1] = frag_t(Qb, 16 * (i + 1), 0, g, c16);
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) dkt[i][ks] = mfma16x16x32(fr[i & 1], sb[ks], dkt[i][ks]);
            }
        }
        // keep the loop-carried accumulators in AGPRs (the MFMA accumulate
        // file) when one wave holds the whole register file; with two waves
        // per SIMD the compiler's own split spills less
        if constexpr (NWV == 4) {
#pragma unroll
            for (int i = 0; i < DSUB; ++i)
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) asm volatile("" : "+a"(dvt[i][ks]), "+a"(dkt[i][ks]));
        }
    };
    for (int it0 = 0; it0 < niter; it0 += NBUF) {
        step(it0, std::integral_constant<int, 0>{});
        if (it0 + 1 < niter) step(it0 + 1, std::integral_constant<int, 1>{});
        if (it0 + 2 < niter) step(it0 + 2, std::integral_constant<int, 2>{});
    }
    // head-group exchange through the (now idle) tile arena
    wait_vm0();
    __syncthreads();
    f32x4 *xs = reinterpret_cast<f32x4 *>(smem + (sl * 2 + hg) * XSLOT);
    const f32x4 *xp = reinterpret_cast<const f32x4 *>(smem + (sl * 2 + (1 - hg)) * XSLOT);
    // group 0 hands over dK^T and keeps dV^T; group 1 the other way round
    auto give = [&](const f32x4 (&a)[DSUB][KS]) {
#pragma unroll
        for (int i = 0; i < DSUB; ++i)
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) xs[(i * KS + ks) * 64 + lane] = a[i][ks];
    };
    auto keep = [&](const f32x4 (&a)[DSUB][KS], float *base, long ld, float sc_) {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            float *out = base + ((long)b * s.n_kv + kw0 + 16 * ks + c16) * ld + kvh * HD;
#pragma unroll
            for (int i = 0; i < DSUB; ++i) {
                const f32x4 v = a[i][ks] + xp[(i * KS + ks) * 64 + lane];
                *reinterpret_cast<float4 *>(out + 16 * i + 4 * g) =
                    make_float4(v[0] * sc_, v[1] * sc_, v[2] * sc_, v[3] * sc_);
            }
        }
    };
    if (hg == 0) give(dkt);
    else give(dvt);
    __syncthreads();
    if constexpr (PARTS > 1) {
        const long R = (long)s.n_batch * s.n_kv, kvd = (long)s.n_kv_heads * HD;
        float *wk = p.split_ws + (long)zp * 2 * R * kvd, *wv = wk + R * kvd;
        if (hg == 0) keep(dvt, wv, kvd, 1.0f);
        else keep(dkt, wk, kvd, s.inv_sqrt_dim);
    } else if constexpr (!QKE) {
        if (hg == 0) keep(dvt, p.dv, p.lddv, 1.0f);
        else keep(dkt, p.dk, p.lddk, s.inv_sqrt_dim);
    } else {
        // bf16 rows of the fused [T, (H + 2 Hkv) hd] gradient: dV as is, dK
        // back through RoPE and the K-RMSNorm (gain partials per block)
        __shared__ float red[NS * 128];
        const QkEpi &e = p.qk;
        float dw[8][4] = {};
        const int kcol = s.n_heads * HD + kvh * HD, vcol = kcol + s.n_kv_heads * HD;
        auto rows = [&](const f32x4(&a)[DSUB][KS], bool is_k) {
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const int key = kw0 + 16 * ks + c16;
                const long t = (long)b * s.n_kv + key;
                const float sc_ = is_k ? s.inv_sqrt_dim : 1.0f;
                float v[8][4];
#pragma unroll
                for (int i = 0; i < DSUB; ++i) {
                    const f32x4 w = a[i][ks] + xp[(i * KS + ks) * 64 + lane];
#pragma unroll
                    for (int r = 0; r < 4; ++r) v[i][r] = w[r] * sc_;
                }
                if (is_k) qk_row_bwd(v, dw, true, e, e.x + t * e.ldx + kcol, e.gk, key, g);
                st_row_bf16(e.out + t * e.ldout + (is_k ? kcol : vcol), v, g);
            }
        };
        if (hg == 0) rows(dvt, false);
        else rows(dkt, true);
        if (e.gk) {
            const int blk = blockIdx.y * gridDim.x + blockIdx.x;
            qk_dw_block(dw, red, sl, NS, hg == 1, lane, e.pk + (long)blk * 128);
        }
    }
}

// The two slices of a split dK / dV launch (p.split_ws: [part][dK, dV][rows][kvd]
// fp32) added in part order, then written as the unsplit kernel writes them:
// with the fused epilogue (QKE) dV as bf16 and dK through RoPE^T and the
// K-RMSNorm backward as bf16 into the gradient rows, the gain gradient as one
// 128-wide partial row per block; otherwise fp32 dK and dV.  Block = 64 rows
// of one KV head, 4 waves of 16 rows in the accumulator row layout
// (lane (g, c) holds elements 16 i + 4 g + r of row c).
template <bool QKE>
__global__ __launch_bounds__(256) void fa_dkv_combine_k(AttnShape s, AttnPtrs p) {
    constexpr int HD = 128;
    __shared__ float red[4 * HD];
    const int kvh = blockIdx.y;
    const int lane = threadIdx.x % 64, g = lane / 16, c16 = lane % 16;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const long R = (long)s.n_batch * s.n_kv, kvd = (long)s.n_kv_heads * HD;
    const long t = (long)blockIdx.x * 64 + 16 * wave + c16;  // row b * n_kv + key
    const bool ok = t < R;
    const long tt = ok ? t : 0;
    const float *k0 = p.split_ws + tt * kvd + kvh * HD + 4 * g, *k1 = k0 + 2 * R * kvd;
    const float *v0 = k0 + R * kvd, *v1 = k1 + R * kvd;
    float vk[8][4], vv[8][4];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        float4 a = make_float4(0.f, 0.f, 0.f, 0.f), bb = a, c = a, d = a;
        if (ok) {
            a = *reinterpret_cast<const float4 *>(k0 + 16 * i);
            bb = *reinterpret_cast<const float4 *>(k1 + 16 * i);
            c = *reinterpret_cast<const float4 *>(v0 + 16 * i);
            d = *reinterpret_cast<const float4 *>(v1 + 16 * i);
        }
        vk[i][0] = a.x + bb.x; vk[i][1] = a.y + bb.y; vk[i][2] = a.z + bb.z; vk[i][3] = a.w + bb.w;
        vv[i][0] = c.x + d.x; vv[i][1] = c.y + d.y; vv[i][2] = c.z + d.z; vv[i][3] = c.w + d.w;
    }
    if constexpr (QKE) {
        const QkEpi &e = p.qk;
        float dw[8][4] = {};
        const int kcol = s.n_heads * HD + kvh * HD, vcol = kcol + s.n_kv_heads * HD;
        const int pos = (int)(tt % s.n_kv);
        qk_row_bwd(vk, dw, ok, e, e.x + tt * e.ldx + kcol, e.gk, pos, g);
        if (ok) {
            st_row_bf16(e.out + tt * e.ldout + kcol, vk, g);
            st_row_bf16(e.out + tt * e.ldout + vcol, vv, g);
        }
        if (e.gk && e.pk)  // uniform
            qk_dw_block(dw, red, wave, 4, true, lane,
                        e.pk + ((long)blockIdx.y * gridDim.x + blockIdx.x) * HD);
    } else if (ok) {
        float *dk = p.dk + t * p.lddk + kvh * HD + 4 * g, *dv = p.dv + t * p.lddv + kvh * HD + 4 * g;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            *reinterpret_cast<float4 *>(dk + 16 * i) = make_float4(vk[i][0], vk[i][1], vk[i][2], vk[i][3]);
            *reinterpret_cast<float4 *>(dv + 16 * i) = make_float4(vv[i][0], vv[i][1], vv[i][2], vv[i][3]);
        }
    }
}

namespace dq4 {
constexpr int HD = 128, BN = 32;
constexpr int KS = BN / 16, DS = HD / 32, DSUB = HD / 16;
constexpr int TILE = BN * HD * 2;  // 8 KB: one K or V tile
constexpr int NBUF = 3;
}  // namespace dq4

// dQ.  Block = BQ (256 or 128) queries of one (sequence, head) on NWV waves
// (8: two per SIMD, BQ / 8 queries each); wave w owns
// the 16-row query sub-tiles Q0 + 16 (NWV j + w), interleaved so that under a
// causal mask every wave has work until the block's last key tile.  Q and dO
// of those rows sit in VGPRs as B operands; per 32-key tile (K and V by DMA,
// three buffers)
//   S^T = K Q^T, dP^T = V dO^T         (A = K / V rows from LDS, b128)
//   P^T = exp2(S^T c - lse), dS^T = P^T (dP^T - D)   (lse, D: one query per lane)
//   dQ^T += K^T dS^T                   (A = transposing reads of the K tile)
// Key tiles ascend from 0, so all query blocks of a (sequence, head) read
// the same K / V tile at about the same time; the heaviest query blocks
// (highest queries) start first.
// WITH_D: D = rowsum(O dO) of the block's rows is formed here from bf16 O (the
// lane's 32 products in fp64, then the row's four lanes) and stored to p.d
// for the dK/dV kernel, which then runs after this one; no separate pass.
template <int NWV, bool WITH_D, bool QKE, int BQ>
__global__ __launch_bounds__(NWV * 64, 1) void fa_bwd_dq4_k(AttnShape s, AttnPtrs p) {
    using namespace dq4;
    constexpr int QSUB = BQ / 16 / NWV;  // 16-row query sub-tiles per wave
    constexpr int QST = 16 * NWV;        // row stride between a wave's sub-tiles
    constexpr int RPW = BN / NWV;        // K / V tile rows each wave moves by DMA
    using dkv3::frag_row;
    using dkv3::frag_t;
    __shared__ __attribute__((aligned(16))) char Kt[NBUF][TILE];
    __shared__ __attribute__((aligned(16))) char Vt[NBUF][TILE];

    const int qblk = s.causal ? (int)gridDim.y - 1 - (int)blockIdx.y : (int)blockIdx.y;
    const int h = blockIdx.x % s.n_heads, b = blockIdx.x / s.n_heads;
    const int kvh = h / (s.n_heads / s.n_kv_heads);
    const int tid = threadIdx.x, lane = tid % 64, g = lane / 16, c16 = lane % 16;
    const int wave = __builtin_amdgcn_readfirstlane(tid / 64);
    const int q00 = qblk * BQ + 16 * wave;  // first row of sub-tile j is q00 + QST j
    const float c2 = s.inv_sqrt_dim * LOG2E;

    bf16x8 qr[QSUB][DS], orr[QSUB][DS];
    float lq[QSUB], dd[QSUB];
#pragma unroll
    for (int j = 0; j < QSUB; ++j) {
        const int q = q00 + QST * j + c16;
        const bool ok = q < s.n_q;
        const long t = (long)b * s.n_q + q;
        const bf16 *qp = (const bf16 *)p.q + t * p.ldq + h * HD + 8 * g;
        const bf16 *op = (const bf16 *)p.dout + t * p.lddo + h * HD + 8 * g;
#pragma unroll
        for (int ds = 0; ds < DS; ++ds) {
            qr[j][ds] = ok ? ld_frag(qp + 32 * ds) : bf16x8{};
            orr[j][ds] = ok ? ld_frag(op + 32 * ds) : bf16x8{};
        }
        const float l = ok ? p.lse[t * s.n_heads + h] : -INFINITY;
        // rows past n_q and fully masked rows (lse = -inf) get P = 0
        lq[j] = l == -INFINITY ? INFINITY : l * LOG2E;
        if constexpr (WITH_D) {
            const bf16 *opo = (const bf16 *)p.o16 + t * p.ldo16 + h * HD + 8 * g;
            double acc = 0;
#pragma unroll
            for (int ds = 0; ds < DS; ++ds) {
                const bf16x8 ov = ok ? ld_frag(opo + 32 * ds) : bf16x8{};
#pragma unroll
                for (int e = 0; e < 8; ++e) acc += (double)(float)ov[e] * (double)(float)orr[j][ds][e];
            }
            acc += __shfl_xor(acc, 16, 64);
            acc += __shfl_xor(acc, 32, 64);
            dd[j] = ok ? (float)acc : 0.f;
            if (ok && g == 0) p.d[t * s.n_heads + h] = dd[j];
        } else {
            dd[j] = ok ? p.d[t * s.n_heads + h] : 0.f;
        }
    }
    wait_vm0();
    f32x4 acc[DSUB][QSUB];
#pragma unroll
    for (int i = 0; i < DSUB; ++i)
#pragma unroll
        for (int j = 0; j < QSUB; ++j) acc[i][j] = f32x4{0, 0, 0, 0};

    const int kend = s.causal ? min(s.n_kv, qblk * BQ + BQ) : s.n_kv;
    const int ntl = (kend + BN - 1) / BN;
    const sgpr4 rk = rsrc4((const bf16 *)p.k + (long)b * s.n_kv * p.ldk,
                           (unsigned)((long)s.n_kv * p.ldk * 2));
    const sgpr4 rv = rsrc4((const bf16 *)p.v + (long)b * s.n_kv * p.ldv,
                           (unsigned)((long)s.n_kv * p.ldv * 2));
    // wave w moves rows RPW w .. RPW w + RPW - 1 of the K and V tiles
    // (RPW / 2 operations)
    auto dma = [&](int t, int buf) {
        const int kk = t * BN;
#pragma unroll
        for (int i = 0; i < RPW / 4; ++i) {
            const int r = RPW * wave + 4 * i + g;
            const int col = kvh * HD + 8 * (c16 ^ dkv3::swz(r));
            const int lo = (RPW * wave + 4 * i) * HD * 2;
            dma16_async(rk, Kt[buf] + lo, (unsigned)(((kk + r) * (int)p.ldk + col) * 2));
            dma16_async(rv, Vt[buf] + lo, (unsigned)(((kk + r) * (int)p.ldv + col) * 2));
        }
    };
    if (ntl > 0) dma(0, 0);
    if (ntl > 1) dma(1, 1);
    // The tile loop is unrolled over the three buffers, so every LDS address
    // is a per-lane base plus a compile-time offset (no per-tile VALU adds).
    auto step = [&](const int t, auto bufc) {
        constexpr int buf = decltype(bufc)::value;
        if (t + 1 < ntl) __builtin_amdgcn_s_waitcnt(0x0f70 | (RPW / 2));
        else wait_vm0();
        lds_barrier();
        if (t + 2 < ntl) dma(t + 2, (buf + 2) % NBUF);
        const int kk = t * BN;
        const char *Kb = Kt[buf], *Vb = Vt[buf];
        // P = 0 where key kk + 16 ks + 4 g + r lies above query q00 + 64 j + c16,
        // i.e. 16 ks + r > lim[j] (branch-free compare against a per-lane limit)
        int lim[QSUB];
#pragma unroll
        for (int j = 0; j < QSUB; ++j)
            lim[j] = min(s.causal ? q00 + QST * j + c16 - kk - 4 * g : (1 << 30), s.n_kv - 1 - kk - 4 * g);
        const bool diag = (s.causal && kk + BN - 1 > q00) || kk + BN > s.n_kv;
        // the dP^T accumulators start at -D (one query per lane), so they end as dP^T - D
        f32x4 st[KS][QSUB], dpt[KS][QSUB];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
            for (int j = 0; j < QSUB; ++j) {
                st[ks][j] = f32x4{0, 0, 0, 0};
                dpt[ks][j] = f32x4{-dd[j], -dd[j], -dd[j], -dd[j]};
            }
        // The three phases walk 24 operand fragments in one sequence (slots
        // 0-7: K rows for S^T, f = (ds, ks) = (f / 2, f % 2); 8-15: V rows for
        // dP^T; 16-23: transposed K for dQ^T), each slot's LDS read issued PD
        // slots ahead of its MFMAs through a ring of PD + 1 fragments.
        constexpr int PD = 2, RING = PD + 1;
        auto ldslot = [&](int n) -> bf16x8 {
            if (n < 8) return frag_row(Kb, 16 * (n % 2) + c16, 32 * (n / 2) + 8 * g);
            if (n < 16) return frag_row(Vb, 16 * ((n - 8) % 2) + c16, 32 * ((n - 8) / 2) + 8 * g);
            return frag_t(Kb, 16 * (n - 16), 0, g, c16);
        };
        bf16x8 fr[RING];
#pragma unroll
        for (int n = 0; n < PD; ++n) fr[n] = ldslot(n);
        // S^T = K Q^T
#pragma unroll
        for (int f = 0; f < 8; ++f) {
            const int ds = f / 2, ks = f % 2, n = f;
            fr[(n + PD) % RING] = ldslot(n + PD);
#pragma unroll
            for (int j = 0; j < QSUB; ++j) st[ks][j] = mfma16x16x32(fr[n % RING], qr[j][ds], st[ks][j]);
        }
        // dP^T = V dO^T, with P^T = exp2(S^T c - lse) of one (ks, j) tile per step
#pragma unroll
        for (int f = 0; f < 8; ++f) {
            const int ds = f / 2, ks = f % 2, n = 8 + f;
            fr[(n + PD) % RING] = ldslot(n + PD);
#pragma unroll
            for (int j = 0; j < QSUB; ++j) dpt[ks][j] = mfma16x16x32(fr[n % RING], orr[j][ds], dpt[ks][j]);
            // the KS * QSUB score tiles spread evenly over the 8 steps
            constexpr int EVERY = 8 / (KS * QSUB);
            static_assert(EVERY >= 1 && EVERY * KS * QSUB == 8, "exp schedule");
            if (f % EVERY == 0) {
                const int t2 = f / EVERY, ks2 = t2 / QSUB, j2 = t2 % QSUB;
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    st[ks2][j2][r] = __builtin_amdgcn_exp2f(st[ks2][j2][r] * c2 - lq[j2]);
            }
        }
        if (diag) {  // keys above a query of this wave (uniform; no MFMA inside)
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
#pragma unroll
                for (int j = 0; j < QSUB; ++j)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (16 * ks + r > lim[j]) st[ks][j][r] = 0.f;
        }
        // dS^T = P^T (dP^T - D) -> bf16 B operands (contraction = keys)
        bf16x8 sb[QSUB];
#pragma unroll
        for (int j = 0; j < QSUB; ++j) {
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
#pragma unroll
                for (int r = 0; r < 4; ++r) dpt[ks][j][r] = st[ks][j][r] * dpt[ks][j][r];
            sb[j] = frag_acc(dpt[0][j], dpt[1][j]);
        }
        // dQ^T += K^T dS^T
#pragma unroll
        for (int i = 0; i < DSUB; ++i) {
            const int n = 16 + i;
            if (n + PD < 24) fr[(n + PD) % RING] = ldslot(n + PD);
#pragma unroll
            for (int j = 0; j < QSUB; ++j) acc[i][j] = mfma16x16x32(fr[n % RING], sb[j], acc[i][j]);
        }
    };
    for (int t0 = 0; t0 < ntl; t0 += NBUF) {
        step(t0, std::integral_constant<int, 0>{});
        if (t0 + 1 < ntl) step(t0 + 1, std::integral_constant<int, 1>{});
        if (t0 + 2 < ntl) step(t0 + 2, std::integral_constant<int, 2>{});
    }
    // acc[i][j][r] = dQ^T[16 i + 4 g + r][q00 + 64 j + c16]
    if constexpr (QKE) {
        // bf16 rows of the fused gradient, back through RoPE and the Q-RMSNorm
        __shared__ float red[NWV * 128];
        const QkEpi &e = p.qk;
        float dw[8][4] = {};
#pragma unroll
        for (int j = 0; j < QSUB; ++j) {
            const int q = q00 + QST * j + c16;
            const bool ok = q < s.n_q;
            const long t = (long)b * s.n_q + (ok ? q : 0);
            float v[8][4];
#pragma unroll
            for (int i = 0; i < DSUB; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) v[i][r] = acc[i][j][r] * s.inv_sqrt_dim;
            qk_row_bwd(v, dw, ok, e, e.x + t * e.ldx + h * HD, e.gq, ok ? q : 0, g);
            if (ok) st_row_bf16(e.out + t * e.ldout + h * HD, v, g);
        }
        if (e.gq) {
            const int blk = blockIdx.y * gridDim.x + blockIdx.x;
            qk_dw_block(dw, red, wave, NWV, true, lane, e.pq + (long)blk * 128);
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < QSUB; ++j) {
        const int q = q00 + QST * j + c16;
        if (q >= s.n_q) continue;
        float *dqr = p.dq + ((long)b * s.n_q + q) * p.lddq + h * HD;
        const float sc_ = s.inv_sqrt_dim;
#pragma unroll
        for (int i = 0; i < DSUB; ++i) {
            const f32x4 a = acc[i][j];
            *reinterpret_cast<float4 *>(dqr + 16 * i + 4 * g) =
                make_float4(a[0] * sc_, a[1] * sc_, a[2] * sc_, a[3] * sc_);
        }
    }
}

// ── forward v3 (head_dim 128): DMA-staged K / V tiles ────────────────────
// One (q tile of 64 QS rows, head, sequence) per block, 4 waves x 16 QS queries
// (QS = 1 where 128-query blocks would be at most one per CU: config 3's 256
// become 512 blocks of 64, two per CU: the step 19.06-19.10 -> 18.86-18.89
// ms),
// Q fragments in registers.  64-key K and V tiles arrive by DMA into the
// swizzled LDS layout of the backward kernel (two buffers, the next tile in
// flight while the current one computes, one barrier per tile); K feeds the
// score MFMAs as row fragments and V^T comes straight from the row-major V
// tile through the transposing LDS read (no transposed staging copy).
// Causal q tiles go heaviest first (a zigzag order, zigzag in common.hpp,
// measured 77.6 against 78.9 us at config 4's 512-block grid: within noise).
template <int QS>
__global__ __launch_bounds__(256, 2) void fa_fwd3_k(AttnShape s, const bf16 *q, long ldq,
                                                     const bf16 *k, long ldk, const bf16 *v,
                                                     long ldv, float *o, long ldo, float *lse,
                                                     bf16 *ob, long ldob) {
    using namespace dkv3;
    constexpr int FBM = 64 * QS, FBN = 64, KT = FBN * HD * 2;
    __shared__ __attribute__((aligned(16))) char Ks[2][KT];
    __shared__ __attribute__((aligned(16))) char Vs[2][KT];

    const int nqt = (s.n_q + FBM - 1) / FBM;
    // blockIdx.x = (head, sequence), blockIdx.y = q tile, heaviest (last) first
    const int qt = s.causal ? nqt - 1 - (int)blockIdx.y : (int)blockIdx.y;
    const int h = blockIdx.x % s.n_heads, b = blockIdx.x / s.n_heads;
    const int kvh = h / (s.n_heads / s.n_kv_heads);
    const int tid = threadIdx.x, lane = tid % 64, g = lane / 16, c16 = lane % 16;
    const int wave = __builtin_amdgcn_readfirstlane(tid / 64);
    const int q0 = qt * FBM, qw0 = q0 + wave * 16 * QS;
    const int off = s.n_kv - s.n_q;
    const bf16 *qb = q + (long)b * s.n_q * ldq + h * HD;
    const float c2 = s.inv_sqrt_dim * LOG2E;

    bf16x8 qf[QS][DS];
#pragma unroll
    for (int qs = 0; qs < QS; ++qs) {
        const int qr = qw0 + 16 * qs + c16;
#pragma unroll
        for (int ds = 0; ds < DS; ++ds)
            qf[qs][ds] = qr < s.n_q ? ld_frag(qb + (long)qr * ldq + 32 * ds + 8 * g) : bf16x8{};
    }
    wait_vm0();  // Q fragments are in registers before any DMA is queued
    f32x4 oacc[DSUB][QS];
    float m[QS], l[QS];
#pragma unroll
    for (int qs = 0; qs < QS; ++qs) {
        m[qs] = -INFINITY;
        l[qs] = 0.f;
#pragma unroll
        for (int i = 0; i < DSUB; ++i) oacc[i][qs] = f32x4{0, 0, 0, 0};
    }

    int kend = s.n_kv;
    if (s.causal) kend = min(s.n_kv, q0 + FBM + off);
    const int nkt = (kend + FBN - 1) / FBN;
    const sgpr4 rk = rsrc4(k + (long)b * s.n_kv * ldk, (unsigned)((long)s.n_kv * ldk * 2));
    const sgpr4 rv = rsrc4(v + (long)b * s.n_kv * ldv, (unsigned)((long)s.n_kv * ldv * 2));
    // wave w moves rows 16 w .. 16 w + 15 of the K and V tiles (keys past
    // n_kv read as zero through the buffer bound)
    auto dma = [&](int kt, int buf) {
        const int k0 = kt * FBN;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = 16 * wave + 4 * i + g;
            const int c = c16 ^ swz(r);
            dma16_async(rk, Ks[buf] + (16 * wave + 4 * i) * HD * 2,
                        (unsigned)(((k0 + r) * (int)ldk + kvh * HD + 8 * c) * 2));
            dma16_async(rv, Vs[buf] + (16 * wave + 4 * i) * HD * 2,
                        (unsigned)(((k0 + r) * (int)ldv + kvh * HD + 8 * c) * 2));
        }
    };
    if (nkt > 0) dma(0, 0);
    const int wave_last_q = min(qw0 + 16 * QS - 1, s.n_q - 1);
    for (int kt = 0; kt < nkt; ++kt) {
        const int k0 = kt * FBN, buf = kt & 1;
        wait_vm0();
        lds_barrier();  // tile kt landed; everyone is done with buffer buf ^ 1
        if (kt + 1 < nkt) dma(kt + 1, buf ^ 1);
        // keys beyond this wave's last visible key are masked; skip if all are
        if (s.causal && k0 > wave_last_q + off) continue;
        const char *Kb = Ks[buf], *Vb = Vs[buf];

        f32x4 st[4][QS];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
#pragma unroll
            for (int qs = 0; qs < QS; ++qs) st[ks][qs] = f32x4{0, 0, 0, 0};
#pragma unroll
        for (int ds = 0; ds < DS; ++ds)
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const bf16x8 kf = frag_row(Kb, 16 * ks + c16, 32 * ds + 8 * g);
#pragma unroll
                for (int qs = 0; qs < QS; ++qs) st[ks][qs] = mfma16x16x32(kf, qf[qs][ds], st[ks][qs]);
            }
        const bool edge = (s.causal && k0 + FBN - 1 > qw0 + off) || k0 + FBN > s.n_kv;
        bf16x8 pf[QS][2];
#pragma unroll
        for (int qs = 0; qs < QS; ++qs) {
            const int qa = qw0 + 16 * qs + c16;
            float mt = -INFINITY;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    float x = st[ks][qs][r] * c2;
                    if (edge) {
                        const int ka = k0 + 16 * ks + 4 * g + r;
                        if (ka >= s.n_kv || (s.causal && ka > qa + off)) x = -INFINITY;
                    }
                    st[ks][qs][r] = x;
                    mt = fmaxf(mt, x);
                }
            mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
            mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
            const float mn = fmaxf(m[qs], mt);
            const float so = (m[qs] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m[qs] - mn);
            float lt = 0.f;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float x = st[ks][qs][r];
                    const float pv = (x == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(x - mn);
                    st[ks][qs][r] = pv;
                    lt += pv;
                }
            lt += __shfl_xor(lt, 16, 64);
            lt += __shfl_xor(lt, 32, 64);
            l[qs] = l[qs] * so + lt;
            m[qs] = mn;
#pragma unroll
            for (int i = 0; i < DSUB; ++i) oacc[i][qs] *= so;
            pf[qs][0] = frag_acc(st[0][qs], st[1][qs]);
            pf[qs][1] = frag_acc(st[2][qs], st[3][qs]);
        }
#pragma unroll
        for (int kst = 0; kst < 2; ++kst)
#pragma unroll
            for (int i = 0; i < DSUB; ++i) {
                const bf16x8 vf = frag_t(Vb, 16 * i, 32 * kst, g, c16);
#pragma unroll
                for (int qs = 0; qs < QS; ++qs) oacc[i][qs] = mfma16x16x32(vf, pf[qs][kst], oacc[i][qs]);
            }
    }
#pragma unroll
    for (int qs = 0; qs < QS; ++qs) {
        const int qa = qw0 + 16 * qs + c16;
        if (qa >= s.n_q) continue;
        const float inv = l[qs] > 0.f ? 1.0f / l[qs] : 0.f;
        float *orow = o + ((long)b * s.n_q + qa) * ldo + h * HD;
#pragma unroll
        for (int i = 0; i < DSUB; ++i) {
            const f32x4 a = oacc[i][qs];
            const float4 ov = make_float4(a[0] * inv, a[1] * inv, a[2] * inv, a[3] * inv);
            if (o) *reinterpret_cast<float4 *>(orow + 16 * i + 4 * g) = ov;
            if (ob) {
                bf16x4 bv;
                bv[0] = (bf16)ov.x; bv[1] = (bf16)ov.y; bv[2] = (bf16)ov.z; bv[3] = (bf16)ov.w;
                *reinterpret_cast<bf16x4 *>(ob + ((long)b * s.n_q + qa) * ldob + h * HD + 16 * i + 4 * g) = bv;
            }
        }
        if (lse && g == 0)
            lse[((long)b * s.n_q + qa) * s.n_heads + h] =
                l[qs] > 0.f ? (m[qs] + log2f(l[qs])) * LN2 : -INFINITY;
    }
}

// dQ[q, :] = inv_sqrt_dim * sum_{k visible} dS[q, k] K[k, :]: one 128 x HD
// output tile per (q tile, head, sequence) on the GEMM tile routine (A = dS
// from its transposed [k][q] store, B = K rows; both MN-major).
template <int HD, int BMQ = 128, int WGM = 2, int WGN = 2>
__global__ __launch_bounds__(WGM * WGN * 64, 1) void fa_dq_gemm_k(AttnShape s, AttnPtrs p,
                                                                  const bf16 *dsw) {
    using Cfg = Tile16<BMQ, HD, WGM, WGN>;
    constexpr int TM = BMQ / WGM / 16, TN = HD / WGN / 16;
    __shared__ __attribute__((aligned(16))) char smem[Cfg::LDS];
    const int qt = s.causal ? (int)gridDim.y - 1 - (int)blockIdx.y : (int)blockIdx.y;
    const int h = blockIdx.x % s.n_heads, b = blockIdx.x / s.n_heads;
    const int kvh = h / (s.n_heads / s.n_kv_heads);
    const int q0 = qt * BMQ;
    const int off = s.n_kv - s.n_q;
    const int kend = s.causal ? min(s.n_kv, q0 + BMQ + off) : s.n_kv;
    // A(q, k) = dS^T[k][q]: MN-major
    const Op16 a{dsw + ((long)b * s.n_heads + h) * s.n_q * s.n_kv, s.n_q,
                 (unsigned)((size_t)s.n_q * s.n_kv * 2)};
    const Op16 bk{(const bf16 *)p.k + (long)b * s.n_kv * p.ldk + kvh * HD, p.ldk,
                  (unsigned)(((size_t)(s.n_kv - 1) * p.ldk + HD) * 2)};
    f32x4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    gemm16_tile_dma<Cfg, Lay::MN, Lay::MN, TM, TN>(a, bk, q0, 0, s.n_q, HD, 0, (kend + 63) / 64, kend,
                                              acc, smem);
    const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
    const int row0 = q0 + (wave / WGN) * (BMQ / WGM), col0 = (wave % WGN) * (HD / WGN);
    const float sc_ = s.inv_sqrt_dim;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int q = row0 + 16 * i + 4 * (lane / 16) + r;
            if (q >= s.n_q) continue;
            float *dqr = p.dq + ((long)b * s.n_q + q) * p.lddq + h * HD;
#pragma unroll
            for (int j = 0; j < TN; ++j) dqr[col0 + 16 * j + lane % 16] = acc[i][j][r] * sc_;
        }
}

// ── fp32 path: one wave per row ──────────────────────────────────────

constexpr int MAXE = 4;  // head_dim <= 256

VKH_DEV float dot_wave(const float (&a)[MAXE], const float (&b)[MAXE]) {
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < MAXE; ++i) acc += a[i] * b[i];
    return wave_sum(acc);
}

VKH_DEV void load_row(float (&x)[MAXE], const float *p, int hd, int lane) {
#pragma unroll
    for (int i = 0; i < MAXE; ++i) {
        const int e = lane + 64 * i;
        x[i] = e < hd ? p[e] : 0.f;
    }
}

// fa_forward.comp: wave per (query, head)
__global__ void fa_fwd_f32_k(AttnShape s, const float *q, long ldq, const float *k, long ldk,
                             const float *v, long ldv, float *o, long ldo, float *lse) {
    const int lane = threadIdx.x % 64;
    const long row = (long)blockIdx.x * (NT / 64) + threadIdx.x / 64;
    const long rows = (long)s.n_batch * s.n_q * s.n_heads;
    if (row >= rows) return;
    const int h = (int)(row % s.n_heads);
    const long t = row / s.n_heads;
    const int b = (int)(t / s.n_q), qi = (int)(t % s.n_q);
    const int kvh = h / (s.n_heads / s.n_kv_heads), hd = s.head_dim;
    float qr[MAXE], orow[MAXE] = {0, 0, 0, 0};
    load_row(qr, q + t * ldq + h * hd, hd, lane);
    const int klim = s.causal ? min(s.n_kv - 1, qi + s.n_kv - s.n_q) : s.n_kv - 1;
    float m = -INFINITY, l = 0.f;
    for (int kk = 0; kk <= klim; ++kk) {
        const long kt = (long)b * s.n_kv + kk;
        float kr[MAXE], vr[MAXE];
        load_row(kr, k + kt * ldk + kvh * hd, hd, lane);
        const float sc = dot_wave(qr, kr) * s.inv_sqrt_dim;
        const float mn = fmaxf(m, sc);
        const float so = m == -INFINITY ? 0.f : expf(m - mn);
        const float pv = expf(sc - mn);
        load_row(vr, v + kt * ldv + kvh * hd, hd, lane);
#pragma unroll
        for (int i = 0; i < MAXE; ++i) orow[i] = orow[i] * so + pv * vr[i];
        l = l * so + pv;
        m = mn;
    }
    const float inv = l > 0.f ? 1.0f / l : 0.f;
#pragma unroll
    for (int i = 0; i < MAXE; ++i) {
        const int e = lane + 64 * i;
        if (e < hd) o[t * ldo + h * hd + e] = orow[i] * inv;
    }
    if (lse && lane == 0) lse[t * s.n_heads + h] = l > 0.f ? m + logf(l) : -INFINITY;
}

// fa_bw_dq.comp: wave per (query, head)
__global__ void fa_bwd_dq_f32_k(AttnShape s, AttnPtrs p) {
    const int lane = threadIdx.x % 64;
    const long row = (long)blockIdx.x * (NT / 64) + threadIdx.x / 64;
    const long rows = (long)s.n_batch * s.n_q * s.n_heads;
    if (row >= rows) return;
    const int h = (int)(row % s.n_heads);
    const long t = row / s.n_heads;
    const int b = (int)(t / s.n_q), qi = (int)(t % s.n_q);
    const int kvh = h / (s.n_heads / s.n_kv_heads), hd = s.head_dim;
    const float *Q = (const float *)p.q, *K = (const float *)p.k, *V = (const float *)p.v,
                *dO = (const float *)p.dout;
    float qr[MAXE], dor[MAXE], acc[MAXE] = {0, 0, 0, 0};
    const float lq = p.lse[t * s.n_heads + h], dd = p.d[t * s.n_heads + h];
    if (lq != -INFINITY) {
        load_row(qr, Q + t * p.ldq + h * hd, hd, lane);
        load_row(dor, dO + t * p.lddo + h * hd, hd, lane);
        const int klim = s.causal ? min(s.n_kv - 1, qi + s.n_kv - s.n_q) : s.n_kv - 1;
        for (int kk = 0; kk <= klim; ++kk) {
            const long kt = (long)b * s.n_kv + kk;
            float kr[MAXE], vr[MAXE];
            load_row(kr, K + kt * p.ldk + kvh * hd, hd, lane);
            load_row(vr, V + kt * p.ldv + kvh * hd, hd, lane);
            const float pv = expf(dot_wave(qr, kr) * s.inv_sqrt_dim - lq);
            const float ds = pv * (dot_wave(dor, vr) - dd) * s.inv_sqrt_dim;
#pragma unroll
            for (int i = 0; i < MAXE; ++i) acc[i] += ds * kr[i];
        }
    }
#pragma unroll
    for (int i = 0; i < MAXE; ++i) {
        const int e = lane + 64 * i;
        if (e < hd) p.dq[t * p.lddq + h * hd + e] = acc[i];
    }
}

// fa_bw_dkv.comp: wave per (key, kv head), GQA fold inside
__global__ void fa_bwd_dkv_f32_k(AttnShape s, AttnPtrs p) {
    const int lane = threadIdx.x % 64;
    const long row = (long)blockIdx.x * (NT / 64) + threadIdx.x / 64;
    const long rows = (long)s.n_batch * s.n_kv * s.n_kv_heads;
    if (row >= rows) return;
    const int kvh = (int)(row % s.n_kv_heads);
    const long t = row / s.n_kv_heads;
    const int b = (int)(t / s.n_kv), ki = (int)(t % s.n_kv);
    const int hpk = s.n_heads / s.n_kv_heads, hd = s.head_dim;
    const float *Q = (const float *)p.q, *K = (const float *)p.k, *V = (const float *)p.v,
                *dO = (const float *)p.dout;
    float kr[MAXE], vr[MAXE], dk[MAXE] = {0, 0, 0, 0}, dv[MAXE] = {0, 0, 0, 0};
    load_row(kr, K + t * p.ldk + kvh * hd, hd, lane);
    load_row(vr, V + t * p.ldv + kvh * hd, hd, lane);
    const int off = s.n_kv - s.n_q;
    const int qmin = s.causal ? max(0, ki - off) : 0;
    for (int hh = 0; hh < hpk; ++hh) {
        const int h = kvh * hpk + hh;
        for (int qi = qmin; qi < s.n_q; ++qi) {
            const long qt = (long)b * s.n_q + qi;
            const float lq = p.lse[qt * s.n_heads + h];
            if (lq == -INFINITY) continue;
            float qr[MAXE], dor[MAXE];
            load_row(qr, Q + qt * p.ldq + h * hd, hd, lane);
            load_row(dor, dO + qt * p.lddo + h * hd, hd, lane);
            const float pv = expf(dot_wave(qr, kr) * s.inv_sqrt_dim - lq);
            const float ds = pv * (dot_wave(dor, vr) - p.d[qt * s.n_heads + h]) * s.inv_sqrt_dim;
#pragma unroll
            for (int i = 0; i < MAXE; ++i) {
                dv[i] += pv * dor[i];
                dk[i] += ds * qr[i];
            }
        }
    }
#pragma unroll
    for (int i = 0; i < MAXE; ++i) {
        const int e = lane + 64 * i;
        if (e < hd) {
            p.dk[t * p.lddk + kvh * hd + e] = dk[i];
            p.dv[t * p.lddv + kvh * hd + e] = dv[i];
        }
    }
}

bool bf16_ok(const AttnShape &s) { return s.head_dim == 64 || s.head_dim == 128; }

inline unsigned rows_grid(long rows) { return (unsigned)((rows + (NT / 64) - 1) / (NT / 64)); }

}  // namespace

hipError_t fa_forward(const AttnShape &s, const void *q, long ldq, const void *k, long ldk,
                      const void *v, long ldv, float *o, long ldo, float *lse, DType dt,
                      bf16 *ob, long ldob, hipStream_t st) {
    if (s.n_batch <= 0 || s.n_q <= 0) return hipSuccess;
    if (s.n_kv_heads <= 0 || s.n_heads % s.n_kv_heads) return hipErrorInvalidValue;
    if (dt == DType::BF16) {
        if (!bf16_ok(s)) return hipErrorInvalidValue;
        if (ob && (ldob % 4 || ((uintptr_t)ob & 7u))) return hipErrorInvalidValue;
        dim3 grid(s.n_heads * s.n_batch, (s.n_q + 127) / 128);
        const bool dma_ok = ((uintptr_t)k & 15) == 0 && ((uintptr_t)v & 15) == 0 && ldk % 8 == 0 &&
                            ldv % 8 == 0 && (long)s.n_kv * std::max(ldk, ldv) * 2 < (1L << 31);
        // grids of 128-query blocks that leave the CUs one block each or fewer
        // (short sequences: config 3's 256) take 64-query blocks, two per CU
        const bool q64 = (long)grid.x * grid.y <= cu_count();
        if (s.head_dim == 128 && dma_ok && q64)
            hipLaunchKernelGGL(fa_fwd3_k<1>, dim3(grid.x, (s.n_q + 63) / 64), dim3(NT), 0, st, s,
                               (const bf16 *)q, ldq, (const bf16 *)k, ldk, (const bf16 *)v, ldv, o,
                               ldo, lse, ob, ldob);
        else if (s.head_dim == 128 && dma_ok)
            hipLaunchKernelGGL(fa_fwd3_k<2>, grid, dim3(NT), 0, st, s, (const bf16 *)q, ldq,
                               (const bf16 *)k, ldk, (const bf16 *)v, ldv, o, ldo, lse, ob, ldob);
        else if (s.head_dim == 128)
            hipLaunchKernelGGL(fa_fwd_bf16_k<128>, grid, dim3(NT), 0, st, s, (const bf16 *)q, ldq,
                               (const bf16 *)k, ldk, (const bf16 *)v, ldv, o, ldo, lse, ob, ldob);
        else
            hipLaunchKernelGGL(fa_fwd_bf16_k<64>, grid, dim3(NT), 0, st, s, (const bf16 *)q, ldq,
                               (const bf16 *)k, ldk, (const bf16 *)v, ldv, o, ldo, lse, ob, ldob);
    } else {
        if (s.head_dim > 64 * MAXE || ob) return hipErrorInvalidValue;
        if (fa_f32m_fwd(s, (const float *)q, ldq, (const float *)k, ldk, (const float *)v, ldv, o,
                        ldo, lse, st))
            return hipGetLastError();
        hipLaunchKernelGGL(fa_fwd_f32_k, dim3(rows_grid((long)s.n_batch * s.n_q * s.n_heads)),
                           dim3(NT), 0, st, s, (const float *)q, ldq, (const float *)k, ldk,
                           (const float *)v, ldv, o, ldo, lse);
    }
    return hipGetLastError();
}

hipError_t fa_bw_d(const AttnShape &s, const float *o, long ldo, const float *dout, long lddo,
                   float *d, bf16 *dout_bf16, long lddo16, hipStream_t st) {
    const long rows = (long)s.n_batch * s.n_q * s.n_heads;
    if (rows <= 0) return hipSuccess;
    const bool al = ((uintptr_t)o & 15) == 0 && ((uintptr_t)dout & 15) == 0 && ldo % 4 == 0 &&
                    lddo % 4 == 0 && (!dout_bf16 || (((uintptr_t)dout_bf16 & 15) == 0 && lddo16 % 8 == 0));
    if ((s.head_dim == 128 || s.head_dim == 64) && al) {
        const int lph = s.head_dim / 8, per_block = (NT / 64) * (64 / lph);
        const long grid = std::min<long>(4096, (rows + 2L * per_block - 1) / (2L * per_block));
        if (lph == 16)
            hipLaunchKernelGGL((fa_bw_d8_k<16, float>), dim3((unsigned)grid), dim3(NT), 0, st, s, o,
                               ldo, dout, lddo, d, dout_bf16, lddo16);
        else
            hipLaunchKernelGGL((fa_bw_d8_k<8, float>), dim3((unsigned)grid), dim3(NT), 0, st, s, o,
                               ldo, dout, lddo, d, dout_bf16, lddo16);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(fa_bw_d_k, dim3(rows_grid(rows)), dim3(NT), 0, st, s, o, ldo, dout, lddo, d,
                       dout_bf16, lddo16);
    return hipGetLastError();
}

hipError_t fa_bw_d_bf16(const AttnShape &s, const bf16 *o, long ldo, const bf16 *dout, long lddo,
                        float *d, hipStream_t st) {
    const long rows = (long)s.n_batch * s.n_q * s.n_heads;
    if (rows <= 0) return hipSuccess;
    if ((s.head_dim != 128 && s.head_dim != 64) || ((uintptr_t)o & 15) || ((uintptr_t)dout & 15) ||
        ldo % 8 || lddo % 8)
        return hipErrorInvalidValue;
    const int lph = s.head_dim / 8, per_block = (NT / 64) * (64 / lph);
    const long grid = std::min<long>(4096, (rows + 2L * per_block - 1) / (2L * per_block));
    if (lph == 16)
        hipLaunchKernelGGL((fa_bw_d8_k<16, bf16>), dim3((unsigned)grid), dim3(NT), 0, st, s, o, ldo,
                           dout, lddo, d, (bf16 *)nullptr, 0L);
    else
        hipLaunchKernelGGL((fa_bw_d8_k<8, bf16>), dim3((unsigned)grid), dim3(NT), 0, st, s, o, ldo,
                           dout, lddo, d, (bf16 *)nullptr, 0L);
    return hipGetLastError();
}

hipError_t fa_bw_dq(const AttnShape &s, const AttnPtrs &p, hipStream_t st) {
    if (s.n_batch <= 0 || s.n_q <= 0) return hipSuccess;
    if (s.n_kv_heads <= 0 || s.n_heads % s.n_kv_heads) return hipErrorInvalidValue;
    if (p.dt == DType::BF16) {
        if (!bf16_ok(s)) return hipErrorInvalidValue;
        dim3 grid(s.n_heads * s.n_batch, (s.n_q + 127) / 128);
        if (s.head_dim == 128)
            hipLaunchKernelGGL(fa_bwd_dq_bf16_k<128>, grid, dim3(NT), 0, st, s, p);
        else
            hipLaunchKernelGGL(fa_bwd_dq_bf16_k<64>, grid, dim3(NT), 0, st, s, p);
    } else {
        if (s.head_dim > 64 * MAXE) return hipErrorInvalidValue;
        if (fa_f32m_dq(s, p, st)) return hipGetLastError();
        if (p.qk_fp32) return hipErrorInvalidValue;  // the fused epilogue has no per-row form
        hipLaunchKernelGGL(fa_bwd_dq_f32_k, dim3(rows_grid((long)s.n_batch * s.n_q * s.n_heads)),
                           dim3(NT), 0, st, s, p);
    }
    return hipGetLastError();
}

#ifndef FA_BM
#define FA_BM 64
#endif

bool fa_bw_fused_ok(const AttnShape &s) {
    return bf16_ok(s) && s.n_q % 64 == 0 && s.n_kv % 64 == 0 && (!s.causal || s.n_q == s.n_kv) &&
           (size_t)s.n_q * s.n_kv * 2 < (1ull << 31) && s.n_kv_heads > 0 &&
           s.n_heads % s.n_kv_heads == 0;
}

// The recompute kernels (fa_bwd_dkv4_k + fa_bwd_dq4_k): head_dim 128, an even
// number of query heads per KV head, 128-key blocks; no dS workspace.
bool fa_bw_v4_ok(const AttnShape &s) {
    return fa_bw_fused_ok(s) && s.head_dim == 128 && (s.n_heads / s.n_kv_heads) % 2 == 0 &&
           s.n_kv % 128 == 0;
}

// They pay off once the dK/dV grid gives every CU a block (>= 128 blocks of 8
// waves: the training step's B = 4 x 512 keys x 8 KV heads measured 22.16 ms
// against 22.37 ms on the dS-GEMM path; config 2's 512 blocks 0.266 against
// 0.327 ms); below that the two-kernel dS path keeps more blocks in flight.
bool fa_bw_v4_preferred(const AttnShape &s) {
    return fa_bw_v4_ok(s) && (long)s.n_batch * s.n_kv_heads * (s.n_kv / 128) >= 128;
}

// The dK/dV recompute kernel with the head-group size as a constant where it
// is one of the common ones.
template <int W, bool QKE>
void launch_dkv4(const AttnShape &s, const AttnPtrs &p, hipStream_t st) {
    const int nh = s.n_heads / s.n_kv_heads / 2;
    if (p.split_ws && fa_bw_v4_split(s)) {
        // two blocks per (sequence, KV head, key block), then their sum and the epilogue
        const dim3 gkv(s.n_kv_heads * s.n_batch, s.n_kv / dkv4::BN, 2);
        if (nh == 2) hipLaunchKernelGGL((fa_bwd_dkv4_k<W, false, 2, 2>), gkv, dim3(W * 64), 0, st, s, p);
        else hipLaunchKernelGGL((fa_bwd_dkv4_k<W, false, 0, 2>), gkv, dim3(W * 64), 0, st, s, p);
        const dim3 gc((unsigned)(((long)s.n_batch * s.n_kv + 63) / 64), s.n_kv_heads);
        hipLaunchKernelGGL(fa_dkv_combine_k<QKE>, gc, dim3(256), 0, st, s, p);
        return;
    }
    const dim3 gkv(s.n_kv_heads * s.n_batch, s.n_kv / dkv4::BN);
    if (nh == 1) hipLaunchKernelGGL((fa_bwd_dkv4_k<W, QKE, 1>), gkv, dim3(W * 64), 0, st, s, p);
    else if (nh == 2) hipLaunchKernelGGL((fa_bwd_dkv4_k<W, QKE, 2>), gkv, dim3(W * 64), 0, st, s, p);
    else hipLaunchKernelGGL((fa_bwd_dkv4_k<W, QKE, 0>), gkv, dim3(W * 64), 0, st, s, p);
}

// dQ blocks of 256 queries, or of 128 where 256 would leave fewer blocks than
// CUs: there a causal grid is also short of work at its end, since a block's
// work grows with its last query (config 3, 4 x 512: 128 blocks of 256 rows,
// the later block of each sequence twice the earlier); with 256-query blocks
// filling the chip, 128 loses (config 2: 0.268 against 0.250 ms per call)
int dq4_bq(const AttnShape &s) {
    const long b256 = (long)s.n_heads * s.n_batch * ((s.n_q + 255) / 256);
    return b256 < 256 ? 128 : 256;
}
template <bool WITH_D, bool QKE>
void launch_dq4(const AttnShape &s, const AttnPtrs &p, hipStream_t st) {
    constexpr int W = 8;
    const int bq = dq4_bq(s);
    const dim3 gq(s.n_heads * s.n_batch, (s.n_q + bq - 1) / bq);
    if (bq == 128)
        hipLaunchKernelGGL((fa_bwd_dq4_k<W, WITH_D, QKE, 128>), gq, dim3(W * 64), 0, st, s, p);
    else
        hipLaunchKernelGGL((fa_bwd_dq4_k<W, WITH_D, QKE, 256>), gq, dim3(W * 64), 0, st, s, p);
}

// One of the two recompute kernels alone (D already in p.d): which = 0 the
// dK/dV kernel, 1 the dQ kernel, so a caller can run them on two streams.
hipError_t fa_bw_v4_part(const AttnShape &s, const AttnPtrs &p, int which, hipStream_t st) {
    if (s.n_batch <= 0 || s.n_q <= 0) return hipSuccess;
    if (p.dt != DType::BF16 || !fa_bw_v4_ok(s) || p.o16) return hipErrorInvalidValue;
    if ((long)s.n_q * std::max(p.ldq, p.lddo) * 2 >= (1l << 31) ||
        (long)s.n_kv * std::max(p.ldk, p.ldv) * 2 >= (1l << 31))
        return hipErrorInvalidValue;
    const QkEpi &e = p.qk;
    if (e.out && (!fa_bw_qk_epi_ok(s, e.rot) || !e.x || e.ldout % 8 || e.ldx % 4 ||
                  ((uintptr_t)e.out & 15) || ((uintptr_t)e.x & 15) || (e.rot && !e.rope) ||
                  (bool)e.gq != (bool)e.gk || (e.gq && (!e.pq || !e.pk))))
        return hipErrorInvalidValue;
    constexpr int W = 8;
    if (which == 0) {
        if (e.out) launch_dkv4<W, true>(s, p, st);
        else launch_dkv4<W, false>(s, p, st);
    } else {
        if (e.out) launch_dq4<false, true>(s, p, st);
        else launch_dq4<false, false>(s, p, st);
    }
    return hipGetLastError();
}

int fa_bw_v4_q_blocks(const AttnShape &s) {
    const int bq = dq4_bq(s);
    return s.n_heads * s.n_batch * ((s.n_q + bq - 1) / bq);
}
int fa_bw_v4_q_rows(const AttnShape &s) { return dq4_bq(s); }
int fa_bw_v4_kv_blocks(const AttnShape &s) { return s.n_kv_heads * s.n_batch * (s.n_kv / dkv4::BN); }
// The split dK/dV launch: where the (sequence, KV head, key block) grid has
// fewer blocks than CUs and each head group holds an even number of query
// heads to divide (config 4: 128 blocks of 4-head groups at 1 x 2048 -> 256).
bool fa_bw_v4_split(const AttnShape &s) {
    return fa_bw_v4_ok(s) && (s.n_heads / s.n_kv_heads / 2) % 2 == 0 && fa_bw_v4_kv_blocks(s) < 256;
}
size_t fa_bw_v4_split_ws_floats(const AttnShape &s) {
    return fa_bw_v4_split(s) ? (size_t)4 * s.n_batch * s.n_kv * s.n_kv_heads * dkv4::HD : 0;
}
int fa_bw_v4_kv_launch_blocks(const AttnShape &s, bool split) {
    return split && fa_bw_v4_split(s) ? 2 * fa_bw_v4_kv_blocks(s) : fa_bw_v4_kv_blocks(s);
}
int fa_bw_v4_k_gain_parts(const AttnShape &s, bool split) {
    if (split && fa_bw_v4_split(s))
        return (int)(((long)s.n_batch * s.n_kv + 63) / 64) * s.n_kv_heads;
    return fa_bw_v4_kv_blocks(s);
}
// The epilogue's row layout assumes head_dim 128 and a rotary span of 0 or
// the whole head (pairs 64 apart).
bool fa_bw_qk_epi_ok(const AttnShape &s, int rotary_dim) {
    return fa_bw_v4_ok(s) && (rotary_dim == 0 || rotary_dim == s.head_dim);
}

size_t fa_bw_ws_bytes(const AttnShape &s, bool v4) {
    if (v4) return 0;
    return (size_t)s.n_batch * s.n_heads * s.n_q * s.n_kv * sizeof(bf16);
}

hipError_t fa_bw_fused(const AttnShape &s, const AttnPtrs &p, bf16 *ds_ws, bool v4, hipStream_t st) {
    if (s.n_batch <= 0 || s.n_q <= 0) return hipSuccess;
    if (p.dt != DType::BF16 || !fa_bw_fused_ok(s) || (v4 && !fa_bw_v4_ok(s)))
        return hipErrorInvalidValue;
    if (v4) {
        // the DMA offsets are 32-bit: rows of the q / k / v / dO views must fit
        if ((long)s.n_q * std::max(p.ldq, p.lddo) * 2 >= (1l << 31) ||
            (long)s.n_kv * std::max(p.ldk, p.ldv) * 2 >= (1l << 31))
            return hipErrorInvalidValue;
        if (p.o16 && (long)s.n_q * p.ldo16 * 2 >= (1l << 31)) return hipErrorInvalidValue;
        constexpr int DKV_WAVES = 8;
        const QkEpi &e = p.qk;
        if (e.out) {
            // fused q/k epilogue: dQ forms D (needs bf16 O), then dK/dV
            if (!p.o16 || !fa_bw_qk_epi_ok(s, e.rot) || !e.x || e.ldout % 8 || e.ldx % 4 ||
                ((uintptr_t)e.out & 15) || ((uintptr_t)e.x & 15) || (e.rot && !e.rope) ||
                (bool)e.gq != (bool)e.gk || (e.gq && (!e.pq || !e.pk)))
                return hipErrorInvalidValue;
            launch_dq4<true, true>(s, p, st);
            launch_dkv4<DKV_WAVES, true>(s, p, st);
        } else if (p.o16) {  // dQ forms D, then dK/dV reads it
            launch_dq4<true, false>(s, p, st);
            launch_dkv4<DKV_WAVES, false>(s, p, st);
        } else {
            launch_dkv4<DKV_WAVES, false>(s, p, st);
            launch_dq4<false, false>(s, p, st);
        }
        return hipGetLastError();
    }
    if (!ds_ws) return hipErrorInvalidValue;
    dim3 gkv(s.n_kv_heads * s.n_batch, (s.n_kv + 127) / 128);
    dim3 gq(s.n_heads * s.n_batch, (s.n_q + 127) / 128);
    if (s.head_dim == 128) {
        hipLaunchKernelGGL(fa_bwd_dkv3_k, gkv, dim3(dkv3::NT3), 0, st, s, p, ds_ws);
        constexpr int DQ_BM = 128, DQ_WGM = 2, DQ_WGN = 2;
        const dim3 gq2(s.n_heads * s.n_batch, (s.n_q + DQ_BM - 1) / DQ_BM);
        hipLaunchKernelGGL((fa_dq_gemm_k<128, DQ_BM, DQ_WGM, DQ_WGN>), gq2,
                           dim3(DQ_WGM * DQ_WGN * 64), 0, st, s, p, (const bf16 *)ds_ws);
    } else {
        hipLaunchKernelGGL((fa_bwd_dkv2_k<64, FA_BM>), gkv, dim3(NT), 0, st, s, p, ds_ws);
        hipLaunchKernelGGL(fa_dq_gemm_k<64>, gq, dim3(NT), 0, st, s, p, (const bf16 *)ds_ws);
    }
    return hipGetLastError();
}

hipError_t fa_bw_dkv(const AttnShape &s, const AttnPtrs &p, hipStream_t st) {
    if (s.n_batch <= 0 || s.n_kv <= 0) return hipSuccess;
    if (s.n_kv_heads <= 0 || s.n_heads % s.n_kv_heads) return hipErrorInvalidValue;
    if (p.dt == DType::BF16) {
        if (!bf16_ok(s)) return hipErrorInvalidValue;
        dim3 grid(s.n_kv_heads * s.n_batch, (s.n_kv + 127) / 128);
        if (s.head_dim == 128)
            hipLaunchKernelGGL(fa_bwd_dkv_bf16_k<128>, grid, dim3(NT), 0, st, s, p);
        else
            hipLaunchKernelGGL(fa_bwd_dkv_bf16_k<64>, grid, dim3(NT), 0, st, s, p);
    } else {
        if (s.head_dim > 64 * MAXE) return hipErrorInvalidValue;
        if (fa_f32m_dkv(s, p, st)) return hipGetLastError();
        if (p.qk_fp32) return hipErrorInvalidValue;  // the fused epilogue has no per-row form
        hipLaunchKernelGGL(fa_bwd_dkv_f32_k,
                           dim3(rows_grid((long)s.n_batch * s.n_kv * s.n_kv_heads)), dim3(NT), 0,
                           st, s, p);
    }
    return hipGetLastError();
}

}  // namespace vkh
