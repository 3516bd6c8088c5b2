// MFMA GEMM for gfx950:  C[m, n] = sum_k A(m, k) * B(n, k)   (then an epilogue)
//
// One template covers the three contractions of a linear layer
// (reference: shaders/matmul_nt_v2.comp, linear_backward_dx_batched.comp,
// linear_backward_dw_batched.comp) by describing each operand's storage:
//
//   Lay::K   element (r, k) at p[r * ld + k]   (k contiguous)
//   Lay::MN  element (r, k) at p[k * ld + r]   (r contiguous)
//
//   forward  y  = x W^T :  A = x  (K),  B = W  (K)
//   dx       dx = dy W  :  A = dy (K),  B = W  (MN)
//   dW       dW = dy^T x:  A = dy (MN), B = x  (MN)
//
// Tiles are staged global -> registers -> LDS with the conversion to the
// compute type (bf16 or fp32) done in registers, so fp32 activations and
// weights never need a separate cast pass.  LDS rows are k-contiguous so
// each lane's MFMA operand is one 16-byte ds_read; operands stored MN-major
// in HBM are transposed in registers on their way into LDS.
//
// Compute types:
//   bf16: v_mfma_f32_16x16x32_bf16, fp32 accumulate
//   fp32: v_mfma_f32_16x16x4_f32,   fp32 accumulate (exact products)
//
// 256 threads = 4 waves arranged 2 x 2; each wave owns a (BM/2) x (BN/2)
// sub-tile made of 16x16 MFMA accumulators.  The block -> tile map is
// XCD-aware: consecutive hardware workgroup ids land on different XCDs, so
// ids are regrouped to give each XCD a contiguous band of tiles (shared
// operand panels stay in that XCD's L2).
#pragma once

#include "common.hpp"

namespace vkh {

enum class Lay { K, MN };

struct GemmOperand {
    const void *p;
    long ld;
    bool vec;  // pointer and ld allow vector loads (16 B fp32 / 16 B bf16 K, 8 B bf16 MN)
};

struct GemmShape {
    int M, N, K;
};

template <bool BF16>
struct Prec;
template <>
struct Prec<true> {
    using T = bf16;
    static constexpr int V = 8;      // k values per lane per MFMA operand
    static constexpr int KSTEP = 32;  // k per MFMA
};
template <>
struct Prec<false> {
    using T = float;
    static constexpr int V = 4;
    static constexpr int KSTEP = 16;  // 4 MFMAs of k=4 consume one float4 per lane
};

VKH_DEV float ld1(const float *p) { return *p; }
VKH_DEV float ld1(const bf16 *p) { return (float)*p; }

// Load V consecutive elements (fp32 registers) from p; vector path when legal.
template <typename TS, int V>
VKH_DEV void load_vec(float (&r)[V], const TS *p, bool full_vec) {
    if constexpr (sizeof(TS) == 4) {
        if (full_vec) {
#pragma unroll
            for (int i = 0; i < V; i += 4) {
                float4 t = *reinterpret_cast<const float4 *>(p + i);
                r[i] = t.x; r[i + 1] = t.y; r[i + 2] = t.z; r[i + 3] = t.w;
            }
            return;
        }
    } else {
        if (full_vec) {
            if constexpr (V == 8) {
                bf16x8 t = *reinterpret_cast<const bf16x8 *>(p);
#pragma unroll
                for (int i = 0; i < 8; ++i) r[i] = (float)t[i];
            } else {
                bf16x4 t = *reinterpret_cast<const bf16x4 *>(p);
#pragma unroll
                for (int i = 0; i < 4; ++i) r[i] = (float)t[i];
            }
            return;
        }
    }
#pragma unroll
    for (int i = 0; i < V; ++i) r[i] = ld1(p + i);
}

// Loads an R x BK operand tile into LDS[R][BK + PAD] (k contiguous).
template <typename TS, Lay L, bool BF16, int R, int BK, int NT>
struct TileLoader {
    using CT = typename Prec<BF16>::T;
    static constexpr int V = Prec<BF16>::V;
    static constexpr int UNITS = (L == Lay::K) ? R * (BK / V) : (BK / V) * (R / 4);
    static constexpr int PER_T = (UNITS + NT - 1) / NT;
    static constexpr int NREG = (L == Lay::K) ? V : V * 4;
    float r[PER_T][NREG];

    // rows [row0, row0 + R) of the operand, k in [k0, k0 + BK)
    VKH_DEV void load(const GemmOperand &op, int row0, int rmax, int k0, int kmax, int tid) {
        const TS *base = reinterpret_cast<const TS *>(op.p);
#pragma unroll
        for (int p = 0; p < PER_T; ++p) {
            const int u = tid + p * NT;
            if (UNITS % NT != 0 && u >= UNITS) break;
            if constexpr (L == Lay::K) {
                const int row = u / (BK / V), kv = u % (BK / V);
                const int gr = row0 + row, gk = k0 + kv * V;
                float(&v)[V] = *reinterpret_cast<float(*)[V]>(&r[p][0]);
                if (gr < rmax && gk + V <= kmax) {
                    load_vec<TS, V>(v, base + (long)gr * op.ld + gk, op.vec);
                } else {
#pragma unroll
                    for (int i = 0; i < V; ++i)
                        v[i] = (gr < rmax && gk + i < kmax) ? ld1(base + (long)gr * op.ld + gk + i) : 0.f;
                }
            } else {
                const int kv = u / (R / 4), r4 = u % (R / 4);
                const int gr = row0 + r4 * 4, gk = k0 + kv * V;
#pragma unroll
                for (int kk = 0; kk < V; ++kk) {
                    float(&v)[4] = *reinterpret_cast<float(*)[4]>(&r[p][kk * 4]);
                    const int k = gk + kk;
                    if (k < kmax && gr + 4 <= rmax) {
                        load_vec<TS, 4>(v, base + (long)k * op.ld + gr, op.vec);
                    } else {
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            v[i] = (k < kmax && gr + i < rmax) ? ld1(base + (long)k * op.ld + gr + i) : 0.f;
                    }
                }
            }
        }
    }

    template <int LDW>
    VKH_DEV void store(CT (*lds)[LDW], int tid) {
#pragma unroll
        for (int p = 0; p < PER_T; ++p) {
            const int u = tid + p * NT;
            if (UNITS % NT != 0 && u >= UNITS) break;
            if constexpr (L == Lay::K) {
                const int row = u / (BK / V), kv = u % (BK / V);
                if constexpr (BF16) {
                    *reinterpret_cast<bf16x8 *>(&lds[row][kv * V]) =
                        cvt8(r[p][0], r[p][1], r[p][2], r[p][3], r[p][4], r[p][5], r[p][6], r[p][7]);
                } else {
                    *reinterpret_cast<float4 *>(&lds[row][kv * V]) =
                        make_float4(r[p][0], r[p][1], r[p][2], r[p][3]);
                }
            } else {
                const int kv = u / (R / 4), r4 = u % (R / 4);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if constexpr (BF16) {
                        *reinterpret_cast<bf16x8 *>(&lds[r4 * 4 + i][kv * V]) =
                            cvt8(r[p][0 * 4 + i], r[p][1 * 4 + i], r[p][2 * 4 + i], r[p][3 * 4 + i],
                                 r[p][4 * 4 + i], r[p][5 * 4 + i], r[p][6 * 4 + i], r[p][7 * 4 + i]);
                    } else {
                        *reinterpret_cast<float4 *>(&lds[r4 * 4 + i][kv * V]) =
                            make_float4(r[p][0 * 4 + i], r[p][1 * 4 + i], r[p][2 * 4 + i], r[p][3 * 4 + i]);
                    }
                }
            }
        }
    }
};

template <int BM_, int BN_, int BK_>
struct TileCfg {
    static constexpr int BM = BM_, BN = BN_, BK = BK_;
};

// Output tile (bm, bn) of linear tile index t.  Tiles go in groups of `grp`
// tile rows (0: all of them), column by column inside a group, so the blocks
// that run at the same time on one XCD (consecutive t after the XCD
// regrouping) cover a few rows x a few columns of tiles and share operand
// panels in that XCD's L2, instead of one column of tiles that each bring
// their own row panel.  Group height by operand layout, measured on the bf16
// training step (T = 2048: 8 / 2 rows, 20.2 ms against 21.8 in plain column
// order) and the 8192-token step (593 against 618 ms): 8 rows when the A
// operand is K-major (forward, dx), 2 for the weight gradients (both
// operands MN-major).
template <Lay LA, Lay LB>
constexpr int tile_group_rows() {
    return LA == Lay::MN && LB == Lay::MN ? 2 : 8;
}
VKH_DEV void tile_rc(int t, int nbm, int nbn, int grp, int &bm, int &bn) {
    if (grp <= 0 || grp > nbm) grp = nbm;
    const int per = grp * nbn;
    const int g = t / per, r = t - g * per;
    const int gm = min(grp, nbm - g * grp);
    // wave-uniform: kept in scalar registers (the tile loops of the largest
    // kernels have no vector register to spare)
    bm = __builtin_amdgcn_readfirstlane(g * grp + r % gm);
    bn = __builtin_amdgcn_readfirstlane(r / gm);
}

// Fragment coordinates handed to epilogues: accumulator acc[i][j][r] holds
// C[row0 + 16 i + 4 (lane / 16) + r][col0 + 16 j + lane % 16].
struct FragPos {
    int row0, col0, lane;
};

template <class Cfg, bool BF16, typename TA, Lay LA, typename TB, Lay LB, class Epi>
__global__ __launch_bounds__(256, 2) void gemm_kernel(GemmOperand a, GemmOperand b, GemmShape s,
                                                      Epi epi) {
    constexpr int BM = Cfg::BM, BN = Cfg::BN, BK = Cfg::BK;
    constexpr int NT = 256;
    using CT = typename Prec<BF16>::T;
    constexpr int V = Prec<BF16>::V;
    constexpr int KSTEP = Prec<BF16>::KSTEP;
    constexpr int PAD = BF16 ? 8 : 4;
    constexpr int LDW = BK + PAD;
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int TM = WM / 16, TN = WN / 16;

    __shared__ __attribute__((aligned(16))) CT As[2][BM][LDW];
    __shared__ __attribute__((aligned(16))) CT Bs[2][BN][LDW];

    const int tid = threadIdx.x;
    const int lane = tid % 64, wave = tid / 64;
    const int wm = wave / 2, wn = wave % 2;

    const int nbm = (s.M + BM - 1) / BM, nbn = (s.N + BN - 1) / BN;
    const int nb = nbm * nbn;
    int bid = blockIdx.x;
    if (nb % 8 == 0) bid = (bid % 8) * (nb / 8) + bid / 8;
    int bm, bn;
    tile_rc(bid, nbm, nbn, tile_group_rows<LA, LB>(), bm, bn);
    const int m0 = bm * BM, n0 = bn * BN;

    TileLoader<TA, LA, BF16, BM, BK, NT> la;
    TileLoader<TB, LB, BF16, BN, BK, NT> lb;

    f32x4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int nk = (s.K + BK - 1) / BK;
    la.load(a, m0, s.M, 0, s.K, tid);
    lb.load(b, n0, s.N, 0, s.K, tid);
    la.template store<LDW>(As[0], tid);
    lb.template store<LDW>(Bs[0], tid);
    __syncthreads();

    const int fr = lane % 16, fg = lane / 16;
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < nk) {
            la.load(a, m0, s.M, (kt + 1) * BK, s.K, tid);
            lb.load(b, n0, s.N, (kt + 1) * BK, s.K, tid);
        }
#pragma unroll
        for (int ks = 0; ks < BK / KSTEP; ++ks) {
            if constexpr (BF16) {
                bf16x8 af[TM], bfr[TN];
#pragma unroll
                for (int i = 0; i < TM; ++i)
                    af[i] = *reinterpret_cast<const bf16x8 *>(&As[cur][wm * WM + 16 * i + fr][ks * KSTEP + fg * V]);
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    bfr[j] = *reinterpret_cast<const bf16x8 *>(&Bs[cur][wn * WN + 16 * j + fr][ks * KSTEP + fg * V]);
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j) acc[i][j] = mfma16x16x32(af[i], bfr[j], acc[i][j]);
            } else {
                float4 af[TM], bfr[TN];
#pragma unroll
                for (int i = 0; i < TM; ++i)
                    af[i] = *reinterpret_cast<const float4 *>(&As[cur][wm * WM + 16 * i + fr][ks * KSTEP + fg * V]);
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    bfr[j] = *reinterpret_cast<const float4 *>(&Bs[cur][wn * WN + 16 * j + fr][ks * KSTEP + fg * V]);
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j) {
                        acc[i][j] = mfma16x16x4(af[i].x, bfr[j].x, acc[i][j]);
                        acc[i][j] = mfma16x16x4(af[i].y, bfr[j].y, acc[i][j]);
                        acc[i][j] = mfma16x16x4(af[i].z, bfr[j].z, acc[i][j]);
                        acc[i][j] = mfma16x16x4(af[i].w, bfr[j].w, acc[i][j]);
                    }
            }
        }
        if (kt + 1 < nk) {
            la.template store<LDW>(As[cur ^ 1], tid);
            lb.template store<LDW>(Bs[cur ^ 1], tid);
        }
        __syncthreads();
    }

    FragPos fp{m0 + wm * WM, n0 + wn * WN, lane};
    epi.template apply<TM, TN>(acc, fp, s);
}

// ── epilogues ──────────────────────────────────────────────────────────

// C = alpha * acc (+ beta * C_old) (+ R), fp32 row-major.
struct EpiStore {
    float *C;
    long ldc;
    const float *R;  // optional residual, same shape as C
    long ldr;
    float alpha;
    float beta;  // 0 => overwrite (C_old not read)

    template <int TM, int TN>
    VKH_DEV void apply(const f32x4 (&acc)[TM][TN], const FragPos &fp, const GemmShape &s) const {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = fp.row0 + 16 * i + 4 * (fp.lane / 16) + r;
                    const int col = fp.col0 + 16 * j + fp.lane % 16;
                    if (row < s.M && col < s.N) {
                        float v = alpha * acc[i][j][r];
                        float *c = C + (long)row * ldc + col;
                        if (beta != 0.f) v += beta * *c;
                        if (R) v += R[(long)row * ldr + col];
                        *c = v;
                    }
                }
    }
};

// C_bf16 = bf16(alpha * acc)
struct EpiStoreBf16 {
    bf16 *C;
    long ldc;
    float alpha;
    template <int TM, int TN>
    VKH_DEV void apply(const f32x4 (&acc)[TM][TN], const FragPos &fp, const GemmShape &s) const {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = fp.row0 + 16 * i + 4 * (fp.lane / 16) + r;
                    const int col = fp.col0 + 16 * j + fp.lane % 16;
                    if (row < s.M && col < s.N) C[(long)row * ldc + col] = (bf16)(alpha * acc[i][j][r]);
                }
    }
};

// ── host-side launch ───────────────────────────────────────────────────

template <class Cfg, bool BF16, typename TA, Lay LA, typename TB, Lay LB, class Epi>
hipError_t launch_gemm(const GemmOperand &a, const GemmOperand &b, const GemmShape &s,
                       const Epi &epi, hipStream_t st) {
    if (s.M <= 0 || s.N <= 0) return hipSuccess;
    const unsigned nb = ceil_div(s.M, Cfg::BM) * ceil_div(s.N, Cfg::BN);
    hipLaunchKernelGGL((gemm_kernel<Cfg, BF16, TA, LA, TB, LB, Epi>), dim3(nb), dim3(256), 0, st, a,
                       b, s, epi);
    return hipGetLastError();
}

// Tile choice: the largest tile that still gives >= 2 blocks per CU.
enum class Tile { T128x128, T128x64, T64x128, T64x64 };

inline Tile pick_tile(int M, int N) {
    const long target = 512;
    auto nb = [&](int bm, int bn) { return (long)ceil_div(M, bm) * (long)ceil_div(N, bn); };
    if (nb(128, 128) >= target) return Tile::T128x128;
    if (M >= N) {
        if (nb(128, 64) >= target) return Tile::T128x64;
        if (nb(64, 128) >= target) return Tile::T64x128;
    } else {
        if (nb(64, 128) >= target) return Tile::T64x128;
        if (nb(128, 64) >= target) return Tile::T128x64;
    }
    return Tile::T64x64;
}

template <bool BF16, typename TA, Lay LA, typename TB, Lay LB, class Epi>
hipError_t gemm_dispatch(const GemmOperand &a, const GemmOperand &b, const GemmShape &s,
                         const Epi &epi, hipStream_t st) {
    constexpr int BK = BF16 ? 64 : 32;
    switch (pick_tile(s.M, s.N)) {
    case Tile::T128x128:
        return launch_gemm<TileCfg<128, 128, BK>, BF16, TA, LA, TB, LB>(a, b, s, epi, st);
    case Tile::T128x64:
        return launch_gemm<TileCfg<128, 64, BK>, BF16, TA, LA, TB, LB>(a, b, s, epi, st);
    case Tile::T64x128:
        return launch_gemm<TileCfg<64, 128, BK>, BF16, TA, LA, TB, LB>(a, b, s, epi, st);
    default:
        return launch_gemm<TileCfg<64, 64, BK>, BF16, TA, LA, TB, LB>(a, b, s, epi, st);
    }
}

inline bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

// vector-load legality for an operand of element size `es` and layout `L`
inline bool vec_ok(const void *p, long ld, int es, Lay L) {
    if (!aligned16(p)) return false;
    if (es == 4) return ld % 4 == 0;
    return L == Lay::K ? (ld % 8 == 0) : (ld % 4 == 0 && ((uintptr_t)p & 7u) == 0);
}

}  // namespace vkh
