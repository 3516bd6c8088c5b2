// Rank-r LoRA products (train/lora.zig:99-251) for the fused projections of a
// decoder layer.  Each launch serves up to three adapters that share one
// operand (q/k/v read the same normed input, gate/up the same n2, and their
// gradients are column blocks of one fused dy):
//
//   lora_rows    U_s[t, i]  = alpha sum_c X[t, col_s + c] F_s(c, i)
//                forward intermediate x A^T (F = A^T), backward dy B (F = B)
//   lora_cols    G_s(c, i)  = alpha sum_t X[t, col_s + c] U_s[t, i]
//                dA = aor (dy B)^T x,  dB = aor dy^T inter   (overwrite)
//   lora_update  Y[t, col_s + c] += alpha sum_s sum_i U_s[t, i] F_s(c, i)
//                y += aor inter B^T,  dx += aor (dy B) A
//
// The adapter factors, the intermediate and dy B stay fp32; X is the fp32 or
// bf16 activation the base GEMM reads, widened exactly.  Products are fp32
// (v_mfma_f32_16x16x4_f32 for rows / cols, fp32 FMA for the update), sums in
// fp32 in a fixed order (no atomics), so results are deterministic.
//
// Why not the general GEMMs: r = 16 gives an N (or M) of 16, so a 64..256
// wide GEMM tile wastes most of its work, and a split over T = 2048 rows
// leaves a few dozen workgroups.  Here every launch spreads T (rows) or the
// wide dimension (cols) over >= 100 workgroups and reduces inside the block.
#include <algorithm>

#include "ops.hpp"

namespace vkh {
namespace {

// 8 consecutive X values widened to fp32 (16-byte loads).
VKH_DEV void ld8(float (&v)[8], const bf16 *p) {
    const bf16x8 t = *reinterpret_cast<const bf16x8 *>(p);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (float)t[e];
}
VKH_DEV void ld8(float (&v)[8], const float *p) {
    const float4 a = *reinterpret_cast<const float4 *>(p);
    const float4 b = *reinterpret_cast<const float4 *>(p + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

// ── lora_rows ───────────────────────────────────────────────────────────
// Block = 32 rows (two 16-row MFMA tiles) x all r outputs of one adapter
// (blockIdx.y); its 8 waves split the reduction columns in 32-column groups
// and the partial tiles are summed through LDS.  Lane (fr, fg) of an MFMA
// supplies A[fr][fg] = X[t0 + fr][c + 8 fg + m] and B[fg][fr] =
// F(c + 8 fg + m, 16 j + fr) for m = 0..7: one 16-byte X load feeds eight
// MFMAs per row tile.  FK: F(c, i) = f[i * fsi + c] (A's [r, K] layout;
// 16-byte loads), else f[c * fsc + i] (B's [N, r] layout).  Each wave keeps
// kStages column groups of loads in flight (a register ring).
constexpr int kRowsWaves = 8, kRowsRT = 2, kStages = 4;

// raw 16-byte X load (converted at use)
template <typename TX> struct Raw16;
template <> struct Raw16<bf16> {
    bf16x8 v;
    VKH_DEV void ld(const bf16 *p) { v = *reinterpret_cast<const bf16x8 *>(p); }
    VKH_DEV void zero() { v = bf16x8{}; }
    VKH_DEV float operator[](int e) const { return (float)v[e]; }
};
template <> struct Raw16<float> {
    float4 a, b;
    VKH_DEV void ld(const float *p) {
        a = *reinterpret_cast<const float4 *>(p);
        b = *reinterpret_cast<const float4 *>(p + 4);
    }
    VKH_DEV void zero() { a = b = make_float4(0.f, 0.f, 0.f, 0.f); }
    VKH_DEV float operator[](int e) const {  // e is a compile-time index at every use
        return e == 0 ? a.x : e == 1 ? a.y : e == 2 ? a.z : e == 3 ? a.w
             : e == 4 ? b.x : e == 5 ? b.y : e == 6 ? b.z : b.w;
    }
};

template <typename TX, int NR, bool FK>
__global__ __launch_bounds__(kRowsWaves * 64) void lora_rows_k(const TX *__restrict__ x, long ldx,
                                                              int T, int r, LoraSegs sg,
                                                              float alpha) {
    __shared__ f32x4 red[kRowsWaves][kRowsRT][NR][64];
    const LoraSeg &s = sg.s[blockIdx.y];
    const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
    const int fr = lane % 16, fg = lane / 16;
    const int t0 = blockIdx.x * 16 * kRowsRT;
    const int ng = s.ncols / 32;
    const int g0 = wave * ng / kRowsWaves, g1 = (wave + 1) * ng / kRowsWaves;

    const TX *xr[kRowsRT];
    bool rok[kRowsRT];
#pragma unroll
    for (int a = 0; a < kRowsRT; ++a) {
        const int t = t0 + 16 * a + fr;
        rok[a] = t < T;
        xr[a] = x + (long)(rok[a] ? t : 0) * ldx + s.col + 8 * fg;
    }
    const float *fp[NR];
    bool iok[NR];
#pragma unroll
    for (int j = 0; j < NR; ++j) {
        const int i = 16 * j + fr;
        iok[j] = i < r;
        fp[j] = s.f + (iok[j] ? i : 0) * (FK ? s.fsi : 1) + (FK ? 8 * fg : 8 * fg * s.fsc);
    }
    f32x4 acc[kRowsRT][NR];
#pragma unroll
    for (int a = 0; a < kRowsRT; ++a)
#pragma unroll
        for (int j = 0; j < NR; ++j) acc[a][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    struct Stage {
        Raw16<TX> x[kRowsRT];
        float f[NR][8];
    };
    auto load = [&](int g, Stage &st) {
        const int c = 32 * g;
#pragma unroll
        for (int a = 0; a < kRowsRT; ++a) {
            if (rok[a]) st.x[a].ld(xr[a] + c);
            else st.x[a].zero();
        }
#pragma unroll
        for (int j = 0; j < NR; ++j) {
            if (!iok[j]) {
#pragma unroll
                for (int e = 0; e < 8; ++e) st.f[j][e] = 0.f;
            } else if constexpr (FK) {
                ld8(st.f[j], fp[j] + c);
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) st.f[j][e] = fp[j][(long)(c + e) * s.fsc];
            }
        }
    };
    // ring of kStages: group g + kStages - 1 is requested before group g computes
    Stage st[kStages];
#pragma unroll
    for (int k = 0; k < kStages - 1; ++k)
        if (g0 + k < g1) load(g0 + k, st[k]);
    for (int g = g0; g < g1; g += kStages) {
#pragma unroll
        for (int k = 0; k < kStages; ++k) {
            const int gg = g + k;
            if (gg >= g1) break;
            if (gg + kStages - 1 < g1) load(gg + kStages - 1, st[(k + kStages - 1) % kStages]);
#pragma unroll
            for (int m = 0; m < 8; ++m)
#pragma unroll
                for (int a = 0; a < kRowsRT; ++a)
#pragma unroll
                    for (int j = 0; j < NR; ++j)
                        acc[a][j] = mfma16x16x4(st[k].x[a][m], st[k].f[j][m], acc[a][j]);
        }
    }
#pragma unroll
    for (int a = 0; a < kRowsRT; ++a)
#pragma unroll
        for (int j = 0; j < NR; ++j) red[wave][a][j][lane] = acc[a][j];
    __syncthreads();
    // acc[a][j][q] of lane ln is C[16 a + 4 (ln / 16) + q][16 j + ln % 16]
    for (int e = threadIdx.x; e < kRowsRT * NR * 64; e += kRowsWaves * 64) {
        const int ln = e % 64, j = (e / 64) % NR, a = e / 64 / NR;
        f32x4 v = red[0][a][j][ln];
#pragma unroll
        for (int w = 1; w < kRowsWaves; ++w) v += red[w][a][j][ln];
        const int i = 16 * j + ln % 16;
        if (i >= r) continue;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int t = t0 + 16 * a + 4 * (ln / 16) + q;
            if (t < T) s.u[(long)t * s.ldu + i] = alpha * v[q];
        }
    }
}

// ── lora_cols ───────────────────────────────────────────────────────────
// Block = 64 columns of one adapter (blockIdx.y) x all r outputs; 8 waves:
// wave w owns column tile w % 4 over row half w / 4.  Each half stages
// 64-row chunks of X (fp32, row stride 80 floats: lanes reading four rows of
// 16 consecutive columns hit disjoint bank halves) and of U through LDS, with
// the next chunk prefetched into registers; the MFMA takes A[fr][fg] =
// X[t + fg][c + fr] (a column tile as its rows, rows as k) and B[fg][fr] =
// U[t + fg][16 j + fr].  The two halves are summed through LDS.
constexpr int kColsCW = 64, kColsRows = 64, kXS = kColsCW + 16;

template <int NR>
constexpr int cols_us() { return (NR % 2) ? 16 * NR : 16 * NR + 16; }

template <typename TX, int NR>
__global__ __launch_bounds__(512) void lora_cols_k(const TX *__restrict__ x, long ldx, int T,
                                                  int r, LoraSegs sg, float alpha) {
    constexpr int US = cols_us<NR>();
    constexpr int UL = (kColsRows * 16 * NR / 4 + 255) / 256;  // U float4 loads per thread
    __shared__ float xs[2][kColsRows][kXS];
    __shared__ float us[2][kColsRows][US];
    __shared__ f32x4 red[4][NR][64];
    const LoraSeg &s = sg.s[blockIdx.y];
    const int c0 = blockIdx.x * kColsCW;
    if (c0 >= s.ncols) return;  // whole block: this adapter has fewer column tiles
    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
    const int h = wave / 4, q = wave % 4, ht = tid % 256;
    const int fr = lane % 16, fg = lane / 16;
    const int half = (T + 1) / 2, tb = h * half, te = h ? T : half;
    const int nch = (half + kColsRows - 1) / kColsRows;  // same count for both halves

    const TX *xb = x + s.col + c0;
    // a chunk's loads, raw (converted when stored to LDS); kStages chunks in
    // flight per thread (a register ring)
    constexpr int XE = 8;  // X values per ring entry (bf16: one 16-byte load, fp32: two)
    constexpr int XN = kColsRows * kColsCW / XE / 256;  // entries per thread per chunk
    struct Stage {
        Raw16<TX> x[XN];
        float4 u[UL];
    };
    auto load = [&](int ch, Stage &st) {
        const int r0 = tb + ch * kColsRows;
#pragma unroll
        for (int k = 0; k < XN; ++k) {
            const int e = (ht + 256 * k) * XE, row = e / kColsCW, col = e % kColsCW;
            const int t = r0 + row;
            if (t < te) st.x[k].ld(xb + (long)t * ldx + col);
            else st.x[k].zero();
        }
#pragma unroll
        for (int k = 0; k < UL; ++k) {
            const int e = (ht + 256 * k) * 4, row = e / (16 * NR), col = e % (16 * NR);
            const int t = r0 + row;
            st.u[k] = float4{0.f, 0.f, 0.f, 0.f};
            if (row < kColsRows && t < te && col < r)
                st.u[k] = *reinterpret_cast<const float4 *>(s.u + (long)t * s.ldu + col);
        }
    };
    auto store = [&](const Stage &st) {
#pragma unroll
        for (int k = 0; k < XN; ++k) {
            const int e = (ht + 256 * k) * XE, row = e / kColsCW, col = e % kColsCW;
            float4 *d = reinterpret_cast<float4 *>(&xs[h][row][col]);
            d[0] = make_float4(st.x[k][0], st.x[k][1], st.x[k][2], st.x[k][3]);
            d[1] = make_float4(st.x[k][4], st.x[k][5], st.x[k][6], st.x[k][7]);
        }
#pragma unroll
        for (int k = 0; k < UL; ++k) {
            const int e = (ht + 256 * k) * 4, row = e / (16 * NR), col = e % (16 * NR);
            if (row < kColsRows) *reinterpret_cast<float4 *>(&us[h][row][col]) = st.u[k];
        }
    };
    f32x4 acc[NR];
#pragma unroll
    for (int j = 0; j < NR; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    Stage st[kStages];
#pragma unroll
    for (int k = 0; k < kStages - 1; ++k)
        if (k < nch) load(k, st[k]);
    // nch is the same for every thread: the barriers below are uniform
    for (int ch0 = 0; ch0 < nch; ch0 += kStages) {
#pragma unroll
        for (int k = 0; k < kStages; ++k) {
            const int ch = ch0 + k;
            if (ch >= nch) break;
            __syncthreads();  // the previous chunk's reads are done
            store(st[k]);
            __syncthreads();
            if (ch + kStages - 1 < nch) load(ch + kStages - 1, st[(k + kStages - 1) % kStages]);
#pragma unroll
            for (int kk = 0; kk < kColsRows / 4; ++kk) {
                const float a = xs[h][4 * kk + fg][16 * q + fr];
#pragma unroll
                for (int j = 0; j < NR; ++j) acc[j] = mfma16x16x4(a, us[h][4 * kk + fg][16 * j + fr], acc[j]);
            }
        }
    }
    __syncthreads();
    if (h == 1)
#pragma unroll
        for (int j = 0; j < NR; ++j) red[q][j][lane] = acc[j];
    __syncthreads();
    if (h == 1) return;
    // acc[j][k] of lane ln is C[4 (ln / 16) + k][16 j + ln % 16]: column
    // c0 + 16 q + 4 (ln / 16) + k, rank index 16 j + ln % 16
#pragma unroll
    for (int j = 0; j < NR; ++j) {
        const f32x4 v = acc[j] + red[q][j][lane];
        const int i = 16 * j + fr;
        if (i >= r) continue;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const long c = c0 + 16 * q + 4 * fg + k;
            s.g[c * s.gsc + (long)i * s.gsi] = alpha * v[k];
        }
    }
}

// ── lora_update ─────────────────────────────────────────────────────────
// Block = kUpdRows rows x 1024 columns of Y; thread = those rows x 4
// consecutive columns (float4 in and out).  The adapters' U rows of the block
// go through LDS once (read back as broadcasts); each thread loads its
// columns' factor values once per 4 rank indices and applies them to all
// kUpdRows rows.  Adapters whose column range holds the thread's columns add
// their rank-r product (FK: F(c, i) = f[i * fsi + c], one float4 per i; else
// f[c * fsc + i], one float4 per column and four i).
constexpr int kUpdCols = 1024, kUpdRows = 16;

template <bool FK>
__global__ __launch_bounds__(256) void lora_update_k(float *__restrict__ y, long ldy, int T, int r,
                                                     LoraSegs sg, float alpha) {
    __shared__ float4 ush[3][kUpdRows][16];  // U rows t0.. of each adapter (r <= 64)
    const int c = blockIdx.x * kUpdCols + threadIdx.x * 4;
    const int t0 = blockIdx.y * kUpdRows;
    for (int e = threadIdx.x; e < sg.n * kUpdRows * 16; e += 256) {
        const int si = e / (kUpdRows * 16), row = (e / 16) % kUpdRows, q4 = e % 16;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (t0 + row < T && 4 * q4 < r)
            v = *reinterpret_cast<const float4 *>(sg.s[si].u + (long)(t0 + row) * sg.s[si].ldu + 4 * q4);
        ush[si][row][q4] = v;
    }
    __syncthreads();
    float acc[kUpdRows][4] = {};
    bool any = false;
    for (int si = 0; si < sg.n; ++si) {
        const LoraSeg &s = sg.s[si];
        if (c < s.col || c >= s.col + s.ncols) continue;
        any = true;
        const long cc = c - s.col;
        for (int i = 0; i < r; i += 4) {
            // f4[e] = F(cc + 0..3, i + e) as a float4 over the 4 columns
            float4 f4[4];
            if constexpr (FK) {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    f4[e] = *reinterpret_cast<const float4 *>(s.f + (long)(i + e) * s.fsi + cc);
            } else {
                float4 fc[4];  // fc[col] = F(cc + col, i .. i + 3)
#pragma unroll
                for (int col = 0; col < 4; ++col)
                    fc[col] = *reinterpret_cast<const float4 *>(s.f + (cc + col) * s.fsc + i);
                f4[0] = make_float4(fc[0].x, fc[1].x, fc[2].x, fc[3].x);
                f4[1] = make_float4(fc[0].y, fc[1].y, fc[2].y, fc[3].y);
                f4[2] = make_float4(fc[0].z, fc[1].z, fc[2].z, fc[3].z);
                f4[3] = make_float4(fc[0].w, fc[1].w, fc[2].w, fc[3].w);
            }
#pragma unroll
            for (int a = 0; a < kUpdRows; ++a) {
                const float4 u = ush[si][a][i / 4];
                const float uu[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    acc[a][0] += uu[e] * f4[e].x;
                    acc[a][1] += uu[e] * f4[e].y;
                    acc[a][2] += uu[e] * f4[e].z;
                    acc[a][3] += uu[e] * f4[e].w;
                }
            }
        }
    }
    if (!any) return;
#pragma unroll
    for (int a = 0; a < kUpdRows; ++a) {
        const int t = t0 + a;
        if (t >= T) break;
        float4 *yp = reinterpret_cast<float4 *>(y + (long)t * ldy + c);
        float4 v = *yp;
        v.x += alpha * acc[a][0]; v.y += alpha * acc[a][1];
        v.z += alpha * acc[a][2]; v.w += alpha * acc[a][3];
        *yp = v;
    }
}

bool al16(const void *p) { return ((uintptr_t)p & 15) == 0; }

template <typename TX>
hipError_t rows_launch(const TX *x, long ldx, int T, int r, const LoraSegs &g, float alpha,
                       bool fk, hipStream_t st) {
    const dim3 grid((T + 16 * kRowsRT - 1) / (16 * kRowsRT), g.n), blk(kRowsWaves * 64);
    const int nr = (r + 15) / 16;
#define VKH_ROWS(NR)                                                                          \
    if (nr == NR) {                                                                           \
        if (fk) hipLaunchKernelGGL((lora_rows_k<TX, NR, true>), grid, blk, 0, st, x, ldx, T, r, g, alpha); \
        else hipLaunchKernelGGL((lora_rows_k<TX, NR, false>), grid, blk, 0, st, x, ldx, T, r, g, alpha);   \
        return hipGetLastError();                                                             \
    }
    VKH_ROWS(1) VKH_ROWS(2) VKH_ROWS(3) VKH_ROWS(4)
#undef VKH_ROWS
    return hipErrorInvalidValue;
}

template <typename TX>
hipError_t cols_launch(const TX *x, long ldx, int T, int r, const LoraSegs &g, float alpha,
                       hipStream_t st) {
    int nb = 0;
    for (int i = 0; i < g.n; ++i) nb = std::max(nb, g.s[i].ncols / kColsCW);
    const dim3 grid(nb, g.n), blk(512);
    const int nr = (r + 15) / 16;
#define VKH_COLS(NR)                                                                            \
    if (nr == NR) {                                                                             \
        hipLaunchKernelGGL((lora_cols_k<TX, NR>), grid, blk, 0, st, x, ldx, T, r, g, alpha);    \
        return hipGetLastError();                                                               \
    }
    VKH_COLS(1) VKH_COLS(2) VKH_COLS(3) VKH_COLS(4)
#undef VKH_COLS
    return hipErrorInvalidValue;
}

}  // namespace

// Shapes the three kernels take: r <= 64 and a multiple of 4, every adapter's
// columns a multiple of 64 starting on a 16-byte boundary of X / Y, rows of
// X, Y and U 16-byte aligned, factor layouts that allow float4 loads.
LoraGroupSegs lora_group_segs(const LoraAdapter *ad, int na, int r) {
    LoraGroupSegs g;
    for (int i = 0; i < na && i < 3; ++i) {
        const LoraAdapter &a = ad[i];
        g.fwd_rows.s[g.fwd_rows.n++] = LoraSeg{0, a.k, a.a, 1, (long)a.k, a.inter, (long)r};
        g.fwd_upd.s[g.fwd_upd.n++] = LoraSeg{a.col, a.n, a.b, (long)r, 1, a.inter, (long)r};
        g.bwd_rows.s[g.bwd_rows.n++] = LoraSeg{a.col, a.n, a.b, (long)r, 1, a.dyb, (long)r};
        g.bwd_upd.s[g.bwd_upd.n++] = LoraSeg{0, a.k, a.a, 1, (long)a.k, a.dyb, (long)r};
        g.bwd_da.s[g.bwd_da.n++] =
            LoraSeg{0, a.k, nullptr, 1, 1, a.dyb, (long)r, a.da, 1, (long)a.k};
        g.bwd_db.s[g.bwd_db.n++] =
            LoraSeg{a.col, a.n, nullptr, 1, 1, a.inter, (long)r, a.db, (long)r, 1};
    }
    return g;
}

bool lora_fast_ok(DType xt, const void *x, long ldx, int r, const LoraSegs &g) {
    if (r < 1 || r > 64 || r % 4 || g.n < 1 || g.n > 3) return false;
    const long xv = xt == DType::BF16 ? 8 : 4;
    if (x && (!al16(x) || ldx % xv)) return false;
    for (int i = 0; i < g.n; ++i) {
        const LoraSeg &s = g.s[i];
        if (s.ncols <= 0 || s.ncols % kColsCW || s.col % xv) return false;
        if (s.u && (!al16(s.u) || s.ldu % 4)) return false;
        if (s.f) {
            if (!al16(s.f)) return false;
            if (s.fsc == 1 ? s.fsi % 4 : s.fsc % 4) return false;
        }
    }
    return true;
}

bool lora_update_ok(const float *y, long ldy, int r, const LoraSegs &g) {
    if (!al16(y) || ldy % 4) return false;
    for (int i = 1; i < g.n; ++i)
        if ((g.s[i].fsc == 1) != (g.s[0].fsc == 1)) return false;
    return lora_fast_ok(DType::F32, nullptr, 0, r, g);
}

hipError_t lora_rows(DType xt, const void *x, long ldx, int T, int r, const LoraSegs &g,
                     float alpha, hipStream_t st) {
    if (T <= 0) return hipSuccess;
    const bool fk = g.s[0].fsc == 1;
    for (int i = 1; i < g.n; ++i)
        if ((g.s[i].fsc == 1) != fk) return hipErrorInvalidValue;
    if (xt == DType::BF16) return rows_launch((const bf16 *)x, ldx, T, r, g, alpha, fk, st);
    return rows_launch((const float *)x, ldx, T, r, g, alpha, fk, st);
}

hipError_t lora_cols(DType xt, const void *x, long ldx, int T, int r, const LoraSegs &g,
                     float alpha, hipStream_t st) {
    if (T <= 0) return hipSuccess;
    if (xt == DType::BF16) return cols_launch((const bf16 *)x, ldx, T, r, g, alpha, st);
    return cols_launch((const float *)x, ldx, T, r, g, alpha, st);
}

hipError_t lora_update(float *y, long ldy, int T, int r, const LoraSegs &g, float alpha,
                       hipStream_t st) {
    if (T <= 0) return hipSuccess;
    if (!al16(y) || ldy % 4) return hipErrorInvalidValue;
    const bool fk = g.s[0].fsc == 1;
    long cols = 0;
    for (int i = 0; i < g.n; ++i) {
        if ((g.s[i].fsc == 1) != fk) return hipErrorInvalidValue;
        cols = std::max(cols, g.s[i].col + g.s[i].ncols);
    }
    const dim3 grid((cols + kUpdCols - 1) / kUpdCols, (T + kUpdRows - 1) / kUpdRows), blk(256);
    if (fk) hipLaunchKernelGGL(lora_update_k<true>, grid, blk, 0, st, y, ldy, T, r, g, alpha);
    else hipLaunchKernelGGL(lora_update_k<false>, grid, blk, 0, st, y, ldy, T, r, g, alpha);
    return hipGetLastError();
}

}  // namespace vkh
