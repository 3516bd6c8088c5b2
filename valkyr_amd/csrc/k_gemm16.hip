// Linear-layer GEMMs on bf16 operands (the bf16 precision of the training
// step): forward y = x W^T (matmul_nt_v2.comp), dx = dy W
// (linear_backward_dx_batched.comp) and dW = dy^T x
// (linear_backward_dw_batched.comp), on the gemm16 kernel.
//
// Tile plan (measured on MI355X with DMA staging, T = 2048-token step shapes):
//   * >= 512 tiles of 256 x 256       -> 256 x 256, 8 waves (vocab-sized GEMMs)
//   * >= 512 tiles of 128 x 128       -> 128 x 128, 8 waves of 64 x 32
//   * K >= 16384 and >= 256 tiles of 128 x 128 -> 256 x 256 split-K 3 ways
//   * K >= 4096 and >= 256 tiles of 128 x 128  -> 128 x 128, 8 waves
//   * K >= 16384 and < 256 such tiles -> 256 x 256 split-K 8 ways (head dh)
//   * < 384 tiles of 128 x 64, K >= 2048 -> 128 x 64 split-K 2 ways
//   * otherwise                       -> 128 x 64
// Operands that break the kernel's layout rules (16-byte alignment, ld and
// the contiguous extent multiples of 8, < 2 GiB) take the generic MFMA GEMM.
#include <algorithm>

#include "gemm16.hpp"
#include "ops.hpp"
#include "qkv8.hpp"

namespace vkh {

namespace {

using TBig = Tile16<256, 256, 2, 4>;
using T128 = Tile16<128, 128, 2, 2>;
using T128x64 = Tile16<128, 64, 2, 2>;
using T128w8 = Tile16<128, 128, 2, 4>;  // 8 waves of 64 x 32
// The in-block split-K block (two 4-wave groups, one block per CU whatever its
// LDS) with three slab buffers per group (144 KB): two slabs in flight per
// group for these latency-bound N = 1024 shapes.  Alone: o / down forward
// 20.0 / 27.8 -> 18.4 / 24.5 us, gate/up and q/k/v dx 50.3 / 34.7 -> 48.4 / 33.6
// us; the bf16 step 19.33-19.34 -> 19.31-19.32 ms.  (In fp32 mode, whose slabs
// are half as deep, it made the fp32 step slower: 77.3 against 76.65 ms.)
using T128x64s3 = Tile16<128, 64, 2, 2, 3>;
// (Three slab buffers were measured slower for these tiles: the larger LDS
// footprint drops a block per CU.  Staging the slabs through VGPRs two slabs
// ahead, which doubles the time a load has to arrive without more LDS, was
// measured equal on every per-layer shape alone and in the step: slab
// latency is not what bounds these GEMMs.)

constexpr bool kUseKs2 = true;

enum class Pick { Big, T128, T128x64, T128w8, T128x64ks2 };
struct Plan {
    Pick tile;
    int splits;
    bool column_order = false;  // tiles in plain column order (no row groups)
};

size_t ws_for(const Plan &p, const GemmShape &s) {
    if (p.splits <= 1) return 0;
    switch (p.tile) {
    case Pick::Big: return gemm16_ws_bytes<TBig>(s, p.splits);
    case Pick::T128: return gemm16_ws_bytes<T128>(s, p.splits);
    case Pick::T128w8: return gemm16_ws_bytes<T128w8>(s, p.splits);
    default: return gemm16_ws_bytes<T128x64>(s, p.splits);
    }
}

Plan plan(const GemmShape &s, size_t ws_bytes) {
    auto tiles = [&](int bm, int bn) { return (long)ceil_div(s.M, bm) * (long)ceil_div(s.N, bn); };
    if (tiles(256, 256) >= 512) return {Pick::Big, 1};
    const long t128 = tiles(128, 128), t64 = tiles(128, 64);
    if (t128 >= 512) return {Pick::T128w8, 1};
    const int nk = (s.K + 63) / 64;
    Plan p{Pick::T128x64, 1};
    if (s.K >= 16384 && t128 >= 256)
        // a long contraction onto at least a chip-wide wave of 128 x 128 tiles
        // (Qwen3-4B gate/up dx, K = 19456): 256 x 256 split 3 ways, 199 us
        // against 236 (128 x 128, 8 waves) and 361 (128 x 64)
        p = Plan{Pick::Big, 3};
    else if (s.K >= 4096 && t128 >= 256)
        // Qwen3-4B o / down forward and q/k/v dx (N = 2560, K = 4096..9728):
        // 128 x 128 on 8 waves, 50 / 113 / 79 us against 56 / 167 / 104 (128 x 64);
        // in column order (the LoRA step: 66.7 against 68.1 ms with row groups)
        p = Plan{Pick::T128w8, 1, true};
    else if (s.K >= 16384 && t128 < 256)
        // the head's dh at config 3 (M = 2048, N = 1024, K = 151936: 32 tiles of
        // 256 x 256): split 8 ways, 256 blocks; in the step 18.78-18.79 against
        // 18.91 ms for 128 x 128 split 4 (Big split 16: 18.93-18.96; 128 x 128
        // split 8: 19.06-19.10)
        p = Plan{Pick::Big, 8};
    else if (t64 < 384 && s.K >= 2048)
        // two wave groups in one block: alone, faster than split-K + reduce up
        // to K = 4096 and slower at 6144, but in the two-stream step faster
        // for every such shape (22.2 vs 22.5 ms with split-K kept at 6144 and
        // for the weight gradients, 22.8 ms with split-K everywhere)
        p = kUseKs2 ? Plan{Pick::T128x64ks2, 1} : Plan{Pick::T128x64, 2};
    while (p.splits > 1 && (nk / p.splits < 8 || ws_for(p, s) > ws_bytes)) --p.splits;
    return p;
}

// Whether the fused-epilogue forward kernels (8-wave 128 x 128 tiles only) take
// the product: where plan() picks that tile, or, for a launch paired with one
// of the same shape on a second stream (the forward's two half batches), where
// M is whole tiles and the pair together fills a chip-wide round (the config-3
// step's q|k|v and gate/up halves: 256 + 256 and 384 + 384 tiles; the forward
// as two concurrent half batches measured 18.58-18.59 against 18.85 ms).
bool fused_tile_ok(const GemmShape &s, bool paired) {
    const Plan p = plan(s, 0);
    if (p.tile == Pick::T128w8 && p.splits == 1) return true;
    return paired && s.M % 128 == 0 && 2L * (s.M / 128) * ceil_div(s.N, 128) >= 512;
}

template <Lay LA, Lay LB, class Epi>
hipError_t run16(const Op16 &a, const Op16 &b, const GemmShape &s, const Epi &e, const GemmWs &ws,
                 hipStream_t st) {
    const Plan p = plan(s, ws.p ? ws.bytes : 0);
    const SplitK sk{p.splits, (f32x4 *)ws.p};
    const int g = p.column_order ? 0 : tile_group_rows<LA, LB>();
    switch (p.tile) {
    case Pick::Big: return launch_gemm16<TBig, LA, LB>(a, b, s, e, sk, g, st);
    case Pick::T128: return launch_gemm16<T128, LA, LB>(a, b, s, e, sk, g, st);
    case Pick::T128w8: return launch_gemm16<T128w8, LA, LB>(a, b, s, e, sk, g, st);
    case Pick::T128x64ks2: return launch_gemm16_ks2<T128x64s3, LA, LB>(a, b, s, e, g, st);
    default: return launch_gemm16<T128x64, LA, LB>(a, b, s, e, sk, g, st);
    }
}

// ── fp32 operands (the reference-precision step) ───────────────────────
// The same kernels with F32 set: slabs of 32 fp32 values (128-byte tile rows,
// the bf16 slab's layout), four v_mfma_f32_16x16x4_f32 per 16-byte fragment.
// At a sixteenth of the bf16 matrix rate the slab DMA has ample time to land,
// so the plan only has to spread whole rounds of tiles over the 256 CUs.
// Measured per shape alone at the config-3 step's 12 layer GEMMs (T = 2048):
//   * 128 x 128 on 8 waves where its tile count fills rounds at least as
//     evenly as 128 x 64 (q/k/v and gate/up forward, o dx, q/k/v dW: 130-196 us
//     against 143-210 on 128 x 64 and 210-290 on 4-wave 128 x 128 or 256 x 256);
//   * 128 x 64 where that evens the rounds (384 tiles of 128 x 128 = 768 of
//     128 x 64: down dx 107 against 134 us, gate/up dW 209 against 259);
//   * fewer than 512 tiles of 128 x 64 (the N = 1024 outputs and dW of o /
//     down): 128 x 64 with the K range split over the two wave groups of one
//     block.  Alone, split-K over two launches plus the reduce is faster
//     (q/k/v dx 149, gate/up dx 213, down dW 119 us against 174, 254, 154),
//     but in the two-stream step the in-block form is (76.3-77.0 against
//     76.5-77.1 ms in four alternating pairs; plain 128 x 64: 77.3-77.4): the
//     reduce launches' 4.2 ms of partial traffic per step is gone.
Plan plan32(const GemmShape &s, size_t ws_bytes) {
    auto tiles = [&](int bm, int bn) { return (long)ceil_div(s.M, bm) * (long)ceil_div(s.N, bn); };
    auto fill = [](long t) { return (double)t / (256.0 * (double)((t + 255) / 256)); };
    const long t128 = tiles(128, 128), t64 = tiles(128, 64);
    const int nk = (s.K + 31) / 32;
    Plan p{Pick::T128x64, 1};
    if (t128 >= 256 && fill(t128) >= fill(t64)) p = Plan{Pick::T128w8, 1};
    else if (t64 < 512) p = Plan{Pick::T128x64ks2, 1};
    while (p.splits > 1 && (nk / p.splits < 8 || ws_for(p, s) > ws_bytes)) --p.splits;
    return p;
}

template <Lay LA, Lay LB, class Epi>
hipError_t run32(const Op16 &a, const Op16 &b, const GemmShape &s, const Epi &e, const GemmWs &ws,
                 hipStream_t st) {
    const Plan p = plan32(s, ws.p ? ws.bytes : 0);
    const SplitK sk{p.splits, (f32x4 *)ws.p};
    const int g = p.column_order ? 0 : tile_group_rows<LA, LB>();
    switch (p.tile) {
    case Pick::Big: return launch_gemm16<TBig, LA, LB, Epi, true>(a, b, s, e, sk, g, st);
    case Pick::T128: return launch_gemm16<T128, LA, LB, Epi, true>(a, b, s, e, sk, g, st);
    case Pick::T128w8: return launch_gemm16<T128w8, LA, LB, Epi, true>(a, b, s, e, sk, g, st);
    case Pick::T128x64ks2: return launch_gemm16_ks2<T128x64, LA, LB, Epi, true>(a, b, s, e, g, st);
    default: return launch_gemm16<T128x64, LA, LB, Epi, true>(a, b, s, e, sk, g, st);
    }
}

// fp32 operand view: 16-byte aligned, ld and the contiguous run multiples of 4
// floats (whole 16-byte chunks), under 2 GiB (32-bit buffer offsets).
bool make_op32(const float *p, long ld, long rows, long run, Op16 &o) {
    if (((uintptr_t)p & 15u) || ld % 4 || run % 4 || rows <= 0) return false;
    const size_t bytes = ((size_t)(rows - 1) * ld + run) * 4;
    if (bytes >= (1ull << 31)) return false;
    o = Op16{reinterpret_cast<const bf16 *>(p), ld, (unsigned)bytes};
    return true;
}

Mat matf32(const float *p, long ld) { return Mat{p, ld, DType::F32}; }

// Operand of `rows` storage rows whose contiguous run is `run` elements.
bool make_op(const bf16 *p, long ld, long rows, long run, Op16 &o) {
    if (((uintptr_t)p & 15u) || ld % 8 || run % 8 || rows <= 0) return false;
    const size_t bytes = ((size_t)(rows - 1) * ld + run) * 2;
    if (bytes >= (1ull << 31)) return false;
    o = Op16{p, ld, (unsigned)bytes};
    return true;
}

Mat matb(const bf16 *p, long ld) { return Mat{p, ld, DType::BF16}; }

// Rows per chunk when a [rows, ld] bf16 operand view reaches 2 GiB (the DMA
// path's 32-bit offsets): 0 if it fits whole, else a multiple of 64 rows.
int rows_per_2g_chunk(long rows, long ld, long run) {
    if (((rows - 1) * ld + run) * 2 < (1l << 31)) return 0;
    const long fit = ((1l << 31) - 1) / (2 * ld);  // rows whose view fits
    const long n = (rows + fit - 1) / fit;           // chunks
    return (int)(((rows + n - 1) / n + 63) / 64 * 64);
}

// ── LoRA term in the epilogue ──────────────────────────────────────────
// EpiLora<Base> adds rank-r LoRA products (train/lora.zig:99-251) to the tile
// before Base stores it:
//   C[t, col_s + c] = acc + alpha sum_i U_s[t, i] F_s(c, i)
// for every adapter s whose columns [col_s, col_s + ncols) hold c: the
// forward's y += aor inter B^T, or the backward's dx += aor (dy B) A summed
// over the adapters of one shared input.  The output is then written once,
// instead of stored by the GEMM, read back and stored again by a separate
// update pass.  The products run on v_mfma_f32_16x16x4_f32 in the
// accumulator layout: lane (g, c) supplies A[c][k] = alpha U_s[row0 + 16 i + c][k]
// and B[k][c] = F_s(col0 + 16 j + c - col_s, k) for the contraction index
// k = 16 kb + 4 g + e at step e, so the results land on acc[i][j] where Base
// reads them.  Base's own alpha must be 1 (the linear layers' products).
template <class Base>
struct EpiLora {
    Base base;
    LoraSegs sg;
    int r;
    float alpha;

    template <int TM, int TN>
    VKH_DEV void apply(const f32x4 (&acc_in)[TM][TN], const FragPos &fp, const GemmShape &s) const {
        f32x4 acc[TM][TN];
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) acc[i][j] = acc_in[i][j];
        const int g = fp.lane / 16, c = fp.lane % 16;
        for (int si = 0; si < sg.n; ++si) {
            const LoraSeg &q = sg.s[si];
            // wave-uniform: none of the wave's columns in this adapter's range
            if (fp.col0 + 16 * TN <= q.col || fp.col0 >= q.col + q.ncols) continue;
            for (int kb = 0; kb < r; kb += 16) {
                const int k = kb + 4 * g;
                const bool kok = k < r;  // r is a multiple of 4
                f32x4 ua[TM];
#pragma unroll
                for (int i = 0; i < TM; ++i) {
                    const int row = fp.row0 + 16 * i + c;
                    float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
                    if (kok && row < s.M) t = *reinterpret_cast<const float4 *>(q.u + (long)row * q.ldu + k);
                    ua[i] = f32x4{alpha * t.x, alpha * t.y, alpha * t.z, alpha * t.w};
                }
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    const long cb = fp.col0 + 16 * j;  // wave-uniform
                    if (cb < q.col || cb >= q.col + q.ncols) continue;
                    const long cc = cb + c - q.col;
                    f32x4 fb = f32x4{0.f, 0.f, 0.f, 0.f};
                    if (kok) {
                        if (q.fsc == 1) {
#pragma unroll
                            for (int e = 0; e < 4; ++e) fb[e] = q.f[(long)(k + e) * q.fsi + cc];
                        } else {
                            const float4 t = *reinterpret_cast<const float4 *>(q.f + cc * q.fsc + k);
                            fb = f32x4{t.x, t.y, t.z, t.w};
                        }
                    }
#pragma unroll
                    for (int i = 0; i < TM; ++i)
#pragma unroll
                        for (int e = 0; e < 4; ++e) acc[i][j] = mfma16x16x4(ua[i][e], fb[e], acc[i][j]);
                }
            }
        }
        base.template apply<TM, TN>(acc, fp, s);
    }
};

bool al16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

// The adapters' layout rules of EpiLora on an output of n_out columns:
// 16-column blocks, whole 16-byte U rows and factor reads, r <= 64.
bool lora_epi_ok(const LoraSegs &g, int r, int n_out) {
    if (r < 1 || r > 64 || r % 4 || g.n < 1 || g.n > 3) return false;
    for (int i = 0; i < g.n; ++i) {
        const LoraSeg &q = g.s[i];
        if (q.col < 0 || q.col % 16 || q.ncols <= 0 || q.ncols % 16 || q.col + q.ncols > n_out) return false;
        if (!q.u || !al16(q.u) || q.ldu % 4 || q.ldu < r || !q.f) return false;
        if (q.fsc != 1 && (!al16(q.f) || q.fsc % 4 || q.fsi != 1)) return false;
    }
    return true;
}

}  // namespace

bool g16_lora_ok(const bf16 *a, long lda, long arows, long arun, const bf16 *b, long ldb, long brows,
                 long brun, const LoraSegs &g, int r, int n_out) {
    Op16 oa, ob;
    return make_op(a, lda, arows, arun, oa) && make_op(b, ldb, brows, brun, ob) &&
           lora_epi_ok(g, r, n_out);
}

hipError_t g16_nt_lora(const bf16 *x, long ldx, const bf16 *w, long ldw, float *y, long ldy, int M,
                       int N, int K, const float *R, long ldr, const LoraSegs &g, int r,
                       float alpha, const GemmWs &ws, hipStream_t st) {
    Op16 a, b;
    if (!make_op(x, ldx, M, K, a) || !make_op(w, ldw, N, K, b) || !lora_epi_ok(g, r, N))
        return hipErrorInvalidValue;
    EpiLora<EpiStore> e{EpiStore{y, ldy, R, ldr, 1.f, 0.f}, g, r, alpha};
    return run16<Lay::K, Lay::K>(a, b, GemmShape{M, N, K}, e, ws, st);
}

hipError_t g16_nn_lora(const bf16 *dy, long lddy, const bf16 *w, long ldw, float *dx, long lddx,
                       int M, int N, int K, const LoraSegs &g, int r, float alpha, const GemmWs &ws,
                       hipStream_t st) {
    Op16 a, b;
    if (!make_op(dy, lddy, M, N, a) || !make_op(w, ldw, N, K, b) || !lora_epi_ok(g, r, K))
        return hipErrorInvalidValue;
    EpiLora<EpiStore> e{EpiStore{dx, lddx, nullptr, 0, 1.f, 0.f}, g, r, alpha};
    return run16<Lay::K, Lay::MN>(a, b, GemmShape{M, K, N}, e, ws, st);
}

hipError_t g16_nn_bf16_lora(const bf16 *dy, long lddy, const bf16 *w, long ldw, bf16 *dx,
                            long lddx, int M, int N, int K, const LoraSegs &g, int r, float alpha,
                            const GemmWs &ws, hipStream_t st) {
    Op16 a, b;
    if (!make_op(dy, lddy, M, N, a) || !make_op(w, ldw, N, K, b) || !lora_epi_ok(g, r, K))
        return hipErrorInvalidValue;
    EpiLora<EpiStoreBf16> e{EpiStoreBf16{dx, lddx, 1.f}, g, r, alpha};
    return run16<Lay::K, Lay::MN>(a, b, GemmShape{M, K, N}, e, ws, st);
}

hipError_t g16_nt(const bf16 *x, long ldx, const bf16 *w, long ldw, float *y, long ldy, int M,
                  int N, int K, const float *R, long ldr, float alpha, float beta,
                  const GemmWs &ws, hipStream_t st) {
    Op16 a, b;
    if (!make_op(x, ldx, M, K, a) || !make_op(w, ldw, N, K, b))
        return gemm_nt(Precision::BF16, matb(x, ldx), matb(w, ldw), y, ldy, M, N, K, R, ldr, alpha,
                       beta, st);
    EpiStore e{y, ldy, R, ldr, alpha, beta};
    return run16<Lay::K, Lay::K>(a, b, GemmShape{M, N, K}, e, ws, st);
}

// gu[M, 2F] = x[M, K] w_gu[2F, K]^T and gated[M, F] = bf16(swiglu1(gu[:, f], gu[:, F + f])) in
// one launch, where the plain plan for the [M, 2F] product is the 8-wave 128 x 128 tile
// (each block then takes 64 gate and the matching 64 up features); hipErrorNotSupported
// (nothing launched) elsewhere, and the caller runs g16_nt + swiglu_forward.  (The same
// epilogue on the 256 x 256 tile, 128 + 128 features per block and a 128 KB hand-over, was
// parity-green but measured config 4 at 59.93-60.07 against 59.68-59.73 ms and config 5
// unchanged, 584.1-584.6 against 584.0-585.0 ms.)
hipError_t g16_gate_up_swiglu(const bf16 *x, long ldx, const bf16 *w, long ldw, float *gu,
                              long ldgu, bf16 *gated, long ldg, int M, int F, int K, hipStream_t st,
                              bool paired) {
    if (M <= 0 || F <= 0 || F % 64) return hipErrorNotSupported;
    if (!fused_tile_ok(GemmShape{M, 2 * F, K}, paired)) return hipErrorNotSupported;
    Op16 a, b;
    if (!make_op(x, ldx, M, K, a) || !make_op(w, ldw, 2L * F, K, b)) return hipErrorNotSupported;
    const unsigned tiles = (unsigned)(ceil_div(M, T128w8::BM) * (F / (T128w8::BN / 2)));
    hipLaunchKernelGGL((gemm16_swiglu_kernel<T128w8>), dim3(tiles), dim3(T128w8::NT), 0, st, a, b, M,
                       F, K, gu, ldgu, gated, ldg, tile_group_rows<Lay::K, Lay::K>());
    return hipGetLastError();
}

namespace {

template <typename TO>
struct QkvEpi {
    QkvLayout L;
    const float *wq, *wk;  // q / k RMSNorm gains (qk_norm)
    TO *out;               // the attention operand [rows, (Hq + 2 Hkv) hd]
    long ld_out;
    const float2 *tab;     // RoPE cos / sin [seq_len][rotary_dim / 2]
};

// The q|k|v projection with the Q/K-RMSNorm + RoPE forward in its epilogue (head_dim
// 128, so a 128 x 128 tile is 128 rows of one head): the tile stores its fp32
// projection (the backward's pre-norm values), stages it in the idle slab buffers (16-float
// group u of row r at u ^ ((r >> 2) & 3), so the four row groups of a store land on
// different banks), and its waves then run the standalone pass's item code
// (qkv_fwd_item8, 16 lanes per row) on it and write the bf16 attention operand.
template <class Cfg, bool F32 = false, typename TO = bf16>
__global__ __launch_bounds__(Cfg::NT, 1) void gemm16_qkv_kernel(Op16 a, Op16 b, GemmShape s, float *C,
                                                               long ldc, QkvEpi<TO> q, int tgrp) {
    constexpr int BM = Cfg::BM, BN = Cfg::BN, NT = Cfg::NT, NW = NT / 64;
    constexpr int WM = BM / Cfg::WGM, WN = BN / Cfg::WGN;
    constexpr int TM = WM / 16, TN = WN / 16;
    constexpr int LPH = 16, G = 64 / LPH;  // lanes per row, rows per wave
    static_assert(BN == 128 && BM * BN * 4 <= Cfg::LDS && BM % (NW * G) == 0, "one head per tile");
    __shared__ __attribute__((aligned(16))) char smem[Cfg::LDS];
    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
    const int wm = wave / Cfg::WGN, wn = wave % Cfg::WGN;
    const int nbm = (s.M + BM - 1) / BM, nbn = s.N / BN;
    const int nb = nbm * nbn;
    int bid = blockIdx.x;
    if (nb % 8 == 0) bid = (bid % 8) * (nb / 8) + bid / 8;
    int bm, bn;
    tile_rc(bid, nbm, nbn, tgrp, bm, bn);
    const int m0 = bm * BM, n0 = bn * BN;
    f32x4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    constexpr int KW = F32 ? 32 : 64;  // k per slab
    gemm16_tile_dma<Cfg, Lay::K, Lay::K, TM, TN, F32>(a, b, m0, n0, s.M, s.N, 0, (s.K + KW - 1) / KW,
                                                      s.K, acc, smem);
    float *lt = reinterpret_cast<float *>(smem);  // the slab loop ended with a barrier
    const int g = lane / 16, c = lane % 16;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int tr = wm * WM + 16 * i + 4 * g + r, tc = wn * WN + 16 * j + c;
                if (m0 + tr < s.M) C[(long)(m0 + tr) * ldc + n0 + tc] = acc[i][j][r];
                lt[tr * BN + (tc ^ (((tr >> 2) & 3) << 4))] = acc[i][j][r];
            }
    lds_barrier();
    const QkvLayout &L = q.L;
    const int h = bn, half = L.rotary_dim / 2, j8 = lane % LPH;
    const Rope8 rp = rope8(j8, half);
    const bool is_q = h < L.n_q_heads, qkh = h < L.n_q_heads + L.n_kv_heads;
    float gq[8], gk[8];
    if (L.qk_norm) {
        ld8(q.wq + 8 * j8, gq);
        ld8(q.wk + 8 * j8, gk);
    }
    for (int tr = wave * G + lane / LPH; tr < BM; tr += NW * G) {
        const int t = m0 + tr;
        const bool valid = t < s.M, qk = valid && qkh;
        float y[8];
        ld8(lt + tr * BN + ((8 * j8) ^ (((tr >> 2) & 3) << 4)), y);
        float2 cs[8];
        if (qk && rp.rot_lane) {
            const float4 *tp =
                reinterpret_cast<const float4 *>(q.tab + (long)(t % L.seq_len) * half + rp.col);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float4 v = tp[i];
                cs[2 * i] = make_float2(v.x, v.y);
                cs[2 * i + 1] = make_float2(v.z, v.w);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) cs[i] = make_float2(1.f, 0.f);
        }
        qkv_fwd_item8<LPH>(L, y, cs, qk, is_q, gq, gk, rp, lane, half);
        if (valid) st8(q.out + (long)t * q.ld_out + h * BN + 8 * j8, y);
    }
}

}  // namespace

// y[M, N] = x w^T (the fp32 q|k|v projection) and the bf16 attention operand out = RoPE(
// Q/K-RMSNorm(y)) (qkv_prepare_forward's values, bit for bit) in one launch, where head_dim
// is 128 and the product's plain plan is the 8-wave 128 x 128 tile; hipErrorNotSupported
// (nothing launched) elsewhere.
hipError_t g16_qkv_norm_rope(const bf16 *x, long ldx, const bf16 *w, long ldw, float *y, long ldy,
                             int M, int N, int K, const QkvLayout &L, const float *wq,
                             const float *wk, bf16 *out, long ld_out, const float2 *tab,
                             hipStream_t st, bool paired) {
    if (M <= 0 || L.head_dim != 128 || L.n_rows != M || L.seq_len <= 0 || L.rotary_dim % 16 ||
        L.rotary_dim > 128 || N != (L.n_q_heads + 2 * L.n_kv_heads) * 128)
        return hipErrorNotSupported;
    const GemmShape s{M, N, K};
    if (!fused_tile_ok(s, paired)) return hipErrorNotSupported;
    const Plan p = plan(s, 0);  // its tile order where it is this tile
    if (((uintptr_t)out & 15u) || ld_out % 8 || (L.qk_norm && (((uintptr_t)wq | (uintptr_t)wk) & 15u)) ||
        (L.rotary_dim && ((uintptr_t)tab & 15u)))
        return hipErrorNotSupported;
    Op16 a, b;
    if (!make_op(x, ldx, M, K, a) || !make_op(w, ldw, N, K, b)) return hipErrorNotSupported;
    const int g = p.tile == Pick::T128w8 && p.column_order ? 0 : tile_group_rows<Lay::K, Lay::K>();
    const unsigned tiles = (unsigned)(ceil_div(M, T128w8::BM) * (N / T128w8::BN));
    hipLaunchKernelGGL((gemm16_qkv_kernel<T128w8>), dim3(tiles), dim3(T128w8::NT), 0, st, a, b, s, y,
                       ldy, QkvEpi<bf16>{L, wq, wk, out, ld_out, tab}, g);
    return hipGetLastError();
}

// The fp32 forms of the two fused projections (fp32 operands on the DMA-staged kernels'
// fp32 slab mode, fp32 outputs), where the fp32 plan is the 8-wave 128 x 128 tile.
hipError_t g32_qkv_norm_rope(const float *x, long ldx, const float *w, long ldw, float *y, long ldy,
                             int M, int N, int K, const QkvLayout &L, const float *wq,
                             const float *wk, float *out, long ld_out, const float2 *tab,
                             hipStream_t st) {
    if (M <= 0 || L.head_dim != 128 || L.n_rows != M || L.seq_len <= 0 || L.rotary_dim % 16 ||
        L.rotary_dim > 128 || N != (L.n_q_heads + 2 * L.n_kv_heads) * 128)
        return hipErrorNotSupported;
    const GemmShape s{M, N, K};
    const Plan p = plan32(s, 0);
    if (p.tile != Pick::T128w8 || p.splits != 1) return hipErrorNotSupported;
    if (((uintptr_t)out & 15u) || ld_out % 4 || (L.qk_norm && (((uintptr_t)wq | (uintptr_t)wk) & 15u)) ||
        (L.rotary_dim && ((uintptr_t)tab & 15u)))
        return hipErrorNotSupported;
    Op16 a, b;
    if (!make_op32(x, ldx, M, K, a) || !make_op32(w, ldw, N, K, b)) return hipErrorNotSupported;
    const int g = p.column_order ? 0 : tile_group_rows<Lay::K, Lay::K>();
    const unsigned tiles = (unsigned)(ceil_div(M, T128w8::BM) * (N / T128w8::BN));
    hipLaunchKernelGGL((gemm16_qkv_kernel<T128w8, true, float>), dim3(tiles), dim3(T128w8::NT), 0, st,
                       a, b, s, y, ldy, QkvEpi<float>{L, wq, wk, out, ld_out, tab}, g);
    return hipGetLastError();
}

hipError_t g32_gate_up_swiglu(const float *x, long ldx, const float *w, long ldw, float *gu,
                              long ldgu, float *gated, long ldg, int M, int F, int K, hipStream_t st) {
    if (M <= 0 || F <= 0 || F % 64) return hipErrorNotSupported;
    const GemmShape s{M, 2 * F, K};
    const Plan p = plan32(s, 0);
    if (p.tile != Pick::T128w8 || p.splits != 1) return hipErrorNotSupported;
    Op16 a, b;
    if (!make_op32(x, ldx, M, K, a) || !make_op32(w, ldw, 2L * F, K, b)) return hipErrorNotSupported;
    const unsigned tiles = (unsigned)(ceil_div(M, T128w8::BM) * (F / (T128w8::BN / 2)));
    hipLaunchKernelGGL((gemm16_swiglu_kernel<T128w8, true, float>), dim3(tiles), dim3(T128w8::NT), 0,
                       st, a, b, M, F, K, gu, ldgu, gated, ldg, p.column_order ? 0 : tile_group_rows<Lay::K, Lay::K>());
    return hipGetLastError();
}

hipError_t g16_nn(const bf16 *dy, long lddy, const bf16 *w, long ldw, float *dx, long lddx, int M,
                  int N, int K, float alpha, float beta, const GemmWs &ws, hipStream_t st) {
    // an over-2 GiB dy (the head's dz at 8192 tokens): independent row chunks
    if (const int mc = M > 64 ? rows_per_2g_chunk(M, lddy, N) : 0) {
        for (int m0 = 0; m0 < M; m0 += mc) {
            const hipError_t e = g16_nn(dy + (long)m0 * lddy, lddy, w, ldw, dx + (long)m0 * lddx,
                                        lddx, std::min(mc, M - m0), N, K, alpha, beta, ws, st);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    // C[m, k'] = sum_n dy[m, n] W[n, k']: A = dy (K-major over n), B(k', n) = W[n][k'] (MN)
    Op16 a, b;
    if (!make_op(dy, lddy, M, N, a) || !make_op(w, ldw, N, K, b))
        return gemm_nn(Precision::BF16, matb(dy, lddy), matb(w, ldw), dx, lddx, M, N, K, alpha,
                       beta, st);
    EpiStore e{dx, lddx, nullptr, 0, alpha, beta};
    return run16<Lay::K, Lay::MN>(a, b, GemmShape{M, K, N}, e, ws, st);
}

hipError_t g16_nn_bf16(const bf16 *dy, long lddy, const bf16 *w, long ldw, bf16 *dx, long lddx,
                       int M, int N, int K, const GemmWs &ws, hipStream_t st) {
    Op16 a, b;
    if (!make_op(dy, lddy, M, N, a) || !make_op(w, ldw, N, K, b)) return hipErrorInvalidValue;
    EpiStoreBf16 e{dx, lddx, 1.f};
    return run16<Lay::K, Lay::MN>(a, b, GemmShape{M, K, N}, e, ws, st);
}

hipError_t g16_tn(const bf16 *dy, long lddy, const bf16 *x, long ldx, float *dw, long lddw, int M,
                  int N, int K, float alpha, float beta, const GemmWs &ws, hipStream_t st) {
    // an over-2 GiB dy (the head's dz at 8192 tokens): the contraction over m in
    // row chunks, each chunk after the first accumulating (beta = 1)
    const int ca = M > 64 ? rows_per_2g_chunk(M, lddy, N) : 0, cb = M > 64 ? rows_per_2g_chunk(M, ldx, K) : 0;
    if (const int mc = (ca && cb) ? std::min(ca, cb) : std::max(ca, cb)) {
        for (int m0 = 0; m0 < M; m0 += mc) {
            const hipError_t e = g16_tn(dy + (long)m0 * lddy, lddy, x + (long)m0 * ldx, ldx, dw, lddw,
                                        std::min(mc, M - m0), N, K, alpha, m0 ? 1.f : beta, ws, st);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    // C[n, k'] = sum_m dy[m, n] x[m, k']: both operands MN-major over m
    Op16 a, b;
    if (!make_op(dy, lddy, M, N, a) || !make_op(x, ldx, M, K, b))
        return gemm_tn(Precision::BF16, matb(dy, lddy), matb(x, ldx), dw, lddw, M, N, K, alpha,
                       beta, st);
    EpiStore e{dw, lddw, nullptr, 0, alpha, beta};
    return run16<Lay::MN, Lay::MN>(a, b, GemmShape{N, K, M}, e, ws, st);
}

hipError_t g32_nt(const float *x, long ldx, const float *w, long ldw, float *y, long ldy, int M,
                  int N, int K, const float *R, long ldr, float alpha, float beta,
                  const GemmWs &ws, hipStream_t st) {
    Op16 a, b;
    if (!make_op32(x, ldx, M, K, a) || !make_op32(w, ldw, N, K, b))
        return gemm_nt(Precision::FP32, matf32(x, ldx), matf32(w, ldw), y, ldy, M, N, K, R, ldr,
                       alpha, beta, st);
    EpiStore e{y, ldy, R, ldr, alpha, beta};
    return run32<Lay::K, Lay::K>(a, b, GemmShape{M, N, K}, e, ws, st);
}

hipError_t g32_nn(const float *dy, long lddy, const float *w, long ldw, float *dx, long lddx, int M,
                  int N, int K, float alpha, float beta, const GemmWs &ws, hipStream_t st) {
    Op16 a, b;
    if (!make_op32(dy, lddy, M, N, a) || !make_op32(w, ldw, N, K, b))
        return gemm_nn(Precision::FP32, matf32(dy, lddy), matf32(w, ldw), dx, lddx, M, N, K, alpha,
                       beta, st);
    EpiStore e{dx, lddx, nullptr, 0, alpha, beta};
    return run32<Lay::K, Lay::MN>(a, b, GemmShape{M, K, N}, e, ws, st);
}

hipError_t g32_tn(const float *dy, long lddy, const float *x, long ldx, float *dw, long lddw, int M,
                  int N, int K, float alpha, float beta, const GemmWs &ws, hipStream_t st) {
    Op16 a, b;
    if (!make_op32(dy, lddy, M, N, a) || !make_op32(x, ldx, M, K, b))
        return gemm_tn(Precision::FP32, matf32(dy, lddy), matf32(x, ldx), dw, lddw, M, N, K, alpha,
                       beta, st);
    EpiStore e{dw, lddw, nullptr, 0, alpha, beta};
    return run32<Lay::MN, Lay::MN>(a, b, GemmShape{N, K, M}, e, ws, st);
}

size_t g32_ws_bytes_for(int M, int N, int K) {
    const GemmShape s{M, N, K};
    return ws_for(plan32(s, ~size_t(0)), s);
}

size_t g16_ws_bytes_for(int M, int N, int K) {
    const GemmShape s{M, N, K};
    return ws_for(plan(s, ~size_t(0)), s);
}

}  // namespace vkh
