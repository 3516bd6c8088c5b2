// bf16-operand MFMA GEMM for gfx950:  C[m, n] = sum_k A(m, k) * B(n, k).
//
// The training step keeps every GEMM operand resident in HBM as bf16 (weight
// shadows refreshed by the Adam kernel, activation and gradient copies
// written by the kernels that produce them), so this kernel moves half the
// bytes of an fp32-operand GEMM and needs no conversion on the way in.
//
// Operand storage, as in gemm.hpp:
//   Lay::K   element (r, k) at p[r * ld + k]   (k contiguous)
//   Lay::MN  element (r, k) at p[k * ld + r]   (r contiguous)
//
// Structure:
//   * A block of NT = 64 * WGM * WGN threads owns a BM x BN tile; wave
//     (wm, wn) owns a (BM / WGM) x (BN / WGN) sub-tile of 16x16 accumulators
//     fed by v_mfma_f32_16x16x32_bf16.
//   * K advances in 64-wide slabs.  Each slab of A and B sits in LDS as rows
//     of 64 bf16 (eight 16-byte chunks); chunk c of row r is stored at chunk
//     position c ^ (r & 7), so the 16-byte fragment reads of 8 consecutive
//     lanes (8 consecutive rows, same logical chunk) and the staging writes
//     (8 chunks of one row) each touch all 32 banks exactly once.
//   * Global -> LDS by DMA (buffer_load ... lds, see gemm16_tile_dma), two or
//     three LDS buffers (Tile16::ST), one barrier per slab: the next one or
//     two slabs stream in while a slab's MFMAs run.  Loads go through buffer
//     resources: out-of-range rows and k are returned as zero by the
//     hardware range check, so edges need no branches.
//   * MN-major operands stay k-row-major in LDS and their MFMA fragments are
//     read with the transposing LDS load ds_read_b64_tr_b16.
//   * Block ids are regrouped so each XCD (8 on MI355X, round-robin dispatch)
//     gets a contiguous band of tiles, ordered in groups of a few tile rows
//     (tile_rc), so the blocks an XCD runs at one time share operand panels
//     in its L2.
#pragma once

#include "gemm.hpp"

namespace vkh {

using u32x4 = unsigned __attribute__((ext_vector_type(4)));
using u32x2 = unsigned __attribute__((ext_vector_type(2)));

// A bf16 operand: `bytes` bounds the hardware range check (< 2^31).
struct Op16 {
    const bf16 *p;
    long ld;
    unsigned bytes;
};

constexpr unsigned kOOB = 0x80000000u;  // any offset >= bytes reads as zero

// Buffer resource as four SGPR words (base, base_hi | stride 0, num_records,
// flags), the form inline assembly takes.
typedef int sgpr4 __attribute__((ext_vector_type(4)));
VKH_DEV sgpr4 rsrc4(const void *base, unsigned bytes) {
    const unsigned long a = (unsigned long)base;
    sgpr4 r;
    r[0] = __builtin_amdgcn_readfirstlane((int)(unsigned)a);
    r[1] = __builtin_amdgcn_readfirstlane((int)(unsigned)(a >> 32) & 0xffff);
    r[2] = __builtin_amdgcn_readfirstlane((int)bytes);
    r[3] = 0x00020000;
    return r;
}
VKH_DEV sgpr4 rsrc4(const Op16 &o) { return rsrc4(o.p, o.bytes); }

// ST = LDS slab buffers (2: one slab in flight while one computes; 3: two).
template <int BM_, int BN_, int WGM_, int WGN_, int ST_ = 2>
struct Tile16 {
    static constexpr int BM = BM_, BN = BN_, WGM = WGM_, WGN = WGN_, ST = ST_;
    static constexpr int NT = 64 * WGM * WGN;
    static constexpr int LDS = ST * (BM + BN) * 128;
};

// Split-K: `splits` blocks share one output tile, each contracting a
// contiguous range of 64-wide K slabs and storing its partial tile to `ws`
// in accumulator order.  gemm16_reduce_kernel then adds the partials in
// split order (0, 1, ...) and runs the epilogue, so results do not depend
// on scheduling.  (Finishing the sum in the GEMM kernel itself would need
// agent-scope release/acquire fences, which on MI355X write back and
// invalidate a whole XCD L2 per block; a kernel boundary is far cheaper.)
struct SplitK {
    int splits;
    f32x4 *ws;  // [tiles][splits][BM * BN / 4]
};

// ── DMA staging: global -> LDS without registers ─────────────────────
//
// buffer_load_dwordx4 ... lds writes lane l's 16 bytes to M0 + 16 l (the
// LDS base is wave-uniform), so one wave instruction fills 1 KB of LDS and
// the layout is chosen through each lane's global address:
//   * K-major tile (R rows x 64 k): the swizzled rows above; lane l of an
//     instruction covering rows rb..rb+7 fetches row rb + l/8, logical chunk
//     (l % 8) ^ ((l / 8) & 7).
//   * MN-major tile (64 k x R m): stored as its k rows, R m values each, with
//     16-byte chunk c of row k at position c ^ mn_swz(k); MFMA fragments are
//     read with ds_read_b64_tr_b16 (transposing), two reads per fragment.
// The loads are asynchronous: slab k+1 streams into the other LDS buffer
// while slab k computes, with no staging registers and no ds_write.

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4_t;

// Chunk permutation of MN tile row k (R m values per row).  It is even, so
// 32-byte pairs stay together, and the rows one half-wave's transposing read
// touches ({0-3, 8-11} + 4 j) land on disjoint banks: with rows of >= 256 B
// (a multiple of the 64 x 4 B bank width) the eight rows get eight values;
// with 128 B rows, even and odd rows already sit in different bank halves
// and the four rows of each parity get four values.
template <int R>
VKH_DEV int mn_swz(int k) {
    if constexpr (R >= 128) return 2 * ((k & 3) | (((k >> 3) & 1) << 2));
    else return 2 * (((k >> 1) & 1) | (((k >> 3) & 1) << 1));
}

// 16-byte global -> LDS DMA of one wave (lane l lands at lds + 16 l; the LDS
// address is wave-uniform and goes to M0).  Issued as inline assembly so the
// compiler's wait-count tracking does not treat later LDS reads as possible
// aliases of the in-flight slab (it would wait for the DMA before reading the
// current one); the slab loops wait for their DMA explicitly (vmcnt) before
// the barrier that publishes a slab.
VKH_DEV void dma16_async(const sgpr4 &rs, const void *lds, unsigned voff) {
    const unsigned m0 = __builtin_amdgcn_readfirstlane(
        (int)(unsigned)(unsigned long)(const __attribute__((address_space(3))) char *)lds);
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :
                 : "s"(m0), "v"(voff), "s"(rs)
                 : "memory");
}
VKH_DEV void dma4_async(const sgpr4 &rs, const void *lds, unsigned voff) {
    const unsigned m0 = __builtin_amdgcn_readfirstlane(
        (int)(unsigned)(unsigned long)(const __attribute__((address_space(3))) char *)lds);
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen lds"
                 :
                 : "s"(m0), "v"(voff), "s"(rs)
                 : "memory");
}

// Block barrier for LDS hand-offs: this wave's LDS operations complete, then
// s_barrier (no wait on outstanding global operations, unlike __syncthreads'
// fence).  The memory clobber keeps the compiler from moving memory accesses
// across it.
VKH_DEV void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Byte offset (into the operand) of the 16 bytes lane `lane` moves for 1 KB
// piece `ins` of an operand tile's slab (R rows x 64 k at k0); the piece
// lands at tile + 1024 ins + 16 lane.  kOOB past the edges.
// fp32 operands (ES = 4): a slab is 32 k wide, so a K-major tile row is again
// 128 bytes (eight 16-byte chunks of 4 floats, the same swizzle) and an
// MN-major tile is 32 k rows of R floats; their fragments are read one float
// per lane (frag32), so the MN swizzle only has to put the rows 4 fg + e of
// one read (fg = 0..3) on two disjoint bank halves: chunk c of row k at
// c ^ (4 ((k >> 2) & 1)).
VKH_DEV int mn_swz32(int k) { return ((k >> 2) & 1) << 2; }

template <Lay L, int R, int ES = 2>
VKH_DEV unsigned tile_off(const Op16 &o, int ins, int lane, int r0, int rmax, int k0, int kmax) {
    constexpr int EPC = 16 / ES;  // elements per 16-byte chunk
    if constexpr (L == Lay::K) {
        const int r = ins * 8 + lane / 8, c = (lane % 8) ^ ((lane / 8) & 7);
        const int gr = r0 + r, gk = k0 + EPC * c;
        return (gr < rmax && gk < kmax) ? (unsigned)(((long)gr * o.ld + gk) * ES) : kOOB;
    } else {
        constexpr int CPR = R / EPC;      // 16-byte chunks per k row
        static_assert(ES == 4 || R == 64 || R % 128 == 0, "MN tile width");
        static_assert(CPR <= 64 && 64 % CPR == 0, "MN rows per instruction");
        constexpr int RPI = 64 / CPR;     // k rows per instruction
        const int k = ins * RPI + lane / CPR, pch = lane % CPR;
        const int c = pch ^ (ES == 2 ? mn_swz<R>(k) : mn_swz32(k));
        const int gk = k0 + k, gm = r0 + EPC * c;
        return (gk < kmax && gm < rmax) ? (unsigned)(((long)gk * o.ld + gm) * ES) : kOOB;
    }
}

// Issue this wave's share of one slab of an operand tile (R x 64).
template <Lay L, int R, int NW, int ES = 2>
VKH_DEV void dma_tile(const sgpr4 &rs, const Op16 &o, char *tile, int r0, int rmax, int k0,
                      int kmax, int wave, int lane) {
    constexpr int PW = R / 8 / NW;  // 1 KB instructions per wave (a slab is 128 R bytes)
    static_assert(PW >= 1 && PW * NW * 8 == R, "tile / wave mismatch");
#pragma unroll
    for (int j = 0; j < PW; ++j) {
        const int ins = wave * PW + j;
        dma16_async(rs, tile + ins * 1024, tile_off<L, R, ES>(o, ins, lane, r0, rmax, k0, kmax));
    }
}

// Fragment (16 rows of the operand x 32 k at k-step ks) for this lane.
template <Lay L, int R>
VKH_DEV bf16x8 frag16(const char *tile, int row16, int ks, int lane) {
    const int fr = lane % 16, fg = lane / 16;
    if constexpr (L == Lay::K) {
        const int r = row16 + fr;
        return *reinterpret_cast<const bf16x8 *>(tile + r * 128 + ((((ks << 2) + fg) ^ (r & 7)) << 4));
    } else {
        // lane (fg, fr) addresses k row 32 ks + 8 fg + fr / 4 (+4), m = row16 + 4 (fr % 4)
        const int m = row16 + 4 * (fr % 4);
        const int k_lo = 32 * ks + 8 * fg + fr / 4, k_hi = k_lo + 4;
        const char *plo = tile + k_lo * (R * 2) + (((m >> 3) ^ mn_swz<R>(k_lo)) << 4) + (m & 7) * 2;
        const char *phi = tile + k_hi * (R * 2) + (((m >> 3) ^ mn_swz<R>(k_hi)) << 4) + (m & 7) * 2;
        const bf16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4_t *)plo);
        const bf16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4_t *)phi);
        return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    }
}

// fp32 fragment for v_mfma_f32_16x16x4_f32 at k-step ks (16 k): lane (fg, fr)
// holds operand row row16 + fr at k = 16 ks + 4 fg + e in element e, the
// contraction index of MFMA step e (the same index for both operands).
template <Lay L, int R>
VKH_DEV f32x4 frag32(const char *tile, int row16, int ks, int lane) {
    const int fr = lane % 16, fg = lane / 16;
    if constexpr (L == Lay::K) {
        const int r = row16 + fr;
        return *reinterpret_cast<const f32x4 *>(tile + r * 128 + ((((ks << 2) + fg) ^ (r & 7)) << 4));
    } else {
        const int m = row16 + fr;
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int k = 16 * ks + 4 * fg + e;
            v[e] = *reinterpret_cast<const float *>(tile + k * (R * 4) + (((m >> 2) ^ mn_swz32(k)) << 4) +
                                                    (m & 3) * 4);
        }
        return v;
    }
}

VKH_DEV void wait_vm0() { __builtin_amdgcn_s_waitcnt(0x0f70); }  // vmcnt(0), exp/lgkm untouched

// One block's BM x BN output tile over the K slabs [kbase, kbase + KW nk)
// (KW = 64 bf16 or, with F32, 32 fp32 values: 128-byte tile rows either way):
// acc (per wave, accumulator layout) += A(m0.., k) B(n0.., k).  `smem` must
// hold Cfg::LDS bytes.  Shared by the GEMM kernels and the attention dQ kernel.
// `wave` is the wave's index among the Cfg::WGM x Cfg::WGN waves that share
// this tile (-1: threadIdx.x / 64, the whole block).  Every wave of the
// workgroup must run the same number of slabs: the routine's barriers are
// workgroup-wide.
// DUALB: the B tile is two halves of BN / 2 operand rows, n0.. and bsplit + n0..
// (the gate and up rows of one feature range for the fused SwiGLU epilogue).
template <class Cfg, Lay LA, Lay LB, int TM, int TN, bool F32 = false, bool DUALB = false>
VKH_DEV void gemm16_tile_dma(const Op16 &a, const Op16 &b, int m0, int n0, int M, int N, int kbase,
                             int nk, int Kmax, f32x4 (&acc)[TM][TN], char *smem, int wave_in = -1,
                             int bsplit = 0) {
    constexpr int KW = F32 ? 32 : 64, ES = F32 ? 4 : 2;
    constexpr int BM = Cfg::BM, BN = Cfg::BN, NW = Cfg::WGM * Cfg::WGN, ST = Cfg::ST;
    constexpr int WM = BM / Cfg::WGM, WN = BN / Cfg::WGN;
    static_assert(TM == WM / 16 && TN == WN / 16, "fragment grid");
    static_assert(ST == 2 || ST == 3, "slab buffers");
    constexpr int ABYTES = BM * 128, BBYTES = BN * 128, STAGE = ABYTES + BBYTES;
    // DMA instructions one wave issues per slab (the newest slab's count)
    constexpr int PER_SLAB = BM / 8 / NW + BN / 8 / NW;
    static_assert(PER_SLAB <= 15, "vmcnt immediate");
    const int lane = threadIdx.x % 64;
    const int wave = __builtin_amdgcn_readfirstlane(wave_in < 0 ? (int)threadIdx.x / 64 : wave_in);
    const int wm = wave / Cfg::WGN, wn = wave % Cfg::WGN;
    const sgpr4 ra = rsrc4(a), rb = rsrc4(b);
    auto issue = [&](int kt) {
        char *stage = smem + (kt % ST) * STAGE;
        dma_tile<LA, BM, NW, ES>(ra, a, stage, m0, M, kbase + kt * KW, Kmax, wave, lane);
        if constexpr (DUALB) {
            dma_tile<LB, BN / 2, NW, ES>(rb, b, stage + ABYTES, n0, N, kbase + kt * KW, Kmax, wave, lane);
            dma_tile<LB, BN / 2, NW, ES>(rb, b, stage + ABYTES + BN / 2 * 128, bsplit + n0, N,
                                         kbase + kt * KW, Kmax, wave, lane);
        } else {
            dma_tile<LB, BN, NW, ES>(rb, b, stage + ABYTES, n0, N, kbase + kt * KW, Kmax, wave, lane);
        }
    };
    // ST - 1 slabs in flight ahead of the one computing
    for (int j = 0; j < ST - 1 && j < nk; ++j) issue(j);
    for (int kt = 0; kt < nk; ++kt) {
        const char *cur = smem + (kt % ST) * STAGE;
        // slab kt is this wave's oldest outstanding DMA batch: with a newer
        // batch in flight, wait until only that one remains
        if (ST == 3 && kt + 1 < nk) __builtin_amdgcn_s_waitcnt(0x0f70 | PER_SLAB);
        else wait_vm0();
        lds_barrier();  // slab kt landed for every wave; slab kt-1's buffer is free
        if (kt + ST - 1 < nk) issue(kt + ST - 1);
        // Both k-steps' fragments are requested before the first MFMA, so the
        // LDS latency of the second set hides behind the first set's MFMAs.
        if constexpr (F32) {
            f32x4 af[2][TM], bfr[2][TN];
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
                for (int i = 0; i < TM; ++i) af[ks][i] = frag32<LA, BM>(cur, wm * WM + 16 * i, ks, lane);
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    bfr[ks][j] = frag32<LB, BN>(cur + ABYTES, wn * WN + 16 * j, ks, lane);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int ks = 0; ks < 2; ++ks)
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            acc[i][j] = mfma16x16x4(af[ks][i][e], bfr[ks][j][e], acc[i][j]);
            continue;
        }
        bf16x8 af[2][TM], bfr[2][TN];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
            for (int i = 0; i < TM; ++i) af[ks][i] = frag16<LA, BM>(cur, wm * WM + 16 * i, ks, lane);
#pragma unroll
            for (int j = 0; j < TN; ++j)
                bfr[ks][j] = frag16<LB, BN>(cur + ABYTES, wn * WN + 16 * j, ks, lane);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) acc[i][j] = mfma16x16x32(af[ks][i], bfr[ks][j], acc[i][j]);
    }
    lds_barrier();  // the caller may reuse smem
}

template <class Cfg, Lay LA, Lay LB, class Epi, bool F32 = false>
__global__ __launch_bounds__(Cfg::NT, 1) void gemm16_kernel(Op16 a, Op16 b, GemmShape s, Epi epi,
                                                            SplitK sk, int tgrp) {
    constexpr int BM = Cfg::BM, BN = Cfg::BN, NT = Cfg::NT;
    constexpr int WM = BM / Cfg::WGM, WN = BN / Cfg::WGN;
    constexpr int TM = WM / 16, TN = WN / 16;
    __shared__ __attribute__((aligned(16))) char smem[Cfg::LDS];

    const int tid = threadIdx.x;
    const int lane = tid % 64, wave = tid / 64;
    const int wm = wave / Cfg::WGN, wn = wave % Cfg::WGN;

    const int nbm = (s.M + BM - 1) / BM, nbn = (s.N + BN - 1) / BN;
    const int nb = nbm * nbn * sk.splits;
    int bid = blockIdx.x;
    if (nb % 8 == 0) bid = (bid % 8) * (nb / 8) + bid / 8;
    const int split = bid % sk.splits, tile = bid / sk.splits;
    int bm, bn;
    tile_rc(tile, nbm, nbn, tgrp, bm, bn);
    const int m0 = bm * BM, n0 = bn * BN;

    f32x4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    constexpr int KW = F32 ? 32 : 64;  // k per slab
    const int nk_all = (s.K + KW - 1) / KW;
    const int kt0 = (int)((long)nk_all * split / sk.splits);
    const int nk = (int)((long)nk_all * (split + 1) / sk.splits) - kt0;
    gemm16_tile_dma<Cfg, LA, LB, TM, TN, F32>(a, b, m0, n0, s.M, s.N, kt0 * KW, nk, s.K, acc, smem);

    if (sk.splits > 1) {
        f32x4 *own = sk.ws + ((size_t)tile * sk.splits + split) * (BM * BN / 4);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) own[(i * TN + j) * NT + tid] = acc[i][j];
        return;
    }
    FragPos fp{m0 + wm * WM, n0 + wn * WN, lane};
    epi.template apply<TM, TN>(acc, fp, s);
}

// Two wave groups per block on one output tile (split-K inside the block):
// group 0 runs the first half of the K slabs, group 1 the second (padded with
// zero-filled slabs so both run the same count), each in its own LDS region;
// group 1 then hands its accumulators over through LDS and group 0 adds them
// (first half + second half, a fixed order) and runs the epilogue.  For
// shapes with too few tiles to fill the chip this doubles the waves per CU
// without the partial round trip and the second launch of split-K.
template <class Cfg, Lay LA, Lay LB, class Epi, bool F32 = false>
__global__ __launch_bounds__(2 * Cfg::NT, 1) void gemm16_ks2_kernel(Op16 a, Op16 b, GemmShape s,
                                                                   Epi epi, int tgrp) {
    constexpr int BM = Cfg::BM, BN = Cfg::BN, NT = Cfg::NT;
    constexpr int WM = BM / Cfg::WGM, WN = BN / Cfg::WGN;
    constexpr int TM = WM / 16, TN = WN / 16;
    static_assert(BM * BN * 4 <= Cfg::LDS, "hand-over buffer");
    __shared__ __attribute__((aligned(16))) char smem[2 * Cfg::LDS];

    const int tid = threadIdx.x, grp = tid / NT, gt = tid % NT;
    const int lane = gt % 64, wave = gt / 64;
    const int wm = wave / Cfg::WGN, wn = wave % Cfg::WGN;

    const int nbm = (s.M + BM - 1) / BM, nbn = (s.N + BN - 1) / BN;
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

    constexpr int KW = F32 ? 32 : 64;
    const int nkh = ((s.K + KW - 1) / KW + 1) / 2;
    gemm16_tile_dma<Cfg, LA, LB, TM, TN, F32>(a, b, m0, n0, s.M, s.N, grp * nkh * KW, nkh, s.K, acc,
                                         smem + grp * Cfg::LDS, wave);
    f32x4 *hand = reinterpret_cast<f32x4 *>(smem);  // both groups are past their last slab
    if (grp == 1) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) hand[(i * TN + j) * NT + gt] = acc[i][j];
    }
    lds_barrier();
    if (grp == 1) return;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] += hand[(i * TN + j) * NT + gt];
    FragPos fp{m0 + wm * WM, n0 + wn * WN, lane};
    epi.template apply<TM, TN>(acc, fp, s);
}

template <class Cfg, Lay LA, Lay LB, class Epi, bool F32 = false>
hipError_t launch_gemm16_ks2(const Op16 &a, const Op16 &b, const GemmShape &s, const Epi &epi,
                             int tgrp, hipStream_t st) {
    if (s.M <= 0 || s.N <= 0) return hipSuccess;
    const unsigned tiles = ceil_div(s.M, Cfg::BM) * ceil_div(s.N, Cfg::BN);
    hipLaunchKernelGGL((gemm16_ks2_kernel<Cfg, LA, LB, Epi, F32>), dim3(tiles), dim3(2 * Cfg::NT), 0, st,
                       a, b, s, epi, tgrp);
    return hipGetLastError();
}

// The gate/up projection with the SwiGLU forward in its epilogue: a block
// computes 128 tokens x (64 gate features f0.. and the same 64 up features,
// the B rows f0.. and F + f0.. of the stacked [2F, K] weight), so both halves
// of every SwiGLU input are in one block.  Each wave stores its fp32
// pre-activations (gu[:, f] and gu[:, F + f], the backward's inputs); the up
// waves hand their accumulators to the gate waves of the same rows and
// features through the idle slab buffers, which write gated = swiglu1(gate,
// up) in TO (bf16; fp32 in the fp32 slab mode, F32).  One pass instead of the
// GEMM plus a SwiGLU pass that reads the whole gu back.
template <class Cfg, bool F32 = false, typename TO = bf16>
__global__ __launch_bounds__(Cfg::NT, 1) void gemm16_swiglu_kernel(Op16 a, Op16 b, int M, int F, int K,
                                                                  float *gu, long ldgu, TO *gated,
                                                                  long ldg, int tgrp) {
    constexpr int BM = Cfg::BM, BN = Cfg::BN, WGN = Cfg::WGN;
    constexpr int WM = BM / Cfg::WGM, WN = BN / WGN;
    constexpr int TM = WM / 16, TN = WN / 16;
    static_assert(WGN % 2 == 0, "gate and up wave columns");
    static_assert(Cfg::WGM * (WGN / 2) * TM * TN * 64 * 16 <= Cfg::LDS, "hand-over buffer");
    __shared__ __attribute__((aligned(16))) char smem[Cfg::LDS];
    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
    const int wm = wave / WGN, wn = wave % WGN;
    const int nbm = (M + BM - 1) / BM, nbn = F / (BN / 2);
    const int nb = nbm * nbn;
    int bid = blockIdx.x;
    if (nb % 8 == 0) bid = (bid % 8) * (nb / 8) + bid / 8;
    int bm, bn;
    tile_rc(bid, nbm, nbn, tgrp, bm, bn);
    const int m0 = bm * BM, f0 = bn * (BN / 2);
    f32x4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    constexpr int KW = F32 ? 32 : 64;  // k per slab
    gemm16_tile_dma<Cfg, Lay::K, Lay::K, TM, TN, F32, true>(a, b, m0, f0, M, 2 * F, 0,
                                                            (K + KW - 1) / KW, K, acc, smem, -1, F);
    const bool up = wn >= WGN / 2;
    const int ws = wm * (WGN / 2) + (up ? wn - WGN / 2 : wn);  // gate / up wave pair
    const int fw = f0 + (ws % (WGN / 2)) * WN;                 // feature of the wave's column 0
    const int g = lane / 16, c = lane % 16;
    float *dst = gu + (up ? F : 0);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = m0 + wm * WM + 16 * i + 4 * g + r;
                if (row < M) dst[(long)row * ldgu + fw + 16 * j + c] = acc[i][j][r];
            }
    f32x4 *xs = reinterpret_cast<f32x4 *>(smem);  // the slab loop ended with a barrier
    if (up) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) xs[((ws * TM + i) * TN + j) * 64 + lane] = acc[i][j];
    }
    lds_barrier();
    if (up) return;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const f32x4 u = xs[((ws * TM + i) * TN + j) * 64 + lane];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = m0 + wm * WM + 16 * i + 4 * g + r;
                if (row < M) gated[(long)row * ldg + fw + 16 * j + c] = (TO)swiglu1(acc[i][j][r], u[r]);
            }
        }
}

// One block per output tile: sum the split partials in order, then the epilogue.
template <class Cfg, class Epi>
__global__ __launch_bounds__(Cfg::NT) void gemm16_reduce_kernel(GemmShape s, Epi epi, SplitK sk,
                                                                int tgrp) {
    constexpr int BM = Cfg::BM, BN = Cfg::BN, NT = Cfg::NT;
    constexpr int WM = BM / Cfg::WGM, WN = BN / Cfg::WGN;
    constexpr int TM = WM / 16, TN = WN / 16;
    constexpr int TILE4 = BM * BN / 4;
    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
    const int wm = wave / Cfg::WGN, wn = wave % Cfg::WGN;
    const int nbm = (s.M + BM - 1) / BM, nbn = (s.N + BN - 1) / BN;
    const int tile = blockIdx.x;
    int bm, bn;
    tile_rc(tile, nbm, nbn, tgrp, bm, bn);
    const int m0 = bm * BM, n0 = bn * BN;
    const f32x4 *parts = sk.ws + (size_t)tile * sk.splits * TILE4;
    f32x4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int e = (i * TN + j) * NT + tid;
            f32x4 sum = parts[e];
            for (int q = 1; q < sk.splits; ++q) sum += parts[(size_t)q * TILE4 + e];
            acc[i][j] = sum;
        }
    FragPos fp{m0 + wm * WM, n0 + wn * WN, lane};
    epi.template apply<TM, TN>(acc, fp, s);
}

template <class Cfg>
size_t gemm16_ws_bytes(const GemmShape &s, int splits) {
    if (splits <= 1) return 0;
    return (size_t)ceil_div(s.M, Cfg::BM) * ceil_div(s.N, Cfg::BN) * splits * Cfg::BM * Cfg::BN * 4;
}

template <class Cfg, Lay LA, Lay LB, class Epi, bool F32 = false>
hipError_t launch_gemm16(const Op16 &a, const Op16 &b, const GemmShape &s, const Epi &epi,
                         const SplitK &sk, int tgrp, hipStream_t st) {
    if (s.M <= 0 || s.N <= 0) return hipSuccess;
    if (sk.splits < 1 || (sk.splits > 1 && !sk.ws)) return hipErrorInvalidValue;
    const unsigned tiles = ceil_div(s.M, Cfg::BM) * ceil_div(s.N, Cfg::BN);
    hipLaunchKernelGGL((gemm16_kernel<Cfg, LA, LB, Epi, F32>), dim3(tiles * sk.splits), dim3(Cfg::NT),
                       0, st, a, b, s, epi, sk, tgrp);
    if (sk.splits > 1)
        hipLaunchKernelGGL((gemm16_reduce_kernel<Cfg, Epi>), dim3(tiles), dim3(Cfg::NT), 0, st, s,
                           epi, sk, tgrp);
    return hipGetLastError();
}

}  // namespace vkh
