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
//   * Global -> LDS by DMA (buffer_load ... lds, see gemm16_tile_dma), two
//     LDS buffers, one barrier per slab: slab k+1 streams in while slab k's
//     MFMAs run.  Loads go through buffer resources: out-of-range rows and k
//     are returned as zero by the hardware range check, so edges need no
//     branches.  (gemm16_tile is the earlier register-staged form.)
//   * MN-major operands stay k-row-major in LDS and their MFMA fragments are
//     read with the transposing LDS load ds_read_b64_tr_b16 (the register-
//     staged form transposes 8x8 / 4x8 bf16 blocks in registers instead).
//   * Block ids are regrouped so each XCD (8 on MI355X, round-robin dispatch)
//     gets a contiguous band of tiles that share operand panels in its L2.
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

VKH_DEV __amdgpu_buffer_rsrc_t make_rsrc(const Op16 &o) {
    return __builtin_amdgcn_make_buffer_rsrc((void *)o.p, (short)0, (int)o.bytes, 0x00020000);
}

VKH_DEV u32x4 buf_load16(__amdgpu_buffer_rsrc_t r, unsigned off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}

// byte offset of chunk c (0..7) of LDS row r
VKH_DEV int swz(int r, int c) { return r * 128 + ((c ^ (r & 7)) << 4); }

// K-major operand: R rows x 64 k per slab, one 16-byte chunk per unit.
template <int R, int NT>
struct Ld16K {
    static constexpr int PER = R * 8 / NT;
    static_assert(PER >= 1 && (R * 8) % NT == 0, "tile / thread mismatch");
    u32x4 v[PER];
    unsigned base[PER];  // byte offset of the chunk at k = 0, or kOOB

    VKH_DEV void setup(const Op16 &o, int row0, int rmax, int tid) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int u = tid + i * NT, row = u >> 3, c = u & 7;
            const int gr = row0 + row;
            base[i] = gr < rmax ? (unsigned)(((long)gr * o.ld + c * 8) * 2) : kOOB;
        }
    }
    VKH_DEV void load(__amdgpu_buffer_rsrc_t rs, long, int k0, int kmax, int tid) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int c = (tid + i * NT) & 7;
            const bool ok = base[i] != kOOB && k0 + c * 8 < kmax;
            v[i] = buf_load16(rs, ok ? base[i] + (unsigned)k0 * 2 : kOOB);
        }
    }
    VKH_DEV void store(char *lds, int tid) const {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int u = tid + i * NT;
            *reinterpret_cast<u32x4 *>(lds + swz(u >> 3, u & 7)) = v[i];
        }
    }
};

// element j (0..7) of an 8 x bf16 chunk, as the low 16 bits
template <int J>
VKH_DEV unsigned half_of(const u32x4 &x) {
    return J & 1 ? (x[J >> 1] >> 16) : (x[J >> 1] & 0xffffu);
}

// MN-major operand: storage rows are k.  A unit is KR consecutive k rows of
// one 8-wide r chunk (KR = 8, 4 or 2, so that every thread owns whole
// units); it is transposed to 8 r rows of KR k values.
template <int R, int NT>
struct Ld16MN {
    static constexpr int KR = (64 * R / 8) / NT >= 8 ? 8 : (64 * R / 8) / NT >= 4 ? 4 : 2;
    static constexpr int KB = 64 / KR;  // k blocks per slab
    static constexpr int UNITS = KB * (R / 8);
    static constexpr int PER = UNITS / NT;
    static_assert(PER >= 1 && UNITS % NT == 0, "tile / thread mismatch");
    u32x4 v[PER][KR];
    unsigned base[PER];  // byte offset of (k = kb * KR, r chunk) at k0 = 0, or kOOB

    VKH_DEV void setup(const Op16 &o, int row0, int rmax, int tid) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int u = tid + i * NT, kb = u % KB, rb = u / KB;
            const int gr = row0 + rb * 8;
            base[i] = gr < rmax ? (unsigned)(((long)kb * KR * o.ld + gr) * 2) : kOOB;
        }
    }
    VKH_DEV void load(__amdgpu_buffer_rsrc_t rs, long ld, int k0, int kmax, int tid) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int kb = (tid + i * NT) % KB;
#pragma unroll
            for (int q = 0; q < KR; ++q) {
                const int k = k0 + kb * KR + q;
                const bool ok = base[i] != kOOB && k < kmax;
                v[i][q] = buf_load16(rs, ok ? base[i] + (unsigned)(((long)k0 + q) * ld * 2) : kOOB);
            }
        }
    }
    template <int J>
    VKH_DEV void store_row(char *lds, int i, int rb, int kb) const {
        const int r = rb * 8 + J;
        const int kpos = kb * KR;
        char *dst = lds + swz(r, kpos >> 3) + (kpos & 7) * 2;
        if constexpr (KR == 8) {
            u32x4 o;
#pragma unroll
            for (int w = 0; w < 4; ++w)
                o[w] = half_of<J>(v[i][2 * w]) | (half_of<J>(v[i][2 * w + 1]) << 16);
            *reinterpret_cast<u32x4 *>(dst) = o;
        } else if constexpr (KR == 4) {
            u32x2 o;
#pragma unroll
            for (int w = 0; w < 2; ++w)
                o[w] = half_of<J>(v[i][2 * w]) | (half_of<J>(v[i][2 * w + 1]) << 16);
            *reinterpret_cast<u32x2 *>(dst) = o;
        } else {
            *reinterpret_cast<unsigned *>(dst) = half_of<J>(v[i][0]) | (half_of<J>(v[i][1]) << 16);
        }
    }
    VKH_DEV void store(char *lds, int tid) const {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int u = tid + i * NT, kb = u % KB, rb = u / KB;
            store_row<0>(lds, i, rb, kb); store_row<1>(lds, i, rb, kb);
            store_row<2>(lds, i, rb, kb); store_row<3>(lds, i, rb, kb);
            store_row<4>(lds, i, rb, kb); store_row<5>(lds, i, rb, kb);
            store_row<6>(lds, i, rb, kb); store_row<7>(lds, i, rb, kb);
        }
    }
};

template <Lay L, int R, int NT>
struct Ld16Sel;
template <int R, int NT>
struct Ld16Sel<Lay::K, R, NT> {
    using T = Ld16K<R, NT>;
};
template <int R, int NT>
struct Ld16Sel<Lay::MN, R, NT> {
    using T = Ld16MN<R, NT>;
};

// PF = number of K slabs in flight in registers while one computes (1 or 2).
template <int BM_, int BN_, int WGM_, int WGN_, int PF_ = 1>
struct Tile16 {
    static constexpr int BM = BM_, BN = BN_, WGM = WGM_, WGN = WGN_, PF = PF_;
    static constexpr int NT = 64 * WGM * WGN;
    static constexpr int LDS = 2 * (BM + BN) * 128;
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

// One block's BM x BN output tile over the K slabs [kbase, kbase + 64 nk):
// acc (per wave, accumulator layout) += A(m0.., k) B(n0.., k).  `smem` must
// hold 2 (BM + BN) 128 bytes.  Shared by the GEMM kernels and the attention
// dQ kernel.
template <class Cfg, Lay LA, Lay LB, int TM, int TN>
VKH_DEV void gemm16_tile(const Op16 &a, const Op16 &b, int m0, int n0, int M, int N, int kbase,
                         int nk, int Kmax, f32x4 (&acc)[TM][TN], char *smem) {
    constexpr int BM = Cfg::BM, BN = Cfg::BN, NT = Cfg::NT;
    constexpr int WM = BM / Cfg::WGM, WN = BN / Cfg::WGN;
    static_assert(TM == WM / 16 && TN == WN / 16, "fragment grid");
    constexpr int ABYTES = BM * 128, BBYTES = BN * 128, STAGE = ABYTES + BBYTES;
    const int tid = threadIdx.x;
    const int lane = tid % 64, wave = __builtin_amdgcn_readfirstlane(tid / 64);
    const int wm = wave / Cfg::WGN, wn = wave % Cfg::WGN;
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(a), rb = make_rsrc(b);
    // register staging sets (the second is used only with PF == 2)
    typename Ld16Sel<LA, BM, NT>::T la0, la1;
    typename Ld16Sel<LB, BN, NT>::T lb0, lb1;
    la0.setup(a, m0, M, tid);
    lb0.setup(b, n0, N, tid);
    if constexpr (Cfg::PF == 2) {
        la1.setup(a, m0, M, tid);
        lb1.setup(b, n0, N, tid);
    }
    // per-lane fragment offsets: row fr of each 16-row group, chunk (4 ks + fg)
    const int fr = lane % 16, fg = lane / 16;
    const int sw = fg ^ (fr & 7);
    const int a_lane = (wm * WM + fr) * 128, b_lane = (wn * WN + fr) * 128;

    auto compute = [&](const char *sa) {
        const char *sb = sa + ABYTES;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const int coff = (((ks << 2) ^ sw) << 4);
            bf16x8 af[TM], bfr[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i)
                af[i] = *reinterpret_cast<const bf16x8 *>(sa + a_lane + i * 16 * 128 + coff);
#pragma unroll
            for (int j = 0; j < TN; ++j)
                bfr[j] = *reinterpret_cast<const bf16x8 *>(sb + b_lane + j * 16 * 128 + coff);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) acc[i][j] = mfma16x16x32(af[i], bfr[j], acc[i][j]);
        }
    };
    char *const lds0 = smem, *const lds1 = smem + STAGE;

    if constexpr (Cfg::PF == 1) {
        la0.load(ra, a.ld, kbase, Kmax, tid);
        lb0.load(rb, b.ld, kbase, Kmax, tid);
        la0.store(lds0, tid);
        lb0.store(lds0 + ABYTES, tid);
        __syncthreads();
        for (int kt = 0; kt < nk; ++kt) {
            if (kt + 1 < nk) {
                la0.load(ra, a.ld, kbase + (kt + 1) * 64, Kmax, tid);
                lb0.load(rb, b.ld, kbase + (kt + 1) * 64, Kmax, tid);
            }
            compute(kt & 1 ? lds1 : lds0);
            if (kt + 1 < nk) {
                char *nxt = kt & 1 ? lds0 : lds1;
                la0.store(nxt, tid);
                lb0.store(nxt + ABYTES, tid);
            }
            __syncthreads();
        }
    } else {
        // Invariant at an even step kt: lds0 holds slab kt, set 1 holds slab
        // kt+1 and set 0 slab kt+2 (both in flight); odd steps swap roles.
        la0.load(ra, a.ld, kbase, Kmax, tid);
        lb0.load(rb, b.ld, kbase, Kmax, tid);
        if (nk > 1) {
            la1.load(ra, a.ld, kbase + 64, Kmax, tid);
            lb1.load(rb, b.ld, kbase + 64, Kmax, tid);
        }
        la0.store(lds0, tid);
        lb0.store(lds0 + ABYTES, tid);
        if (nk > 2) {
            la0.load(ra, a.ld, kbase + 128, Kmax, tid);
            lb0.load(rb, b.ld, kbase + 128, Kmax, tid);
        }
        __syncthreads();
        for (int kt = 0; kt < nk; kt += 2) {
            compute(lds0);
            if (kt + 1 < nk) {
                la1.store(lds1, tid);
                lb1.store(lds1 + ABYTES, tid);
            }
            if (kt + 3 < nk) {
                la1.load(ra, a.ld, kbase + (kt + 3) * 64, Kmax, tid);
                lb1.load(rb, b.ld, kbase + (kt + 3) * 64, Kmax, tid);
            }
            __syncthreads();
            if (kt + 1 >= nk) break;
            compute(lds1);
            if (kt + 2 < nk) {
                la0.store(lds0, tid);
                lb0.store(lds0 + ABYTES, tid);
            }
            if (kt + 4 < nk) {
                la0.load(ra, a.ld, kbase + (kt + 4) * 64, Kmax, tid);
                lb0.load(rb, b.ld, kbase + (kt + 4) * 64, Kmax, tid);
            }
            __syncthreads();
        }
    }

}

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

VKH_DEV void dma16(__amdgpu_buffer_rsrc_t rs, char *lds_wave_base, unsigned voff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_t *)lds_wave_base, 16, voff, 0, 0, 0);
}

// Issue this wave's share of one slab of an operand tile (R x 64).
template <Lay L, int R, int NW>
VKH_DEV void dma_tile(__amdgpu_buffer_rsrc_t rs, const Op16 &o, char *tile, int r0, int rmax, int k0,
                      int kmax, int wave, int lane) {
    constexpr int PW = R / 8 / NW;  // 1 KB instructions per wave
    static_assert(PW >= 1 && PW * NW * 8 == R, "tile / wave mismatch");
#pragma unroll
    for (int j = 0; j < PW; ++j) {
        const int ins = wave * PW + j;
        char *dst = tile + ins * 1024;
        unsigned off;
        if constexpr (L == Lay::K) {
            const int r = ins * 8 + lane / 8, c = (lane % 8) ^ ((lane / 8) & 7);
            const int gr = r0 + r, gk = k0 + 8 * c;
            off = (gr < rmax && gk < kmax) ? (unsigned)(((long)gr * o.ld + gk) * 2) : kOOB;
        } else {
            constexpr int CPR = R / 8;        // 16-byte chunks per k row
        static_assert(R == 64 || R % 128 == 0, "MN tile width");
            constexpr int RPI = 64 / CPR;     // k rows per instruction
            const int k = ins * RPI + lane / CPR, pch = lane % CPR;
            const int c = pch ^ mn_swz<R>(k);
            const int gk = k0 + k, gm = r0 + 8 * c;
            off = (gk < kmax && gm < rmax) ? (unsigned)(((long)gk * o.ld + gm) * 2) : kOOB;
        }
        dma16(rs, dst, off);
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

VKH_DEV void wait_vm0() { __builtin_amdgcn_s_waitcnt(0x0f70); }  // vmcnt(0), exp/lgkm untouched

template <class Cfg, Lay LA, Lay LB, int TM, int TN>
VKH_DEV void gemm16_tile_dma(const Op16 &a, const Op16 &b, int m0, int n0, int M, int N, int kbase,
                             int nk, int Kmax, f32x4 (&acc)[TM][TN], char *smem) {
    constexpr int BM = Cfg::BM, BN = Cfg::BN, NW = Cfg::WGM * Cfg::WGN;
    constexpr int WM = BM / Cfg::WGM, WN = BN / Cfg::WGN;
    static_assert(TM == WM / 16 && TN == WN / 16, "fragment grid");
    constexpr int ABYTES = BM * 128, BBYTES = BN * 128, STAGE = ABYTES + BBYTES;
    const int lane = threadIdx.x % 64, wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const int wm = wave / Cfg::WGN, wn = wave % Cfg::WGN;
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(a), rb = make_rsrc(b);
    auto issue = [&](int kt, char *stage) {
        dma_tile<LA, BM, NW>(ra, a, stage, m0, M, kbase + kt * 64, Kmax, wave, lane);
        dma_tile<LB, BN, NW>(rb, b, stage + ABYTES, n0, N, kbase + kt * 64, Kmax, wave, lane);
    };
    if (nk > 0) issue(0, smem);
    for (int kt = 0; kt < nk; ++kt) {
        char *cur = smem + (kt & 1) * STAGE;
        wait_vm0();
        __syncthreads();  // slab kt landed for every wave; slab kt-1's buffer is free
        if (kt + 1 < nk) issue(kt + 1, smem + ((kt + 1) & 1) * STAGE);
        // Both k-steps' fragments are requested before the first MFMA, so the
        // LDS latency of the second set hides behind the first set's MFMAs.
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
    __syncthreads();  // the caller may reuse smem
}

template <class Cfg, Lay LA, Lay LB, class Epi>
__global__ __launch_bounds__(Cfg::NT, 1) void gemm16_kernel(Op16 a, Op16 b, GemmShape s, Epi epi,
                                                            SplitK sk) {
    constexpr int BM = Cfg::BM, BN = Cfg::BN, NT = Cfg::NT;
    constexpr int WM = BM / Cfg::WGM, WN = BN / Cfg::WGN;
    constexpr int TM = WM / 16, TN = WN / 16;
    __shared__ __attribute__((aligned(16))) char smem[2 * (BM + BN) * 128];

    const int tid = threadIdx.x;
    const int lane = tid % 64, wave = tid / 64;
    const int wm = wave / Cfg::WGN, wn = wave % Cfg::WGN;

    const int nbm = (s.M + BM - 1) / BM, nbn = (s.N + BN - 1) / BN;
    const int nb = nbm * nbn * sk.splits;
    int bid = blockIdx.x;
    if (nb % 8 == 0) bid = (bid % 8) * (nb / 8) + bid / 8;
    const int split = bid % sk.splits, tile = bid / sk.splits;
    const int bm = tile % nbm, bn = tile / nbm;
    const int m0 = bm * BM, n0 = bn * BN;

    f32x4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int nk_all = (s.K + 63) / 64;
    const int kt0 = (int)((long)nk_all * split / sk.splits);
    const int nk = (int)((long)nk_all * (split + 1) / sk.splits) - kt0;
    gemm16_tile_dma<Cfg, LA, LB, TM, TN>(a, b, m0, n0, s.M, s.N, kt0 * 64, nk, s.K, acc, smem);

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

// One block per output tile: sum the split partials in order, then the epilogue.
template <class Cfg, class Epi>
__global__ __launch_bounds__(Cfg::NT) void gemm16_reduce_kernel(GemmShape s, Epi epi, SplitK sk) {
    constexpr int BM = Cfg::BM, BN = Cfg::BN, NT = Cfg::NT;
    constexpr int WM = BM / Cfg::WGM, WN = BN / Cfg::WGN;
    constexpr int TM = WM / 16, TN = WN / 16;
    constexpr int TILE4 = BM * BN / 4;
    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
    const int wm = wave / Cfg::WGN, wn = wave % Cfg::WGN;
    const int nbm = (s.M + BM - 1) / BM;
    const int tile = blockIdx.x;
    const int m0 = (tile % nbm) * BM, n0 = (tile / nbm) * BN;
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

template <class Cfg, Lay LA, Lay LB, class Epi>
hipError_t launch_gemm16(const Op16 &a, const Op16 &b, const GemmShape &s, const Epi &epi,
                         const SplitK &sk, hipStream_t st) {
    if (s.M <= 0 || s.N <= 0) return hipSuccess;
    if (sk.splits < 1 || (sk.splits > 1 && !sk.ws)) return hipErrorInvalidValue;
    const unsigned tiles = ceil_div(s.M, Cfg::BM) * ceil_div(s.N, Cfg::BN);
    hipLaunchKernelGGL((gemm16_kernel<Cfg, LA, LB, Epi>), dim3(tiles * sk.splits), dim3(Cfg::NT),
                       0, st, a, b, s, epi, sk);
    if (sk.splits > 1)
        hipLaunchKernelGGL((gemm16_reduce_kernel<Cfg, Epi>), dim3(tiles), dim3(Cfg::NT), 0, st, s,
                           epi, sk);
    return hipGetLastError();
}

}  // namespace vkh
