// Q/K-RMSNorm + RoPE forward on rows of the fused q|k|v projection, LPH lanes
// per (row, head) holding 8 consecutive elements each (head_dim 64 / 128 ->
// LPH 8 / 16), shared by the standalone pass (qkv_fwd8_k, k_norm.hip) and the
// QKV GEMM's epilogue (gemm16_qkv_kernel, gemm16.hpp), which run the same
// arithmetic on the same values and so give the same bits.
//
// The per-head reductions stay inside a DPP row (quad swaps, half-row and row
// mirrors, in fp64) and, for full-width RoPE at LPH = 16, the partner element
// i +- 64 sits in lane j ^ 8 of the same row (row rotate by 8).  Requires
// rotary_dim % 16 == 0 so a lane's 8 elements are all on one side of the
// rotation.
#pragma once

#include "ops.hpp"

namespace vkh {

template <int CTRL>
VKH_DEV double dpp_d(double v) {
    const long long b = __builtin_bit_cast(long long, v);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)b, CTRL, 0xf, 0xf, false);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(b >> 32), CTRL, 0xf, 0xf, false);
    return __builtin_bit_cast(double, ((long long)hi << 32) | (long long)(unsigned)lo);
}

template <int LPH>
VKH_DEV double grp_sum(double v) {
    v += dpp_d<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_d<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_d<0x141>(v);  // row_half_mirror: the other quad of the 8 lanes
    if constexpr (LPH == 16) v += dpp_d<0x140>(v);  // row_mirror: the other 8 lanes
    return v;
}

VKH_DEV void ld8(const float *p, float (&v)[8]) {
    const float4 a = reinterpret_cast<const float4 *>(p)[0];
    const float4 b = reinterpret_cast<const float4 *>(p)[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}
VKH_DEV void st8(float *p, const float (&v)[8]) {
    reinterpret_cast<float4 *>(p)[0] = make_float4(v[0], v[1], v[2], v[3]);
    reinterpret_cast<float4 *>(p)[1] = make_float4(v[4], v[5], v[6], v[7]);
}
VKH_DEV void st8(bf16 *p, const float (&v)[8]) {
    *reinterpret_cast<bf16x8 *>(p) = cvt8(v[0], v[1], v[2], v[3], v[4], v[5], v[6], v[7]);
}

struct Item8 {
    float v[8], x[8];
    float2 cs[8];
};

// RoPE geometry of lane slot j (elements 8 j .. 8 j + 7) of a head.
struct Rope8 {
    int rot_lane;   // 0: no rotation, else the table column base of the slot
    int src;        // partner slot within the head
    bool lower;     // slot below half
    int col;        // first table column of the slot
};

VKH_DEV Rope8 rope8(int j, int half) {
    Rope8 r;
    const int e0 = 8 * j;
    r.lower = e0 < half;
    r.rot_lane = e0 < 2 * half;
    r.src = r.lower ? j + half / 8 : j - half / 8;
    r.col = r.lower ? e0 : e0 - half;
    return r;
}

template <int LPH>
VKH_DEV void load8(Item8 &d, const float *vp, const float *xp, const float2 *trow, const Rope8 &rp,
                   bool valid, bool qk) {
    if (!valid) {
#pragma unroll
        for (int i = 0; i < 8; ++i) d.v[i] = d.x[i] = 0.f, d.cs[i] = make_float2(1.f, 0.f);
        return;
    }
    ld8(vp, d.v);
    if (xp) {
        ld8(xp, d.x);
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) d.x[i] = 0.f;
    }
    if (qk && rp.rot_lane) {
        const float4 *tp = reinterpret_cast<const float4 *>(trow + rp.col);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 c = tp[i];
            d.cs[2 * i] = make_float2(c.x, c.y);
            d.cs[2 * i + 1] = make_float2(c.z, c.w);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) d.cs[i] = make_float2(1.f, 0.f);
    }
}

// Partner values of a head's rotation: full-width rope at 16 lanes per head
// is a row rotate by 8; other widths shuffle from the partner lane.
template <int LPH>
VKH_DEV void partner8(const float (&v)[8], float (&pv)[8], int lane, const Rope8 &rp, int half) {
    if (LPH == 16 && half == 64) {
#pragma unroll
        for (int i = 0; i < 8; ++i) pv[i] = dpp_f<0x128>(v[i]);  // row_ror:8
    } else {
        const int src = (lane & ~(LPH - 1)) + (rp.rot_lane ? rp.src : (lane & (LPH - 1)));
#pragma unroll
        for (int i = 0; i < 8; ++i) pv[i] = __shfl(v[i], src, 64);
    }
}


// One (row, head) item: y holds this lane's 8 elements of the head (in: the
// projection; out: normalised and rotated).  qk: a q or k head of a valid row;
// is_q: a q head; cs: the row position's cos / sin for the lane's slots.  Every
// lane of the wave calls it (the reductions and the partner exchange are
// cross-lane).
template <int LPH>
VKH_DEV void qkv_fwd_item8(const QkvLayout &L, float (&y)[8], const float2 (&cs)[8], bool qk,
                           bool is_q, const float (&gq)[8], const float (&gk)[8], const Rope8 &rp,
                           int lane, int half) {
#pragma clang fp contract(off)
    if (L.qk_norm) {
        double ss = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) ss += (double)y[i] * (double)y[i];
        ss = grp_sum<LPH>(ss);
        if (qk) {
            const float ri = 1.0f / sqrtf((float)(ss / (double)L.head_dim) + L.eps);
#pragma unroll
            for (int i = 0; i < 8; ++i) y[i] = (is_q ? gq[i] : gk[i]) * ri * y[i];
        }
    }
    if (half > 0) {
        float pv[8];
        partner8<LPH>(y, pv, lane, rp, half);
        if (qk && rp.rot_lane) {
#pragma unroll
            for (int i = 0; i < 8; ++i)
                y[i] = rp.lower ? y[i] * cs[i].x - pv[i] * cs[i].y : pv[i] * cs[i].y + y[i] * cs[i].x;
        }
    }
}

}  // namespace vkh
