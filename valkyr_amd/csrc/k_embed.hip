// Embedding backward: dE[tok] (+)= sum of dy rows of the positions holding
// `tok`, summed in position order.
//
// Reference: shaders/embedding_backward.comp (one workgroup per vocab row,
// each scanning all n_pos ids: V * n_pos id reads) and the CPU oracle
// train_transformer.zig:351-366 (sequential scatter-add).  Here one workgroup
// per position p scans the ids (4 bytes each, L2-resident): if an earlier
// position holds the same id, p is not the id's owner and the workgroup
// exits; the owner (first position of its id) collects the positions holding
// the id in order (wave ballots compacted through LDS), sums their dy rows
// with plain fp32 adds in that order and writes (or adds to) the output row
// once.  The scatter targets are exact and the sums round exactly like the
// oracle's, so the result is bit-identical to it; no sort, no atomics, no
// work buffer.  embed_own2_k (below) is the form launched wherever rows and
// ids are 16-byte aligned and dim <= 4096.
#include "ops.hpp"
#include "adam.hpp"

namespace vkh {

namespace {

constexpr int EO_NT = 256;

template <bool VEC, bool ADAM>
__global__ __launch_bounds__(EO_NT) void embed_own_k(const float *dy, const uint32_t *ids, int n,
                                                      int dim, float *out, int vocab,
                                                      int accumulate, EmbedAdam ea) {
    __shared__ uint64_t masks[EO_NT / 64];
    __shared__ uint16_t list[kEmbedBwMaxPos];
    const int p = blockIdx.x, lane = threadIdx.x % 64, w = threadIdx.x / 64;
    const uint32_t tok = ids[p];
    if (tok >= (uint32_t)vocab) return;  // uniform over the block
    // an earlier position with the same id owns it
    int dup = 0;
    for (int i = threadIdx.x; i < p; i += EO_NT) dup |= ids[i] == tok;
    if (__syncthreads_or(dup)) return;
    // positions >= p holding tok, in order
    int cnt = 0;  // identical in every thread
    for (int i0 = p; i0 < n; i0 += EO_NT) {
        const int i = i0 + (int)threadIdx.x;
        const bool m = i < n && ids[i] == tok;
        const uint64_t bal = __ballot(m);
        if (lane == 0) masks[w] = bal;
        __syncthreads();
        int before = 0, total = 0;
#pragma unroll
        for (int k = 0; k < EO_NT / 64; ++k) {
            const int c = __popcll(masks[k]);
            before += k < w ? c : 0;
            total += c;
        }
        if (m) list[cnt + before + __popcll(bal & ((1ull << lane) - 1))] = (uint16_t)i;
        cnt += total;
        __syncthreads();
    }
    float *orow = out + (size_t)tok * dim;
    if (VEC) {
        for (int c = threadIdx.x; c < dim / 4; c += EO_NT) {
            float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
            for (int k = 0; k < cnt; ++k) {
                const float4 v = reinterpret_cast<const float4 *>(dy + (size_t)list[k] * dim)[c];
                acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
            }
            if (accumulate) {
                const float4 o = reinterpret_cast<float4 *>(orow)[c];
                acc = make_float4(o.x + acc.x, o.y + acc.y, o.z + acc.z, o.w + acc.w);
            }
            reinterpret_cast<float4 *>(orow)[c] = acc;
            if constexpr (ADAM) {  // the row's gradient is final: its Adam update
                const size_t j = (size_t)tok * (dim / 4) + c;
                f32x4 *p = reinterpret_cast<f32x4 *>(ea.p), *m = reinterpret_cast<f32x4 *>(ea.m),
                      *v = reinterpret_cast<f32x4 *>(ea.v);
                f32x4 pp = p[j], mm = m[j], vv = v[j];
                adam4(pp, f32x4{acc.x, acc.y, acc.z, acc.w}, mm, vv, ea.h);
                p[j] = pp;
                m[j] = mm;
                v[j] = vv;
                if (ea.pb) {
                    bf16x4 b;
                    b[0] = (bf16)pp.x; b[1] = (bf16)pp.y; b[2] = (bf16)pp.z; b[3] = (bf16)pp.w;
                    reinterpret_cast<bf16x4 *>(ea.pb)[j] = b;
                }
            }
        }
    } else {
        for (int c = threadIdx.x; c < dim; c += EO_NT) {
            float acc = 0.f;
            for (int k = 0; k < cnt; ++k) acc += dy[(size_t)list[k] * dim + c];
            orow[c] = accumulate ? orow[c] + acc : acc;
        }
    }
}

// The same owner rule and summation order with the ids read once per chunk
// of 2048 positions: thread t loads ids base + 8 t .. + 7 (two 16-byte
// loads), which settles both the duplicate test (an equal id before p) and
// the thread's matches (equal ids from p on); a wave prefix scan of the match
// counts puts the matching positions into an ordered list of at most 2048
// entries (4 KB of LDS, so occupancy is not bounded by the list), and the
// owner adds their dy rows in that order.  Each thread owns float4 column
// chunks tid + 256 j (dim <= 4096), kept in registers across the chunks.
// Where no other position of a chunk holds the id (every position of a
// batch of distinct ids), the one barrier of the duplicate test also says
// so, and the chunk's list is p alone: no scan, no list, no further barrier.
constexpr int EO_CH = 8 * EO_NT;  // positions per chunk
template <bool ADAM>
__global__ __launch_bounds__(EO_NT) void embed_own2_k(const float *dy, const uint32_t *ids, int n,
                                                       int dim, float *out, int vocab,
                                                       int accumulate, EmbedAdam ea) {
    __shared__ uint16_t list[EO_CH];
    __shared__ int wtot[EO_NT / 64];
    __shared__ int wflag[2][EO_NT / 64];
    const int p = blockIdx.x, t = threadIdx.x, lane = t % 64, w = t / 64;
    const uint32_t tok = ids[p];
    if (tok >= (uint32_t)vocab) return;  // uniform over the block
    const int d4 = dim / 4;
    // issued before the id scan: the rows an owner needs whatever the scan
    // finds (its own dy row, the output row, and its Adam state), so the scan
    // and these loads overlap; p is the first entry of its own list
    float4 own[4], orow_in[4];
    f32x4 pin[4], min_[4], vin[4];
    const float4 *dyp = reinterpret_cast<const float4 *>(dy + (size_t)p * dim);
    const float4 *orow_c = reinterpret_cast<const float4 *>(out + (size_t)tok * dim);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int cc = t + EO_NT * j;
        if (cc < d4) {
            own[j] = dyp[cc];
            if (accumulate) orow_in[j] = orow_c[cc];
            if constexpr (ADAM) {
                const size_t jj = (size_t)tok * d4 + cc;
                pin[j] = reinterpret_cast<const f32x4 *>(ea.p)[jj];
                min_[j] = reinterpret_cast<const f32x4 *>(ea.m)[jj];
                vin[j] = reinterpret_cast<const f32x4 *>(ea.v)[jj];
            }
        }
    }
    float4 acc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int base = 0; base < n; base += EO_CH) {
        const int i0 = base + 8 * t;
        uint32_t id[8];
        if (i0 + 8 <= n) {
            const uint4 a = *reinterpret_cast<const uint4 *>(ids + i0);
            const uint4 b = *reinterpret_cast<const uint4 *>(ids + i0 + 4);
            id[0] = a.x; id[1] = a.y; id[2] = a.z; id[3] = a.w;
            id[4] = b.x; id[5] = b.y; id[6] = b.z; id[7] = b.w;
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) id[j] = i0 + j < n ? ids[i0 + j] : 0xffffffffu;
        }
        int dup = 0;
        unsigned mb = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const bool eq = id[j] == tok;
            dup |= eq && i0 + j < p;
            mb |= (eq && i0 + j >= p) ? 1u << j : 0u;
        }
        // one barrier answers both block-wide questions: does an earlier
        // position hold tok (bit 0), and does a position of this chunk other
        // than p (bit 1); the flags alternate between two slots by chunk
        const unsigned other = mb & ~(p >= i0 && p < i0 + 8 ? 1u << (p - i0) : 0u);
        const int par = (base / EO_CH) & 1;
        const bool any_dup = __ballot(dup) != 0, any_other = __ballot(other != 0) != 0;
        if (lane == 0) wflag[par][w] = (any_dup ? 1 : 0) | (any_other ? 2 : 0);
        __syncthreads();
        int fl = 0;
#pragma unroll
        for (int k = 0; k < EO_NT / 64; ++k) fl |= wflag[par][k];
        if (fl & 1) return;              // an earlier position owns tok
        if (base + EO_CH <= p) continue;  // this chunk holds no position >= p
        if (!(fl & 2)) {
            // no other position of the chunk holds tok: its list would be p
            // alone (p in this chunk) or empty, so neither list nor scan
            if (p >= base) {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if (t + EO_NT * j < d4) {
                        acc[j].x += own[j].x; acc[j].y += own[j].y;
                        acc[j].z += own[j].z; acc[j].w += own[j].w;
                    }
            }
            continue;
        }
        // wave-inclusive prefix of the match counts, then the block offsets
        const int c = __popc(mb);
        int x = c;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int y = __shfl_up(x, o);
            if (lane >= o) x += y;
        }
        if (lane == 63) wtot[w] = x;
        __syncthreads();
        int off = 0, tot = 0;
#pragma unroll
        for (int k = 0; k < EO_NT / 64; ++k) {
            off += k < w ? wtot[k] : 0;
            tot += wtot[k];
        }
        int e = off + x - c;
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (mb >> j & 1u) list[e++] = (uint16_t)(8 * t + j);
        __syncthreads();
        for (int k = 0; k < tot; ++k) {
            const int pos = base + list[k];  // block-uniform
            float4 v[4];
            if (pos == p) {
#pragma unroll
                for (int j = 0; j < 4; ++j) v[j] = own[j];
            } else {
                const float4 *row = reinterpret_cast<const float4 *>(dy + (size_t)pos * dim);
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if (t + EO_NT * j < d4) v[j] = row[t + EO_NT * j];
            }
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (t + EO_NT * j < d4) {
                    acc[j].x += v[j].x; acc[j].y += v[j].y; acc[j].z += v[j].z; acc[j].w += v[j].w;
                }
        }
        __syncthreads();  // the list and wtot are reused by the next chunk
    }
    float4 *orow = reinterpret_cast<float4 *>(out + (size_t)tok * dim);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int cc = t + EO_NT * j;
        if (cc >= d4) continue;
        float4 a = acc[j];
        if (accumulate) {
            const float4 o = orow_in[j];
            a = make_float4(o.x + a.x, o.y + a.y, o.z + a.z, o.w + a.w);
        }
        orow[cc] = a;
        if constexpr (ADAM) {  // the row's gradient is final: its Adam update
            const size_t jj = (size_t)tok * d4 + cc;
            f32x4 *pp = reinterpret_cast<f32x4 *>(ea.p), *mm = reinterpret_cast<f32x4 *>(ea.m),
                  *vv = reinterpret_cast<f32x4 *>(ea.v);
            f32x4 pr = pin[j], mr = min_[j], vr = vin[j];
            adam4(pr, f32x4{a.x, a.y, a.z, a.w}, mr, vr, ea.h);
            pp[jj] = pr;
            mm[jj] = mr;
            vv[jj] = vr;
            if (ea.pb) {
                bf16x4 bb;
                bb[0] = (bf16)pr.x; bb[1] = (bf16)pr.y; bb[2] = (bf16)pr.z; bb[3] = (bf16)pr.w;
                reinterpret_cast<bf16x4 *>(ea.pb)[jj] = bb;
            }
        }
    }
}

// the chunked kernel's preconditions: float4 rows, 16-byte aligned ids and rows
inline bool own2_ok(const float *dy, const uint32_t *ids, const float *out, int dim) {
    return dim % 4 == 0 && dim <= 4 * 4 * EO_NT &&
           (((uintptr_t)dy | (uintptr_t)out | (uintptr_t)ids) & 15u) == 0;
}

}  // namespace

size_t embed_bw_work_bytes(int) { return 16; }

hipError_t embedding_backward(const float *dy, const uint32_t *ids, float *out, int n_pos,
                              int dim, int vocab, bool accumulate, void *work, hipStream_t st) {
    (void)work;
    if (n_pos <= 0) return hipSuccess;
    if (n_pos > kEmbedBwMaxPos) return hipErrorInvalidValue;
    const bool vec = (dim % 4 == 0) && (((uintptr_t)dy | (uintptr_t)out) & 15u) == 0;
    const EmbedAdam none{};
    if (own2_ok(dy, ids, out, dim))
        hipLaunchKernelGGL((embed_own2_k<false>), dim3(n_pos), dim3(EO_NT), 0, st, dy, ids, n_pos,
                           dim, out, vocab, accumulate ? 1 : 0, none);
    else if (vec)
        hipLaunchKernelGGL((embed_own_k<true, false>), dim3(n_pos), dim3(EO_NT), 0, st, dy, ids,
                           n_pos, dim, out, vocab, accumulate ? 1 : 0, none);
    else
        hipLaunchKernelGGL((embed_own_k<false, false>), dim3(n_pos), dim3(EO_NT), 0, st, dy, ids,
                           n_pos, dim, out, vocab, accumulate ? 1 : 0, none);
    return hipGetLastError();
}

hipError_t embedding_backward_adam(const float *dy, const uint32_t *ids, float *out, int n_pos,
                                   int dim, int vocab, bool accumulate, const EmbedAdam &ea,
                                   hipStream_t st) {
    if (n_pos <= 0) return hipSuccess;
    if (n_pos > kEmbedBwMaxPos) return hipErrorInvalidValue;
    const uintptr_t a = (uintptr_t)dy | (uintptr_t)out | (uintptr_t)ea.p | (uintptr_t)ea.m |
                        (uintptr_t)ea.v;
    if (dim % 4 || (a & 15u) || ((uintptr_t)ea.pb & 7u) || !ea.p || !ea.m || !ea.v)
        return hipErrorInvalidValue;
    if (own2_ok(dy, ids, out, dim))
        hipLaunchKernelGGL((embed_own2_k<true>), dim3(n_pos), dim3(EO_NT), 0, st, dy, ids, n_pos,
                           dim, out, vocab, accumulate ? 1 : 0, ea);
    else
        hipLaunchKernelGGL((embed_own_k<true, true>), dim3(n_pos), dim3(EO_NT), 0, st, dy, ids,
                           n_pos, dim, out, vocab, accumulate ? 1 : 0, ea);
    return hipGetLastError();
}

}  // namespace vkh
