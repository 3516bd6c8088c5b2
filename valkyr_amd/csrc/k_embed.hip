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
// work buffer.
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

}  // namespace

size_t embed_bw_work_bytes(int) { return 16; }

hipError_t embedding_backward(const float *dy, const uint32_t *ids, float *out, int n_pos,
                              int dim, int vocab, bool accumulate, void *work, hipStream_t st) {
    (void)work;
    if (n_pos <= 0) return hipSuccess;
    if (n_pos > kEmbedBwMaxPos) return hipErrorInvalidValue;
    const bool vec = (dim % 4 == 0) && (((uintptr_t)dy | (uintptr_t)out) & 15u) == 0;
    const EmbedAdam none{};
    if (vec)
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
    hipLaunchKernelGGL((embed_own_k<true, true>), dim3(n_pos), dim3(EO_NT), 0, st, dy, ids, n_pos,
                       dim, out, vocab, accumulate ? 1 : 0, ea);
    return hipGetLastError();
}

}  // namespace vkh
