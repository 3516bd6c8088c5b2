// Embedding backward: dE[tok] (+)= sum of dy rows of the positions holding
// `tok`, summed in position order.
//
// Reference: shaders/embedding_backward.comp (one workgroup per vocab row,
// each scanning all n_pos ids: V * n_pos id reads) and the CPU oracle
// train_transformer.zig:351-366 (sequential scatter-add).  Here the ids are
// sorted once (bitonic sort of (id << 32 | position) keys in LDS, so equal
// ids stay in position order), split into segments, and one workgroup per
// distinct id sums its rows with plain fp32 adds in position order.  The
// scatter targets are exact and the sums round exactly like the oracle's,
// so the result is bit-identical to it; no atomics.
#include "ops.hpp"

namespace vkh {

namespace {

constexpr int SORT_NT = 1024;

struct EmbedWork {
    uint32_t *pos;        // [n] positions in (id, position) order
    uint32_t *seg_start;  // [n + 1]
    uint32_t *seg_tok;    // [n]
    uint32_t *n_segs;     // [1]
};

inline EmbedWork carve(void *work, int n) {
    uint32_t *w = (uint32_t *)work;
    return EmbedWork{w, w + n, w + 2 * n + 1, w + 3 * n + 1};
}

__global__ __launch_bounds__(SORT_NT) void embed_sort_k(const uint32_t *ids, int n, EmbedWork w) {
    extern __shared__ uint64_t keys[];
    __shared__ uint32_t scan[SORT_NT];
    int np = 1;
    while (np < n) np <<= 1;
    const int tid = threadIdx.x;
    for (int i = tid; i < np; i += SORT_NT)
        keys[i] = i < n ? (((uint64_t)ids[i] << 32) | (uint32_t)i) : ~0ull;
    __syncthreads();
    for (int k = 2; k <= np; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = tid; i < np; i += SORT_NT) {
                const int ixj = i ^ j;
                if (ixj > i) {
                    const uint64_t a = keys[i], b = keys[ixj];
                    const bool up = (i & k) == 0;
                    if ((a > b) == up) { keys[i] = b; keys[ixj] = a; }
                }
            }
            __syncthreads();
        }
    }
    // segment heads, counted per thread over a contiguous chunk
    const int per = (n + SORT_NT - 1) / SORT_NT;
    const int i0 = tid * per, i1 = min(n, i0 + per);
    uint32_t cnt = 0;
    for (int i = i0; i < i1; ++i)
        if (i == 0 || (keys[i] >> 32) != (keys[i - 1] >> 32)) ++cnt;
    scan[tid] = cnt;
    __syncthreads();
    for (int o = 1; o < SORT_NT; o <<= 1) {  // inclusive Hillis-Steele scan
        const uint32_t v = tid >= o ? scan[tid - o] : 0;
        __syncthreads();
        scan[tid] += v;
        __syncthreads();
    }
    uint32_t seg = scan[tid] - cnt;
    for (int i = i0; i < i1; ++i) {
        const uint32_t tok = (uint32_t)(keys[i] >> 32);
        w.pos[i] = (uint32_t)keys[i];
        if (i == 0 || tok != (uint32_t)(keys[i - 1] >> 32)) {
            w.seg_start[seg] = i;
            w.seg_tok[seg] = tok;
            ++seg;
        }
    }
    if (tid == SORT_NT - 1) {
        w.n_segs[0] = scan[tid];
        w.seg_start[scan[tid]] = n;
    }
}

template <bool VEC>
__global__ __launch_bounds__(256) void embed_seg_k(const float *dy, int dim, EmbedWork w,
                                                    float *out, int vocab, int accumulate) {
    const uint32_t sgi = blockIdx.x;
    if (sgi >= w.n_segs[0]) return;
    const uint32_t tok = w.seg_tok[sgi];
    if (tok >= (uint32_t)vocab) return;
    const uint32_t s0 = w.seg_start[sgi], s1 = w.seg_start[sgi + 1];
    float *orow = out + (size_t)tok * dim;
    if (VEC) {
        for (int c = threadIdx.x; c < dim / 4; c += blockDim.x) {
            float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
            for (uint32_t i = s0; i < s1; ++i) {
                const float4 v = reinterpret_cast<const float4 *>(dy + (size_t)w.pos[i] * dim)[c];
                acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
            }
            if (accumulate) {
                const float4 o = reinterpret_cast<float4 *>(orow)[c];
                acc = make_float4(o.x + acc.x, o.y + acc.y, o.z + acc.z, o.w + acc.w);
            }
            reinterpret_cast<float4 *>(orow)[c] = acc;
        }
    } else {
        for (int c = threadIdx.x; c < dim; c += blockDim.x) {
            float acc = 0.f;
            for (uint32_t i = s0; i < s1; ++i) acc += dy[(size_t)w.pos[i] * dim + c];
            orow[c] = accumulate ? orow[c] + acc : acc;
        }
    }
}

}  // namespace

size_t embed_bw_work_bytes(int n_pos) { return (size_t)(4 * n_pos + 2) * sizeof(uint32_t); }

hipError_t embedding_backward(const float *dy, const uint32_t *ids, float *out, int n_pos,
                              int dim, int vocab, bool accumulate, void *work, hipStream_t st) {
    if (n_pos <= 0) return hipSuccess;
    if (n_pos > kEmbedBwMaxPos) return hipErrorInvalidValue;
    EmbedWork w = carve(work, n_pos);
    int np = 1;
    while (np < n_pos) np <<= 1;
    static bool attr_set = false;
    if (!attr_set) {
        // the key array may exceed the 64 KB default dynamic-LDS limit (gfx950 has 160 KB)
        hipError_t e = hipFuncSetAttribute((const void *)embed_sort_k,
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           kEmbedBwMaxPos * (int)sizeof(uint64_t));
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    hipLaunchKernelGGL(embed_sort_k, dim3(1), dim3(SORT_NT), np * sizeof(uint64_t), st, ids, n_pos, w);
    const bool vec = (dim % 4 == 0) && (((uintptr_t)dy | (uintptr_t)out) & 15u) == 0;
    if (vec)
        hipLaunchKernelGGL(embed_seg_k<true>, dim3(n_pos), dim3(256), 0, st, dy, dim, w, out, vocab,
                           accumulate ? 1 : 0);
    else
        hipLaunchKernelGGL(embed_seg_k<false>, dim3(n_pos), dim3(256), 0, st, dy, dim, w, out, vocab,
                           accumulate ? 1 : 0);
    return hipGetLastError();
}

}  // namespace vkh
