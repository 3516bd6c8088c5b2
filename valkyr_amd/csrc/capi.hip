// C ABI for the individual kernels plus the HIP plumbing (memory, streams,
// events) a host without its own HIP bindings needs.  Every function checks
// its arguments, enqueues, and reports launch errors as VKH_ERR_HIP.
#include <math.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <iterator>
#include <map>
#include <mutex>
#include <tuple>
#include <vector>

#include "internal.hpp"

namespace vkh {

static thread_local char g_err[512] = "";

vkh_status fail(vkh_status st, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return st;
}

vkh_status hip_fail(hipError_t e, const char *what) {
    if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation)
        return fail(VKH_ERR_OUT_OF_MEMORY, "%s: %s", what, hipGetErrorString(e));
    return fail(VKH_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

static std::atomic<uint64_t> g_allocations{0};
void note_allocation() { g_allocations.fetch_add(1, std::memory_order_relaxed); }

// RoPE tables for the standalone kernel entry points, cached per
// (device, seq_len, rotary_dim, theta) for the life of the process.
static vkh_status rope_table_cached(int seq_len, int rot, float theta, const float2 **out) {
    static std::mutex mu;
    static std::map<std::tuple<int, int, int, uint32_t>, float2 *> cache;
    int dev = 0;
    VKH_HIP(hipGetDevice(&dev));
    uint32_t tb;
    memcpy(&tb, &theta, 4);
    std::lock_guard<std::mutex> lk(mu);
    auto key = std::make_tuple(dev, seq_len, rot, tb);
    auto it = cache.find(key);
    if (it != cache.end()) { *out = it->second; return VKH_OK; }
    const int half = rot / 2;
    std::vector<float2> tab((size_t)seq_len * (half ? half : 1));
    if (half) rope_table_host(tab.data(), seq_len, rot, theta);
    float2 *d = nullptr;
    note_allocation();
    VKH_HIP(hipMalloc(&d, tab.size() * sizeof(float2)));
    VKH_HIP(hipMemcpy(d, tab.data(), tab.size() * sizeof(float2), hipMemcpyHostToDevice));
    cache[key] = d;
    *out = d;
    return VKH_OK;
}

// Scratch memory of the standalone entry points (gain partials, split-K
// partials): one buffer per (device, stream), grown on demand and reused, so
// a call does not allocate once its stream's buffer is large enough.  Calls
// on one stream are ordered by the stream; calls on different streams use
// different buffers, so no event is recorded or waited for per call (an
// event record costs a few microseconds of device time).  Streams are told
// apart by hipStreamGetId, which is unique for the life of the process, so a
// stream created after another was destroyed never inherits its buffer.  A
// buffer is replaced only after its stream has drained; at most kMaxStreams
// buffers are kept, and making room for another waits for the whole device.
class ScratchLease {
  public:
    vkh_status acquire(size_t bytes, hipStream_t st, void **out) {
        note_allocation();
        constexpr size_t kMaxStreams = 64;
        struct Buf {
            void *p = nullptr;
            size_t bytes = 0;
        };
        static std::mutex mu;
        static std::map<std::pair<int, unsigned long long>, Buf> per_stream;
        lk_ = std::unique_lock<std::mutex>(mu);  // held until the call has enqueued its work
        int dev = 0;
        VKH_HIP(hipGetDevice(&dev));
        unsigned long long sid = 0;
        VKH_HIP(hipStreamGetId(st, &sid));
        const auto key = std::make_pair(dev, sid);
        auto it = per_stream.find(key);
        if (it == per_stream.end()) {
            if (per_stream.size() >= kMaxStreams) {
                // every stream's work done: any kept buffer may go
                VKH_HIP(hipDeviceSynchronize());
                for (auto &kv : per_stream) {
                    if (kv.first.first != dev) continue;
                    VKH_HIP(hipFree(kv.second.p));
                }
                for (auto i = per_stream.begin(); i != per_stream.end();)
                    i = i->first.first == dev ? per_stream.erase(i) : std::next(i);
            }
            it = per_stream.emplace(key, Buf{}).first;
        }
        Buf &b = it->second;
        if (b.bytes < bytes) {
            if (b.p) {
                VKH_HIP(hipStreamSynchronize(st));  // its earlier uses are done
                VKH_HIP(hipFree(b.p));
                b.p = nullptr;
                b.bytes = 0;
            }
            const size_t nb = std::max(bytes, (size_t)1 << 20);
            note_allocation();
            VKH_HIP(hipMalloc(&b.p, nb));
            b.bytes = nb;
        }
        *out = b.p;
        return VKH_OK;
    }

  private:
    std::unique_lock<std::mutex> lk_;
};

}  // namespace vkh

using namespace vkh;

#define CHECK_ARG(cond, msg)                                              \
    do {                                                                  \
        if (!(cond)) return fail(VKH_ERR_INVALID_ARGUMENT, "%s", msg);    \
    } while (0)

static inline hipStream_t S(vkh_stream s) { return (hipStream_t)s; }
static inline Precision PR(uint32_t p) { return p == VKH_PRECISION_BF16 ? Precision::BF16 : Precision::FP32; }

static AttnShape attn_shape(const vkh_attn_params *p) {
    AttnShape s;
    s.n_batch = p->n_batch ? (int)p->n_batch : 1;
    s.n_q = p->n_q; s.n_kv = p->n_kv; s.n_heads = p->n_heads; s.n_kv_heads = p->n_kv_heads;
    s.head_dim = p->head_dim; s.causal = p->causal ? 1 : 0; s.inv_sqrt_dim = p->inv_sqrt_dim;
    return s;
}

static vkh_status check_attn(const vkh_attn_params *p) {
    CHECK_ARG(p, "null params");
    CHECK_ARG(p->n_heads && p->n_kv_heads && p->head_dim && p->n_q && p->n_kv, "zero attention dimension");
    CHECK_ARG(p->n_heads % p->n_kv_heads == 0, "n_heads % n_kv_heads != 0");
    CHECK_ARG(!p->causal || p->n_q <= p->n_kv, "causal attention needs n_q <= n_kv");
    CHECK_ARG(p->dtype <= VKH_BF16, "dtype");
    if (p->dtype == VKH_BF16 && p->head_dim != 64 && p->head_dim != 128)
        return fail(VKH_ERR_UNSUPPORTED, "bf16 attention supports head_dim 64 and 128");
    if (p->head_dim > 256) return fail(VKH_ERR_UNSUPPORTED, "head_dim > 256");
    return VKH_OK;
}

extern "C" {

const char *vkh_last_error(void) { return g_err; }

const char *vkh_build_info(void) { return "vkhip for gfx950 (MI355X), built with hipcc " __VERSION__; }

const char *vkh_status_name(vkh_status s) {
    switch (s) {
    case VKH_OK: return "Ok";
    case VKH_ERR_INVALID_ARGUMENT: return "InvalidArgument";
    case VKH_ERR_HIP: return "HipError";
    case VKH_ERR_OUT_OF_MEMORY: return "OutOfMemory";
    case VKH_ERR_UNSUPPORTED: return "Unsupported";
    case VKH_ERR_NO_DEVICE: return "NoDevice";
    case VKH_ERR_TOKEN_IDS_LEN: return "TokenIdsLen";
    case VKH_ERR_TARGET_LEN: return "TargetLen";
    case VKH_ERR_OUT_LOGITS_LEN: return "OutLogitsLen";
    case VKH_ERR_TOKEN_OUT_OF_RANGE: return "TokenOutOfRange";
    case VKH_ERR_EMBED_SHAPE: return "EmbedShape";
    case VKH_ERR_FINAL_NORM_SHAPE: return "FinalNormShape";
    case VKH_ERR_LM_HEAD_SHAPE: return "LmHeadShape";
    case VKH_ERR_LAYER_COUNT: return "LayerCount";
    case VKH_ERR_LAYER_N1_SHAPE: return "LayerN1Shape";
    case VKH_ERR_LAYER_Q_SHAPE: return "LayerQShape";
    case VKH_ERR_LAYER_K_SHAPE: return "LayerKShape";
    case VKH_ERR_LAYER_V_SHAPE: return "LayerVShape";
    case VKH_ERR_LAYER_O_SHAPE: return "LayerOShape";
    case VKH_ERR_LAYER_N2_SHAPE: return "LayerN2Shape";
    case VKH_ERR_LAYER_GATE_SHAPE: return "LayerGateShape";
    case VKH_ERR_LAYER_UP_SHAPE: return "LayerUpShape";
    case VKH_ERR_LAYER_DOWN_SHAPE: return "LayerDownShape";
    case VKH_ERR_LAYER_Q_NORM_SHAPE: return "LayerQNormShape";
    case VKH_ERR_LAYER_K_NORM_SHAPE: return "LayerKNormShape";
    case VKH_ERR_LORA_RANK_ZERO: return "LoraRankZero";
    case VKH_ERR_LORA_INIT_LEN: return "LoraInitLen";
    case VKH_ERR_INVALID_CHECKPOINT_MAGIC: return "InvalidCheckpointMagic";
    case VKH_ERR_UNSUPPORTED_CHECKPOINT_VERSION: return "UnsupportedCheckpointVersion";
    case VKH_ERR_CHECKPOINT_CONFIG_SIZE_MISMATCH: return "CheckpointConfigSizeMismatch";
    case VKH_ERR_CHECKPOINT_CONFIG_MISMATCH: return "CheckpointConfigMismatch";
    case VKH_ERR_END_OF_STREAM: return "EndOfStream";
    case VKH_ERR_INVALID_LORA_CHECKPOINT_MAGIC: return "InvalidLoraCheckpointMagic";
    case VKH_ERR_UNSUPPORTED_LORA_CHECKPOINT_VERSION: return "UnsupportedLoraCheckpointVersion";
    case VKH_ERR_LORA_CHECKPOINT_CONFIG_SIZE_MISMATCH: return "LoraCheckpointConfigSizeMismatch";
    case VKH_ERR_LORA_CHECKPOINT_CONFIG_MISMATCH: return "LoraCheckpointConfigMismatch";
    case VKH_ERR_LORA_CHECKPOINT_EMPTY: return "LoraCheckpointEmpty";
    case VKH_ERR_IO: return "IoError";
    case VKH_ERR_INPUT_IDS_LEN: return "InputIdsLen";
    case VKH_ERR_TARGET_IDS_LEN: return "TargetIdsLen";
    case VKH_ERR_BATCH_INDEX_OUT_OF_RANGE: return "BatchIndexOutOfRange";
    case VKH_ERR_EMPTY_DATASET: return "EmptyDataset";
    case VKH_ERR_DATASET_TOO_SHORT: return "DatasetTooShort";
    case VKH_ERR_BATCH_IDX_OUT_OF_RANGE: return "BatchIdxOutOfRange";
    case VKH_ERR_HIDDEN_DIM_EXCEEDS_MAX: return "HiddenDimExceedsMax";
    case VKH_ERR_X_DIM_MISMATCH: return "XDimMismatch";
    case VKH_ERR_TARGET_DIM_MISMATCH: return "TargetDimMismatch";
    case VKH_ERR_OUT_DIM_MISMATCH: return "OutDimMismatch";
    case VKH_ERR_BATCH_SIZE_NOT_CONFIGURED: return "BatchSizeNotConfigured";
    case VKH_ERR_BATCH_SIZE_EXCEEDS_MAX: return "BatchSizeExceedsMax";
    case VKH_ERR_X_BATCH_DIM_MISMATCH: return "XBatchDimMismatch";
    case VKH_ERR_TARGET_BATCH_DIM_MISMATCH: return "TargetBatchDimMismatch";
    case VKH_ERR_OUT_BATCH_DIM_MISMATCH: return "OutBatchDimMismatch";
    case VKH_ERR_OUTPUT_TOO_LARGE: return "OutputTooLarge";
    }
    return "Unknown";
}

// ── attention ──────────────────────────────────────────────────────────

vkh_status vkh_fa_forward(const vkh_attn_params *p, const void *q, const void *k, const void *v,
                          float *o, float *lse, vkh_stream stream) {
    VKH_TRY(check_attn(p));
    CHECK_ARG(q && k && v && o, "null pointer");
    const AttnShape s = attn_shape(p);
    const long ldq = (long)p->n_heads * p->head_dim, ldk = (long)p->n_kv_heads * p->head_dim;
    VKH_HIP(fa_forward(s, q, ldq, k, ldk, v, ldk, o, ldq, lse,
                       p->dtype == VKH_BF16 ? DType::BF16 : DType::F32, nullptr, 0, S(stream)));
    return VKH_OK;
}

vkh_status vkh_fa_bw_d(const vkh_attn_params *p, const float *o, const float *dout, float *d,
                       void *dout_bf16, vkh_stream stream) {
    VKH_TRY(check_attn(p));
    CHECK_ARG(o && dout && d, "null pointer");
    const AttnShape s = attn_shape(p);
    const long ld = (long)p->n_heads * p->head_dim;
    VKH_HIP(fa_bw_d(s, o, ld, dout, ld, d, p->dtype == VKH_BF16 ? (bf16 *)dout_bf16 : nullptr, ld,
                    S(stream)));
    return VKH_OK;
}

vkh_status vkh_fa_bw_d_bf16(const vkh_attn_params *p, const void *o_bf16, const void *dout_bf16,
                            float *d, vkh_stream stream) {
    VKH_TRY(check_attn(p));
    CHECK_ARG(o_bf16 && dout_bf16 && d, "null pointer");
    if (p->head_dim != 64 && p->head_dim != 128)
        return fail(VKH_ERR_UNSUPPORTED, "bf16 D preprocess needs head_dim 64 or 128");
    const AttnShape s = attn_shape(p);
    const long ld = (long)p->n_heads * p->head_dim;
    VKH_HIP(fa_bw_d_bf16(s, (const bf16 *)o_bf16, ld, (const bf16 *)dout_bf16, ld, d, S(stream)));
    return VKH_OK;
}

static AttnPtrs attn_ptrs(const vkh_attn_params *p, const void *q, const void *k, const void *v,
                          const void *dout, const float *lse, const float *d) {
    AttnPtrs a{};
    const long ldq = (long)p->n_heads * p->head_dim, ldk = (long)p->n_kv_heads * p->head_dim;
    a.q = q; a.ldq = ldq; a.k = k; a.ldk = ldk; a.v = v; a.ldv = ldk;
    a.dout = dout; a.lddo = ldq; a.lse = lse; a.d = (float *)d;
    a.lddq = ldq; a.lddk = ldk; a.lddv = ldk;
    a.dt = p->dtype == VKH_BF16 ? DType::BF16 : DType::F32;
    return a;
}

vkh_status vkh_fa_bw_dq(const vkh_attn_params *p, const void *q, const void *k, const void *v,
                        const void *dout, const float *lse, const float *d, float *dq,
                        vkh_stream stream) {
    VKH_TRY(check_attn(p));
    CHECK_ARG(q && k && v && dout && lse && d && dq, "null pointer");
    AttnPtrs a = attn_ptrs(p, q, k, v, dout, lse, d);
    a.dq = dq;
    VKH_HIP(fa_bw_dq(attn_shape(p), a, S(stream)));
    return VKH_OK;
}

vkh_status vkh_fa_bw_dkv(const vkh_attn_params *p, const void *q, const void *k, const void *v,
                         const void *dout, const float *lse, const float *d, float *dk,
                         float *dv, vkh_stream stream) {
    VKH_TRY(check_attn(p));
    CHECK_ARG(q && k && v && dout && lse && d && dk && dv, "null pointer");
    AttnPtrs a = attn_ptrs(p, q, k, v, dout, lse, d);
    a.dk = dk;
    a.dv = dv;
    VKH_HIP(fa_bw_dkv(attn_shape(p), a, S(stream)));
    return VKH_OK;
}

size_t vkh_fa_backward_workspace_bytes(const vkh_attn_params *p) {
    if (!p || check_attn(p) != VKH_OK) return 0;
    const AttnShape s = attn_shape(p);
    return p->dtype == VKH_BF16 && fa_bw_fused_ok(s) ? fa_bw_ws_bytes(s, fa_bw_v4_ok(s)) : 0;
}

vkh_status vkh_fa_backward(const vkh_attn_params *p, const void *q, const void *k, const void *v,
                           const void *dout, const float *lse, const float *d, float *dq,
                           float *dk, float *dv, void *workspace, vkh_stream stream) {
    VKH_TRY(check_attn(p));
    CHECK_ARG(q && k && v && dout && lse && d && dq && dk && dv, "null pointer");
    AttnPtrs a = attn_ptrs(p, q, k, v, dout, lse, d);
    a.dq = dq;
    a.dk = dk;
    a.dv = dv;
    const AttnShape s = attn_shape(p);
    hipStream_t st = S(stream);
    if (p->dtype != VKH_BF16 || !fa_bw_fused_ok(s)) {
        VKH_HIP(fa_bw_dkv(s, a, st));
        VKH_HIP(fa_bw_dq(s, a, st));
        return VKH_OK;
    }
    void *ws = workspace;
    // the recompute kernels whenever the shape allows (they need no workspace)
    const bool v4 = fa_bw_v4_ok(s);
    const size_t wsb = fa_bw_ws_bytes(s, v4);
    if (!ws && wsb) {
        note_allocation();
        VKH_HIP(hipMallocAsync(&ws, wsb, st));
    }
    const hipError_t e = fa_bw_fused(s, a, (bf16 *)ws, v4, st);
    if (!workspace && wsb) (void)hipFreeAsync(ws, st);
    if (e != hipSuccess) return hip_fail(e, "fa_backward");
    return VKH_OK;
}

// The whole attention backward from bf16 O: the D preprocess and the two
// gradient kernels.  On the recompute path the dQ kernel forms D itself (no
// separate pass) and the dK/dV kernel reads it; other shapes run the D kernel
// and then vkh_fa_backward.
vkh_status vkh_fa_backward_from_o(const vkh_attn_params *p, const void *q, const void *k,
                                  const void *v, const void *o_bf16, const void *dout_bf16,
                                  const float *lse, float *d, float *dq, float *dk, float *dv,
                                  void *workspace, vkh_stream stream) {
    VKH_TRY(check_attn(p));
    CHECK_ARG(q && k && v && o_bf16 && dout_bf16 && lse && d && dq && dk && dv, "null pointer");
    if (p->dtype != VKH_BF16) return fail(VKH_ERR_INVALID_ARGUMENT, "fa_backward_from_o takes bf16 operands");
    const AttnShape s = attn_shape(p);
    if (fa_bw_fused_ok(s) && fa_bw_v4_ok(s)) {
        AttnPtrs a = attn_ptrs(p, q, k, v, dout_bf16, lse, d);
        a.dq = dq;
        a.dk = dk;
        a.dv = dv;
        a.o16 = o_bf16;
        a.ldo16 = (long)p->n_heads * p->head_dim;
        const hipError_t e = fa_bw_fused(s, a, nullptr, true, S(stream));
        if (e != hipSuccess) return hip_fail(e, "fa_backward_from_o");
        return VKH_OK;
    }
    VKH_TRY(vkh_fa_bw_d_bf16(p, o_bf16, dout_bf16, d, stream));
    return vkh_fa_backward(p, q, k, v, dout_bf16, lse, d, dq, dk, dv, workspace, stream);
}

// ── GEMMs ──────────────────────────────────────────────────────────────

// Split-K workspace for one call (stream-ordered allocation), if the plan wants one.
extern "C++" {
template <class F>
static vkh_status with_ws(size_t bytes, hipStream_t st, const char *what, F &&f) {
    GemmWs ws{nullptr, bytes};
    ScratchLease lease;
    if (ws.bytes) VKH_TRY(lease.acquire(ws.bytes, st, &ws.p));
    const hipError_t e = f(ws);
    if (e != hipSuccess) return hip_fail(e, what);
    return VKH_OK;
}
template <class F>
static vkh_status with_g16_ws(int M, int N, int K, hipStream_t st, const char *what, F &&f) {
    return with_ws(g16_ws_bytes_for(M, N, K), st, what, f);
}
}

// Precision FP32: the DMA-staged fp32 MFMA kernels (g32_*), which take the
// generic kernel for operands outside their layout rules; BF16: operands
// rounded to bf16 on their way into the generic kernel's LDS tiles.
vkh_status vkh_matmul_nt(const float *x, const float *w, float *y, uint32_t M, uint32_t N,
                         uint32_t K, uint32_t precision, vkh_stream stream) {
    CHECK_ARG(x && w && y, "null pointer");
    hipStream_t st = S(stream);
    if (PR(precision) == Precision::FP32)
        return with_ws(g32_ws_bytes_for(M, N, K), st, "matmul_nt", [&](const GemmWs &ws) {
            return g32_nt(x, K, w, K, y, N, M, N, K, nullptr, 0, 1.f, 0.f, ws, st);
        });
    VKH_HIP(gemm_nt(PR(precision), matf(x, K), matf(w, K), y, N, M, N, K, nullptr, 0, 1.f, 0.f, st));
    return VKH_OK;
}

vkh_status vkh_linear_backward_dx(const float *dy, const float *w, float *dx, uint32_t M,
                                  uint32_t N, uint32_t K, uint32_t precision, vkh_stream stream) {
    CHECK_ARG(dy && w && dx, "null pointer");
    hipStream_t st = S(stream);
    if (PR(precision) == Precision::FP32)
        return with_ws(g32_ws_bytes_for(M, K, N), st, "linear_backward_dx", [&](const GemmWs &ws) {
            return g32_nn(dy, N, w, K, dx, K, M, N, K, 1.f, 0.f, ws, st);
        });
    VKH_HIP(gemm_nn(PR(precision), matf(dy, N), matf(w, K), dx, K, M, N, K, 1.f, 0.f, st));
    return VKH_OK;
}

vkh_status vkh_linear_backward_dw(const float *dy, const float *x, float *dw, uint32_t M,
                                  uint32_t N, uint32_t K, uint32_t precision, vkh_stream stream) {
    CHECK_ARG(dy && x && dw, "null pointer");
    hipStream_t st = S(stream);
    if (PR(precision) == Precision::FP32)
        return with_ws(g32_ws_bytes_for(N, K, M), st, "linear_backward_dw", [&](const GemmWs &ws) {
            return g32_tn(dy, N, x, K, dw, K, M, N, K, 1.f, 0.f, ws, st);
        });
    VKH_HIP(gemm_tn(PR(precision), matf(dy, N), matf(x, K), dw, K, M, N, K, 1.f, 0.f, st));
    return VKH_OK;
}

vkh_status vkh_matmul_nt_bf16(const void *x, const void *w, float *y, uint32_t M, uint32_t N,
                              uint32_t K, vkh_stream stream) {
    CHECK_ARG(x && w && y, "null pointer");
    hipStream_t st = S(stream);
    return with_g16_ws(M, N, K, st, "matmul_nt_bf16", [&](const GemmWs &ws) {
        return g16_nt((const bf16 *)x, K, (const bf16 *)w, K, y, N, M, N, K, nullptr, 0, 1.f, 0.f,
                      ws, st);
    });
}

vkh_status vkh_gate_up_swiglu_bf16(const void *x, const void *w_gu, float *gu, void *gated,
                                   uint32_t M, uint32_t F, uint32_t K, vkh_stream stream) {
    CHECK_ARG(x && w_gu && gu && gated, "null pointer");
    CHECK_ARG(2ull * F < (1ull << 31), "F too large");
    hipStream_t st = S(stream);
    const hipError_t e = g16_gate_up_swiglu((const bf16 *)x, K, (const bf16 *)w_gu, K, gu, 2L * F,
                                            (bf16 *)gated, F, (int)M, (int)F, (int)K, st);
    if (e != hipErrorNotSupported) {
        VKH_HIP(e);
        return VKH_OK;
    }
    // the two-pass form: the [M, 2F] product, then the SwiGLU over its halves
    const vkh_status r = vkh_matmul_nt_bf16(x, w_gu, gu, M, 2 * F, K, stream);
    if (r != VKH_OK) return r;
    VKH_HIP(swiglu_forward(gu, 2L * F, gu + F, 2L * F, gated, F, DType::BF16, (int)M, (int)F, st));
    return VKH_OK;
}

vkh_status vkh_gate_up_swiglu(const float *x, const float *w_gu, float *gu, float *gated,
                              uint32_t M, uint32_t F, uint32_t K, int fused, vkh_stream stream) {
    CHECK_ARG(x && w_gu && gu && gated, "null pointer");
    CHECK_ARG(2ull * F < (1ull << 31), "F too large");
    hipStream_t st = S(stream);
    if (fused) {
        const hipError_t e = g32_gate_up_swiglu(x, K, w_gu, K, gu, 2L * F, gated, F, (int)M, (int)F,
                                                (int)K, st);
        if (e != hipErrorNotSupported) {
            VKH_HIP(e);
            return VKH_OK;
        }
    }
    const vkh_status r = vkh_matmul_nt(x, w_gu, gu, M, 2 * F, K, VKH_PRECISION_FP32, stream);
    if (r != VKH_OK) return r;
    VKH_HIP(swiglu_forward(gu, 2L * F, gu + F, 2L * F, gated, F, DType::F32, (int)M, (int)F, st));
    return VKH_OK;
}

vkh_status vkh_linear_backward_dx_bf16(const void *dy, const void *w, float *dx, uint32_t M,
                                       uint32_t N, uint32_t K, vkh_stream stream) {
    CHECK_ARG(dy && w && dx, "null pointer");
    hipStream_t st = S(stream);
    return with_g16_ws(M, K, N, st, "linear_backward_dx_bf16", [&](const GemmWs &ws) {
        return g16_nn((const bf16 *)dy, N, (const bf16 *)w, K, dx, K, M, N, K, 1.f, 0.f, ws, st);
    });
}

vkh_status vkh_linear_backward_dw_bf16(const void *dy, const void *x, float *dw, uint32_t M,
                                       uint32_t N, uint32_t K, vkh_stream stream) {
    CHECK_ARG(dy && x && dw, "null pointer");
    hipStream_t st = S(stream);
    return with_g16_ws(N, K, M, st, "linear_backward_dw_bf16", [&](const GemmWs &ws) {
        return g16_tn((const bf16 *)dy, N, (const bf16 *)x, K, dw, K, M, N, K, 1.f, 0.f, ws, st);
    });
}

vkh_status vkh_lora_forward(const float *x, const float *w, const float *a, const float *b,
                            float *y, float *inter, uint32_t M, uint32_t N, uint32_t K,
                            uint32_t r, float aor, uint32_t precision, vkh_stream stream) {
    CHECK_ARG(x && w && a && b && y && inter, "null pointer");
    CHECK_ARG(r > 0, "rank 0");
    const Precision pr = PR(precision);
    hipStream_t st = S(stream);
    VKH_HIP(gemm_nt(pr, matf(x, K), matf(w, K), y, N, M, N, K, nullptr, 0, 1.f, 0.f, st));
    // rank-r kernels (fp32 factors and products) where the shape allows
    LoraSegs sa, sb;
    sa.n = sb.n = 1;
    sa.s[0] = LoraSeg{0, (int)K, a, 1, (long)K, inter, (long)r};
    sb.s[0] = LoraSeg{0, (int)N, b, (long)r, 1, inter, (long)r};
    if (lora_fast_ok(DType::F32, x, K, (int)r, sa) && lora_update_ok(y, N, (int)r, sb)) {
        VKH_HIP(lora_rows(DType::F32, x, K, (int)M, (int)r, sa, 1.f, st));
        VKH_HIP(lora_update(y, N, (int)M, (int)r, sb, aor, st));
        return VKH_OK;
    }
    VKH_HIP(gemm_nt(pr, matf(x, K), matf(a, K), inter, r, M, r, K, nullptr, 0, 1.f, 0.f, st));
    VKH_HIP(gemm_nt(pr, matf(inter, r), matf(b, r), y, N, M, N, r, nullptr, 0, aor, 1.f, st));
    return VKH_OK;
}

vkh_status vkh_lora_backward(const float *dy, const float *x, const float *w, const float *a,
                             const float *b, const float *inter, float *dx, float *dA,
                             float *dB, uint32_t M, uint32_t N, uint32_t K, uint32_t r,
                             float aor, uint32_t precision, vkh_stream stream) {
    CHECK_ARG(dy && x && w && a && b && inter && dA && dB, "null pointer");
    CHECK_ARG(r > 0, "rank 0");
    const Precision pr = PR(precision);
    hipStream_t st = S(stream);
    float *dyB = nullptr;
    note_allocation();
    VKH_HIP(hipMallocAsync((void **)&dyB, (size_t)M * r * 4 + 256, st));
    LoraSegs sb, sa, sdA, sdB;
    sb.n = sa.n = sdA.n = sdB.n = 1;
    sb.s[0] = LoraSeg{0, (int)N, b, (long)r, 1, dyB, (long)r};
    sa.s[0] = LoraSeg{0, (int)K, a, 1, (long)K, dyB, (long)r};
    sdA.s[0] = LoraSeg{0, (int)K, nullptr, 1, 1, dyB, (long)r, dA, 1, (long)K};
    sdB.s[0] = LoraSeg{0, (int)N, nullptr, 1, 1, (float *)inter, (long)r, dB, (long)r, 1};
    if (lora_fast_ok(DType::F32, dy, N, (int)r, sb) && lora_fast_ok(DType::F32, x, K, (int)r, sdA) &&
        lora_fast_ok(DType::F32, dy, N, (int)r, sdB) && (!dx || lora_update_ok(dx, K, (int)r, sa))) {
        // rank-r kernels (fp32 factors and products)
        hipError_t e = lora_rows(DType::F32, dy, N, (int)M, (int)r, sb, 1.f, st);
        if (e == hipSuccess && dx) e = gemm_nn(pr, matf(dy, N), matf(w, K), dx, K, M, N, K, 1.f, 0.f, st);
        if (e == hipSuccess && dx) e = lora_update(dx, K, (int)M, (int)r, sa, aor, st);
        if (e == hipSuccess) e = lora_cols(DType::F32, x, K, (int)M, (int)r, sdA, aor, st);
        if (e == hipSuccess) e = lora_cols(DType::F32, dy, N, (int)M, (int)r, sdB, aor, st);
        (void)hipFreeAsync(dyB, st);
        if (e != hipSuccess) return hip_fail(e, "lora_backward");
        return VKH_OK;
    }
    hipError_t e = gemm_nn(pr, matf(dy, N), matf(b, r), dyB, r, M, N, r, 1.f, 0.f, st);
    if (e == hipSuccess && dx) e = gemm_nn(pr, matf(dy, N), matf(w, K), dx, K, M, N, K, 1.f, 0.f, st);
    if (e == hipSuccess && dx) e = gemm_nn(pr, matf(dyB, r), matf(a, K), dx, K, M, r, K, aor, 1.f, st);
    if (e == hipSuccess) e = gemm_tn(pr, matf(dyB, r), matf(x, K), dA, K, M, r, K, aor, 0.f, st);
    if (e == hipSuccess) e = gemm_tn(pr, matf(dy, N), matf(inter, r), dB, r, M, N, r, aor, 0.f, st);
    (void)hipFreeAsync(dyB, st);
    if (e != hipSuccess) return hip_fail(e, "lora_backward");
    return VKH_OK;
}

// The training step's grouped LoRA launches on bf16 activations: the segment
// lists come from lora_group_segs, as in the runner.
static vkh_status lora_group_args(const vkh_lora_adapter *ad, uint32_t na, uint32_t r,
                                  LoraAdapter (&out)[3]) {
    CHECK_ARG(ad && na >= 1 && na <= 3, "1 to 3 adapters");
    CHECK_ARG(r > 0, "rank 0");
    for (uint32_t i = 0; i < na; ++i) {
        const vkh_lora_adapter &a = ad[i];
        CHECK_ARG(a.a && a.b && a.inter && a.n && a.k, "adapter: null factor or buffer");
        out[i] = LoraAdapter{(long)a.col, (int)a.n, (int)a.k, a.a, a.b, a.inter, a.dyb, a.da, a.db};
    }
    return VKH_OK;
}

vkh_status vkh_lora_group_forward_bf16(const uint16_t *x, uint32_t ldx, uint32_t T, uint32_t r,
                                       float aor, const vkh_lora_adapter *adapters,
                                       uint32_t n_adapters, float *y, uint32_t ldy,
                                       vkh_stream stream) {
    CHECK_ARG(x && y, "null pointer");
    LoraAdapter ad[3];
    VKH_TRY(lora_group_args(adapters, n_adapters, r, ad));
    for (uint32_t i = 0; i < n_adapters; ++i)
        CHECK_ARG(ad[i].k <= (long)ldx && ad[i].col + ad[i].n <= (long)ldy, "adapter outside the rows");
    const LoraGroupSegs g = lora_group_segs(ad, (int)n_adapters, (int)r);
    if (!lora_fast_ok(DType::BF16, x, ldx, (int)r, g.fwd_rows) ||
        !lora_update_ok(y, ldy, (int)r, g.fwd_upd))
        return fail(VKH_ERR_UNSUPPORTED, "lora_group_forward_bf16: shape or alignment");
    hipStream_t st = S(stream);
    VKH_HIP(lora_rows(DType::BF16, x, ldx, (int)T, (int)r, g.fwd_rows, 1.f, st));
    VKH_HIP(lora_update(y, ldy, (int)T, (int)r, g.fwd_upd, aor, st));
    return VKH_OK;
}

vkh_status vkh_lora_group_backward_bf16(const uint16_t *dy, uint32_t lddy, const uint16_t *x,
                                        uint32_t ldx, uint32_t T, uint32_t r, float aor,
                                        const vkh_lora_adapter *adapters, uint32_t n_adapters,
                                        float *dx, uint32_t lddx, vkh_stream stream) {
    CHECK_ARG(dy && x, "null pointer");
    LoraAdapter ad[3];
    VKH_TRY(lora_group_args(adapters, n_adapters, r, ad));
    for (uint32_t i = 0; i < n_adapters; ++i) {
        CHECK_ARG(ad[i].dyb && ad[i].da && ad[i].db, "adapter: null dyb, da or db");
        CHECK_ARG(ad[i].k <= (long)ldx && ad[i].col + ad[i].n <= (long)lddy &&
                      (!dx || ad[i].k <= (long)lddx),
                  "adapter outside the rows");
    }
    const LoraGroupSegs g = lora_group_segs(ad, (int)n_adapters, (int)r);
    if (!lora_fast_ok(DType::BF16, dy, lddy, (int)r, g.bwd_rows) ||
        !lora_fast_ok(DType::BF16, x, ldx, (int)r, g.bwd_da) ||
        !lora_fast_ok(DType::BF16, dy, lddy, (int)r, g.bwd_db) ||
        (dx && !lora_update_ok(dx, lddx, (int)r, g.bwd_upd)))
        return fail(VKH_ERR_UNSUPPORTED, "lora_group_backward_bf16: shape or alignment");
    hipStream_t st = S(stream);
    VKH_HIP(lora_rows(DType::BF16, dy, lddy, (int)T, (int)r, g.bwd_rows, 1.f, st));
    VKH_HIP(lora_cols(DType::BF16, x, ldx, (int)T, (int)r, g.bwd_da, aor, st));
    VKH_HIP(lora_cols(DType::BF16, dy, lddy, (int)T, (int)r, g.bwd_db, aor, st));
    if (dx) VKH_HIP(lora_update(dx, lddx, (int)T, (int)r, g.bwd_upd, aor, st));
    return VKH_OK;
}

// ── CCE ────────────────────────────────────────────────────────────────

vkh_status vkh_cce_forward(const vkh_cce_params *p, const float *h, const float *w,
                           const uint32_t *targets, float *lse, float *loss_row,
                           float *loss_mean, vkh_stream stream) {
    CHECK_ARG(p && h && w && targets && lse, "null pointer");
    CHECK_ARG(p->n && p->vocab && p->dim, "zero dimension");
    const CceShape s{(int)p->n, (int)p->vocab, (int)p->dim, p->z_loss_scale, p->label_smoothing};
    hipStream_t st = S(stream);
    float *work = nullptr;
    note_allocation();
    VKH_HIP(hipMallocAsync((void **)&work, cce_work_floats(s) * 4, st));
    hipError_t e = cce_forward(PR(p->precision), s, h, w, targets, lse, loss_row, loss_mean, work, st);
    (void)hipFreeAsync(work, st);
    if (e != hipSuccess) return hip_fail(e, "cce_forward");
    return VKH_OK;
}

vkh_status vkh_cce_backward(const vkh_cce_params *p, const float *h, const float *w,
                            const uint32_t *targets, const float *lse, float *dh, float *dw,
                            uint32_t accumulate_dw, vkh_stream stream) {
    CHECK_ARG(p && h && w && targets && lse, "null pointer");
    CHECK_ARG(p->n && p->vocab && p->dim, "zero dimension");
    const CceShape s{(int)p->n, (int)p->vocab, (int)p->dim, p->z_loss_scale, p->label_smoothing};
    hipStream_t st = S(stream);
    void *dz = nullptr;
    const size_t zb = (size_t)p->n * p->vocab * (p->precision == VKH_PRECISION_BF16 ? 2 : 4);
    note_allocation();
    VKH_HIP(hipMallocAsync(&dz, zb, st));
    hipError_t e = cce_backward(PR(p->precision), s, h, w, targets, lse, dz, dh, dw,
                                accumulate_dw ? 1.f : 0.f, st);
    (void)hipFreeAsync(dz, st);
    if (e != hipSuccess) return hip_fail(e, "cce_backward");
    return VKH_OK;
}

// ── norms, rope, elementwise ───────────────────────────────────────────

vkh_status vkh_rmsnorm_forward(const float *x, const float *w, float *y, uint32_t n_rows,
                               uint32_t dim, float eps, uint32_t gq, vkh_stream stream) {
    CHECK_ARG(x && w && y, "null pointer");
    VKH_HIP(rmsnorm_forward(x, w, y, DType::F32, n_rows, dim, eps, gq ? 1 : 0, S(stream)));
    return VKH_OK;
}

vkh_status vkh_rmsnorm_backward(const float *dy, const float *x, const float *w, float *dx,
                                const float *residual, float *dw, uint32_t n_rows, uint32_t dim,
                                float eps, uint32_t gq, vkh_stream stream) {
    CHECK_ARG(dy && x && w && dx, "null pointer");
    if (dim > 4096) return fail(VKH_ERR_UNSUPPORTED, "rmsnorm_backward dim > 4096");
    hipStream_t st = S(stream);
    void *partial = nullptr;
    ScratchLease lease;
    VKH_TRY(lease.acquire(rmsnorm_partial_floats(n_rows, dim) * 4 + 16, st, &partial));
    hipError_t e = rmsnorm_backward(dy, x, w, dx, nullptr, residual, dw, (float *)partial, n_rows,
                                    dim, eps, gq ? 1 : 0, st);
    if (e != hipSuccess) return hip_fail(e, "rmsnorm_backward");
    return VKH_OK;
}

// ── the allocation-free RMSNorm backward ───────────────────────────────
// The gain-gradient partials (one row of `dim` floats per block of the
// backward kernel, at most 512 blocks and dim <= 4096) live in a fixed device
// array instead of the lease above, so a call allocates nothing (for callers
// under graph capture or in loops that must not call hipMalloc).  Each GPU
// holds its own copy for the life of the process; its device address is
// looked up once per device, at the first call on it, and only that address
// is handed to kernels.  Every block overwrites its whole partial row before
// the column sum reads it, so nothing needs clearing between calls.
//
// Calls share the array, so they are ordered like the lease's uses: an event
// per device (created with the address lookup; an event holds no device
// memory) is recorded after each call's launch, and a call on another stream
// first makes its stream wait for it.  While the caller's stream is being
// captured into a graph the event is neither waited for nor recorded (a
// captured stream may not wait on work outside its capture): the caller then
// orders the graph's launches against other uses of the array itself.
constexpr size_t kNoAllocPartialFloats = 512 * 4096;  // 8 MiB
static __device__ __align__(256) float scratch[kNoAllocPartialFloats];

namespace {
constexpr int kMaxDevices = 64;
struct NoAllocScratch {
    float *ptr = nullptr;      // the device address of `scratch` on this device
    hipEvent_t done = nullptr; // recorded after each uncaptured use
    hipStream_t last = nullptr;
    bool used = false;
};
std::mutex g_scratch_mu;
NoAllocScratch g_scratch[kMaxDevices];
}  // namespace

// Set-up of the current device's array (once per device, with the mutex held).
static vkh_status noalloc_scratch_setup(int dev) {
    NoAllocScratch &d = g_scratch[dev];
    if (d.ptr) return VKH_OK;
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    if (!p) return fail(VKH_ERR_HIP, "hipGetSymbolAddress(scratch) returned null");
    VKH_HIP(hipEventCreateWithFlags(&d.done, hipEventDisableTiming | hipEventDisableSystemFence));
    d.ptr = (float *)p;
    return VKH_OK;
}

vkh_status vkh_rmsnorm_backward_noalloc(const float *dy, const float *x, const float *w,
                                        float *dx, const float *residual, float *dw,
                                        uint32_t n_rows, uint32_t dim, float eps, uint32_t gq,
                                        vkh_stream stream) {
    CHECK_ARG(dy && x && w && dx, "null pointer");
    if (dim > 4096) return fail(VKH_ERR_UNSUPPORTED, "rmsnorm_backward_noalloc: dim %u > 4096", dim);
    const size_t need = rmsnorm_partial_floats((int)n_rows, (int)dim);
    if (need > kNoAllocPartialFloats)
        return fail(VKH_ERR_UNSUPPORTED, "rmsnorm_backward_noalloc: %zu partial floats > %zu",
                    need, kNoAllocPartialFloats);
    int dev = 0;
    VKH_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices)
        return fail(VKH_ERR_UNSUPPORTED, "device index %d >= %d", dev, kMaxDevices);
    const hipStream_t st = S(stream);
    std::lock_guard<std::mutex> lk(g_scratch_mu);  // held while the call enqueues
    VKH_TRY(noalloc_scratch_setup(dev));
    NoAllocScratch &d = g_scratch[dev];
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    VKH_HIP(hipStreamIsCapturing(st, &cs));
    const bool captured = cs != hipStreamCaptureStatusNone;
    if (!captured && d.used && d.last != st) VKH_HIP(hipStreamWaitEvent(st, d.done, 0));
    hipError_t e = rmsnorm_backward(dy, x, w, dx, nullptr, residual, dw, d.ptr, n_rows, dim, eps,
                                    gq ? 1 : 0, st);
    if (e != hipSuccess) return hip_fail(e, "rmsnorm_backward_noalloc");
    if (!captured) {
        VKH_HIP(hipEventRecord(d.done, st));
        d.used = true;
        d.last = st;
    }
    return VKH_OK;
}

uint64_t vkh_allocation_count(void) { return g_allocations.load(std::memory_order_relaxed); }

vkh_status vkh_swiglu_forward(const float *pg, const float *up, float *g, size_t n,
                              vkh_stream stream) {
    CHECK_ARG(pg && up && g, "null pointer");
    CHECK_ARG(n < (1ull << 31), "n too large");
    VKH_HIP(swiglu_forward(pg, (long)n, up, (long)n, g, (long)n, DType::F32, 1, (int)n, S(stream)));
    return VKH_OK;
}

vkh_status vkh_swiglu_backward(const float *dg, const float *pg, const float *up, float *dpg,
                               float *dup, size_t n, vkh_stream stream) {
    CHECK_ARG(dg && pg && up && dpg && dup, "null pointer");
    CHECK_ARG(n < (1ull << 31), "n too large");
    VKH_HIP(swiglu_backward(dg, (long)n, pg, (long)n, up, (long)n, dpg, (long)n, dup, (long)n,
                            DType::F32, 1, (int)n, S(stream)));
    return VKH_OK;
}

static vkh_status rope_common(const vkh_rope_params *p, const float *qi, float *qo,
                              const float *ki, float *ko, bool bw, vkh_stream stream) {
    CHECK_ARG(p && qi && qo && ki && ko, "null pointer");
    CHECK_ARG(p->rotary_dim <= p->head_dim && (p->rotary_dim % 2) == 0, "rotary_dim");
    const int seq = p->seq_len ? (int)p->seq_len : (int)p->n_pos;
    const float2 *tab = nullptr;
    VKH_TRY(rope_table_cached(seq, p->rotary_dim, p->theta_base, &tab));
    const long ldq = (long)p->n_q_heads * p->head_dim, ldk = (long)p->n_kv_heads * p->head_dim;
    VKH_HIP(qk_rope(qi, ldq, qo, ldq, ki, ldk, ko, ldk, p->n_pos, p->n_q_heads, p->n_kv_heads,
                    p->head_dim, p->rotary_dim, seq, tab, bw, S(stream)));
    return VKH_OK;
}

vkh_status vkh_qk_rope_forward(const vkh_rope_params *p, const float *q_in, float *q_out,
                               const float *k_in, float *k_out, vkh_stream stream) {
    return rope_common(p, q_in, q_out, k_in, k_out, false, stream);
}

vkh_status vkh_qk_rope_backward(const vkh_rope_params *p, const float *dq_out, float *dq_in,
                                const float *dk_out, float *dk_in, vkh_stream stream) {
    return rope_common(p, dq_out, dq_in, dk_out, dk_in, true, stream);
}

vkh_status vkh_qkv_project_bf16(const vkh_rope_params *p, uint32_t K, float eps, int qk_norm,
                                const void *x, const void *w, const float *wq, const float *wk,
                                float *y, void *out, int fused, vkh_stream stream) {
    CHECK_ARG(p && x && w && y && out, "null pointer");
    CHECK_ARG(!qk_norm || (wq && wk), "null norm gains");
    CHECK_ARG(p->rotary_dim <= p->head_dim && (p->rotary_dim % 2) == 0, "rotary_dim");
    QkvLayout L;
    L.n_rows = (int)p->n_pos; L.n_q_heads = (int)p->n_q_heads; L.n_kv_heads = (int)p->n_kv_heads;
    L.head_dim = (int)p->head_dim; L.seq_len = p->seq_len ? (int)p->seq_len : (int)p->n_pos;
    L.rotary_dim = (int)p->rotary_dim; L.theta = p->theta_base; L.eps = eps; L.qk_norm = qk_norm ? 1 : 0;
    const float2 *tab = nullptr;
    VKH_TRY(rope_table_cached(L.seq_len, L.rotary_dim, L.theta, &tab));
    const uint32_t N = (p->n_q_heads + 2 * p->n_kv_heads) * p->head_dim;
    hipStream_t st = S(stream);
    if (fused) {
        const hipError_t e = g16_qkv_norm_rope((const bf16 *)x, K, (const bf16 *)w, K, y, N, L.n_rows,
                                               (int)N, (int)K, L, wq, wk, (bf16 *)out, N, tab, st);
        if (e != hipErrorNotSupported) {
            VKH_HIP(e);
            return VKH_OK;
        }
    }
    const vkh_status r = vkh_matmul_nt_bf16(x, w, y, p->n_pos, N, K, stream);
    if (r != VKH_OK) return r;
    VKH_HIP(qkv_prepare_forward(L, y, N, wq, wk, out, N, DType::BF16, tab, st));
    return VKH_OK;
}

vkh_status vkh_qkv_project(const vkh_rope_params *p, uint32_t K, float eps, int qk_norm,
                           const float *x, const float *w, const float *wq, const float *wk,
                           float *y, float *out, int fused, vkh_stream stream) {
    CHECK_ARG(p && x && w && y && out, "null pointer");
    CHECK_ARG(!qk_norm || (wq && wk), "null norm gains");
    CHECK_ARG(p->rotary_dim <= p->head_dim && (p->rotary_dim % 2) == 0, "rotary_dim");
    QkvLayout L;
    L.n_rows = (int)p->n_pos; L.n_q_heads = (int)p->n_q_heads; L.n_kv_heads = (int)p->n_kv_heads;
    L.head_dim = (int)p->head_dim; L.seq_len = p->seq_len ? (int)p->seq_len : (int)p->n_pos;
    L.rotary_dim = (int)p->rotary_dim; L.theta = p->theta_base; L.eps = eps; L.qk_norm = qk_norm ? 1 : 0;
    const float2 *tab = nullptr;
    VKH_TRY(rope_table_cached(L.seq_len, L.rotary_dim, L.theta, &tab));
    const uint32_t N = (p->n_q_heads + 2 * p->n_kv_heads) * p->head_dim;
    hipStream_t st = S(stream);
    if (fused) {
        const hipError_t e = g32_qkv_norm_rope(x, K, w, K, y, N, L.n_rows, (int)N, (int)K, L, wq, wk,
                                               out, N, tab, st);
        if (e != hipErrorNotSupported) {
            VKH_HIP(e);
            return VKH_OK;
        }
    }
    const vkh_status r = vkh_matmul_nt(x, w, y, p->n_pos, N, K, VKH_PRECISION_FP32, stream);
    if (r != VKH_OK) return r;
    VKH_HIP(qkv_prepare_forward(L, y, N, wq, wk, out, N, DType::F32, tab, st));
    return VKH_OK;
}

vkh_status vkh_embed_lookup(const float *embed, const uint32_t *ids, float *out, uint32_t n_pos,
                            uint32_t dim, float scale, vkh_stream stream) {
    CHECK_ARG(embed && ids && out, "null pointer");
    VKH_HIP(embed_lookup(embed, ids, out, n_pos, dim, scale, S(stream)));
    return VKH_OK;
}

vkh_status vkh_embedding_backward(const float *dy, const uint32_t *ids, float *dE,
                                  uint32_t n_pos, uint32_t dim, uint32_t vocab,
                                  vkh_stream stream) {
    CHECK_ARG(dy && ids && dE, "null pointer");
    if (n_pos > (uint32_t)kEmbedBwMaxPos) return fail(VKH_ERR_UNSUPPORTED, "n_pos > %d", kEmbedBwMaxPos);
    // the owner kernels need no work buffer (no lease, no ordering event)
    hipError_t e = embedding_backward(dy, ids, dE, n_pos, dim, vocab, true, nullptr, S(stream));
    if (e != hipSuccess) return hip_fail(e, "embedding_backward");
    return VKH_OK;
}

vkh_status vkh_adam_step(float *param, const float *grad, float *m, float *v, size_t n, float lr,
                         float beta1, float beta2, float eps, uint32_t t, float wd,
                         vkh_stream stream) {
    CHECK_ARG(param && grad && m && v, "null pointer");
    CHECK_ARG(t >= 1, "t must be >= 1");
    const float tf = (float)t;
    VKH_HIP(adam_step(param, grad, m, v, n, lr, beta1, beta2, eps, 1.0f - powf(beta1, tf),
                      1.0f - powf(beta2, tf), wd, nullptr, S(stream)));
    return VKH_OK;
}

vkh_status vkh_add_in_place(float *dst, const float *src, size_t n, vkh_stream stream) {
    CHECK_ARG(dst && src, "null pointer");
    VKH_HIP(add_in_place(dst, src, n, S(stream)));
    return VKH_OK;
}

vkh_status vkh_vec_add(const float *a, const float *b, float *c, size_t n, vkh_stream stream) {
    CHECK_ARG(a && b && c, "null pointer");
    VKH_HIP(vec_add(a, b, c, n, S(stream)));
    return VKH_OK;
}

vkh_status vkh_scale(const float *in, float *out, size_t n, float s, vkh_stream stream) {
    CHECK_ARG(in && out, "null pointer");
    VKH_HIP(scale(in, out, n, s, S(stream)));
    return VKH_OK;
}

vkh_status vkh_cast_f32_to_bf16(const float *in, void *out, size_t n, vkh_stream stream) {
    CHECK_ARG(in && out, "null pointer");
    VKH_HIP(cast_f32_to_bf16(in, (bf16 *)out, n, S(stream)));
    return VKH_OK;
}

// ── plumbing ───────────────────────────────────────────────────────────

vkh_status vkh_device_count(int *count) {
    CHECK_ARG(count, "null pointer");
    *count = 0;
    hipError_t e = hipGetDeviceCount(count);
    if (e != hipSuccess) { *count = 0; return fail(VKH_ERR_NO_DEVICE, "%s", hipGetErrorString(e)); }
    return VKH_OK;
}
vkh_status vkh_set_device(int device) { VKH_HIP(hipSetDevice(device)); return VKH_OK; }
vkh_status vkh_malloc(void **ptr, size_t bytes) {
    CHECK_ARG(ptr, "null pointer");
    note_allocation();
    VKH_HIP(hipMalloc(ptr, bytes ? bytes : 1));
    return VKH_OK;
}
vkh_status vkh_free(void *ptr) { VKH_HIP(hipFree(ptr)); return VKH_OK; }
vkh_status vkh_memcpy_h2d(void *dst, const void *src, size_t bytes) {
    VKH_HIP(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
    return VKH_OK;
}
vkh_status vkh_memcpy_d2h(void *dst, const void *src, size_t bytes) {
    VKH_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
    return VKH_OK;
}
vkh_status vkh_memset(void *ptr, int value, size_t bytes) {
    VKH_HIP(hipMemset(ptr, value, bytes));
    return VKH_OK;
}
vkh_status vkh_device_synchronize(void) { VKH_HIP(hipDeviceSynchronize()); return VKH_OK; }
vkh_status vkh_stream_create(vkh_stream *out) {
    CHECK_ARG(out, "null pointer");
    hipStream_t s;
    VKH_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    *out = (vkh_stream)s;
    return VKH_OK;
}
vkh_status vkh_stream_destroy(vkh_stream s) { VKH_HIP(hipStreamDestroy(S(s))); return VKH_OK; }
vkh_status vkh_stream_synchronize(vkh_stream s) { VKH_HIP(hipStreamSynchronize(S(s))); return VKH_OK; }
vkh_status vkh_event_create(vkh_event *out) {
    CHECK_ARG(out, "null pointer");
    hipEvent_t e;
    VKH_HIP(hipEventCreate(&e));
    *out = (vkh_event)e;
    return VKH_OK;
}
vkh_status vkh_event_destroy(vkh_event e) { VKH_HIP(hipEventDestroy((hipEvent_t)e)); return VKH_OK; }
vkh_status vkh_event_record(vkh_event e, vkh_stream s) {
    VKH_HIP(hipEventRecord((hipEvent_t)e, S(s)));
    return VKH_OK;
}
vkh_status vkh_event_synchronize(vkh_event e) { VKH_HIP(hipEventSynchronize((hipEvent_t)e)); return VKH_OK; }
vkh_status vkh_event_elapsed_ms(vkh_event a, vkh_event b, float *ms) {
    CHECK_ARG(ms, "null pointer");
    VKH_HIP(hipEventElapsedTime(ms, (hipEvent_t)a, (hipEvent_t)b));
    return VKH_OK;
}

}  // extern "C"
