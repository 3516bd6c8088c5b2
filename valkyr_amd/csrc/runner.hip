// The training Runner: transformer.zig `Runner` (init / step / forwardLogits /
// checkpoints) re-expressed for one MI355X.
//
// Differences in structure from the reference (same results):
//   * Parameters, gradients and Adam moments live in four arenas with one
//     shared offset table in the canonical collectBlobs order
//     (transformer.zig:1586-1655); q/k/v and gate/up sit back to back, so
//     each pair/triple is one [N_total, dim] matrix and its forward, dx and dW
//     are single GEMMs (the q/k/v dx sum of transformer.zig:2061-2065 comes
//     out of the fused GEMM's contraction).  Adam is one launch per arena
//     span instead of 11L + 3 dispatches (transformer.zig:2072-2149).
//   * Residual adds are fused into GEMM epilogues (forward) and into the
//     RMSNorm backward (backward); norm-gain gradients are reduced on the GPU
//     (no host readbacks, transformer.zig:2151-2191).
//   * One HIP stream, no host round trips inside a step; `step` waits once at
//     the end to stay blocking like the reference.
#include <math.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <chrono>
#include <vector>

#include "internal.hpp"

// Events that only order one stream after another on this device (waited for
// with hipStreamWaitEvent, never by the host): no timing and no system-scope
// fence, which makes each record cheaper; events the host waits on before
// reading pinned memory keep the fence.
constexpr unsigned kOrderEvent = hipEventDisableTiming | hipEventDisableSystemFence;

using namespace vkh;

namespace {

struct Span {
    size_t off = 0, numel = 0;
};

struct LayerSpans {
    Span t[11];
    Span la[7], lb[7];
};

struct Acts {
    float *n1, *qkv, *attn_out, *lse, *mid, *n2, *gu, *gated, *y;
    void *qkv_attn;
    float *inter[7];
    // bf16 precision: GEMM operand copies (n1, attention output, n2, gated)
    bf16 *n1b, *attn_b, *n2b, *gatedb;
};

template <typename TO>
__global__ void init_normal_k(TO *p, size_t n, uint64_t seed, float stddev) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += stride) {
        uint64_t z = seed + 0x9E3779B97F4A7C15ull * (i / 2 + 1);
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        z ^= z >> 31;
        const double u1 = ((double)(z >> 40) + 0.5) * (1.0 / 16777216.0);
        const double u2 = ((double)(z & 0xFFFFFFull) + 0.5) * (1.0 / 16777216.0);
        const double r = sqrt(-2.0 * log(u1));
        const double a = 6.283185307179586 * u2;
        p[i] = (TO)(float)(stddev * r * ((i & 1) ? sin(a) : cos(a)));
    }
}

inline uint64_t mix(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

// Host <-> device transfers of a bf16-only tensor as fp32 values: widening
// is exact; rounding is to nearest even (the device casts' rounding).
uint16_t bf16_bits_rne(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);  // NaN stays NaN
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

vkh_status read_bf16_widened(const bf16 *dev, size_t n, float *host) {
    std::vector<uint16_t> h(n);
    VKH_HIP(hipMemcpy(h.data(), dev, n * 2, hipMemcpyDeviceToHost));
    for (size_t i = 0; i < n; ++i) {
        const uint32_t u = (uint32_t)h[i] << 16;
        memcpy(&host[i], &u, 4);
    }
    return VKH_OK;
}

vkh_status write_bf16_rounded(bf16 *dev, size_t n, const float *host) {
    std::vector<uint16_t> h(n);
    for (size_t i = 0; i < n; ++i) h[i] = bf16_bits_rne(host[i]);
    VKH_HIP(hipMemcpy(dev, h.data(), n * 2, hipMemcpyHostToDevice));
    return VKH_OK;
}

}  // namespace

struct vkh_runner {
    vkh_config cfg{};
    int T = 0, S = 0, B = 0, D = 0, H = 0, Hkv = 0, hd = 0, qd = 0, kvd = 0, qkvd = 0, F = 0,
        V = 0, L = 0, R = 0;
    bool lora = false, tied = false;
    Precision pr = Precision::FP32;
    DType adt = DType::F32;
    float aor = 0.f;

    Span embed, final_norm, lm_head;
    std::vector<LayerSpans> ls;
    size_t total = 0, tb = 0, te = 0, lora_a_begin = 0, lora_b_begin = 0;

    float *P = nullptr, *G = nullptr, *M = nullptr, *Vm = nullptr;
    // LoRA in bf16 precision (a frozen bf16 base): the base matrices (embed,
    // lm_head, the seven projections) are stored in bf16 only, in Pb, and
    // take the arena offsets below p_lo; P holds fp32 from p_lo on (the norm
    // gains and the adapters).  Elsewhere p_lo = 0 and everything has fp32.
    bool fb16 = false;
    size_t p_lo = 0;
    // bf16 precision: bf16 shadow of P (the GEMM weight operands), refreshed
    // by Adam and re-cast whenever parameters change from the host side
    bf16 *Pb = nullptr;
    bool shadow_dirty = true;
    bf16 *fn_outb = nullptr, *d_gub = nullptr, *d_midb = nullptr, *d_qkvb = nullptr,
         *dxb[2] = {nullptr, nullptr};
    bf16 *attn_ds = nullptr;  // bf16 dS of the fused attention backward (when it needs one)
    bool attn_fused = false;  // bf16 attention backward on fa_bw_fused
    bool attn_v4 = false;     // ... on its recompute kernels (no dS workspace)
    float *attn_split = nullptr;  // ... with the dK/dV launch split in two (its workspace)
    bool qk_fused = false;    // ... with RoPE^T / Q/K-norm backward in their epilogues
    // ... with the dQ kernel on a second stream beside dK/dV (one stream
    // otherwise: no side stream, and the dK/dV grid leaves CUs idle)
    bool attn_fork = false;
    // bf16 two-stream mode: the forward runs as two half batches, the first
    // on the main stream and the second on the side stream (forward_halves)
    bool half_fwd = false;
    std::vector<Acts> acts_h[2];
    hipEvent_t ev_hf = nullptr, ev_hj = nullptr;
    // fp32 two-stream mode: the head's dh done on the main stream (the table
    // updates on the side stream wait for it)
    hipEvent_t ev_dh = nullptr;
    // bf16 precision: the head forward's fp32 logits [T, V], from which
    // the backward forms dz in one pass (the fp32 precision keeps them in the
    // fp32 dz buffer itself); null where they would exceed kLogitsCap
    float *zf = nullptr;
    static constexpr size_t kLogitsCap = 8ull << 30;
    hipStream_t aux = nullptr;
    hipEvent_t ev_fork = nullptr, ev_join = nullptr;
    // LoRA: each layer's adapter gradients dA, dB (lora_cols) run on `aux`
    // too; what they read (the fused dy copies, dy B, the layer's inputs) is
    // next overwritten within the layer below's backward, which starts by
    // waiting for this layer's event (ev_laux[l]).
    bool lora_aux = false;
    std::vector<hipEvent_t> ev_laux;
    GemmWs gws{nullptr, 0};
    // Concurrent weight gradients (bf16 full fine-tune): each layer's dW GEMMs
    // and its Adam update run on a second stream one layer behind the main
    // stream's backward, reading per-layer copies of the bf16 gradients.
    struct LayerGrads {
        // the layer's gradient operands of its weight-gradient GEMMs: bf16
        // copies in the bf16 precision, the fp32 tensors themselves in fp32
        bf16 *dyb = nullptr, *gub = nullptr, *midb = nullptr, *qkvb = nullptr;
        float *dyf = nullptr, *guf = nullptr, *midf = nullptr, *qkvf = nullptr;
        // norm-gain partial sums (n1, n2, q/k norm), reduced on the side stream
        float *pn1 = nullptr, *pn2 = nullptr, *pqk = nullptr;
        int qk_parts = 0;
        // where this step's q / k gain partials went: rows of `stride` floats
        // (interleaved q|k rows from the Q/K-norm kernel, or the attention
        // kernels' separate q and k rows)
        float *pq = nullptr, *pk = nullptr;
        int q_parts = 0, k_parts = 0;
        long qk_stride = 0;
    };
    bool concurrent = false;
    // Per-layer activation recompute: each layer keeps its output y (the next
    // layer's input) and its attention output O and LSE; the other activations
    // live in kActSets sets shared in turn (layer l in set l % kActSets), and
    // a layer's forward, attention aside, runs again just before its backward
    // when later layers have reused its set.  The
    // side stream's gradient copies are shared the same way (kGradSets sets,
    // kDyRing for dy, which the layer above writes), and before layer l
    // writes any of them the main stream waits for the side stream to finish
    // layer l + 2, their previous user (ev_sdone).
    static constexpr int kActSets = 2, kGradSets = 2, kDyRing = 3;
    bool recompute = false;
    std::vector<hipEvent_t> ev_sdone;
    hipStream_t side = nullptr;
    std::vector<hipEvent_t> ev_layer;
    hipEvent_t ev_side = nullptr, ev_head = nullptr, ev_lm = nullptr;
    // Split embedding update (concurrent mode with Adam): rows of the table
    // that no token of the step names have their final gradient once the
    // head's weight gradient is written (tied) or are zero (untied), so their
    // Adam update runs on the side stream right after that GEMM; the rows the
    // tokens name (stamped in emb_mark with this step's stamp) are updated by
    // the embedding backward at the end of the step, inside its own launch.
    uint32_t *emb_mark = nullptr;
    uint32_t mark_stamp = 0;
    std::vector<LayerGrads> lg;
    GemmWs gws2{nullptr, 0};
    std::vector<Acts> acts;
    float *x_emb = nullptr, *fn_out = nullptr, *ce_lse = nullptr, *loss_row = nullptr,
          *loss_mean = nullptr;
    float *d_gated = nullptr, *d_gu = nullptr, *d_n = nullptr, *d_mid = nullptr,
          *d_attn_out = nullptr, *fa_d = nullptr, *d_qkv = nullptr, *dx[2] = {nullptr, nullptr},
          *d_fn = nullptr, *partial = nullptr, *cce_work = nullptr, *dyB = nullptr;
    bf16 *dout16 = nullptr;
    void *dz = nullptr, *embed_work = nullptr;
    float2 *rope_tab = nullptr;
    uint32_t *tok_d = nullptr, *tgt_d = nullptr;
    uint32_t *tok_h = nullptr, *tgt_h = nullptr;
    float *loss_h = nullptr;
    // loss staging (pinned): slot 0 for step / forward_backward, slot 1 for
    // the tick API's gate, each with its own event
    hipEvent_t upload_done = nullptr, loss_ready = nullptr, tick_loss_ready = nullptr;
    hipStream_t own = nullptr, cur = nullptr;
    // boundary capture (test introspection): the gradient at each layer
    // boundary l = 0..L from the last backward, (L + 1) x [T, D] fp32
    float *bnd_grad = nullptr;
    bool bnd_capture = false;
    // Ordering across streams: every enqueue ends by recording ev_done on the
    // stream it used; an enqueue on another stream first waits for it, and
    // host-side reads and writes of runner memory wait for it.
    hipEvent_t ev_done = nullptr;
    hipStream_t last_st = nullptr;
    uint32_t step_t = 1;  // transformer.zig:940
    float loss_target = 0.f;
    bool loss_pending = false, tick_loss_pending = false, batch_ready = false;
    // the tick API's cached last loss (runner.zig:932-945)
    bool has_last = false;
    float last_loss_v = 0.f;
    size_t dev_bytes = 0;
    std::vector<void *> allocs;

    ~vkh_runner() {
        if (ev_done && last_st) (void)hipEventSynchronize(ev_done);
        if (own) (void)hipStreamSynchronize(own);
        if (side) (void)hipStreamSynchronize(side);
        if (ev_done) (void)hipEventDestroy(ev_done);
        for (hipEvent_t e : ev_layer) (void)hipEventDestroy(e);
        for (hipEvent_t e : ev_sdone) (void)hipEventDestroy(e);
        if (ev_side) (void)hipEventDestroy(ev_side);
        if (ev_head) (void)hipEventDestroy(ev_head);
        if (ev_lm) (void)hipEventDestroy(ev_lm);
        if (side) (void)hipStreamDestroy(side);
        if (aux) (void)hipStreamSynchronize(aux);
        if (ev_fork) (void)hipEventDestroy(ev_fork);
        if (ev_hf) (void)hipEventDestroy(ev_hf);
        if (ev_dh) (void)hipEventDestroy(ev_dh);
        if (ev_hj) (void)hipEventDestroy(ev_hj);
        if (ev_join) (void)hipEventDestroy(ev_join);
        for (hipEvent_t e : ev_laux) (void)hipEventDestroy(e);
        if (aux) (void)hipStreamDestroy(aux);
        for (void *p : allocs) (void)hipFree(p);
        if (tok_h) (void)hipHostFree(tok_h);
        if (tgt_h) (void)hipHostFree(tgt_h);
        if (loss_h) (void)hipHostFree(loss_h);
        if (upload_done) (void)hipEventDestroy(upload_done);
        if (loss_ready) (void)hipEventDestroy(loss_ready);
        if (tick_loss_ready) (void)hipEventDestroy(tick_loss_ready);
        if (own) (void)hipStreamDestroy(own);
    }

    template <typename T_>
    vkh_status alloc(T_ *&p, size_t count) {
        const size_t bytes = count * sizeof(T_) + 256;
        void *q = nullptr;
        note_allocation();
        hipError_t e = hipMalloc(&q, bytes);
        if (e != hipSuccess)
            return fail(VKH_ERR_OUT_OF_MEMORY, "hipMalloc(%zu bytes) failed: %s", bytes,
                        hipGetErrorString(e));
        allocs.push_back(q);
        dev_bytes += bytes;
        p = (T_ *)q;
        return VKH_OK;
    }

    // ── layout ──────────────────────────────────────────────────────

    void proj_shape(int p, int &N, int &K) const {
        switch (p) {
        case 0: N = qd; K = D; break;
        case 1: case 2: N = kvd; K = D; break;
        case 3: N = D; K = qd; break;
        case 4: case 5: N = F; K = D; break;
        default: N = D; K = F; break;
        }
    }
    bool proj_lora(int p) const { return lora && (cfg.lora_targets & (1u << p)); }

    void build_layout() {
        size_t off = 0;
        auto align = [&]() { off = (off + 63) & ~size_t(63); };
        auto take = [&](Span &s, size_t n) { s.off = off; s.numel = n; off += n; };
        // fb16: the norm gains go after all matrices (from p_lo on, with fp32)
        const bool gains_here = !fb16;
        align(); take(embed, (size_t)V * D);
        if (gains_here) { align(); take(final_norm, D); }
        if (tied) lm_head = embed; else { align(); take(lm_head, (size_t)V * D); }
        ls.assign(L, LayerSpans{});
        for (int l = 0; l < L; ++l) {
            LayerSpans &s = ls[l];
            if (gains_here) { align(); take(s.t[0], D); }
            align(); take(s.t[1], (size_t)qd * D);
            take(s.t[2], (size_t)kvd * D);  // k, v directly after q: one [qkvd, D] matrix
            take(s.t[3], (size_t)kvd * D);
            align(); take(s.t[4], (size_t)D * qd);
            if (gains_here) { align(); take(s.t[5], D); }
            align(); take(s.t[6], (size_t)F * D);
            take(s.t[7], (size_t)F * D);    // up directly after gate: one [2F, D] matrix
            align(); take(s.t[8], (size_t)D * F);
            if (gains_here && cfg.qk_norm) { align(); take(s.t[9], hd); align(); take(s.t[10], hd); }
        }
        align();
        p_lo = 0;
        if (fb16) {
            p_lo = off;
            take(final_norm, D);
            for (int l = 0; l < L; ++l) {
                LayerSpans &s = ls[l];
                align(); take(s.t[0], D);
                align(); take(s.t[5], D);
                if (cfg.qk_norm) { align(); take(s.t[9], hd); align(); take(s.t[10], hd); }
            }
            align();
        }
        tb = 0;
        if (lora) {
            // all A tensors, then all B tensors (two Adam spans: lr and lr * b_scale)
            lora_a_begin = off;
            for (int p = 0; p < 7; ++p) {
                if (!proj_lora(p)) continue;
                int N, K;
                proj_shape(p, N, K);
                for (int l = 0; l < L; ++l) { align(); take(ls[l].la[p], (size_t)R * K); }
            }
            align();
            lora_b_begin = off;
            for (int p = 0; p < 7; ++p) {
                if (!proj_lora(p)) continue;
                int N, K;
                proj_shape(p, N, K);
                for (int l = 0; l < L; ++l) { align(); take(ls[l].lb[p], (size_t)N * R); }
            }
            align();
            tb = lora_a_begin;
        }
        total = off;
        te = total;
    }

    const Span *find(int layer, int which) const {
        if (layer < 0) {
            if (which == 0) return &embed;
            if (which == 1) return &final_norm;
            if (which == 2) return &lm_head;
            return nullptr;
        }
        if (layer >= L) return nullptr;
        if (which >= 0 && which < 11) return ls[layer].t[which].numel ? &ls[layer].t[which] : nullptr;
        if (which >= 16 && which < 30) {
            const int p = (which - 16) / 2;
            const Span &s = ((which - 16) % 2 == 0) ? ls[layer].la[p] : ls[layer].lb[p];
            return s.numel ? &s : nullptr;
        }
        return nullptr;
    }

    float *ptr(int kind, const Span &s) const {
        if (kind == VKH_PARAM) return bf16_only(s) ? nullptr : W(s);
        if (s.off < tb || s.off + s.numel > te) return nullptr;  // not trainable
        float *base = kind == VKH_GRAD ? G : kind == VKH_ADAM_M ? M : Vm;
        return base + (s.off - tb);
    }
    float *Pat(size_t off) const { return P + (off - p_lo); }
    float *W(const Span &s) const { return Pat(s.off); }
    bool bf16_only(const Span &s) const { return fb16 && s.numel && s.off < p_lo; }
    const bf16 *Wb(const Span &s) const { return Pb + s.off; }
    bool b16() const { return pr == Precision::BF16; }
    float *Gd(const Span &s) const { return lora ? nullptr : G + (s.off - tb); }

    // ── init ────────────────────────────────────────────────────────

    vkh_status init(const vkh_config &c) {
        cfg = c;
        if (cfg.n_seqs == 0) cfg.n_seqs = 1;
        S = cfg.n_pos; B = cfg.n_seqs; T = S * B;
        D = cfg.dim; H = cfg.n_heads; Hkv = cfg.n_kv_heads; hd = cfg.head_dim; F = cfg.ff_dim;
        V = cfg.vocab_size; L = cfg.n_layers; R = cfg.lora_rank;
        if (!D || !H || !Hkv || !hd || !F || !S || !L || !V)
            return fail(VKH_ERR_INVALID_ARGUMENT, "config has a zero dimension");
        if (H % Hkv) return fail(VKH_ERR_INVALID_ARGUMENT, "n_heads %% n_kv_heads != 0");
        if (cfg.rotary_dim > (uint32_t)hd || (cfg.rotary_dim & 1))
            return fail(VKH_ERR_INVALID_ARGUMENT, "rotary_dim must be even and <= head_dim");
        if (D % 4 || hd % 4 || F % 4)
            return fail(VKH_ERR_UNSUPPORTED, "dim, head_dim and ff_dim must be multiples of 4");
        if (hd > 256) return fail(VKH_ERR_UNSUPPORTED, "head_dim > 256");
        if (D > 4096) return fail(VKH_ERR_UNSUPPORTED, "dim > 4096");
        if (T > kEmbedBwMaxPos) return fail(VKH_ERR_UNSUPPORTED, "n_seqs * n_pos > %d", kEmbedBwMaxPos);
        if (cfg.precision > 1) return fail(VKH_ERR_INVALID_ARGUMENT, "precision");
        lora = cfg.lora_targets != 0;
        if (lora && R == 0) return fail(VKH_ERR_LORA_RANK_ZERO, "lora_rank = 0 with lora_targets");
        tied = cfg.tied_embeddings != 0;
        pr = cfg.precision == VKH_PRECISION_BF16 ? Precision::BF16 : Precision::FP32;
        adt = (pr == Precision::BF16 && (hd == 64 || hd == 128)) ? DType::BF16 : DType::F32;
        aor = lora ? cfg.lora_alpha / (float)R : 0.f;
        fb16 = lora && pr == Precision::BF16;
        qd = H * hd; kvd = Hkv * hd; qkvd = qd + 2 * kvd;
        build_layout();

        VKH_HIP(hipStreamCreateWithFlags(&own, hipStreamNonBlocking));
        cur = own;
        VKH_HIP(hipEventCreateWithFlags(&upload_done, hipEventDisableTiming));
        VKH_HIP(hipEventCreateWithFlags(&loss_ready, hipEventDisableTiming));
        VKH_HIP(hipEventCreateWithFlags(&tick_loss_ready, hipEventDisableTiming));
        VKH_HIP(hipEventCreateWithFlags(&ev_done, hipEventDisableTiming));
        note_allocation();
        VKH_HIP(hipHostMalloc((void **)&tok_h, (size_t)T * 4, hipHostMallocDefault));
        VKH_HIP(hipHostMalloc((void **)&tgt_h, (size_t)T * 4, hipHostMallocDefault));
        VKH_HIP(hipHostMalloc((void **)&loss_h, 16, hipHostMallocDefault));

        VKH_TRY(alloc(P, total - p_lo));
        VKH_HIP(hipMemsetAsync(P, 0, (total - p_lo) * 4, own));
        if (b16()) VKH_TRY(alloc(Pb, total));
        // bf16-only base matrices start at zero like the fp32 ones (the shadow
        // cast never writes them)
        if (p_lo) VKH_HIP(hipMemsetAsync(Pb, 0, p_lo * sizeof(bf16), own));
        const size_t nt = te - tb;
        VKH_TRY(alloc(G, nt));
        VKH_TRY(alloc(M, nt));
        VKH_TRY(alloc(Vm, nt));
        VKH_HIP(hipMemsetAsync(G, 0, nt * 4, own));
        VKH_HIP(hipMemsetAsync(M, 0, nt * 4, own));
        VKH_HIP(hipMemsetAsync(Vm, 0, nt * 4, own));
        // norm gains start at one
        auto ones = [&](const Span &s) -> vkh_status {
            if (s.numel) VKH_HIP(fill_f32(W(s), s.numel, 1.0f, own));
            return VKH_OK;
        };
        VKH_TRY(ones(final_norm));
        for (int l = 0; l < L; ++l) {
            VKH_TRY(ones(ls[l].t[0])); VKH_TRY(ones(ls[l].t[5]));
            VKH_TRY(ones(ls[l].t[9])); VKH_TRY(ones(ls[l].t[10]));
        }

        const size_t asz = adt == DType::BF16 ? 2 : 4;
        recompute = cfg.recompute != 0;
        concurrent = !lora;
        const int n_sets = recompute ? std::min(L, kActSets) : L;
        acts.assign(L, Acts{});
        for (int l = 0; l < L; ++l) {
            Acts &a = acts[l];
            if (l >= n_sets) {
                // recompute: set l % n_sets, own output y and own attention
                // output O and LSE (the recompute reruns projections, norms and
                // SwiGLU, not the attention)
                a = acts[l % n_sets];
                VKH_TRY(alloc(a.y, (size_t)T * D));
                VKH_TRY(alloc(a.lse, (size_t)T * H));
                if (b16()) VKH_TRY(alloc(a.attn_b, (size_t)T * qd));
                if (!(b16() && adt == DType::BF16)) VKH_TRY(alloc(a.attn_out, (size_t)T * qd));
                continue;
            }
            if (b16()) {
                VKH_TRY(alloc(a.n1b, (size_t)T * D));
                VKH_TRY(alloc(a.attn_b, (size_t)T * qd));
                VKH_TRY(alloc(a.n2b, (size_t)T * D));
                VKH_TRY(alloc(a.gatedb, (size_t)T * F));
            } else {
                VKH_TRY(alloc(a.n1, (size_t)T * D));
                VKH_TRY(alloc(a.n2, (size_t)T * D));
                VKH_TRY(alloc(a.gated, (size_t)T * F));
            }
            VKH_TRY(alloc(a.qkv, (size_t)T * qkvd));
            char *qa = nullptr;
            VKH_TRY(alloc(qa, (size_t)T * qkvd * asz));
            a.qkv_attn = qa;
            // the fp32 O feeds only the fp32 path: the bf16 path keeps O in
            // bf16 (the O projection's operand and the D preprocess's input)
            if (!(b16() && adt == DType::BF16)) VKH_TRY(alloc(a.attn_out, (size_t)T * qd));
            VKH_TRY(alloc(a.lse, (size_t)T * H));
            VKH_TRY(alloc(a.mid, (size_t)T * D));
            VKH_TRY(alloc(a.gu, (size_t)T * 2 * F));
            VKH_TRY(alloc(a.y, (size_t)T * D));
            for (int p = 0; p < 7; ++p) {
                a.inter[p] = nullptr;
                if (proj_lora(p)) VKH_TRY(alloc(a.inter[p], (size_t)T * R));
            }
        }
        VKH_TRY(alloc(x_emb, (size_t)T * D));
        if (b16()) {
            VKH_TRY(alloc(fn_outb, (size_t)T * D));
            if (!concurrent) {  // concurrent mode uses the per-layer copies (lg)
                VKH_TRY(alloc(d_gub, (size_t)T * 2 * F));
                VKH_TRY(alloc(d_midb, (size_t)T * D));
                VKH_TRY(alloc(d_qkvb, (size_t)T * qkvd));
                VKH_TRY(alloc(dxb[0], (size_t)T * D));
                VKH_TRY(alloc(dxb[1], (size_t)T * D));
            }
            attn_fused = adt == DType::BF16 && fa_bw_fused_ok(attn_shape());
            attn_v4 = attn_fused && fa_bw_v4_preferred(attn_shape());
            qk_fused = attn_v4 && fa_bw_qk_epi_ok(attn_shape(), (int)cfg.rotary_dim);
            attn_fork = attn_v4 && lora && fa_bw_v4_kv_blocks(attn_shape()) < 256;
            if (attn_v4 && fa_bw_v4_split(attn_shape()))
                VKH_TRY(alloc(attn_split, fa_bw_v4_split_ws_floats(attn_shape())));
            if (attn_fused && fa_bw_ws_bytes(attn_shape(), attn_v4))
                VKH_TRY(alloc(attn_ds, fa_bw_ws_bytes(attn_shape(), attn_v4) / sizeof(bf16)));
            // split-K workspace: the largest the planner asks for over the step's GEMMs
            size_t wsb = 0;
            auto need = [&](int m, int n, int k) { wsb = std::max(wsb, g16_ws_bytes_for(m, n, k)); };
            need(T, qkvd, D); need(T, D, qd); need(T, 2 * F, D); need(T, D, F);
            need(T, F, D); need(T, D, 2 * F); need(T, qd, D); need(T, D, qkvd);
            need(D, F, T); need(2 * F, D, T); need(D, qd, T); need(qkvd, D, T);
            need(T, D, V); need(V, D, T);
            if (wsb) {
                char *w = nullptr;
                VKH_TRY(alloc(w, wsb));
                gws = GemmWs{w, wsb};
            }
        } else {
            VKH_TRY(alloc(fn_out, (size_t)T * D));
            // split-K workspace of the fp32 GEMMs (g32_*), if their plan asks for one
            size_t wsb = 0;
            auto need = [&](int m, int n, int k) { wsb = std::max(wsb, g32_ws_bytes_for(m, n, k)); };
            need(T, qkvd, D); need(T, D, qd); need(T, 2 * F, D); need(T, D, F);
            need(T, F, D); need(T, D, 2 * F); need(T, qd, D); need(T, D, qkvd);
            need(D, F, T); need(2 * F, D, T); need(D, qd, T); need(qkvd, D, T);
            if (wsb) {
                char *w = nullptr;
                VKH_TRY(alloc(w, wsb));
                gws = GemmWs{w, wsb};
            }
        }
        if (concurrent) {
            // the side stream (weight gradients, Adam) and each layer's gradient
            // operands for it, in the step's precision
            VKH_HIP(hipStreamCreateWithFlags(&side, hipStreamNonBlocking));
            ev_layer.assign(L, nullptr);
            for (int l = 0; l < L; ++l)
                VKH_HIP(hipEventCreateWithFlags(&ev_layer[l], kOrderEvent));
            VKH_HIP(hipEventCreateWithFlags(&ev_dh, kOrderEvent));
            half_fwd = b16() && !recompute && B % 2 == 0;
            if (half_fwd) {
                VKH_HIP(hipEventCreateWithFlags(&ev_hf, kOrderEvent));
                VKH_HIP(hipEventCreateWithFlags(&ev_hj, kOrderEvent));
            }
            if (recompute) {
                ev_sdone.assign(L, nullptr);
                for (int l = 0; l < L; ++l)
                    VKH_HIP(hipEventCreateWithFlags(&ev_sdone[l], kOrderEvent));
            }
            VKH_HIP(hipEventCreateWithFlags(&ev_side, kOrderEvent));
            VKH_HIP(hipEventCreateWithFlags(&ev_head, kOrderEvent));
            VKH_HIP(hipEventCreateWithFlags(&ev_lm, kOrderEvent));
            if (embed_split_ok()) {
                VKH_TRY(alloc(emb_mark, (size_t)V));
                VKH_HIP(fill_f32(reinterpret_cast<float *>(emb_mark), (size_t)V, 0.f, own));
            }
            lg.assign(L, LayerGrads{});
            const int n_g = recompute ? std::min(L, kGradSets) : L;
            const int n_dy = recompute ? std::min(L, kDyRing) : L;
            for (int l = 0; l < L; ++l) {
                if (l < n_dy) {
                    if (b16()) VKH_TRY(alloc(lg[l].dyb, (size_t)T * D));
                    else VKH_TRY(alloc(lg[l].dyf, (size_t)T * D));
                } else {
                    lg[l].dyb = lg[l % n_dy].dyb;
                    lg[l].dyf = lg[l % n_dy].dyf;
                }
                if (l >= n_g) {
                    const LayerGrads &o = lg[l % n_g];
                    lg[l].gub = o.gub; lg[l].midb = o.midb; lg[l].qkvb = o.qkvb;
                    lg[l].guf = o.guf; lg[l].midf = o.midf; lg[l].qkvf = o.qkvf;
                    lg[l].pn1 = o.pn1; lg[l].pn2 = o.pn2; lg[l].pqk = o.pqk;
                    continue;
                }
                if (b16()) {
                    VKH_TRY(alloc(lg[l].gub, (size_t)T * 2 * F));
                    VKH_TRY(alloc(lg[l].midb, (size_t)T * D));
                    VKH_TRY(alloc(lg[l].qkvb, (size_t)T * qkvd));
                } else {
                    VKH_TRY(alloc(lg[l].guf, (size_t)T * 2 * F));
                    VKH_TRY(alloc(lg[l].midf, (size_t)T * D));
                    VKH_TRY(alloc(lg[l].qkvf, (size_t)T * qkvd));
                }
                VKH_TRY(alloc(lg[l].pn1, rmsnorm_partial_floats(T, D)));
                VKH_TRY(alloc(lg[l].pn2, rmsnorm_partial_floats(T, D)));
                if (cfg.qk_norm) VKH_TRY(alloc(lg[l].pqk, qk_partial_floats()));
            }
            // the side stream's own split-K workspace
            size_t wsb2 = 0;
            auto need2 = [&](int m, int n, int k) {
                wsb2 = std::max(wsb2, b16() ? g16_ws_bytes_for(m, n, k) : g32_ws_bytes_for(m, n, k));
            };
            need2(D, F, T); need2(2 * F, D, T); need2(D, qd, T); need2(qkvd, D, T); need2(V, D, T);
            if (wsb2) {
                char *w = nullptr;
                VKH_TRY(alloc(w, wsb2));
                gws2 = GemmWs{w, wsb2};
            }
        }
        VKH_TRY(alloc(ce_lse, T));
        VKH_TRY(alloc(loss_row, T));
        VKH_TRY(alloc(loss_mean, 4));
        VKH_TRY(alloc(d_gated, (size_t)T * F));
        if (!b16()) VKH_TRY(alloc(d_gu, (size_t)T * 2 * F));
        VKH_TRY(alloc(d_n, (size_t)T * D));
        VKH_TRY(alloc(d_mid, (size_t)T * D));
        VKH_TRY(alloc(d_attn_out, (size_t)T * qd));
        VKH_TRY(alloc(fa_d, (size_t)T * H));
        VKH_TRY(alloc(d_qkv, (size_t)T * qkvd));
        VKH_TRY(alloc(dx[0], (size_t)T * D));
        VKH_TRY(alloc(dx[1], (size_t)T * D));
        VKH_TRY(alloc(d_fn, (size_t)T * D));
        if (adt == DType::BF16) VKH_TRY(alloc(dout16, (size_t)T * qd));
        size_t pf = rmsnorm_partial_floats(T, D);
        if (qk_partial_floats() > pf) pf = qk_partial_floats();
        VKH_TRY(alloc(partial, pf));
        CceShape cs{T, V, D, 0.f, 0.f};
        VKH_TRY(alloc(cce_work, cce_work_floats(cs)));
        char *z = nullptr;
        VKH_TRY(alloc(z, (size_t)T * V * (b16() ? 2 : 4)));
        // 18.41-18.47 -> 18.27-18.29 ms at config 3 (1.24 GB), same losses; config 5
        // (8192 tokens, 4.98 GB): 587.4 -> 581.4-581.7 ms in 157.1 GiB
        if (b16() && (size_t)T * V * 4 <= kLogitsCap) VKH_TRY(alloc(zf, (size_t)T * V));
        dz = z;
        char *ew = nullptr;
        VKH_TRY(alloc(ew, embed_bw_work_bytes(T)));
        embed_work = ew;
        if (lora) VKH_TRY(alloc(dyB, (size_t)7 * T * R));  // dy B of each adapter
        lora_aux = lora;
        if (attn_fork || lora_aux) {
            VKH_HIP(hipStreamCreateWithFlags(&aux, hipStreamNonBlocking));
            VKH_HIP(hipEventCreateWithFlags(&ev_fork, kOrderEvent));
            VKH_HIP(hipEventCreateWithFlags(&ev_join, kOrderEvent));
        }
        if (lora_aux) {
            ev_laux.assign(L, nullptr);
            for (int l = 0; l < L; ++l)
                VKH_HIP(hipEventCreateWithFlags(&ev_laux[l], kOrderEvent));
        }
        VKH_TRY(alloc(tok_d, T));
        VKH_TRY(alloc(tgt_d, T));
        if (cfg.rotary_dim > 0) {
            const int half = cfg.rotary_dim / 2;
            std::vector<float2> tab((size_t)S * half);
            rope_table_host(tab.data(), S, cfg.rotary_dim, cfg.rope_theta);
            VKH_TRY(alloc(rope_tab, tab.size()));
            VKH_HIP(hipMemcpy(rope_tab, tab.data(), tab.size() * sizeof(float2), hipMemcpyHostToDevice));
        }
        VKH_HIP(hipStreamSynchronize(own));
        return VKH_OK;
    }

    // floats of q / k gain partials one layer's backward writes (either path)
    size_t qk_partial_floats() const {
        size_t n = qkv_partial_floats(qkv_layout());
        if (!b16() && cfg.qk_norm) {  // the fp32 tile kernels' fused epilogue
            const AttnShape as = attn_shape();
            if (fa_f32m_ok(as))
                n = std::max(n, (size_t)(fa_f32m_dq_blocks(as) + fa_f32m_dkv_blocks(as)) * hd);
        }
        if (qk_fused) {
            const AttnShape as = attn_shape();
            n = std::max(n, (size_t)(fa_bw_v4_q_blocks(as) + fa_bw_v4_k_gain_parts(as, attn_split)) * hd);
        }
        return n;
    }

    QkvLayout qkv_layout() const {
        QkvLayout q;
        q.n_rows = T; q.n_q_heads = H; q.n_kv_heads = Hkv; q.head_dim = hd;
        q.seq_len = S; q.rotary_dim = cfg.rotary_dim; q.theta = cfg.rope_theta;
        q.eps = cfg.rms_eps; q.qk_norm = cfg.qk_norm ? 1 : 0;
        return q;
    }

    AttnShape attn_shape() const {
        AttnShape s;
        s.n_batch = B; s.n_q = S; s.n_kv = S; s.n_heads = H; s.n_kv_heads = Hkv;
        s.head_dim = hd; s.causal = cfg.causal ? 1 : 0;
        s.inv_sqrt_dim = 1.0f / sqrtf((float)hd);
        return s;
    }

    // a bf16-only base matrix from host fp32 values (rounded to nearest even)
    vkh_status upload_bf16(const Span &s, const float *host) {
        return write_bf16_rounded(Pb + s.off, s.numel, host);
    }

    vkh_status upload_weights(const vkh_init_weights &w) {
        const size_t qdim = (size_t)qd, kvdim = (size_t)kvd;
        if (w.embed.len != (size_t)V * D) return fail(VKH_ERR_EMBED_SHAPE, "embed len %zu", w.embed.len);
        if (w.final_norm.len != (size_t)D) return fail(VKH_ERR_FINAL_NORM_SHAPE, "final_norm len");
        if (!tied && w.lm_head.len != (size_t)V * D) return fail(VKH_ERR_LM_HEAD_SHAPE, "lm_head len");
        if (w.n_layers != (size_t)L || (!w.layers && L)) return fail(VKH_ERR_LAYER_COUNT, "layer count");
        for (int l = 0; l < L; ++l) {
            const vkh_layer_weights &lw = w.layers[l];
            if (lw.w_n1.len != (size_t)D) return fail(VKH_ERR_LAYER_N1_SHAPE, "layer %d n1", l);
            if (lw.w_q.len != qdim * D) return fail(VKH_ERR_LAYER_Q_SHAPE, "layer %d q", l);
            if (lw.w_k.len != kvdim * D) return fail(VKH_ERR_LAYER_K_SHAPE, "layer %d k", l);
            if (lw.w_v.len != kvdim * D) return fail(VKH_ERR_LAYER_V_SHAPE, "layer %d v", l);
            if (lw.w_o.len != (size_t)D * qdim) return fail(VKH_ERR_LAYER_O_SHAPE, "layer %d o", l);
            if (lw.w_n2.len != (size_t)D) return fail(VKH_ERR_LAYER_N2_SHAPE, "layer %d n2", l);
            if (lw.w_gate.len != (size_t)F * D) return fail(VKH_ERR_LAYER_GATE_SHAPE, "layer %d gate", l);
            if (lw.w_up.len != (size_t)F * D) return fail(VKH_ERR_LAYER_UP_SHAPE, "layer %d up", l);
            if (lw.w_down.len != (size_t)D * F) return fail(VKH_ERR_LAYER_DOWN_SHAPE, "layer %d down", l);
            if (cfg.qk_norm) {
                if (lw.w_q_norm.len != (size_t)hd) return fail(VKH_ERR_LAYER_Q_NORM_SHAPE, "layer %d q_norm", l);
                if (lw.w_k_norm.len != (size_t)hd) return fail(VKH_ERR_LAYER_K_NORM_SHAPE, "layer %d k_norm", l);
            }
        }
        for (int p = 0; p < 7; ++p)
            if (proj_lora(p) && w.lora[p] && w.lora_len[p] != (size_t)L)
                return fail(VKH_ERR_LORA_INIT_LEN, "lora init for projection %d has %zu layers", p, w.lora_len[p]);
        auto up = [&](const Span &s, const vkh_tensor &t) -> vkh_status {
            if (!s.numel || !t.data) return VKH_OK;
            if (bf16_only(s)) return upload_bf16(s, t.data);
            VKH_HIP(hipMemcpy(W(s), t.data, s.numel * 4, hipMemcpyHostToDevice));
            return VKH_OK;
        };
        VKH_TRY(up(embed, w.embed));
        VKH_TRY(up(final_norm, w.final_norm));
        if (!tied) VKH_TRY(up(lm_head, w.lm_head));
        for (int l = 0; l < L; ++l) {
            const vkh_layer_weights &lw = w.layers[l];
            const vkh_tensor *tt[11] = {&lw.w_n1, &lw.w_q, &lw.w_k, &lw.w_v, &lw.w_o, &lw.w_n2,
                                        &lw.w_gate, &lw.w_up, &lw.w_down, &lw.w_q_norm, &lw.w_k_norm};
            for (int i = 0; i < 11; ++i) VKH_TRY(up(ls[l].t[i], *tt[i]));
        }
        for (int p = 0; p < 7; ++p) {
            if (!proj_lora(p)) continue;
            if (w.lora[p]) {
                for (int l = 0; l < L; ++l) {
                    int N, K;
                    proj_shape(p, N, K);
                    if (w.lora[p][l].a.len != (size_t)R * K || w.lora[p][l].b.len != (size_t)N * R)
                        return fail(VKH_ERR_LORA_INIT_LEN, "lora init shape, projection %d layer %d", p, l);
                    VKH_TRY(up(ls[l].la[p], w.lora[p][l].a));
                    VKH_TRY(up(ls[l].lb[p], w.lora[p][l].b));
                }
            } else {
                VKH_TRY(lora_default_init(p));
            }
        }
        return VKH_OK;
    }

    // transformer.zig:2568-2574: A ~ N(0, 1/sqrt(r)) from a fixed seed, B = 0
    vkh_status lora_default_init(int p) {
        const float sigma = 1.0f / sqrtf((float)R);
        for (int l = 0; l < L; ++l) {
            const Span &a = ls[l].la[p];
            hipLaunchKernelGGL(init_normal_k<float>, dim3(256), dim3(256), 0, own, W(a), a.numel,
                               mix(0x10AAFADEull ^ ((uint64_t)p << 32) ^ (uint64_t)l), sigma);
            VKH_HIP(hipGetLastError());
        }
        return VKH_OK;
    }

    vkh_status init_random(uint64_t seed, float std_, float lora_std) {
        VKH_TRY(host_wait());
        shadow_dirty = true;
        auto normal = [&](const Span &s, uint64_t tag, float sd) -> vkh_status {
            if (!s.numel) return VKH_OK;
            const unsigned g = (unsigned)std::min<size_t>(4096, (s.numel + 255) / 256);
            if (bf16_only(s))
                hipLaunchKernelGGL(init_normal_k<bf16>, dim3(g ? g : 1), dim3(256), 0, own, Pb + s.off,
                                   s.numel, mix(seed ^ mix(tag)), sd);
            else
                hipLaunchKernelGGL(init_normal_k<float>, dim3(g ? g : 1), dim3(256), 0, own, W(s),
                                   s.numel, mix(seed ^ mix(tag)), sd);
            VKH_HIP(hipGetLastError());
            return VKH_OK;
        };
        auto ones = [&](const Span &s) -> vkh_status {
            if (s.numel) VKH_HIP(fill_f32(W(s), s.numel, 1.0f, own));
            return VKH_OK;
        };
        VKH_TRY(normal(embed, 1, std_));
        VKH_TRY(ones(final_norm));
        if (!tied) VKH_TRY(normal(lm_head, 2, std_));
        for (int l = 0; l < L; ++l)
            for (int t = 0; t < 11; ++t) {
                if (t == 0 || t == 5 || t == 9 || t == 10) VKH_TRY(ones(ls[l].t[t]));
                else VKH_TRY(normal(ls[l].t[t], 1000 + 16 * (uint64_t)l + t, std_));
            }
        for (int p = 0; p < 7; ++p)
            for (int l = 0; l < L; ++l) {
                if (ls[l].la[p].numel) VKH_TRY(normal(ls[l].la[p], 500000 + 64 * (uint64_t)p + l, lora_std));
                if (ls[l].lb[p].numel) VKH_HIP(hipMemsetAsync(W(ls[l].lb[p]), 0, ls[l].lb[p].numel * 4, own));
            }
        VKH_HIP(hipStreamSynchronize(own));
        return VKH_OK;
    }

    // ── forward ─────────────────────────────────────────────────────

    // y = x W^T for one projection p, plus the LoRA term when p is a target
    // (train/lora.zig:99-129; oracle lora.zig:75-121).
    vkh_status lora_fwd(int l, int p, Mat x, float *y, long ldy) {
        int N, K;
        proj_shape(p, N, K);
        float *Bm = W(ls[l].lb[p]);
        float *inter = acts[l].inter[p];
        VKH_TRY(lora_inter(l, p, x));
        VKH_HIP(gemm_nt(pr, matf(inter, R), matf(Bm, R), y, ldy, T, N, R, nullptr, 0, aor, 1.f, cur));
        return VKH_OK;
    }
    // column of projection p in its fused output (and fused gradient)
    long proj_col(int p) const {
        return p == 1 ? qd : p == 2 ? qd + kvd : p == 5 ? F : 0;
    }
    // The LoRA terms of the targets among projections `ps`, which share the
    // input x: inter_p = x A_p^T (one launch), then, with need_y, y[:, col_p
    // ..] += aor inter_p B_p^T (one launch); the rank-r kernels where the
    // shapes allow, else the general GEMMs per projection.
    // The adapters of layer l among projections ps (one group of the fused layout).
    int lora_adapters(int l, std::initializer_list<int> ps, LoraAdapter (&ad)[3]) {
        int na = 0;
        for (int p : ps) {
            if (!proj_lora(p)) continue;
            LoraAdapter &a = ad[na++];
            proj_shape(p, a.n, a.k);
            a.col = proj_col(p);
            a.a = W(ls[l].la[p]);
            a.b = W(ls[l].lb[p]);
            a.inter = acts[l].inter[p];
            a.dyb = dyB + (size_t)p * T * R;
            a.da = G + (ls[l].la[p].off - tb);
            a.db = G + (ls[l].lb[p].off - tb);
        }
        return na;
    }
    vkh_status lora_fwd_group(int l, std::initializer_list<int> ps, Mat x, float *y, long ldy,
                              bool need_y = true) {
        LoraAdapter ad[3];
        const int na = lora_adapters(l, ps, ad);
        if (!na) return VKH_OK;
        const LoraGroupSegs gs = lora_group_segs(ad, na, R);
        const LoraSegs &sa = gs.fwd_rows, &sb = gs.fwd_upd;
        if (lora_fast_ok(x.dt, x.p, x.ld, R, sa) && (!need_y || lora_update_ok(y, ldy, R, sb))) {
            VKH_HIP(lora_rows(x.dt, x.p, x.ld, T, R, sa, 1.f, cur));
            if (need_y) VKH_HIP(lora_update(y, ldy, T, R, sb, aor, cur));
            return VKH_OK;
        }
        for (int p : ps) {
            if (!proj_lora(p)) continue;
            if (need_y) VKH_TRY(lora_fwd(l, p, x, y + proj_col(p), ldy));
            else VKH_TRY(lora_inter(l, p, x));
        }
        return VKH_OK;
    }
    // y = x W^T (+ Rr) with the LoRA terms of the targets among `ps`: in the
    // bf16 precision the update rides in the GEMM's epilogue (inter first,
    // then one GEMM), else the GEMM and lora_fwd_group's update pass.
    vkh_status linear_fwd_lora(int l, std::initializer_list<int> ps, Mat x, const Span &w, float *y,
                               long ldy, int N, int K, const float *Rr, long ldr) {
        LoraAdapter ad[3];
        const int na = b16() ? lora_adapters(l, ps, ad) : 0;
        if (na) {
            const LoraGroupSegs gs = lora_group_segs(ad, na, R);
            if (lora_fast_ok(x.dt, x.p, x.ld, R, gs.fwd_rows) &&
                g16_lora_ok((const bf16 *)x.p, x.ld, T, K, Wb(w), K, N, K, gs.fwd_upd, R, N)) {
                VKH_HIP(lora_rows(x.dt, x.p, x.ld, T, R, gs.fwd_rows, 1.f, cur));
                VKH_HIP(g16_nt_lora((const bf16 *)x.p, x.ld, Wb(w), K, y, ldy, T, N, K, Rr, ldr,
                                    gs.fwd_upd, R, aor, gws, cur));
                return VKH_OK;
            }
        }
        VKH_TRY(linear_fwd(x, w, y, ldy, N, K, Rr, ldr));
        return lora_fwd_group(l, ps, x, y, ldy);
    }
    // Whether dx_lora can fuse the LoRA dx term of `ps` into the dx GEMM.
    bool dx_lora_fused(int l, std::initializer_list<int> ps, Mat dy, Mat x, const Span &w, int N,
                       int K) {
        LoraAdapter ad[3];
        const int na = b16() ? lora_adapters(l, ps, ad) : 0;
        if (!na) return false;
        const LoraGroupSegs gs = lora_group_segs(ad, na, R);
        return lora_fast_ok(dy.dt, dy.p, dy.ld, R, gs.bwd_rows) &&
               lora_fast_ok(x.dt, x.p, x.ld, R, gs.bwd_da) &&
               lora_fast_ok(dy.dt, dy.p, dy.ld, R, gs.bwd_db) &&
               g16_lora_ok((const bf16 *)dy.p, dy.ld, T, N, Wb(w), K, N, K, gs.bwd_upd, R, K);
    }
    // dx = dy W plus the LoRA backward of the targets among `ps` (dx term,
    // dA, dB): where dx_lora_fused holds, dy B first, dA / dB on the side
    // stream, and the dx term in the dx GEMM's epilogue (fp32 dx, or bf16
    // into dxb); otherwise the GEMM then lora_bwd_group (fp32 dx only).
    vkh_status dx_lora(int l, std::initializer_list<int> ps, Mat dy, Mat x, const Span &w, float *dx,
                       bf16 *dxb, long lddx, int N, int K) {
        if (!dx_lora_fused(l, ps, dy, x, w, N, K)) {
            if (dxb) return fail(VKH_ERR_UNSUPPORTED, "bf16 dx with an unfused LoRA term");
            VKH_TRY(linear_dx(dy, w, dx, lddx, N, K));
            return lora_bwd_group(l, ps, dy, x, dx, lddx);
        }
        LoraAdapter ad[3];
        const int na = lora_adapters(l, ps, ad);
        const LoraGroupSegs gs = lora_group_segs(ad, na, R);
        VKH_HIP(lora_rows(dy.dt, dy.p, dy.ld, T, R, gs.bwd_rows, 1.f, cur));
        hipStream_t cs = cur;
        if (lora_aux) {
            VKH_HIP(hipEventRecord(ev_fork, cur));
            VKH_HIP(hipStreamWaitEvent(aux, ev_fork, 0));
            cs = aux;
        }
        VKH_HIP(lora_cols(x.dt, x.p, x.ld, T, R, gs.bwd_da, aor, cs));
        VKH_HIP(lora_cols(dy.dt, dy.p, dy.ld, T, R, gs.bwd_db, aor, cs));
        if (dxb)
            VKH_HIP(g16_nn_bf16_lora((const bf16 *)dy.p, dy.ld, Wb(w), K, dxb, lddx, T, N, K,
                                     gs.bwd_upd, R, aor, gws, cur));
        else
            VKH_HIP(g16_nn_lora((const bf16 *)dy.p, dy.ld, Wb(w), K, dx, lddx, T, N, K, gs.bwd_upd, R,
                                aor, gws, cur));
        return VKH_OK;
    }
    // inter = x A^T, the rank-r intermediate the LoRA backward reads (dB)
    vkh_status lora_inter(int l, int p, Mat x) {
        int N, K;
        proj_shape(p, N, K);
        VKH_HIP(gemm_nt(pr, x, matf(W(ls[l].la[p]), K), acts[l].inter[p], R, T, R, K, nullptr, 0,
                        1.f, 0.f, cur));
        return VKH_OK;
    }

    static Mat matb(const bf16 *p, long ld) { return Mat{p, ld, DType::BF16}; }

    // y[T, N] = x[T, K] W[N, K]^T (+ R residual): bf16 shadow operands in the
    // bf16 precision, fp32 operands otherwise.
    vkh_status linear_fwd(Mat x, const Span &w, float *y, long ldy, int N, int K, const float *R,
                          long ldr) {
        if (b16())
            VKH_HIP(g16_nt((const bf16 *)x.p, x.ld, Wb(w), K, y, ldy, T, N, K, R, ldr, 1.f, 0.f, gws, cur));
        else
            VKH_HIP(g32_nt((const float *)x.p, x.ld, W(w), K, y, ldy, T, N, K, R, ldr, 1.f, 0.f, gws, cur));
        return VKH_OK;
    }
    // dx[T, K] = dy[T, N] W[N, K]
    vkh_status linear_dx(Mat dy, const Span &w, float *dx, long lddx, int N, int K) {
        if (b16())
            VKH_HIP(g16_nn((const bf16 *)dy.p, dy.ld, Wb(w), K, dx, lddx, T, N, K, 1.f, 0.f, gws, cur));
        else
            VKH_HIP(g32_nn((const float *)dy.p, dy.ld, W(w), K, dx, lddx, T, N, K, 1.f, 0.f, gws, cur));
        return VKH_OK;
    }
    // dW[N, K] = dy[T, N]^T x[T, K] (overwrite)
    vkh_status linear_dw(Mat dy, Mat x, const Span &w, int N, int K) {
        return linear_dw_on(dy, x, w, N, K, gws, cur);
    }
    vkh_status linear_dw_on(Mat dy, Mat x, const Span &w, int N, int K, const GemmWs &ws,
                            hipStream_t st) {
        if (lora) return VKH_OK;  // base weights frozen
        if (b16())
            VKH_HIP(g16_tn((const bf16 *)dy.p, dy.ld, (const bf16 *)x.p, x.ld, Gd(w), K, T, N, K, 1.f,
                           0.f, ws, st));
        else
            VKH_HIP(g32_tn((const float *)dy.p, dy.ld, (const float *)x.p, x.ld, Gd(w), K, T, N, K, 1.f,
                           0.f, ws, st));
        return VKH_OK;
    }
    // The four weight-gradient GEMMs of layer l on the side stream (concurrent
    // mode); with gains_in_adam the norm-gain gradients are left as partials
    // for adam_layer_side to reduce.
    vkh_status layer_dw_side(int l, bool gains_in_adam) {
        Acts &a = acts[l];
        LayerSpans &s = ls[l];
        const LayerGrads &g = lg[l];
        const bool h = b16();
        VKH_TRY(linear_dw_on(h ? matb(g.dyb, D) : matf(g.dyf, D), m_gated(a), s.t[8], D, F, gws2, side));
        VKH_TRY(linear_dw_on(h ? matb(g.gub, 2 * F) : matf(g.guf, 2 * F), m_n2(a), s.t[6], 2 * F, D,
                             gws2, side));
        VKH_TRY(linear_dw_on(h ? matb(g.midb, D) : matf(g.midf, D), m_attn(a), s.t[4], D, qd, gws2, side));
        VKH_TRY(linear_dw_on(h ? matb(g.qkvb, qkvd) : matf(g.qkvf, qkvd), m_n1(a), s.t[1], qkvd, D,
                             gws2, side));
        if (gains_in_adam) return VKH_OK;
        // norm-gain gradients from the partial sums the main stream wrote
        const int rp = rmsnorm_partial_rows(T);
        VKH_HIP(column_sums(g.pn2, rp, D, D, Gd(s.t[5]), side));
        VKH_HIP(column_sums(g.pn1, rp, D, D, Gd(s.t[0]), side));
        if (cfg.qk_norm) {
            VKH_HIP(column_sums(g.pq, g.q_parts, g.qk_stride, hd, Gd(s.t[9]), side));
            VKH_HIP(column_sums(g.pk, g.k_parts, g.qk_stride, hd, Gd(s.t[10]), side));
        }
        return VKH_OK;
    }

    // operand views of the per-layer activations in the current precision
    Mat m_n1(const Acts &a) const { return b16() ? matb(a.n1b, D) : matf(a.n1, D); }
    Mat m_n2(const Acts &a) const { return b16() ? matb(a.n2b, D) : matf(a.n2, D); }
    Mat m_attn(const Acts &a) const { return b16() ? matb(a.attn_b, qd) : matf(a.attn_out, qd); }
    Mat m_gated(const Acts &a) const { return b16() ? matb(a.gatedb, F) : matf(a.gated, F); }
    static Mat shift(Mat m, long cols) {
        m.p = (const char *)m.p + cols * (m.dt == DType::BF16 ? 2 : 4);
        return m;
    }

    vkh_status sync_shadow() {
        if (b16() && shadow_dirty) {
            VKH_HIP(cast_f32_to_bf16(P, Pb + p_lo, total - p_lo, cur));
            shadow_dirty = false;
        }
        return VKH_OK;
    }

    // need_y = false (a recompute before the backward): stop before the down
    // projection, whose output y the layer keeps anyway.
    vkh_status layer_forward(int l, bool need_y = true) {
        Acts &a = acts[l];
        LayerSpans &s = ls[l];
        const float *x_in = l == 0 ? x_emb : acts[l - 1].y;
        const DType odt = b16() ? DType::BF16 : DType::F32;
        // transformer.zig:1794-1885
        VKH_HIP(rmsnorm_forward(x_in, W(s.t[0]), b16() ? (void *)a.n1b : (void *)a.n1, odt, T, D,
                                cfg.rms_eps, 0, cur));
        const Mat n1 = m_n1(a);
        const QkvLayout ql = qkv_layout();
        // the Q/K-norm + RoPE in the q|k|v GEMM's epilogue where the fused form applies
        hipError_t fq = hipErrorNotSupported;
        if (b16() && adt == DType::BF16 && !proj_lora(0) && !proj_lora(1) && !proj_lora(2))
            fq = g16_qkv_norm_rope((const bf16 *)n1.p, n1.ld, Wb(s.t[1]), D, a.qkv, qkvd, T, qkvd, D,
                                   ql, cfg.qk_norm ? W(s.t[9]) : nullptr,
                                   cfg.qk_norm ? W(s.t[10]) : nullptr, (bf16 *)a.qkv_attn, qkvd,
                                   rope_tab, cur, half_fwd);
        else if (!b16() && adt == DType::F32 && !lora)
            fq = g32_qkv_norm_rope((const float *)n1.p, n1.ld, W(s.t[1]), D, a.qkv, qkvd, T, qkvd, D,
                                   ql, cfg.qk_norm ? W(s.t[9]) : nullptr,
                                   cfg.qk_norm ? W(s.t[10]) : nullptr, (float *)a.qkv_attn, qkvd,
                                   rope_tab, cur);
        if (fq != hipErrorNotSupported) {
            VKH_HIP(fq);
        } else {
            VKH_TRY(linear_fwd_lora(l, {0, 1, 2}, n1, s.t[1], a.qkv, qkvd, qkvd, D, nullptr, 0));
            VKH_HIP(qkv_prepare_forward(ql, a.qkv, qkvd, cfg.qk_norm ? W(s.t[9]) : nullptr,
                                        cfg.qk_norm ? W(s.t[10]) : nullptr, a.qkv_attn, qkvd, adt,
                                        rope_tab, cur));
        }
        const AttnShape as = attn_shape();
        const size_t es = adt == DType::BF16 ? 2 : 4;
        const char *qa = (const char *)a.qkv_attn;
        const bool ob = b16() && adt == DType::BF16;
        // a recompute keeps the layer's O and LSE from the forward pass
        if (need_y) {
            VKH_HIP(fa_forward(as, qa, qkvd, qa + qd * es, qkvd, qa + (qd + kvd) * es, qkvd,
                               ob ? nullptr : a.attn_out, qd, a.lse, adt, ob ? a.attn_b : nullptr, qd,
                               cur));
            if (b16() && !ob) VKH_HIP(cast_f32_to_bf16(a.attn_out, a.attn_b, (size_t)T * qd, cur));
        }
        // mid = x_in + attn_out W_o^T (+ LoRA)
        const Mat att = m_attn(a);
        VKH_TRY(linear_fwd_lora(l, {3}, att, s.t[4], a.mid, D, D, qd, x_in, D));
        VKH_HIP(rmsnorm_forward(a.mid, W(s.t[5]), b16() ? (void *)a.n2b : (void *)a.n2, odt, T, D,
                                cfg.rms_eps, 0, cur));
        const Mat n2 = m_n2(a);
        // gate/up with the SwiGLU in its epilogue where the fused form applies
        hipError_t fused = hipErrorNotSupported;
        if (b16() && !proj_lora(4) && !proj_lora(5))
            fused = g16_gate_up_swiglu((const bf16 *)n2.p, n2.ld, Wb(s.t[6]), D, a.gu, 2 * F,
                                       a.gatedb, F, T, F, D, cur, half_fwd);
        else if (!b16() && !lora)
            fused = g32_gate_up_swiglu((const float *)n2.p, n2.ld, W(s.t[6]), D, a.gu, 2 * F, a.gated,
                                       F, T, F, D, cur);
        if (fused != hipErrorNotSupported) {
            VKH_HIP(fused);
        } else {
            VKH_TRY(linear_fwd_lora(l, {4, 5}, n2, s.t[6], a.gu, 2 * F, 2 * F, D, nullptr, 0));
            VKH_HIP(swiglu_forward(a.gu, 2 * F, a.gu + F, 2 * F,
                                   b16() ? (void *)a.gatedb : (void *)a.gated, F, odt, T, F, cur));
        }
        const Mat gt = m_gated(a);
        if (!need_y) return lora_fwd_group(l, {6}, gt, nullptr, 0, false);
        // y = mid + gated W_down^T (+ LoRA)
        VKH_TRY(linear_fwd_lora(l, {6}, gt, s.t[8], a.y, D, D, F, a.mid, D));
        return VKH_OK;
    }

    // The layers' forward as two half batches of whole sequences at once, the
    // first half on the main stream and the second on the side stream (idle
    // in the forward).  Every forward kernel works on rows, attention on whole
    // sequences, so the halves exchange nothing until the final norm, and one
    // stream's kernel tails and launch gaps overlap the other's work: the
    // config-3 step 18.85 -> 18.58-18.59 ms with the same losses (the fp32
    // step, whose forward GEMMs are compute-bound, measured slower: 76.55
    // against 75.9 ms).  Each half is layer_forward on the row range: T, B,
    // the stream, its split-K workspace, the input rows and the activation
    // pointers are switched for the call and restored after it.
    vkh_status forward_halves() {
        const int T0 = T, B0 = B;
        const long th = T0 / 2;
        const size_t es = adt == DType::BF16 ? 2 : 4;
        for (int h = 0; h < 2; ++h) {
            acts_h[h] = acts;
            const long r0 = h * th;
            auto off = [&](auto *&ptr, long ld) {
                if (ptr) ptr += r0 * ld;
            };
            for (Acts &a : acts_h[h]) {
                off(a.n1, D); off(a.qkv, qkvd); off(a.attn_out, qd); off(a.lse, H); off(a.mid, D);
                off(a.n2, D); off(a.gu, 2 * F); off(a.gated, F); off(a.y, D);
                off(a.n1b, D); off(a.attn_b, qd); off(a.n2b, D); off(a.gatedb, F);
                if (a.qkv_attn) a.qkv_attn = (char *)a.qkv_attn + r0 * qkvd * (long)es;
            }
        }
        hipStream_t c0 = cur;
        const GemmWs w0 = gws;
        float *x0 = x_emb;
        VKH_HIP(hipEventRecord(ev_hf, c0));
        VKH_HIP(hipStreamWaitEvent(side, ev_hf, 0));
        vkh_status st = VKH_OK;
        T = (int)th;
        B = B0 / 2;
        for (int l = 0; l < L && st == VKH_OK; ++l)
            for (int h = 0; h < 2 && st == VKH_OK; ++h) {
                cur = h ? side : c0;
                gws = h ? gws2 : w0;
                x_emb = x0 + h * th * D;
                std::swap(acts, acts_h[h]);
                st = layer_forward(l);
                std::swap(acts, acts_h[h]);
            }
        T = T0; B = B0; cur = c0; gws = w0; x_emb = x0;
        VKH_TRY(st);
        VKH_HIP(hipEventRecord(ev_hj, side));
        VKH_HIP(hipStreamWaitEvent(cur, ev_hj, 0));
        return VKH_OK;
    }

    vkh_status forward_all() {
        VKH_TRY(sync_shadow());
        if (bf16_only(embed)) VKH_HIP(embed_lookup_bf16(Wb(embed), tok_d, x_emb, T, D, 1.0f, cur));
        else VKH_HIP(embed_lookup(W(embed), tok_d, x_emb, T, D, 1.0f, cur));
        if (half_fwd) VKH_TRY(forward_halves());
        else
            for (int l = 0; l < L; ++l) VKH_TRY(layer_forward(l));
        VKH_HIP(rmsnorm_forward(acts[L - 1].y, W(final_norm), b16() ? (void *)fn_outb : (void *)fn_out,
                                b16() ? DType::BF16 : DType::F32, T, D, cfg.rms_eps, 0, cur));
        return VKH_OK;
    }

    // ── backward ────────────────────────────────────────────────────

    // LoRA backward of projection p after the base dx GEMM (train/lora.zig:137-251):
    // dx += aor (dy B) A;  dA = aor (dy B)^T x;  dB = aor dy^T inter.
    vkh_status lora_bwd(int l, int p, Mat dy, Mat x, float *dxo, long lddx) {
        int N, K;
        proj_shape(p, N, K);
        float *A = W(ls[l].la[p]), *Bm = W(ls[l].lb[p]);
        float *dA = G + (ls[l].la[p].off - tb), *dB = G + (ls[l].lb[p].off - tb);
        VKH_HIP(gemm_nn(pr, dy, matf(Bm, R), dyB, R, T, N, R, 1.f, 0.f, cur));
        if (dxo) VKH_HIP(gemm_nn(pr, matf(dyB, R), matf(A, K), dxo, lddx, T, R, K, aor, 1.f, cur));
        VKH_HIP(gemm_tn(pr, matf(dyB, R), x, dA, K, T, R, K, aor, 0.f, cur));
        VKH_HIP(gemm_tn(pr, dy, matf(acts[l].inter[p], R), dB, R, T, N, R, aor, 0.f, cur));
        return VKH_OK;
    }

    // LoRA backward of the targets among projections `ps`, which share the
    // input x; dy is their fused output gradient (projection p at column
    // proj_col(p)).  dy B for all of them, dx += aor (dy B) A, dA and dB:
    // one launch each on the rank-r kernels where the shapes allow.
    vkh_status lora_bwd_group(int l, std::initializer_list<int> ps, Mat dy, Mat x, float *dxo,
                              long lddx) {
        LoraAdapter ad[3];
        const int na = lora_adapters(l, ps, ad);
        if (!na) return VKH_OK;
        const LoraGroupSegs gs = lora_group_segs(ad, na, R);
        const LoraSegs &sb = gs.bwd_rows, &sa = gs.bwd_upd, &sda = gs.bwd_da, &sdb = gs.bwd_db;
        if (lora_fast_ok(dy.dt, dy.p, dy.ld, R, sb) && lora_fast_ok(x.dt, x.p, x.ld, R, sda) &&
            lora_fast_ok(dy.dt, dy.p, dy.ld, R, sdb) && (!dxo || lora_update_ok(dxo, lddx, R, sa))) {
            VKH_HIP(lora_rows(dy.dt, dy.p, dy.ld, T, R, sb, 1.f, cur));
            // dA, dB beside the rest of the backward (ordering: ev_laux)
            hipStream_t cs = cur;
            if (lora_aux) {
                VKH_HIP(hipEventRecord(ev_fork, cur));
                VKH_HIP(hipStreamWaitEvent(aux, ev_fork, 0));
                cs = aux;
            }
            VKH_HIP(lora_cols(x.dt, x.p, x.ld, T, R, sda, aor, cs));
            VKH_HIP(lora_cols(dy.dt, dy.p, dy.ld, T, R, sdb, aor, cs));
            if (dxo) VKH_HIP(lora_update(dxo, lddx, T, R, sa, aor, cur));
            return VKH_OK;
        }
        for (int p : ps)
            if (proj_lora(p)) VKH_TRY(lora_bwd(l, p, shift(dy, proj_col(p)), x, dxo, lddx));
        return VKH_OK;
    }

    // dy / dyb: the residual-stream gradient (fp32) and its bf16 copy; the
    // layer input gradient goes to dxo / dxob.
    vkh_status layer_backward(int l, const float *dy, const bf16 *dyb, float *dxo, bf16 *dxob) {
        if (lora_aux && l + 1 < L) VKH_HIP(hipStreamWaitEvent(cur, ev_laux[l + 1], 0));
        VKH_TRY(layer_backward_body(l, dy, dyb, dxo, dxob));
        if (lora_aux) VKH_HIP(hipEventRecord(ev_laux[l], aux));
        return VKH_OK;
    }
    vkh_status layer_backward_body(int l, const float *dy, const bf16 *dyb, float *dxo, bf16 *dxob) {
        Acts &a = acts[l];
        LayerSpans &s = ls[l];
        const float *x_in = l == 0 ? x_emb : acts[l - 1].y;
        // concurrent mode: this layer's own gradient operands (bf16 copies, or
        // in fp32 the tensors themselves); dW is deferred to the side stream
        const bool c32 = concurrent && !b16();
        bf16 *d_gub = concurrent ? lg[l].gub : this->d_gub;
        bf16 *d_midb = concurrent ? lg[l].midb : this->d_midb;
        bf16 *d_qkvb = concurrent ? lg[l].qkvb : this->d_qkvb;
        float *d_gu = c32 ? lg[l].guf : this->d_gu;
        float *d_mid = c32 ? lg[l].midf : this->d_mid;
        float *d_qkv = c32 ? lg[l].qkvf : this->d_qkv;
        auto linear_dw = [&](Mat dy_, Mat x_, const Span &w_, int N_, int K_) -> vkh_status {
            if (concurrent) return VKH_OK;
            return this->linear_dw(dy_, x_, w_, N_, K_);
        };
        const Mat mdy = b16() ? matb(dyb, D) : matf(dy, D);
        // transformer.zig:1967-2070 (order), train_decoder.zig:340-498 (math)
        // down: d_gated = dy W_down;  dW_down = dy^T gated
        VKH_TRY(dx_lora(l, {6}, mdy, m_gated(a), s.t[8], d_gated, nullptr, F, D, F));
        VKH_TRY(linear_dw(mdy, m_gated(a), s.t[8], D, F));
        // swiglu: d_gu = [d_gate | d_up] (bf16 copy only in the bf16 precision)
        if (b16())
            VKH_HIP(swiglu_backward(d_gated, F, a.gu, 2 * F, a.gu + F, 2 * F, d_gub, 2 * F, d_gub + F,
                                    2 * F, DType::BF16, T, F, cur));
        else
            VKH_HIP(swiglu_backward(d_gated, F, a.gu, 2 * F, a.gu + F, 2 * F, d_gu, 2 * F, d_gu + F,
                                    2 * F, DType::F32, T, F, cur));
        const Mat mdgu = b16() ? matb(d_gub, 2 * F) : matf(d_gu, 2 * F);
        // gate/up (one [2F, D] matrix): d_n2 = d_gu W_gu; dW_gu = d_gu^T n2
        VKH_TRY(dx_lora(l, {4, 5}, mdgu, m_n2(a), s.t[6], d_n, nullptr, D, 2 * F, D));
        VKH_TRY(linear_dw(mdgu, m_n2(a), s.t[6], 2 * F, D));
        // n2: d_mid = rmsnorm_bw(d_n2) + dy
        VKH_HIP(rmsnorm_backward(d_n, a.mid, W(s.t[5]), d_mid, d_midb, dy,
                                 concurrent ? nullptr : Gd(s.t[5]), concurrent ? lg[l].pn2 : partial,
                                 T, D, cfg.rms_eps, 0, cur));
        const Mat mdmid = b16() ? matb(d_midb, D) : matf(d_mid, D);
        // o: d_attn_out = d_mid W_o; dW_o = d_mid^T attn_out.  On the bf16
        // attention path without a LoRA term on o, dO goes straight to bf16 (the
        // attention kernels' operand) and D = rowsum(O dO) reads both in bf16.
        const AttnShape as = attn_shape();
        const bool o_lora = proj_lora(3);
        const bool do_bf16 = b16() && adt == DType::BF16 &&
                             (!o_lora || dx_lora_fused(l, {3}, mdmid, m_attn(a), s.t[4], D, qd));
        if (do_bf16 && !o_lora)
            VKH_HIP(g16_nn_bf16((const bf16 *)mdmid.p, mdmid.ld, Wb(s.t[4]), qd, dout16, qd, T, D,
                                qd, gws, cur));
        else
            VKH_TRY(dx_lora(l, {3}, mdmid, m_attn(a), s.t[4], d_attn_out, do_bf16 ? dout16 : nullptr,
                            qd, D, qd));
        VKH_TRY(linear_dw(mdmid, m_attn(a), s.t[4], D, qd));
        // attention: D, dK/dV, dQ into the fused d_qkv buffer
        if (b16() && adt == DType::BF16) {
            if (!do_bf16) VKH_HIP(cast_f32_to_bf16(d_attn_out, dout16, (size_t)T * qd, cur));
            // the recompute kernels form D themselves (from the bf16 O below),
            // unless dQ runs beside dK/dV
            if (!attn_v4 || attn_fork) VKH_HIP(fa_bw_d_bf16(as, a.attn_b, qd, dout16, qd, fa_d, cur));
        } else {
            VKH_HIP(fa_bw_d(as, a.attn_out, qd, d_attn_out, qd, fa_d, dout16, qd, cur));
        }
        const size_t es = adt == DType::BF16 ? 2 : 4;
        const char *qa = (const char *)a.qkv_attn;
        AttnPtrs ap;
        ap.q = qa; ap.ldq = qkvd;
        ap.k = qa + qd * es; ap.ldk = qkvd;
        ap.v = qa + (qd + kvd) * es; ap.ldv = qkvd;
        ap.o = a.attn_out; ap.ldo = qd;
        ap.dout = adt == DType::BF16 ? (const void *)dout16 : (const void *)d_attn_out; ap.lddo = qd;
        ap.lse = a.lse; ap.d = fa_d;
        ap.dq = d_qkv; ap.lddq = qkvd;
        ap.dk = d_qkv + qd; ap.lddk = qkvd;
        ap.dv = d_qkv + qd + kvd; ap.lddv = qkvd;
        ap.dt = adt;
        ap.split_ws = attn_split;
        if (attn_v4 && !attn_fork) {
            ap.o16 = a.attn_b;
            ap.ldo16 = qd;
        }
        // the recompute (or dS-GEMM) kernels; forked: dQ on the second stream
        auto attn_bw = [&]() -> vkh_status {
            if (attn_fork) {
                VKH_HIP(hipEventRecord(ev_fork, cur));
                VKH_HIP(hipStreamWaitEvent(aux, ev_fork, 0));
                VKH_HIP(fa_bw_v4_part(as, ap, 1, aux));
                VKH_HIP(fa_bw_v4_part(as, ap, 0, cur));
                VKH_HIP(hipEventRecord(ev_join, aux));
                VKH_HIP(hipStreamWaitEvent(cur, ev_join, 0));
                return VKH_OK;
            }
            VKH_HIP(fa_bw_fused(as, ap, attn_ds, attn_v4, cur));
            return VKH_OK;
        };
        const bool qk_side = concurrent && cfg.qk_norm;
        float *qkp = qk_side ? lg[l].pqk : partial;
        if (qk_fused) {
            // RoPE^T and the Q/K-norm backward in the attention kernels'
            // epilogues, straight into the bf16 gradient copy
            QkEpi &e = ap.qk;
            e.out = d_qkvb; e.ldout = qkvd;
            e.x = a.qkv; e.ldx = qkvd;
            e.gq = cfg.qk_norm ? W(s.t[9]) : nullptr;
            e.gk = cfg.qk_norm ? W(s.t[10]) : nullptr;
            e.eps = cfg.rms_eps;
            e.rope = rope_tab; e.rot = (int)cfg.rotary_dim;
            const int nq = fa_bw_v4_q_blocks(as);
            e.pq = qkp;
            e.pk = qkp + (size_t)nq * hd;
            VKH_TRY(attn_bw());
            if (qk_side) {
                lg[l].pq = e.pq; lg[l].pk = e.pk;
                lg[l].q_parts = nq; lg[l].k_parts = fa_bw_v4_k_gain_parts(as, attn_split);
                lg[l].qk_stride = hd;
            } else if (cfg.qk_norm && !lora) {
                VKH_HIP(column_sums(e.pq, nq, hd, hd, Gd(s.t[9]), cur));
                VKH_HIP(column_sums(e.pk, fa_bw_v4_k_gain_parts(as, attn_split), hd, hd, Gd(s.t[10]), cur));
            }
        } else {
            // fp32 with the gains on the side stream: RoPE^T and the Q/K-norm
            // backward in the fp32 dQ and dK/dV kernels' epilogues (gain partials
            // per block), where those kernels take the shape
            bool qk32 = false;
            if (adt == DType::F32 && !b16() && qk_side && !attn_fused &&
                (cfg.rotary_dim == 0 || (int)cfg.rotary_dim == hd)) {
                QkEpi &e = ap.qk;
                e.x = a.qkv; e.ldx = qkvd;
                e.gq = W(s.t[9]); e.gk = W(s.t[10]);
                e.eps = cfg.rms_eps;
                e.rope = rope_tab; e.rot = (int)cfg.rotary_dim;
                e.pq = qkp;
                e.pk = qkp + (size_t)fa_f32m_dq_blocks(as) * hd;
                qk32 = fa_f32m_qk_ok(as, ap);
                ap.qk_fp32 = qk32;
            }
            if (attn_fused) {
                VKH_TRY(attn_bw());
            } else {
                VKH_HIP(fa_bw_dkv(as, ap, cur));
                VKH_HIP(fa_bw_dq(as, ap, cur));
            }
            if (qk32) {
                lg[l].pq = ap.qk.pq; lg[l].pk = ap.qk.pk;
                lg[l].q_parts = fa_f32m_dq_blocks(as);
                lg[l].k_parts = fa_f32m_dkv_blocks(as);
                lg[l].qk_stride = hd;
            } else {
                // RoPE^T and Q/K-norm backward on the q/k columns (in place, or into the bf16 copy)
                const QkvLayout ql = qkv_layout();
                VKH_HIP(qkv_prepare_backward(ql, d_qkv, qkvd, a.qkv, qkvd, cfg.qk_norm ? W(s.t[9]) : nullptr,
                                             cfg.qk_norm ? W(s.t[10]) : nullptr,
                                             cfg.qk_norm && !qk_side ? Gd(s.t[9]) : nullptr,
                                             cfg.qk_norm && !qk_side ? Gd(s.t[10]) : nullptr, qkp,
                                             rope_tab, b16() ? d_qkvb : nullptr, qkvd, cur,
                                             qk_side ? &lg[l].qk_parts : nullptr));
                if (qk_side) {
                    lg[l].pq = qkp; lg[l].pk = qkp + hd;
                    lg[l].q_parts = lg[l].k_parts = lg[l].qk_parts;
                    lg[l].qk_stride = 2L * hd;
                }
            }
        }
        const Mat mdqkv = b16() ? matb(d_qkvb, qkvd) : matf(d_qkv, qkvd);
        // q/k/v (one [qkvd, D] matrix): d_n1 = d_qkv W_qkv; dW_qkv = d_qkv^T n1
        VKH_TRY(dx_lora(l, {0, 1, 2}, mdqkv, m_n1(a), s.t[1], d_n, nullptr, D, qkvd, D));
        VKH_TRY(linear_dw(mdqkv, m_n1(a), s.t[1], qkvd, D));
        // n1: d_x_in = rmsnorm_bw(d_n1) + d_mid
        VKH_HIP(rmsnorm_backward(d_n, x_in, W(s.t[0]), dxo, dxob, d_mid,
                                 concurrent ? nullptr : Gd(s.t[0]), concurrent ? lg[l].pn1 : partial,
                                 T, D, cfg.rms_eps, 0, cur));
        return VKH_OK;
    }

    vkh_status capture_boundary(int l, const float *g) {
        if (!bnd_capture) return VKH_OK;
        VKH_HIP(hipMemcpyAsync(bnd_grad + (size_t)l * T * D, g, (size_t)T * D * 4,
                               hipMemcpyDeviceToDevice, cur));
        return VKH_OK;
    }

    // with_adam: the concurrent mode applies Adam inside the backward (per layer
    // on the side stream); otherwise the caller enqueues adam_enqueue() after.
    vkh_status forward_backward_enqueue(bool with_adam) {
        VKH_TRY(forward_all());
        const CceShape cs{T, V, D, 0.f, 0.f};
        // head backward: dh and dW_lm (tied: the embed grad slot)
        float *dw_lm = lora ? nullptr : Gd(lm_head);
        const bool split = with_adam && embed_split_ok();
        if (b16()) {
            VKH_HIP(cce_forward16(cs, fn_outb, Wb(lm_head), tgt_d, ce_lse, loss_row, loss_mean,
                                  cce_work, cur, zf));
            VKH_HIP(cce_backward16(cs, fn_outb, Wb(lm_head), tgt_d, ce_lse, (bf16 *)dz, d_fn,
                                   concurrent ? nullptr : dw_lm, 0.f, gws, cur, zf));
            if (concurrent && dw_lm) {
                if (split) {  // this step's token rows, for the split embedding update
                    if (++mark_stamp == 0) {
                        VKH_HIP(fill_f32(reinterpret_cast<float *>(emb_mark), (size_t)V, 0.f, cur));
                        mark_stamp = 1;
                    }
                    VKH_HIP(mark_rows(tok_d, T, emb_mark, V, mark_stamp, cur));
                }
                // dW_lm = dz^T h on the side stream; the tied embedding scatter
                // below adds into the same gradient and waits for it
                VKH_HIP(hipEventRecord(ev_head, cur));
                VKH_HIP(hipStreamWaitEvent(side, ev_head, 0));
                VKH_HIP(g16_tn((const bf16 *)dz, V, fn_outb, D, dw_lm, D, T, V, D, 1.f, 0.f, gws2, side));
                if (split) VKH_TRY(embed_adam_early());
                VKH_HIP(hipEventRecord(ev_lm, side));
            }
        } else {
            // the fp32 logits kept in the dz buffer, which the backward turns
            // into dz in place (no second logits GEMM)
            VKH_HIP(cce_forward(pr, cs, fn_out, W(lm_head), tgt_d, ce_lse, loss_row, loss_mean,
                                cce_work, cur, (float *)dz));
            // two streams: dW_lm on the side stream starts as soon as dz is
            // written, beside dh on the main stream (fp32: 75.97-75.99 -> 75.30 ms,
            // same losses; the bf16 step, whose dh is the short split-K form,
            // measured 0.05-0.09 ms slower this way and keeps dh first)
            const bool dw_early = concurrent && dw_lm;
            VKH_HIP(cce_backward(pr, cs, fn_out, W(lm_head), tgt_d, ce_lse, dz, dw_early ? nullptr : d_fn,
                                 concurrent ? nullptr : dw_lm, 0.f, cur, (const float *)dz));
            if (concurrent && dw_lm) {  // as above, on the fp32 logits gradient
                if (split) {
                    if (++mark_stamp == 0) {
                        VKH_HIP(fill_f32(reinterpret_cast<float *>(emb_mark), (size_t)V, 0.f, cur));
                        mark_stamp = 1;
                    }
                    VKH_HIP(mark_rows(tok_d, T, emb_mark, V, mark_stamp, cur));
                }
                VKH_HIP(hipEventRecord(ev_head, cur));
                VKH_HIP(hipStreamWaitEvent(side, ev_head, 0));
                VKH_HIP(g32_tn((const float *)dz, V, fn_out, D, dw_lm, D, T, V, D, 1.f, 0.f, gws2, side));
                // dh = dz W_lm (cce_backward's own call); the table's Adam on the
                // side stream rewrites W_lm, so it waits for dh
                VKH_HIP(g32_nn((const float *)dz, V, W(lm_head), D, d_fn, D, T, V, D, 1.f, 0.f,
                               GemmWs{nullptr, 0}, cur));
                VKH_HIP(hipEventRecord(ev_dh, cur));
                VKH_HIP(hipStreamWaitEvent(side, ev_dh, 0));
                if (split) VKH_TRY(embed_adam_early());
                VKH_HIP(hipEventRecord(ev_lm, side));
            }
        }
        // fp32 concurrent: each layer's dy is its own buffer (the side stream's
        // dW_down reads it after the main stream has moved on)
        const bool c32 = concurrent && !b16();
        float *top = c32 ? lg[L - 1].dyf : dx[0];
        VKH_HIP(rmsnorm_backward(d_fn, acts[L - 1].y, W(final_norm), top,
                                 b16() ? (concurrent ? lg[L - 1].dyb : dxb[0]) : nullptr, nullptr,
                                 Gd(final_norm), partial, T, D, cfg.rms_eps, 0, cur));
        VKH_TRY(capture_boundary(L, top));
        int c = 0;
        for (int l = L - 1; l >= 0; --l) {
            if (recompute) {
                // shared sets: the side stream is done with layer l + 2's
                if (concurrent && l + 2 < L) VKH_HIP(hipStreamWaitEvent(cur, ev_sdone[l + 2], 0));
                // the set holds layer l + kActSets's activations: run l's forward again
                if (l + kActSets < L) VKH_TRY(layer_forward(l, false));
            }
            float *out = c32 && l > 0 ? lg[l - 1].dyf : dx[c ^ 1];
            if (concurrent) {
                VKH_TRY(layer_backward(l, c32 ? lg[l].dyf : dx[c], c32 ? nullptr : lg[l].dyb, out,
                                       !c32 && l > 0 ? lg[l - 1].dyb : nullptr));
                // layer l's gradient inputs are final: its dW GEMMs (and, with Adam,
                // its update) run on the side stream while the main stream goes on
                VKH_HIP(hipEventRecord(ev_layer[l], cur));
                VKH_HIP(hipStreamWaitEvent(side, ev_layer[l], 0));
                VKH_TRY(layer_dw_side(l, with_adam));
                if (with_adam) VKH_TRY(adam_layer_side(l));
                if (recompute) VKH_HIP(hipEventRecord(ev_sdone[l], side));
            } else {
                VKH_TRY(layer_backward(l, dx[c], dxb[c], dx[c ^ 1], dxb[c ^ 1]));
            }
            VKH_TRY(capture_boundary(l, out));
            c ^= 1;
        }
        // the adapters' last gradients before Adam and the next forward
        if (lora_aux) VKH_HIP(hipStreamWaitEvent(cur, ev_laux[0], 0));
        if (!lora) {
            float *dE = Gd(embed);
            if (concurrent) VKH_HIP(hipStreamWaitEvent(cur, ev_lm, 0));
            if (split) {
                // the scatter completes the token rows' gradient: their update in the same launch
                const EmbedAdam ea{W(embed), M + embed.off, Vm + embed.off,
                                   b16() ? Pb + embed.off : nullptr, adam_hyper(cfg.lr)};
                VKH_HIP(embedding_backward_adam(dx[c], tok_d, dE, T, D, V, tied, ea, cur));
            } else {
                if (!tied) VKH_HIP(fill_f32(dE, embed.numel, 0.f, cur));
                VKH_HIP(embedding_backward(dx[c], tok_d, dE, T, D, V, tied, embed_work, cur));
            }
        }
        if (concurrent) {
            // embed, final norm, lm_head: the span before layer 0 (split: the
            // embedding and lm_head are done, the final norm remains)
            if (split) VKH_TRY(adam_span(final_norm.off, final_norm.off + final_norm.numel, cur));
            else if (with_adam) VKH_TRY(adam_span(0, ls[0].t[0].off, cur));
            VKH_HIP(hipEventRecord(ev_side, side));
            VKH_HIP(hipStreamWaitEvent(cur, ev_side, 0));
        }
        return VKH_OK;
    }

    // Adam over layer l's span on the side stream, reducing its norm-gain
    // partials (n1, n2, q/k norm) inside the same launch.
    vkh_status adam_layer_side(int l) {
        const LayerSpans &ss = ls[l];
        const LayerGrads &g = lg[l];
        const size_t b = ss.t[0].off, e = layer_end(l);
        const int rp = rmsnorm_partial_rows(T);
        AdamGains gs{};
        auto add = [&](const Span &sp, const float *part, int nparts, long stride) {
            gs.g[gs.n++] = AdamGain{sp.off - b, (unsigned)sp.numel, part, nparts, stride};
        };
        add(ss.t[0], g.pn1, rp, D);
        add(ss.t[5], g.pn2, rp, D);
        if (cfg.qk_norm) {
            add(ss.t[9], g.pq, g.q_parts, g.qk_stride);
            add(ss.t[10], g.pk, g.k_parts, g.qk_stride);
        }
        const float t = (float)step_t;
        const float bc1 = 1.0f - powf(cfg.beta1, t);
        const float bc2 = 1.0f - powf(cfg.beta2, t);
        // bf16 without recompute: three blocks per CU walk the layer's chunks, so the
        // update streams beside the main stream's latency-bound backward kernels
        // at a lower share of HBM (config 3: 18.07-18.33 -> 17.74-18.01 ms in three
        // alternating pairs, same losses; on one box 3 / 2 / 4 / 5 per CU measured
        // 18.02-18.04 / 18.23-18.26 / 18.09-18.12 / 18.36-18.37).  The
        // fp32 step (71.30-71.35 against 70.90-70.94) and config 5 (582.3 against
        // 578.7), whose side streams have no slack to spare, keep the full grid.
        const unsigned cap = b16() && !recompute ? 3u * (unsigned)cu_count() : 0u;
        VKH_HIP(adam_step_gains(Pat(b), G + b, M + b, Vm + b, e - b, cfg.lr, cfg.beta1, cfg.beta2,
                                cfg.eps_adam, bc1, bc2, 0.f, b16() ? Pb + b : nullptr, gs, side, cap));
        return VKH_OK;
    }

    // end (arena offset) of layer l's tensors
    size_t layer_end(int l) const {
        const LayerSpans &s = ls[l];
        const Span &last = s.t[10].numel ? s.t[10] : s.t[8];
        return last.off + last.numel;
    }

    AdamHyper adam_hyper(float lr) const {
        const float t = (float)step_t;
        return AdamHyper{lr, cfg.beta1, cfg.beta2, cfg.eps_adam, 1.0f - powf(cfg.beta1, t),
                         1.0f - powf(cfg.beta2, t), 0.f};
    }
    // the split embedding update needs whole float4 rows
    bool embed_split_ok() const { return concurrent && !lora && D % 4 == 0; }

    // Side stream, after the head's weight-gradient GEMM: Adam over the table
    // rows no token of this step names (and, untied, over lm_head, whose
    // gradient is complete, after zeroing the embedding gradient the scatter
    // writes into).
    vkh_status embed_adam_early() {
        const AdamHyper h = adam_hyper(cfg.lr);
        if (!tied) {
            VKH_TRY(adam_span(lm_head.off, lm_head.off + lm_head.numel, side));
            VKH_HIP(fill_f32(Gd(embed), embed.numel, 0.f, side));
        }
        VKH_HIP(adam_rows_unmarked(W(embed), Gd(embed), M + embed.off, Vm + embed.off,
                                   b16() ? Pb + embed.off : nullptr, V, D, emb_mark, mark_stamp, h,
                                   side));
        return VKH_OK;
    }

    // Adam over the arena range [b, e) of a full fine-tune (adam_step.comp:45-61)
    vkh_status adam_span(size_t b, size_t e, hipStream_t st) {
        const float t = (float)step_t;
        const float bc1 = 1.0f - powf(cfg.beta1, t);
        const float bc2 = 1.0f - powf(cfg.beta2, t);
        VKH_HIP(adam_step(Pat(b), G + b, M + b, Vm + b, e - b, cfg.lr, cfg.beta1, cfg.beta2,
                          cfg.eps_adam, bc1, bc2, 0.f, b16() ? Pb + b : nullptr, st));
        return VKH_OK;
    }

    vkh_status adam_enqueue() {
        const float t = (float)step_t;
        const float bc1 = 1.0f - powf(cfg.beta1, t);
        const float bc2 = 1.0f - powf(cfg.beta2, t);
        bf16 *pb = b16() ? Pb : nullptr;
        if (!lora) {
            VKH_HIP(adam_step(Pat(0), G, M, Vm, total, cfg.lr, cfg.beta1, cfg.beta2, cfg.eps_adam, bc1, bc2,
                              0.f, pb, cur));
        } else {
            const size_t na = lora_b_begin - lora_a_begin, nb = total - lora_b_begin;
            VKH_HIP(adam_step(Pat(lora_a_begin), G, M, Vm, na, cfg.lr, cfg.beta1, cfg.beta2, cfg.eps_adam,
                              bc1, bc2, 0.f, pb ? pb + lora_a_begin : nullptr, cur));
            VKH_HIP(adam_step(Pat(lora_b_begin), G + na, M + na, Vm + na, nb, cfg.lr * cfg.lora_lr_b_scale,
                              cfg.beta1, cfg.beta2, cfg.eps_adam, bc1, bc2, 0.f,
                              pb ? pb + lora_b_begin : nullptr, cur));
        }
        return VKH_OK;
    }

    vkh_status check_ids(const uint32_t *tok, size_t nt, const uint32_t *tgt, size_t ng) {
        if (nt != (size_t)T) return fail(VKH_ERR_TOKEN_IDS_LEN, "token_ids len %zu != %d", nt, T);
        if (tgt && ng != (size_t)T) return fail(VKH_ERR_TARGET_LEN, "target_ids len %zu != %d", ng, T);
        if (!tok || (ng && !tgt)) return fail(VKH_ERR_INVALID_ARGUMENT, "null ids");
        for (int i = 0; i < T; ++i)
            if (tok[i] >= (uint32_t)V || (tgt && tgt[i] >= (uint32_t)V))
                return fail(VKH_ERR_TOKEN_OUT_OF_RANGE, "id at %d out of range [0, %d)", i, V);
        return VKH_OK;
    }

    vkh_status upload_ids(const uint32_t *tok, const uint32_t *tgt) {
        VKH_HIP(hipEventSynchronize(upload_done));  // staging reuse
        memcpy(tok_h, tok, (size_t)T * 4);
        VKH_HIP(hipMemcpyAsync(tok_d, tok_h, (size_t)T * 4, hipMemcpyHostToDevice, cur));
        if (tgt) {
            memcpy(tgt_h, tgt, (size_t)T * 4);
            VKH_HIP(hipMemcpyAsync(tgt_d, tgt_h, (size_t)T * 4, hipMemcpyHostToDevice, cur));
        }
        VKH_HIP(hipEventRecord(upload_done, cur));
        return VKH_OK;
    }

    vkh_status record_loss() {
        VKH_HIP(hipMemcpyAsync(loss_h, loss_mean, 4, hipMemcpyDeviceToHost, cur));
        VKH_HIP(hipEventRecord(loss_ready, cur));
        loss_pending = true;
        return VKH_OK;
    }
    // the tick API's staging: only ticks write it, so the gate sees what
    // earlier ticks measured whatever other calls ran in between
    vkh_status record_tick_loss() {
        VKH_HIP(hipMemcpyAsync(loss_h + 1, loss_mean, 4, hipMemcpyDeviceToHost, cur));
        VKH_HIP(hipEventRecord(tick_loss_ready, cur));
        tick_loss_pending = true;
        return VKH_OK;
    }

    // Start enqueueing on stream s after the runner's last work, whichever
    // stream that went to (on the same stream the wait is already implied;
    // it is issued anyway, so a caller stream destroyed and re-created at the
    // same address cannot skip it).
    vkh_status begin_on(hipStream_t s) {
        cur = s;
        if (last_st) VKH_HIP(hipStreamWaitEvent(s, ev_done, 0));
        return VKH_OK;
    }
    // Close an enqueue: later work on any stream (or the host) orders after it.
    vkh_status end_on() {
        hipStream_t s = cur;
        cur = own;
        VKH_HIP(hipEventRecord(ev_done, s));
        last_st = s;
        return VKH_OK;
    }
    // Before the host reads or writes runner memory.
    vkh_status host_wait() {
        if (last_st) VKH_HIP(hipEventSynchronize(ev_done));
        VKH_HIP(hipStreamSynchronize(own));
        return VKH_OK;
    }

    // Forward + CE loss of the staged batch into the loss staging (the
    // loss evaluation runner.zig:967-973 records every tick under a loss
    // target, so a new batch whose loss is above the target resumes training).
    vkh_status loss_eval_enqueue() {
        VKH_TRY(forward_all());
        const CceShape cs{T, V, D, 0.f, 0.f};
        if (b16())
            VKH_HIP(cce_forward16(cs, fn_outb, Wb(lm_head), tgt_d, ce_lse, loss_row, loss_mean,
                                  cce_work, cur));
        else
            VKH_HIP(cce_forward(pr, cs, fn_out, W(lm_head), tgt_d, ce_lse, loss_row, loss_mean,
                                cce_work, cur));
        return record_tick_loss();
    }

    vkh_status step_enqueue(bool with_adam) {
        VKH_TRY(forward_backward_enqueue(with_adam));
        VKH_TRY(record_loss());
        if (with_adam) {
            if (!concurrent) VKH_TRY(adam_enqueue());
            step_t += 1;  // transformer.zig:1318
        }
        return VKH_OK;
    }
};

// ── checkpoint I/O ─────────────────────────────────────────────────────

namespace {

struct CkptHeader {
    char magic[4];
    uint32_t version, step_t, cfg_size;
};
static_assert(sizeof(CkptHeader) == 16, "checkpoint header is 16 bytes");

// The config block is std.mem.asBytes(&cfg) of the reference's `Config`
// (transformer.zig:31-77, written at :1405-1406).  `Config` is an auto-layout
// Zig struct: the compiler orders its fields by descending alignment, keeping
// declaration order among equals, so the nineteen 4-byte fields come first in
// declaration order, then the two bools (causal, qk_norm), then two bytes of
// padding: @sizeOf(Config) = 80.  Padding is written as zero.  The order is
// inferred from those rules, not checked against a reference-written file
// (none exists); this encoder and zig_cfg_decode are the only places it lives.
constexpr uint32_t kZigCfgSize = 80;

void put32(uint8_t *p, uint32_t v) { memcpy(p, &v, 4); }
void putf(uint8_t *p, float v) { memcpy(p, &v, 4); }
uint32_t get32(const uint8_t *p) { uint32_t v; memcpy(&v, p, 4); return v; }
float getf(const uint8_t *p) { float v; memcpy(&v, p, 4); return v; }

void zig_cfg_encode(const vkh_config &c, uint8_t *o) {
    memset(o, 0, kZigCfgSize);
    put32(o + 0, c.dim); put32(o + 4, c.n_heads); put32(o + 8, c.n_kv_heads);
    put32(o + 12, c.head_dim); put32(o + 16, c.ff_dim); put32(o + 20, c.n_pos);
    put32(o + 24, c.n_layers); put32(o + 28, c.vocab_size); putf(o + 32, c.rms_eps);
    put32(o + 36, c.rotary_dim); putf(o + 40, c.rope_theta); putf(o + 44, c.lr);
    putf(o + 48, c.beta1); putf(o + 52, c.beta2); putf(o + 56, c.eps_adam);
    put32(o + 60, c.lora_targets); put32(o + 64, c.lora_rank); putf(o + 68, c.lora_alpha);
    putf(o + 72, c.lora_lr_b_scale);
    o[76] = c.causal ? 1 : 0;
    o[77] = c.qk_norm ? 1 : 0;
}

// Fills the reference's fields; the extensions (n_seqs, tied_embeddings,
// precision) are left as they are in `c`.
void zig_cfg_decode(const uint8_t *o, vkh_config &c) {
    c.dim = get32(o + 0); c.n_heads = get32(o + 4); c.n_kv_heads = get32(o + 8);
    c.head_dim = get32(o + 12); c.ff_dim = get32(o + 16); c.n_pos = get32(o + 20);
    c.n_layers = get32(o + 24); c.vocab_size = get32(o + 28); c.rms_eps = getf(o + 32);
    c.rotary_dim = get32(o + 36); c.rope_theta = getf(o + 40); c.lr = getf(o + 44);
    c.beta1 = getf(o + 48); c.beta2 = getf(o + 52); c.eps_adam = getf(o + 56);
    c.lora_targets = get32(o + 60); c.lora_rank = get32(o + 64); c.lora_alpha = getf(o + 68);
    c.lora_lr_b_scale = getf(o + 72);
    c.causal = o[76] != 0;
    c.qk_norm = o[77] != 0;
}

// transformer.zig:197-205 cfgShapeMatches
bool shape_matches(const vkh_config &a, const vkh_config &b) {
    return a.dim == b.dim && a.n_heads == b.n_heads && a.n_kv_heads == b.n_kv_heads &&
           a.head_dim == b.head_dim && a.ff_dim == b.ff_dim && a.n_pos == b.n_pos &&
           a.n_layers == b.n_layers && a.vocab_size == b.vocab_size && a.rms_eps == b.rms_eps &&
           (a.causal != 0) == (b.causal != 0) && a.rotary_dim == b.rotary_dim &&
           a.rope_theta == b.rope_theta && (a.qk_norm != 0) == (b.qk_norm != 0) &&
           a.lora_targets == b.lora_targets && a.lora_rank == b.lora_rank;
}

struct Blob {
    float *dev;   // nullptr => zeros (m/v of frozen tensors), unless dev16
    size_t numel;
    int alias;    // >= 0: the tied lm_head, the same memory as blob `alias`
    bf16 *dev16 = nullptr;  // a base matrix stored in bf16 only: widened / rounded
};

}  // namespace

namespace vkh {


// transformer.zig:1586-1655 collectBlobs.  A tied runner has one embedding
// matrix; its lm_head blobs are the embedding's (param, m, v) again, which is
// how the reference itself represents a tied head (load_real.zig:14-19 copies
// embed_tokens into a separate lm_head), so the file loads in the reference.
static void collect_blobs(vkh_runner *r, std::vector<Blob> &out) {
    auto add3 = [&](const Span &s, int alias) {
        if (r->bf16_only(s)) out.push_back({nullptr, s.numel, alias, r->Pb + s.off});
        else out.push_back({r->W(s), s.numel, alias});
        out.push_back({r->ptr(VKH_ADAM_M, s), s.numel, alias < 0 ? -1 : alias + 1});
        out.push_back({r->ptr(VKH_ADAM_V, s), s.numel, alias < 0 ? -1 : alias + 2});
    };
    add3(r->embed, -1);
    add3(r->final_norm, -1);
    add3(r->lm_head, r->tied ? 0 : -1);
    for (int l = 0; l < r->L; ++l) {
        for (int t = 0; t < 9; ++t) add3(r->ls[l].t[t], -1);
        if (r->cfg.qk_norm) { add3(r->ls[l].t[9], -1); add3(r->ls[l].t[10], -1); }
    }
}

static void collect_lora_blobs(vkh_runner *r, std::vector<Blob> &out) {
    for (int p = 0; p < 7; ++p) {
        if (!r->proj_lora(p)) continue;
        for (int l = 0; l < r->L; ++l) {
            const Span &a = r->ls[l].la[p], &b = r->ls[l].lb[p];
            out.push_back({r->W(a), a.numel, -1});
            out.push_back({r->ptr(VKH_ADAM_M, a), a.numel, -1});
            out.push_back({r->ptr(VKH_ADAM_V, a), a.numel, -1});
            out.push_back({r->W(b), b.numel, -1});
            out.push_back({r->ptr(VKH_ADAM_M, b), b.numel, -1});
            out.push_back({r->ptr(VKH_ADAM_V, b), b.numel, -1});
        }
    }
}

static vkh_status save_blobs(vkh_runner *r, const char *path, const char magic[4],
                             const std::vector<Blob> &blobs) {
    VKH_TRY(r->host_wait());
    FILE *f = fopen(path, "wb");
    if (!f) return fail(VKH_ERR_IO, "cannot open %s for writing", path);
    CkptHeader h;
    memcpy(h.magic, magic, 4);
    h.version = 1;
    h.step_t = r->step_t;
    h.cfg_size = kZigCfgSize;
    uint8_t cb[kZigCfgSize];
    zig_cfg_encode(r->cfg, cb);
    bool ok = fwrite(&h, sizeof(h), 1, f) == 1 && fwrite(cb, kZigCfgSize, 1, f) == 1;
    std::vector<float> buf;
    for (const Blob &b : blobs) {
        if (!ok) break;
        buf.assign(b.numel, 0.f);
        if (b.dev) {
            hipError_t e = hipMemcpy(buf.data(), b.dev, b.numel * 4, hipMemcpyDeviceToHost);
            if (e != hipSuccess) { fclose(f); return hip_fail(e, "checkpoint readback"); }
        } else if (b.dev16) {
            const vkh_status e = read_bf16_widened(b.dev16, b.numel, buf.data());
            if (e != VKH_OK) { fclose(f); return e; }
        }
        ok = fwrite(buf.data(), 4, b.numel, f) == b.numel;
    }
    if (fclose(f) != 0) ok = false;
    return ok ? VKH_OK : fail(VKH_ERR_IO, "write to %s failed", path);
}

static vkh_status load_blobs(vkh_runner *r, const char *path, const char magic[4], bool lora_file,
                             const std::vector<Blob> &blobs) {
    FILE *f = fopen(path, "rb");
    if (!f) return fail(VKH_ERR_IO, "cannot open %s", path);
    CkptHeader h;
    uint8_t cb[kZigCfgSize];
    vkh_config saved = r->cfg;
    vkh_status st = VKH_OK;
    const vkh_status mismatch =
        lora_file ? VKH_ERR_LORA_CHECKPOINT_CONFIG_MISMATCH : VKH_ERR_CHECKPOINT_CONFIG_MISMATCH;
    if (fread(&h, sizeof(h), 1, f) != 1) st = fail(VKH_ERR_END_OF_STREAM, "truncated header");
    else if (memcmp(h.magic, magic, 4) != 0)
        st = fail(lora_file ? VKH_ERR_INVALID_LORA_CHECKPOINT_MAGIC : VKH_ERR_INVALID_CHECKPOINT_MAGIC, "bad magic");
    else if (h.version != 1)
        st = fail(lora_file ? VKH_ERR_UNSUPPORTED_LORA_CHECKPOINT_VERSION : VKH_ERR_UNSUPPORTED_CHECKPOINT_VERSION,
                  "version %u", h.version);
    else if (h.cfg_size != kZigCfgSize)
        st = fail(lora_file ? VKH_ERR_LORA_CHECKPOINT_CONFIG_SIZE_MISMATCH : VKH_ERR_CHECKPOINT_CONFIG_SIZE_MISMATCH,
                  "cfg_size %u != %u", h.cfg_size, kZigCfgSize);
    else if (fread(cb, kZigCfgSize, 1, f) != 1) st = fail(VKH_ERR_END_OF_STREAM, "truncated config");
    else {
        zig_cfg_decode(cb, saved);
        if (!shape_matches(saved, r->cfg)) st = fail(mismatch, "config shape mismatch");
    }
    std::vector<std::vector<float>> data;
    if (st == VKH_OK) {
        data.resize(blobs.size());
        for (size_t i = 0; i < blobs.size(); ++i) {
            data[i].resize(blobs[i].numel);
            if (fread(data[i].data(), 4, blobs[i].numel, f) != blobs[i].numel) {
                st = fail(VKH_ERR_END_OF_STREAM, "truncated body");
                break;
            }
        }
    }
    fclose(f);
    // a tied runner holds one matrix: the file's lm_head must be its embedding
    for (size_t i = 0; st == VKH_OK && i < blobs.size(); ++i)
        if (blobs[i].alias >= 0 && data[i] != data[(size_t)blobs[i].alias])
            st = fail(mismatch, "the file's lm_head differs from its embedding (untied) but the "
                                "runner ties them");
    if (st != VKH_OK) return st;
    VKH_TRY(r->host_wait());
    for (size_t i = 0; i < blobs.size(); ++i) {
        if (blobs[i].alias >= 0) continue;
        if (blobs[i].dev)
            VKH_HIP(hipMemcpy(blobs[i].dev, data[i].data(), blobs[i].numel * 4, hipMemcpyHostToDevice));
        else if (blobs[i].dev16)
            VKH_TRY(write_bf16_rounded(blobs[i].dev16, blobs[i].numel, data[i].data()));
    }
    // transformer.zig:1444-1448, :1538-1544
    r->step_t = h.step_t;
    r->cfg.lr = saved.lr;
    r->cfg.beta1 = saved.beta1;
    r->cfg.beta2 = saved.beta2;
    r->cfg.eps_adam = saved.eps_adam;
    if (lora_file) {
        r->cfg.lora_alpha = saved.lora_alpha;
        r->cfg.lora_lr_b_scale = saved.lora_lr_b_scale;
        r->aor = r->R ? saved.lora_alpha / (float)r->R : 0.f;
    }
    return VKH_OK;
}

}  // namespace vkh

// ── C ABI: runner ─────────────────────────────────────────────────────

extern "C" {

vkh_status vkh_runner_create(const vkh_config *cfg, const vkh_init_weights *weights,
                             vkh_runner **out) {
    if (!cfg || !out) return fail(VKH_ERR_INVALID_ARGUMENT, "null argument");
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) return fail(VKH_ERR_NO_DEVICE, "no HIP device");
    vkh_runner *r = new vkh_runner();
    vkh_status st = r->init(*cfg);
    if (st == VKH_OK && weights) st = r->upload_weights(*weights);
    if (st == VKH_OK && !weights && r->lora)
        for (int p = 0; p < 7 && st == VKH_OK; ++p)
            if (r->proj_lora(p)) st = r->lora_default_init(p);
    if (st == VKH_OK) {
        hipError_t e = hipStreamSynchronize(r->own);
        if (e != hipSuccess) st = hip_fail(e, "init");
    }
    if (st != VKH_OK) {
        delete r;
        return st;
    }
    *out = r;
    return VKH_OK;
}

void vkh_runner_destroy(vkh_runner *r) { delete r; }

vkh_status vkh_runner_init_random(vkh_runner *r, uint64_t seed, float std_, float lora_std) {
    if (!r) return fail(VKH_ERR_INVALID_ARGUMENT, "null runner");
    return r->init_random(seed, std_, lora_std);
}

static vkh_status run_step(vkh_runner *r, const uint32_t *tok, size_t nt, const uint32_t *tgt,
                           size_t ng, hipStream_t st, bool adam, bool wait) {
    if (!r) return fail(VKH_ERR_INVALID_ARGUMENT, "null runner");
    VKH_TRY(r->check_ids(tok, nt, tgt, ng));
    VKH_TRY(r->begin_on(st ? st : r->own));
    vkh_status s = r->upload_ids(tok, tgt);
    if (s == VKH_OK) s = r->step_enqueue(adam);
    const vkh_status se = r->end_on();
    if (s == VKH_OK) s = se;
    if (s == VKH_OK && wait) {
        hipError_t e = hipEventSynchronize(r->ev_done);
        if (e != hipSuccess) s = hip_fail(e, "step");
    }
    return s;
}

vkh_status vkh_runner_step(vkh_runner *r, const uint32_t *token_ids, size_t n_tokens,
                           const uint32_t *target_ids, size_t n_targets) {
    return run_step(r, token_ids, n_tokens, target_ids, n_targets, nullptr, true, true);
}

vkh_status vkh_runner_step_async(vkh_runner *r, const uint32_t *token_ids, size_t n_tokens,
                                 const uint32_t *target_ids, size_t n_targets,
                                 vkh_stream stream) {
    return run_step(r, token_ids, n_tokens, target_ids, n_targets, (hipStream_t)stream, true, false);
}

vkh_status vkh_runner_forward_backward(vkh_runner *r, const uint32_t *token_ids,
                                       size_t n_tokens, const uint32_t *target_ids,
                                       size_t n_targets) {
    return run_step(r, token_ids, n_tokens, target_ids, n_targets, nullptr, false, true);
}

vkh_status vkh_runner_last_loss(vkh_runner *r, float *loss) {
    if (!r || !loss) return fail(VKH_ERR_INVALID_ARGUMENT, "null argument");
    if (!r->loss_pending) return fail(VKH_ERR_INVALID_ARGUMENT, "no step has run");
    VKH_HIP(hipEventSynchronize(r->loss_ready));
    *loss = r->loss_h[0];
    return VKH_OK;
}

vkh_status vkh_runner_synchronize(vkh_runner *r) {
    if (!r) return fail(VKH_ERR_INVALID_ARGUMENT, "null runner");
    return r->host_wait();
}

vkh_status vkh_runner_forward_logits(vkh_runner *r, const uint32_t *token_ids, size_t n_tokens,
                                     float *out_logits, size_t out_len) {
    if (!r || !out_logits) return fail(VKH_ERR_INVALID_ARGUMENT, "null argument");
    VKH_TRY(r->check_ids(token_ids, n_tokens, nullptr, 0));
    if (out_len != (size_t)r->T * r->V) return fail(VKH_ERR_OUT_LOGITS_LEN, "out_logits len %zu", out_len);
    VKH_TRY(r->begin_on(r->own));
    vkh_status s = r->upload_ids(token_ids, nullptr);
    if (s == VKH_OK) s = r->forward_all();
    const vkh_status se = r->end_on();
    if (s == VKH_OK) s = se;
    if (s != VKH_OK) return s;
    float *logits = nullptr;
    note_allocation();
    VKH_HIP(hipMallocAsync((void **)&logits, (size_t)r->T * r->V * 4, r->own));
    hipError_t e =
        r->b16() ? g16_nt(r->fn_outb, r->D, r->Wb(r->lm_head), r->D, logits, r->V, r->T, r->V, r->D,
                          nullptr, 0, 1.f, 0.f, r->gws, r->own)
                 : gemm_nt(r->pr, matf(r->fn_out, r->D), matf(r->W(r->lm_head), r->D), logits, r->V,
                           r->T, r->V, r->D, nullptr, 0, 1.f, 0.f, r->own);
    if (e == hipSuccess)
        e = hipMemcpyAsync(out_logits, logits, (size_t)r->T * r->V * 4, hipMemcpyDeviceToHost, r->own);
    (void)hipFreeAsync(logits, r->own);
    if (e == hipSuccess) e = hipEventRecord(r->ev_done, r->own);
    if (e == hipSuccess) e = hipStreamSynchronize(r->own);
    if (e != hipSuccess) return hip_fail(e, "forward_logits");
    return VKH_OK;
}

uint32_t vkh_runner_step_t(const vkh_runner *r) { return r ? r->step_t : 0; }

vkh_status vkh_runner_set_step_t(vkh_runner *r, uint32_t t) {
    if (!r || t == 0) return fail(VKH_ERR_INVALID_ARGUMENT, "step_t must be >= 1");
    r->step_t = t;
    return VKH_OK;
}

float vkh_runner_get_lr(const vkh_runner *r) { return r ? r->cfg.lr : 0.f; }

vkh_status vkh_runner_set_lr(vkh_runner *r, float lr) {
    if (!r) return fail(VKH_ERR_INVALID_ARGUMENT, "null runner");
    r->cfg.lr = lr;
    return VKH_OK;
}

vkh_status vkh_runner_get_config(const vkh_runner *r, vkh_config *out) {
    if (!r || !out) return fail(VKH_ERR_INVALID_ARGUMENT, "null argument");
    *out = r->cfg;
    return VKH_OK;
}

size_t vkh_runner_param_count(const vkh_runner *r) {
    if (!r) return 0;
    size_t n = r->embed.numel + r->final_norm.numel + (r->tied ? 0 : r->lm_head.numel);
    if (r->lora) {
        n = 0;
        for (const auto &l : r->ls)
            for (int p = 0; p < 7; ++p) n += l.la[p].numel + l.lb[p].numel;
        return n;
    }
    for (const auto &l : r->ls)
        for (int t = 0; t < 11; ++t) n += l.t[t].numel;
    return n;
}

size_t vkh_runner_device_bytes(const vkh_runner *r) { return r ? r->dev_bytes : 0; }

uint32_t vkh_runner_attention_backward_path(const vkh_runner *r) {
    if (!r) return VKH_ATTN_BW_ROWWISE;
    if (r->attn_v4) return VKH_ATTN_BW_RECOMPUTE;
    if (r->attn_fused) return VKH_ATTN_BW_DS_GEMM;
    return VKH_ATTN_BW_ROWWISE;
}

vkh_status vkh_runner_attention_backward_plan(const vkh_runner *r, uint32_t out[5]) {
    if (!r || !out) return fail(VKH_ERR_INVALID_ARGUMENT, "null argument");
    out[0] = vkh_runner_attention_backward_path(r);
    out[1] = out[2] = out[3] = out[4] = 0;
    if (r->attn_v4) {
        const AttnShape s = r->attn_shape();
        out[1] = (uint32_t)fa_bw_v4_q_rows(s);
        out[2] = (uint32_t)fa_bw_v4_q_blocks(s);
        out[3] = (uint32_t)fa_bw_v4_kv_launch_blocks(s, r->attn_split != nullptr);
        out[4] = r->qk_fused ? 1u : 0u;
    }
    return VKH_OK;
}

vkh_status vkh_runner_tensor_numel(const vkh_runner *r, int kind, int layer, int which,
                                   size_t *numel) {
    if (!r || !numel) return fail(VKH_ERR_INVALID_ARGUMENT, "null argument");
    const Span *s = r->find(layer, which);
    if (!s || kind < 0 || kind > 3) return fail(VKH_ERR_INVALID_ARGUMENT, "no tensor (%d, %d, %d)", kind, layer, which);
    if (kind != VKH_PARAM && !r->ptr(kind, *s)) return fail(VKH_ERR_INVALID_ARGUMENT, "tensor is frozen");
    *numel = s->numel;
    return VKH_OK;
}

static vkh_status tensor_ptr(vkh_runner *r, int kind, int layer, int which, float **dptr,
                             size_t *numel, bf16 **dptr16 = nullptr) {
    if (!r || !dptr) return fail(VKH_ERR_INVALID_ARGUMENT, "null argument");
    size_t n = 0;
    VKH_TRY(vkh_runner_tensor_numel(r, kind, layer, which, &n));
    const Span &s = *r->find(layer, which);
    *dptr = r->ptr(kind, s);
    if (dptr16) *dptr16 = kind == VKH_PARAM && r->bf16_only(s) ? r->Pb + s.off : nullptr;
    if (numel) *numel = n;
    return VKH_OK;
}

// The caller may write parameters through the returned pointer, so the bf16
// weight shadow is re-cast before the next forward pass.
vkh_status vkh_runner_tensor_device_ptr(vkh_runner *r, int kind, int layer, int which,
                                        float **dptr, size_t *numel) {
    VKH_TRY(tensor_ptr(r, kind, layer, which, dptr, numel));
    if (!*dptr)
        return fail(VKH_ERR_UNSUPPORTED, "a frozen base matrix of a bf16 LoRA runner has no fp32 copy");
    if (kind == VKH_PARAM) r->shadow_dirty = true;
    return VKH_OK;
}

vkh_status vkh_runner_get_tensor(vkh_runner *r, int kind, int layer, int which, float *host,
                                 size_t numel) {
    float *d = nullptr;
    bf16 *d16 = nullptr;
    size_t n = 0;
    VKH_TRY(tensor_ptr(r, kind, layer, which, &d, &n, &d16));
    if (numel != n || !host) return fail(VKH_ERR_INVALID_ARGUMENT, "numel %zu != %zu", numel, n);
    VKH_TRY(r->host_wait());
    if (d16) return read_bf16_widened(d16, n, host);  // bf16-only base matrix
    VKH_HIP(hipMemcpy(host, d, n * 4, hipMemcpyDeviceToHost));
    return VKH_OK;
}

vkh_status vkh_runner_set_boundary_capture(vkh_runner *r, uint32_t on) {
    if (!r) return fail(VKH_ERR_INVALID_ARGUMENT, "null runner");
    VKH_TRY(r->host_wait());
    if (on && !r->bnd_grad) VKH_TRY(r->alloc(r->bnd_grad, (size_t)(r->L + 1) * r->T * r->D));
    r->bnd_capture = on != 0;
    return VKH_OK;
}

vkh_status vkh_runner_boundary_read(vkh_runner *r, uint32_t l, uint32_t which, float *host,
                                    size_t numel) {
    if (!r || !host) return fail(VKH_ERR_INVALID_ARGUMENT, "null argument");
    if ((int)l > r->L || which > 1) return fail(VKH_ERR_INVALID_ARGUMENT, "boundary %u / %u", l, which);
    const size_t n = (size_t)r->T * r->D;
    if (numel != n) return fail(VKH_ERR_INVALID_ARGUMENT, "numel %zu != %zu", numel, n);
    const float *src;
    if (which == 0) {
        src = l == 0 ? r->x_emb : r->acts[l - 1].y;
    } else {
        if (!r->bnd_grad) return fail(VKH_ERR_INVALID_ARGUMENT, "boundary capture was never on");
        src = r->bnd_grad + (size_t)l * n;
    }
    VKH_TRY(r->host_wait());
    VKH_HIP(hipMemcpy(host, src, n * 4, hipMemcpyDeviceToHost));
    return VKH_OK;
}

vkh_status vkh_runner_set_tensor(vkh_runner *r, int kind, int layer, int which,
                                 const float *host, size_t numel) {
    float *d = nullptr;
    bf16 *d16 = nullptr;
    size_t n = 0;
    VKH_TRY(tensor_ptr(r, kind, layer, which, &d, &n, &d16));
    if (numel != n || !host) return fail(VKH_ERR_INVALID_ARGUMENT, "numel %zu != %zu", numel, n);
    VKH_TRY(r->host_wait());
    if (d16) return write_bf16_rounded(d16, n, host);  // bf16-only base matrix
    VKH_HIP(hipMemcpy(d, host, n * 4, hipMemcpyHostToDevice));
    if (kind == VKH_PARAM) r->shadow_dirty = true;
    return VKH_OK;
}

vkh_status vkh_runner_save_checkpoint(vkh_runner *r, const char *path) {
    if (!r || !path) return fail(VKH_ERR_INVALID_ARGUMENT, "null argument");
    std::vector<Blob> b;
    collect_blobs(r, b);
    return save_blobs(r, path, "VKPT", b);
}

vkh_status vkh_runner_load_checkpoint(vkh_runner *r, const char *path) {
    if (!r || !path) return fail(VKH_ERR_INVALID_ARGUMENT, "null argument");
    std::vector<Blob> b;
    collect_blobs(r, b);
    r->shadow_dirty = true;
    return load_blobs(r, path, "VKPT", false, b);
}

vkh_status vkh_runner_save_lora_checkpoint(vkh_runner *r, const char *path) {
    if (!r || !path) return fail(VKH_ERR_INVALID_ARGUMENT, "null argument");
    if (!r->lora) return fail(VKH_ERR_LORA_CHECKPOINT_EMPTY, "runner has no LoRA state");
    std::vector<Blob> b;
    collect_lora_blobs(r, b);
    return save_blobs(r, path, "VLKP", b);
}

vkh_status vkh_runner_load_lora_checkpoint(vkh_runner *r, const char *path) {
    if (!r || !path) return fail(VKH_ERR_INVALID_ARGUMENT, "null argument");
    if (!r->lora) return fail(VKH_ERR_LORA_CHECKPOINT_EMPTY, "runner has no LoRA state");
    std::vector<Blob> b;
    collect_lora_blobs(r, b);
    r->shadow_dirty = true;
    return load_blobs(r, path, "VLKP", true, b);
}

vkh_status vkh_runner_upload_train_batch(vkh_runner *r, const uint32_t *token_ids,
                                         size_t n_tokens, const uint32_t *target_ids,
                                         size_t n_targets) {
    if (!r) return fail(VKH_ERR_INVALID_ARGUMENT, "null runner");
    VKH_TRY(r->check_ids(token_ids, n_tokens, target_ids, n_targets));
    VKH_TRY(r->begin_on(r->own));
    vkh_status s = r->upload_ids(token_ids, target_ids);
    const vkh_status se = r->end_on();
    if (s == VKH_OK) s = se;
    if (s != VKH_OK) return s;
    VKH_HIP(hipStreamSynchronize(r->own));
    r->batch_ready = true;
    return VKH_OK;
}

vkh_status vkh_runner_set_loss_target(vkh_runner *r, float target) {
    if (!r) return fail(VKH_ERR_INVALID_ARGUMENT, "null runner");
    r->loss_target = target;
    return VKH_OK;
}

// runner.zig:904-986 tickFrameTrain over the transformer step: up to the
// budget of steps on the staged batch, enqueued on the caller's stream.  The
// loss reported is the one staged by an earlier tick, once its copy has
// landed.  With a loss target, that loss gates training (idle while it is at
// or below the target) and every tick enqueues a fresh loss evaluation of the
// staged batch after its steps, so uploading a batch whose loss is above the
// target resumes training; without one, the loss of the tick's last step is
// staged.
vkh_status vkh_runner_tick_frame_train(vkh_runner *r, vkh_stream stream,
                                       vkh_train_budget budget, vkh_tick_result *out) {
    if (!r || !out) return fail(VKH_ERR_INVALID_ARGUMENT, "null argument");
    memset(out, 0, sizeof(*out));
    if (!r->batch_ready) return fail(VKH_ERR_INVALID_ARGUMENT, "no train batch uploaded");
    if (budget.mode > VKH_BUDGET_EITHER) return fail(VKH_ERR_INVALID_ARGUMENT, "unknown budget mode %u", budget.mode);
    const auto t0 = std::chrono::steady_clock::now();
    if (r->tick_loss_pending && hipEventQuery(r->tick_loss_ready) == hipSuccess) {
        r->last_loss_v = r->loss_h[1];
        r->has_last = true;
    }
    out->has_loss = r->has_last ? 1u : 0u;
    out->last_loss = r->has_last ? r->last_loss_v : 0.f;
    const uint32_t max_steps = budget.mode == VKH_BUDGET_MICROSECONDS ? UINT32_MAX : budget.steps;
    const uint64_t us_cap = budget.mode == VKH_BUDGET_STEPS ? UINT64_MAX : budget.microseconds;
    if (max_steps == 0 || us_cap == 0) {  // runner.zig:924-926
        out->idle = 1;
        return VKH_OK;
    }
    const bool decay = r->loss_target > 0.f;
    const bool should_train = !decay || !r->has_last || r->last_loss_v > r->loss_target;
    VKH_TRY(r->begin_on(stream ? (hipStream_t)stream : r->own));
    vkh_status st = VKH_OK;
    uint32_t n = 0;
    while (should_train && n < max_steps) {
        st = r->forward_backward_enqueue(true);
        if (st == VKH_OK && !r->concurrent) st = r->adam_enqueue();
        if (st != VKH_OK) break;
        r->step_t += 1;
        ++n;
        const uint64_t us = (uint64_t)std::chrono::duration_cast<std::chrono::microseconds>(
                                std::chrono::steady_clock::now() - t0).count();
        if (us >= us_cap) break;
    }
    if (st == VKH_OK) {
        if (decay) st = r->loss_eval_enqueue();
        else if (n > 0) st = r->record_tick_loss();
    }
    const vkh_status se = r->end_on();
    if (st == VKH_OK) st = se;
    out->steps_completed = n;
    out->idle = should_train ? 0u : 1u;
    out->elapsed_us = (uint64_t)std::chrono::duration_cast<std::chrono::microseconds>(
                          std::chrono::steady_clock::now() - t0).count();
    return st;
}

// The checkpoint config block (the reference's Config bytes) as a codec, for
// hosts and tests that read or write checkpoint files themselves.
vkh_status vkh_checkpoint_config_encode(const vkh_config *cfg, void *out, size_t out_len) {
    if (!cfg || !out) return fail(VKH_ERR_INVALID_ARGUMENT, "null argument");
    if (out_len < kZigCfgSize) return fail(VKH_ERR_INVALID_ARGUMENT, "out_len %zu < %u", out_len, kZigCfgSize);
    zig_cfg_encode(*cfg, (uint8_t *)out);
    return VKH_OK;
}

vkh_status vkh_checkpoint_config_decode(const void *in, size_t in_len, vkh_config *out) {
    if (!in || !out) return fail(VKH_ERR_INVALID_ARGUMENT, "null argument");
    if (in_len != kZigCfgSize)
        return fail(VKH_ERR_CHECKPOINT_CONFIG_SIZE_MISMATCH, "in_len %zu != %u", in_len, kZigCfgSize);
    memset(out, 0, sizeof(*out));
    out->n_seqs = 1;
    zig_cfg_decode((const uint8_t *)in, *out);
    return VKH_OK;
}

}  // extern "C"
