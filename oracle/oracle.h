/*
 * CPU oracle for the valkyr transformer-training hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker the parity tests,
 * `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` compare
 * the HIP path against.  Nothing in the product (`valkyr_amd/`) links, loads
 * or calls it, and the product fails loudly when its own HIP library is
 * missing instead of falling back here.
 *
 * It restates, in plain C, the reference's scalar CPU oracles
 * (the `src/cpu/` Zig files of `/root/reference`, which cannot be compiled in this
 * image) plus the GPU Runner semantics that those oracles do not encode
 * (the Adam shader form, the FA + CCE + QK-norm + RoPE step order of
 * `src/train/transformer.zig`).  Loop orders and the fp64 accumulators are
 * kept where the Zig has them; every function cites the file:line it follows.
 *
 * It also restates the tiny-MLP trainer (`src/cpu/train.zig` and the batched
 * semantics of `src/train/runner.zig`), including `Mlp.init`'s generator:
 * Zig 0.14's DefaultPrng (xoshiro256++ seeded by SplitMix64, pinned by the
 * published vectors of both) and `Random.float(f32)`.  Parity unpinned: which
 * bits of the draw `Random.float(f32)` uses for the mantissa (restated from
 * Zig's std source; no Zig toolchain or Zig-written vector exists here).
 *
 * Extensions over the reference (documented where they appear):
 *   - a batch axis: T = n_seqs * seq_len rows; attention is block-diagonal
 *     per sequence and the RoPE position of row r is r % seq_len;
 *   - tied embeddings (lm_head aliases embed, grad = dE + dW_lm);
 *   - an optional bf16-operand mode that rounds GEMM / attention operands to
 *     bf16 (round-to-nearest-even) before each contraction.
 */
#ifndef VALKYR_ORACLE_H
#define VALKYR_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ── threads (OpenMP over independent outputs; results do not depend on the
 * thread count) ─────────────────────────────────────────────────────────── */
void orc_set_threads(int n);
int orc_get_threads(void);

/* ── seeded generator (SplitMix64 + Box-Muller) ─────────────────────────── */
uint64_t orc_splitmix64(uint64_t *state);
void orc_fill_normal(float *x, size_t n, uint64_t seed, float mean, float stddev);
void orc_fill_uniform(float *x, size_t n, uint64_t seed, float lo, float hi);
void orc_fill_ids(uint32_t *x, size_t n, uint64_t seed, uint32_t hi);

/* ── bf16 (upper 16 bits of fp32, round-to-nearest-even) ────────────────── */
uint16_t orc_f32_to_bf16(float f);
float orc_bf16_to_f32(uint16_t h);
void orc_round_bf16(float *x, size_t n);
void orc_to_bf16(const float *x, uint16_t *out, size_t n);

/* ── train_transformer.zig primitives ───────────────────────────────────── */
float orc_rmsnorm_forward_row(const float *x, const float *w, size_t dim, float eps,
                              int gemma_quirk, float *y);
void orc_rmsnorm_forward(const float *x, const float *w, size_t n_rows, size_t dim,
                         float eps, int gemma_quirk, float *y);
void orc_rmsnorm_backward(const float *dy, const float *x, const float *w, size_t n_rows,
                          size_t dim, float eps, int gemma_quirk, float *dx, float *dw_accum);
void orc_embedding_forward(const float *embed, const uint32_t *ids, size_t n_pos,
                           size_t dim, float *out);
void orc_embedding_backward(const float *dy, const uint32_t *ids, size_t n_pos,
                            size_t vocab, size_t dim, float *dE);
int orc_rope_forward_batched(float *out, const float *in, size_t n_rows, size_t n_heads,
                             size_t head_dim, size_t rotary_dim, float theta,
                             size_t seq_len);
int orc_rope_backward_batched(float *d_in, const float *d_out, size_t n_rows,
                              size_t n_heads, size_t head_dim, size_t rotary_dim,
                              float theta, size_t seq_len);
void orc_attention_forward(const float *Q, const float *K, const float *V, size_t n_q,
                           size_t n_kv, size_t n_heads, size_t n_kv_heads, size_t head_dim,
                           int causal, float *scores, float *attn, float *out);
void orc_attention_backward(const float *d_out, const float *Q, const float *K,
                            const float *V, const float *attn, size_t n_q, size_t n_kv,
                            size_t n_heads, size_t n_kv_heads, size_t head_dim,
                            float *d_scores, float *dQ, float *dK, float *dV);
void orc_swiglu_forward(const float *pre_gate, const float *up, size_t n, float *gated);
void orc_swiglu_backward(const float *d_gated, const float *pre_gate, const float *up,
                         size_t n, float *d_pre_gate, float *d_up);

/* ── flash_attn.zig ─────────────────────────────────────────────────────── */
void orc_flash_attention_forward(const float *Q, const float *K, const float *V,
                                 size_t n_q, size_t n_kv, size_t n_heads,
                                 size_t n_kv_heads, size_t head_dim, int causal,
                                 size_t Br, size_t Bc, float *out, float *lse);
void orc_flash_attention_backward(const float *Q, const float *K, const float *V,
                                  const float *O, const float *dO, const float *lse,
                                  size_t n_q, size_t n_kv, size_t n_heads,
                                  size_t n_kv_heads, size_t head_dim, int causal,
                                  float *dQ, float *dK, float *dV);
/* The same with the bf16-operand model of the MFMA kernels (an extension:
 * the reference is fp32 throughout): P rounds to bf16 where it multiplies V
 * (forward, 64-key tiles) and dO (dV); the unscaled dS = P (dP - D) rounds to
 * bf16 where it multiplies Q and K, and 1/sqrt(d) scales the accumulated dQ
 * and dK.  Inputs are expected already rounded to bf16. */
void orc_flash_attention_forward_bf16ops(const float *Q, const float *K, const float *V,
                                         size_t n_q, size_t n_kv, size_t n_heads,
                                         size_t n_kv_heads, size_t head_dim, int causal,
                                         float *out, float *lse);
void orc_flash_attention_backward_bf16ops(const float *Q, const float *K, const float *V,
                                          const float *O, const float *dO, const float *lse,
                                          size_t n_q, size_t n_kv, size_t n_heads,
                                          size_t n_kv_heads, size_t head_dim, int causal,
                                          float *dQ, float *dK, float *dV);
/* FA-2 preprocess of fa_bw_d.comp: D[q,h] = sum_d O*dO (fp64 as in
 * flash_attn.zig:330-334). */
void orc_fa_bw_d(const float *O, const float *dO, size_t n_q, size_t n_heads,
                 size_t head_dim, float *D);

/* ── train_decoder.zig ──────────────────────────────────────────────────── */
void orc_matmul_nt(float *out, const float *x, const float *W, size_t M, size_t N,
                   size_t K);
void orc_linear_backward(const float *dout, const float *x, const float *W, size_t M,
                         size_t N, size_t K, float *dx /* nullable */,
                         float *dW /* accumulated, nullable */);

/* ── cce.zig ────────────────────────────────────────────────────────────── */
float orc_cce_forward(const float *h, const float *w_lm, const uint32_t *tgt, size_t n,
                      size_t vocab, size_t dim, size_t chunk, float z_loss_scale,
                      float label_smoothing, float *lse_out, float *loss_row_out);
void orc_cce_backward(const float *h, const float *w_lm, const uint32_t *tgt,
                      const float *lse, size_t n, size_t vocab, size_t dim, size_t chunk,
                      float z_loss_scale, float label_smoothing, float *d_h,
                      float *dW /* accumulated, nullable */);
/* bf16-operand model of the MFMA path: dz rounded to bf16 before dh and dW. */
void orc_cce_backward_bf16ops(const float *h, const float *w_lm, const uint32_t *tgt,
                              const float *lse, size_t n, size_t vocab, size_t dim,
                              float z_loss_scale, float label_smoothing, float *d_h, float *dW);
/* train_decoder.zig:738-785: materialised softmax-CE loss and d_logits. */
float orc_softmax_ce_loss(const float *logits, const uint32_t *tgt, size_t n_pos,
                          size_t vocab);
void orc_softmax_ce_loss_grad(float *d_logits, const float *logits, const uint32_t *tgt,
                              size_t n_pos, size_t vocab);

/* ── lora.zig ───────────────────────────────────────────────────────────── */
void orc_lora_forward(const float *x, const float *w, const float *a, const float *b,
                      size_t M, size_t N, size_t K, size_t r, float alpha_over_r,
                      float *y_out, float *intermediate_out);
void orc_lora_backward(const float *dy, const float *x, const float *w, const float *a,
                       const float *b, const float *intermediate, size_t M, size_t N,
                       size_t K, size_t r, float alpha_over_r, float *dx /* nullable */,
                       float *dA /* accumulated */, float *dB /* accumulated */);

/* ── Adam ───────────────────────────────────────────────────────────────── */
void orc_adam_step(float *param, const float *grad, float *m, float *v, size_t n,
                   float lr, float beta1, float beta2, float eps, uint32_t t,
                   float weight_decay);
void orc_adam_step_folded(float *param, const float *grad, float *m, float *v, size_t n,
                          float lr, float beta1, float beta2, float eps, uint32_t t);

/* ── whole-model step (GPU Runner semantics) ────────────────────────────── */
typedef struct {
    uint32_t dim, n_heads, n_kv_heads, head_dim, ff_dim;
    uint32_t seq_len;   /* reference Config.n_pos: positions per sequence */
    uint32_t n_seqs;    /* batch extension; T = n_seqs * seq_len */
    uint32_t n_layers, vocab_size;
    float rms_eps;
    uint32_t causal, rotary_dim;
    float rope_theta;
    uint32_t qk_norm;
    float lr, beta1, beta2, eps_adam;
    uint32_t lora_targets, lora_rank;
    float lora_alpha, lora_lr_b_scale;
    uint32_t tied_embeddings;
    uint32_t bf16_operands; /* round contraction operands to bf16 */
} orc_model_config;

/* Tensor kinds / ids shared with the HIP runner's layout. */
enum { ORC_PARAM = 0, ORC_GRAD = 1, ORC_ADAM_M = 2, ORC_ADAM_V = 3 };
enum {
    ORC_T_EMBED = 0, ORC_T_FINAL_NORM = 1, ORC_T_LM_HEAD = 2,
    ORC_T_N1 = 0, ORC_T_Q = 1, ORC_T_K = 2, ORC_T_V = 3, ORC_T_O = 4, ORC_T_N2 = 5,
    ORC_T_GATE = 6, ORC_T_UP = 7, ORC_T_DOWN = 8, ORC_T_Q_NORM = 9, ORC_T_K_NORM = 10,
    ORC_T_LORA_A = 16, ORC_T_LORA_B = 17
};

typedef struct orc_model orc_model;
orc_model *orc_model_create(const orc_model_config *cfg);
void orc_model_destroy(orc_model *m);
/* Pointer to a tensor: layer = -1 for stack-level tensors.  For LoRA tensors
 * `which` = 16 + 2*proj (A) or 17 + 2*proj (B), proj in q,k,v,o,gate,up,down. */
float *orc_model_tensor(orc_model *m, int kind, int layer, int which, size_t *numel);
/* Deterministic random init of the configs' distribution: matrices ~N(0,std),
 * norm gains = 1, LoRA A ~N(0, lora_std), B = 0. */
void orc_model_init_random(orc_model *m, uint64_t seed, float std, float lora_std);
/* forward + CCE loss + backward (grads written, not applied). Returns loss. */
float orc_model_forward_backward(orc_model *m, const uint32_t *tokens,
                                 const uint32_t *targets);
/* The stages of orc_model_forward_backward on caller-given inputs (the same
 * code it runs), for stage-by-stage comparisons: the head on the last layer's
 * output y (loss returned; writes the gradient at y, the final-norm gain and
 * lm_head gradients), one layer's forward and backward from its input and the
 * gradient at its output (writes the layer's gradients and the gradient at
 * its input; its stored activations are replaced), and the embedding gradient
 * from the gradient at the embedding output (tied: plus the head's dW_lm from
 * the last head call). */
float orc_model_head_forward_backward(orc_model *m, const float *y, const uint32_t *targets,
                                      float *d_y);
void orc_model_layer_forward_backward(orc_model *m, int l, const float *x_in, const float *d_y,
                                      float *d_x_in);
void orc_model_embedding_backward(orc_model *m, const uint32_t *tokens, const float *d_x0);
/* Layer l's output y from the last forward (l = -1: the embedding output). */
void orc_model_layer_output(const orc_model *m, int l, float *out);
/* Adam over every trainable tensor with t = step_t, then step_t += 1. */
void orc_model_adam(orc_model *m);
float orc_model_step(orc_model *m, const uint32_t *tokens, const uint32_t *targets);
uint32_t orc_model_step_t(const orc_model *m);
void orc_model_set_step_t(orc_model *m, uint32_t t);
/* Wall seconds spent per phase since the last reset (timing for the CPU
 * baseline): layer forwards and backwards (attention included), the attention
 * inside them, the head (embedding, final norm, CCE, tied sum) and Adam. */
enum {
    ORC_PHASE_LAYER_FWD = 0, ORC_PHASE_LAYER_BWD = 1, ORC_PHASE_ATTN_FWD = 2,
    ORC_PHASE_ATTN_BWD = 3, ORC_PHASE_HEAD = 4, ORC_PHASE_ADAM = 5, ORC_N_PHASES = 6
};
void orc_model_phase_seconds(const orc_model *m, double *out);
void orc_model_reset_phases(orc_model *m);
/* forward only: logits [T, vocab] (runner forwardLogits). */
void orc_model_forward_logits(orc_model *m, const uint32_t *tokens, float *logits);

/* ── tiny-MLP TrainingRunner (cpu/train.zig, runner.zig) ────────────────────
 * Parameter blob: [W1 (H x I) | b1 (H) | W2 (O x H) | b2 (O)]. */
void orc_zig_prng_seed(uint64_t s[4], uint64_t seed);
uint64_t orc_zig_prng_next(uint64_t s[4]);
float orc_zig_float32(uint64_t s[4]);
size_t orc_mlp_param_count(size_t I, size_t H, size_t O);
void orc_mlp_init(float *P, size_t I, size_t H, size_t O, float init_scale, uint64_t seed);
void orc_mlp_forward(const float *P, size_t I, size_t H, size_t O, const float *x, float *h_pre,
                     float *h, float *y);
float orc_mse_loss(const float *y, const float *t, size_t n);
void orc_mse_loss_grad(float *dy, const float *y, const float *t, size_t n);
void orc_mlp_backward(const float *P, size_t I, size_t H, size_t O, const float *x,
                      const float *h_pre, const float *h, const float *dy, float *G);
void orc_sgd_step(float *p, const float *g, size_t n, float lr, float weight_decay);
float orc_mlp_train_step(float *P, float *G, size_t I, size_t H, size_t O, const float *x,
                         const float *t, float lr);
void orc_softmax_ce_grad_row(float *dy, const float *y, const float *t, size_t n);
float orc_mlp_batch_loss(const float *P, size_t I, size_t H, size_t O, const float *x,
                         const float *t, size_t N, int cross_entropy);
void orc_mlp_batch_step(float *P, float *G, float *M, float *V, size_t I, size_t H, size_t O,
                        const float *x, const float *t, size_t N, int cross_entropy, int adam,
                        float lr, float weight_decay, float beta1, float beta2, float eps,
                        uint32_t t_step);

/* time helpers for the CPU baseline */
double orc_now_seconds(void);

#ifdef __cplusplus
}
#endif
#endif
