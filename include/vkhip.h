/*
 * vkhip — MI355X (gfx950) training backward path of valkyr, C ABI.
 *
 * Drop-in boundary for valkyr's transformer training step
 * (src/train/transformer.zig `Runner`) and the kernels it records.  All entry
 * points are `extern "C"`, take plain pointers and sizes, and return a
 * `vkh_status`; no C++ or framework types cross the boundary.  A Zig host
 * binds this header with `@cImport` / `extern fn`.
 *
 * Conventions
 *   - Errors: `vkh_status`, mirroring the Zig error names of the reference;
 *     `vkh_last_error()` returns a thread-local message for the last failure.
 *   - Ownership: input pointers are borrowed; the runner owns its device memory.
 *   - Threading: one runner per thread; a runner is never called concurrently.
 *   - Streams: `vkh_stream` is a `hipStream_t` (NULL = the runner's own
 *     stream for runner calls, the null stream for kernel calls).  Kernel
 *     entry points only enqueue; runner `step`/`forward_logits`/checkpoint
 *     calls are blocking like the reference's.  A runner orders its own work
 *     across streams: work enqueued on a caller stream (step_async,
 *     tick_frame_train) completes before any later runner call reads or
 *     writes the same memory, on any stream or from the host.
 *   - Layout: weights are [N, K] row-major with y = x W^T; activations are
 *     [T, dim] with T = n_seqs * n_pos rows; Q, O, dO are [T, n_heads, head_dim]
 *     and K, V are [T, n_kv_heads, head_dim]; LSE and D are [T, n_heads].
 */
#ifndef VKHIP_H
#define VKHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t *vkh_stream;
typedef struct ihipEvent_t *vkh_event;

typedef enum vkh_status {
    VKH_OK = 0,
    VKH_ERR_INVALID_ARGUMENT = 1,
    VKH_ERR_HIP = 2,               /* a HIP runtime call or kernel launch failed */
    VKH_ERR_OUT_OF_MEMORY = 3,
    VKH_ERR_UNSUPPORTED = 4,       /* shape outside what the kernels implement */
    VKH_ERR_NO_DEVICE = 5,
    /* Runner.step / forwardLogits: transformer.zig:1259-1260, :1326-1327 */
    VKH_ERR_TOKEN_IDS_LEN = 10,
    VKH_ERR_TARGET_LEN = 11,
    VKH_ERR_OUT_LOGITS_LEN = 12,
    VKH_ERR_TOKEN_OUT_OF_RANGE = 13,
    /* Runner.init shape validation: transformer.zig:497-515 */
    VKH_ERR_EMBED_SHAPE = 20,
    VKH_ERR_FINAL_NORM_SHAPE = 21,
    VKH_ERR_LM_HEAD_SHAPE = 22,
    VKH_ERR_LAYER_COUNT = 23,
    VKH_ERR_LAYER_N1_SHAPE = 24,
    VKH_ERR_LAYER_Q_SHAPE = 25,
    VKH_ERR_LAYER_K_SHAPE = 26,
    VKH_ERR_LAYER_V_SHAPE = 27,
    VKH_ERR_LAYER_O_SHAPE = 28,
    VKH_ERR_LAYER_N2_SHAPE = 29,
    VKH_ERR_LAYER_GATE_SHAPE = 30,
    VKH_ERR_LAYER_UP_SHAPE = 31,
    VKH_ERR_LAYER_DOWN_SHAPE = 32,
    VKH_ERR_LAYER_Q_NORM_SHAPE = 33,
    VKH_ERR_LAYER_K_NORM_SHAPE = 34,
    VKH_ERR_LORA_RANK_ZERO = 35,
    VKH_ERR_LORA_INIT_LEN = 36,
    /* checkpoints: transformer.zig:1434-1440, :1480, :1527-1533 */
    VKH_ERR_INVALID_CHECKPOINT_MAGIC = 40,
    VKH_ERR_UNSUPPORTED_CHECKPOINT_VERSION = 41,
    VKH_ERR_CHECKPOINT_CONFIG_SIZE_MISMATCH = 42,
    VKH_ERR_CHECKPOINT_CONFIG_MISMATCH = 43,
    VKH_ERR_END_OF_STREAM = 44,    /* truncated file (readNoEof) */
    VKH_ERR_INVALID_LORA_CHECKPOINT_MAGIC = 45,
    VKH_ERR_UNSUPPORTED_LORA_CHECKPOINT_VERSION = 46,
    VKH_ERR_LORA_CHECKPOINT_CONFIG_SIZE_MISMATCH = 47,
    VKH_ERR_LORA_CHECKPOINT_CONFIG_MISMATCH = 48,
    VKH_ERR_LORA_CHECKPOINT_EMPTY = 49,
    VKH_ERR_IO = 50,
    /* dataset / fine-tune loop: train/dataset.zig:52-62, :140; commands/finetune.zig:132-135 */
    VKH_ERR_INPUT_IDS_LEN = 60,
    VKH_ERR_TARGET_IDS_LEN = 61,
    VKH_ERR_BATCH_INDEX_OUT_OF_RANGE = 62,
    VKH_ERR_EMPTY_DATASET = 63,
    VKH_ERR_DATASET_TOO_SHORT = 64,
    VKH_ERR_BATCH_IDX_OUT_OF_RANGE = 65,
    /* tiny-MLP TrainingRunner (train/runner.zig) */
    VKH_ERR_HIDDEN_DIM_EXCEEDS_MAX = 70,
    VKH_ERR_X_DIM_MISMATCH = 71,
    VKH_ERR_TARGET_DIM_MISMATCH = 72,
    VKH_ERR_OUT_DIM_MISMATCH = 73,
    VKH_ERR_BATCH_SIZE_NOT_CONFIGURED = 74,
    VKH_ERR_BATCH_SIZE_EXCEEDS_MAX = 75,
    VKH_ERR_X_BATCH_DIM_MISMATCH = 76,
    VKH_ERR_TARGET_BATCH_DIM_MISMATCH = 77,
    VKH_ERR_OUT_BATCH_DIM_MISMATCH = 78,
    VKH_ERR_OUTPUT_TOO_LARGE = 79
} vkh_status;

typedef enum vkh_precision {
    VKH_PRECISION_FP32 = 0, /* fp32 operands on v_mfma_f32_16x16x4_f32 (reference numerics) */
    VKH_PRECISION_BF16 = 1  /* bf16 operands, fp32 accumulate, fp32 master weights/optimizer */
} vkh_precision;

typedef enum vkh_dtype { VKH_F32 = 0, VKH_BF16 = 1 } vkh_dtype;

/* LoRA target bits: transformer.zig:82-98 (LoraTarget). */
enum {
    VKH_LORA_Q = 1u << 0, VKH_LORA_K = 1u << 1, VKH_LORA_V = 1u << 2, VKH_LORA_O = 1u << 3,
    VKH_LORA_GATE = 1u << 4, VKH_LORA_UP = 1u << 5, VKH_LORA_DOWN = 1u << 6,
    VKH_LORA_ALL_ATTN = 0xFu, VKH_LORA_ALL_FFN = 0x70u, VKH_LORA_ALL = 0x7Fu
};

/* transformer.zig:31-77 (Config) plus four extensions at the end. */
typedef struct vkh_config {
    uint32_t dim, n_heads, n_kv_heads, head_dim, ff_dim;
    uint32_t n_pos;            /* positions per sequence */
    uint32_t n_layers, vocab_size;
    float rms_eps;
    uint32_t causal;
    uint32_t rotary_dim;
    float rope_theta;
    uint32_t qk_norm;
    float lr, beta1, beta2, eps_adam;
    uint32_t lora_targets, lora_rank;
    float lora_alpha, lora_lr_b_scale;
    /* extensions */
    uint32_t n_seqs;           /* sequences per step (0 means 1); T = n_seqs * n_pos */
    uint32_t tied_embeddings;  /* lm_head aliases embed; grad = dE + dW_lm */
    uint32_t precision;        /* vkh_precision */
    uint32_t recompute;        /* 1: per-layer activation recompute -- each layer keeps only
                                  its input and its attention output O and LSE; the rest of
                                  its forward (projections, norms, SwiGLU) runs again just
                                  before its backward (same kernels, so the same gradients
                                  bit for bit) */
} vkh_config;

/* A borrowed host fp32 tensor (a Zig slice: pointer + element count). */
typedef struct vkh_tensor {
    const float *data;
    size_t len;
} vkh_tensor;

/* transformer.zig:113-127 (LayerWeights). */
typedef struct vkh_layer_weights {
    vkh_tensor w_n1, w_q, w_k, w_v, w_o, w_n2, w_gate, w_up, w_down, w_q_norm, w_k_norm;
} vkh_layer_weights;

/* transformer.zig:152-155 (LoraInitWeights). */
typedef struct vkh_lora_init {
    vkh_tensor a; /* [r, K_proj] */
    vkh_tensor b; /* [N_proj, r] */
} vkh_lora_init;

/* transformer.zig:129-150 (InitWeights).  `lora[p]` is NULL (default init:
 * A ~ N(0, 1/sqrt(r)) from a fixed seed, B = 0) or an array of n_layers. */
typedef struct vkh_init_weights {
    vkh_tensor embed, final_norm, lm_head;
    const vkh_layer_weights *layers;
    size_t n_layers;
    const vkh_lora_init *lora[7];
    size_t lora_len[7];
} vkh_init_weights;

typedef struct vkh_runner vkh_runner;

/* Tensor addressing for get/set: stack-level tensors use layer = -1 and
 * which = 0 embed, 1 final_norm, 2 lm_head; per-layer which = 0 n1, 1 q, 2 k,
 * 3 v, 4 o, 5 n2, 6 gate, 7 up, 8 down, 9 q_norm, 10 k_norm; LoRA adapters
 * which = 16 + 2 * proj (A) and 17 + 2 * proj (B), proj = 0..6 (q..down). */
typedef enum vkh_kind { VKH_PARAM = 0, VKH_GRAD = 1, VKH_ADAM_M = 2, VKH_ADAM_V = 3 } vkh_kind;

/* ── runner (transformer.zig Runner) ─────────────────────────────────── */

/* Runner.init (transformer.zig:482).  `weights` may be NULL: matrices start
 * at zero and norm gains at one, to be filled with vkh_runner_set_tensor or
 * vkh_runner_init_random. */
vkh_status vkh_runner_create(const vkh_config *cfg, const vkh_init_weights *weights,
                             vkh_runner **out);
/* Runner.deinit (transformer.zig:1125) */
void vkh_runner_destroy(vkh_runner *r);
/* Device-side deterministic random init of the synthetic configs: matrices
 * ~N(0, std), norm gains 1, LoRA A ~N(0, lora_std), B = 0. */
vkh_status vkh_runner_init_random(vkh_runner *r, uint64_t seed, float std, float lora_std);

/* Runner.step (transformer.zig:1257): one Adam step on n_seqs * n_pos
 * tokens; blocking; step_t += 1 afterwards. */
vkh_status vkh_runner_step(vkh_runner *r, const uint32_t *token_ids, size_t n_tokens,
                           const uint32_t *target_ids, size_t n_targets);
/* The same step enqueued on `stream` without waiting (NULL = runner stream). */
vkh_status vkh_runner_step_async(vkh_runner *r, const uint32_t *token_ids, size_t n_tokens,
                                 const uint32_t *target_ids, size_t n_targets,
                                 vkh_stream stream);
/* Mean CE loss of the last completed step (waits for it). */
vkh_status vkh_runner_last_loss(vkh_runner *r, float *loss);
/* Runner.forwardLogits (transformer.zig:1324): logits [T, vocab] fp32. */
vkh_status vkh_runner_forward_logits(vkh_runner *r, const uint32_t *token_ids, size_t n_tokens,
                                     float *out_logits, size_t out_len);
/* Forward + loss + backward only (grads written, Adam not applied). */
vkh_status vkh_runner_forward_backward(vkh_runner *r, const uint32_t *token_ids,
                                       size_t n_tokens, const uint32_t *target_ids,
                                       size_t n_targets);
vkh_status vkh_runner_synchronize(vkh_runner *r);

uint32_t vkh_runner_step_t(const vkh_runner *r);
vkh_status vkh_runner_set_step_t(vkh_runner *r, uint32_t step_t);
float vkh_runner_get_lr(const vkh_runner *r);
vkh_status vkh_runner_set_lr(vkh_runner *r, float lr); /* cfg.lr is mutable between steps */
vkh_status vkh_runner_get_config(const vkh_runner *r, vkh_config *out);
size_t vkh_runner_param_count(const vkh_runner *r);          /* trainable params */
size_t vkh_runner_device_bytes(const vkh_runner *r);

/* Which attention-backward kernels the runner's step uses (fixed at create
 * from the shape and precision): the recompute MFMA kernels (bf16, head_dim
 * 128, an even GQA group, n_pos a multiple of 128 and at least 128 key blocks
 * of 128), the MFMA kernels with a bf16 dS workspace (other bf16 shapes with
 * n_pos a multiple of 64), or the per-row kernels (fp32 precision and the
 * remaining shapes). */
typedef enum vkh_attn_bw_path {
    VKH_ATTN_BW_ROWWISE = 0,
    VKH_ATTN_BW_DS_GEMM = 1,
    VKH_ATTN_BW_RECOMPUTE = 2
} vkh_attn_bw_path;
uint32_t vkh_runner_attention_backward_path(const vkh_runner *r);
/* The step's attention-backward launch plan (introspection for tests and
 * tuning; the reference has no counterpart): out[0] the path as above,
 * out[1] query rows per dQ block (128, or 256 where that still gives at least
 * one block per CU), out[2] dQ blocks, out[3] dK/dV blocks, out[4] 1 when
 * RoPE^T and the Q/K-norm backward run in the kernels' epilogues.  out[1..4]
 * are 0 off the recompute path. */
vkh_status vkh_runner_attention_backward_plan(const vkh_runner *r, uint32_t out[5]);

/* Stage-by-stage test introspection (the reference has no counterpart).
 * With capture on, every forward/backward keeps the gradient of the loss at
 * each layer boundary: L + 1 fp32 [T, dim] tensors, allocated when capture is
 * first turned on.  vkh_runner_boundary_read copies boundary l in [0, L]:
 * which = 0 the residual-stream tensor there (l = 0 the embedding output,
 * 0 < l <= L the output of layer l - 1, so l = L is the head's input), which
 * = 1 the gradient at it from the last backward run with capture on.
 * Blocking. */
vkh_status vkh_runner_set_boundary_capture(vkh_runner *r, uint32_t on);
vkh_status vkh_runner_boundary_read(vkh_runner *r, uint32_t l, uint32_t which, float *dst,
                                    size_t numel);

/* Tensor access (host <-> device copies, blocking).  A LoRA runner in bf16
 * precision keeps its frozen base matrices (embed, lm_head, q..down) in bf16
 * only: get returns their bf16 values widened to fp32, set rounds to nearest
 * even, and tensor_device_ptr refuses them (VKH_ERR_UNSUPPORTED). */
vkh_status vkh_runner_tensor_numel(const vkh_runner *r, int kind, int layer, int which,
                                   size_t *numel);
vkh_status vkh_runner_get_tensor(vkh_runner *r, int kind, int layer, int which, float *host,
                                 size_t numel);
vkh_status vkh_runner_set_tensor(vkh_runner *r, int kind, int layer, int which,
                                 const float *host, size_t numel);
/* Device pointer of a tensor (valid until vkh_runner_destroy). */
vkh_status vkh_runner_tensor_device_ptr(vkh_runner *r, int kind, int layer, int which,
                                        float **dptr, size_t *numel);

/* Checkpoints, byte layout of transformer.zig:157-205, :1390-1655:
 * 16-byte header {magic, version 1, step_t, cfg_size = 80} + the 80 bytes of
 * the reference's `Config` (VKH_CHECKPOINT_CONFIG_BYTES, see
 * vkh_checkpoint_config_encode) + positional fp32 blobs (.vkpt: (param, m, v)
 * per tensor in collectBlobs order, lm_head included: a tied runner writes
 * its embedding's blobs there and loads only files whose lm_head equals the
 * embedding; .lvkpt: (A, mA, vA, B, mB, vB) per enabled projection and
 * layer).  Loading compares the shape fields of cfgShapeMatches
 * (transformer.zig:197-205) and restores step_t, lr, beta1, beta2, eps_adam
 * (and lora_alpha, lora_lr_b_scale from .lvkpt). */
vkh_status vkh_runner_save_checkpoint(vkh_runner *r, const char *path);
vkh_status vkh_runner_load_checkpoint(vkh_runner *r, const char *path);
vkh_status vkh_runner_save_lora_checkpoint(vkh_runner *r, const char *path);
vkh_status vkh_runner_load_lora_checkpoint(vkh_runner *r, const char *path);

/* The checkpoint config block: std.mem.asBytes(&cfg) of the reference's
 * auto-layout `Config` (transformer.zig:31-77), fields ordered by descending
 * alignment with declaration order kept among equals: offsets 0-28 dim,
 * n_heads, n_kv_heads, head_dim, ff_dim, n_pos, n_layers, vocab_size (u32);
 * 32 rms_eps (f32); 36 rotary_dim (u32); 40 rope_theta, 44 lr, 48 beta1,
 * 52 beta2, 56 eps_adam (f32); 60 lora_targets, 64 lora_rank (u32);
 * 68 lora_alpha, 72 lora_lr_b_scale (f32); 76 causal, 77 qk_norm (bool, one
 * byte); 78-79 padding (written as zero).  That order is inferred from the
 * Zig compiler's auto-layout rules (the reference's `Config` is not extern,
 * transformer.zig:190-193) and is unpinned against any reference-written
 * file.  Host-only: no device work.
 * decode fills the reference's fields and sets the extensions to n_seqs = 1,
 * untied, fp32 precision. */
#define VKH_CHECKPOINT_CONFIG_BYTES 80
vkh_status vkh_checkpoint_config_encode(const vkh_config *cfg, void *out, size_t out_len);
vkh_status vkh_checkpoint_config_decode(const void *in, size_t in_len, vkh_config *out);

/* ── cooperative per-frame API (shape of runner.zig:129-176, :904-986) ── */
typedef enum vkh_budget_mode {
    VKH_BUDGET_STEPS = 0,
    VKH_BUDGET_MICROSECONDS = 1,
    VKH_BUDGET_EITHER = 2
} vkh_budget_mode;

typedef struct vkh_train_budget {
    uint32_t mode;         /* vkh_budget_mode */
    uint32_t steps;        /* max steps this tick */
    uint64_t microseconds; /* max host enqueue time this tick */
} vkh_train_budget;

typedef struct vkh_tick_result {
    uint32_t steps_completed; /* steps enqueued this tick */
    uint32_t has_loss;        /* last_loss valid (one-tick latency) */
    float last_loss;
    uint32_t idle;            /* loss target reached: nothing enqueued */
    uint64_t elapsed_us;
} vkh_tick_result;

/* runner.zig:797 uploadTrainBatch: the batch the following ticks train on. */
vkh_status vkh_runner_upload_train_batch(vkh_runner *r, const uint32_t *token_ids,
                                         size_t n_tokens, const uint32_t *target_ids,
                                         size_t n_targets);
/* runner.zig:61-68 LossDecay target: ticks go idle once last_loss <= target
 * (target <= 0 disables). */
vkh_status vkh_runner_set_loss_target(vkh_runner *r, float target);
/* runner.zig:904 tickFrameTrain: enqueue up to the budget of steps on the
 * caller's stream and return without waiting; the loss staged by an earlier
 * tick is reported once its copy has landed.  A budget of 0 steps or 0 us
 * returns idle with the cached loss (runner.zig:924-926); an unknown mode is
 * VKH_ERR_INVALID_ARGUMENT.  With a loss target (> 0), a tick whose cached
 * loss is <= target is idle (no steps) and every tick enqueues a fresh loss
 * evaluation (forward + CE) of the staged batch, so a newly uploaded batch
 * above the target resumes training (runner.zig:948-973). */
vkh_status vkh_runner_tick_frame_train(vkh_runner *r, vkh_stream stream,
                                       vkh_train_budget budget, vkh_tick_result *out);

/* ── host feed: packed token stream and the fine-tune loop ───────────── */

/* train/dataset.zig Dataset: examples packed into one stream with `eos_id`
 * between them (none after the last), read as sliding windows of n_pos + 1
 * tokens: batch idx = (packed[idx .. idx + n_pos], packed[idx + 1 .. idx + n_pos
 * + 1]), num_batches = len - n_pos (0 when len <= n_pos).  Token ids only:
 * the tokenizer is not part of this library. */
typedef struct vkh_dataset vkh_dataset;

/* buildFromExamples (dataset.zig:76-96) on already-tokenized examples. */
vkh_status vkh_dataset_from_examples(const uint32_t *const *examples, const size_t *lens,
                                     size_t n_examples, uint32_t n_pos, uint32_t eos_id,
                                     vkh_dataset **out);
/* buildFromJsonl (dataset.zig:98-148) with the token ids of a line in an
 * integer array field "ids" (the reference tokenizes a "text" field): empty or
 * whitespace-only lines, lines that do not parse as a JSON object and objects
 * without an "ids" array of integers in [0, 2^32) are skipped; EOS goes
 * between accepted lines.  VKH_ERR_EMPTY_DATASET when no line is usable. */
vkh_status vkh_dataset_from_jsonl(const char *path, uint32_t n_pos, uint32_t eos_id,
                                  vkh_dataset **out);
void vkh_dataset_destroy(vkh_dataset *d);
size_t vkh_dataset_num_batches(const vkh_dataset *d); /* numBatches (dataset.zig:42-47) */
size_t vkh_dataset_packed_len(const vkh_dataset *d);
/* the packed stream itself (n = packed_len) */
vkh_status vkh_dataset_packed(const vkh_dataset *d, uint32_t *out, size_t n);
/* batch (dataset.zig:50-66): errors InputIdsLen, TargetIdsLen, BatchIndexOutOfRange. */
vkh_status vkh_dataset_batch(const vkh_dataset *d, size_t idx, uint32_t *input_ids, size_t n_input,
                             uint32_t *target_ids, size_t n_target);
/* n_seqs windows for one batched step (the n_seqs extension): window s is
 * batch (idx + s * stride) mod num_batches, written at offset s * n_pos. */
vkh_status vkh_dataset_batch_seqs(const vkh_dataset *d, size_t idx, size_t stride, uint32_t n_seqs,
                                  uint32_t *input_ids, uint32_t *target_ids);

/* computeMeanCe (commands/finetune.zig:256-268): mean over rows of
 * log-sum-exp(logits[p]) - logits[p][target[p]], fp64 accumulation. */
float vkh_mean_ce(const float *logits, const uint32_t *target_ids, size_t n_rows, size_t vocab);

typedef struct vkh_finetune_result {
    float ce_initial;   /* on the batch at batch_idx, before the first step */
    float ce_final;     /* same batch after the last step */
    double total_ms;    /* wall time of the step loop */
    double mean_step_ms;
} vkh_finetune_result;

/* The training loop of commands/finetune.zig:155-196: CE on batch `batch_idx`
 * (forward_logits + vkh_mean_ce), n_steps Runner steps on batch `batch_idx`
 * or, with rotate, on (step + batch_idx) mod num_batches, then CE again on
 * `batch_idx`.  With n_seqs > 1 each step trains on n_seqs windows n_pos apart
 * (vkh_dataset_batch_seqs).  Errors: DatasetTooShort (no batch),
 * BatchIdxOutOfRange, and the Runner's own. */
vkh_status vkh_runner_finetune(vkh_runner *r, const vkh_dataset *d, uint32_t batch_idx,
                               uint32_t n_steps, uint32_t rotate, vkh_finetune_result *out);

/* ── tiny-MLP TrainingRunner (train/runner.zig; oracle cpu/train.zig) ───
 * Linear -> ReLU -> Linear trained in place on the GPU, one runner per
 * trained function.  Parameters, gradients and Adam moments are each one fp32
 * blob [W1 (H x I) | b1 (H) | W2 (O x H) | b2 (O)], W row-major with
 * y = W x + b.  Batches are sample-major [N, dim]. */
#define VKH_MLP_MAX_HIDDEN 64 /* MLP2_MAX_HIDDEN, runner.zig:128 */

typedef enum vkh_mlp_optimizer { VKH_MLP_SGD = 0, VKH_MLP_ADAM = 1 } vkh_mlp_optimizer;
typedef enum vkh_mlp_loss { VKH_MLP_MSE = 0, VKH_MLP_CROSS_ENTROPY = 1 } vkh_mlp_loss;
typedef enum vkh_mlp_decay {
    VKH_MLP_DECAY_NONE = 0,
    VKH_MLP_DECAY_LOSS_TARGET = 1 /* idle while last loss <= decay_target */
} vkh_mlp_decay;

/* Mlp2Config (runner.zig:70-123); defaults from vkh_mlp_config_default. */
typedef struct vkh_mlp_config {
    uint32_t dim_in, dim_hidden, dim_out;
    float lr;                /* mutable later: vkh_mlp_set_lr */
    float init_scale;        /* W ~ U(-init_scale, init_scale); 0.3 */
    uint32_t max_batch_size; /* 0 disables the batched surface */
    uint64_t init_seed;      /* Zig DefaultPrng seed of Mlp.init; 0xCAFE */
    uint32_t optimizer;      /* vkh_mlp_optimizer; SGD */
    float adam_beta1, adam_beta2, adam_eps; /* 0.9, 0.999, 1e-8 */
    uint32_t loss;           /* vkh_mlp_loss; MSE */
    uint32_t decay;          /* vkh_mlp_decay; NONE */
    float decay_target;      /* LossDecay.loss_target.target */
    float weight_decay;      /* decoupled, W1 / W2 only; mutable: vkh_mlp_set_weight_decay */
} vkh_mlp_config;

typedef struct vkh_mlp vkh_mlp;

void vkh_mlp_config_default(vkh_mlp_config *c, uint32_t dim_in, uint32_t dim_hidden,
                            uint32_t dim_out, float lr);
/* TrainingRunner.init (runner.zig:329-544): weights from Mlp.init(seed),
 * biases and Adam moments zero.  HiddenDimExceedsMax when dim_hidden > 64. */
vkh_status vkh_mlp_create(const vkh_mlp_config *cfg, vkh_mlp **out);
void vkh_mlp_destroy(vkh_mlp *m); /* deinit (runner.zig:546-592) */
vkh_status vkh_mlp_get_config(const vkh_mlp *m, vkh_mlp_config *out);
vkh_status vkh_mlp_set_lr(vkh_mlp *m, float lr);            /* runner.lr */
float vkh_mlp_get_lr(const vkh_mlp *m);
vkh_status vkh_mlp_set_weight_decay(vkh_mlp *m, float wd);  /* runner.weight_decay */
uint32_t vkh_mlp_adam_step(const vkh_mlp *m);               /* runner.adam_step */

/* Standalone (blocking) calls.  Lengths are element counts of the caller's
 * slices; mismatches return the reference's error names. */
/* tickStep (runner.zig:598-620): one-sample MSE + SGD step; out_pred (may be
 * NULL) gets the prediction before the update.  XDimMismatch,
 * TargetDimMismatch, OutDimMismatch. */
vkh_status vkh_mlp_tick_step(vkh_mlp *m, const float *x, size_t x_len, const float *target,
                             size_t target_len, float *out_pred, size_t out_len);
/* tickPredict (runner.zig:626-637). */
vkh_status vkh_mlp_tick_predict(vkh_mlp *m, const float *x, size_t x_len, float *out_pred,
                                size_t out_len);
/* tickPredictBatch (runner.zig:705-733): BatchSizeNotConfigured,
 * XBatchDimMismatch, BatchSizeExceedsMax, OutBatchDimMismatch. */
vkh_status vkh_mlp_tick_predict_batch(vkh_mlp *m, const float *x_batch, size_t x_len,
                                      float *out_y, size_t out_len);
/* tickStepBatch (runner.zig:746-763): one step on the mean gradient of the
 * batch with the configured loss and optimizer.  TargetBatchDimMismatch too. */
vkh_status vkh_mlp_tick_step_batch(vkh_mlp *m, const float *x_batch, size_t x_len,
                                   const float *target_batch, size_t target_len);

/* Cooperative (attach) calls: enqueue on the caller's stream (NULL: the
 * runner's own) and return without waiting. */
/* uploadTrainBatch / uploadPredictInputs (runner.zig:784-803): blocking
 * copies into the runner's batch buffers; call them when no enqueued work
 * still reads the previous batch. */
vkh_status vkh_mlp_upload_train_batch(vkh_mlp *m, const float *x_batch, size_t x_len,
                                      const float *target_batch, size_t target_len);
vkh_status vkh_mlp_upload_predict_inputs(vkh_mlp *m, const float *x_batch, size_t x_len);
/* tickStepRecord / tickPredictRecord (runner.zig:655-678). */
vkh_status vkh_mlp_tick_step_record(vkh_mlp *m, vkh_stream stream, const float *x, size_t x_len,
                                    const float *target, size_t target_len);
vkh_status vkh_mlp_tick_predict_record(vkh_mlp *m, vkh_stream stream, const float *x,
                                       size_t x_len);
/* tickStepBatchRecord / tickPredictBatchRecord (runner.zig:768-773, :1001-1021). */
vkh_status vkh_mlp_tick_step_batch_record(vkh_mlp *m, vkh_stream stream, uint32_t n_samples);
vkh_status vkh_mlp_tick_predict_batch_record(vkh_mlp *m, vkh_stream stream, uint32_t n_samples);
/* recordPredictReadback / readPredictStaging (runner.zig:815-863): y_batch to
 * pinned staging, read after the stream is synchronized.  OutputTooLarge. */
vkh_status vkh_mlp_record_predict_readback(vkh_mlp *m, vkh_stream stream, uint32_t n_samples);
vkh_status vkh_mlp_read_predict_staging(vkh_mlp *m, float *out_y, size_t out_len);
/* tickFrameTrain (runner.zig:904-986): up to `budget` steps on the uploaded
 * batch; with VKH_MLP_DECAY_LOSS_TARGET the previous tick's loss gates
 * training (idle when <= decay_target) and a fresh loss evaluation is
 * enqueued every tick.  last_loss is reported only under that policy. */
vkh_status vkh_mlp_tick_frame_train(vkh_mlp *m, vkh_stream stream, vkh_train_budget budget,
                                    uint32_t n_samples, vkh_tick_result *out);
/* getLastLoss (runner.zig:991-993). */
vkh_status vkh_mlp_get_last_loss(const vkh_mlp *m, float *loss, uint32_t *has_loss);

/* Device buffers, for GPU-resident consumers of the predictions (the
 * reference binds runner.y / y_batch as shader inputs) and for tests. */
typedef enum vkh_mlp_buffer_id {
    VKH_MLP_BUF_PARAMS = 0, VKH_MLP_BUF_GRADS = 1, VKH_MLP_BUF_ADAM_M = 2,
    VKH_MLP_BUF_ADAM_V = 3, VKH_MLP_BUF_Y = 4, VKH_MLP_BUF_X_BATCH = 5,
    VKH_MLP_BUF_Y_BATCH = 6, VKH_MLP_BUF_X_TRAIN = 7, VKH_MLP_BUF_TARGET = 8,
    VKH_MLP_BUF_H_PRE_TRAIN = 9, VKH_MLP_BUF_H_TRAIN = 10, VKH_MLP_BUF_Y_TRAIN = 11,
    VKH_MLP_BUF_DY_TRAIN = 12, VKH_MLP_BUF_DH_PRE_TRAIN = 13
} vkh_mlp_buffer_id;
vkh_status vkh_mlp_buffer(vkh_mlp *m, uint32_t which, float **dptr, size_t *numel);
/* blocking copy of the first numel floats, after the device is idle */
vkh_status vkh_mlp_read_buffer(vkh_mlp *m, uint32_t which, float *host, size_t numel);
/* readWeights (runner.zig:684-689). */
vkh_status vkh_mlp_read_weights(vkh_mlp *m, float *w1, size_t w1_len, float *b1, size_t b1_len,
                                float *w2, size_t w2_len, float *b2, size_t b2_len);

/* ── kernels (device pointers; enqueue on `stream`) ─────────────────── */

/* Attention shape shared by the FA entry points: FaForwardPush,
 * FaBwDPush, FaBwDqPush, FaBwDkvPush (runtime.zig:377-416) plus n_batch
 * (sequences stacked along rows, block-diagonal attention). */
typedef struct vkh_attn_params {
    uint32_t n_batch, n_q, n_kv, n_heads, n_kv_heads, head_dim;
    uint32_t causal;
    float inv_sqrt_dim;
    uint32_t dtype; /* vkh_dtype of q, k, v, dO; bf16 requires head_dim 64 or 128 */
} vkh_attn_params;

/* shaders/fa_forward.comp (write_lse = 1 when lse != NULL): O fp32. */
vkh_status vkh_fa_forward(const vkh_attn_params *p, const void *q, const void *k, const void *v,
                          float *o, float *lse, vkh_stream stream);
/* shaders/fa_bw_d.comp: D[t, h] = sum_d O * dO.  With p->dtype == bf16, dO is
 * fp32 and `dout_bf16` (if non-NULL) receives its bf16 copy, D pairing with it. */
vkh_status vkh_fa_bw_d(const vkh_attn_params *p, const float *o, const float *dout, float *d,
                       void *dout_bf16, vkh_stream stream);
/* shaders/fa_bw_d.comp with O and dO stored in bf16 (the operand precision of
 * the bf16 attention path: config 2's bf16 dO, the forward's bf16 O): D[t, h] =
 * sum_d O * dO, fp32 out; head_dim 64 or 128. */
vkh_status vkh_fa_bw_d_bf16(const vkh_attn_params *p, const void *o_bf16, const void *dout_bf16,
                            float *d, vkh_stream stream);
/* shaders/fa_bw_dq.comp: dQ fp32 (overwrite). */
vkh_status vkh_fa_bw_dq(const vkh_attn_params *p, const void *q, const void *k, const void *v,
                        const void *dout, const float *lse, const float *d, float *dq,
                        vkh_stream stream);
/* shaders/fa_bw_dkv.comp: dK, dV fp32 (overwrite), GQA fold inside. */
vkh_status vkh_fa_bw_dkv(const vkh_attn_params *p, const void *q, const void *k, const void *v,
                         const void *dout, const float *lse, const float *d, float *dk,
                         float *dv, vkh_stream stream);

/* The FA-2 backward of one attention call after vkh_fa_bw_d (the
 * fa_bw_dkv.comp + fa_bw_dq.comp pair of the reference's attention
 * backward): dK, dV, dQ fp32 (overwrite).  With bf16 operands (head_dim 64 or
 * 128, n_q and n_kv multiples of 64, self-attention when causal):
 *   - head_dim 128, an even number of query heads per KV head and n_kv a
 *     multiple of 128: a dK/dV kernel and a dQ kernel that each form S and
 *     dP themselves (no workspace: vkh_fa_backward_workspace_bytes is 0);
 *   - otherwise dK/dV write dS = P (dP - D) once as bf16 into `workspace` and
 *     dQ = dS K is a GEMM.
 * Other shapes run the two kernels above.  `workspace` may be NULL (allocated
 * per call on the stream when needed) or hold
 * vkh_fa_backward_workspace_bytes(p) bytes. */
size_t vkh_fa_backward_workspace_bytes(const vkh_attn_params *p);
vkh_status vkh_fa_backward(const vkh_attn_params *p, const void *q, const void *k, const void *v,
                           const void *dout, const float *lse, const float *d, float *dq,
                           float *dk, float *dv, void *workspace, vkh_stream stream);
/* The three shaders of the reference's attention backward recorded back to
 * back (fa_bw_d.comp, fa_bw_dkv.comp, fa_bw_dq.comp; transformer.zig:2004-2050)
 * from bf16 O and dO: D = rowsum(O dO) is written to `d` and dK, dV, dQ as in
 * vkh_fa_backward.  On the recompute path the dQ kernel forms D itself (no
 * separate pass); other shapes run vkh_fa_bw_d_bf16 then vkh_fa_backward.
 * bf16 operands only. */
vkh_status vkh_fa_backward_from_o(const vkh_attn_params *p, const void *q, const void *k,
                                  const void *v, const void *o_bf16, const void *dout_bf16,
                                  const float *lse, float *d, float *dq, float *dk, float *dv,
                                  void *workspace, vkh_stream stream);

/* shaders/matmul_nt_v2.comp (MatmulPush {m, n, k}): y[M,N] = x[M,K] w[N,K]^T. */
vkh_status vkh_matmul_nt(const float *x, const float *w, float *y, uint32_t M, uint32_t N,
                         uint32_t K, uint32_t precision, vkh_stream stream);
/* shaders/linear_backward_dx_batched.comp (LinearBatchedPush {M, N, K}):
 * dx[M,K] = dy[M,N] w[N,K]  (overwrite). */
vkh_status vkh_linear_backward_dx(const float *dy, const float *w, float *dx, uint32_t M,
                                  uint32_t N, uint32_t K, uint32_t precision, vkh_stream stream);
/* shaders/linear_backward_dw_batched.comp: dw[N,K] = dy[M,N]^T x[M,K]  (overwrite). */
vkh_status vkh_linear_backward_dw(const float *dy, const float *x, float *dw, uint32_t M,
                                  uint32_t N, uint32_t K, uint32_t precision, vkh_stream stream);

/* bf16-operand forms of the three GEMMs above: every operand is bf16 (RNE
 * bits, as uint16), accumulation and output fp32.  These are the contractions
 * the bf16 training step runs (VKH_PRECISION_BF16 keeps all GEMM operands
 * resident as bf16); the reference's shaders take fp32 buffers only, so they
 * have no direct counterpart there beyond the three entry points above. */
vkh_status vkh_matmul_nt_bf16(const void *x, const void *w, float *y, uint32_t M, uint32_t N,
                              uint32_t K, vkh_stream stream);
/* The bf16 step's gate/up projection and SwiGLU forward: gu[M, 2F] = x[M, K]
 * w_gu[2F, K]^T (w_gu = the gate rows, then the up rows, as Runner stacks
 * them), gated[M, F] = bf16(swiglu(gu[:, f], gu[:, F + f])).  No single
 * counterpart in the reference: it is matmul_nt_v2.comp for w_gate and w_up
 * followed by swiglu_forward.comp (train_transformer.zig:839-851), run as one
 * launch with the SwiGLU in the GEMM's epilogue where the tile plan allows
 * (the 8-wave 128 x 128 tile) and as the two passes elsewhere, with the same
 * bits either way. */
vkh_status vkh_gate_up_swiglu_bf16(const void *x, const void *w_gu, float *gu, void *gated,
                                   uint32_t M, uint32_t F, uint32_t K, vkh_stream stream);
/* The same at the reference's precision (the fp32 step's): fp32 x, w_gu and gated;
 * fused = 0 forces the two passes. */
vkh_status vkh_gate_up_swiglu(const float *x, const float *w_gu, float *gu, float *gated,
                              uint32_t M, uint32_t F, uint32_t K, int fused, vkh_stream stream);
vkh_status vkh_linear_backward_dx_bf16(const void *dy, const void *w, float *dx, uint32_t M,
                                       uint32_t N, uint32_t K, vkh_stream stream);
vkh_status vkh_linear_backward_dw_bf16(const void *dy, const void *x, float *dw, uint32_t M,
                                       uint32_t N, uint32_t K, vkh_stream stream);

/* train/lora.zig:99-129: y = x w^T + (alpha/r) (x a^T) b^T; inter = x a^T. */
vkh_status vkh_lora_forward(const float *x, const float *w, const float *a, const float *b,
                            float *y, float *inter, uint32_t M, uint32_t N, uint32_t K,
                            uint32_t r, float alpha_over_r, uint32_t precision,
                            vkh_stream stream);
/* train/lora.zig:137-251: dx = dy w + (alpha/r) (dy b) a (overwrite, if dx);
 * dA = (alpha/r) (dy b)^T x;  dB = (alpha/r) dy^T inter  (overwrite). */
vkh_status vkh_lora_backward(const float *dy, const float *x, const float *w, const float *a,
                             const float *b, const float *inter, float *dx, float *dA,
                             float *dB, uint32_t M, uint32_t N, uint32_t K, uint32_t r,
                             float alpha_over_r, uint32_t precision, vkh_stream stream);

/* CceForwardPush / CceBackwardPush {N, V, D, z_loss, label_smoothing}
 * (runtime.zig:484-496). */
typedef struct vkh_cce_params {
    uint32_t n, vocab, dim;
    float z_loss_scale, label_smoothing;
    uint32_t precision;
} vkh_cce_params;
/* shaders/cce_forward.comp: lse[n], loss_row[n] (and the mean if non-NULL). */
vkh_status vkh_cce_forward(const vkh_cce_params *p, const float *h, const float *w,
                           const uint32_t *targets, float *lse, float *loss_row,
                           float *loss_mean, vkh_stream stream);
/* One adapter of a grouped LoRA call: output columns [col, col + n) of the
 * group's fused y / dy, input width k, the fp32 factors and per-adapter
 * buffers. */
typedef struct vkh_lora_adapter {
    uint32_t col, n, k;
    const float *a;  /* A [r, k] */
    const float *b;  /* B [n, r] */
    float *inter;    /* x A^T [T, r]: written by the forward, read by the backward */
    float *dyb;      /* dy B [T, r]: written by the backward */
    float *da;       /* dA [r, k] (overwrite) */
    float *db;       /* dB [n, r] (overwrite) */
} vkh_lora_adapter;

/* train/lora.zig:99-129 (forward) and :137-251 (backward) for up to three
 * adapters that share one bf16 activation, launched as the training step
 * launches them on its fused projections (q/k/v on the first norm's output,
 * gate/up on the second's, o and down alone): x and dy are bf16 [T, *] with
 * leading dimensions ldx / lddy (in elements), factors, intermediates and
 * products fp32, fixed summation order.  Forward: inter = x A^T and
 * y[:, col..col+n) += aor inter B^T.  Backward: dyb = dy B, dx += aor dyb A
 * (dx may be NULL), dA = aor dyb^T x, dB = aor dy^T inter.  The rank-r
 * kernels need r a multiple of 4 up to 64, 16-byte aligned rows, and k, n
 * and col multiples of the kernels' column groups; other shapes return
 * VKH_ERR_UNSUPPORTED.  The reference has no grouped call: each adapter is
 * its lora.zig call. */
vkh_status vkh_lora_group_forward_bf16(const uint16_t *x, uint32_t ldx, uint32_t T, uint32_t r,
                                       float aor, const vkh_lora_adapter *adapters,
                                       uint32_t n_adapters, float *y, uint32_t ldy,
                                       vkh_stream stream);
vkh_status vkh_lora_group_backward_bf16(const uint16_t *dy, uint32_t lddy, const uint16_t *x,
                                        uint32_t ldx, uint32_t T, uint32_t r, float aor,
                                        const vkh_lora_adapter *adapters, uint32_t n_adapters,
                                        float *dx, uint32_t lddx, vkh_stream stream);

/* shaders/cce_backward_dh.comp + cce_backward_dw.comp in one pass:
 * dh overwritten (if non-NULL); dw += (accumulate_dw) or = dz^T h (if non-NULL). */
vkh_status vkh_cce_backward(const vkh_cce_params *p, const float *h, const float *w,
                            const uint32_t *targets, const float *lse, float *dh, float *dw,
                            uint32_t accumulate_dw, vkh_stream stream);

/* shaders/rmsnorm.comp (RmsnormPush {dim, eps, gemma_quirk}) */
vkh_status vkh_rmsnorm_forward(const float *x, const float *w, float *y, uint32_t n_rows,
                               uint32_t dim, float eps, uint32_t gemma_quirk, vkh_stream stream);
/* shaders/rmsnorm_backward.comp with the gain gradient reduced on the GPU:
 * dx [n_rows, dim] (+ residual if non-NULL), dw [dim] (overwrite, if non-NULL). */
vkh_status vkh_rmsnorm_backward(const float *dy, const float *x, const float *w, float *dx,
                                const float *residual, float *dw, uint32_t n_rows, uint32_t dim,
                                float eps, uint32_t gemma_quirk, vkh_stream stream);
/* No counterpart in the reference: vkh_rmsnorm_backward for callers that
 * cannot allocate (code under HIP graph capture, serving loops, harnesses that
 * forbid hipMalloc).  Same kernels and results (bit for bit); the gain-gradient
 * partials live in a fixed 8 MiB per-device array inside the library instead
 * of memory it allocates, so the call allocates nothing.  Limit: dim <= 4096
 * (VKH_ERR_UNSUPPORTED beyond).  Calls on one GPU share that array and are
 * ordered on the device like the allocating form's scratch uses (a call on
 * another stream waits for the previous call), except while the caller's
 * stream is being captured into a graph: there the captured launch is not
 * ordered against other uses of the array, and the caller must not run the
 * graph while another call on the same GPU may still be in flight (they
 * race). */
vkh_status vkh_rmsnorm_backward_noalloc(const float *dy, const float *x, const float *w,
                                        float *dx, const float *residual, float *dw,
                                        uint32_t n_rows, uint32_t dim, float eps,
                                        uint32_t gemma_quirk, vkh_stream stream);
/* No counterpart in the reference (test introspection): the number of
 * allocations this library has made in the process so far (device and pinned
 * host memory, and leases of the shared scratch buffer that the standalone
 * entry points use), so a test can check that an entry point allocates
 * nothing. */
uint64_t vkh_allocation_count(void);
/* shaders/swiglu_forward.comp / swiglu_backward.comp (SwigluPush {n}) */
vkh_status vkh_swiglu_forward(const float *pre_gate, const float *up, float *gated, size_t n,
                              vkh_stream stream);
vkh_status vkh_swiglu_backward(const float *d_gated, const float *pre_gate, const float *up,
                               float *d_pre_gate, float *d_up, size_t n, vkh_stream stream);
/* shaders/qk_rope_partial_batched.comp / qk_rope_backward_batched.comp
 * (QkRopeBatchedPush, runtime.zig:221-228) + seq_len: position = row % seq_len. */
typedef struct vkh_rope_params {
    uint32_t n_pos, n_q_heads, n_kv_heads, head_dim, rotary_dim;
    float theta_base;
    uint32_t seq_len; /* 0 means n_pos */
} vkh_rope_params;
vkh_status vkh_qk_rope_forward(const vkh_rope_params *p, const float *q_in, float *q_out,
                               const float *k_in, float *k_out, vkh_stream stream);
vkh_status vkh_qk_rope_backward(const vkh_rope_params *p, const float *dq_out, float *dq_in,
                                const float *dk_out, float *dk_in, vkh_stream stream);
/* The bf16 step's q|k|v projection and attention operand: y[n_pos, (Hq + 2 Hkv) hd]
 * = x[n_pos, K] w^T (bf16 operands, fp32 y: the backward's pre-norm values) and
 * out = bf16 of the q and k heads Q/K-RMSNorm'd (qk_norm, gains wq / wk, eps) and
 * rotated (p), the v heads as they are.  No single counterpart in the reference:
 * it is matmul_nt_v2.comp for w_q, w_k and w_v, rmsnorm.comp over each q and k
 * head, and qk_rope_partial_batched.comp (transformer.zig's forward order),
 * run as one launch with the norm and rotation in the GEMM's epilogue where
 * head_dim is 128 and the tile plan allows (fused != 0), as the two passes
 * otherwise (fused = 0 forces them); the same bits either way. */
vkh_status vkh_qkv_project_bf16(const vkh_rope_params *p, uint32_t K, float eps, int qk_norm,
                                const void *x, const void *w, const float *wq, const float *wk,
                                float *y, void *out, int fused, vkh_stream stream);
/* The same at the reference's precision (the fp32 step's): fp32 x, w and out. */
vkh_status vkh_qkv_project(const vkh_rope_params *p, uint32_t K, float eps, int qk_norm,
                           const float *x, const float *w, const float *wq, const float *wk,
                           float *y, float *out, int fused, vkh_stream stream);
/* shaders/embed_lookup_batched.comp (EmbedLookupBatchedPush {dim, n_pos, scale}) */
vkh_status vkh_embed_lookup(const float *embed, const uint32_t *ids, float *out, uint32_t n_pos,
                            uint32_t dim, float scale, vkh_stream stream);
/* shaders/embedding_backward.comp (EmbeddingBackwardPush {dim, n_pos, vocab}):
 * dE[tok] += sum of dy rows holding tok (position order); other rows untouched.
 * n_pos <= 16384. */
vkh_status vkh_embedding_backward(const float *dy, const uint32_t *ids, float *dE,
                                  uint32_t n_pos, uint32_t dim, uint32_t vocab,
                                  vkh_stream stream);
/* shaders/adam_step.comp (AdamStepPush {n, lr, beta1, beta2, eps, t, wd}) */
vkh_status vkh_adam_step(float *param, const float *grad, float *m, float *v, size_t n, float lr,
                         float beta1, float beta2, float eps, uint32_t t, float weight_decay,
                         vkh_stream stream);
/* shaders/add_in_place.comp, vec_add.comp, scale.comp */
vkh_status vkh_add_in_place(float *dst, const float *src, size_t n, vkh_stream stream);
vkh_status vkh_vec_add(const float *a, const float *b, float *c, size_t n, vkh_stream stream);
vkh_status vkh_scale(const float *in, float *out, size_t n, float scale, vkh_stream stream);
vkh_status vkh_cast_f32_to_bf16(const float *in, void *out, size_t n, vkh_stream stream);

/* ── device memory, streams, events (HIP plumbing for hosts without HIP) ── */
vkh_status vkh_device_count(int *count);
vkh_status vkh_set_device(int device);
vkh_status vkh_malloc(void **ptr, size_t bytes);
vkh_status vkh_free(void *ptr);
vkh_status vkh_memcpy_h2d(void *dst, const void *src, size_t bytes);
vkh_status vkh_memcpy_d2h(void *dst, const void *src, size_t bytes);
vkh_status vkh_memset(void *ptr, int value, size_t bytes);
vkh_status vkh_device_synchronize(void);
vkh_status vkh_stream_create(vkh_stream *out);
vkh_status vkh_stream_destroy(vkh_stream s);
vkh_status vkh_stream_synchronize(vkh_stream s);
vkh_status vkh_event_create(vkh_event *out);
vkh_status vkh_event_destroy(vkh_event e);
vkh_status vkh_event_record(vkh_event e, vkh_stream s);
vkh_status vkh_event_synchronize(vkh_event e);
vkh_status vkh_event_elapsed_ms(vkh_event start, vkh_event stop, float *ms);

const char *vkh_last_error(void);
const char *vkh_status_name(vkh_status s);
/* "gfx950" build info; 0 on success. */
const char *vkh_build_info(void);

#ifdef __cplusplus
}
#endif

#endif /* VKHIP_H */
