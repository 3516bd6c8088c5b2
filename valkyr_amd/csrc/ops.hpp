// Host-side entry points of the HIP kernels (internal to libvkhip; the C ABI
// in include/vkhip.h wraps them).  All pointers are device pointers; every
// function only enqueues on `st` and returns the launch status.
#pragma once

#include "common.hpp"
#include "adam.hpp"

namespace vkh {

enum class DType : int { F32 = 0, BF16 = 1 };
enum class Precision : int { FP32 = 0, BF16 = 1 };

struct Mat {
    const void *p;
    long ld;
    DType dt;
};

inline Mat matf(const float *p, long ld) { return Mat{p, ld, DType::F32}; }

// ── GEMMs (k_gemm.hip) ────────────────────────────────────────────────
// y[M,N] = alpha * x[M,K] W[N,K]^T  (+ R[M,N] residual, optional; + beta*y_old)
hipError_t gemm_nt(Precision pr, Mat x, Mat w, float *y, long ldy, int M, int N, int K,
                   const float *R, long ldr, float alpha, float beta, hipStream_t st);
// dx[M,K] = dy[M,N] W[N,K]  (+ beta*dx_old)
hipError_t gemm_nn(Precision pr, Mat dy, Mat w, float *dx, long lddx, int M, int N, int K,
                   float alpha, float beta, hipStream_t st);
// dW[N,K] = dy[M,N]^T x[M,K]  (+ beta*dW_old)
hipError_t gemm_tn(Precision pr, Mat dy, Mat x, float *dw, long lddw, int M, int N, int K,
                   float alpha, float beta, hipStream_t st);
// ── bf16-operand GEMMs (k_gemm16.hip) ─────────────────────────────────
// Same contractions as gemm_nt / gemm_nn / gemm_tn with every operand bf16
// (fp32 accumulate and output).  `ws` is the split-K workspace (may be
// empty: no split); g16_ws_bytes_for(M, N, K) of the C = [M, N] x K product
// is the size the planner would like for that shape.
struct GemmWs {
    void *p;
    size_t bytes;
};
hipError_t g16_nt(const bf16 *x, long ldx, const bf16 *w, long ldw, float *y, long ldy, int M,
                  int N, int K, const float *R, long ldr, float alpha, float beta,
                  const GemmWs &ws, hipStream_t st);
// The gate/up projection with the SwiGLU forward fused into its epilogue (gu fp32 for
// the backward, gated bf16 for the down projection); hipErrorNotSupported, launching
// nothing, where the [M, 2F] product's plan is not the 8-wave 128 x 128 tile.
// paired: the caller runs another M rows of the same product on a second stream at
// the same time, so the tile is taken wherever the two launches together give it a
// chip-wide round (fused_tile_ok).
hipError_t g16_gate_up_swiglu(const bf16 *x, long ldx, const bf16 *w, long ldw, float *gu,
                              long ldgu, bf16 *gated, long ldg, int M, int F, int K, hipStream_t st,
                              bool paired = false);
hipError_t g16_nn(const bf16 *dy, long lddy, const bf16 *w, long ldw, float *dx, long lddx, int M,
                  int N, int K, float alpha, float beta, const GemmWs &ws, hipStream_t st);
// dx as bf16 (the operand precision of the next kernel), no split-K / fp32 copy.
hipError_t g16_nn_bf16(const bf16 *dy, long lddy, const bf16 *w, long ldw, bf16 *dx, long lddx,
                       int M, int N, int K, const GemmWs &ws, hipStream_t st);
hipError_t g16_tn(const bf16 *dy, long lddy, const bf16 *x, long ldx, float *dw, long lddw, int M,
                  int N, int K, float alpha, float beta, const GemmWs &ws, hipStream_t st);
size_t g16_ws_bytes_for(int M, int N, int K);
// fp32 operands on the same DMA-staged kernels (fp32 matrix cores); operands
// the DMA path cannot take (alignment, ld or extent not a multiple of 4, over
// 2 GiB) go to gemm_nt / gemm_nn / gemm_tn at Precision::FP32.
hipError_t g32_nt(const float *x, long ldx, const float *w, long ldw, float *y, long ldy, int M,
                  int N, int K, const float *R, long ldr, float alpha, float beta,
                  const GemmWs &ws, hipStream_t st);
hipError_t g32_nn(const float *dy, long lddy, const float *w, long ldw, float *dx, long lddx, int M,
                  int N, int K, float alpha, float beta, const GemmWs &ws, hipStream_t st);
hipError_t g32_tn(const float *dy, long lddy, const float *x, long ldx, float *dw, long lddw, int M,
                  int N, int K, float alpha, float beta, const GemmWs &ws, hipStream_t st);
size_t g32_ws_bytes_for(int M, int N, int K);

// ── LoRA rank-r products (k_lora.hip) ───────────────────────────────────
// One adapter of a launch: its columns [col, col + ncols) of the shared X
// (or of Y for the update), its factor F(c, i) = f[c * fsc + i * fsi] (A^T:
// fsc = 1, fsi = K; B: fsc = r, fsi = 1), its [T, r] operand u, and for
// lora_cols the gradient g(c, i) = g[c * gsc + i * gsi].
struct LoraSeg {
    long col = 0;
    int ncols = 0;
    const float *f = nullptr;
    long fsc = 1, fsi = 1;
    float *u = nullptr;
    long ldu = 0;
    float *g = nullptr;
    long gsc = 1, gsi = 1;
};
struct LoraSegs {
    LoraSeg s[3];
    int n = 0;
};
// U_s = alpha X[:, cols_s] F_s            (X fp32 or bf16, [T, ldx])
hipError_t lora_rows(DType xt, const void *x, long ldx, int T, int r, const LoraSegs &g,
                     float alpha, hipStream_t st);
// g_s = alpha X[:, cols_s]^T U_s          (overwrite)
hipError_t lora_cols(DType xt, const void *x, long ldx, int T, int r, const LoraSegs &g,
                     float alpha, hipStream_t st);
// Y[:, cols_s] += alpha U_s F_s^T          (every adapter whose columns hold c)
hipError_t lora_update(float *y, long ldy, int T, int r, const LoraSegs &g, float alpha,
                       hipStream_t st);
bool lora_fast_ok(DType xt, const void *x, long ldx, int r, const LoraSegs &g);
bool lora_update_ok(const float *y, long ldy, int r, const LoraSegs &g);
// The bf16-operand GEMMs with lora_update's term added in their epilogue
// (k_gemm16.hip): the output written once, U_s and F_s as for lora_update
// (alpha the LoRA scale; the base product unscaled).  g16_lora_ok: both
// operands ([arows, arun] and [brows, brun] views) and the adapters fit the
// fused form on an output of n_out columns; the entry points return
// hipErrorInvalidValue where it does not.
bool g16_lora_ok(const bf16 *a, long lda, long arows, long arun, const bf16 *b, long ldb, long brows,
                 long brun, const LoraSegs &g, int r, int n_out);
hipError_t g16_nt_lora(const bf16 *x, long ldx, const bf16 *w, long ldw, float *y, long ldy, int M,
                       int N, int K, const float *R, long ldr, const LoraSegs &g, int r,
                       float alpha, const GemmWs &ws, hipStream_t st);
hipError_t g16_nn_lora(const bf16 *dy, long lddy, const bf16 *w, long ldw, float *dx, long lddx,
                       int M, int N, int K, const LoraSegs &g, int r, float alpha, const GemmWs &ws,
                       hipStream_t st);
hipError_t g16_nn_bf16_lora(const bf16 *dy, long lddy, const bf16 *w, long ldw, bf16 *dx,
                            long lddx, int M, int N, int K, const LoraSegs &g, int r, float alpha,
                            const GemmWs &ws, hipStream_t st);

// One projection group's adapters (train/lora.zig:99-251 for each): up to
// three adapters that read one activation x [T, k] and own column blocks
// [col, col + n) of the group's fused output y / gradient dy.
struct LoraAdapter {
    long col = 0;
    int n = 0, k = 0;
    const float *a = nullptr, *b = nullptr;  // A [r, k], B [n, r]
    float *inter = nullptr;                  // x A^T [T, r]
    float *dyb = nullptr;                    // dy B [T, r]
    float *da = nullptr, *db = nullptr;      // gradients (overwrite)
};
// The segment lists the group's launches take: forward rows (inter = x A^T)
// and update (y += aor inter B^T); backward rows (dyb = dy B), update
// (dx += aor dyb A), dA = aor dyb^T x and dB = aor dy^T inter.
struct LoraGroupSegs {
    LoraSegs fwd_rows, fwd_upd, bwd_rows, bwd_upd, bwd_da, bwd_db;
};
LoraGroupSegs lora_group_segs(const LoraAdapter *ad, int na, int r);

// bf16-output forward GEMM (used for LoRA intermediates and bf16 copies)
hipError_t gemm_nt_bf16out(Mat x, Mat w, bf16 *y, long ldy, int M, int N, int K, float alpha,
                           hipStream_t st);

// ── elementwise / normalisation (k_elementwise.hip, k_norm.hip) ───────
hipError_t fill_f32(float *p, size_t n, float v, hipStream_t st);
hipError_t add_in_place(float *dst, const float *src, size_t n, hipStream_t st);
hipError_t vec_add(const float *a, const float *b, float *c, size_t n, hipStream_t st);
hipError_t scale(const float *in, float *out, size_t n, float s, hipStream_t st);
hipError_t cast_f32_to_bf16(const float *in, bf16 *out, size_t n, hipStream_t st);
// SwiGLU outputs are fp32 or bf16 (the GEMM-operand copy) per `gdt` / `odt`.
hipError_t swiglu_forward(const float *pg, long ldpg, const float *up, long ldup, void *g,
                          long ldg, DType gdt, int rows, int cols, hipStream_t st);
hipError_t swiglu_backward(const float *dg, long lddg, const float *pg, long ldpg,
                           const float *up, long ldup, void *dpg, long lddpg, void *dup,
                           long lddup, DType odt, int rows, int cols, hipStream_t st);
hipError_t embed_lookup(const float *embed, const uint32_t *ids, float *out, int n_pos, int dim,
                        float scale, hipStream_t st);
// the lookup from a bf16 table (dim % 4 == 0), widened to fp32
hipError_t embed_lookup_bf16(const bf16 *embed, const uint32_t *ids, float *out, int n_pos,
                             int dim, float scale, hipStream_t st);
// Adam (adam_step.comp): bc1 = 1 - beta1^t, bc2 = 1 - beta2^t computed by the caller.
// pb (optional) receives bf16(p) after the update.
hipError_t adam_step(float *p, const float *g, float *m, float *v, size_t n, float lr,
                     float beta1, float beta2, float eps, float bc1, float bc2, float wd,
                     bf16 *pb, hipStream_t st);
// Up to kAdamMaxGains norm gains inside an Adam span whose gradients are still
// RMSNorm-backward partial sums: gradient = column sums of partial[nparts][stride]
// (the column-sum kernel's order), stored into g, then the update.  Gains must
// cover whole float4 vectors (offsets and lengths multiples of 4).
constexpr int kAdamMaxGains = 4;
struct AdamGain {
    size_t off;           // element offset from the span start
    unsigned dim;
    const float *partial;
    int nparts;
    long stride;
};
struct AdamGains {
    AdamGain g[kAdamMaxGains];
    int n;
};
// max_blocks (0: one block per chunk): at most that many blocks walk the span's
// chunks, lowering the update's instantaneous share of HBM beside other work.
hipError_t adam_step_gains(float *p, float *g, float *m, float *v, size_t n, float lr, float beta1,
                           float beta2, float eps, float bc1, float bc2, float wd, bf16 *pb,
                           const AdamGains &gs, hipStream_t st, unsigned max_blocks = 0);

// y (fp32 or bf16 per ydt) = rmsnorm(x) * w
hipError_t rmsnorm_forward(const float *x, const float *w, void *y, DType ydt, int rows, int dim,
                           float eps, int gemma_quirk, hipStream_t st);
// dx = rmsnorm_bw(dy) (+ residual add), dxb (optional) = bf16(dx), dw (reduced
// over rows, overwrite); `partial` must hold rmsnorm_partial_floats(rows, dim) floats.
hipError_t rmsnorm_backward(const float *dy, const float *x, const float *w, float *dx,
                            bf16 *dxb, const float *residual, float *dw, float *partial, int rows,
                            int dim, float eps, int gemma_quirk, hipStream_t st);
size_t rmsnorm_partial_floats(int rows, int dim);
// Rows of per-block partial sums rmsnorm_backward writes for `rows` rows.
int rmsnorm_partial_rows(int rows);
// out[c] = sum over b < nparts of partial[b * stride + c], c < dim, summed in a
// fixed order (the gain-gradient reduction of the norm backwards; callers
// that pass dw = nullptr there run it themselves, e.g. on another stream).
hipError_t column_sums(const float *partial, int nparts, long stride, int dim, float *out,
                       hipStream_t st);

// RoPE cos/sin table [seq_len][rotary_dim/2] as float2, built on the host
// with the fp32 formula of qk_rope_partial_batched.comp:76-81.
void rope_table_host(float2 *tab, int seq_len, int rotary_dim, float theta);
// qk_rope_partial_batched.comp / qk_rope_backward_batched.comp (position of
// row r = r % seq_len).
hipError_t qk_rope(const float *q_in, long ldq_in, float *q_out, long ldq_out, const float *k_in,
                   long ldk_in, float *k_out, long ldk_out, int n_rows, int n_q_heads,
                   int n_kv_heads, int head_dim, int rotary_dim, int seq_len, const float2 *tab,
                   bool backward, hipStream_t st);

// Fused per-head Q/K RMSNorm + RoPE forward, emitting the attention
// operands (fp32 or bf16) for q, k and (copy/cast of) v.
struct QkvLayout {
    int n_rows, n_q_heads, n_kv_heads, head_dim;
    int seq_len, rotary_dim;
    float theta, eps;
    int qk_norm;
};
hipError_t qkv_prepare_forward(const QkvLayout &L, const float *qkv, long ld_qkv,
                               const float *wq, const float *wk, void *out, long ld_out,
                               DType out_dt, const float2 *rope_tab, hipStream_t st);
// The q|k|v projection y = x w^T (bf16 operands, fp32 y) with qkv_prepare_forward's
// bf16 output fused into the GEMM's epilogue (the same values bit for bit);
// hipErrorNotSupported, launching nothing, unless head_dim is 128 and the product's
// plan is the 8-wave 128 x 128 tile (paired: as for g16_gate_up_swiglu).
hipError_t g16_qkv_norm_rope(const bf16 *x, long ldx, const bf16 *w, long ldw, float *y, long ldy,
                             int M, int N, int K, const QkvLayout &L, const float *wq,
                             const float *wk, bf16 *out, long ld_out, const float2 *tab,
                             hipStream_t st, bool paired = false);
// fp32 forms (fp32 operands and outputs), where the fp32 plan is the 8-wave 128 x 128 tile.
hipError_t g32_qkv_norm_rope(const float *x, long ldx, const float *w, long ldw, float *y, long ldy,
                             int M, int N, int K, const QkvLayout &L, const float *wq,
                             const float *wk, float *out, long ld_out, const float2 *tab,
                             hipStream_t st);
hipError_t g32_gate_up_swiglu(const float *x, long ldx, const float *w, long ldw, float *gu,
                              long ldgu, float *gated, long ldg, int M, int F, int K, hipStream_t st);
// Backward of the above on the fused d_qkv buffer: d(post-rope) ->
// d(pre-norm) for the q/k columns, in place, or (outb non-null) written with
// the v columns to the bf16 copy outb; dwq/dwk reduced gains (overwrite).
// nparts (optional) receives the number of partial rows written (q gains in
// columns [0, hd), k gains in [hd, 2 hd), row stride 2 hd).
hipError_t qkv_prepare_backward(const QkvLayout &L, float *dqkv, long ld, const float *qkv,
                                long ld_qkv, const float *wq, const float *wk, float *dwq,
                                float *dwk, float *partial, const float2 *rope_tab,
                                bf16 *outb, long ldb, hipStream_t st, int *nparts = nullptr);
size_t qkv_partial_floats(const QkvLayout &L);

// ── embedding backward (k_embed.hip) ─────────────────────────────────
// out[tok] = (accumulate ? out[tok] : 0) + sum over positions p with
// ids[p] == tok of dy[p] (position order).  Rows of untouched tokens are not
// written.  `work` is not used (embed_bw_work_bytes is a 16-byte placeholder,
// kept so callers that pass a buffer stay valid).
hipError_t embedding_backward(const float *dy, const uint32_t *ids, float *out, int n_pos,
                              int dim, int vocab, bool accumulate, void *work, hipStream_t st);
size_t embed_bw_work_bytes(int n_pos);
// The same scatter, and then the Adam update of every row it wrote (dim % 4
// == 0, 16-byte aligned rows): for a step whose table gradient is complete
// once the scatter is (the head's weight gradient came first).
struct EmbedAdam {
    float *p, *m, *v;
    bf16 *pb;  // optional bf16 copy of the updated rows
    AdamHyper h;
};
hipError_t embedding_backward_adam(const float *dy, const uint32_t *ids, float *out, int n_pos,
                                   int dim, int vocab, bool accumulate, const EmbedAdam &ea,
                                   hipStream_t st);
// Adam over the rows of a [rows, dim] table (dim % 4 == 0, 16-byte aligned)
// whose mark differs from `stamp`; mark_rows stamps the rows named by ids.
hipError_t adam_rows_unmarked(float *p, const float *g, float *m, float *v, bf16 *pb, int rows,
                              int dim, const uint32_t *mark, uint32_t stamp, const AdamHyper &h,
                              hipStream_t st);
hipError_t mark_rows(const uint32_t *ids, int n, uint32_t *mark, int rows, uint32_t stamp,
                     hipStream_t st);
constexpr int kEmbedBwMaxPos = 16384;

// ── attention (k_attn.hip) ───────────────────────────────────────────
struct AttnShape {
    int n_batch, n_q, n_kv, n_heads, n_kv_heads, head_dim;
    int causal;
    float inv_sqrt_dim;
};
// Fused q/k gradient epilogue of the recompute attention backward: dQ, dK
// and dV leave the kernels as bf16 rows of one [T, (H + 2 Hkv) hd] matrix
// (q heads, then k, then v), dQ and dK already taken back through RoPE and
// the Q/K-RMSNorm (the gradient w.r.t. the pre-norm projection output), with
// the norm-gain gradient as one head_dim row of partial sums per block.
struct QkEpi {
    bf16 *out = nullptr;                      // set: the epilogue runs
    long ldout = 0;
    const float *x = nullptr;                 // pre-norm q / k rows (same column layout)
    long ldx = 0;
    const float *gq = nullptr, *gk = nullptr; // norm gains (null: no Q/K-RMSNorm)
    float eps = 0.f;
    const float2 *rope = nullptr;             // [n_pos][head_dim / 2] (cos, sin)
    int rot = 0;                              // rotary_dim: 0 or head_dim
    float *pq = nullptr, *pk = nullptr;       // gain partials [blocks][head_dim]
};

struct AttnPtrs {
    const void *q; long ldq;   // [T, n_heads*hd] rows, elements of dtype dt
    const void *k; long ldk;
    const void *v; long ldv;
    const float *o; long ldo;  // fp32 forward output (for D)
    const void *dout; long lddo; // upstream gradient (dtype dt)
    const float *lse;          // [T, n_heads]
    float *d;                  // [T, n_heads]
    float *dq; long lddq;
    float *dk; long lddk;
    float *dv; long lddv;
    DType dt;
    // bf16 O: when set on the recompute path, the dQ kernel forms
    // D = rowsum(O dO) for its rows itself (written to d) and runs first
    const void *o16 = nullptr; long ldo16 = 0;
    QkEpi qk;  // recompute path, and the fp32 tile kernels with qk_fp32
    // fp32 tile kernels: dQ / dK leave through p.qk's RoPE^T and Q/K-norm
    // backward (fa_f32m_qk_ok must hold; fa_bw_dq / fa_bw_dkv fail otherwise)
    bool qk_fp32 = false;
    // recompute path: workspace of fa_bw_v4_split_ws_floats(s) floats; when set
    // on a shape fa_bw_v4_split accepts, the dK / dV launch is split in two
    float *split_ws = nullptr;
};
// fp32 attention on the matrix cores (k_attn_f32.hip) for the shapes
// fa_f32m_ok accepts; each launcher returns false, launching nothing, for a
// shape or alignment it does not take (the caller then uses the per-row
// kernels).
bool fa_f32m_ok(const AttnShape &s);
bool fa_f32m_fwd(const AttnShape &s, const float *q, long ldq, const float *k, long ldk,
                 const float *v, long ldv, float *o, long ldo, float *lse, hipStream_t st);
bool fa_f32m_dkv(const AttnShape &s, const AttnPtrs &p, hipStream_t st);
bool fa_f32m_dq(const AttnShape &s, const AttnPtrs &p, hipStream_t st);
bool fa_f32m_qk_ok(const AttnShape &s, const AttnPtrs &p);
// blocks of the fp32 dQ and dK/dV grids: the fused epilogue's gain partials
int fa_f32m_dq_blocks(const AttnShape &s);
int fa_f32m_dkv_blocks(const AttnShape &s);
// ob (optional, bf16 operands only): bf16 copy of O for the output projection.
hipError_t fa_forward(const AttnShape &s, const void *q, long ldq, const void *k, long ldk,
                      const void *v, long ldv, float *o, long ldo, float *lse, DType dt,
                      bf16 *ob, long ldob, hipStream_t st);
// D = rowsum(O * dO); optionally also writes dO as bf16 (dout_bf16, ld lddo16)
hipError_t fa_bw_d(const AttnShape &s, const float *o, long ldo, const float *dout, long lddo,
                   float *d, bf16 *dout_bf16, long lddo16, hipStream_t st);
// D = rowsum(O * dO) from bf16 O and dO (head_dim 64 / 128, 16-byte aligned).
hipError_t fa_bw_d_bf16(const AttnShape &s, const bf16 *o, long ldo, const bf16 *dout, long lddo,
                        float *d, hipStream_t st);
hipError_t fa_bw_dq(const AttnShape &s, const AttnPtrs &p, hipStream_t st);
hipError_t fa_bw_dkv(const AttnShape &s, const AttnPtrs &p, hipStream_t st);
// Fused bf16 backward.  Requires fa_bw_fused_ok(s) (bf16 head_dim 64/128, n_q
// and n_kv multiples of 64, self-attention when causal).  v4 (requires
// fa_bw_v4_ok: head_dim 128, even GQA group, n_kv % 128 == 0): dK/dV and dQ
// kernels that each recompute S and dP, no workspace.  Otherwise dK/dV writes
// bf16 dS into ds_ws (fa_bw_ws_bytes) and dQ = dS K is a GEMM.
// fa_bw_v4_preferred: the shapes on which v4 is the faster of the two.
bool fa_bw_fused_ok(const AttnShape &s);
bool fa_bw_v4_ok(const AttnShape &s);
bool fa_bw_v4_preferred(const AttnShape &s);
// Gain-partial rows the fused q/k epilogue writes (dQ kernel: q gains; dK/dV
// kernel: k gains), and whether a shape / rotary_dim can take it.
hipError_t fa_bw_v4_part(const AttnShape &s, const AttnPtrs &p, int which, hipStream_t st);
int fa_bw_v4_q_blocks(const AttnShape &s);
int fa_bw_v4_q_rows(const AttnShape &s);  // query rows per dQ block
bool fa_bw_v4_split(const AttnShape &s);
size_t fa_bw_v4_split_ws_floats(const AttnShape &s);
// dK/dV blocks launched, and K-gain partial rows written, with or without the split
int fa_bw_v4_kv_launch_blocks(const AttnShape &s, bool split);
int fa_bw_v4_k_gain_parts(const AttnShape &s, bool split);
int fa_bw_v4_kv_blocks(const AttnShape &s);
bool fa_bw_qk_epi_ok(const AttnShape &s, int rotary_dim);
size_t fa_bw_ws_bytes(const AttnShape &s, bool v4);
hipError_t fa_bw_fused(const AttnShape &s, const AttnPtrs &p, bf16 *ds_ws, bool v4, hipStream_t st);

// ── cut cross-entropy (k_cce.hip) ────────────────────────────────────
struct CceShape {
    int N, V, D;
    float z_loss_scale, label_smoothing;
};
size_t cce_work_floats(const CceShape &s);
// z_out (optional): the fp32 logits [N, V] are stored there too, for
// cce_backward's z.
hipError_t cce_forward(Precision pr, const CceShape &s, const float *h, const float *w,
                       const uint32_t *tgt, float *lse, float *loss_row, float *loss_mean,
                       float *work, hipStream_t st, float *z_out = nullptr);
// bf16-operand forms (h, W bf16; dz bf16), on the gemm16 kernel.
hipError_t cce_forward16(const CceShape &s, const bf16 *h, const bf16 *w, const uint32_t *tgt,
                         float *lse, float *loss_row, float *loss_mean, float *work,
                         hipStream_t st, float *z_out = nullptr);
hipError_t cce_backward16(const CceShape &s, const bf16 *h, const bf16 *w, const uint32_t *tgt,
                          const float *lse, bf16 *dz, float *dh, float *dw, float dw_beta,
                          const GemmWs &ws, hipStream_t st, const float *z = nullptr);
// dz (bf16 for Precision::BF16 else fp32) [N, V] is materialised in `dz`;
// dh overwritten (if non-null); dW = beta*dW + dz^T h (if non-null).  z: the
// logits cce_forward stored with z_out (may be dz itself), read instead of
// recomputing them; nullptr recomputes.
hipError_t cce_backward(Precision pr, const CceShape &s, const float *h, const float *w,
                        const uint32_t *tgt, const float *lse, void *dz, float *dh, float *dw,
                        float dw_beta, hipStream_t st, const float *z = nullptr);

}  // namespace vkh
