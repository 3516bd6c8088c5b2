/*
 * CPU oracle for the valkyr transformer-training hot path — TEST
 * INFRASTRUCTURE ONLY (see oracle.h).  Built with -ffp-contract=off so every
 * fp32 operation rounds exactly where the reference's Zig does.
 */
#define _POSIX_C_SOURCE 199309L
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define NEG_INF (-INFINITY)

/* ── threads ───────────────────────────────────────────────────────────────
 * Parallel loops run only over outputs that are independent of each other,
 * and every accumulation keeps the sequential loop's order, so any thread
 * count gives bit-identical results. */

void orc_set_threads(int n) {
#ifdef _OPENMP
    omp_set_num_threads(n > 0 ? n : 1);
#else
    (void)n;
#endif
}

int orc_get_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ── generator ─────────────────────────────────────────────────────────── */

uint64_t orc_splitmix64(uint64_t *state) {
    uint64_t z = (*state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static double u01(uint64_t *s) { /* (0, 1) exclusive of 0 */
    return ((double)(orc_splitmix64(s) >> 11) + 0.5) * (1.0 / 9007199254740992.0);
}

/* The j-th draw (0-based) of a SplitMix64 stream started at `seed` is the
 * mix of seed + (j + 1) * gamma, so the Box-Muller pairs can be formed in
 * any order: the values are those of the sequential stream. */
void orc_fill_normal(float *x, size_t n, uint64_t seed, float mean, float stddev) {
    const long long npairs = (long long)((n + 1) / 2);
#pragma omp parallel for schedule(static)
    for (long long p = 0; p < npairs; ++p) {
        const size_t i = 2 * (size_t)p;
        uint64_t s = seed + 0x9E3779B97F4A7C15ull * (uint64_t)i;
        double u1 = u01(&s), u2 = u01(&s);
        double r = sqrt(-2.0 * log(u1));
        double a = 6.283185307179586 * u2;
        x[i] = (float)(mean + stddev * r * cos(a));
        if (i + 1 < n) x[i + 1] = (float)(mean + stddev * r * sin(a));
    }
}

void orc_fill_uniform(float *x, size_t n, uint64_t seed, float lo, float hi) {
    uint64_t s = seed;
    for (size_t i = 0; i < n; ++i) x[i] = (float)(lo + (hi - lo) * u01(&s));
}

void orc_fill_ids(uint32_t *x, size_t n, uint64_t seed, uint32_t hi) {
    uint64_t s = seed;
    for (size_t i = 0; i < n; ++i) x[i] = (uint32_t)(orc_splitmix64(&s) % hi);
}

/* ── bf16 ───────────────────────────────────────────────────────────────── */

uint16_t orc_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40); /* quiet NaN */
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;
    return (uint16_t)(u >> 16);
}

float orc_bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

void orc_round_bf16(float *x, size_t n) {
    for (size_t i = 0; i < n; ++i) x[i] = orc_bf16_to_f32(orc_f32_to_bf16(x[i]));
}

void orc_to_bf16(const float *x, uint16_t *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_f32_to_bf16(x[i]);
}

/* ── RMSNorm: src/cpu/train_transformer.zig:41-164 ─────────────────────── */

float orc_rmsnorm_forward_row(const float *x, const float *w, size_t dim, float eps,
                              int gemma_quirk, float *y) {
    double s = 0;
    for (size_t i = 0; i < dim; ++i) s += (double)x[i] * (double)x[i];
    double m = s / (double)dim;
    float ri = 1.0f / sqrtf((float)m + eps);
    for (size_t i = 0; i < dim; ++i) {
        float gain = gemma_quirk ? w[i] + 1.0f : w[i];
        y[i] = gain * ri * x[i];
    }
    return ri;
}

void orc_rmsnorm_forward(const float *x, const float *w, size_t n_rows, size_t dim,
                         float eps, int gemma_quirk, float *y) {
    for (size_t r = 0; r < n_rows; ++r)
        orc_rmsnorm_forward_row(x + r * dim, w, dim, eps, gemma_quirk, y + r * dim);
}

/* train_transformer.zig:68-111 (row) and :137-164 (rows; dw accumulates
 * across rows in row order, fp32). */
void orc_rmsnorm_backward(const float *dy, const float *x, const float *w, size_t n_rows,
                          size_t dim, float eps, int gemma_quirk, float *dx,
                          float *dw_accum) {
    for (size_t r = 0; r < n_rows; ++r) {
        const float *dyr = dy + r * dim, *xr = x + r * dim;
        float *dxr = dx + r * dim;
        double s = 0;
        for (size_t i = 0; i < dim; ++i) s += (double)xr[i] * (double)xr[i];
        double m = s / (double)dim;
        float ri = 1.0f / sqrtf((float)m + eps);
        double A = 0;
        for (size_t i = 0; i < dim; ++i) {
            float gain = gemma_quirk ? w[i] + 1.0f : w[i];
            A += (double)dyr[i] * (double)gain * (double)xr[i];
        }
        float ri3_over_D = ri * ri * ri / (float)dim;
        float A_f32 = (float)A;
        for (size_t i = 0; i < dim; ++i) {
            float gain = gemma_quirk ? w[i] + 1.0f : w[i];
            dxr[i] = ri * gain * dyr[i] - ri3_over_D * xr[i] * A_f32;
            if (dw_accum) dw_accum[i] += dyr[i] * ri * xr[i];
        }
    }
}

/* ── embedding: train_decoder.zig:713-718 (lookup), train_transformer.zig:351-366 */

void orc_embedding_forward(const float *embed, const uint32_t *ids, size_t n_pos,
                           size_t dim, float *out) {
    for (size_t p = 0; p < n_pos; ++p)
        memcpy(out + p * dim, embed + (size_t)ids[p] * dim, dim * sizeof(float));
}

void orc_embedding_backward(const float *dy, const uint32_t *ids, size_t n_pos,
                            size_t vocab, size_t dim, float *dE) {
    (void)vocab;
    for (size_t p = 0; p < n_pos; ++p) {
        const float *src = dy + p * dim;
        float *dst = dE + (size_t)ids[p] * dim;
        for (size_t i = 0; i < dim; ++i) dst[i] += src[i];
    }
}

/* ── RoPE: train_transformer.zig:489-563.  Batch extension: the position of
 * row r is r % seq_len (seq_len = n_rows reproduces the reference). ───── */

static int rope_apply(float *out, const float *in, size_t n_rows, size_t n_heads,
                      size_t head_dim, size_t rotary_dim, float theta, size_t seq_len,
                      int backward) {
    if (rotary_dim > head_dim) return -1;
    if (rotary_dim % 2 != 0) return -2;
    if (seq_len == 0) seq_len = n_rows;
    size_t half = rotary_dim / 2;
    float rdim_f = (float)rotary_dim;
    size_t row_stride = n_heads * head_dim;
    for (size_t p = 0; p < n_rows; ++p) {
        float pos_f = (float)(p % seq_len);
        for (size_t h = 0; h < n_heads; ++h) {
            size_t off = p * row_stride + h * head_dim;
            for (size_t j = 0; j < half; ++j) {
                float freq = 1.0f / powf(theta, (2.0f * (float)j) / rdim_f);
                float angle = pos_f * freq;
                float c = cosf(angle), s = sinf(angle);
                float a = in[off + j], b = in[off + j + half];
                if (!backward) {
                    out[off + j] = a * c - b * s;
                    out[off + j + half] = a * s + b * c;
                } else {
                    out[off + j] = c * a + s * b;
                    out[off + j + half] = -s * a + c * b;
                }
            }
            for (size_t i = rotary_dim; i < head_dim; ++i) out[off + i] = in[off + i];
        }
    }
    return 0;
}

int orc_rope_forward_batched(float *out, const float *in, size_t n_rows, size_t n_heads,
                             size_t head_dim, size_t rotary_dim, float theta,
                             size_t seq_len) {
    return rope_apply(out, in, n_rows, n_heads, head_dim, rotary_dim, theta, seq_len, 0);
}

int orc_rope_backward_batched(float *d_in, const float *d_out, size_t n_rows,
                              size_t n_heads, size_t head_dim, size_t rotary_dim,
                              float theta, size_t seq_len) {
    return rope_apply(d_in, d_out, n_rows, n_heads, head_dim, rotary_dim, theta, seq_len, 1);
}

/* ── 3-pass attention: train_transformer.zig:614-796 ───────────────────── */

void orc_attention_forward(const float *Q, const float *K, const float *V, size_t n_q,
                           size_t n_kv, size_t n_heads, size_t n_kv_heads, size_t head_dim,
                           int causal, float *scores, float *attn, float *out) {
    size_t hpk = n_heads / n_kv_heads;
    float inv_sqrt_d = 1.0f / sqrtf((float)head_dim);
    for (size_t q = 0; q < n_q; ++q) {
        size_t k_limit = causal ? q + (n_kv - n_q) : n_kv - 1;
        for (size_t h = 0; h < n_heads; ++h) {
            size_t kv_h = h / hpk;
            size_t q_off = q * n_heads * head_dim + h * head_dim;
            size_t s_row = q * n_heads * n_kv + h * n_kv;
            for (size_t k = 0; k < n_kv; ++k) {
                if (causal && k > k_limit) { scores[s_row + k] = NEG_INF; continue; }
                size_t k_off = k * n_kv_heads * head_dim + kv_h * head_dim;
                double s = 0;
                for (size_t d = 0; d < head_dim; ++d) s += (double)Q[q_off + d] * (double)K[k_off + d];
                scores[s_row + k] = (float)s * inv_sqrt_d;
            }
            float max_s = NEG_INF;
            for (size_t k = 0; k < n_kv; ++k) if (scores[s_row + k] > max_s) max_s = scores[s_row + k];
            double sum = 0;
            for (size_t k = 0; k < n_kv; ++k) {
                float v = scores[s_row + k];
                float e = (isinf(v) && v < 0) ? 0.0f : expf(v - max_s);
                attn[s_row + k] = e;
                sum += e;
            }
            float inv_sum = sum > 0 ? 1.0f / (float)sum : 0.0f;
            for (size_t k = 0; k < n_kv; ++k) attn[s_row + k] *= inv_sum;
            size_t o_off = q_off;
            for (size_t d = 0; d < head_dim; ++d) out[o_off + d] = 0.0f;
            for (size_t k = 0; k < n_kv; ++k) {
                size_t v_off = k * n_kv_heads * head_dim + kv_h * head_dim;
                float w = attn[s_row + k];
                if (w == 0.0f) continue;
                for (size_t d = 0; d < head_dim; ++d) out[o_off + d] += w * V[v_off + d];
            }
        }
    }
}

/* train_transformer.zig:385-396 softmaxBackwardRow (fp64 reduction) */
static void softmax_backward_row(const float *dy, const float *y, size_t n, float *dx) {
    double S = 0;
    for (size_t i = 0; i < n; ++i) S += (double)dy[i] * (double)y[i];
    float S_f = (float)S;
    for (size_t i = 0; i < n; ++i) dx[i] = y[i] * (dy[i] - S_f);
}

void orc_attention_backward(const float *d_out, const float *Q, const float *K,
                            const float *V, const float *attn, size_t n_q, size_t n_kv,
                            size_t n_heads, size_t n_kv_heads, size_t head_dim,
                            float *d_scores, float *dQ, float *dK, float *dV) {
    size_t hpk = n_heads / n_kv_heads;
    float inv_sqrt_d = 1.0f / sqrtf((float)head_dim);
    memset(dQ, 0, n_q * n_heads * head_dim * sizeof(float));
    memset(dK, 0, n_kv * n_kv_heads * head_dim * sizeof(float));
    memset(dV, 0, n_kv * n_kv_heads * head_dim * sizeof(float));
    for (size_t q = 0; q < n_q; ++q)
        for (size_t h = 0; h < n_heads; ++h) {
            size_t kv_h = h / hpk;
            size_t dout_off = q * n_heads * head_dim + h * head_dim;
            size_t a_row = q * n_heads * n_kv + h * n_kv;
            for (size_t k = 0; k < n_kv; ++k) {
                size_t v_off = k * n_kv_heads * head_dim + kv_h * head_dim;
                float a = attn[a_row + k];
                if (a != 0.0f)
                    for (size_t d = 0; d < head_dim; ++d) dV[v_off + d] += a * d_out[dout_off + d];
                double dot = 0;
                for (size_t d = 0; d < head_dim; ++d) dot += (double)d_out[dout_off + d] * (double)V[v_off + d];
                d_scores[a_row + k] = (float)dot;
            }
        }
    for (size_t r = 0; r < n_q * n_heads; ++r)
        softmax_backward_row(d_scores + r * n_kv, attn + r * n_kv, n_kv, d_scores + r * n_kv);
    for (size_t q = 0; q < n_q; ++q)
        for (size_t h = 0; h < n_heads; ++h) {
            size_t kv_h = h / hpk;
            size_t q_off = q * n_heads * head_dim + h * head_dim;
            size_t ds_row = q * n_heads * n_kv + h * n_kv;
            for (size_t k = 0; k < n_kv; ++k) {
                size_t k_off = k * n_kv_heads * head_dim + kv_h * head_dim;
                float ds = d_scores[ds_row + k];
                if (ds == 0.0f) continue;
                float dss = ds * inv_sqrt_d;
                for (size_t d = 0; d < head_dim; ++d) {
                    dQ[q_off + d] += dss * K[k_off + d];
                    dK[k_off + d] += dss * Q[q_off + d];
                }
            }
        }
}

/* ── SwiGLU: train_transformer.zig:832-875 ─────────────────────────────── */

static float sigmoidf_(float z) { return 1.0f / (1.0f + expf(-z)); }

void orc_swiglu_forward(const float *pre_gate, const float *up, size_t n, float *gated) {
    for (size_t i = 0; i < n; ++i) {
        float z = pre_gate[i];
        float sig = sigmoidf_(z);
        float silu_z = z * sig;
        gated[i] = silu_z * up[i];
    }
}

void orc_swiglu_backward(const float *d_gated, const float *pre_gate, const float *up,
                         size_t n, float *d_pre_gate, float *d_up) {
    for (size_t i = 0; i < n; ++i) {
        float z = pre_gate[i], u = up[i], dg = d_gated[i];
        float sig = sigmoidf_(z);
        float silu_z = z * sig;
        float silu_grad = sig + silu_z * (1.0f - sig);
        d_up[i] = dg * silu_z;
        d_pre_gate[i] = dg * u * silu_grad;
    }
}

/* ── FlashAttention: src/cpu/flash_attn.zig:91-376 ─────────────────────── */

static float bf16r(float x) { return orc_bf16_to_f32(orc_f32_to_bf16(x)); }

/* bf16_ops: the bf16-operand model of the MFMA kernels.  Every product's
 * operands are bf16, including the probabilities: P is formed in fp32 (l sums
 * the fp32 values) and rounded to bf16 where it multiplies V. */
static void flash_forward(const float *Q, const float *K, const float *V, size_t n_q,
                          size_t n_kv, size_t n_heads, size_t n_kv_heads, size_t head_dim,
                          int causal, size_t Br, size_t Bc, int bf16_ops, float *out,
                          float *lse) {
    size_t hpk = n_heads / n_kv_heads;
    float inv_sqrt_d = 1.0f / sqrtf((float)head_dim);
    /* every (query block, head) is independent: parallel over them */
    const long long n_qb = (long long)((n_q + Br - 1) / Br), n_work = n_qb * (long long)n_heads;
#pragma omp parallel
    {
    float *s_tile = malloc(Br * Bc * sizeof(float));
    float *p_tile = malloc(Br * Bc * sizeof(float));
    float *o_acc = malloc(Br * head_dim * sizeof(float));
    float *m_acc = malloc(Br * sizeof(float));
    float *l_acc = malloc(Br * sizeof(float));
#pragma omp for schedule(dynamic, 1)
    for (long long wi = 0; wi < n_work; ++wi) {
        const size_t qb = (size_t)(wi / (long long)n_heads) * Br, h = (size_t)(wi % (long long)n_heads);
        size_t qe = qb + Br < n_q ? qb + Br : n_q, qlen = qe - qb;
        {
            size_t kv_h = h / hpk;
            for (size_t qi = 0; qi < qlen; ++qi) { m_acc[qi] = NEG_INF; l_acc[qi] = 0.0f; }
            for (size_t i = 0; i < qlen * head_dim; ++i) o_acc[i] = 0.0f;
            for (size_t kb = 0; kb < n_kv; kb += Bc) {
                size_t ke = kb + Bc < n_kv ? kb + Bc : n_kv, klen = ke - kb;
                for (size_t qi = 0; qi < qlen; ++qi) {
                    size_t q = qb + qi;
                    size_t k_limit = causal ? q + (n_kv - n_q) : n_kv - 1;
                    size_t q_off = q * n_heads * head_dim + h * head_dim;
                    for (size_t ki = 0; ki < klen; ++ki) {
                        size_t k = kb + ki;
                        if (causal && k > k_limit) { s_tile[qi * Bc + ki] = NEG_INF; continue; }
                        size_t k_off = k * n_kv_heads * head_dim + kv_h * head_dim;
                        double s = 0;
                        for (size_t d = 0; d < head_dim; ++d) s += (double)Q[q_off + d] * (double)K[k_off + d];
                        s_tile[qi * Bc + ki] = (float)s * inv_sqrt_d;
                    }
                }
                for (size_t qi = 0; qi < qlen; ++qi) {
                    float m_tile = NEG_INF;
                    for (size_t ki = 0; ki < klen; ++ki)
                        if (s_tile[qi * Bc + ki] > m_tile) m_tile = s_tile[qi * Bc + ki];
                    float m_old = m_acc[qi];
                    float m_new = m_tile > m_old ? m_tile : m_old;
                    double l_tile = 0;
                    for (size_t ki = 0; ki < klen; ++ki) {
                        float s = s_tile[qi * Bc + ki];
                        float p = (s == NEG_INF) ? 0.0f : expf(s - m_new);
                        p_tile[qi * Bc + ki] = p;
                        l_tile += p;
                    }
                    float scale_old = (m_old == NEG_INF) ? 0.0f : expf(m_old - m_new);
                    for (size_t d = 0; d < head_dim; ++d) o_acc[qi * head_dim + d] *= scale_old;
                    for (size_t ki = 0; ki < klen; ++ki) {
                        float p = p_tile[qi * Bc + ki];
                        if (p == 0.0f) continue;
                        if (bf16_ops) p = bf16r(p);
                        size_t v_off = (kb + ki) * n_kv_heads * head_dim + kv_h * head_dim;
                        for (size_t d = 0; d < head_dim; ++d) o_acc[qi * head_dim + d] += p * V[v_off + d];
                    }
                    m_acc[qi] = m_new;
                    l_acc[qi] = scale_old * l_acc[qi] + (float)l_tile;
                }
            }
            for (size_t qi = 0; qi < qlen; ++qi) {
                size_t q = qb + qi;
                float inv_l = l_acc[qi] > 0 ? 1.0f / l_acc[qi] : 0.0f;
                size_t o_off = q * n_heads * head_dim + h * head_dim;
                for (size_t d = 0; d < head_dim; ++d) out[o_off + d] = o_acc[qi * head_dim + d] * inv_l;
                if (lse) lse[q * n_heads + h] = l_acc[qi] > 0 ? m_acc[qi] + logf(l_acc[qi]) : NEG_INF;
            }
        }
    }
    free(s_tile); free(p_tile); free(o_acc); free(m_acc); free(l_acc);
    }
}

void orc_flash_attention_forward(const float *Q, const float *K, const float *V,
                                 size_t n_q, size_t n_kv, size_t n_heads,
                                 size_t n_kv_heads, size_t head_dim, int causal,
                                 size_t Br, size_t Bc, float *out, float *lse) {
    flash_forward(Q, K, V, n_q, n_kv, n_heads, n_kv_heads, head_dim, causal, Br, Bc, 0, out, lse);
}

/* bf16_ops: P rounds to bf16 where it multiplies dO (dV), and the unscaled
 * dS = P (dP - D) rounds to bf16 where it multiplies Q and K (dK, dQ); the
 * 1/sqrt(d) scale is applied to the accumulated dQ and dK, which is where the
 * MFMA kernels apply it. */
static void flash_backward(const float *Q, const float *K, const float *V, const float *O,
                           const float *dO, const float *lse, size_t n_q, size_t n_kv,
                           size_t n_heads, size_t n_kv_heads, size_t head_dim, int causal,
                           int bf16_ops, float *dQ, float *dK, float *dV) {
    size_t hpk = n_heads / n_kv_heads;
    float inv_sqrt_d = 1.0f / sqrtf((float)head_dim);
    memset(dQ, 0, n_q * n_heads * head_dim * sizeof(float));
    memset(dK, 0, n_kv * n_kv_heads * head_dim * sizeof(float));
    memset(dV, 0, n_kv * n_kv_heads * head_dim * sizeof(float));
    /* The KV heads are independent.  Within one, dK / dV rows take their
     * terms in the sequential loop's order (q ascending, then the group's
     * heads ascending), and dQ[q, h] its terms k ascending. */
#pragma omp parallel for schedule(static, 1)
    for (size_t kv_h = 0; kv_h < n_kv_heads; ++kv_h)
    for (size_t q = 0; q < n_q; ++q)
        for (size_t h = kv_h * hpk; h < (kv_h + 1) * hpk; ++h) {
            size_t o_off = q * n_heads * head_dim + h * head_dim;
            float lse_qh = lse[q * n_heads + h];
            if (lse_qh == NEG_INF) continue;
            double D = 0;
            for (size_t d = 0; d < head_dim; ++d) D += (double)O[o_off + d] * (double)dO[o_off + d];
            float D_f32 = (float)D;
            size_t k_limit = causal ? q + (n_kv - n_q) : n_kv - 1;
            for (size_t k = 0; k < n_kv; ++k) {
                if (causal && k > k_limit) continue;
                size_t k_off = k * n_kv_heads * head_dim + kv_h * head_dim;
                double s = 0;
                for (size_t d = 0; d < head_dim; ++d) s += (double)Q[o_off + d] * (double)K[k_off + d];
                float S = (float)s * inv_sqrt_d;
                float P = expf(S - lse_qh);
                if (P == 0.0f) continue;
                const float Pv = bf16_ops ? bf16r(P) : P;
                for (size_t d = 0; d < head_dim; ++d) dV[k_off + d] += Pv * dO[o_off + d];
                double dP = 0;
                for (size_t d = 0; d < head_dim; ++d) dP += (double)dO[o_off + d] * (double)V[k_off + d];
                float dS_scaled = bf16_ops ? bf16r(P * ((float)dP - D_f32))
                                           : P * ((float)dP - D_f32) * inv_sqrt_d;
                for (size_t d = 0; d < head_dim; ++d) {
                    dQ[o_off + d] += dS_scaled * K[k_off + d];
                    dK[k_off + d] += dS_scaled * Q[o_off + d];
                }
            }
        }
    if (bf16_ops) {
        for (size_t i = 0; i < n_q * n_heads * head_dim; ++i) dQ[i] *= inv_sqrt_d;
        for (size_t i = 0; i < n_kv * n_kv_heads * head_dim; ++i) dK[i] *= inv_sqrt_d;
    }
}

void orc_flash_attention_backward(const float *Q, const float *K, const float *V,
                                  const float *O, const float *dO, const float *lse,
                                  size_t n_q, size_t n_kv, size_t n_heads,
                                  size_t n_kv_heads, size_t head_dim, int causal,
                                  float *dQ, float *dK, float *dV) {
    flash_backward(Q, K, V, O, dO, lse, n_q, n_kv, n_heads, n_kv_heads, head_dim, causal, 0, dQ,
                   dK, dV);
}

void orc_flash_attention_forward_bf16ops(const float *Q, const float *K, const float *V,
                                         size_t n_q, size_t n_kv, size_t n_heads,
                                         size_t n_kv_heads, size_t head_dim, int causal,
                                         float *out, float *lse) {
    flash_forward(Q, K, V, n_q, n_kv, n_heads, n_kv_heads, head_dim, causal, 16, 64, 1, out, lse);
}

void orc_flash_attention_backward_bf16ops(const float *Q, const float *K, const float *V,
                                          const float *O, const float *dO, const float *lse,
                                          size_t n_q, size_t n_kv, size_t n_heads,
                                          size_t n_kv_heads, size_t head_dim, int causal,
                                          float *dQ, float *dK, float *dV) {
    flash_backward(Q, K, V, O, dO, lse, n_q, n_kv, n_heads, n_kv_heads, head_dim, causal, 1, dQ,
                   dK, dV);
}

void orc_fa_bw_d(const float *O, const float *dO, size_t n_q, size_t n_heads,
                 size_t head_dim, float *D) {
    for (size_t q = 0; q < n_q; ++q)
        for (size_t h = 0; h < n_heads; ++h) {
            size_t off = q * n_heads * head_dim + h * head_dim;
            double acc = 0;
            for (size_t d = 0; d < head_dim; ++d) acc += (double)O[off + d] * (double)dO[off + d];
            D[q * n_heads + h] = (float)acc;
        }
}

/* ── linear layers: train_decoder.zig:45-58 and :294-332 ───────────────── */

void orc_matmul_nt(float *out, const float *x, const float *W, size_t M, size_t N,
                   size_t K) {
    /* every output is its own fp32 k-ascending sum: parallel over outputs.
     * Rows go MM_G at a time over a transposed copy of their x values, so
     * the MM_G sums of one W row advance together (vectorised across rows,
     * each still summed in k order). */
    enum { MM_G = 64 };
    const size_t ng = M / MM_G;
    float *xt = malloc((ng ? ng : 1) * K * MM_G * sizeof(float));
#pragma omp parallel for schedule(static)
    for (size_t g = 0; g < ng; ++g)
        for (size_t j = 0; j < MM_G; ++j)
            for (size_t k = 0; k < K; ++k) xt[(g * K + k) * MM_G + j] = x[(g * MM_G + j) * K + k];
    const long long tasks = (long long)ng * (long long)N;
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < tasks; ++i) {
        const size_t g = (size_t)i / N, n = (size_t)i % N;
        const float *xg = xt + g * K * MM_G, *wr = W + n * K;
        float acc[MM_G];
        for (int j = 0; j < MM_G; ++j) acc[j] = 0;
        for (size_t k = 0; k < K; ++k) {
            const float w = wr[k];
            for (int j = 0; j < MM_G; ++j) acc[j] += xg[k * MM_G + j] * w;
        }
        for (int j = 0; j < MM_G; ++j) out[(g * MM_G + j) * N + n] = acc[j];
    }
    free(xt);
    const long long rest = (long long)(M - ng * MM_G) * (long long)N;
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < rest; ++i) {
        const size_t m = ng * MM_G + (size_t)i / N, n = (size_t)i % N;
        const float *xr = x + m * K, *wr = W + n * K;
        float acc = 0;
        for (size_t k = 0; k < K; ++k) acc += xr[k] * wr[k];
        out[m * N + n] = acc;
    }
}

void orc_linear_backward(const float *dout, const float *x, const float *W, size_t M,
                         size_t N, size_t K, float *dx, float *dW) {
    /* LB_G independent outputs rows advance together per streamed row of the
     * other operand; each output is still its own fp64 sum in the stated order */
    enum { LB_G = 8 };
    if (dx) {
        /* dx[m,k] = sum_n dout[m,n] W[n,k]; fp64 per output, n ascending
         * (rows of dx are independent). */
        const size_t nb = (M + LB_G - 1) / LB_G;
#pragma omp parallel
        {
            double *acc = malloc(LB_G * K * sizeof(double));
#pragma omp for schedule(static)
            for (size_t b = 0; b < nb; ++b) {
                const size_t m0 = b * LB_G, mr = m0 + LB_G <= M ? LB_G : M - m0;
                for (size_t i = 0; i < mr * K; ++i) acc[i] = 0;
                for (size_t n = 0; n < N; ++n) {
                    const float *wr = W + n * K;
                    for (size_t r = 0; r < mr; ++r) {
                        const double g = dout[(m0 + r) * N + n];
                        double *ar = acc + r * K;
                        for (size_t k = 0; k < K; ++k) ar[k] += g * (double)wr[k];
                    }
                }
                for (size_t r = 0; r < mr; ++r)
                    for (size_t k = 0; k < K; ++k) dx[(m0 + r) * K + k] = (float)acc[r * K + k];
            }
            free(acc);
        }
    }
    if (dW) {
        /* dW[n,k] += sum_m dout[m,n] x[m,k]; fp64 per output, m ascending
         * (rows of dW are independent). */
        const size_t nb = (N + LB_G - 1) / LB_G;
#pragma omp parallel
        {
            double *acc = malloc(LB_G * K * sizeof(double));
#pragma omp for schedule(static)
            for (size_t b = 0; b < nb; ++b) {
                const size_t n0 = b * LB_G, nr = n0 + LB_G <= N ? LB_G : N - n0;
                for (size_t i = 0; i < nr * K; ++i) acc[i] = 0;
                for (size_t m = 0; m < M; ++m) {
                    const float *xr = x + m * K;
                    for (size_t r = 0; r < nr; ++r) {
                        const double g = dout[m * N + n0 + r];
                        double *ar = acc + r * K;
                        for (size_t k = 0; k < K; ++k) ar[k] += g * (double)xr[k];
                    }
                }
                for (size_t r = 0; r < nr; ++r)
                    for (size_t k = 0; k < K; ++k) dW[(n0 + r) * K + k] += (float)acc[r * K + k];
            }
            free(acc);
        }
    }
}

/* ── cut cross-entropy: src/cpu/cce.zig:89-268 ─────────────────────────── */

/* Rows are taken CCE_RB at a time; the logits of a block are formed vocab
 * row by vocab row (z_t[v * nr + r], each an fp64 dot rounded to fp32 as in
 * cce.zig), so the head matrix streams once per block.  The per-row online
 * softmax then walks the chunks exactly as cce.zig does.  Within a block, 32
 * rows' dots advance together over a transposed copy of their h values (32
 * independent fp64 sums, vectorised across the rows); each is still its own
 * k-ascending sum, so the values do not depend on the grouping. */
#define CCE_RB 128
#define CCE_G 32

static void cce_logits_block(const float *h, const float *w_lm, size_t r0, size_t nr,
                             size_t vocab, size_t dim, float *z_t) {
    const size_t ng = nr / CCE_G;
    float *ht = malloc((ng ? ng : 1) * dim * CCE_G * sizeof(float));
    for (size_t g = 0; g < ng; ++g)
        for (size_t j = 0; j < CCE_G; ++j) {
            const float *hr = h + (r0 + g * CCE_G + j) * dim;
            for (size_t k = 0; k < dim; ++k) ht[(g * dim + k) * CCE_G + j] = hr[k];
        }
#pragma omp parallel for schedule(static)
    for (size_t v = 0; v < vocab; ++v) {
        const float *wr = w_lm + v * dim;
        for (size_t g = 0; g < ng; ++g) {
            const float *hg = ht + g * dim * CCE_G;
            double s[CCE_G];
            for (int j = 0; j < CCE_G; ++j) s[j] = 0;
            for (size_t k = 0; k < dim; ++k) {
                const double w = (double)wr[k];
                for (int j = 0; j < CCE_G; ++j) s[j] += (double)hg[k * CCE_G + j] * w;
            }
            for (int j = 0; j < CCE_G; ++j) z_t[v * nr + g * CCE_G + j] = (float)s[j];
        }
        for (size_t r = ng * CCE_G; r < nr; ++r) {
            const float *hr = h + (r0 + r) * dim;
            double s = 0;
            for (size_t k = 0; k < dim; ++k) s += (double)hr[k] * (double)wr[k];
            z_t[v * nr + r] = (float)s;
        }
    }
    free(ht);
}

float orc_cce_forward(const float *h, const float *w_lm, const uint32_t *tgt, size_t n,
                      size_t vocab, size_t dim, size_t chunk, float z_loss_scale,
                      float label_smoothing, float *lse_out, float *loss_row_out) {
    float eps = label_smoothing;
    float t_scale = 1.0f - eps;
    float *z_t = malloc((size_t)CCE_RB * vocab * sizeof(float));
    double *row_loss = malloc(n * sizeof(double));
    for (size_t r0 = 0; r0 < n; r0 += CCE_RB) {
        const size_t nr = r0 + CCE_RB < n ? CCE_RB : n - r0;
        cce_logits_block(h, w_lm, r0, nr, vocab, dim, z_t);
#pragma omp parallel for schedule(static)
        for (size_t r = 0; r < nr; ++r) {
            const size_t row = r0 + r;
            float m = NEG_INF;
            double d_acc = 0, z_sum = 0;
            float z_target = 0;
            size_t t = tgt[row];
            for (size_t c0 = 0; c0 < vocab; c0 += chunk) {
                size_t c1 = c0 + chunk < vocab ? c0 + chunk : vocab;
                float chunk_max = NEG_INF;
                for (size_t v = c0; v < c1; ++v) {
                    float zi = z_t[v * nr + r];
                    if (zi > chunk_max) chunk_max = zi;
                    z_sum += (double)zi;
                }
                float m_new = m > chunk_max ? m : chunk_max;
                double chunk_sum = 0;
                for (size_t v = c0; v < c1; ++v) chunk_sum += exp((double)z_t[v * nr + r] - (double)m_new);
                double rescale = isinf(m) ? 0.0 : exp((double)m - (double)m_new);
                d_acc = d_acc * rescale + chunk_sum;
                m = m_new;
                if (t >= c0 && t < c1) z_target = z_t[t * nr + r];
            }
            float lse = (float)(log(d_acc) + (double)m);
            lse_out[row] = lse;
            double z_mean = z_sum / (double)vocab;
            double ce = (double)lse - (double)t_scale * (double)z_target - (double)eps * z_mean;
            double zp = (double)z_loss_scale * (double)lse * (double)lse;
            if (loss_row_out) loss_row_out[row] = (float)(ce + zp);
            row_loss[row] = ce + zp;
        }
    }
    double total_loss = 0;
    for (size_t row = 0; row < n; ++row) total_loss += row_loss[row];
    free(z_t);
    free(row_loss);
    return (float)(total_loss / (double)n);
}

/* dh[row, :] accumulates dz * W[v, :] with v ascending and dW[v, :]
 * accumulates dz * h[row, :] with rows ascending, in fp32, as cce.zig's
 * row-by-row loop does; the block structure only changes which of these
 * independent sums is advanced when. */
static void cce_backward(const float *h, const float *w_lm, const uint32_t *tgt,
                         const float *lse, size_t n, size_t vocab, size_t dim,
                         float z_loss_scale, float label_smoothing, int bf16_ops, float *d_h,
                         float *dW) {
    memset(d_h, 0, n * dim * sizeof(float));
    float inv_n = 1.0f / (float)n;
    float eps = label_smoothing;
    float eps_over_v = eps / (float)vocab;
    float t_scale = 1.0f - eps;
    float *z_t = malloc((size_t)CCE_RB * vocab * sizeof(float));
    for (size_t r0 = 0; r0 < n; r0 += CCE_RB) {
        const size_t nr = r0 + CCE_RB < n ? CCE_RB : n - r0;
        cce_logits_block(h, w_lm, r0, nr, vocab, dim, z_t);
        /* z -> dz in place */
#pragma omp parallel for schedule(static)
        for (size_t v = 0; v < vocab; ++v)
            for (size_t r = 0; r < nr; ++r) {
                const size_t row = r0 + r;
                float lse_row = lse[row];
                float softmax_factor = 1.0f + 2.0f * z_loss_scale * lse_row;
                float p = (float)exp((double)z_t[v * nr + r] - (double)lse_row);
                float ti = (v == tgt[row]) ? t_scale : 0.0f;
                const float dz = (softmax_factor * p - ti - eps_over_v) * inv_n;
                /* bf16 operands: dz is an operand of both products */
                z_t[v * nr + r] = bf16_ops ? orc_bf16_to_f32(orc_f32_to_bf16(dz)) : dz;
            }
        /* dh: each thread owns whole rows and walks the vocabulary in tiles
         * of 64 head rows (reused from cache by all its rows) */
#pragma omp parallel
        {
            size_t ra = 0, rb = nr;
#ifdef _OPENMP
            const size_t nt = (size_t)omp_get_num_threads(), ti = (size_t)omp_get_thread_num();
            ra = nr * ti / nt;
            rb = nr * (ti + 1) / nt;
#endif
            for (size_t v0 = 0; v0 < vocab && ra < rb; v0 += 64) {
                const size_t v1 = v0 + 64 < vocab ? v0 + 64 : vocab;
                for (size_t r = ra; r < rb; ++r) {
                    float *dhr = d_h + (r0 + r) * dim;
                    for (size_t v = v0; v < v1; ++v) {
                        const float dz = z_t[v * nr + r];
                        const float *wr = w_lm + v * dim;
                        for (size_t k = 0; k < dim; ++k) dhr[k] += dz * wr[k];
                    }
                }
            }
        }
        if (dW) {
            /* each dW element takes the block's rows in ascending order; 64
             * columns of a vocabulary row are held in registers across them */
#pragma omp parallel for schedule(static)
            for (size_t v = 0; v < vocab; ++v) {
                float *dwr = dW + v * dim;
                const float *zr = z_t + v * nr;
                size_t k0 = 0;
                for (; k0 + 64 <= dim; k0 += 64) {
                    float acc[64];
                    for (int k = 0; k < 64; ++k) acc[k] = dwr[k0 + k];
                    for (size_t r = 0; r < nr; ++r) {
                        const float dz = zr[r];
                        const float *hr = h + (r0 + r) * dim + k0;
                        for (int k = 0; k < 64; ++k) acc[k] += dz * hr[k];
                    }
                    for (int k = 0; k < 64; ++k) dwr[k0 + k] = acc[k];
                }
                for (size_t r = 0; r < nr && k0 < dim; ++r) {
                    const float dz = zr[r];
                    const float *hr = h + (r0 + r) * dim;
                    for (size_t k = k0; k < dim; ++k) dwr[k] += dz * hr[k];
                }
            }
        }
    }
    free(z_t);
}

void orc_cce_backward(const float *h, const float *w_lm, const uint32_t *tgt,
                      const float *lse, size_t n, size_t vocab, size_t dim, size_t chunk,
                      float z_loss_scale, float label_smoothing, float *d_h, float *dW) {
    (void)chunk; /* the chunking of cce.zig does not change any value here */
    cce_backward(h, w_lm, tgt, lse, n, vocab, dim, z_loss_scale, label_smoothing, 0, d_h, dW);
}

/* The bf16-operand model of the MFMA path: dz rounds to bf16 (the operand
 * of dh = dz W and dW = dz^T h); h and W are expected already rounded. */
void orc_cce_backward_bf16ops(const float *h, const float *w_lm, const uint32_t *tgt,
                              const float *lse, size_t n, size_t vocab, size_t dim,
                              float z_loss_scale, float label_smoothing, float *d_h, float *dW) {
    cce_backward(h, w_lm, tgt, lse, n, vocab, dim, z_loss_scale, label_smoothing, 1, d_h, dW);
}

float orc_softmax_ce_loss(const float *logits, const uint32_t *tgt, size_t n_pos,
                          size_t vocab) {
    double total = 0;
    for (size_t p = 0; p < n_pos; ++p) {
        const float *l = logits + p * vocab;
        float m = NEG_INF;
        for (size_t o = 0; o < vocab; ++o) m = l[o] > m ? l[o] : m;
        double sum_e = 0;
        for (size_t o = 0; o < vocab; ++o) sum_e += exp((double)l[o] - (double)m);
        double log_z = (double)m + log(sum_e);
        total -= (double)l[tgt[p]] - log_z;
    }
    return (float)(total / (double)n_pos);
}

void orc_softmax_ce_loss_grad(float *d_logits, const float *logits, const uint32_t *tgt,
                              size_t n_pos, size_t vocab) {
    float inv_n = 1.0f / (float)n_pos;
    for (size_t p = 0; p < n_pos; ++p) {
        const float *l = logits + p * vocab;
        float m = NEG_INF;
        for (size_t o = 0; o < vocab; ++o) m = l[o] > m ? l[o] : m;
        double sum_e = 0;
        for (size_t o = 0; o < vocab; ++o) sum_e += exp((double)l[o] - (double)m);
        double inv_sum = 1.0 / sum_e;
        for (size_t o = 0; o < vocab; ++o) {
            double p_o = exp((double)l[o] - (double)m) * inv_sum;
            float t_o = (o == tgt[p]) ? 1.0f : 0.0f;
            d_logits[p * vocab + o] = inv_n * ((float)p_o - t_o);
        }
    }
}

/* ── LoRA: src/cpu/lora.zig:75-199 ─────────────────────────────────────── */

/* out[m, n] = (float) sum_k (double) x[m, k] * (double) W[n, k]: every output its own
 * fp64 sum, k ascending.  Rows go DR_G at a time over a transposed copy of their x
 * values, so the DR_G sums of one W row advance together (vectorised across rows, each
 * still summed in k order: the values do not depend on the grouping). */
static void dot_rows_f64(float *out, const float *x, const float *W, size_t M, size_t N,
                         size_t K) {
    enum { DR_G = 16 };
    const size_t ng = M / DR_G;
    float *xt = malloc((ng ? ng : 1) * K * DR_G * sizeof(float));
#pragma omp parallel for schedule(static)
    for (size_t g = 0; g < ng; ++g)
        for (size_t j = 0; j < DR_G; ++j)
            for (size_t k = 0; k < K; ++k) xt[(g * K + k) * DR_G + j] = x[(g * DR_G + j) * K + k];
    const long long tasks = (long long)ng * (long long)N;
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < tasks; ++i) {
        const size_t g = (size_t)i / N, n = (size_t)i % N;
        const float *xg = xt + g * K * DR_G, *wr = W + n * K;
        double acc[DR_G];
        for (int j = 0; j < DR_G; ++j) acc[j] = 0;
        for (size_t k = 0; k < K; ++k) {
            const double wv = (double)wr[k];
            for (int j = 0; j < DR_G; ++j) acc[j] += (double)xg[k * DR_G + j] * wv;
        }
        for (int j = 0; j < DR_G; ++j) out[(g * DR_G + j) * N + n] = (float)acc[j];
    }
    free(xt);
    const long long rest = (long long)(M - ng * DR_G) * (long long)N;
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < rest; ++i) {
        const size_t m = ng * DR_G + (size_t)i / N, n = (size_t)i % N;
        double s = 0;
        for (size_t k = 0; k < K; ++k) s += (double)x[m * K + k] * (double)W[n * K + k];
        out[m * N + n] = (float)s;
    }
}

/* y = x w^T (fp64 sums, k ascending), inter = x a^T, then y += alpha/r * (inter b^T
 * summed in fp64, i ascending, rounded to fp32 before the scale). */
void orc_lora_forward(const float *x, const float *w, const float *a, const float *b,
                      size_t M, size_t N, size_t K, size_t r, float alpha_over_r,
                      float *y_out, float *inter) {
    dot_rows_f64(y_out, x, w, M, N, K);
    dot_rows_f64(inter, x, a, M, r, K);
#pragma omp parallel for schedule(static)
    for (size_t m = 0; m < M; ++m)
        for (size_t n = 0; n < N; ++n) {
            double s = 0;
            for (size_t i = 0; i < r; ++i) s += (double)inter[m * r + i] * (double)b[n * r + i];
            y_out[m * N + n] += (float)s * alpha_over_r;
        }
}

/* dy_B = dy b (fp64 over n ascending); dx = dy w + alpha/r * dy_B a, the base part an
 * fp64 sum over n ascending and the update an fp64 sum over i ascending, added in fp64;
 * dA += alpha/r * dy_B^T x and dB += alpha/r * dy^T inter, fp64 sums over m ascending.
 * Parallel over independent outputs; every output keeps its own summation order. */
void orc_lora_backward(const float *dy, const float *x, const float *w, const float *a,
                       const float *b, const float *inter, size_t M, size_t N, size_t K,
                       size_t r, float alpha_over_r, float *dx, float *dA, float *dB) {
    float *dy_B = malloc((M ? M : 1) * (r ? r : 1) * sizeof(float));
    float *bt = malloc((N ? N : 1) * (r ? r : 1) * sizeof(float));
    for (size_t n = 0; n < N; ++n)
        for (size_t i = 0; i < r; ++i) bt[i * N + n] = b[n * r + i];
    dot_rows_f64(dy_B, dy, bt, M, r, N);
    free(bt);
    if (dx) {
        enum { LX_G = 8 };
        const size_t nb = (M + LX_G - 1) / LX_G;
#pragma omp parallel
        {
            double *acc = malloc(LX_G * K * sizeof(double));
#pragma omp for schedule(static)
            for (size_t blk = 0; blk < nb; ++blk) {
                const size_t m0 = blk * LX_G, mr = m0 + LX_G <= M ? LX_G : M - m0;
                for (size_t i = 0; i < mr * K; ++i) acc[i] = 0;
                for (size_t n = 0; n < N; ++n) {
                    const float *wr = w + n * K;
                    for (size_t q = 0; q < mr; ++q) {
                        const double g = dy[(m0 + q) * N + n];
                        double *aq = acc + q * K;
                        for (size_t k = 0; k < K; ++k) aq[k] += g * (double)wr[k];
                    }
                }
                for (size_t q = 0; q < mr; ++q) {
                    const size_t m = m0 + q;
                    for (size_t k = 0; k < K; ++k) {
                        double s_lora = 0;
                        for (size_t i = 0; i < r; ++i)
                            s_lora += (double)dy_B[m * r + i] * (double)a[i * K + k];
                        dx[m * K + k] = (float)(acc[q * K + k] + alpha_over_r * s_lora);
                    }
                }
            }
            free(acc);
        }
    }
    {
        enum { LA_KC = 256 };
        const size_t nkc = (K + LA_KC - 1) / LA_KC;
#pragma omp parallel
        {
            double *acc = malloc((r ? r : 1) * LA_KC * sizeof(double));
#pragma omp for schedule(static)
            for (size_t c = 0; c < nkc; ++c) {
                const size_t k0 = c * LA_KC, kn = k0 + LA_KC <= K ? LA_KC : K - k0;
                for (size_t i = 0; i < r * LA_KC; ++i) acc[i] = 0;
                for (size_t m = 0; m < M; ++m) {
                    const float *xr = x + m * K + k0;
                    for (size_t i = 0; i < r; ++i) {
                        const double g = dy_B[m * r + i];
                        double *ai = acc + i * LA_KC;
                        for (size_t k = 0; k < kn; ++k) ai[k] += g * (double)xr[k];
                    }
                }
                for (size_t i = 0; i < r; ++i)
                    for (size_t k = 0; k < kn; ++k)
                        dA[i * K + k0 + k] += alpha_over_r * (float)acc[i * LA_KC + k];
            }
            free(acc);
        }
    }
    {
        enum { LB_NC = 64 };
        const size_t nnc = (N + LB_NC - 1) / LB_NC;
#pragma omp parallel
        {
            double *acc = malloc(LB_NC * (r ? r : 1) * sizeof(double));
#pragma omp for schedule(static)
            for (size_t c = 0; c < nnc; ++c) {
                const size_t n0 = c * LB_NC, nn = n0 + LB_NC <= N ? LB_NC : N - n0;
                for (size_t i = 0; i < LB_NC * r; ++i) acc[i] = 0;
                for (size_t m = 0; m < M; ++m) {
                    const float *ir = inter + m * r;
                    for (size_t q = 0; q < nn; ++q) {
                        const double g = dy[m * N + n0 + q];
                        double *aq = acc + q * r;
                        for (size_t i = 0; i < r; ++i) aq[i] += g * (double)ir[i];
                    }
                }
                for (size_t q = 0; q < nn; ++q)
                    for (size_t i = 0; i < r; ++i)
                        dB[(n0 + q) * r + i] += alpha_over_r * (float)acc[q * r + i];
            }
            free(acc);
        }
    }
    free(dy_B);
}

/* ── Adam: shaders/adam_step.comp:41-62 (GPU Runner form) and
 * train_decoder.zig:938-962 (CPU Stack folded-lr form) ──────────────── */

void orc_adam_step(float *param, const float *grad, float *m, float *v, size_t n,
                   float lr, float beta1, float beta2, float eps, uint32_t t,
                   float weight_decay) {
    float t_f = (float)t;
    float bc1 = 1.0f - powf(beta1, t_f);
    float bc2 = 1.0f - powf(beta2, t_f);
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; ++i) {
        float g = grad[i];
        float nm = beta1 * m[i] + (1.0f - beta1) * g;
        float nv = beta2 * v[i] + (1.0f - beta2) * g * g;
        m[i] = nm;
        v[i] = nv;
        float m_hat = nm / bc1, v_hat = nv / bc2;
        float p = param[i];
        if (weight_decay > 0.0f) p = p * (1.0f - lr * weight_decay);
        param[i] = p - lr * m_hat / (sqrtf(v_hat) + eps);
    }
}

void orc_adam_step_folded(float *param, const float *grad, float *m, float *v, size_t n,
                          float lr, float beta1, float beta2, float eps, uint32_t t) {
    float t_f = (float)t;
    float bc1 = 1.0f - powf(beta1, t_f);
    float bc2 = 1.0f - powf(beta2, t_f);
    float lr_t = lr * sqrtf(bc2) / bc1;
    for (size_t i = 0; i < n; ++i) {
        m[i] = beta1 * m[i] + (1.0f - beta1) * grad[i];
        v[i] = beta2 * v[i] + (1.0f - beta2) * grad[i] * grad[i];
        param[i] -= lr_t * m[i] / (sqrtf(v[i]) + eps);
    }
}

/* ── whole model ───────────────────────────────────────────────────────── */

#define N_PROJ 7
typedef struct { size_t off, numel; } span;

typedef struct {
    span t[11];      /* n1,q,k,v,o,n2,gate,up,down,q_norm,k_norm */
    span lora_a[N_PROJ], lora_b[N_PROJ];
} layer_spans;

typedef struct {
    float *n1, *q_pre_norm, *k_pre_norm, *q_normed, *k_normed, *q, *k, *v, *attn_out,
        *lse, *mid, *n2, *pre_gate, *up, *gated, *y;
    float *inter[N_PROJ];
} layer_acts;

struct orc_model {
    orc_model_config cfg;
    size_t T, qd, kvd;
    span embed, final_norm, lm_head;
    layer_spans *ls;
    size_t total;
    float *arena[4];
    layer_acts *acts;
    float *x_emb, *fn_out, *lse, *loss_row;
    uint32_t step_t;
    uint32_t *tokens;
    /* wall seconds spent per phase since the last reset (ORC_PHASE_*) */
    double phase_s[ORC_N_PHASES];
    float *dW_lm_tied; /* the tied head's dW_lm, kept between steps (zeroed per step) */
};

static double now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

void orc_model_phase_seconds(const orc_model *m, double *out) {
    for (int i = 0; i < ORC_N_PHASES; ++i) out[i] = m->phase_s[i];
}

void orc_model_reset_phases(orc_model *m) {
    for (int i = 0; i < ORC_N_PHASES; ++i) m->phase_s[i] = 0;
}

static void proj_shape(const orc_model *m, int p, size_t *N, size_t *K) {
    const orc_model_config *c = &m->cfg;
    switch (p) {
    case 0: *N = m->qd; *K = c->dim; break;
    case 1: case 2: *N = m->kvd; *K = c->dim; break;
    case 3: *N = c->dim; *K = m->qd; break;
    case 4: case 5: *N = c->ff_dim; *K = c->dim; break;
    default: *N = c->dim; *K = c->ff_dim; break;
    }
}

orc_model *orc_model_create(const orc_model_config *cfg) {
    orc_model *m = calloc(1, sizeof(*m));
    m->cfg = *cfg;
    if (m->cfg.n_seqs == 0) m->cfg.n_seqs = 1;
    const orc_model_config *c = &m->cfg;
    m->T = (size_t)c->seq_len * c->n_seqs;
    m->qd = (size_t)c->n_heads * c->head_dim;
    m->kvd = (size_t)c->n_kv_heads * c->head_dim;
    size_t D = c->dim, V = c->vocab_size, F = c->ff_dim, off = 0;
#define TAKE(sp, n) do { (sp).off = off; (sp).numel = (n); off += (n); } while (0)
    TAKE(m->embed, V * D);
    TAKE(m->final_norm, D);
    if (c->tied_embeddings) { m->lm_head = m->embed; } else { TAKE(m->lm_head, V * D); }
    m->ls = calloc(c->n_layers, sizeof(layer_spans));
    for (uint32_t l = 0; l < c->n_layers; ++l) {
        layer_spans *s = &m->ls[l];
        TAKE(s->t[0], D);
        TAKE(s->t[1], m->qd * D);
        TAKE(s->t[2], m->kvd * D);
        TAKE(s->t[3], m->kvd * D);
        TAKE(s->t[4], D * m->qd);
        TAKE(s->t[5], D);
        TAKE(s->t[6], F * D);
        TAKE(s->t[7], F * D);
        TAKE(s->t[8], D * F);
        if (c->qk_norm) { TAKE(s->t[9], c->head_dim); TAKE(s->t[10], c->head_dim); }
    }
    if (c->lora_targets) {
        for (int p = 0; p < N_PROJ; ++p) {
            if (!(c->lora_targets & (1u << p))) continue;
            size_t N, K;
            proj_shape(m, p, &N, &K);
            for (uint32_t l = 0; l < c->n_layers; ++l) {
                TAKE(m->ls[l].lora_a[p], (size_t)c->lora_rank * K);
                TAKE(m->ls[l].lora_b[p], N * c->lora_rank);
            }
        }
    }
#undef TAKE
    m->total = off;
    for (int k = 0; k < 4; ++k) m->arena[k] = calloc(off ? off : 1, sizeof(float));
    size_t T = m->T, H = c->n_heads;
    m->acts = calloc(c->n_layers, sizeof(layer_acts));
    for (uint32_t l = 0; l < c->n_layers; ++l) {
        layer_acts *a = &m->acts[l];
        a->n1 = malloc(T * D * sizeof(float));
        a->q_pre_norm = malloc(T * m->qd * sizeof(float));
        a->k_pre_norm = malloc(T * m->kvd * sizeof(float));
        a->q_normed = malloc(T * m->qd * sizeof(float));
        a->k_normed = malloc(T * m->kvd * sizeof(float));
        a->q = malloc(T * m->qd * sizeof(float));
        a->k = malloc(T * m->kvd * sizeof(float));
        a->v = malloc(T * m->kvd * sizeof(float));
        a->attn_out = malloc(T * m->qd * sizeof(float));
        a->lse = malloc(T * H * sizeof(float));
        a->mid = malloc(T * D * sizeof(float));
        a->n2 = malloc(T * D * sizeof(float));
        a->pre_gate = malloc(T * F * sizeof(float));
        a->up = malloc(T * F * sizeof(float));
        a->gated = malloc(T * F * sizeof(float));
        a->y = malloc(T * D * sizeof(float));
        for (int p = 0; p < N_PROJ; ++p)
            if (c->lora_targets & (1u << p)) a->inter[p] = malloc(T * c->lora_rank * sizeof(float));
    }
    m->x_emb = malloc(T * D * sizeof(float));
    m->fn_out = malloc(T * D * sizeof(float));
    m->lse = malloc(T * sizeof(float));
    m->loss_row = malloc(T * sizeof(float));
    m->tokens = malloc(T * sizeof(uint32_t));
    m->step_t = 1; /* transformer.zig:940 */
    return m;
}

void orc_model_destroy(orc_model *m) {
    if (!m) return;
    for (uint32_t l = 0; l < m->cfg.n_layers; ++l) {
        layer_acts *a = &m->acts[l];
        free(a->n1); free(a->q_pre_norm); free(a->k_pre_norm); free(a->q_normed);
        free(a->k_normed); free(a->q); free(a->k); free(a->v); free(a->attn_out);
        free(a->lse); free(a->mid); free(a->n2); free(a->pre_gate); free(a->up);
        free(a->gated); free(a->y);
        for (int p = 0; p < N_PROJ; ++p) free(a->inter[p]);
    }
    free(m->acts); free(m->ls);
    for (int k = 0; k < 4; ++k) free(m->arena[k]);
    free(m->x_emb); free(m->fn_out); free(m->lse); free(m->loss_row); free(m->tokens);
    free(m->dW_lm_tied);
    free(m);
}

float *orc_model_tensor(orc_model *m, int kind, int layer, int which, size_t *numel) {
    span sp = {0, 0};
    if (kind < 0 || kind > 3) return NULL;
    if (layer < 0) {
        if (which == ORC_T_EMBED) sp = m->embed;
        else if (which == ORC_T_FINAL_NORM) sp = m->final_norm;
        else if (which == ORC_T_LM_HEAD) sp = m->lm_head;
        else return NULL;
    } else {
        if ((uint32_t)layer >= m->cfg.n_layers) return NULL;
        if (which >= 0 && which < 11) sp = m->ls[layer].t[which];
        else if (which >= ORC_T_LORA_A && which < ORC_T_LORA_A + 2 * N_PROJ) {
            int p = (which - ORC_T_LORA_A) / 2;
            sp = ((which - ORC_T_LORA_A) % 2 == 0) ? m->ls[layer].lora_a[p] : m->ls[layer].lora_b[p];
        } else return NULL;
    }
    if (numel) *numel = sp.numel;
    if (sp.numel == 0) return NULL;
    return m->arena[kind] + sp.off;
}

uint32_t orc_model_step_t(const orc_model *m) { return m->step_t; }

/* step_t as a checkpoint restores it (transformer.zig:1444) */
void orc_model_set_step_t(orc_model *m, uint32_t t) { m->step_t = t; }

void orc_model_init_random(orc_model *m, uint64_t seed, float std, float lora_std) {
    const orc_model_config *c = &m->cfg;
    float *P = m->arena[ORC_PARAM];
    uint64_t s = seed;
    orc_fill_normal(P + m->embed.off, m->embed.numel, orc_splitmix64(&s), 0, std);
    for (size_t i = 0; i < m->final_norm.numel; ++i) P[m->final_norm.off + i] = 1.0f;
    if (!c->tied_embeddings)
        orc_fill_normal(P + m->lm_head.off, m->lm_head.numel, orc_splitmix64(&s), 0, std);
    for (uint32_t l = 0; l < c->n_layers; ++l) {
        layer_spans *ls = &m->ls[l];
        for (int t = 0; t < 11; ++t) {
            span sp = ls->t[t];
            if (!sp.numel) continue;
            uint64_t ts = orc_splitmix64(&s);
            if (t == 0 || t == 5 || t == 9 || t == 10)
                for (size_t i = 0; i < sp.numel; ++i) P[sp.off + i] = 1.0f;
            else orc_fill_normal(P + sp.off, sp.numel, ts, 0, std);
        }
    }
    /* LoRA adapters draw from their own stream so the base weights do not
     * depend on whether LoRA is enabled. */
    uint64_t ls_seed = seed ^ 0x10AAFADEull;
    for (int p = 0; p < N_PROJ; ++p)
        for (uint32_t l = 0; l < c->n_layers; ++l) {
            span a = m->ls[l].lora_a[p];
            if (a.numel) orc_fill_normal(P + a.off, a.numel, orc_splitmix64(&ls_seed), 0, lora_std);
            /* B = 0 */
        }
}

/* bf16 operand staging for the optional bf16-operand mode */
typedef struct { float *buf; size_t cap; } scratch_t;
static const float *maybe_bf16(const orc_model *m, const float *x, size_t n, scratch_t *sc) {
    if (!m->cfg.bf16_operands) return x;
    if (sc->cap < n) { free(sc->buf); sc->buf = malloc(n * sizeof(float)); sc->cap = n; }
    memcpy(sc->buf, x, n * sizeof(float));
    orc_round_bf16(sc->buf, n);
    return sc->buf;
}

static int proj_is_lora(const orc_model *m, int p) {
    return m->cfg.lora_targets && (m->cfg.lora_targets & (1u << p)) && m->cfg.lora_rank > 0;
}

/* y[T,N] = x W^T, or the LoRA-augmented projection (lora.zig:75-121). The
 * GPU Runner's forward matmul is matmul_nt (train_decoder.zig:45-58). */
static void proj_forward(orc_model *m, int l, int p, const float *x, const float *W,
                         float *y, scratch_t *s1, scratch_t *s2) {
    size_t N, K, T = m->T;
    proj_shape(m, p, &N, &K);
    const float *xx = maybe_bf16(m, x, T * K, s1);
    const float *ww = maybe_bf16(m, W, N * K, s2);
    if (proj_is_lora(m, p)) {
        float *P = m->arena[ORC_PARAM];
        const float *A = P + m->ls[l].lora_a[p].off, *B = P + m->ls[l].lora_b[p].off;
        orc_lora_forward(xx, ww, A, B, T, N, K, m->cfg.lora_rank,
                         m->cfg.lora_alpha / (float)m->cfg.lora_rank, y, m->acts[l].inter[p]);
    } else {
        orc_matmul_nt(y, xx, ww, T, N, K);
    }
}

/* Backward of one projection: dx overwritten; dW (or dA/dB) written. */
static void proj_backward(orc_model *m, int l, int p, const float *dy, const float *x,
                          const float *W, float *dx, float *dW, scratch_t *s1,
                          scratch_t *s2, scratch_t *s3) {
    size_t N, K, T = m->T;
    proj_shape(m, p, &N, &K);
    const float *dd = maybe_bf16(m, dy, T * N, s1);
    const float *xx = maybe_bf16(m, x, T * K, s2);
    const float *ww = maybe_bf16(m, W, N * K, s3);
    if (proj_is_lora(m, p)) {
        float *P = m->arena[ORC_PARAM], *G = m->arena[ORC_GRAD];
        layer_spans *ls = &m->ls[l];
        memset(G + ls->lora_a[p].off, 0, ls->lora_a[p].numel * sizeof(float));
        memset(G + ls->lora_b[p].off, 0, ls->lora_b[p].numel * sizeof(float));
        orc_lora_backward(dd, xx, ww, P + ls->lora_a[p].off, P + ls->lora_b[p].off,
                          m->acts[l].inter[p], T, N, K, m->cfg.lora_rank,
                          m->cfg.lora_alpha / (float)m->cfg.lora_rank, dx,
                          G + ls->lora_a[p].off, G + ls->lora_b[p].off);
    } else {
        if (dW) memset(dW, 0, N * K * sizeof(float));
        orc_linear_backward(dd, xx, ww, T, N, K, dx, m->cfg.lora_targets ? NULL : dW);
    }
}

static void layer_forward(orc_model *m, int l, const float *x_in, scratch_t *sc) {
    const orc_model_config *c = &m->cfg;
    float *P = m->arena[ORC_PARAM];
    layer_spans *s = &m->ls[l];
    layer_acts *a = &m->acts[l];
    size_t T = m->T, D = c->dim, S = c->seq_len, H = c->n_heads, Hkv = c->n_kv_heads,
           hd = c->head_dim, F = c->ff_dim;
    /* transformer.zig:1789-1885 */
    orc_rmsnorm_forward(x_in, P + s->t[0].off, T, D, c->rms_eps, 0, a->n1);
    proj_forward(m, l, 0, a->n1, P + s->t[1].off, a->q_pre_norm, &sc[0], &sc[1]);
    proj_forward(m, l, 1, a->n1, P + s->t[2].off, a->k_pre_norm, &sc[0], &sc[1]);
    proj_forward(m, l, 2, a->n1, P + s->t[3].off, a->v, &sc[0], &sc[1]);
    const float *qn = a->q_pre_norm, *kn = a->k_pre_norm;
    if (c->qk_norm) {
        orc_rmsnorm_forward(a->q_pre_norm, P + s->t[9].off, T * H, hd, c->rms_eps, 0, a->q_normed);
        orc_rmsnorm_forward(a->k_pre_norm, P + s->t[10].off, T * Hkv, hd, c->rms_eps, 0, a->k_normed);
        qn = a->q_normed; kn = a->k_normed;
    }
    if (c->rotary_dim > 0) {
        orc_rope_forward_batched(a->q, qn, T, H, hd, c->rotary_dim, c->rope_theta, S);
        orc_rope_forward_batched(a->k, kn, T, Hkv, hd, c->rotary_dim, c->rope_theta, S);
    } else {
        memcpy(a->q, qn, T * m->qd * sizeof(float));
        memcpy(a->k, kn, T * m->kvd * sizeof(float));
    }
    const float *qq = maybe_bf16(m, a->q, T * m->qd, &sc[0]);
    const float *kk = maybe_bf16(m, a->k, T * m->kvd, &sc[1]);
    const float *vv = maybe_bf16(m, a->v, T * m->kvd, &sc[2]);
    /* bf16 operands: the kernels' 64-key tiles and bf16 P (flash_forward) */
    const double ta = now_s();
    for (uint32_t b = 0; b < c->n_seqs; ++b)
        flash_forward(qq + b * S * m->qd, kk + b * S * m->kvd, vv + b * S * m->kvd, S, S, H, Hkv,
                      hd, c->causal != 0, 16, c->bf16_operands ? 64 : 16, c->bf16_operands != 0,
                      a->attn_out + b * S * m->qd, a->lse + b * S * H);
    m->phase_s[ORC_PHASE_ATTN_FWD] += now_s() - ta;
    float *o = malloc(T * D * sizeof(float));
    proj_forward(m, l, 3, a->attn_out, P + s->t[4].off, o, &sc[0], &sc[1]);
    for (size_t i = 0; i < T * D; ++i) a->mid[i] = x_in[i] + o[i];
    free(o);
    orc_rmsnorm_forward(a->mid, P + s->t[5].off, T, D, c->rms_eps, 0, a->n2);
    proj_forward(m, l, 4, a->n2, P + s->t[6].off, a->pre_gate, &sc[0], &sc[1]);
    proj_forward(m, l, 5, a->n2, P + s->t[7].off, a->up, &sc[0], &sc[1]);
    orc_swiglu_forward(a->pre_gate, a->up, T * F, a->gated);
    float *ff = malloc(T * D * sizeof(float));
    proj_forward(m, l, 6, a->gated, P + s->t[8].off, ff, &sc[0], &sc[1]);
    for (size_t i = 0; i < T * D; ++i) a->y[i] = a->mid[i] + ff[i];
    free(ff);
}

/* transformer.zig:1967-2070 (order), train_decoder.zig:340-498 (math). */
static void layer_backward(orc_model *m, int l, const float *x_in, const float *d_y,
                           float *d_x_in, scratch_t *sc) {
    const orc_model_config *c = &m->cfg;
    float *P = m->arena[ORC_PARAM], *G = m->arena[ORC_GRAD];
    layer_spans *s = &m->ls[l];
    layer_acts *a = &m->acts[l];
    size_t T = m->T, D = c->dim, S = c->seq_len, H = c->n_heads, Hkv = c->n_kv_heads,
           hd = c->head_dim, F = c->ff_dim;
    int lora = c->lora_targets != 0;
    float *d_gated = malloc(T * F * sizeof(float));
    float *d_pre_gate = malloc(T * F * sizeof(float));
    float *d_up = malloc(T * F * sizeof(float));
    float *d_n2 = malloc(T * D * sizeof(float));
    float *tmp = malloc(T * D * sizeof(float));
    float *d_mid = malloc(T * D * sizeof(float));
    proj_backward(m, l, 6, d_y, a->gated, P + s->t[8].off, d_gated, G + s->t[8].off, &sc[0], &sc[1], &sc[2]);
    orc_swiglu_backward(d_gated, a->pre_gate, a->up, T * F, d_pre_gate, d_up);
    proj_backward(m, l, 4, d_pre_gate, a->n2, P + s->t[6].off, d_n2, G + s->t[6].off, &sc[0], &sc[1], &sc[2]);
    proj_backward(m, l, 5, d_up, a->n2, P + s->t[7].off, tmp, G + s->t[7].off, &sc[0], &sc[1], &sc[2]);
    for (size_t i = 0; i < T * D; ++i) d_n2[i] += tmp[i];
    float *dw_n2 = G + s->t[5].off;
    if (!lora) memset(dw_n2, 0, D * sizeof(float));
    orc_rmsnorm_backward(d_n2, a->mid, P + s->t[5].off, T, D, c->rms_eps, 0, tmp, lora ? NULL : dw_n2);
    for (size_t i = 0; i < T * D; ++i) d_mid[i] = d_y[i] + tmp[i];
    float *d_attn_out = malloc(T * m->qd * sizeof(float));
    proj_backward(m, l, 3, d_mid, a->attn_out, P + s->t[4].off, d_attn_out, G + s->t[4].off, &sc[0], &sc[1], &sc[2]);
    float *dQ = malloc(T * m->qd * sizeof(float)), *dK = malloc(T * m->kvd * sizeof(float));
    float *dV = malloc(T * m->kvd * sizeof(float));
    const float *qq = maybe_bf16(m, a->q, T * m->qd, &sc[0]);
    const float *kk = maybe_bf16(m, a->k, T * m->kvd, &sc[1]);
    const float *vv = maybe_bf16(m, a->v, T * m->kvd, &sc[2]);
    const float *dd = maybe_bf16(m, d_attn_out, T * m->qd, &sc[3]);
    /* bf16 operands: D = rowsum(O dO) over the bf16 O the kernels keep */
    const float *oo = maybe_bf16(m, a->attn_out, T * m->qd, &sc[4]);
    const double ta = now_s();
    for (uint32_t b = 0; b < c->n_seqs; ++b)
        flash_backward(qq + b * S * m->qd, kk + b * S * m->kvd, vv + b * S * m->kvd,
                       oo + b * S * m->qd, dd + b * S * m->qd, a->lse + b * S * H, S, S, H, Hkv,
                       hd, c->causal != 0, c->bf16_operands != 0, dQ + b * S * m->qd,
                       dK + b * S * m->kvd, dV + b * S * m->kvd);
    m->phase_s[ORC_PHASE_ATTN_BWD] += now_s() - ta;
    float *dQ2 = malloc(T * m->qd * sizeof(float)), *dK2 = malloc(T * m->kvd * sizeof(float));
    if (c->rotary_dim > 0) {
        orc_rope_backward_batched(dQ2, dQ, T, H, hd, c->rotary_dim, c->rope_theta, S);
        orc_rope_backward_batched(dK2, dK, T, Hkv, hd, c->rotary_dim, c->rope_theta, S);
        memcpy(dQ, dQ2, T * m->qd * sizeof(float));
        memcpy(dK, dK2, T * m->kvd * sizeof(float));
    }
    if (c->qk_norm) {
        float *dwq = G + s->t[9].off, *dwk = G + s->t[10].off;
        if (!lora) { memset(dwq, 0, hd * sizeof(float)); memset(dwk, 0, hd * sizeof(float)); }
        orc_rmsnorm_backward(dQ, a->q_pre_norm, P + s->t[9].off, T * H, hd, c->rms_eps, 0, dQ2, lora ? NULL : dwq);
        orc_rmsnorm_backward(dK, a->k_pre_norm, P + s->t[10].off, T * Hkv, hd, c->rms_eps, 0, dK2, lora ? NULL : dwk);
        memcpy(dQ, dQ2, T * m->qd * sizeof(float));
        memcpy(dK, dK2, T * m->kvd * sizeof(float));
    }
    float *d_n1 = malloc(T * D * sizeof(float));
    proj_backward(m, l, 0, dQ, a->n1, P + s->t[1].off, d_n1, G + s->t[1].off, &sc[0], &sc[1], &sc[2]);
    proj_backward(m, l, 1, dK, a->n1, P + s->t[2].off, tmp, G + s->t[2].off, &sc[0], &sc[1], &sc[2]);
    for (size_t i = 0; i < T * D; ++i) d_n1[i] += tmp[i];
    proj_backward(m, l, 2, dV, a->n1, P + s->t[3].off, tmp, G + s->t[3].off, &sc[0], &sc[1], &sc[2]);
    for (size_t i = 0; i < T * D; ++i) d_n1[i] += tmp[i];
    float *dw_n1 = G + s->t[0].off;
    if (!lora) memset(dw_n1, 0, D * sizeof(float));
    orc_rmsnorm_backward(d_n1, x_in, P + s->t[0].off, T, D, c->rms_eps, 0, d_x_in, lora ? NULL : dw_n1);
    for (size_t i = 0; i < T * D; ++i) d_x_in[i] += d_mid[i];
    free(d_gated); free(d_pre_gate); free(d_up); free(d_n2); free(tmp); free(d_mid);
    free(d_attn_out); free(dQ); free(dK); free(dV); free(dQ2); free(dK2); free(d_n1);
}

static void model_forward(orc_model *m, const uint32_t *tokens, scratch_t *sc) {
    const orc_model_config *c = &m->cfg;
    float *P = m->arena[ORC_PARAM];
    size_t T = m->T, D = c->dim;
    memcpy(m->tokens, tokens, T * sizeof(uint32_t));
    double t0 = now_s();
    orc_embedding_forward(P + m->embed.off, tokens, T, D, m->x_emb);
    double t1 = now_s();
    for (uint32_t l = 0; l < c->n_layers; ++l)
        layer_forward(m, l, l == 0 ? m->x_emb : m->acts[l - 1].y, sc);
    double t2 = now_s();
    orc_rmsnorm_forward(m->acts[c->n_layers - 1].y, P + m->final_norm.off, T, D, c->rms_eps, 0, m->fn_out);
    m->phase_s[ORC_PHASE_LAYER_FWD] += t2 - t1;
    m->phase_s[ORC_PHASE_HEAD] += (t1 - t0) + (now_s() - t2);
}

/* The head on the last layer's output y: final RMSNorm, the chunked CE
 * forward and backward (cce_backward: dh overwritten, dW_lm accumulated into
 * zero; tied: kept in m->dW_lm_tied for the embedding's sum) and the final
 * norm's backward, which writes d_y (the gradient at y) and the gain
 * gradient (transformer.zig:1917-1960). */
static float head_forward_backward(orc_model *m, const float *y, const uint32_t *targets,
                                   float *d_y, scratch_t *sc) {
    const orc_model_config *c = &m->cfg;
    float *P = m->arena[ORC_PARAM], *G = m->arena[ORC_GRAD];
    size_t T = m->T, D = c->dim, V = c->vocab_size;
    int lora = c->lora_targets != 0;
    orc_rmsnorm_forward(y, P + m->final_norm.off, T, D, c->rms_eps, 0, m->fn_out);
    const float *hh = maybe_bf16(m, m->fn_out, T * D, &sc[0]);
    const float *ww = maybe_bf16(m, P + m->lm_head.off, V * D, &sc[1]);
    size_t chunk = V < 1024 ? V : 1024;
    float loss = orc_cce_forward(hh, ww, targets, T, V, D, chunk, 0, 0, m->lse, m->loss_row);
    float *d_fn = malloc(T * D * sizeof(float));
    float *dW_lm = NULL;
    if (!lora) {
        if (c->tied_embeddings && !m->dW_lm_tied) m->dW_lm_tied = malloc(V * D * sizeof(float));
        dW_lm = c->tied_embeddings ? m->dW_lm_tied : G + m->lm_head.off;
        memset(dW_lm, 0, V * D * sizeof(float));
    }
    cce_backward(hh, ww, targets, m->lse, T, V, D, 0, 0, c->bf16_operands != 0, d_fn, dW_lm);
    float *dw_fn = G + m->final_norm.off;
    if (!lora) memset(dw_fn, 0, D * sizeof(float));
    orc_rmsnorm_backward(d_fn, y, P + m->final_norm.off, T, D, c->rms_eps, 0, d_y,
                         lora ? NULL : dw_fn);
    free(d_fn);
    return loss;
}

/* The embedding gradient from the gradient at the embedding output (the
 * scatter in position order; tied: plus the head's dW_lm). */
static void embed_backward(orc_model *m, const uint32_t *tokens, const float *d_x0) {
    const orc_model_config *c = &m->cfg;
    if (c->lora_targets) return;
    float *G = m->arena[ORC_GRAD];
    size_t T = m->T, D = c->dim, V = c->vocab_size;
    float *dE = G + m->embed.off;
    memset(dE, 0, V * D * sizeof(float));
    orc_embedding_backward(d_x0, tokens, T, V, D, dE);
    if (c->tied_embeddings) {
        /* tied: grad = dE (position-order row sums) + dW_lm */
        const float *dW_lm = m->dW_lm_tied;
        for (size_t i = 0; i < V * D; ++i) dE[i] = dW_lm[i] + dE[i];
    }
}

float orc_model_forward_backward(orc_model *m, const uint32_t *tokens,
                                 const uint32_t *targets) {
    const orc_model_config *c = &m->cfg;
    size_t T = m->T, D = c->dim;
    scratch_t sc[5] = {{0}};
    model_forward(m, tokens, sc);
    double t0 = now_s();
    float *d_y = malloc(T * D * sizeof(float)), *d_x = malloc(T * D * sizeof(float));
    float loss = head_forward_backward(m, m->acts[c->n_layers - 1].y, targets, d_y, sc);
    double t1 = now_s();
    for (int l = (int)c->n_layers - 1; l >= 0; --l) {
        layer_backward(m, l, l == 0 ? m->x_emb : m->acts[l - 1].y, d_y, d_x, sc);
        float *t = d_y; d_y = d_x; d_x = t;
    }
    double t2 = now_s();
    embed_backward(m, tokens, d_y);
    free(d_y); free(d_x);
    for (int k = 0; k < 5; ++k) free(sc[k].buf);
    m->phase_s[ORC_PHASE_LAYER_BWD] += t2 - t1;
    m->phase_s[ORC_PHASE_HEAD] += (t1 - t0) + (now_s() - t2);
    return loss;
}

float orc_model_head_forward_backward(orc_model *m, const float *y, const uint32_t *targets,
                                      float *d_y) {
    scratch_t sc[5] = {{0}};
    float loss = head_forward_backward(m, y, targets, d_y, sc);
    for (int k = 0; k < 5; ++k) free(sc[k].buf);
    return loss;
}

void orc_model_layer_forward_backward(orc_model *m, int l, const float *x_in, const float *d_y,
                                      float *d_x_in) {
    scratch_t sc[5] = {{0}};
    layer_forward(m, l, x_in, sc);
    layer_backward(m, l, x_in, d_y, d_x_in, sc);
    for (int k = 0; k < 5; ++k) free(sc[k].buf);
}

void orc_model_embedding_backward(orc_model *m, const uint32_t *tokens, const float *d_x0) {
    embed_backward(m, tokens, d_x0);
}

void orc_model_layer_output(const orc_model *m, int l, float *out) {
    const float *src = l < 0 ? m->x_emb : m->acts[l].y;
    memcpy(out, src, m->T * m->cfg.dim * sizeof(float));
}

static void adam_span(orc_model *m, span sp, float lr) {
    if (!sp.numel) return;
    const orc_model_config *c = &m->cfg;
    orc_adam_step(m->arena[ORC_PARAM] + sp.off, m->arena[ORC_GRAD] + sp.off,
                  m->arena[ORC_ADAM_M] + sp.off, m->arena[ORC_ADAM_V] + sp.off, sp.numel,
                  lr, c->beta1, c->beta2, c->eps_adam, m->step_t, 0.0f);
}

/* transformer.zig:2072-2149: every tensor in full mode; only LoRA A/B (B at
 * lr * lora_lr_b_scale) when LoRA is active. */
void orc_model_adam(orc_model *m) {
    const orc_model_config *c = &m->cfg;
    const double t0 = now_s();
    if (!c->lora_targets) {
        adam_span(m, m->embed, c->lr);
        for (uint32_t l = 0; l < c->n_layers; ++l)
            for (int t = 0; t < 11; ++t) adam_span(m, m->ls[l].t[t], c->lr);
        adam_span(m, m->final_norm, c->lr);
        if (!c->tied_embeddings) adam_span(m, m->lm_head, c->lr);
    } else {
        for (uint32_t l = 0; l < c->n_layers; ++l)
            for (int p = 0; p < N_PROJ; ++p) {
                adam_span(m, m->ls[l].lora_a[p], c->lr);
                adam_span(m, m->ls[l].lora_b[p], c->lr * c->lora_lr_b_scale);
            }
    }
    m->phase_s[ORC_PHASE_ADAM] += now_s() - t0;
    m->step_t += 1;
}

float orc_model_step(orc_model *m, const uint32_t *tokens, const uint32_t *targets) {
    float loss = orc_model_forward_backward(m, tokens, targets);
    orc_model_adam(m);
    return loss;
}

void orc_model_forward_logits(orc_model *m, const uint32_t *tokens, float *logits) {
    scratch_t sc[5] = {{0}};
    model_forward(m, tokens, sc);
    const orc_model_config *c = &m->cfg;
    const float *hh = maybe_bf16(m, m->fn_out, m->T * c->dim, &sc[0]);
    const float *ww = maybe_bf16(m, m->arena[ORC_PARAM] + m->lm_head.off,
                                 (size_t)c->vocab_size * c->dim, &sc[1]);
    orc_matmul_nt(logits, hh, ww, m->T, c->vocab_size, c->dim);
    for (int k = 0; k < 5; ++k) free(sc[k].buf);
}

double orc_now_seconds(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

/* ══ Tiny-MLP TrainingRunner (src/cpu/train.zig; src/train/runner.zig) ══════
 *
 * Parameters travel as one blob [W1 (H x I) | b1 (H) | W2 (O x H) | b2 (O)],
 * row-major, y = W x + b (cpu/train.zig:25-41). */

/* Zig 0.14 std.Random.DefaultPrng = Xoshiro256++ (Blackman & Vigna), seeded
 * by four SplitMix64 outputs (std/Random/Xoshiro256.zig init/seed). */
void orc_zig_prng_seed(uint64_t s[4], uint64_t seed) {
    uint64_t sm = seed;
    for (int i = 0; i < 4; ++i) s[i] = orc_splitmix64(&sm);
}

static uint64_t rotl64(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

uint64_t orc_zig_prng_next(uint64_t s[4]) {
    const uint64_t r = rotl64(s[0] + s[3], 23) + s[0];
    const uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl64(s[3], 45);
    return r;
}

/* std.Random.float(f32): 23 low bits of one u64 draw are the mantissa; the
 * count of leading zeros of that draw (extended by further draws while the
 * top 41 bits are all zero) picks the exponent 2^-(1+lz), so the result is
 * in [0, 1) with every representable value reachable. */
float orc_zig_float32(uint64_t s[4]) {
    const uint64_t r = orc_zig_prng_next(s);
    unsigned lz = r ? (unsigned)__builtin_clzll(r) : 64u;
    if (lz >= 41) {
        const uint64_t r2 = orc_zig_prng_next(s);
        lz = 41 + (r2 ? (unsigned)__builtin_clzll(r2) : 64u);
        if (lz == 41 + 64) {
            const uint32_t r3 = (uint32_t)orc_zig_prng_next(s);
            lz += (unsigned)__builtin_clz(r3 | 0x7FFu);
        }
    }
    const uint32_t bits = ((uint32_t)(126 - lz) << 23) | (uint32_t)(r & 0x7FFFFFu);
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

size_t orc_mlp_param_count(size_t I, size_t H, size_t O) { return H * I + H + O * H + O; }

/* Mlp.init (cpu/train.zig:47-81): W1 then W2 drawn as (u*2 - 1)*scale with
 * u = rng.float(f32) from DefaultPrng(seed); biases zero. */
void orc_mlp_init(float *P, size_t I, size_t H, size_t O, float init_scale, uint64_t seed) {
    uint64_t s[4];
    orc_zig_prng_seed(s, seed);
    float *w1 = P, *b1 = P + H * I, *w2 = b1 + H, *b2 = w2 + O * H;
    for (size_t k = 0; k < H * I; ++k) w1[k] = (orc_zig_float32(s) * 2.0f - 1.0f) * init_scale;
    for (size_t k = 0; k < O * H; ++k) w2[k] = (orc_zig_float32(s) * 2.0f - 1.0f) * init_scale;
    memset(b1, 0, H * sizeof(float));
    memset(b2, 0, O * sizeof(float));
}

/* forward (cpu/train.zig:146-173). */
void orc_mlp_forward(const float *P, size_t I, size_t H, size_t O, const float *x, float *h_pre,
                     float *h, float *y) {
    const float *w1 = P, *b1 = P + H * I, *w2 = b1 + H, *b2 = w2 + O * H;
    for (size_t i = 0; i < H; ++i) {
        float acc = b1[i];
        for (size_t j = 0; j < I; ++j) acc += w1[i * I + j] * x[j];
        h_pre[i] = acc;
        h[i] = acc > 0 ? acc : 0;
    }
    for (size_t i = 0; i < O; ++i) {
        float acc = b2[i];
        for (size_t j = 0; j < H; ++j) acc += w2[i * H + j] * h[j];
        y[i] = acc;
    }
}

/* mseLoss / mseLossGrad (cpu/train.zig:180-196): L = 1/2 sum (y - t)^2. */
float orc_mse_loss(const float *y, const float *t, size_t n) {
    float acc = 0;
    for (size_t i = 0; i < n; ++i) {
        const float d = y[i] - t[i];
        acc += d * d;
    }
    return 0.5f * acc;
}

void orc_mse_loss_grad(float *dy, const float *y, const float *t, size_t n) {
    for (size_t i = 0; i < n; ++i) dy[i] = y[i] - t[i];
}

/* backward (cpu/train.zig:214-254): overwrites G (blob layout). */
void orc_mlp_backward(const float *P, size_t I, size_t H, size_t O, const float *x,
                      const float *h_pre, const float *h, const float *dy, float *G) {
    const float *w2 = P + H * I + H;
    float *dw1 = G, *db1 = G + H * I, *dw2 = db1 + H, *db2 = dw2 + O * H;
    for (size_t i = 0; i < O; ++i) {
        db2[i] = dy[i];
        for (size_t j = 0; j < H; ++j) dw2[i * H + j] = dy[i] * h[j];
    }
    float *dh = (float *)calloc(H ? H : 1, sizeof(float));
    for (size_t i = 0; i < O; ++i)
        for (size_t j = 0; j < H; ++j) dh[j] += dy[i] * w2[i * H + j];
    for (size_t j = 0; j < H; ++j) {
        const float mask = h_pre[j] > 0 ? 1.0f : 0.0f;
        const float dpre = dh[j] * mask;
        db1[j] = dpre;
        for (size_t k = 0; k < I; ++k) dw1[j * I + k] = dpre * x[k];
    }
    free(dh);
}

/* sgd_step.comp:15-25 (decoupled weight decay on the W spans only, as the
 * runner pushes weight_decay = 0 for biases, runner.zig:1178-1186);
 * cpu/train.zig:261-270 is the weight_decay = 0 case. */
void orc_sgd_step(float *p, const float *g, size_t n, float lr, float weight_decay) {
    for (size_t i = 0; i < n; ++i) {
        float v = p[i];
        if (weight_decay > 0.0f) v = v * (1.0f - lr * weight_decay);
        p[i] = v - lr * g[i];
    }
}

/* trainStep (cpu/train.zig:280-306): forward, MSE, backward, SGD; returns the
 * loss before the update.  `G` receives the gradients. */
float orc_mlp_train_step(float *P, float *G, size_t I, size_t H, size_t O, const float *x,
                         const float *t, float lr) {
    float *buf = (float *)malloc((2 * H + 2 * O + 1) * sizeof(float));
    float *h_pre = buf, *h = buf + H, *y = h + H, *dy = y + O;
    orc_mlp_forward(P, I, H, O, x, h_pre, h, y);
    const float loss = orc_mse_loss(y, t, O);
    orc_mse_loss_grad(dy, y, t, O);
    orc_mlp_backward(P, I, H, O, x, h_pre, h, dy, G);
    orc_sgd_step(P, G, orc_mlp_param_count(I, H, O), lr, 0.0f);
    free(buf);
    return loss;
}

/* Stable softmax cross-entropy gradient of one row, before the 1/N of the
 * batch mean (softmax_ce_loss_grad_batched.comp:30-60): dy = softmax(y) - t. */
void orc_softmax_ce_grad_row(float *dy, const float *y, const float *t, size_t n) {
    float m = y[0];
    for (size_t i = 1; i < n; ++i) m = y[i] > m ? y[i] : m;
    float sum_e = 0;
    for (size_t i = 0; i < n; ++i) sum_e += expf(y[i] - m);
    for (size_t i = 0; i < n; ++i) dy[i] = expf(y[i] - m) / sum_e - t[i];
}

/* Batch loss of the loss-target gate: mlp2_mse_loss_batched.comp (1/2 sum of
 * squares over N x O, / N) and mlp2_ce_loss_batched.comp (-sum t log softmax,
 * / N), sequential fp32 as in the shaders. */
float orc_mlp_batch_loss(const float *P, size_t I, size_t H, size_t O, const float *x,
                         const float *t, size_t N, int cross_entropy) {
    float *buf = (float *)malloc((2 * H + O) * sizeof(float));
    float *h_pre = buf, *h = buf + H, *y = h + H;
    float total = 0;
    for (size_t n = 0; n < N; ++n) {
        orc_mlp_forward(P, I, H, O, x + n * I, h_pre, h, y);
        const float *tn = t + n * O;
        if (!cross_entropy) {
            for (size_t o = 0; o < O; ++o) {
                const float d = y[o] - tn[o];
                total += d * d;
            }
        } else {
            float m = y[0];
            for (size_t o = 1; o < O; ++o) m = y[o] > m ? y[o] : m;
            float sum_e = 0;
            for (size_t o = 0; o < O; ++o) sum_e += expf(y[o] - m);
            const float log_z = m + logf(sum_e);
            for (size_t o = 0; o < O; ++o) total -= tn[o] * (y[o] - log_z);
        }
    }
    free(buf);
    return cross_entropy ? total / (float)N : (total * 0.5f) / (float)N;
}

/* One batched step with the runner's semantics (runner.zig:1053-1220), in
 * the form of the reference's own CPU check (smoke/training.zig:1576-1612,
 * :2066-2101): per-sample gradients summed over the batch, times 1/N, then
 * SGD or Adam (adam_step.comp form, t = the 1-based step) with decoupled
 * weight decay on W1 and W2 only.  G receives the mean gradient; M and V may
 * be NULL for SGD. */
void orc_mlp_batch_step(float *P, float *G, float *M, float *V, size_t I, size_t H, size_t O,
                        const float *x, const float *t, size_t N, int cross_entropy, int adam,
                        float lr, float weight_decay, float beta1, float beta2, float eps,
                        uint32_t t_step) {
    const size_t np = orc_mlp_param_count(I, H, O);
    float *gs = (float *)malloc(np * sizeof(float));
    float *buf = (float *)malloc((2 * H + 2 * O) * sizeof(float));
    float *h_pre = buf, *h = buf + H, *y = h + H, *dy = y + O;
    memset(G, 0, np * sizeof(float));
    for (size_t n = 0; n < N; ++n) {
        orc_mlp_forward(P, I, H, O, x + n * I, h_pre, h, y);
        if (cross_entropy)
            orc_softmax_ce_grad_row(dy, y, t + n * O, O);
        else
            orc_mse_loss_grad(dy, y, t + n * O, O);
        orc_mlp_backward(P, I, H, O, x + n * I, h_pre, h, dy, gs);
        for (size_t k = 0; k < np; ++k) G[k] += gs[k];
    }
    const float inv_n = 1.0f / (float)N;
    for (size_t k = 0; k < np; ++k) G[k] *= inv_n;
    /* spans: W1, b1, W2, b2 */
    const size_t off[5] = {0, H * I, H * I + H, H * I + H + O * H, np};
    for (int s = 0; s < 4; ++s) {
        const size_t a = off[s], n = off[s + 1] - off[s];
        const float wd = (s == 0 || s == 2) ? weight_decay : 0.0f;
        if (adam)
            orc_adam_step(P + a, G + a, M + a, V + a, n, lr, beta1, beta2, eps, t_step, wd);
        else
            orc_sgd_step(P + a, G + a, n, lr, wd);
    }
    free(buf);
    free(gs);
}
