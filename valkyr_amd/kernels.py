"""Python mirror of the reference's per-kernel dispatches.

Each function takes `DeviceBuffer`s (or raw device addresses) and the fields
of the reference push-constant struct it replaces (runtime.zig push ABI),
and enqueues the gfx950 kernel through the C ABI.  Nothing here computes on
the host.
"""
from __future__ import annotations

import ctypes as C
import math

from ._lib import AttnParams, CceParams, LoraAdapter, RopeParams, check, lib

F32, BF16 = 0, 1
PRECISION_FP32, PRECISION_BF16 = 0, 1


def _p(x):
    if x is None:
        return None
    if isinstance(x, C.c_void_p):
        return x
    if isinstance(x, int):
        return C.c_void_p(x)
    return x.ptr


def _s(stream):
    return stream.handle if stream is not None else None


def attn_params(n_q, n_kv, n_heads, n_kv_heads, head_dim, causal=True, n_batch=1, dtype=F32,
                inv_sqrt_dim=None):
    """FaForwardPush / FaBwDqPush / FaBwDkvPush (runtime.zig:377-416) + n_batch."""
    return AttnParams(n_batch, n_q, n_kv, n_heads, n_kv_heads, head_dim, 1 if causal else 0,
                      inv_sqrt_dim if inv_sqrt_dim is not None else 1.0 / math.sqrt(head_dim), dtype)


def fa_forward(p, q, k, v, o, lse=None, stream=None):
    check(lib().vkh_fa_forward(C.byref(p), _p(q), _p(k), _p(v), _p(o), _p(lse), _s(stream)))


def fa_bw_d(p, o, dout, d, dout_bf16=None, stream=None):
    check(lib().vkh_fa_bw_d(C.byref(p), _p(o), _p(dout), _p(d), _p(dout_bf16), _s(stream)))


def fa_bw_d_bf16(p, o16, dout16, d, stream=None):
    """D = rowsum(O dO) with O and dO stored in bf16."""
    check(lib().vkh_fa_bw_d_bf16(C.byref(p), _p(o16), _p(dout16), _p(d), _s(stream)))


def fa_bw_dq(p, q, k, v, dout, lse, d, dq, stream=None):
    check(lib().vkh_fa_bw_dq(C.byref(p), _p(q), _p(k), _p(v), _p(dout), _p(lse), _p(d), _p(dq),
                             _s(stream)))


def fa_bw_dkv(p, q, k, v, dout, lse, d, dk, dv, stream=None):
    check(lib().vkh_fa_bw_dkv(C.byref(p), _p(q), _p(k), _p(v), _p(dout), _p(lse), _p(d), _p(dk),
                              _p(dv), _s(stream)))


def fa_backward_workspace_bytes(p):
    return lib().vkh_fa_backward_workspace_bytes(C.byref(p))


def fa_backward(p, q, k, v, dout, lse, d, dq, dk, dv, workspace=None, stream=None):
    """dK, dV and dQ of one attention call (after fa_bw_d); bf16 shapes take
    the fused dS path (workspace of fa_backward_workspace_bytes(p) bytes, or
    None to allocate per call)."""
    check(lib().vkh_fa_backward(C.byref(p), _p(q), _p(k), _p(v), _p(dout), _p(lse), _p(d),
                                _p(dq), _p(dk), _p(dv), _p(workspace), _s(stream)))


def fa_backward_from_o(p, q, k, v, o16, dout16, lse, d, dq, dk, dv, workspace=None, stream=None):
    """D = rowsum(O dO) (written to d) and dK, dV, dQ from bf16 O and dO in one
    call; on the recompute path the dQ kernel forms D itself."""
    check(lib().vkh_fa_backward_from_o(C.byref(p), _p(q), _p(k), _p(v), _p(o16), _p(dout16),
                                       _p(lse), _p(d), _p(dq), _p(dk), _p(dv), _p(workspace),
                                       _s(stream)))


def matmul_nt(x, w, y, M, N, K, precision=PRECISION_FP32, stream=None):
    """matmul_nt_v2.comp: y[M,N] = x[M,K] w[N,K]^T."""
    check(lib().vkh_matmul_nt(_p(x), _p(w), _p(y), M, N, K, precision, _s(stream)))


def linear_backward_dx(dy, w, dx, M, N, K, precision=PRECISION_FP32, stream=None):
    check(lib().vkh_linear_backward_dx(_p(dy), _p(w), _p(dx), M, N, K, precision, _s(stream)))


def linear_backward_dw(dy, x, dw, M, N, K, precision=PRECISION_FP32, stream=None):
    check(lib().vkh_linear_backward_dw(_p(dy), _p(x), _p(dw), M, N, K, precision, _s(stream)))


def matmul_nt_bf16(x, w, y, M, N, K, stream=None):
    """y[M,N] = x[M,K] w[N,K]^T on bf16 operands (the bf16 training step's GEMM)."""
    check(lib().vkh_matmul_nt_bf16(_p(x), _p(w), _p(y), M, N, K, _s(stream)))


def gate_up_swiglu_bf16(x, w_gu, gu, gated, M, F, K, stream=None):
    """gu[M, 2F] = x w_gu^T and gated[M, F] = bf16 SwiGLU of its halves (bf16 operands)."""
    check(lib().vkh_gate_up_swiglu_bf16(_p(x), _p(w_gu), _p(gu), _p(gated), M, F, K, _s(stream)))


def qkv_project_bf16(p, K, eps, qk_norm, x, w, wq, wk, y, out, fused=True, stream=None):
    """y = x w^T (q|k|v, bf16 operands) and the bf16 attention operand out (Q/K-RMSNorm +
    RoPE of the q and k heads); fused=False forces the two passes."""
    check(lib().vkh_qkv_project_bf16(C.byref(p), K, eps, 1 if qk_norm else 0, _p(x), _p(w), _p(wq),
                                     _p(wk), _p(y), _p(out), 1 if fused else 0, _s(stream)))


def qkv_project(p, K, eps, qk_norm, x, w, wq, wk, y, out, fused=True, stream=None):
    """The fp32 form of qkv_project_bf16 (fp32 x, w and out)."""
    check(lib().vkh_qkv_project(C.byref(p), K, eps, 1 if qk_norm else 0, _p(x), _p(w), _p(wq),
                                _p(wk), _p(y), _p(out), 1 if fused else 0, _s(stream)))


def gate_up_swiglu(x, w_gu, gu, gated, M, F, K, fused=True, stream=None):
    """The fp32 form of gate_up_swiglu_bf16 (fp32 operands and gated)."""
    check(lib().vkh_gate_up_swiglu(_p(x), _p(w_gu), _p(gu), _p(gated), M, F, K, 1 if fused else 0,
                                   _s(stream)))


def linear_backward_dx_bf16(dy, w, dx, M, N, K, stream=None):
    """dx[M,K] = dy[M,N] w[N,K] on bf16 operands."""
    check(lib().vkh_linear_backward_dx_bf16(_p(dy), _p(w), _p(dx), M, N, K, _s(stream)))


def linear_backward_dw_bf16(dy, x, dw, M, N, K, stream=None):
    """dw[N,K] = dy[M,N]^T x[M,K] on bf16 operands."""
    check(lib().vkh_linear_backward_dw_bf16(_p(dy), _p(x), _p(dw), M, N, K, _s(stream)))


def lora_forward(x, w, a, b, y, inter, M, N, K, r, alpha_over_r, precision=PRECISION_FP32,
                 stream=None):
    check(lib().vkh_lora_forward(_p(x), _p(w), _p(a), _p(b), _p(y), _p(inter), M, N, K, r,
                                 alpha_over_r, precision, _s(stream)))


def lora_backward(dy, x, w, a, b, inter, dx, dA, dB, M, N, K, r, alpha_over_r,
                  precision=PRECISION_FP32, stream=None):
    check(lib().vkh_lora_backward(_p(dy), _p(x), _p(w), _p(a), _p(b), _p(inter), _p(dx), _p(dA),
                                  _p(dB), M, N, K, r, alpha_over_r, precision, _s(stream)))


def lora_adapters(specs):
    """ctypes array of vkh_lora_adapter from dicts with keys col, n, k, a, b,
    inter, dyb, da, db (buffers or None)."""
    def addr(x):
        p = _p(x)
        return None if p is None else p.value

    arr = (LoraAdapter * len(specs))()
    for i, d in enumerate(specs):
        arr[i] = LoraAdapter(d["col"], d["n"], d["k"],
                             *(addr(d.get(f)) for f in ("a", "b", "inter", "dyb", "da", "db")))
    return arr


def lora_group_forward_bf16(x16, ldx, T, r, aor, adapters, y, ldy, stream=None):
    """The training step's grouped rank-r forward on a bf16 activation:
    inter = x A^T and y[:, col:col+n] += aor inter B^T for each adapter."""
    check(lib().vkh_lora_group_forward_bf16(_p(x16), ldx, T, r, aor, adapters, len(adapters),
                                            _p(y), ldy, _s(stream)))


def lora_group_backward_bf16(dy16, lddy, x16, ldx, T, r, aor, adapters, dx=None, lddx=0,
                             stream=None):
    """The grouped rank-r backward on bf16 dy and x: dyb = dy B, dA, dB and
    dx += aor dyb A."""
    check(lib().vkh_lora_group_backward_bf16(_p(dy16), lddy, _p(x16), ldx, T, r, aor, adapters,
                                             len(adapters), _p(dx), lddx, _s(stream)))


def cce_params(n, vocab, dim, z_loss_scale=0.0, label_smoothing=0.0, precision=PRECISION_FP32):
    return CceParams(n, vocab, dim, z_loss_scale, label_smoothing, precision)


def cce_forward(p, h, w, targets, lse, loss_row=None, loss_mean=None, stream=None):
    check(lib().vkh_cce_forward(C.byref(p), _p(h), _p(w), _p(targets), _p(lse), _p(loss_row),
                                _p(loss_mean), _s(stream)))


def cce_backward(p, h, w, targets, lse, dh=None, dw=None, accumulate_dw=False, stream=None):
    check(lib().vkh_cce_backward(C.byref(p), _p(h), _p(w), _p(targets), _p(lse), _p(dh), _p(dw),
                                 1 if accumulate_dw else 0, _s(stream)))


def rmsnorm_forward(x, w, y, n_rows, dim, eps, gemma_quirk=False, stream=None):
    check(lib().vkh_rmsnorm_forward(_p(x), _p(w), _p(y), n_rows, dim, eps, int(gemma_quirk),
                                    _s(stream)))


def rmsnorm_backward(dy, x, w, dx, dw=None, n_rows=0, dim=0, eps=1e-6, gemma_quirk=False,
                     residual=None, stream=None):
    check(lib().vkh_rmsnorm_backward(_p(dy), _p(x), _p(w), _p(dx), _p(residual), _p(dw), n_rows,
                                     dim, eps, int(gemma_quirk), _s(stream)))


def rmsnorm_backward_noalloc(dy, x, w, dx, dw=None, n_rows=0, dim=0, eps=1e-6,
                             gemma_quirk=False, residual=None, stream=None):
    """vkh_rmsnorm_backward with the gain partials in the library's fixed
    per-device array: no allocation; calls on one GPU must not overlap."""
    check(lib().vkh_rmsnorm_backward_noalloc(_p(dy), _p(x), _p(w), _p(dx), _p(residual), _p(dw),
                                             n_rows, dim, eps, int(gemma_quirk), _s(stream)))


def swiglu_forward(pre_gate, up, gated, n, stream=None):
    check(lib().vkh_swiglu_forward(_p(pre_gate), _p(up), _p(gated), n, _s(stream)))


def swiglu_backward(d_gated, pre_gate, up, d_pre_gate, d_up, n, stream=None):
    check(lib().vkh_swiglu_backward(_p(d_gated), _p(pre_gate), _p(up), _p(d_pre_gate), _p(d_up), n,
                                    _s(stream)))


def rope_params(n_pos, n_q_heads, n_kv_heads, head_dim, rotary_dim, theta_base, seq_len=0):
    """QkRopeBatchedPush (runtime.zig:221-228) + seq_len."""
    return RopeParams(n_pos, n_q_heads, n_kv_heads, head_dim, rotary_dim, theta_base, seq_len)


def qk_rope_forward(p, q_in, q_out, k_in, k_out, stream=None):
    check(lib().vkh_qk_rope_forward(C.byref(p), _p(q_in), _p(q_out), _p(k_in), _p(k_out), _s(stream)))


def qk_rope_backward(p, dq_out, dq_in, dk_out, dk_in, stream=None):
    check(lib().vkh_qk_rope_backward(C.byref(p), _p(dq_out), _p(dq_in), _p(dk_out), _p(dk_in),
                                     _s(stream)))


def embed_lookup(embed, ids, out, n_pos, dim, scale=1.0, stream=None):
    check(lib().vkh_embed_lookup(_p(embed), _p(ids), _p(out), n_pos, dim, scale, _s(stream)))


def embedding_backward(dy, ids, dE, n_pos, dim, vocab, stream=None):
    check(lib().vkh_embedding_backward(_p(dy), _p(ids), _p(dE), n_pos, dim, vocab, _s(stream)))


def adam_step(param, grad, m, v, n, lr, beta1, beta2, eps, t, weight_decay=0.0, stream=None):
    check(lib().vkh_adam_step(_p(param), _p(grad), _p(m), _p(v), n, lr, beta1, beta2, eps, t,
                              weight_decay, _s(stream)))


def add_in_place(dst, src, n, stream=None):
    check(lib().vkh_add_in_place(_p(dst), _p(src), n, _s(stream)))


def vec_add(a, b, c, n, stream=None):
    check(lib().vkh_vec_add(_p(a), _p(b), _p(c), n, _s(stream)))


def scale(x, out, n, s, stream=None):
    check(lib().vkh_scale(_p(x), _p(out), n, s, _s(stream)))


def cast_f32_to_bf16(x, out, n, stream=None):
    check(lib().vkh_cast_f32_to_bf16(_p(x), _p(out), n, _s(stream)))
