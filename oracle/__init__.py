"""ctypes binding of the C oracle (`oracle/liboracle.so`).

TEST INFRASTRUCTURE ONLY: imported by `tests/`, `__graft_entry__.smoke()` and
the `cpu_baseline` leg of `bench.py`, as the checker.  The product package
`valkyr_amd` never imports this module.

Every function restates a reference CPU oracle from the valkyr tree
(`src/cpu/*.zig`); the C source cites file:line for each.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

F32P = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
U32P = np.ctypeslib.ndpointer(dtype=np.uint32, flags="C_CONTIGUOUS")
U16P = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
SZ = C.c_size_t


def build() -> None:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = C.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


class ModelConfig(C.Structure):
    _fields_ = [
        ("dim", C.c_uint32), ("n_heads", C.c_uint32), ("n_kv_heads", C.c_uint32),
        ("head_dim", C.c_uint32), ("ff_dim", C.c_uint32), ("seq_len", C.c_uint32),
        ("n_seqs", C.c_uint32), ("n_layers", C.c_uint32), ("vocab_size", C.c_uint32),
        ("rms_eps", C.c_float), ("causal", C.c_uint32), ("rotary_dim", C.c_uint32),
        ("rope_theta", C.c_float), ("qk_norm", C.c_uint32), ("lr", C.c_float),
        ("beta1", C.c_float), ("beta2", C.c_float), ("eps_adam", C.c_float),
        ("lora_targets", C.c_uint32), ("lora_rank", C.c_uint32),
        ("lora_alpha", C.c_float), ("lora_lr_b_scale", C.c_float),
        ("tied_embeddings", C.c_uint32), ("bf16_operands", C.c_uint32),
    ]


def _declare(L):
    def d(name, res, *args):
        f = getattr(L, name)
        f.restype = res
        f.argtypes = list(args)

    d("orc_set_threads", None, C.c_int)
    d("orc_get_threads", C.c_int)
    d("orc_fill_normal", None, F32P, SZ, C.c_uint64, C.c_float, C.c_float)
    d("orc_fill_uniform", None, F32P, SZ, C.c_uint64, C.c_float, C.c_float)
    d("orc_fill_ids", None, U32P, SZ, C.c_uint64, C.c_uint32)
    d("orc_f32_to_bf16", C.c_uint16, C.c_float)
    d("orc_bf16_to_f32", C.c_float, C.c_uint16)
    d("orc_round_bf16", None, F32P, SZ)
    d("orc_to_bf16", None, F32P, U16P, SZ)
    d("orc_rmsnorm_forward", None, F32P, F32P, SZ, SZ, C.c_float, C.c_int, F32P)
    d("orc_rmsnorm_backward", None, F32P, F32P, F32P, SZ, SZ, C.c_float, C.c_int, F32P, F32P)
    d("orc_embedding_forward", None, F32P, U32P, SZ, SZ, F32P)
    d("orc_embedding_backward", None, F32P, U32P, SZ, SZ, SZ, F32P)
    d("orc_rope_forward_batched", C.c_int, F32P, F32P, SZ, SZ, SZ, SZ, C.c_float, SZ)
    d("orc_rope_backward_batched", C.c_int, F32P, F32P, SZ, SZ, SZ, SZ, C.c_float, SZ)
    d("orc_attention_forward", None, F32P, F32P, F32P, SZ, SZ, SZ, SZ, SZ, C.c_int,
      F32P, F32P, F32P)
    d("orc_attention_backward", None, F32P, F32P, F32P, F32P, F32P, SZ, SZ, SZ, SZ, SZ,
      F32P, F32P, F32P, F32P)
    d("orc_swiglu_forward", None, F32P, F32P, SZ, F32P)
    d("orc_swiglu_backward", None, F32P, F32P, F32P, SZ, F32P, F32P)
    d("orc_flash_attention_forward", None, F32P, F32P, F32P, SZ, SZ, SZ, SZ, SZ, C.c_int,
      SZ, SZ, F32P, F32P)
    d("orc_flash_attention_backward", None, F32P, F32P, F32P, F32P, F32P, F32P, SZ, SZ,
      SZ, SZ, SZ, C.c_int, F32P, F32P, F32P)
    d("orc_flash_attention_forward_bf16ops", None, F32P, F32P, F32P, SZ, SZ, SZ, SZ, SZ,
      C.c_int, F32P, F32P)
    d("orc_flash_attention_backward_bf16ops", None, F32P, F32P, F32P, F32P, F32P, F32P, SZ, SZ,
      SZ, SZ, SZ, C.c_int, F32P, F32P, F32P)
    d("orc_fa_bw_d", None, F32P, F32P, SZ, SZ, SZ, F32P)
    d("orc_matmul_nt", None, F32P, F32P, F32P, SZ, SZ, SZ)
    d("orc_linear_backward", None, F32P, F32P, F32P, SZ, SZ, SZ, C.c_void_p, C.c_void_p)
    d("orc_cce_forward", C.c_float, F32P, F32P, U32P, SZ, SZ, SZ, SZ, C.c_float, C.c_float,
      F32P, F32P)
    d("orc_cce_backward", None, F32P, F32P, U32P, F32P, SZ, SZ, SZ, SZ, C.c_float,
      C.c_float, F32P, C.c_void_p)
    d("orc_cce_backward_bf16ops", None, F32P, F32P, U32P, F32P, SZ, SZ, SZ, C.c_float,
      C.c_float, F32P, C.c_void_p)
    d("orc_softmax_ce_loss", C.c_float, F32P, U32P, SZ, SZ)
    d("orc_softmax_ce_loss_grad", None, F32P, F32P, U32P, SZ, SZ)
    d("orc_lora_forward", None, F32P, F32P, F32P, F32P, SZ, SZ, SZ, SZ, C.c_float, F32P, F32P)
    d("orc_lora_backward", None, F32P, F32P, F32P, F32P, F32P, F32P, SZ, SZ, SZ, SZ,
      C.c_float, C.c_void_p, F32P, F32P)
    d("orc_adam_step", None, F32P, F32P, F32P, F32P, SZ, C.c_float, C.c_float, C.c_float,
      C.c_float, C.c_uint32, C.c_float)
    d("orc_adam_step_folded", None, F32P, F32P, F32P, F32P, SZ, C.c_float, C.c_float,
      C.c_float, C.c_float, C.c_uint32)
    d("orc_model_create", C.c_void_p, C.POINTER(ModelConfig))
    d("orc_model_destroy", None, C.c_void_p)
    d("orc_model_tensor", C.POINTER(C.c_float), C.c_void_p, C.c_int, C.c_int, C.c_int,
      C.POINTER(C.c_size_t))
    d("orc_model_init_random", None, C.c_void_p, C.c_uint64, C.c_float, C.c_float)
    d("orc_model_forward_backward", C.c_float, C.c_void_p, U32P, U32P)
    d("orc_model_head_forward_backward", C.c_float, C.c_void_p, F32P, U32P, F32P)
    d("orc_model_layer_forward_backward", None, C.c_void_p, C.c_int, F32P, F32P, F32P)
    d("orc_model_embedding_backward", None, C.c_void_p, U32P, F32P)
    d("orc_model_layer_output", None, C.c_void_p, C.c_int, F32P)
    d("orc_model_adam", None, C.c_void_p)
    d("orc_model_step", C.c_float, C.c_void_p, U32P, U32P)
    d("orc_model_step_t", C.c_uint32, C.c_void_p)
    d("orc_model_set_step_t", None, C.c_void_p, C.c_uint32)
    d("orc_model_phase_seconds", None, C.c_void_p, np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS"))
    d("orc_model_reset_phases", None, C.c_void_p)
    d("orc_model_forward_logits", None, C.c_void_p, U32P, F32P)
    d("orc_now_seconds", C.c_double)
    U64P = np.ctypeslib.ndpointer(dtype=np.uint64, flags="C_CONTIGUOUS")
    d("orc_zig_prng_seed", None, U64P, C.c_uint64)
    d("orc_zig_prng_next", C.c_uint64, U64P)
    d("orc_zig_float32", C.c_float, U64P)
    d("orc_splitmix64", C.c_uint64, C.POINTER(C.c_uint64))
    d("orc_mlp_param_count", SZ, SZ, SZ, SZ)
    d("orc_mlp_init", None, F32P, SZ, SZ, SZ, C.c_float, C.c_uint64)
    d("orc_mlp_forward", None, F32P, SZ, SZ, SZ, F32P, F32P, F32P, F32P)
    d("orc_mse_loss", C.c_float, F32P, F32P, SZ)
    d("orc_mse_loss_grad", None, F32P, F32P, F32P, SZ)
    d("orc_mlp_backward", None, F32P, SZ, SZ, SZ, F32P, F32P, F32P, F32P, F32P)
    d("orc_sgd_step", None, F32P, F32P, SZ, C.c_float, C.c_float)
    d("orc_mlp_train_step", C.c_float, F32P, F32P, SZ, SZ, SZ, F32P, F32P, C.c_float)
    d("orc_softmax_ce_grad_row", None, F32P, F32P, F32P, SZ)
    d("orc_mlp_batch_loss", C.c_float, F32P, SZ, SZ, SZ, F32P, F32P, SZ, C.c_int)
    d("orc_mlp_batch_step", None, F32P, F32P, C.c_void_p, C.c_void_p, SZ, SZ, SZ, F32P, F32P,
      SZ, C.c_int, C.c_int, C.c_float, C.c_float, C.c_float, C.c_float, C.c_float, C.c_uint32)


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


# ── array helpers ────────────────────────────────────────────────────────

def set_threads(n: int) -> None:
    """OpenMP threads of the oracle's parallel loops (results are identical
    for every thread count: only independent outputs run in parallel)."""
    lib().orc_set_threads(int(n))


def get_threads() -> int:
    return int(lib().orc_get_threads())


def normal(n, seed, std=1.0, mean=0.0):
    x = np.empty(int(n), np.float32)
    lib().orc_fill_normal(x, x.size, seed, mean, std)
    return x


def uniform(n, seed, lo=-1.0, hi=1.0):
    x = np.empty(int(n), np.float32)
    lib().orc_fill_uniform(x, x.size, seed, lo, hi)
    return x


def ids(n, seed, hi):
    x = np.empty(int(n), np.uint32)
    lib().orc_fill_ids(x, x.size, seed, hi)
    return x


def round_bf16(x):
    y = np.ascontiguousarray(x, np.float32).copy()
    lib().orc_round_bf16(y, y.size)
    return y


def to_bf16_bits(x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_to_bf16(x.reshape(-1), out.reshape(-1), x.size)
    return out


def f32(x):
    return np.ascontiguousarray(x, dtype=np.float32)


# ── primitives ───────────────────────────────────────────────────────────

def rmsnorm_forward(x, w, eps, gemma_quirk=False):
    x, w = f32(x), f32(w)
    y = np.empty_like(x)
    lib().orc_rmsnorm_forward(x.reshape(-1), w, x.size // w.size, w.size, eps, int(gemma_quirk),
                              y.reshape(-1))
    return y


def rmsnorm_backward(dy, x, w, eps, gemma_quirk=False):
    dy, x, w = f32(dy), f32(x), f32(w)
    dx = np.empty_like(x)
    dw = np.zeros_like(w)
    lib().orc_rmsnorm_backward(dy.reshape(-1), x.reshape(-1), w, x.size // w.size, w.size,
                               eps, int(gemma_quirk), dx.reshape(-1), dw)
    return dx, dw


def embedding_forward(embed, tok, dim):
    embed, tok = f32(embed), np.ascontiguousarray(tok, np.uint32)
    out = np.empty(tok.size * dim, np.float32)
    lib().orc_embedding_forward(embed.reshape(-1), tok, tok.size, dim, out)
    return out


def embedding_backward(dy, tok, vocab, dim, dE=None):
    dy, tok = f32(dy), np.ascontiguousarray(tok, np.uint32)
    dE = np.zeros(vocab * dim, np.float32) if dE is None else f32(dE).copy()
    lib().orc_embedding_backward(dy.reshape(-1), tok, tok.size, vocab, dim, dE.reshape(-1))
    return dE


def rope_forward(x, n_rows, n_heads, head_dim, rotary_dim, theta, seq_len=0):
    x = f32(x)
    out = np.empty_like(x)
    rc = lib().orc_rope_forward_batched(out.reshape(-1), x.reshape(-1), n_rows, n_heads,
                                        head_dim, rotary_dim, theta, seq_len)
    if rc != 0:
        raise ValueError(f"rope: error {rc}")
    return out


def rope_backward(dy, n_rows, n_heads, head_dim, rotary_dim, theta, seq_len=0):
    dy = f32(dy)
    out = np.empty_like(dy)
    rc = lib().orc_rope_backward_batched(out.reshape(-1), dy.reshape(-1), n_rows, n_heads,
                                         head_dim, rotary_dim, theta, seq_len)
    if rc != 0:
        raise ValueError(f"rope: error {rc}")
    return out


def attention_forward(Q, K, V, n_q, n_kv, H, Hkv, hd, causal):
    Q, K, V = f32(Q), f32(K), f32(V)
    scores = np.empty(n_q * H * n_kv, np.float32)
    attn = np.empty_like(scores)
    out = np.empty(n_q * H * hd, np.float32)
    lib().orc_attention_forward(Q.reshape(-1), K.reshape(-1), V.reshape(-1), n_q, n_kv, H,
                                Hkv, hd, int(causal), scores, attn, out)
    return out, attn


def attention_backward(dO, Q, K, V, attn, n_q, n_kv, H, Hkv, hd):
    dO, Q, K, V, attn = f32(dO), f32(Q), f32(K), f32(V), f32(attn)
    ds = np.empty(n_q * H * n_kv, np.float32)
    dQ = np.empty(n_q * H * hd, np.float32)
    dK = np.empty(n_kv * Hkv * hd, np.float32)
    dV = np.empty_like(dK)
    lib().orc_attention_backward(dO.reshape(-1), Q.reshape(-1), K.reshape(-1), V.reshape(-1),
                                 attn.reshape(-1), n_q, n_kv, H, Hkv, hd, ds, dQ, dK, dV)
    return dQ, dK, dV


def swiglu_forward(pg, up):
    pg, up = f32(pg), f32(up)
    out = np.empty_like(pg)
    lib().orc_swiglu_forward(pg.reshape(-1), up.reshape(-1), pg.size, out.reshape(-1))
    return out


def swiglu_backward(dg, pg, up):
    dg, pg, up = f32(dg), f32(pg), f32(up)
    dpg, dup = np.empty_like(pg), np.empty_like(pg)
    lib().orc_swiglu_backward(dg.reshape(-1), pg.reshape(-1), up.reshape(-1), pg.size,
                              dpg.reshape(-1), dup.reshape(-1))
    return dpg, dup


def flash_forward(Q, K, V, n_q, n_kv, H, Hkv, hd, causal, Br=16, Bc=16, bf16_ops=False):
    """flash_attn.zig forward; bf16_ops: the MFMA kernels' operand rounding
    (P to bf16 where it multiplies V, 64-key tiles; Br / Bc ignored)."""
    Q, K, V = f32(Q), f32(K), f32(V)
    out = np.empty(n_q * H * hd, np.float32)
    lse = np.empty(n_q * H, np.float32)
    if bf16_ops:
        lib().orc_flash_attention_forward_bf16ops(Q.reshape(-1), K.reshape(-1), V.reshape(-1),
                                                  n_q, n_kv, H, Hkv, hd, int(causal), out, lse)
    else:
        lib().orc_flash_attention_forward(Q.reshape(-1), K.reshape(-1), V.reshape(-1), n_q,
                                          n_kv, H, Hkv, hd, int(causal), Br, Bc, out, lse)
    return out, lse


def flash_backward(Q, K, V, O, dO, lse, n_q, n_kv, H, Hkv, hd, causal, bf16_ops=False):
    """flash_attn.zig backward; bf16_ops: P and the unscaled dS rounded to bf16
    where they meet dO / Q / K, 1/sqrt(d) applied to the accumulated dQ, dK."""
    Q, K, V, O, dO, lse = (f32(a) for a in (Q, K, V, O, dO, lse))
    dQ = np.empty(n_q * H * hd, np.float32)
    dK = np.empty(n_kv * Hkv * hd, np.float32)
    dV = np.empty_like(dK)
    fn = (lib().orc_flash_attention_backward_bf16ops if bf16_ops
          else lib().orc_flash_attention_backward)
    fn(Q.reshape(-1), K.reshape(-1), V.reshape(-1), O.reshape(-1), dO.reshape(-1),
       lse.reshape(-1), n_q, n_kv, H, Hkv, hd, int(causal), dQ, dK, dV)
    return dQ, dK, dV


def fa_bw_d(O, dO, n_q, H, hd):
    O, dO = f32(O), f32(dO)
    D = np.empty(n_q * H, np.float32)
    lib().orc_fa_bw_d(O.reshape(-1), dO.reshape(-1), n_q, H, hd, D)
    return D


def matmul_nt(x, W, M, N, K):
    x, W = f32(x), f32(W)
    out = np.empty(M * N, np.float32)
    lib().orc_matmul_nt(out, x.reshape(-1), W.reshape(-1), M, N, K)
    return out


def linear_backward(dout, x, W, M, N, K, want_dx=True, want_dw=True):
    dout, x, W = f32(dout), f32(x), f32(W)
    dx = np.empty(M * K, np.float32) if want_dx else None
    dW = np.zeros(N * K, np.float32) if want_dw else None
    lib().orc_linear_backward(dout.reshape(-1), x.reshape(-1), W.reshape(-1), M, N, K,
                              _ptr(dx), _ptr(dW))
    return dx, dW


def cce_forward(h, w, tgt, n, vocab, dim, chunk=1024, z_loss=0.0, ls=0.0):
    h, w = f32(h), f32(w)
    tgt = np.ascontiguousarray(tgt, np.uint32)
    lse = np.empty(n, np.float32)
    loss_row = np.empty(n, np.float32)
    loss = lib().orc_cce_forward(h.reshape(-1), w.reshape(-1), tgt, n, vocab, dim,
                                 min(chunk, vocab), z_loss, ls, lse, loss_row)
    return loss, lse, loss_row


def cce_backward(h, w, tgt, lse, n, vocab, dim, chunk=1024, z_loss=0.0, ls=0.0, want_dw=True,
                 bf16_ops=False):
    """cce.zig backward; bf16_ops: dz rounded to bf16 before both products."""
    h, w, lse = f32(h), f32(w), f32(lse)
    tgt = np.ascontiguousarray(tgt, np.uint32)
    dh = np.empty(n * dim, np.float32)
    dW = np.zeros(vocab * dim, np.float32) if want_dw else None
    if bf16_ops:
        lib().orc_cce_backward_bf16ops(h.reshape(-1), w.reshape(-1), tgt, lse, n, vocab, dim,
                                       z_loss, ls, dh, _ptr(dW))
    else:
        lib().orc_cce_backward(h.reshape(-1), w.reshape(-1), tgt, lse, n, vocab, dim,
                               min(chunk, vocab), z_loss, ls, dh, _ptr(dW))
    return dh, dW


def softmax_ce_loss(logits, tgt, n, vocab):
    return lib().orc_softmax_ce_loss(f32(logits).reshape(-1), np.ascontiguousarray(tgt, np.uint32),
                                     n, vocab)


def softmax_ce_loss_grad(logits, tgt, n, vocab):
    d = np.empty(n * vocab, np.float32)
    lib().orc_softmax_ce_loss_grad(d, f32(logits).reshape(-1), np.ascontiguousarray(tgt, np.uint32),
                                   n, vocab)
    return d


def lora_forward(x, w, a, b, M, N, K, r, aor):
    x, w, a, b = f32(x), f32(w), f32(a), f32(b)
    y = np.empty(M * N, np.float32)
    inter = np.empty(M * r, np.float32)
    lib().orc_lora_forward(x.reshape(-1), w.reshape(-1), a.reshape(-1), b.reshape(-1), M, N,
                           K, r, aor, y, inter)
    return y, inter


def lora_backward(dy, x, w, a, b, inter, M, N, K, r, aor, want_dx=True, dA=None, dB=None):
    dy, x, w, a, b, inter = (f32(t) for t in (dy, x, w, a, b, inter))
    dx = np.empty(M * K, np.float32) if want_dx else None
    dA = np.zeros(r * K, np.float32) if dA is None else f32(dA).copy()
    dB = np.zeros(N * r, np.float32) if dB is None else f32(dB).copy()
    lib().orc_lora_backward(dy.reshape(-1), x.reshape(-1), w.reshape(-1), a.reshape(-1),
                            b.reshape(-1), inter.reshape(-1), M, N, K, r, aor, _ptr(dx), dA, dB)
    return dx, dA, dB


def adam_step(p, g, m, v, lr, b1, b2, eps, t, wd=0.0):
    """In place on p, m, v (float32 arrays)."""
    lib().orc_adam_step(p.reshape(-1), f32(g).reshape(-1), m.reshape(-1), v.reshape(-1), p.size,
                        lr, b1, b2, eps, t, wd)


def adam_step_folded(p, g, m, v, lr, b1, b2, eps, t):
    lib().orc_adam_step_folded(p.reshape(-1), f32(g).reshape(-1), m.reshape(-1),
                               v.reshape(-1), p.size, lr, b1, b2, eps, t)


def now():
    return lib().orc_now_seconds()


# ── whole model ──────────────────────────────────────────────────────────

class Model:
    """Oracle model with the GPU Runner's step semantics (see oracle.c)."""

    PARAM, GRAD, M, V = 0, 1, 2, 3

    def __init__(self, **cfg):
        self.cfg = ModelConfig(**cfg)
        self._h = lib().orc_model_create(C.byref(self.cfg))
        c = self.cfg
        self.T = c.seq_len * max(1, c.n_seqs)

    def __del__(self):
        if getattr(self, "_h", None):
            lib().orc_model_destroy(self._h)
            self._h = None

    def tensor(self, kind, layer, which):
        n = C.c_size_t(0)
        p = lib().orc_model_tensor(self._h, kind, layer, which, C.byref(n))
        if not p or n.value == 0:
            return None
        return np.ctypeslib.as_array(p, shape=(n.value,))

    def init_random(self, seed, std=0.02, lora_std=0.02):
        lib().orc_model_init_random(self._h, seed, std, lora_std)

    def forward_backward(self, tokens, targets):
        return lib().orc_model_forward_backward(self._h, np.ascontiguousarray(tokens, np.uint32),
                                                np.ascontiguousarray(targets, np.uint32))

    # the stages of forward_backward on given inputs (stage-by-stage checks)
    def head_forward_backward(self, y, targets):
        """Final norm + CE + their backward from the last layer's output y:
        returns (loss, gradient at y); writes the final-norm gain and lm_head
        gradients (tied: kept for embedding_backward)."""
        y = np.ascontiguousarray(y, np.float32).ravel()
        d_y = np.empty_like(y)
        loss = lib().orc_model_head_forward_backward(
            self._h, y, np.ascontiguousarray(targets, np.uint32), d_y)
        return loss, d_y

    def layer_forward_backward(self, l, x_in, d_y):
        """Layer l's forward from x_in and backward from the gradient d_y at
        its output: writes its gradients, returns the gradient at x_in."""
        x_in = np.ascontiguousarray(x_in, np.float32).ravel()
        d_x = np.empty_like(x_in)
        lib().orc_model_layer_forward_backward(self._h, int(l), x_in,
                                               np.ascontiguousarray(d_y, np.float32).ravel(), d_x)
        return d_x

    def layer_output(self, l):
        """Layer l's output from the last forward (l = -1: the embedding output)."""
        out = np.empty(self.T * self.cfg.dim, np.float32)
        lib().orc_model_layer_output(self._h, int(l), out)
        return out

    def embedding_backward(self, tokens, d_x0):
        lib().orc_model_embedding_backward(self._h, np.ascontiguousarray(tokens, np.uint32),
                                           np.ascontiguousarray(d_x0, np.float32).ravel())

    def adam(self):
        lib().orc_model_adam(self._h)

    def step(self, tokens, targets):
        return lib().orc_model_step(self._h, np.ascontiguousarray(tokens, np.uint32),
                                    np.ascontiguousarray(targets, np.uint32))

    @property
    def step_t(self):
        return lib().orc_model_step_t(self._h)

    @step_t.setter
    def step_t(self, t):
        lib().orc_model_set_step_t(self._h, int(t))

    PHASES = ("layer_fwd", "layer_bwd", "attn_fwd", "attn_bwd", "head", "adam")

    def phase_seconds(self):
        """Wall seconds per phase since the last reset_phases(): layer forwards
        and backwards (attention included), the attention inside them, the head
        (embedding, final norm, CCE, tied sum) and Adam."""
        out = np.zeros(len(self.PHASES), np.float64)
        lib().orc_model_phase_seconds(self._h, out)
        return dict(zip(self.PHASES, out.tolist()))

    def reset_phases(self):
        lib().orc_model_reset_phases(self._h)

    def forward_logits(self, tokens):
        out = np.empty(self.T * self.cfg.vocab_size, np.float32)
        lib().orc_model_forward_logits(self._h, np.ascontiguousarray(tokens, np.uint32), out)
        return out


# ── tiny-MLP TrainingRunner (cpu/train.zig; runner.zig batched semantics) ──

def splitmix64_stream(seed, n):
    st = C.c_uint64(seed)
    return [lib().orc_splitmix64(C.byref(st)) for _ in range(n)]


class ZigPrng:
    """std.Random.DefaultPrng (xoshiro256++ seeded by SplitMix64)."""

    def __init__(self, seed=None, state=None):
        self.s = np.zeros(4, np.uint64)
        if state is not None:
            self.s[:] = np.asarray(state, np.uint64)
        else:
            lib().orc_zig_prng_seed(self.s, seed)

    def next(self):
        return int(lib().orc_zig_prng_next(self.s))

    def float32(self):
        return np.float32(lib().orc_zig_float32(self.s))


class Mlp:
    """Parameter blob [W1 (H x I) | b1 | W2 (O x H) | b2] plus its views."""

    def __init__(self, dim_in, dim_hidden, dim_out, init_scale=0.3, seed=0xCAFE, params=None):
        self.I, self.H, self.O = dim_in, dim_hidden, dim_out
        self.n = int(lib().orc_mlp_param_count(self.I, self.H, self.O))
        if params is None:
            self.P = np.empty(self.n, np.float32)
            lib().orc_mlp_init(self.P, self.I, self.H, self.O, init_scale, seed)
        else:
            self.P = f32(params).reshape(-1).copy()
            assert self.P.size == self.n
        self.G = np.zeros(self.n, np.float32)
        self.M = np.zeros(self.n, np.float32)
        self.V = np.zeros(self.n, np.float32)

    def spans(self):
        I, H, O = self.I, self.H, self.O
        o = np.cumsum([0, H * I, H, O * H, O])
        return {k: slice(o[i], o[i + 1]) for i, k in enumerate(("w1", "b1", "w2", "b2"))}

    def view(self, name, which="P"):
        return getattr(self, which)[self.spans()[name]]

    def forward(self, x):
        x = f32(x).reshape(-1)
        hp, h, y = (np.empty(self.H, np.float32), np.empty(self.H, np.float32),
                    np.empty(self.O, np.float32))
        lib().orc_mlp_forward(self.P, self.I, self.H, self.O, x, hp, h, y)
        return hp, h, y

    def backward(self, x, h_pre, h, dy):
        lib().orc_mlp_backward(self.P, self.I, self.H, self.O, f32(x).reshape(-1), f32(h_pre),
                               f32(h), f32(dy), self.G)
        return self.G

    def train_step(self, x, t, lr):
        return lib().orc_mlp_train_step(self.P, self.G, self.I, self.H, self.O,
                                        f32(x).reshape(-1), f32(t).reshape(-1), lr)

    def batch_loss(self, x, t, n, cross_entropy=False):
        return lib().orc_mlp_batch_loss(self.P, self.I, self.H, self.O, f32(x).reshape(-1),
                                        f32(t).reshape(-1), n, int(cross_entropy))

    def batch_step(self, x, t, n, lr, cross_entropy=False, adam=False, weight_decay=0.0,
                   beta1=0.9, beta2=0.999, eps=1e-8, t_step=1):
        lib().orc_mlp_batch_step(self.P, self.G, _ptr(self.M), _ptr(self.V), self.I, self.H,
                                 self.O, f32(x).reshape(-1), f32(t).reshape(-1), n,
                                 int(cross_entropy), int(adam), lr, weight_decay, beta1, beta2,
                                 eps, t_step)


def mse_loss(y, t):
    y, t = f32(y).reshape(-1), f32(t).reshape(-1)
    return lib().orc_mse_loss(y, t, y.size)


def softmax_ce_grad_row(y, t):
    y, t = f32(y).reshape(-1), f32(t).reshape(-1)
    d = np.empty_like(y)
    lib().orc_softmax_ce_grad_row(d, y, t, y.size)
    return d


def sgd_step(p, g, lr, wd=0.0):
    lib().orc_sgd_step(p.reshape(-1), f32(g).reshape(-1), p.size, lr, wd)
