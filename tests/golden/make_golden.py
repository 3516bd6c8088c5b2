"""Writes the golden fixtures of this directory (run from the repository root:
`python tests/golden/make_golden.py`).

The reference commits no golden vectors for the training path: its tests
generate inputs at run time from Zig's PRNG and compare the GPU against its
CPU oracle (src/cpu/*.zig).  The fixtures here are therefore of two kinds:

* known answers that need no oracle: the duplicated-id embedding scatter of
  gpu_train.zig:4855-4884 (ids {3, 7, 3, 11, 7, 3}) with dyadic dy values, so
  the expected sums are exact and are formed here by a plain loop;
* outputs of the C oracle (oracle/oracle.c, itself pinned by
  tests/test_oracle.py against closed forms, finite differences and the
  reference's own test cases) on small seeded inputs, frozen so that the GPU
  tests have fixed expected values and the oracle cannot drift unnoticed.

Every file is a plain .npz (no pickled objects); `meta` holds a JSON string.
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle as O  # noqa: E402  (test infrastructure: the checker)


def save(name, meta, **arrays):
    path = os.path.join(HERE, name)
    np.savez_compressed(path, meta=np.array(json.dumps(meta, sort_keys=True)), **arrays)
    print(f"{name}: {os.path.getsize(path)} bytes")


# ── embedding backward: duplicated ids (gpu_train.zig:4855-4884) ─────────

def kat_embedding():
    ids = np.array([3, 7, 3, 11, 7, 3], np.uint32)
    V, D = 16, 5
    # dy[p][j] = (p + 1) + j / 8: dyadic, every partial sum exact in fp32
    dy = np.array([[(p + 1) + j / 8 for j in range(D)] for p in range(len(ids))], np.float32)
    dE = np.zeros((V, D), np.float32)
    for p, t in enumerate(ids):  # position order, as embedding_backward.comp sums
        for j in range(D):
            dE[t, j] = np.float32(dE[t, j] + dy[p, j])
    save("kat_embedding_dup_ids.npz", {"V": V, "D": D, "source": "gpu_train.zig:4855-4884"},
         ids=ids, dy=dy.ravel(), dE=dE.ravel())


# ── FlashAttention fwd + bwd ─────────────────────────────────────────────

FA_CASES = {  # name: (B, n_q, n_kv, H, Hkv, hd, causal, bf16 inputs)
    "ref_4x4": (1, 4, 4, 4, 2, 16, 1, False),        # smoke/cpu.zig:909-916 shapes
    "ref_10x12": (1, 10, 12, 4, 2, 16, 1, False),
    "ref_noncausal": (1, 4, 8, 4, 2, 16, 0, False),
    "bf16_64": (2, 64, 64, 4, 2, 64, 1, True),       # fused MFMA backward shape
}


def fa():
    arrays, meta = {}, {}
    for i, (name, (B, n_q, n_kv, H, Hkv, hd, causal, bf)) in enumerate(FA_CASES.items()):
        gen = O.normal if bf else (lambda n, s, std=1.0: O.uniform(n, s, -0.5 * std, 0.5 * std))
        Q = gen(B * n_q * H * hd, 700 + 10 * i)
        K = gen(B * n_kv * Hkv * hd, 701 + 10 * i)
        V = gen(B * n_kv * Hkv * hd, 702 + 10 * i)
        dO = gen(B * n_q * H * hd, 703 + 10 * i, 0.1 if bf else 1.0)
        if bf:
            Q, K, V, dO = (O.round_bf16(x) for x in (Q, K, V, dO))
        outs = {k: [] for k in ("O", "lse", "D", "dQ", "dK", "dV")}
        for b in range(B):
            sq = slice(b * n_q * H * hd, (b + 1) * n_q * H * hd)
            sk = slice(b * n_kv * Hkv * hd, (b + 1) * n_kv * Hkv * hd)
            o, lse = O.flash_forward(Q[sq], K[sk], V[sk], n_q, n_kv, H, Hkv, hd, causal)
            dq, dk, dv = O.flash_backward(Q[sq], K[sk], V[sk], o, dO[sq], lse, n_q, n_kv, H, Hkv,
                                          hd, causal)
            d = O.fa_bw_d(o, dO[sq], n_q, H, hd)
            for k, x in zip(outs, (o, lse, d, dq, dk, dv)):
                outs[k].append(x)
        for k, x in (("Q", Q), ("K", K), ("V", V), ("dO", dO)):
            arrays[f"{name}_{k}"] = x
        for k, xs in outs.items():
            arrays[f"{name}_{k}"] = np.concatenate(xs)
        meta[name] = dict(B=B, n_q=n_q, n_kv=n_kv, H=H, Hkv=Hkv, hd=hd, causal=causal, bf16=bf)
    save("fa.npz", meta, **arrays)


# ── cut cross-entropy ────────────────────────────────────────────────────

def cce():
    n, V, D, zl, ls = 32, 512, 64, 1e-4, 0.1
    h = O.round_bf16(O.normal(n * D, 801))  # bf16-representable: same operands for both precisions
    w = O.round_bf16(O.normal(V * D, 802, 0.05))
    t = O.ids(n, 803, V)
    loss, lse, row = O.cce_forward(h, w, t, n, V, D, 128, zl, ls)
    dh, dW = O.cce_backward(h, w, t, lse, n, V, D, 128, zl, ls)
    save("cce.npz", dict(n=n, V=V, D=D, z_loss=zl, label_smoothing=ls, chunk=128),
         h=h, w=w, targets=t, loss=np.float32(loss), lse=lse, loss_row=row, dh=dh, dW=dW)


# ── bandwidth kernels and GEMMs ──────────────────────────────────────────

def ops():
    a = {}
    rows, dim, eps = 8, 64, 1e-6
    x, w, dy = O.normal(rows * dim, 901), O.uniform(dim, 902, 0.5, 1.5), O.normal(rows * dim, 903)
    dx, dw = O.rmsnorm_backward(dy, x, w, eps)
    a.update(rms_x=x, rms_w=w, rms_dy=dy, rms_y=O.rmsnorm_forward(x, w, eps), rms_dx=dx,
             rms_dw=dw)

    n = 256
    z, u, dg = O.normal(n, 911, 2.0), O.normal(n, 912), O.normal(n, 913)
    dz, du = O.swiglu_backward(dg, z, u)
    a.update(sw_z=z, sw_u=u, sw_dg=dg, sw_g=O.swiglu_forward(z, u), sw_dz=dz, sw_du=du)

    S, B, Hq, Hkv, hd, theta = 8, 2, 2, 1, 16, 1e6
    q, k = O.normal(S * B * Hq * hd, 921), O.normal(S * B * Hkv * hd, 922)
    a.update(rope_q=q, rope_k=k)
    for rot in (16, 8):
        a[f"rope{rot}_q_out"] = O.rope_forward(q, S * B, Hq, hd, rot, theta, S)
        a[f"rope{rot}_k_out"] = O.rope_forward(k, S * B, Hkv, hd, rot, theta, S)
        a[f"rope{rot}_dq_in"] = O.rope_backward(q, S * B, Hq, hd, rot, theta, S)
        a[f"rope{rot}_dk_in"] = O.rope_backward(k, S * B, Hkv, hd, rot, theta, S)

    na = 64
    p, g = O.normal(na, 931), O.normal(na, 932, 1e-2)
    m, v = O.normal(na, 933, 1e-3), np.abs(O.normal(na, 934, 1e-5))
    a.update(adam_p0=p.copy(), adam_g=g, adam_m0=m.copy(), adam_v0=v.copy())
    for t in (1, 2, 3):
        O.adam_step(p, g, m, v, 1e-3, 0.9, 0.999, 1e-8, t)
    a.update(adam_p3=p, adam_m3=m, adam_v3=v)

    M, N, K = 16, 24, 32
    xm, W, dym = O.normal(M * K, 941), O.normal(N * K, 942), O.normal(M * N, 943)
    dxm, dWm = O.linear_backward(dym, xm, W, M, N, K)
    a.update(lin_x=xm, lin_w=W, lin_dy=dym, lin_y=O.matmul_nt(xm, W, M, N, K), lin_dx=dxm,
             lin_dw=dWm)
    save("ops.npz", dict(rms=dict(rows=rows, dim=dim, eps=eps), swiglu=dict(n=n),
                         rope=dict(S=S, B=B, Hq=Hq, Hkv=Hkv, hd=hd, theta=theta),
                         adam=dict(n=na, lr=1e-3, b1=0.9, b2=0.999, eps=1e-8, t=[1, 2, 3]),
                         linear=dict(M=M, N=N, K=K)), **a)


# ── one whole training step ──────────────────────────────────────────────

STEP_CFG = dict(dim=32, n_heads=2, n_kv_heads=1, head_dim=16, ff_dim=64, seq_len=16, n_seqs=2,
                n_layers=2, vocab_size=256, rms_eps=1e-6, causal=1, rotary_dim=16,
                rope_theta=1e6, qk_norm=1, lr=1e-3, beta1=0.9, beta2=0.999, eps_adam=1e-8,
                lora_targets=0, lora_rank=0, lora_alpha=0.0, lora_lr_b_scale=1.0,
                tied_embeddings=0, bf16_operands=0)


def step_keys(cfg):
    """(layer, which) of every trainable tensor in collectBlobs order."""
    keys = [(-1, 0), (-1, 1)] + ([] if cfg["tied_embeddings"] else [(-1, 2)])
    for l in range(cfg["n_layers"]):
        keys += [(l, w) for w in range(9)]
        if cfg["qk_norm"]:
            keys += [(l, 9), (l, 10)]
    return keys


def step():
    cfg = STEP_CFG
    m = O.Model(**cfg)
    m.init_random(1001, std=0.05)
    keys = step_keys(cfg)
    T = cfg["seq_len"] * cfg["n_seqs"]
    tok, tgt = O.ids(T, 1002, cfg["vocab_size"]), O.ids(T, 1003, cfg["vocab_size"])

    def cat(kind):
        return np.concatenate([m.tensor(kind, *k).copy() for k in keys])

    p0 = cat(0)
    loss = m.forward_backward(tok, tgt)
    g = cat(1)
    m.adam()
    save("step_tiny.npz", dict(cfg=cfg, keys=keys,
                               sizes=[int(m.tensor(0, *k).size) for k in keys]),
         tokens=tok, targets=tgt, params0=p0, loss=np.float32(loss), grads=g, params1=cat(0),
         adam_m1=cat(2), adam_v1=cat(3))


if __name__ == "__main__":
    kat_embedding()
    fa()
    cce()
    ops()
    step()
