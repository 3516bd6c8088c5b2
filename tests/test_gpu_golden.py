"""The HIP kernels and the Runner (through the C ABI) against the committed
golden fixtures of tests/golden/ (fixed inputs, fixed expected outputs).

Bars: bit-exact for the embedding scatter; rel-L2 <= 1e-3 (fp32 operands) and
<= 1e-2 (bf16 operands) for contractions; the formula-identical elementwise
kernels at max-relative 1e-5.
"""
import json
import os

import numpy as np
import pytest

from helpers import bf16_dev, dev, grel, host, note, rel_l2, zeros

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
LAYER_KEYS = ["w_n1", "w_q", "w_k", "w_v", "w_o", "w_n2", "w_gate", "w_up", "w_down", "w_q_norm",
              "w_k_norm"]


def load(name):
    z = np.load(os.path.join(GOLDEN, name))
    return {k: z[k] for k in z.files}, json.loads(str(z["meta"]))


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    import valkyr_amd as v

    assert v.device_count() > 0, "no GPU visible"


def test_golden_embedding_duplicate_ids():
    from valkyr_amd import kernels as K

    a, m = load("kat_embedding_dup_ids.npz")
    note("golden embedding {3,7,3,11,7,3}")
    bE = zeros(m["V"] * m["D"])
    K.embedding_backward(dev(a["dy"]), dev(a["ids"]), bE, a["ids"].size, m["D"], m["V"])
    assert np.array_equal(host(bE), a["dE"])


@pytest.mark.parametrize("name", ["ref_4x4", "ref_10x12", "ref_noncausal", "bf16_64"])
def test_golden_flash_attention(name):
    from valkyr_amd import kernels as K

    a, meta = load("fa.npz")
    c = meta[name]
    B, n_q, n_kv, H, Hkv, hd = (c[k] for k in ("B", "n_q", "n_kv", "H", "Hkv", "hd"))
    note(f"golden fa {name} {c}")
    g = {k: a[f"{name}_{k}"] for k in ("Q", "K", "V", "dO", "O", "lse", "D", "dQ", "dK", "dV")}
    nq, nk, nr = B * n_q * H * hd, B * n_kv * Hkv * hd, B * n_q * H
    if c["bf16"]:
        p = K.attn_params(n_q, n_kv, H, Hkv, hd, c["causal"], B, K.BF16)
        q, k, v = bf16_dev(g["Q"])[0], bf16_dev(g["K"])[0], bf16_dev(g["V"])[0]
        do16 = zeros(nq // 2 + 8)
        tol = 1e-2
    else:
        p = K.attn_params(n_q, n_kv, H, Hkv, hd, c["causal"], B, K.F32)
        q, k, v = dev(g["Q"]), dev(g["K"]), dev(g["V"])
        do16 = None
        tol = 1e-3
    bo, blse, bd = zeros(nq), zeros(nr), zeros(nr)
    K.fa_forward(p, q, k, v, bo, blse)
    dof = dev(g["dO"])
    K.fa_bw_d(p, bo, dof, bd, do16)
    bdq, bdk, bdv = zeros(nq), zeros(nk), zeros(nk)
    ws_bytes = K.fa_backward_workspace_bytes(p)
    ws = zeros(ws_bytes // 4 + 1) if ws_bytes else None
    K.fa_backward(p, q, k, v, do16 if do16 is not None else dof, blse, bd, bdq, bdk, bdv, ws)
    e = {"O": rel_l2(g["O"], host(bo)), "D": rel_l2(g["D"], host(bd)),
         "dQ": rel_l2(g["dQ"], host(bdq)), "dK": rel_l2(g["dK"], host(bdk)),
         "dV": rel_l2(g["dV"], host(bdv))}
    note("  rel-L2 " + " ".join(f"{k}={x:.2e}" for k, x in e.items()))
    assert np.abs(g["lse"] - host(blse)).max() < (2e-2 if c["bf16"] else 1e-5)
    assert all(x < tol for x in e.values()), e


@pytest.mark.parametrize("prec", [0, 1])
def test_golden_cce(prec):
    from valkyr_amd import kernels as K

    a, m = load("cce.npz")
    n, V, D = m["n"], m["V"], m["D"]
    note(f"golden cce prec={prec}")
    p = K.cce_params(n, V, D, m["z_loss"], m["label_smoothing"], prec)
    bh, bw, bt = dev(a["h"]), dev(a["w"]), dev(a["targets"])
    blse, brow, bmean = zeros(n), zeros(n), zeros(1)
    K.cce_forward(p, bh, bw, bt, blse, brow, bmean)
    assert grel(a["lse"], host(blse)) < 1e-5
    assert abs(host(bmean)[0] - a["loss"]) < 1e-4 * abs(a["loss"])
    bdh, bdW = zeros(n * D), zeros(V * D)
    K.cce_backward(p, bh, bw, bt, blse, bdh, bdW)
    tol = 1e-3 if prec == 0 else 1e-2
    assert rel_l2(a["dh"], host(bdh)) < tol
    assert rel_l2(a["dW"], host(bdW)) < tol


def test_golden_bandwidth_kernels_and_gemms():
    from valkyr_amd import kernels as K

    a, m = load("ops.npz")
    note("golden ops")
    r = m["rms"]
    n = r["rows"] * r["dim"]
    by, bdx, bdw = zeros(n), zeros(n), zeros(r["dim"])
    bx, bw = dev(a["rms_x"]), dev(a["rms_w"])
    K.rmsnorm_forward(bx, bw, by, r["rows"], r["dim"], r["eps"])
    K.rmsnorm_backward(dev(a["rms_dy"]), bx, bw, bdx, bdw, r["rows"], r["dim"], r["eps"])
    assert grel(a["rms_y"], host(by)) < 1e-5
    assert grel(a["rms_dx"], host(bdx)) < 1e-5 and grel(a["rms_dw"], host(bdw)) < 1e-5

    ns = m["swiglu"]["n"]
    bz, bu = dev(a["sw_z"]), dev(a["sw_u"])
    bg, bdz, bdu = zeros(ns), zeros(ns), zeros(ns)
    K.swiglu_forward(bz, bu, bg, ns)
    K.swiglu_backward(dev(a["sw_dg"]), bz, bu, bdz, bdu, ns)
    assert grel(a["sw_g"], host(bg)) < 1e-5
    assert grel(a["sw_dz"], host(bdz)) < 1e-5 and grel(a["sw_du"], host(bdu)) < 1e-5

    ro = m["rope"]
    rows = ro["S"] * ro["B"]
    bq, bk = dev(a["rope_q"]), dev(a["rope_k"])
    for rot in (16, 8):
        p = K.rope_params(rows, ro["Hq"], ro["Hkv"], ro["hd"], rot, ro["theta"], ro["S"])
        oq, ok = zeros(a["rope_q"].size), zeros(a["rope_k"].size)
        K.qk_rope_forward(p, bq, oq, bk, ok)
        assert grel(a[f"rope{rot}_q_out"], host(oq)) < 1e-5
        assert grel(a[f"rope{rot}_k_out"], host(ok)) < 1e-5
        K.qk_rope_backward(p, bq, oq, bk, ok)
        assert grel(a[f"rope{rot}_dq_in"], host(oq)) < 1e-5
        assert grel(a[f"rope{rot}_dk_in"], host(ok)) < 1e-5

    ad = m["adam"]
    bp, bm, bv = dev(a["adam_p0"]), dev(a["adam_m0"]), dev(a["adam_v0"])
    bg2 = dev(a["adam_g"])
    for t in ad["t"]:
        K.adam_step(bp, bg2, bm, bv, ad["n"], ad["lr"], ad["b1"], ad["b2"], ad["eps"], t)
    assert grel(a["adam_p3"], host(bp)) < 1e-6
    assert grel(a["adam_m3"], host(bm)) < 1e-6 and grel(a["adam_v3"], host(bv)) < 1e-6

    L = m["linear"]
    M, N, Kd = L["M"], L["N"], L["K"]
    for prec in (0, 1):
        tol = 1e-3 if prec == 0 else 1e-2
        bxl, bwl, bdy = dev(a["lin_x"]), dev(a["lin_w"]), dev(a["lin_dy"])
        y, dx, dW = zeros(M * N), zeros(M * Kd), zeros(N * Kd)
        K.matmul_nt(bxl, bwl, y, M, N, Kd, prec)
        K.linear_backward_dx(bdy, bwl, dx, M, N, Kd, prec)
        K.linear_backward_dw(bdy, bxl, dW, M, N, Kd, prec)
        assert rel_l2(a["lin_y"], host(y)) < tol
        assert rel_l2(a["lin_dx"], host(dx)) < tol and rel_l2(a["lin_dw"], host(dW)) < tol


def test_golden_training_step():
    import valkyr_amd as v

    a, m = load("step_tiny.npz")
    cfg, keys, sizes = m["cfg"], [tuple(k) for k in m["keys"]], m["sizes"]
    note(f"golden step {cfg}")
    offs = np.concatenate([[0], np.cumsum(sizes)])
    t = {k: a["params0"][offs[i]:offs[i + 1]] for i, k in enumerate(keys)}
    weights = {"embed": t[(-1, 0)], "final_norm": t[(-1, 1)], "lm_head": t.get((-1, 2)),
               "layers": [{LAYER_KEYS[w]: t.get((l, w)) for w in range(11)}
                          for l in range(cfg["n_layers"])]}
    rc = v.make_config(dim=cfg["dim"], n_heads=cfg["n_heads"], n_kv_heads=cfg["n_kv_heads"],
                       head_dim=cfg["head_dim"], ff_dim=cfg["ff_dim"], n_pos=cfg["seq_len"],
                       n_layers=cfg["n_layers"], vocab_size=cfg["vocab_size"],
                       rms_eps=cfg["rms_eps"], causal=cfg["causal"], rotary_dim=cfg["rotary_dim"],
                       rope_theta=cfg["rope_theta"], qk_norm=cfg["qk_norm"], lr=cfg["lr"],
                       beta1=cfg["beta1"], beta2=cfg["beta2"], eps_adam=cfg["eps_adam"],
                       n_seqs=cfg["n_seqs"], tied_embeddings=cfg["tied_embeddings"], precision=0)
    with v.Runner(rc, weights) as r:
        r.step(a["tokens"], a["targets"])
        loss = r.last_loss()
        note(f"  loss golden {float(a['loss']):.6f} gpu {loss:.6f}")
        assert abs(loss - float(a["loss"])) < 1e-5 * abs(float(a["loss"]))
        assert r.step_t == 2  # Adam's t starts at 1 and is incremented after the update
        worst = 0.0
        for i, k in enumerate(keys):
            s = slice(offs[i], offs[i + 1])
            eg = rel_l2(a["grads"][s], r.get(1, *k))
            ep = rel_l2(a["params1"][s], r.get(0, *k))
            em = rel_l2(a["adam_m1"][s], r.get(2, *k))
            worst = max(worst, eg, ep, em)
            assert eg < 1e-3 and ep < 1e-3 and em < 1e-3, (k, eg, ep, em)
        note(f"  worst rel-L2 over grads / params / Adam m: {worst:.2e}")
