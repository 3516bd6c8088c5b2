"""The committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py) against the C oracle, on the CPU.

The duplicated-id embedding fixture is a known answer formed without the
oracle (gpu_train.zig:4855-4884); the others are frozen oracle outputs, so
these tests fail if the oracle's arithmetic changes.
"""
import json
import os

import numpy as np
import pytest

import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    z = np.load(os.path.join(GOLDEN, name))  # allow_pickle stays False
    return {k: z[k] for k in z.files}, json.loads(str(z["meta"]))


def close(ref, got, tol=1e-6):
    ref, got = np.asarray(ref, np.float64), np.asarray(got, np.float64)
    scale = max(np.abs(ref).max(), 1e-30)
    return np.abs(ref - got).max() / scale <= tol


def test_fixtures_are_plain_arrays():
    for name in sorted(os.listdir(GOLDEN)):
        if name.endswith(".npz"):
            z = np.load(os.path.join(GOLDEN, name))
            assert all(z[k].dtype != object for k in z.files), name


def test_embedding_duplicate_ids_known_answer():
    a, meta = load("kat_embedding_dup_ids.npz")
    V, D = meta["V"], meta["D"]
    ids, dy, dE = a["ids"], a["dy"].reshape(-1, D), a["dE"].reshape(V, D)
    assert list(ids) == [3, 7, 3, 11, 7, 3]
    # by hand: token 3 collects positions 0, 2, 5 -> (1 + 3 + 6) + 3 j / 8
    assert np.array_equal(dE[3], np.array([10 + 3 * j / 8 for j in range(D)], np.float32))
    assert np.array_equal(dE[7], np.array([(2 + 5) + 2 * j / 8 for j in range(D)], np.float32))
    assert np.array_equal(dE[11], dy[3])
    untouched = [t for t in range(V) if t not in (3, 7, 11)]
    assert not dE[untouched].any()
    assert np.array_equal(O.embedding_backward(a["dy"], ids, V, D), a["dE"])


def test_oracle_reproduces_flash_attention_fixture():
    a, meta = load("fa.npz")
    for name, c in meta.items():
        B, n_q, n_kv, H, Hkv, hd, causal = (c[k] for k in ("B", "n_q", "n_kv", "H", "Hkv", "hd",
                                                          "causal"))
        for b in range(B):
            sq = slice(b * n_q * H * hd, (b + 1) * n_q * H * hd)
            sk = slice(b * n_kv * Hkv * hd, (b + 1) * n_kv * Hkv * hd)
            sr = slice(b * n_q * H, (b + 1) * n_q * H)
            Q, K, V, dO = (a[f"{name}_{k}"][s] for k, s in (("Q", sq), ("K", sk), ("V", sk),
                                                          ("dO", sq)))
            o, lse = O.flash_forward(Q, K, V, n_q, n_kv, H, Hkv, hd, causal)
            dq, dk, dv = O.flash_backward(Q, K, V, o, dO, lse, n_q, n_kv, H, Hkv, hd, causal)
            assert close(a[f"{name}_O"][sq], o) and close(a[f"{name}_lse"][sr], lse), name
            assert close(a[f"{name}_D"][sr], O.fa_bw_d(o, dO, n_q, H, hd)), name
            assert close(a[f"{name}_dQ"][sq], dq), name
            assert close(a[f"{name}_dK"][sk], dk) and close(a[f"{name}_dV"][sk], dv), name


def test_oracle_reproduces_cce_fixture():
    a, m = load("cce.npz")
    n, V, D = m["n"], m["V"], m["D"]
    loss, lse, row = O.cce_forward(a["h"], a["w"], a["targets"], n, V, D, m["chunk"], m["z_loss"],
                                   m["label_smoothing"])
    dh, dW = O.cce_backward(a["h"], a["w"], a["targets"], lse, n, V, D, m["chunk"], m["z_loss"],
                            m["label_smoothing"])
    assert close(a["loss"], loss) and close(a["lse"], lse) and close(a["loss_row"], row)
    assert close(a["dh"], dh) and close(a["dW"], dW)
    # independent of chunking (cce.zig:461-512)
    loss2, lse2, _ = O.cce_forward(a["h"], a["w"], a["targets"], n, V, D, 1024, m["z_loss"],
                                   m["label_smoothing"])
    assert close(a["lse"], lse2, 1e-6) and abs(loss2 - a["loss"]) <= 1e-6 * abs(a["loss"])


def test_oracle_reproduces_ops_fixture():
    a, m = load("ops.npz")
    eps = m["rms"]["eps"]
    assert close(a["rms_y"], O.rmsnorm_forward(a["rms_x"], a["rms_w"], eps))
    dx, dw = O.rmsnorm_backward(a["rms_dy"], a["rms_x"], a["rms_w"], eps)
    assert close(a["rms_dx"], dx) and close(a["rms_dw"], dw)
    dz, du = O.swiglu_backward(a["sw_dg"], a["sw_z"], a["sw_u"])
    assert close(a["sw_g"], O.swiglu_forward(a["sw_z"], a["sw_u"]))
    assert close(a["sw_dz"], dz) and close(a["sw_du"], du)
    r = m["rope"]
    n = r["S"] * r["B"]
    for rot in (16, 8):
        assert close(a[f"rope{rot}_q_out"],
                     O.rope_forward(a["rope_q"], n, r["Hq"], r["hd"], rot, r["theta"], r["S"]))
        assert close(a[f"rope{rot}_dk_in"],
                     O.rope_backward(a["rope_k"], n, r["Hkv"], r["hd"], rot, r["theta"], r["S"]))
    p, mm, v = a["adam_p0"].copy(), a["adam_m0"].copy(), a["adam_v0"].copy()
    for t in m["adam"]["t"]:
        O.adam_step(p, a["adam_g"], mm, v, 1e-3, 0.9, 0.999, 1e-8, t)
    assert close(a["adam_p3"], p) and close(a["adam_m3"], mm) and close(a["adam_v3"], v)
    L = m["linear"]
    assert close(a["lin_y"], O.matmul_nt(a["lin_x"], a["lin_w"], L["M"], L["N"], L["K"]))
    dxm, dWm = O.linear_backward(a["lin_dy"], a["lin_x"], a["lin_w"], L["M"], L["N"], L["K"])
    assert close(a["lin_dx"], dxm) and close(a["lin_dw"], dWm)


def test_oracle_reproduces_step_fixture():
    a, m = load("step_tiny.npz")
    cfg, keys, sizes = m["cfg"], [tuple(k) for k in m["keys"]], m["sizes"]
    model = O.Model(**cfg)
    offs = np.concatenate([[0], np.cumsum(sizes)])
    for i, k in enumerate(keys):
        model.tensor(0, *k)[:] = a["params0"][offs[i]:offs[i + 1]]
    loss = model.forward_backward(a["tokens"], a["targets"])
    assert abs(loss - float(a["loss"])) <= 1e-6 * abs(float(a["loss"]))
    for i, k in enumerate(keys):
        s = slice(offs[i], offs[i + 1])
        assert close(a["grads"][s], model.tensor(1, *k), 1e-5), k
    model.adam()
    for i, k in enumerate(keys):
        s = slice(offs[i], offs[i + 1])
        assert close(a["params1"][s], model.tensor(0, *k), 1e-6), k
        assert close(a["adam_m1"][s], model.tensor(2, *k), 1e-5), k


@pytest.mark.parametrize("name", ["fa.npz", "cce.npz", "ops.npz", "step_tiny.npz"])
def test_fixture_outputs_are_finite(name):
    a, _ = load(name)
    for k, x in a.items():
        if x.dtype.kind == "f":
            assert np.isfinite(x).all(), (name, k)
