"""Whole-step parity: the HIP Runner vs the C oracle's GPU-Runner semantics on
identical seeded weights and tokens (the tiny parity config and variants), plus
the Runner API behaviour (checkpoints, tick API, error paths).

Per-tensor bars: fp32 precision rel-L2 <= 1e-3 for every gradient and Adam
moment; bf16-operand precision rel-L2 <= 1e-2 against the oracle run with
bf16-rounded contraction operands.
"""
import os
import struct

import numpy as np
import pytest

import oracle as O
from helpers import note, rel_l2

pytestmark = pytest.mark.gpu

CONFIG1 = dict(dim=256, n_heads=4, n_kv_heads=2, head_dim=64, ff_dim=768, seq_len=128, n_seqs=1,
               n_layers=2, vocab_size=4096, rms_eps=1e-6, causal=1, rotary_dim=64,
               rope_theta=1e6, qk_norm=1, lr=1e-4, beta1=0.9, beta2=0.999, eps_adam=1e-8,
               lora_targets=0, lora_rank=0, lora_alpha=0.0, lora_lr_b_scale=1.0,
               tied_embeddings=0, bf16_operands=0)

LAYER_KEYS = ["w_n1", "w_q", "w_k", "w_v", "w_o", "w_n2", "w_gate", "w_up", "w_down", "w_q_norm",
              "w_k_norm"]


def build_pair(precision=0, seed=1234, lora_std=0.02, **over):
    import valkyr_amd as v

    cfg = dict(CONFIG1)
    cfg.update(over)
    if precision == 1:
        cfg["bf16_operands"] = 1
    m = O.Model(**cfg)
    m.init_random(seed, std=0.02, lora_std=lora_std)
    L = cfg["n_layers"]
    if precision == 1 and cfg["lora_targets"]:
        # a bf16 LoRA runner stores its frozen base matrices in bf16: the
        # oracle takes the same bf16 values
        mats = [(-1, 0)] + ([] if cfg["tied_embeddings"] else [(-1, 2)]) + \
            [(l, w) for l in range(L) for w in (1, 2, 3, 4, 6, 7, 8)]
        for k in mats:
            t = m.tensor(0, *k)
            t[:] = O.round_bf16(t)
    weights = {
        "embed": m.tensor(0, -1, 0).copy(),
        "final_norm": m.tensor(0, -1, 1).copy(),
        "lm_head": None if cfg["tied_embeddings"] else m.tensor(0, -1, 2).copy(),
        "layers": [{LAYER_KEYS[w]: (m.tensor(0, l, w).copy() if m.tensor(0, l, w) is not None else None)
                    for w in range(11)} for l in range(L)],
    }
    if cfg["lora_targets"]:
        weights["lora"] = {p: [{"a": m.tensor(0, l, 16 + 2 * p).copy(),
                                "b": m.tensor(0, l, 17 + 2 * p).copy()} for l in range(L)]
                           for p in range(7) if cfg["lora_targets"] & (1 << p)}
    rc = v.make_config(dim=cfg["dim"], n_heads=cfg["n_heads"], n_kv_heads=cfg["n_kv_heads"],
                       head_dim=cfg["head_dim"], ff_dim=cfg["ff_dim"], n_pos=cfg["seq_len"],
                       n_layers=L, vocab_size=cfg["vocab_size"], rms_eps=cfg["rms_eps"],
                       causal=cfg["causal"], rotary_dim=cfg["rotary_dim"],
                       rope_theta=cfg["rope_theta"], qk_norm=cfg["qk_norm"], lr=cfg["lr"],
                       beta1=cfg["beta1"], beta2=cfg["beta2"], eps_adam=cfg["eps_adam"],
                       lora_targets=cfg["lora_targets"], lora_rank=cfg["lora_rank"],
                       lora_alpha=cfg["lora_alpha"], lora_lr_b_scale=cfg["lora_lr_b_scale"],
                       n_seqs=cfg["n_seqs"], tied_embeddings=cfg["tied_embeddings"],
                       precision=precision)
    r = v.Runner(rc, weights)
    T = cfg["seq_len"] * cfg["n_seqs"]
    tok = O.ids(T, seed + 1, cfg["vocab_size"])
    tgt = O.ids(T, seed + 2, cfg["vocab_size"])
    return m, r, tok, tgt, cfg


def tensor_keys(cfg):
    keys = [(-1, 0), (-1, 1)] + ([] if cfg["tied_embeddings"] else [(-1, 2)])
    for l in range(cfg["n_layers"]):
        keys += [(l, w) for w in range(9)]
        if cfg["qk_norm"]:
            keys += [(l, 9), (l, 10)]
    return keys


def lora_keys(cfg):
    return [(l, 16 + 2 * p + ab) for l in range(cfg["n_layers"]) for p in range(7)
            if cfg["lora_targets"] & (1 << p) for ab in (0, 1)]


def compare(m, r, keys, kind, tol, what):
    """rel-L2 of every tensor in `keys`; fails listing the worst ones."""
    errs = {k: rel_l2(m.tensor(kind, *k), r.get(kind, *k)) for k in keys}
    worst = sorted(errs.items(), key=lambda kv: -kv[1])
    note(f"  {what}: worst rel-L2 " + ", ".join(f"{k}: {e:.2e}" for k, e in worst[:4]))
    bad = [(k, e) for k, e in worst if not e < tol]
    assert not bad, f"{what} rel-L2 >= {tol}: " + ", ".join(f"{k}: {e:.3e}" for k, e in bad[:8])
    return worst[0][1]


def stage_compare(m, r, tok, tgt, cfg, tol, what):
    """The runner's step against the oracle stage by stage, each stage on the
    GPU's own inputs (the residual-stream tensor and the gradient at every
    layer boundary, captured by the runner): the head from the last layer's
    output, each layer's forward from its input and backward from the
    gradient at its output, the embedding gradient from the gradient at the
    embedding output.  Compares every layer output, boundary gradient and
    trainable gradient at `tol`; returns the errors."""
    L = cfg["n_layers"]
    lora = bool(cfg["lora_targets"])
    r.set_boundary_capture(True)
    loss = r.forward_backward(tok, tgt)
    xs = [r.boundary(l, 0) for l in range(L + 1)]
    gs = [r.boundary(l, 1) for l in range(L + 1)]
    errs = {}
    loss_ref, g_ref = m.head_forward_backward(xs[L], tgt)
    note(f"  head: loss oracle {loss_ref:.6f} gpu {loss:.6f}")
    assert abs(loss - loss_ref) < 1e-5 * abs(loss_ref)
    errs["g(L)"] = rel_l2(g_ref, gs[L])
    if not lora:
        errs["final_norm"] = rel_l2(m.tensor(1, -1, 1), r.get(1, -1, 1))
    for l in range(L - 1, -1, -1):
        g_ref = m.layer_forward_backward(l, xs[l], gs[l + 1])
        errs[f"y{l}"] = rel_l2(m.layer_output(l), xs[l + 1])
        errs[f"g({l})"] = rel_l2(g_ref, gs[l])
        ws = [k[1] for k in lora_keys(cfg) if k[0] == l] if lora else \
            [w for w in range(11) if cfg["qk_norm"] or w < 9]
        for w in ws:
            errs[(l, w)] = rel_l2(m.tensor(1, l, w), r.get(1, l, w))
    if not lora:
        m.embedding_backward(tok, gs[0])
        errs["embed"] = rel_l2(m.tensor(1, -1, 0), r.get(1, -1, 0))
    worst = sorted(errs.items(), key=lambda kv: -kv[1])
    note(f"  {what}: worst rel-L2 " + ", ".join(f"{k}: {e:.2e}" for k, e in worst[:8]))
    bad = [(k, e) for k, e in worst if not e < tol]
    assert not bad, f"{what} rel-L2 >= {tol}: {bad}"
    return errs


HD128 = {"head_dim": 128, "n_heads": 2, "n_kv_heads": 1, "rotary_dim": 128}  # Qwen3 head size


@pytest.mark.parametrize("variant", [{}, {"tied_embeddings": 1}, {"n_seqs": 2, "seq_len": 64},
                                     {"qk_norm": 0, "rotary_dim": 32}, HD128,
                                     dict(HD128, rotary_dim=64, n_seqs=2, seq_len=64)])
def test_step_parity_fp32(variant):
    note(f"step fp32 {variant}")
    m, r, tok, tgt, cfg = build_pair(0, **variant)
    keys = tensor_keys(cfg)
    p0 = {k: m.tensor(0, *k).copy() for k in keys}
    loss_ref = m.forward_backward(tok, tgt)
    loss = r.forward_backward(tok, tgt)
    note(f"  loss oracle {loss_ref:.6f} gpu {loss:.6f}")
    assert abs(loss - loss_ref) < 1e-5 * abs(loss_ref)
    compare(m, r, keys, 1, 1e-3, "grad")
    m.adam()
    r.step(tok, tgt)  # same grads again (weights unchanged), then Adam
    assert r.step_t == m.step_t == 2
    compare(m, r, keys, 2, 1e-3, "adam m")
    compare(m, r, keys, 3, 1e-3, "adam v")
    for k in keys:
        # updated weights ...
        assert rel_l2(m.tensor(0, *k), r.get(0, *k)) < 1e-3
        # ... and the update itself: at t = 1 Adam moves every weight by about
        # lr * sign(g), so entries with |g| near eps are sign-sensitive; 1e-2
        du_ref = m.tensor(0, *k) - p0[k]
        du = r.get(0, *k) - p0[k]
        assert rel_l2(du_ref, du) < 1e-2, (k, rel_l2(du_ref, du))


# The step's recompute attention-backward kernels need bf16, head_dim 128, an
# even GQA group and >= 128 key blocks of 128: 16 sequences x 128 positions x
# 8 KV heads (the Qwen3-0.6B head layout) at a small width.
RECOMPUTE = dict(HD128, n_heads=16, n_kv_heads=8, n_seqs=16, seq_len=128, n_layers=1, dim=256,
                 ff_dim=512, vocab_size=1024)


# GQA 4:1 on the recompute path with 128 dK/dV blocks (fewer than the CUs): the
# dK/dV launch splits each block's head group over two blocks and a combine
# kernel adds the halves before the epilogue (config 4's case at 1 x 2048);
# with a 64-wide rotary span the fused epilogue is off and the combine writes
# fp32 dK / dV
RECOMPUTE_GQA4 = dict(HD128, n_heads=16, n_kv_heads=4, n_seqs=16, seq_len=256, n_layers=1,
                      dim=256, ff_dim=512, vocab_size=1024)
RECOMPUTE_GQA4_ROT64 = dict(RECOMPUTE_GQA4, rotary_dim=64)
SPLIT_VARIANTS = (RECOMPUTE_GQA4, RECOMPUTE_GQA4_ROT64)

# The fused q/k epilogue's other branches: RoPE^T without the Q/K-norm
# backward (a Llama-style hd-128 model), and the Q/K-norm backward without RoPE.
RECOMPUTE_NO_QK_NORM = dict(RECOMPUTE, qk_norm=0)
RECOMPUTE_NO_ROPE = dict(RECOMPUTE, rotary_dim=0)
RECOMPUTE_VARIANTS = (RECOMPUTE, RECOMPUTE_NO_QK_NORM, RECOMPUTE_NO_ROPE)


@pytest.mark.parametrize("variant", [{}, HD128, RECOMPUTE, RECOMPUTE_NO_QK_NORM,
                                     RECOMPUTE_NO_ROPE, RECOMPUTE_GQA4, RECOMPUTE_GQA4_ROT64],
                         ids=["config1", "hd128", "recompute", "recompute-no-qk-norm",
                              "recompute-no-rope", "recompute-gqa4-split",
                              "recompute-gqa4-split-rot64"])
def test_step_parity_bf16(variant):
    """bf16-operand step vs the oracle with the same operand rounding (every
    MFMA operand, the attention P and dS and the CCE dz included), every
    gradient and Adam moment within rel-L2 1e-2 (the bf16-operand bar).
    Measured worst: 6.0e-3 (config 1), 3.2e-3 (recompute attention path), at
    the floor of the bf16-operand step's own sensitivity (a one-ulp change of
    10 % of the fp32 master weights moves the oracle's gradients by 6.0e-3 on
    the same tensors; tests/test_oracle.py)."""
    note(f"step bf16 {variant}")
    m, r, tok, tgt, cfg = build_pair(1, **variant)
    if any(variant is x for x in RECOMPUTE_VARIANTS):
        assert r.attention_backward_path() == "recompute"
        plan = r.attention_backward_plan()
        note(f"  attention backward plan {plan}")
        assert plan["qk_epilogue"], plan
    if any(variant is x for x in SPLIT_VARIANTS):
        plan = r.attention_backward_plan()
        note(f"  attention backward plan {plan}")
        # 16 sequences x 4 KV heads x 2 key blocks = 128, launched as 2 x 128
        assert plan["path"] == "recompute" and plan["dkv_blocks"] == 256, plan
        assert plan["qk_epilogue"] == (variant is RECOMPUTE_GQA4), plan
    keys = tensor_keys(cfg)
    loss_ref = m.forward_backward(tok, tgt)
    loss = r.forward_backward(tok, tgt)
    note(f"  loss oracle(bf16 operands) {loss_ref:.6f} gpu {loss:.6f}")
    assert abs(loss - loss_ref) < 1e-3 * abs(loss_ref)
    compare(m, r, keys, 1, 1e-2, "grad")
    m.adam()
    r.step(tok, tgt)
    compare(m, r, keys, 2, 1e-2, "adam m")
    compare(m, r, keys, 3, 1e-2, "adam v")
    for k in keys:  # updated weights
        assert rel_l2(m.tensor(0, *k), r.get(0, *k)) < 1e-2


# Per-layer activation recompute (config 5's mode) at 5 layers, so that the
# two shared activation sets, the two gradient-copy sets and the three-deep
# dy ring are all reused: the same kernels run on the same inputs, so every
# gradient, moment and weight must equal the stored-activation runner's bit
# for bit, through forward_backward and three Adam steps.
RECOMPUTE_MODE_BASE = dict(dim=256, n_heads=4, n_kv_heads=2, head_dim=64, ff_dim=768, n_pos=128,
                           n_layers=5, vocab_size=4096, rms_eps=1e-6, causal=1, rotary_dim=64,
                           rope_theta=1e6, qk_norm=1, lr=1e-3)
LORA_QV = dict(lora_targets=0x5 | 0x40, lora_rank=8, lora_alpha=16.0)


@pytest.mark.parametrize("precision,over", [
    (0, {}), (1, {}), (1, dict(tied_embeddings=1, n_seqs=2, n_pos=64)), (0, LORA_QV),
    (1, LORA_QV),
    (1, dict(head_dim=128, n_heads=16, n_kv_heads=8, rotary_dim=128, n_seqs=16, n_pos=128,
             ff_dim=512, vocab_size=1024, n_layers=4)),
    (1, dict(head_dim=128, n_heads=16, n_kv_heads=8, rotary_dim=128, n_seqs=16, n_pos=128,
             ff_dim=512, vocab_size=1024, n_layers=4, **LORA_QV)),
    # GQA 4:1 with the split dK/dV launch
    (1, dict(head_dim=128, n_heads=16, n_kv_heads=4, rotary_dim=128, n_seqs=16, n_pos=256,
             ff_dim=512, vocab_size=1024, n_layers=4))])
def test_activation_recompute_bit_identical(precision, over):
    import valkyr_amd as v
    from valkyr_amd.runner import ADAM_M, ADAM_V, GRAD, PARAM

    c = dict(RECOMPUTE_MODE_BASE, **over)
    note(f"activation recompute precision={precision} {over}")
    lora = bool(c.get("lora_targets"))
    L = c["n_layers"]
    T = c["n_pos"] * c.get("n_seqs", 1)
    with v.Runner(v.make_config(**c, precision=precision)) as a, \
            v.Runner(v.make_config(**c, precision=precision, recompute=1)) as b:
        for r in (a, b):
            r.init_random(seed=21, std=0.02, lora_std=0.02)
        note(f"  device bytes stored {a.device_bytes():,}, recompute {b.device_bytes():,}")
        assert b.device_bytes() < a.device_bytes()
        if over.get("head_dim") == 128:
            assert b.attention_backward_path() == "recompute"
        cf = {**c, "tied_embeddings": c.get("tied_embeddings", 0),
              "qk_norm": c["qk_norm"]}
        base = tensor_keys(cf)
        trainable = lora_keys(cf) if lora else base
        tok, tgt = O.ids(T, 5, c["vocab_size"]), O.ids(T, 6, c["vocab_size"])

        def same(kind, keys, what):
            for k in keys:
                x, y = a.get(kind, *k), b.get(kind, *k)
                assert np.array_equal(x, y), (what, k, rel_l2(x, y))

        la, lb = a.forward_backward(tok, tgt), b.forward_backward(tok, tgt)
        assert la == lb, (la, lb)
        same(GRAD, trainable, "grad")
        for i in range(3):
            tok, tgt = O.ids(T, 7 + i, c["vocab_size"]), O.ids(T, 17 + i, c["vocab_size"])
            a.step(tok, tgt)
            b.step(tok, tgt)
            assert a.last_loss() == b.last_loss()
        same(GRAD, trainable, "grad after steps")
        same(ADAM_M, trainable, "adam m")
        same(ADAM_V, trainable, "adam v")
        same(PARAM, base + (lora_keys(cf) if lora else []), "param")
        note(f"  loss {la:.5f} -> {b.last_loss():.5f}, identical")


# Qwen3-0.6B widths (config 3) at 2 layers: dim 1024, 16/8 heads of 128,
# QK-norm, FFN 3072, the full 151936 vocabulary with tied embeddings, theta
# 1e6, eps 1e-6.  "1x128" pins the CCE's dh and dW over the full vocabulary,
# the tied-embedding sum and the vocabulary-sized GEMM plans; "4x512" is
# config 3's own batch layout (B = 4 x S = 512, 2048 rows), so the step runs
# exactly the kernels the benchmark runs: the M = 2048 GEMM plans with their
# residual / bf16 / CCE epilogues, and in bf16 the recompute attention
# backward with 128-query dQ blocks (256 of them; 128 dK/dV blocks), RoPE
# positions up to 511 over four key blocks per sequence and the fused RoPE^T /
# Q/K-norm epilogue.
QWEN3_06B_WIDTHS = dict(dim=1024, n_heads=16, n_kv_heads=8, head_dim=128, ff_dim=3072,
                        vocab_size=151936, tied_embeddings=1, rotary_dim=128, seq_len=128,
                        n_seqs=1, n_layers=2)
QWEN3_06B_LAYOUTS = {"1x128": {}, "4x512": dict(seq_len=512, n_seqs=4)}
CONFIG3_PLAN = {"path": "recompute", "dq_block_rows": 128, "dq_blocks": 256, "dkv_blocks": 128,
                "qk_epilogue": True}


# Whole-step comparisons.  bf16 at 4 x 512 is held to the oracle stage by
# stage instead (test_step_stages_qwen3_06b_widths): there the oracle's own
# bf16 model moves by up to 1.18e-2 under a one-ulp change of its master
# weights, above the 1e-2 bar.
WHOLE_CASES = [("1x128", 0), ("4x512", 0), ("1x128", 1)]


@pytest.mark.parametrize("layout,precision", WHOLE_CASES,
                         ids=[f"{'bf16' if p else 'fp32'}-{l}" for l, p in WHOLE_CASES])
def test_step_parity_qwen3_06b_widths(layout, precision):
    """One Adam step at config-3 widths against the oracle: every gradient,
    Adam moment and updated weight within 1e-3 (fp32 precision) or 1e-2
    (bf16 operands, against the oracle with the same rounding)."""
    tol = 1e-3 if precision == 0 else 1e-2
    note(f"step at Qwen3-0.6B widths, layout {layout}, precision {precision}")
    m, r, tok, tgt, cfg = build_pair(precision, **{**QWEN3_06B_WIDTHS, **QWEN3_06B_LAYOUTS[layout]})
    keys = tensor_keys(cfg)
    p0 = {k: m.tensor(0, *k).copy() for k in keys}
    loss_ref = m.forward_backward(tok, tgt)
    m.adam()
    r.step(tok, tgt)
    loss = r.last_loss()
    note(f"  loss oracle {loss_ref:.6f} gpu {loss:.6f}")
    assert abs(loss - loss_ref) < (1e-5 if precision == 0 else 1e-3) * abs(loss_ref)
    assert r.step_t == m.step_t == 2
    compare(m, r, keys, 1, tol, "grad")
    compare(m, r, keys, 2, tol, "adam m")
    compare(m, r, keys, 3, tol, "adam v")
    worst = 0.0
    for k in keys:
        e = rel_l2(m.tensor(0, *k), r.get(0, *k))
        worst = max(worst, e)
        assert e < tol, (k, e)
        if precision == 0:
            # the update itself: at t = 1 Adam moves every weight by about
            # lr * sign(g), so entries with |g| near the gradient error flip
            du_ref, du = m.tensor(0, *k) - p0[k], r.get(0, *k) - p0[k]
            assert rel_l2(du_ref, du) < 1e-2, (k, rel_l2(du_ref, du))
    note(f"  updated weights: worst rel-L2 {worst:.2e}")


# (layout, precision) of the whole-step comparisons that the bf16 model's
# sensitivity floor makes non-discriminating (below), checked stage by stage
STAGE_CASES = [("4x512", 1), ("1x128", 1), ("4x512", 0)]


@pytest.mark.parametrize("layout,precision", STAGE_CASES,
                         ids=[f"{l}-{'bf16' if p else 'fp32'}" for l, p in STAGE_CASES])
def test_step_stages_qwen3_06b_widths(layout, precision):
    """The step at config-3 widths held to the oracle stage by stage, each
    stage on the GPU's own inputs (its residual-stream tensor and the gradient
    arriving at it, captured at every layer boundary): the head (final norm,
    CE over the full tied 151936 vocabulary and their backward) from the last
    layer's output, each layer's forward from its input and backward from the
    gradient at its output, and the embedding gradient from the gradient at
    the embedding output plus the head's dW.  Every layer output, boundary
    gradient and parameter gradient within 1e-2 (bf16 operands, against the
    oracle with the same rounding) or 1e-3 (fp32).

    Why stages: two correct bf16-operand steps drift apart by about a bf16
    ulp wherever they differ in the last fp32 bit before a rounding, and the
    drift compounds over the stages.  Moving 10 % of the oracle's fp32 master
    weights by one ulp moves its own bf16 gradients by up to 1.2e-2 at 4 x 512
    (9.2e-3 at 1 x 128) on the q / k side, so a whole-step comparison at 1e-2
    cannot tell a correct step from a wrong one there; one stage on identical
    inputs can."""
    tol = 1e-2 if precision == 1 else 1e-3
    note(f"step stages at Qwen3-0.6B widths, layout {layout}, precision {precision}")
    m, r, tok, tgt, cfg = build_pair(precision, **{**QWEN3_06B_WIDTHS, **QWEN3_06B_LAYOUTS[layout]})
    if precision == 1 and layout == "4x512":
        plan = r.attention_backward_plan()
        note(f"  attention backward plan {plan}")
        assert plan == CONFIG3_PLAN, plan
    stage_compare(m, r, tok, tgt, cfg, tol, "stages")


@pytest.mark.parametrize("tied", [1, 0], ids=["tied", "untied"])
def test_split_embedding_update_bit_identical(tied):
    """The two-stream bf16 step updates the embedding table in two parts: rows
    no token names on the second stream right after the head's weight
    gradient, the token rows inside the embedding-backward launch.  Over two
    steps (the second with non-zero moments) the table's gradient, Adam
    moments and weights (and the untied head's and the final norm's) equal,
    bit for bit, one full-table Adam update (the library's own span kernel)
    applied to the gradient a forward/backward-only pass produces from the
    same state."""
    import valkyr_amd as v
    from valkyr_amd import kernels as K
    from valkyr_amd.runner import ADAM_M, ADAM_V, GRAD, PARAM

    from helpers import dev, host

    c = dict(dim=256, n_heads=4, n_kv_heads=2, head_dim=64, ff_dim=512, n_pos=128, n_seqs=2,
             n_layers=2, vocab_size=4096, rms_eps=1e-6, rotary_dim=64, rope_theta=1e6,
             qk_norm=1, lr=1e-3, tied_embeddings=tied)
    T, V = 256, 4096
    keys = [(-1, 0), (-1, 1)] + ([] if tied else [(-1, 2)])
    with v.Runner(v.make_config(**c, precision=1)) as a, \
            v.Runner(v.make_config(**c, precision=1)) as b:
        for r in (a, b):
            r.init_random(seed=31, std=0.02)
        for it in range(2):
            # ids from a narrow range: repeated ids (the owner sums them) and
            # most of the table untouched
            tok = (O.ids(T, 40 + it, 97) * 37 + 5).astype(np.uint32) % V
            tgt = O.ids(T, 50 + it, V)
            state = {k: [a.get(kind, *k) for kind in (PARAM, ADAM_M, ADAM_V)] for k in keys}
            t = a.step_t
            b.step_t = t
            lb = b.forward_backward(tok, tgt)
            a.step(tok, tgt)
            assert a.last_loss() == lb
            for k in keys:
                g = b.get(GRAD, *k)
                assert np.array_equal(a.get(GRAD, *k), g), (it, k, "grad")
                p, m, vv = (dev(x) for x in state[k])
                n = g.size
                K.adam_step(p, dev(g), m, vv, n, c["lr"], 0.9, 0.999, 1e-8, t)
                for kind, buf in ((PARAM, p), (ADAM_M, m), (ADAM_V, vv)):
                    want = host(buf, n)
                    got = a.get(kind, *k)
                    assert np.array_equal(got, want), (it, k, kind, rel_l2(want, got))
            # b follows a's state for the next step's gradient
            for k in [(-1, 0), (-1, 1)] + ([] if tied else [(-1, 2)]) + \
                    [(l, w) for l in range(2) for w in range(11)]:
                for kind in (PARAM, ADAM_M, ADAM_V):
                    b.set(kind, *k, a.get(kind, *k))
        note(f"  split embedding update tied={tied}: bit-identical over 2 steps")


def test_step_bf16_vs_pure_fp32_oracle():
    """bf16-operand GPU path against the unrounded fp32 oracle (reported; 5e-2 bar)."""
    m, r, tok, tgt, cfg = build_pair(0)
    import valkyr_amd as v
    rb = v.Runner(v.make_config(**{f: getattr(r.cfg, f) for f, _ in r.cfg._fields_ if f != "precision"},
                                precision=1),
                  {"embed": m.tensor(0, -1, 0), "final_norm": m.tensor(0, -1, 1),
                   "lm_head": m.tensor(0, -1, 2),
                   "layers": [{LAYER_KEYS[w]: m.tensor(0, l, w) for w in range(11)} for l in range(2)]})
    m.forward_backward(tok, tgt)
    rb.forward_backward(tok, tgt)
    compare(m, rb, tensor_keys(cfg), 1, 5e-2, "grad bf16-vs-fp32")


@pytest.mark.parametrize("precision,over", [
    (0, dict(lora_targets=0xF)), (1, dict(lora_targets=0xF)),
    (1, dict(lora_targets=0x7F, n_layers=3)), (0, dict(lora_targets=0x55, lora_rank=8)),
    (1, dict(HD128, lora_targets=0xF)),
    # the recompute attention path at a grid that leaves CUs idle: dQ runs on
    # a second stream beside dK/dV (and with GQA 4:1, the split dK/dV launch)
    (1, dict(RECOMPUTE, lora_targets=0xF)), (1, dict(RECOMPUTE_GQA4, lora_targets=0xF))])
def test_lora_step_parity(precision, over):
    """Config-4 shape class: LoRA r=16 on q/k/v/o (and every projection, and
    a rank-8 subset), B = 0 init, frozen base.  fp32: every adapter gradient
    within 1e-3; bf16: against the oracle with bf16 base-GEMM operands and fp32
    adapter factors (the rank-r kernels' numerics) within 1e-2."""
    note(f"lora step precision={precision} {over}")
    over = dict(dict(lora_rank=16, lora_alpha=32.0, lora_lr_b_scale=1.0), **over)
    m, r, tok, tgt, cfg = build_pair(precision, **over)
    tol, ltol = (1e-3, 1e-5) if precision == 0 else (1e-2, 1e-3)
    lk = lora_keys(cfg)
    loss_ref = m.forward_backward(tok, tgt)
    loss = r.forward_backward(tok, tgt)
    assert abs(loss - loss_ref) < ltol * abs(loss_ref)
    for (l, w) in lk:
        if w % 2 == 0:  # dA == 0 exactly at B = 0 (lora.zig:449-505)
            assert np.all(r.get(1, l, w) == 0)
    compare(m, r, [k for k in lk if k[1] % 2 == 1], 1, tol, "dB")
    base_before = r.get(0, 0, 1).copy()
    m.adam()
    r.step(tok, tgt)
    if precision == 1:
        # Adam at t = 1 moves each entry by about lr * sign(g): where dB is
        # near zero, the bf16-level difference in dB flips the step, so the
        # oracle continues from the runner's updated adapters (step-2
        # gradients from identical weights)
        for k in lk:
            m.tensor(0, *k)[:] = r.get(0, *k)
    # second step: B != 0, dA flows; frozen base unchanged bit-for-bit.  bf16:
    # stage by stage (the adapter gradients of each layer from the GPU's own
    # boundary tensors) at the 1e-2 bar.  The whole-step distance of the
    # adapter-on-every-projection case is 1.05e-2 on its top layer's q / k B
    # gradients, at the bf16 step's own sensitivity floor (two correct bf16
    # steps drift apart by about a bf16 ulp once any rounding differs), so a
    # whole-step comparison cannot discriminate there; the grouped rank-r
    # kernels themselves match the oracle within 1e-5 on identical inputs
    # (test_lora_group_bf16_matches_oracle).
    if precision == 0:
        loss_ref = m.forward_backward(tok, tgt)
        loss = r.forward_backward(tok, tgt)
        assert abs(loss - loss_ref) < ltol * abs(loss_ref)
        compare(m, r, lk, 1, tol, "lora grad step 2")
    else:
        stage_compare(m, r, tok, tgt, cfg, tol, "lora step 2 stages")
    assert np.array_equal(base_before, r.get(0, 0, 1))


QWEN3_4B_WIDTHS = dict(dim=2560, n_heads=32, n_kv_heads=8, head_dim=128, ff_dim=9728,
                       vocab_size=151936, tied_embeddings=1, rotary_dim=128, seq_len=2048,
                       n_seqs=1, n_layers=2, lora_targets=0xF, lora_rank=16, lora_alpha=32.0,
                       lora_lr_b_scale=1.0)


@pytest.fixture(scope="module")
def qwen3_4b_pair():
    """Config 4 in every respect except n_layers = 2 (Qwen3-4B widths, 1 x 2048,
    32 / 8 heads of 128, V = 151936 tied, LoRA r = 16 on q/k/v/o over a frozen bf16
    base) and the oracle on the same weights, shared by the step-1 and step-2 tests
    below (each about a minute of oracle work)."""
    note("lora step at Qwen3-4B widths, 2 layers")
    m, r, tok, tgt, cfg = build_pair(1, **QWEN3_4B_WIDTHS)
    yield m, r, tok, tgt, cfg
    r.close()


def test_lora_step_qwen3_4b_widths(qwen3_4b_pair):
    """The kernels the config-4 step launches at their real shapes, i.e. the base
    GEMMs with the rank-16 update in their epilogues on the 128 x 128 plans and the
    split dK/dV grid (8 KV heads x 16 key blocks, launched as 256 blocks), held to
    the oracle's bf16-operand model stage by stage (each layer's output, boundary
    gradient and adapter gradients from the GPU's own boundary tensors) at 1e-2, at
    step 1 (B = 0: dA exactly 0).  Stage by stage because the whole-step bf16
    distance of dB at these widths measured 9.8e-3, at the bf16 step's own
    sensitivity floor."""
    m, r, tok, tgt, cfg = qwen3_4b_pair
    plan = r.attention_backward_plan()
    note(f"  attention backward plan {plan}")
    assert plan["path"] == "recompute" and plan["dkv_blocks"] == 256 and plan["qk_epilogue"], plan
    stage_compare(m, r, tok, tgt, cfg, 1e-2, "lora step 1 stages")
    for (l, w) in lora_keys(cfg):
        if w % 2 == 0:  # dA == 0 exactly at B = 0
            assert np.all(r.get(1, l, w) == 0)


def test_lora_step2_qwen3_4b_widths(qwen3_4b_pair):
    """Step 2 at the same widths (B != 0 after one Adam step, so both adapter
    gradients and the update in the epilogues are live), stage by stage at 1e-2
    from adapters copied to the oracle (see test_lora_step_parity)."""
    m, r, tok, tgt, cfg = qwen3_4b_pair
    r.step(tok, tgt)
    for k in lora_keys(cfg):
        m.tensor(0, *k)[:] = r.get(0, *k)
    stage_compare(m, r, tok, tgt, cfg, 1e-2, "lora step 2 stages")


def test_lora_bf16_base_stored_in_bf16(tmp_path):
    """A bf16 LoRA runner (frozen bf16 base, config 4's class) holds its base
    matrices in bf16 only: no fp32 copy in device memory, set_tensor rounds to
    nearest even and get_tensor returns the bf16 values, the device pointer of
    a base matrix is refused, and a .vkpt checkpoint carries the widened bf16
    values and loads back bit for bit."""
    import valkyr_amd as v
    from valkyr_amd import VkhError
    from valkyr_amd.runner import PARAM

    V = 16384
    c = dict(dim=256, n_heads=4, n_kv_heads=2, head_dim=64, ff_dim=512, n_pos=64, n_layers=2,
             vocab_size=V, rotary_dim=64, qk_norm=1, lora_targets=0b1111, lora_rank=8,
             lora_alpha=16.0)
    with v.Runner(v.make_config(**c, precision=1)) as rb, \
            v.Runner(v.make_config(**c, precision=0)) as rf:
        # embed, lm_head and per layer q, k, v, o, gate, up, down
        base = 2 * V * 256 + 2 * (256 * 256 + 2 * 128 * 256 + 256 * 256 + 3 * 512 * 256)
        # the fp32 runner holds 4 bytes per base weight, the bf16 one 2 (an fp32
        # copy beside the bf16 one would make it 6); activations are small here
        note(f"  device bytes: bf16 base {rb.device_bytes():,}, fp32 base {rf.device_bytes():,}")
        assert rb.device_bytes() < rf.device_bytes() - base
        rng = np.random.default_rng(3)
        x = (0.02 * rng.standard_normal(256 * 256)).astype(np.float32)
        rb.set(PARAM, 0, 1, x)  # q: [256, 256]
        assert np.array_equal(rb.get(PARAM, 0, 1), O.round_bf16(x))
        with pytest.raises(VkhError):
            rb.device_ptr(PARAM, 0, 1)
        rb.device_ptr(PARAM, 0, 16)  # LoRA A of q: fp32
        rb.device_ptr(PARAM, 0, 0)   # n1 gain: fp32
        rb.init_random(seed=4, std=0.02, lora_std=0.02)
        keys = [(-1, 0), (-1, 1), (-1, 2)] + [(l, w) for l in range(2) for w in range(11)]
        for k in keys:
            if k in ((-1, 1),) or k[1] in (0, 5, 9, 10):
                continue
            t = rb.get(PARAM, *k)
            assert np.array_equal(t, O.round_bf16(t)), k  # representable in bf16
        path = str(tmp_path / "b.vkpt")
        rb.save_checkpoint(path)
        with v.Runner(v.make_config(**c, precision=1)) as rc:
            rc.load_checkpoint(path)
            for k in keys:
                assert np.array_equal(rb.get(PARAM, *k), rc.get(PARAM, *k)), k
        # the file holds fp32 values: the embedding blob is the widened bf16 table
        raw = np.fromfile(path, np.uint8)
        body = raw[16 + 80:].view(np.float32)
        assert np.array_equal(body[:V * 256], rb.get(PARAM, -1, 0))


def test_forward_logits_matches_oracle():
    m, r, tok, tgt, cfg = build_pair(0)
    ref = m.forward_logits(tok)
    got = r.forward_logits(tok)
    assert rel_l2(ref, got) < 1e-4


def test_forward_logits_bf16_half_batches():
    """bf16 with an even number of sequences: the forward runs as two concurrent
    half batches (sequence 0 on the main stream, 1 on the second).  The logits
    of the two-sequence batch against the oracle's bf16-operand model."""
    m, r, tok, tgt, cfg = build_pair(1, n_seqs=2, seq_len=64)
    ref = m.forward_logits(tok)
    got = r.forward_logits(tok)
    e = rel_l2(ref, got)
    note(f"  bf16 half-batch forward logits rel-L2 {e:.2e}")
    assert e < 5e-3


def test_loss_decreases_over_steps():
    m, r, tok, tgt, cfg = build_pair(0, lr=1e-3)
    losses = []
    for _ in range(8):
        r.step(tok, tgt)
        losses.append(r.last_loss())
    note(f"  losses {losses[0]:.4f} -> {losses[-1]:.4f}")
    assert losses[-1] < losses[0]
    assert all(np.isfinite(losses))


def test_checkpoint_roundtrip_and_errors(tmp_path):
    import valkyr_amd as v

    m, r, tok, tgt, cfg = build_pair(0, lr=1e-3)
    for _ in range(2):
        r.step(tok, tgt)
    path = str(tmp_path / "a.vkpt")
    r.save_checkpoint(path)
    with open(path, "rb") as f:
        head = f.read(16)
    assert head[:4] == b"VKPT"
    assert int.from_bytes(head[4:8], "little") == 1
    assert int.from_bytes(head[8:12], "little") == 3  # step_t after two steps
    r.step(tok, tgt)
    after_a = r.get(0, 0, 1)
    # a fresh runner resumes from the checkpoint and reproduces the next step bit-for-bit
    m2, r2, _, _, _ = build_pair(0, seed=99, lr=5e-2)
    r2.load_checkpoint(path)
    assert r2.step_t == 3 and abs(r2.lr - 1e-3) < 1e-9
    r2.step(tok, tgt)
    assert np.array_equal(after_a, r2.get(0, 0, 1))
    # corrupted magic, truncated file, config mismatch
    bad = tmp_path / "bad.vkpt"
    data = open(path, "rb").read()
    bad.write_bytes(b"XXXX" + data[4:])
    with pytest.raises(v.VkhError) as e:
        r2.load_checkpoint(str(bad))
    assert e.value.name == "InvalidCheckpointMagic"
    bad.write_bytes(data[: len(data) // 2])
    with pytest.raises(v.VkhError) as e:
        r2.load_checkpoint(str(bad))
    assert e.value.name == "EndOfStream"
    _, r3, _, _, _ = build_pair(0, n_layers=1)
    with pytest.raises(v.VkhError) as e:
        r3.load_checkpoint(path)
    assert e.value.name == "CheckpointConfigMismatch"
    assert int.from_bytes(head[12:16], "little") == 80  # @sizeOf(Config)


# The reference's Config as bytes (transformer.zig:31-77 written by
# std.mem.asBytes): an auto-layout Zig struct, fields by descending alignment
# with declaration order among equals: 19 four-byte fields, the two bools,
# two bytes of padding.
ZIG_CFG = struct.Struct("<8If If 4f 2I 2f 2B 2x")
assert ZIG_CFG.size == 80


def zig_cfg_fields(cfg):
    f32 = lambda x: float(np.float32(x))  # noqa: E731
    return (cfg["dim"], cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"], cfg["ff_dim"],
            cfg["seq_len"], cfg["n_layers"], cfg["vocab_size"], f32(cfg["rms_eps"]),
            cfg["rotary_dim"], f32(cfg["rope_theta"]), f32(cfg["lr"]), f32(cfg["beta1"]),
            f32(cfg["beta2"]), f32(cfg["eps_adam"]), cfg["lora_targets"], cfg["lora_rank"],
            f32(cfg["lora_alpha"]), f32(cfg["lora_lr_b_scale"]), cfg["causal"], cfg["qk_norm"])


def blob_order(cfg):
    """collectBlobs (transformer.zig:1586-1655): (layer, which, numel) per
    tensor, each written as (param, m, v); lm_head is always present."""
    D, F, hd, V = cfg["dim"], cfg["ff_dim"], cfg["head_dim"], cfg["vocab_size"]
    qd, kvd = cfg["n_heads"] * hd, cfg["n_kv_heads"] * hd
    out = [(-1, 0, V * D), (-1, 1, D), (-1, 2, V * D)]
    sizes = [D, qd * D, kvd * D, kvd * D, D * qd, D, F * D, F * D, D * F, hd, hd]
    for l in range(cfg["n_layers"]):
        out += [(l, w, sizes[w]) for w in range(11 if cfg["qk_norm"] else 9)]
    return out


@pytest.mark.parametrize("tied", [0, 1], ids=["untied", "tied"])
def test_checkpoint_file_layout(tmp_path, tied):
    """A saved .vkpt parsed without the loader: header, the reference's
    80-byte Config block, then every blob in collectBlobs order equal to
    get_tensor; a tied runner writes its embedding as lm_head."""
    m, r, tok, tgt, cfg = build_pair(0, lr=1e-3, tied_embeddings=tied)
    r.step(tok, tgt)
    r.step(tok, tgt)
    path = tmp_path / "c.vkpt"
    r.save_checkpoint(str(path))
    data = path.read_bytes()
    assert struct.unpack_from("<4sIII", data, 0) == (b"VKPT", 1, 3, 80)
    assert ZIG_CFG.unpack_from(data, 16) == zig_cfg_fields(cfg)
    off = 16 + 80
    for (l, w, n) in blob_order(cfg):
        src = (-1, 0) if (tied and (l, w) == (-1, 2)) else (l, w)
        for kind in (0, 2, 3):
            blob = np.frombuffer(data, np.float32, n, off)
            off += 4 * n
            assert np.array_equal(blob, r.get(kind, *src)), (l, w, kind)
    assert off == len(data)


def test_checkpoint_written_by_hand_loads(tmp_path):
    """A file laid out as the reference writes it (built here with struct,
    not with the library's writer) loads: every tensor, step_t and the Adam
    hyperparameters; a tied runner takes it only when lm_head = embed."""
    import valkyr_amd as v

    m, r, tok, tgt, cfg = build_pair(0)
    rng = np.random.default_rng(17)
    saved = dict(cfg, lr=3e-3, beta1=0.8, beta2=0.99, eps_adam=1e-7)

    def write(path, cfg_, lm_same_as_embed, cfg_size=80):
        blobs = {}
        with open(path, "wb") as f:
            f.write(struct.pack("<4sIII", b"VKPT", 1, 7, cfg_size))
            f.write(ZIG_CFG.pack(*zig_cfg_fields(cfg_)))
            for (l, w, n) in blob_order(cfg_):
                for kind in (0, 2, 3):
                    if lm_same_as_embed and (l, w) == (-1, 2):
                        a = blobs[(-1, 0, kind)]
                    else:
                        a = rng.standard_normal(n).astype(np.float32) * 0.02
                        if kind == 3:
                            a = np.abs(a)
                    blobs[(l, w, kind)] = a
                    f.write(a.tobytes())
        return blobs

    p1 = str(tmp_path / "ref.vkpt")
    blobs = write(p1, saved, False)
    r.load_checkpoint(p1)
    assert r.step_t == 7 and abs(r.lr - 3e-3) < 1e-9
    for (l, w, kind), a in blobs.items():
        assert np.array_equal(r.get(kind, l, w), a), (l, w, kind)
    # the restored Adam state steps like an oracle restored the same way
    mo = O.Model(**saved)
    for (l, w, kind), a in blobs.items():
        mo.tensor(kind, l, w)[:] = a
    mo.step_t = 7
    mo.step(tok, tgt)
    r.step(tok, tgt)
    compare(mo, r, tensor_keys(cfg), 0, 1e-5, "params after resuming")
    compare(mo, r, tensor_keys(cfg), 2, 1e-3, "adam m after resuming")
    # tied runners: lm_head must equal the embedding
    _, rt, _, _, _ = build_pair(0, tied_embeddings=1)
    p2 = str(tmp_path / "tied_ok.vkpt")
    b2 = write(p2, dict(saved, tied_embeddings=1), True)
    rt.load_checkpoint(p2)
    assert np.array_equal(rt.get(0, -1, 0), b2[(-1, 0, 0)])
    with pytest.raises(v.VkhError) as e:
        rt.load_checkpoint(p1)
    assert e.value.name == "CheckpointConfigMismatch"
    p3 = str(tmp_path / "size.vkpt")
    write(p3, saved, False, cfg_size=84)
    with pytest.raises(v.VkhError) as e:
        r.load_checkpoint(p3)
    assert e.value.name == "CheckpointConfigSizeMismatch"


def test_lora_checkpoint_roundtrip(tmp_path):
    import valkyr_amd as v

    over = dict(lora_targets=0xF, lora_rank=16, lora_alpha=32.0, lora_lr_b_scale=4.0, lr=1e-3)
    m, r, tok, tgt, cfg = build_pair(0, **over)
    for _ in range(2):
        r.step(tok, tgt)
    path = str(tmp_path / "a.lvkpt")
    r.save_lora_checkpoint(path)
    assert open(path, "rb").read(4) == b"VLKP"
    _, r2, _, _, _ = build_pair(0, seed=7, **over)
    r2.load_lora_checkpoint(path)
    for k in lora_keys(cfg):
        assert np.array_equal(r.get(0, *k), r2.get(0, *k))
    _, rf, _, _, _ = build_pair(0)
    with pytest.raises(v.VkhError) as e:
        rf.save_lora_checkpoint(path)
    assert e.value.name == "LoraCheckpointEmpty"


def test_tick_frame_train_budget_and_loss_latency():
    from valkyr_amd.device import Stream

    m, r, tok, tgt, cfg = build_pair(0, lr=1e-3)
    r.upload_train_batch(tok, tgt)
    s = Stream()
    res = r.tick_frame_train(steps=3, stream=s)
    assert res.steps_completed == 3 and not res.has_loss
    s.synchronize()
    res2 = r.tick_frame_train(steps=1, stream=s)
    assert res2.has_loss and np.isfinite(res2.last_loss)
    s.synchronize()
    assert r.step_t == 5
    r.set_loss_target(1e9)  # any loss is below: the next tick goes idle
    res3 = r.tick_frame_train(steps=2, stream=s)
    assert res3.idle and res3.steps_completed == 0


def test_tick_frame_train_loss_target_resumes_on_new_batch():
    """runner.zig:948-973: under a loss target every tick stages a fresh loss
    evaluation, so a newly uploaded batch whose loss is above the target
    resumes training after an idle tick."""
    from valkyr_amd.device import Stream

    m, r, tok, tgt, cfg = build_pair(0, lr=1e-2)
    tok_b = O.ids(len(tok), 555, cfg["vocab_size"])
    tgt_b = O.ids(len(tok), 556, cfg["vocab_size"])
    s = Stream()
    r.upload_train_batch(tok, tgt)
    r.set_loss_target(1e9)
    res = r.tick_frame_train(steps=3, stream=s)  # nothing measured yet: trains
    assert res.steps_completed == 3 and not res.idle and not res.has_loss
    s.synchronize()
    res = r.tick_frame_train(steps=3, stream=s)  # staged eval <= 1e9: idle
    assert res.idle and res.steps_completed == 0 and res.has_loss
    loss_a = res.last_loss
    assert loss_a == r.forward_backward(tok, tgt)  # the eval of batch A, bit for bit
    loss_b = r.forward_backward(tok_b, tgt_b)
    note(f"  loss A after 3 steps {loss_a:.4f}, batch B {loss_b:.4f}")
    assert loss_b > loss_a
    r.set_loss_target(0.5 * (loss_a + loss_b))
    r.upload_train_batch(tok_b, tgt_b)
    res = r.tick_frame_train(steps=2, stream=s)  # still A's loss: idle, stages B's
    assert res.idle and res.steps_completed == 0 and res.last_loss == loss_a
    s.synchronize()
    res = r.tick_frame_train(steps=2, stream=s)  # B's loss > target: trains again
    assert not res.idle and res.steps_completed == 2 and res.last_loss == loss_b
    s.synchronize()
    assert r.step_t == 6


def test_tick_frame_train_budget_edges():
    """runner.zig:924-926: a zero step or microsecond budget is an idle tick
    that reports the cached loss; an unknown budget mode is an error."""
    import valkyr_amd as v
    from valkyr_amd.runner import BUDGET_EITHER, BUDGET_MICROSECONDS

    m, r, tok, tgt, cfg = build_pair(0)
    r.upload_train_batch(tok, tgt)
    assert r.tick_frame_train(steps=1).steps_completed == 1
    r.synchronize()
    for kw in (dict(steps=0), dict(mode=BUDGET_MICROSECONDS, microseconds=0),
               dict(mode=BUDGET_EITHER, steps=0, microseconds=10**6),
               dict(mode=BUDGET_EITHER, steps=5, microseconds=0)):
        res = r.tick_frame_train(**kw)
        assert res.idle and res.steps_completed == 0 and res.has_loss, kw
    assert r.step_t == 2
    with pytest.raises(v.VkhError) as e:
        r.tick_frame_train(steps=1, mode=7)
    assert e.value.name == "InvalidArgument"
    res = r.tick_frame_train(mode=BUDGET_EITHER, steps=3, microseconds=10**9)
    assert res.steps_completed == 3


def test_caller_stream_work_orders_before_later_calls(tmp_path):
    """Steps enqueued on a caller stream are complete before a later
    get_tensor / save_checkpoint / step on the runner stream touches the same
    memory, with no synchronisation by the caller."""
    from valkyr_amd.device import Stream

    m, r1, tok, tgt, cfg = build_pair(0, lr=1e-3)
    _, r2, _, _, _ = build_pair(0, lr=1e-3)
    tok2 = O.ids(len(tok), 77, cfg["vocab_size"])
    s = Stream()
    for i in range(3):
        r1.step_async(tok if i % 2 == 0 else tok2, tgt, stream=s)
        r2.step(tok if i % 2 == 0 else tok2, tgt)
    for k in tensor_keys(cfg):
        assert np.array_equal(r1.get(0, *k), r2.get(0, *k)), k
    r1.step_async(tok, tgt, stream=s)
    r1.save_checkpoint(str(tmp_path / "1.vkpt"))
    r2.step(tok, tgt)
    r2.save_checkpoint(str(tmp_path / "2.vkpt"))
    assert (tmp_path / "1.vkpt").read_bytes() == (tmp_path / "2.vkpt").read_bytes()
    # caller stream, then the runner's own stream, then the caller stream again
    r1.step_async(tok2, tgt, stream=s)
    r1.step(tok, tgt)
    r1.step_async(tok2, tgt, stream=s)
    for t in (tok2, tok, tok2):
        r2.step(t, tgt)
    assert r1.last_loss() == r2.last_loss()
    for k in tensor_keys(cfg):
        assert np.array_equal(r1.get(2, *k), r2.get(2, *k)), k


def test_runner_error_paths():
    import valkyr_amd as v

    m, r, tok, tgt, cfg = build_pair(0)
    with pytest.raises(v.VkhError) as e:
        r.step(tok[:-1], tgt)
    assert e.value.name == "TokenIdsLen"
    with pytest.raises(v.VkhError) as e:
        r.step(tok, tgt[:-1])
    assert e.value.name == "TargetLen"
    bad = tok.copy()
    bad[3] = cfg["vocab_size"]
    with pytest.raises(v.VkhError) as e:
        r.step(bad, tgt)
    assert e.value.name == "TokenOutOfRange"
    w = {"embed": np.zeros(10, np.float32), "final_norm": np.ones(256, np.float32),
         "lm_head": None, "layers": []}
    with pytest.raises(v.VkhError) as e:
        v.Runner(r.cfg, w)
    assert e.value.name == "EmbedShape"


def test_nonfinite_weights_give_nonfinite_loss():
    m, r, tok, tgt, cfg = build_pair(0)
    w = r.get(0, 0, 1)
    w[5] = np.nan
    r.set(0, 0, 1, w)
    loss = r.forward_backward(tok, tgt)
    assert not np.isfinite(loss)


def test_finetune_loop_matches_manual_steps():
    """vkh_runner_finetune (commands/finetune.zig:155-196) against the same loop
    driven step by step from the host: identical weights and CE values."""
    from valkyr_amd.dataset import Dataset, finetune, mean_ce

    note("finetune loop")
    cfg = dict(CONFIG1, n_seqs=2, seq_len=64)
    m, r1, _, _, _ = build_pair(0, n_seqs=2, seq_len=64)
    _, r2, _, _, _ = build_pair(0, n_seqs=2, seq_len=64)
    rng = np.random.default_rng(3)
    ex = [rng.integers(0, cfg["vocab_size"], rng.integers(20, 200)).tolist() for _ in range(12)]
    ds = Dataset.from_examples(ex, n_pos=64, eos_id=1)
    nb = ds.num_batches()
    res = finetune(r1, ds, batch_idx=5, n_steps=4, rotate=True)
    # the same loop by hand on the second runner
    V, T = cfg["vocab_size"], 128
    tok, tgt = ds.batch_seqs(5, 64, 2)
    ce0 = mean_ce(r2.forward_logits(tok), tgt, V)
    for step in range(4):
        a, b = ds.batch_seqs((step + 5) % nb, 64, 2)
        r2.step(a, b)
    ce1 = mean_ce(r2.forward_logits(tok), tgt, V)
    note(f"  CE {res['ce_initial']:.4f} -> {res['ce_final']:.4f} (manual {ce0:.4f} -> {ce1:.4f}), "
         f"{res['mean_step_ms']:.2f} ms/step")
    assert res["ce_initial"] == ce0 and res["ce_final"] == ce1
    assert res["ce_final"] < res["ce_initial"]
    for k in tensor_keys(cfg):
        assert np.array_equal(r1.get(0, *k), r2.get(0, *k)), k
    # errors of finetune.zig:132-135
    import valkyr_amd as v
    short = Dataset.from_examples([[1, 2, 3]], n_pos=64, eos_id=1)
    with pytest.raises(v.VkhError) as e:
        finetune(r1, short, 0, 1)
    assert e.value.name == "DatasetTooShort"
    with pytest.raises(v.VkhError) as e:
        finetune(r1, ds, nb, 1)
    assert e.value.name == "BatchIdxOutOfRange"
