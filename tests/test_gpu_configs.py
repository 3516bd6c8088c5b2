"""The metric's configs 3, 4 and 5 at full size through the C ABI, held to the
size-independent properties those shapes allow (no oracle runs at this size;
config 3's widths are held to the oracle at 2 layers in test_gpu_runner.py):

* the loss of a random init: after the unit-gain final RMSNorm every logit of
  a N(0, s^2) head is N(0, D s^2), so the mean CE is ln V + D s^2 / 2 up to the
  target logits' sampling noise, std sqrt(D s^2 / T);
* config 3 (Qwen3-0.6B shape, 4 x 512, 28 layers, tied 151936 vocabulary):
  the step takes the recompute attention backward, gradients of sampled
  tensors are finite and non-zero, the bf16-operand gradients agree with the
  fp32-precision runner's on the same weights, and the loss falls over
  repeated steps on one batch;
* config 4 (Qwen3-4B shape, LoRA r16 on q/k/v/o, frozen base): at step 1
  B = 0 makes every dA exactly zero (lora.zig:449-505), dB is live, and A and
  the frozen base weights are unchanged bit for bit after the update;
* config 5 (Qwen3-8B shape, 1 x 8192, full fine-tune with per-layer
  activation recompute): the runner fits in 160 GiB (fp32 master weights, their
  bf16 copy, gradients and two Adam moments are 137 GiB of it), gradients are
  finite, and a second step on the same batch lowers the loss.

A box without the memory for a configuration skips it (OutOfMemory) rather
than failing.
"""
import math

import numpy as np
import pytest

from helpers import note

pytestmark = pytest.mark.gpu

BASE = dict(head_dim=128, n_heads=32, n_kv_heads=8, vocab_size=151936, rms_eps=1e-6, causal=1,
            rotary_dim=128, rope_theta=1e6, qk_norm=1, lr=1e-4, beta1=0.9, beta2=0.999,
            eps_adam=1e-8, n_seqs=1)
CONFIG3 = dict(BASE, n_heads=16, dim=1024, ff_dim=3072, n_pos=512, n_seqs=4, n_layers=28,
               tied_embeddings=1)
CONFIG4 = dict(BASE, dim=2560, ff_dim=9728, n_pos=2048, n_layers=36, tied_embeddings=1,
               lora_targets=0xF, lora_rank=16, lora_alpha=32.0, lora_lr_b_scale=1.0)
CONFIG5 = dict(BASE, dim=4096, ff_dim=12288, n_pos=8192, n_layers=36, tied_embeddings=0,
               recompute=1)


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    import valkyr_amd as v

    assert v.device_count() > 0, "no GPU visible"


def runner(c, precision=1):
    import valkyr_amd as v

    try:
        r = v.Runner(v.make_config(**c, precision=precision))
    except v.VkhError as e:
        if e.name == "OutOfMemory":
            pytest.skip(f"not enough device memory: {e.message}")
        raise
    r.init_random(seed=7, std=0.02, lora_std=0.02)
    return r


def batch(c, seed):
    rng = np.random.default_rng(seed)
    T = c["n_pos"] * c["n_seqs"]
    return (rng.integers(0, c["vocab_size"], T, dtype=np.uint32),
            rng.integers(0, c["vocab_size"], T, dtype=np.uint32))


def loss_closed_form_ok(c, loss):
    var, T = c["dim"] * 0.02 ** 2, c["n_pos"] * c["n_seqs"]
    want = math.log(c["vocab_size"]) + var / 2
    note(f"  loss {loss:.4f}, closed form {want:.4f} +- {math.sqrt(var / T):.4f}")
    return abs(loss - want) < 4 * math.sqrt(var / T) + 0.01


def test_config3_qwen3_06b_full_size():
    from helpers import rel_l2
    from valkyr_amd.runner import DOWN, GATE, GRAD, K, N1, N2, O, Q, Q_NORM, UP

    c = CONFIG3
    note("config 3 full size: Qwen3-0.6B shape, 4 x 512, 28 layers, tied vocabulary")
    sampled = [(-1, 0), (-1, 1), (0, Q), (0, N1), (0, DOWN), (9, K), (13, N2), (13, UP),
               (20, Q_NORM), (27, O), (27, GATE)]
    tok, tgt = batch(c, 3)
    with runner(c) as r:
        assert r.param_count() == 596_049_920
        assert r.attention_backward_path() == "recompute"
        loss = r.forward_backward(tok, tgt)  # first-step gradients, no update
        assert loss_closed_form_ok(c, loss)
        g16 = {k: r.get(GRAD, *k) for k in sampled}
        for k, g in g16.items():
            assert np.isfinite(g).all() and g.any(), k
        with runner(c, precision=0) as r32:  # same seed: same fp32 weights
            loss32 = r32.forward_backward(tok, tgt)
            note(f"  first-step loss bf16 {loss:.5f}, fp32 {loss32:.5f}")
            assert abs(loss - loss32) < 1e-3 * loss32
            errs = {k: rel_l2(r32.get(GRAD, *k), g16[k]) for k in sampled}
        note("  bf16 vs fp32 gradient rel-L2: " + ", ".join(f"{k}: {e:.2e}" for k, e in errs.items()))
        assert max(errs.values()) < 5e-2, errs
        losses = []
        for _ in range(4):
            r.step(tok, tgt)
            losses.append(r.last_loss())
        note(f"  losses over 4 steps on one batch: {losses}")
        assert all(np.isfinite(losses)) and losses[-1] < losses[0] and losses[0] == loss
        assert r.step_t == 5


def test_config4_qwen3_4b_lora_first_step():
    from valkyr_amd.runner import DOWN, GRAD, PARAM, Q, lora_a, lora_b

    c = CONFIG4
    note("config 4 full size: Qwen3-4B shape, LoRA r16 q/k/v/o, 1 x 2048")
    with runner(c) as r:
        assert r.param_count() == 11_796_480  # the 11.8 M trainable parameters
        L = c["n_layers"]
        a0 = {(l, p): r.get(PARAM, l, lora_a(p)) for l in (0, L // 2, L - 1) for p in range(4)}
        w0 = {(l, w): r.get(PARAM, l, w) for l, w in ((0, Q), (L - 1, DOWN))}
        tok, tgt = batch(c, 4)
        r.step(tok, tgt)
        assert loss_closed_form_ok(c, r.last_loss())
        for l in range(L):
            for p in range(4):
                assert not r.get(GRAD, l, lora_a(p)).any(), (l, p)
        for l in (0, L - 1):
            for p in range(4):
                g = r.get(GRAD, l, lora_b(p))
                assert np.isfinite(g).all() and g.any(), (l, p)
        for (l, p), a in a0.items():
            assert np.array_equal(r.get(PARAM, l, lora_a(p)), a), (l, p)
        for (l, w), x in w0.items():
            assert np.array_equal(r.get(PARAM, l, w), x), (l, w)
        r.step(tok, tgt)  # B is no longer zero: dA comes alive
        assert r.get(GRAD, 0, lora_a(0)).any()


def test_config5_qwen3_8b_long_context_first_steps():
    from valkyr_amd.runner import GRAD, Q

    c = CONFIG5
    note("config 5 full size: Qwen3-8B shape, full fine-tune, 1 x 8192")
    with runner(c) as r:
        note(f"  {r.param_count():,} params, {r.device_bytes() / 2**30:.1f} GiB")
        assert r.device_bytes() < 160 * 2**30
        tok, tgt = batch(c, 5)
        r.step(tok, tgt)
        l0 = r.last_loss()
        assert loss_closed_form_ok(c, l0)
        g = r.get(GRAD, 0, Q)
        assert np.isfinite(g).all() and g.any()
        r.step(tok, tgt)
        l1 = r.last_loss()
        note(f"  second step loss {l1:.4f}")
        assert l1 < l0
