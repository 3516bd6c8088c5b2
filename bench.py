"""Benchmark: the headline training metric on one MI355X.

  train tokens/s of a Qwen3-0.6B-shaped fwd + bwd + Adam step (config 3:
  28 layers, dim 1024, 16/8 heads, head_dim 128, QK-norm, SwiGLU 3072,
  vocab 151936 tied, batch 4 x seq 512, bf16 operands with fp32 master
  weights / accumulation / Adam), synthetic random-init weights and
  uniform token ids.

One JSON line on stdout.  `roofline` is the FA-2 backward (the D row-dot
preprocess + dK/dV + dQ, one call) at config 2 (B=4, S=2048, 16/8 heads, hd 128, causal, bf16
Q/K/V/dO and bf16 O from the forward), timed with HIP events on the stream it
runs on; its algorithmic work is 10 * B * Hq * hd * S(S+1)/2 = 171.88 GFLOP
per call.
`reference_precision_step` is the same step with fp32 operands throughout (the
reference's own precision).
`cpu_baseline` is the C oracle (a restatement of valkyr's CPU reference path,
fp64 accumulators) timed on this host on a bounded sample, each cost timed
directly, scaled to tokens/s of the same step (see `sample`): all host threads
(`value`, OpenMP over independent outputs, same bits as one thread) and one
thread (`single_thread`).

usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--precision bf16|fp32]
                       [--no-cpu-baseline] [--no-configs] [--fa-reps R]
                       [--only all|step|fa|mlp|bw|gemms|config4|config5] [--calib-copy]

`bandwidth_kernels` times the HBM-bound backward kernels alone through the C ABI at
config-3 shapes (RMSNorm, SwiGLU, RoPE backward, Adam, embedding backward) against
the 8 TB/s HBM peak.
`--only gemms` times the twelve per-layer GEMMs of config 3 alone through the C ABI,
with hipBLASLt (torch.mm) on the same shapes when torch is importable.
`mlp_runner` times the tiny-MLP TrainingRunner (train/runner.zig): the
reference's `--train-demo` loop and tickFrameTrain on batches.  `configs` runs
the metric's Qwen3-4B LoRA (config 4) and Qwen3-8B long-context full fine-tune
with per-layer activation recompute (config 5) at full size: device memory,
step time, TFLOP/s of the step's algorithmic work, size-independent checks
(`--only config4` / `--only config5` run one alone, `--no-configs` skips them).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
FP32_PEAK_TFLOPS = 157.3

# config 3 of the metric: the Qwen3-0.6B-shaped full fine-tune step
QWEN3_06B = dict(dim=1024, n_heads=16, n_kv_heads=8, head_dim=128, ff_dim=3072, n_pos=512,
                 n_layers=28, vocab_size=151936, rms_eps=1e-6, causal=1, rotary_dim=128,
                 rope_theta=1e6, qk_norm=1, lr=1e-4, beta1=0.9, beta2=0.999, eps_adam=1e-8,
                 n_seqs=4, tied_embeddings=1)


# configs 4 and 5 of the metric (parity / capacity cases, not the headline line)
QWEN3_4B_LORA = dict(dim=2560, n_heads=32, n_kv_heads=8, head_dim=128, ff_dim=9728, n_pos=2048,
                     n_layers=36, vocab_size=151936, rms_eps=1e-6, causal=1, rotary_dim=128,
                     rope_theta=1e6, qk_norm=1, lr=1e-4, beta1=0.9, beta2=0.999, eps_adam=1e-8,
                     n_seqs=1, tied_embeddings=1, lora_targets=0xF, lora_rank=16,
                     lora_alpha=32.0, lora_lr_b_scale=1.0)
QWEN3_8B = dict(dim=4096, n_heads=32, n_kv_heads=8, head_dim=128, ff_dim=12288, n_pos=8192,
                n_layers=36, vocab_size=151936, rms_eps=1e-6, causal=1, rotary_dim=128,
                rope_theta=1e6, qk_norm=1, lr=1e-4, beta1=0.9, beta2=0.999, eps_adam=1e-8,
                n_seqs=1, tied_embeddings=0, recompute=1)


def step_flops(c) -> float:
    """Algorithmic FLOP of one step: 6 * tokens * matmul params (4 with a frozen
    base: no weight gradients), the CCE head (6 T V D; 4 when frozen), causal
    attention (forward 2 GEMMs, backward 5), and each LoRA adapter's six rank-r
    products (6 T r (K + N)).  Activation recompute is not counted: it is work
    the step repeats, not work the model needs."""
    T = c["n_pos"] * c["n_seqs"]
    D, F, V, L = c["dim"], c["ff_dim"], c["vocab_size"], c["n_layers"]
    qd, kvd = c["n_heads"] * c["head_dim"], c["n_kv_heads"] * c["head_dim"]
    p_mat = L * (D * (qd + 2 * kvd) + qd * D + 3 * D * F)
    lora = c.get("lora_targets", 0)
    gemm = (4.0 if lora else 6.0) * T * p_mat
    cce = (4.0 if lora else 6.0) * T * V * D
    S, H, hd = c["n_pos"], c["n_heads"], c["head_dim"]
    causal_pairs = c["n_seqs"] * S * (S + 1) / 2
    attn = L * H * hd * causal_pairs * (4 + 10)  # fwd 2 GEMMs (4), bwd 5 GEMMs (10)
    nk = [(qd, D), (kvd, D), (kvd, D), (D, qd), (F, D), (F, D), (D, F)]  # (N, K) per projection
    adapters = sum(6.0 * T * c["lora_rank"] * (n + k) for p, (n, k) in enumerate(nk)
                   if lora & (1 << p)) * L
    return gemm + cce + attn + adapters


def bench_step(args, dev_info, precision=None, steps=None, warmup=None):
    import valkyr_amd as v
    from valkyr_amd.device import Event

    c = dict(QWEN3_06B)
    precision = precision or args.precision
    steps = steps or args.steps
    warmup = args.warmup if warmup is None else warmup
    prec = 1 if precision == "bf16" else 0
    cfg = v.make_config(**c, precision=prec)
    r = v.Runner(cfg)
    r.init_random(seed=20261201, std=0.02)
    T = c["n_pos"] * c["n_seqs"]
    rng = np.random.default_rng(1)
    tok = rng.integers(0, c["vocab_size"], T, dtype=np.uint32)
    tgt = rng.integers(0, c["vocab_size"], T, dtype=np.uint32)
    print(f"[bench] runner ready: {r.param_count():,} params, "
          f"{r.device_bytes() / 2**30:.1f} GiB device memory", file=sys.stderr, flush=True)
    for _ in range(warmup):
        r.step_async(tok, tgt)
    r.synchronize()
    loss0 = r.last_loss()
    e0, e1 = Event(), Event()
    r.synchronize()
    t0 = time.perf_counter()
    e0.record()
    for _ in range(steps):
        r.step_async(tok, tgt)
    r.synchronize()
    e1.record()
    e1.synchronize()
    t1 = time.perf_counter()
    wall = t1 - t0
    loss1 = r.last_loss()
    ms = 1000.0 * wall / steps
    tokens_s = T * steps / wall
    flops = step_flops(c)
    print(f"[bench] {precision} step {ms:.2f} ms, {tokens_s:,.0f} tok/s, loss {loss0:.4f} -> {loss1:.4f}",
          file=sys.stderr, flush=True)
    r.close()
    return dict(ms=ms, tokens_s=tokens_s, T=T, flops=flops, loss_first=loss0, loss_last=loss1,
                params=None)


def bench_fa_bwd(args):
    """FA-2 backward at config 2, events on the launch stream."""
    from valkyr_amd import kernels as K
    from valkyr_amd.device import DeviceBuffer, Event, Stream, f32_to_bf16_bits

    B, S, H, Hkv, hd = 4, 2048, 16, 8, 128
    rng = np.random.default_rng(2)
    nq, nk = B * S * H * hd, B * S * Hkv * hd
    q = DeviceBuffer.from_numpy(f32_to_bf16_bits(rng.standard_normal(nq, np.float32)))
    k = DeviceBuffer.from_numpy(f32_to_bf16_bits(rng.standard_normal(nk, np.float32)))
    vv = DeviceBuffer.from_numpy(f32_to_bf16_bits(rng.standard_normal(nk, np.float32)))
    # config 2: dO ~N(0, 1e-2) in bf16; O (bf16) and LSE from the forward of the same inputs
    dout16 = DeviceBuffer.from_numpy(
        f32_to_bf16_bits((0.1 * rng.standard_normal(nq)).astype(np.float32)))
    o = DeviceBuffer(nq * 4)
    o16 = DeviceBuffer(nq * 2)
    lse = DeviceBuffer(B * S * H * 4)
    d = DeviceBuffer(B * S * H * 4)
    dq, dk, dv = DeviceBuffer(nq * 4), DeviceBuffer(nk * 4), DeviceBuffer(nk * 4)
    p = K.attn_params(S, S, H, Hkv, hd, True, B, K.BF16)
    ws = DeviceBuffer(max(K.fa_backward_workspace_bytes(p), 4))  # bf16 dS if the shape needs it
    s = Stream()
    K.fa_forward(p, q, k, vv, o, lse, stream=s)  # O and LSE of the same inputs
    K.cast_f32_to_bf16(o, o16, nq, stream=s)

    def once():  # D preprocess + dK/dV + dQ
        K.fa_backward_from_o(p, q, k, vv, o16, dout16, lse, d, dq, dk, dv, ws, stream=s)

    # the GPU clock ramps up over the first ~100 back-to-back calls (0.39 ms ->
    # 0.33 ms per call); the timed calls measure the settled state, as in training
    for _ in range(args.fa_warmup):
        once()
    s.synchronize()
    e0, e1 = Event(), Event()
    e0.record(s)
    for _ in range(args.fa_reps):
        once()
    e1.record(s)
    e1.synchronize()
    ms = e0.elapsed_ms(e1) / args.fa_reps
    flops = 10.0 * B * H * hd * S * (S + 1) / 2
    tflops = flops / (ms * 1e-3) / 1e12
    print(f"[bench] fa-bwd {ms:.3f} ms, {tflops:.1f} TFLOP/s", file=sys.stderr, flush=True)
    return dict(ms=ms, flops=flops, tflops=tflops)


HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, AMD published


def bench_bandwidth(args):
    """The bandwidth-bound backward kernels alone, through the C ABI, at config-3 shapes.

    Each kernel cycles through enough independent buffer sets that the data
    cannot stay in the 256 MB Infinity Cache (>= 768 MB per kernel), so the
    rate is an HBM rate; HIP events on the launch stream around R calls.
    `bytes` is each call's algorithmic traffic (compulsory reads + writes,
    fp32), `frac` the fraction of the 8 TB/s HBM peak, `frac_of_copy` the
    fraction of the measured streaming-copy rate at the same byte count
    (`copy_GB_s`: a read+write stream's ceiling falls with its size, from
    ~6.2 TB/s at >= 512 MB to under 4 TB/s at 8 MB)."""
    from valkyr_amd import kernels as K
    from valkyr_amd.device import DeviceBuffer, Event, Stream

    T, D, F, H, Hkv, hd = 2048, 1024, 3072, 16, 8, 128
    rng = np.random.default_rng(11)
    s = Stream()

    def sets_for(nbytes):
        return max(2, int(np.ceil(768e6 / nbytes)))

    def rand_like(n, nsets, scale=1.0):
        host = (scale * rng.standard_normal(n)).astype(np.float32)
        first = DeviceBuffer.from_numpy(host)
        out = [first]
        for _ in range(nsets - 1):
            b = DeviceBuffer(n * 4)
            K.scale(first, b, n, 1.0, stream=s)
            out.append(b)
        return out

    def timed(call, nsets, reps):
        for i in range(2 * nsets):
            call(i % nsets)
        s.synchronize()
        e0, e1 = Event(), Event()
        e0.record(s)
        for i in range(reps):
            call(i % nsets)
        e1.record(s)
        e1.synchronize()
        return e0.elapsed_ms(e1) / reps

    res = {}

    def copy_ceiling(nbytes):
        """The library's streaming copy (vkh_scale: chunked, non-temporal, n
        floats in and n out) moving the same bytes per call, cycled over the
        same >= 768 MB of buffer sets: the rate this part gives a plain
        read+write stream of that size."""
        n = max(4, int(nbytes) // 8 // 4 * 4)
        k = sets_for(8 * n)
        src = [DeviceBuffer(n * 4) for _ in range(k)]
        dst = [DeviceBuffer(n * 4) for _ in range(k)]
        ms = timed(lambda i: K.scale(src[i], dst[i], n, 1.0, stream=s), k, 4 * k)
        return 8 * n / (ms * 1e-3) / 1e9

    def row(name, ms, nbytes, shape):
        gbs = nbytes / (ms * 1e-3) / 1e9
        ceil = copy_ceiling(nbytes)
        res[name] = {"shape": shape, "us": round(ms * 1e3, 2), "bytes": int(nbytes),
                     "GB_s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "copy_GB_s": round(ceil, 1), "frac_of_copy": round(gbs / ceil, 4)}
        print(f"[bench] {name}: {ms * 1e3:.1f} us, {gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS:.1%} of "
              f"8 TB/s, {gbs / ceil:.1%} of the {ceil:.0f} GB/s copy of the same bytes)",
              file=sys.stderr, flush=True)

    # RMSNorm backward with residual add and gain gradient: dy, x, res in; dx out
    n = T * D
    nb = 4 * n * 4
    k = sets_for(nb)
    dy, x, res_, dx = rand_like(n, k), rand_like(n, k), rand_like(n, k), rand_like(n, k)
    w = DeviceBuffer.from_numpy(np.ones(D, np.float32))
    dw = DeviceBuffer(D * 4)
    ms = timed(lambda i: K.rmsnorm_backward(dy[i], x[i], w, dx[i], dw, T, D, 1e-6, residual=res_[i],
                                            stream=s), k, 8 * k)
    row("rmsnorm_backward", ms, nb + 2 * D * 4, f"[{T}, {D}] + residual, gain gradient")
    del dy, x, res_, dx
    # SwiGLU backward: d_gated, pre_gate, up in; d_pre_gate, d_up out
    n = T * F
    nb = 5 * n * 4
    k = sets_for(nb)
    dg, pg, up, dpg, dup = (rand_like(n, k) for _ in range(5))
    ms = timed(lambda i: K.swiglu_backward(dg[i], pg[i], up[i], dpg[i], dup[i], n, stream=s), k, 4 * k)
    row("swiglu_backward", ms, nb, f"[{T}, {F}]")
    del dg, pg, up, dpg, dup
    # RoPE backward over q and k (qk_rope_backward_batched): in and out
    nq, nk = T * H * hd, T * Hkv * hd
    nb = 2 * (nq + nk) * 4
    k = sets_for(nb)
    rp = K.rope_params(T, H, Hkv, hd, hd, 1e6, seq_len=512)
    dqo, dqi, dko, dki = rand_like(nq, k), rand_like(nq, k), rand_like(nk, k), rand_like(nk, k)
    ms = timed(lambda i: K.qk_rope_backward(rp, dqo[i], dqi[i], dko[i], dki[i], stream=s), k, 8 * k)
    row("qk_rope_backward", ms, nb, f"q [{T}, {H}, {hd}] + k [{T}, {Hkv}, {hd}], seq 512")
    del dqo, dqi, dko, dki
    # Adam over a 128 Mi-parameter span: p, g, m, v in; p, m, v out
    n = 128 << 20
    nb = 7 * n * 4
    pp, gg = rand_like(n, 1, 0.02), rand_like(n, 1, 1e-3)
    mm, vv = DeviceBuffer.zeros(n * 4), DeviceBuffer.zeros(n * 4)
    ms = timed(lambda i: K.adam_step(pp[0], gg[0], mm, vv, n, 1e-4, 0.9, 0.999, 1e-8, 1, stream=s),
               1, 5)
    row("adam_step", ms, nb, f"{n} params")
    del pp, gg, mm, vv
    # Embedding backward (accumulate into dE): dy read, touched dE rows read + written
    V = 151936
    ids_h = rng.integers(0, V, T).astype(np.uint32)
    distinct = len(np.unique(ids_h))
    nb = T * D * 4 + 2 * distinct * D * 4
    ids = DeviceBuffer.from_numpy(ids_h)
    dyb = rand_like(T * D, 1)
    dE = DeviceBuffer.zeros(V * D * 4)
    ms = timed(lambda i: K.embedding_backward(dyb[0], ids, dE, T, D, V, stream=s), 1, 20)
    row("embedding_backward", ms, nb, f"{T} ids into [{V}, {D}], accumulate")
    return res


# The twelve linear-layer GEMMs of one config-3 layer (T = 2048 tokens): name, kind
# (nt: y = x W^T forward; dx: dx = dy W; dw: dW = dy^T x), M (tokens), N (outputs), K (inputs)
LAYER_GEMMS = [("qkv fwd", "nt", 2048, 4096, 1024), ("o fwd", "nt", 2048, 1024, 2048),
               ("gate/up fwd", "nt", 2048, 6144, 1024), ("down fwd", "nt", 2048, 1024, 3072),
               ("down dx", "dx", 2048, 1024, 3072), ("gate/up dx", "dx", 2048, 6144, 1024),
               ("o dx", "dx", 2048, 1024, 2048), ("qkv dx", "dx", 2048, 4096, 1024),
               ("down dW", "dw", 2048, 1024, 3072), ("gate/up dW", "dw", 2048, 6144, 1024),
               ("o dW", "dw", 2048, 1024, 2048), ("qkv dW", "dw", 2048, 4096, 1024)]


def bench_gemms(args):
    """The per-layer GEMMs of config 3 alone, through the C ABI (bf16 operands, fp32
    out; the kernels the step launches, without the second stream sharing the chip),
    HIP events on the launch stream around 50 calls after 10 warm-up calls.  With
    --hipblaslt, hipBLASLt (torch.mm, bf16 operands and output) is timed on the same
    shapes beside them as a library reference point (torch is not imported otherwise,
    so counter runs of this leg see only the library's kernels)."""
    from valkyr_amd import kernels as K
    from valkyr_amd.device import DeviceBuffer, Event, Stream, f32_to_bf16_bits

    rng = np.random.default_rng(5)
    s = Stream()
    reps = 50

    def ev_time(call):
        for _ in range(10):
            call()
        s.synchronize()
        e0, e1 = Event(), Event()
        e0.record(s)
        for _ in range(reps):
            call()
        e1.record(s)
        e1.synchronize()
        return e0.elapsed_ms(e1) / reps

    have_torch = False
    if args.hipblaslt:
        try:
            import torch
            have_torch = torch.cuda.is_available()
            if not have_torch:
                print("[bench] --hipblaslt: torch sees no GPU", file=sys.stderr, flush=True)
        except Exception as e:
            print(f"[bench] --hipblaslt: torch unavailable ({e})", file=sys.stderr, flush=True)

    def torch_time(call):
        for _ in range(10):
            call()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            call()
        e1.record()
        e1.synchronize()
        return e0.elapsed_time(e1) / reps

    def bf16_buf(n):
        return DeviceBuffer.from_numpy(f32_to_bf16_bits(rng.standard_normal(n, np.float32)))

    rows, tot, tot_lib = {}, 0.0, 0.0
    for name, kind, M, N, Kd in LAYER_GEMMS:
        flops = 2.0 * M * N * Kd
        if kind == "nt":
            a, b, y = bf16_buf(M * Kd), bf16_buf(N * Kd), DeviceBuffer(M * N * 4)
            call = lambda: K.matmul_nt_bf16(a, b, y, M, N, Kd, stream=s)
        elif kind == "dx":
            a, b, y = bf16_buf(M * N), bf16_buf(N * Kd), DeviceBuffer(M * Kd * 4)
            call = lambda: K.linear_backward_dx_bf16(a, b, y, M, N, Kd, stream=s)
        else:
            a, b, y = bf16_buf(M * N), bf16_buf(M * Kd), DeviceBuffer(N * Kd * 4)
            call = lambda: K.linear_backward_dw_bf16(a, b, y, M, N, Kd, stream=s)
        ms = ev_time(call)
        tot += ms
        row = {"M": M, "N": N, "K": Kd, "us": round(ms * 1e3, 1),
               "TFLOP_s": round(flops / (ms * 1e-3) / 1e12, 1)}
        if have_torch:
            dev = torch.device("cuda")
            g = torch.Generator(device=dev).manual_seed(5)
            if kind == "nt":
                ta = torch.randn(M, Kd, device=dev, generator=g).bfloat16()
                tb = torch.randn(N, Kd, device=dev, generator=g).bfloat16().t()
            elif kind == "dx":
                ta = torch.randn(M, N, device=dev, generator=g).bfloat16()
                tb = torch.randn(N, Kd, device=dev, generator=g).bfloat16()
            else:
                ta = torch.randn(M, N, device=dev, generator=g).bfloat16().t()
                tb = torch.randn(M, Kd, device=dev, generator=g).bfloat16()
            lms = torch_time(lambda: torch.mm(ta, tb))
            tot_lib += lms
            row["hipblaslt_us"] = round(lms * 1e3, 1)
            del ta, tb
        rows[name] = row
        print(f"[bench] gemm {name}: {row}", file=sys.stderr, flush=True)
        del a, b, y
    out = {"shapes": rows, "layer_us": round(tot * 1e3, 1),
           "layer_TFLOP_s": round(sum(2.0 * M * N * Kd for _, _, M, N, Kd in LAYER_GEMMS)
                                  / (tot * 1e-3) / 1e12, 1)}
    if have_torch:
        out["hipblaslt_layer_us"] = round(tot_lib * 1e3, 1)
    print(f"[bench] per-layer GEMMs alone: {out['layer_us']} us"
          + (f" (hipBLASLt {out['hipblaslt_layer_us']} us)" if have_torch else ""),
          file=sys.stderr, flush=True)
    return out


def calib_copy():
    """Copy-type kernel of known size for counter calibration."""
    from valkyr_amd import kernels as K
    from valkyr_amd.device import DeviceBuffer, synchronize

    n = 64 << 20
    src = DeviceBuffer.from_numpy(np.ones(n, np.float32))
    dst = DeviceBuffer(n * 4)
    for _ in range(3):
        K.scale(src, dst, n, 1.0)
    synchronize()
    print(f"[bench] calibration copy: {n * 4} bytes read + {n * 4} written per dispatch",
          file=sys.stderr, flush=True)


def measured_traffic(name):
    """HBM bytes per call recorded by the rocprofv3 counter runs (None if absent)."""
    path = os.path.join(ROOT, "profiles", name)
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_call:"):
                return int(line.split(":")[1])
    except OSError:
        pass
    return None


def cpu_baseline(args):
    """valkyr's CPU reference path (the C oracle: a restatement of src/cpu/*.zig with its
    fp64 accumulators, parallel only over independent outputs, so every thread count gives
    the same bits) on this host, scaled to tokens/s of the config-3 step.

    Each cost is timed directly, not as a difference of two runs: the oracle model keeps
    per-phase wall clocks.  Sample: the config-3 widths with 2 layers and the full tied
    151936 vocabulary on one sequence of 32 tokens (16 for the one-thread figure; one
    warm-up pass, then timed passes);
    the causal attention at the real sequence length timed separately on one 256-position
    sequence (16/8 heads of 128) and scaled by (512 / 256)^2; Adam over the sample's
    187 M parameters scaled to 596 M.  Extrapolated per step:
      t = 28 * (2048 * c_layer + 4 * t_attn(512)) + 2048 * c_head + t_adam(596 M),
    with c_layer the per-token layer cost net of attention.  Reported for all host threads
    (value) and for one thread (the reference oracle is single-threaded scalar code)."""
    import oracle as O

    c = dict(QWEN3_06B)
    Sa, L = 256, 2
    T = c["n_pos"] * c["n_seqs"]
    n_full = 596_049_920
    H, Hkv, hd = c["n_heads"], c["n_kv_heads"], c["head_dim"]
    qa, ka, va = O.normal(Sa * H * hd, 21), O.normal(Sa * Hkv * hd, 22), O.normal(Sa * Hkv * hd, 23)
    doa = O.normal(Sa * H * hd, 24, 0.1)
    all_threads = O.get_threads()

    def model(Ts):
        m = O.Model(dim=c["dim"], n_heads=H, n_kv_heads=Hkv, head_dim=hd, ff_dim=c["ff_dim"],
                    seq_len=Ts, n_seqs=1, n_layers=L, vocab_size=c["vocab_size"],
                    rms_eps=c["rms_eps"], causal=1, rotary_dim=c["rotary_dim"],
                    rope_theta=c["rope_theta"], qk_norm=1, lr=1e-4, beta1=0.9, beta2=0.999,
                    eps_adam=1e-8, lora_targets=0, lora_rank=0, lora_alpha=0.0,
                    lora_lr_b_scale=1.0, tied_embeddings=1, bf16_operands=0)
        m.init_random(3, std=0.02)
        return m

    def measure(threads, reps, Ts):
        O.set_threads(all_threads)
        m = model(Ts)
        n_sample = sum(m.tensor(0, l, w).size for l, w in [(-1, 0), (-1, 1)] +
                       [(l, i) for l in range(L) for i in range(11)])
        tok, tgt = O.ids(Ts, 11, c["vocab_size"]), O.ids(Ts, 12, c["vocab_size"])
        m.forward_backward(tok, tgt)  # warm-up: first touch of the sample's memory
        m.adam()
        O.set_threads(threads)
        runs = []
        for _ in range(reps):
            m.reset_phases()
            m.forward_backward(tok, tgt)
            m.adam()
            ph = m.phase_seconds()
            t0 = O.now()
            o, lse = O.flash_forward(qa, ka, va, Sa, Sa, H, Hkv, hd, True)
            O.flash_backward(qa, ka, va, o, doa, lse, Sa, Sa, H, Hkv, hd, True)
            ph["attn_256"] = O.now() - t0
            runs.append(ph)
        del m
        ph = {k: float(np.median([r[k] for r in runs])) for k in runs[0]}
        c_layer = (ph["layer_fwd"] + ph["layer_bwd"] - ph["attn_fwd"] - ph["attn_bwd"]) / (L * Ts)
        t_attn512 = ph["attn_256"] * (c["n_pos"] / Sa) ** 2
        c_head = ph["head"] / Ts
        t_adam = ph["adam"] * n_full / n_sample
        t_step = c["n_layers"] * (T * c_layer + c["n_seqs"] * t_attn512) + T * c_head + t_adam
        return dict(tokens_s=T / t_step, s_per_step=t_step, per_token_layer_s=c_layer,
                    attn_seq512_s=t_attn512, per_token_head_s=c_head, adam_596m_s=t_adam,
                    measured_s=sum(sum(r.values()) for r in runs), runs=reps, tokens=Ts,
                    n_sample=n_sample)

    try:
        multi = measure(all_threads, 3, 32)
        single = measure(1, 1, 16)
    finally:
        O.set_threads(all_threads)
    return dict(value=round(multi["tokens_s"], 3), unit="tokens/s", cores=all_threads,
                kind="port",
                sample=(f"C oracle (src/cpu/*.zig restatement, fp64 accumulators, OpenMP over "
                        f"independent outputs) on this host: config-3 widths, {L} layers, tied "
                        f"151936 vocabulary, 32 tokens (median of {multi['runs']} passes; 16 tokens, "
                        f"1 pass on 1 thread) + causal "
                        f"attention on one {Sa}-position sequence scaled by (512/{Sa})^2, Adam "
                        f"scaled from {multi['n_sample']:,} to {n_full:,} params; per step = 28 layers x "
                        f"2048 tokens (extrapolated): {multi['s_per_step']:,.0f} s on "
                        f"{all_threads} threads, {single['s_per_step']:,.0f} s on 1 thread"),
                single_thread={"value": round(single["tokens_s"], 3), "cores": 1,
                               "s_per_step": round(single["s_per_step"], 1)},
                all_threads={k: (round(v, 6) if isinstance(v, float) else v)
                             for k, v in multi.items()},
                single_thread_detail={k: (round(v, 6) if isinstance(v, float) else v)
                                      for k, v in single.items()},
                seconds_measured=round(multi["measured_s"] + single["measured_s"], 1))


def bench_config(name, args):
    """Config 4 (Qwen3-4B shape, frozen bf16-operand base + LoRA r16 on q/k/v/o, 1 x 2048)
    or config 5 (Qwen3-8B shape, full fine-tune with per-layer activation recompute,
    1 x 8192, untied head) at full size:
    device memory, step time, and the size-independent checks the shapes allow (loss of a
    random init = ln V within 0.5; for LoRA at step 1: B = 0 makes every dA exactly zero,
    dB non-zero, A and the frozen base unchanged bit for bit)."""
    import valkyr_amd as v
    from valkyr_amd.runner import GRAD, PARAM, Q, DOWN, lora_a, lora_b

    c = dict(QWEN3_4B_LORA if name == "config4" else QWEN3_8B)
    lora = bool(c.get("lora_targets"))
    T = c["n_pos"] * c["n_seqs"]
    out = {"shape": {k: c[k] for k in ("dim", "n_heads", "n_kv_heads", "head_dim", "ff_dim",
                                       "n_layers", "vocab_size")},
           "tokens_per_step": T}
    try:
        r = v.Runner(v.make_config(**c, precision=1))
    except v.VkhError as e:
        out["error"] = f"{e.name}: {e.message}"
        return out
    r.init_random(seed=20261202, std=0.02, lora_std=0.02)
    out["trainable_params"] = r.param_count()
    out["device_gib"] = round(r.device_bytes() / 2**30, 1)
    rng = np.random.default_rng(2)
    tok = rng.integers(0, c["vocab_size"], T, dtype=np.uint32)
    tgt = rng.integers(0, c["vocab_size"], T, dtype=np.uint32)
    print(f"[bench] {name}: {out['trainable_params']:,} trainable params, "
          f"{out['device_gib']} GiB", file=sys.stderr, flush=True)
    checks = {}
    L = c["n_layers"]
    if lora:
        a0 = {(l, p): r.get(PARAM, l, lora_a(p)) for l in (0, L - 1) for p in range(4)}
        w0 = {(l, w): r.get(PARAM, l, w) for l, w in ((0, Q), (L - 1, DOWN))}
    t0 = time.perf_counter()
    r.step(tok, tgt)
    first_s = time.perf_counter() - t0
    loss0 = r.last_loss()
    # after the unit-gain final RMSNorm every logit of a N(0, std^2) head is
    # N(0, D std^2): the mean CE of a random init is ln V + D std^2 / 2, and the
    # target logits' mean over T tokens adds noise of std sqrt(D std^2 / T)
    var = c["dim"] * 0.02 ** 2
    want = math.log(c["vocab_size"]) + var / 2
    checks["loss_init"] = round(loss0, 4)
    checks["loss_init_closed_form"] = round(want, 4)
    ok = math.isfinite(loss0) and abs(loss0 - want) < 4 * math.sqrt(var / T) + 0.01
    if lora:
        dA_zero = all(not r.get(GRAD, l, lora_a(p)).any() for l in range(L) for p in range(4))
        dB_live = all(r.get(GRAD, l, lora_b(p)).any() for l in (0, L - 1) for p in range(4))
        a_same = all(np.array_equal(r.get(PARAM, l, lora_a(p)), a) for (l, p), a in a0.items())
        w_same = all(np.array_equal(r.get(PARAM, l, w), x) for (l, w), x in w0.items())
        checks.update(dA_exactly_zero_at_step1=dA_zero, dB_nonzero=dB_live,
                      A_unchanged=a_same, frozen_base_unchanged=w_same)
        ok = ok and dA_zero and dB_live and a_same and w_same
    else:
        g = r.get(GRAD, 0, Q)
        checks["grad_layer0_q_finite_nonzero"] = bool(np.isfinite(g).all() and g.any())
        ok = ok and checks["grad_layer0_q_finite_nonzero"]
    checks["all_passed"] = bool(ok)
    K = max(1, min(args.steps, 10 if name == "config4" else 3))
    r.step_async(tok, tgt)
    r.synchronize()
    t0 = time.perf_counter()
    for _ in range(K):
        r.step_async(tok, tgt)
    r.synchronize()
    wall = time.perf_counter() - t0
    loss1 = r.last_loss()
    r.close()
    tflops = step_flops(c) / (wall / K) / 1e12
    out.update(steps=K, ms_per_step=round(1000 * wall / K, 2), tokens_s=round(T * K / wall, 1),
               tflops=round(tflops, 1), frac_bf16_peak=round(tflops / BF16_PEAK_TFLOPS, 4),
               first_step_s=round(first_s, 2), loss=[round(loss0, 4), round(loss1, 4)],
               checks=checks)
    if c.get("recompute"):
        out["activation_recompute"] = "per layer (each layer keeps its input and its attention " \
                                      "output O / LSE; projections, norms and SwiGLU rerun " \
                                      "before its backward; not counted in tflops)"
    print(f"[bench] {name}: {out['ms_per_step']} ms/step, {out['tokens_s']:,.0f} tok/s, "
          f"checks {checks}", file=sys.stderr, flush=True)
    return out


def bench_mlp(args):
    """The tiny-MLP TrainingRunner (train/runner.zig): the reference's
    `--train-demo` loop (4 -> 16 -> 4, one-sample tickStep with the prediction
    read back, 600 steps; docs/embedding.md:894-897 quotes ~730 steps/s on an
    RTX 3090, Debug build) and tickFrameTrain throughput on batches, timed with
    HIP events on the stream the steps are enqueued on."""
    import valkyr_amd as v
    from valkyr_amd.device import Event, Stream

    out = {}
    with v.TrainingRunner(4, 16, 4, 0.05, init_seed=0xDEDEDED0) as r:
        x, t = np.empty(4, np.float32), np.empty(4, np.float32)

        def demo(steps):
            for k in range(steps):
                tt = k * 0.05
                x[:] = (math.sin(tt), math.cos(tt), math.sin(2 * tt), math.cos(2 * tt))
                t[:] = (0.5 + 0.5 * math.sin(tt), 0.5 + 0.5 * math.cos(tt),
                        0.5 + 0.333 * math.sin(3 * tt), 0.0)
                pred = r.tick_step(x, t)
            return float(0.5 * np.sum((pred - t) ** 2))

        demo(50)
        t0 = time.perf_counter()
        last = demo(600)
        dt = time.perf_counter() - t0
        out["train_demo"] = {"config": "4-16-4 sgd lr 0.05, 600 blocking tick_step",
                             "steps_s": round(600 / dt, 1), "us_per_step": round(dt / 600 * 1e6, 2),
                             "last_loss": round(last, 6),
                             "reference_steps_s": 730, "reference_hw": "RTX 3090, Debug build"}
    s = Stream()
    for name, (I, H, O, N, opt) in {"uv_grid": (5, 16, 3, 256, "adam"),
                                    "large_batch": (32, 64, 32, 16384, "sgd")}.items():
        with v.TrainingRunner(I, H, O, 5e-3, max_batch_size=N, optimizer=opt) as r:
            X = np.random.default_rng(1).uniform(-1, 1, N * I).astype(np.float32)
            T = np.random.default_rng(2).uniform(0, 1, N * O).astype(np.float32)
            r.upload_train_batch(X, T)
            r.tick_frame_train(N, steps=8, stream=s)
            s.synchronize()
            K = 256 if N <= 1024 else 32
            e0, e1 = Event(), Event()
            e0.record(s)
            res = r.tick_frame_train(N, steps=K, stream=s)
            e1.record(s)
            s.synchronize()
            ms = e0.elapsed_ms(e1)
            out[name] = {"config": f"{I}-{H}-{O} {opt} batch {N}, tick_frame_train steps={K}",
                         "device_us_per_step": round(ms * 1e3 / K, 2),
                         "host_enqueue_us_per_step": round(res.elapsed_us / K, 2),
                         "samples_s": round(N * K / (ms * 1e-3), 1)}
    # the C oracle on the same demo step, one core (the tiny case is latency
    # work: a CPU core beats any GPU round trip here)
    try:
        import oracle as O

        m = O.Mlp(4, 16, 4, seed=0xDEDEDED0)
        xs, ts = np.zeros(4, np.float32), np.zeros(4, np.float32)
        t0 = time.perf_counter()
        for k in range(2000):
            m.train_step(xs, ts, 0.05)
        out["train_demo"]["cpu_oracle_steps_s"] = round(2000 / (time.perf_counter() - t0), 1)
    except Exception as e:  # the oracle is optional on the GPU box
        out["train_demo"]["cpu_oracle_steps_s"] = f"unavailable: {e}"
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--precision", default="bf16", choices=["bf16", "fp32"])
    ap.add_argument("--fa-reps", type=int, default=100)
    ap.add_argument("--fa-warmup", type=int, default=150)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the full-size config 4 / config 5 steps")
    ap.add_argument("--only", default="all",
                    choices=["all", "step", "fa", "mlp", "bw", "gemms", "config4", "config5"],
                    help="run only the step or only the attention benchmark (profiling runs)")
    ap.add_argument("--hipblaslt", action="store_true",
                    help="--only gemms: also time hipBLASLt (torch.mm) on the same shapes")
    ap.add_argument("--calib-copy", action="store_true",
                    help="after the benchmarks, run a copy-type kernel of known size "
                         "(vkh_scale over 64 Mi floats: 256 MiB read + 256 MiB written, 3x) "
                         "to calibrate rocprofv3 FETCH_SIZE / WRITE_SIZE")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: this build has no multi-GPU path "
              "(the design shards the step data-parallel, one process per GPU, but only one "
              "GPU is measured here); run with --gpus 1",
              file=sys.stderr)
        sys.exit(2)

    if args.hipblaslt:
        try:  # before the library loads: torch then sees the GPU
            import torch  # noqa: F401
        except Exception:
            pass
    import valkyr_amd as v

    if v.device_count() < 1:
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    if args.only == "fa":
        fa = bench_fa_bwd(args)
        if args.calib_copy:
            calib_copy()
        print(json.dumps({"fa_bwd_ms": round(fa["ms"], 4), "fa_bwd_tflops": round(fa["tflops"], 1)}),
              flush=True)
        return
    if args.only == "mlp":
        print(json.dumps({"mlp_runner": bench_mlp(args)}), flush=True)
        return
    if args.only == "bw":
        bw = bench_bandwidth(args)
        if args.calib_copy:
            calib_copy()
        print(json.dumps({"bandwidth": bw}), flush=True)
        return
    if args.only == "gemms":
        print(json.dumps({"layer_gemms": bench_gemms(args)}), flush=True)
        return
    if args.only in ("config4", "config5"):
        print(json.dumps({args.only: bench_config(args.only, args)}), flush=True)
        return
    st = bench_step(args, None)
    if args.only == "step":
        print(json.dumps({"ms_per_step": round(st["ms"], 3), "tokens_s": round(st["tokens_s"], 1)}),
              flush=True)
        return
    # the same step at the reference's own precision (fp32 operands throughout)
    st32 = bench_step(args, None, precision="fp32", steps=max(3, args.steps // 4), warmup=2)
    fa = bench_fa_bwd(args)
    if args.calib_copy:
        calib_copy()
    mlp = bench_mlp(args)
    bw = bench_bandwidth(args)
    cfgs = {} if args.no_configs else {n: bench_config(n, args) for n in ("config4", "config5")}
    cpu = None if args.no_cpu_baseline else cpu_baseline(args)
    peak = BF16_PEAK_TFLOPS if args.precision == "bf16" else FP32_PEAK_TFLOPS
    mfu = st["flops"] / (st["ms"] * 1e-3) / 1e12 / peak
    out = {
        "metric": "train tokens/s, Qwen3-0.6B fwd+bwd+Adam",
        "value": round(st["tokens_s"], 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(st["ms"], 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if args.precision == "bf16" else "fp32",
        "data": "synthetic (random-init weights ~N(0,0.02), uniform token ids)",
        "config": {"workload": "qwen3-0.6b full fine-tune step, config 3 of the metric",
                   "global_batch": st["T"], "seq_len": QWEN3_06B["n_pos"], "batch": 4,
                   "layers": 28, "vocab": 151936, "tied_embeddings": True,
                   "master_weights": "fp32", "optimizer": "adam",
                   "parallelism": "single GPU"},
        "step_tflops": round(st["flops"] / (st["ms"] * 1e-3) / 1e12, 1),
        "reference_precision_step": {
            "dtype": "fp32", "note": "config 3 with fp32 operands on v_mfma_f32_16x16x4_f32 "
                                     "(the reference computes in fp32 throughout)",
            "ms_per_step": round(st32["ms"], 3), "tokens_s": round(st32["tokens_s"], 1),
            "steps": max(3, args.steps // 4),
            "tflops": round(st32["flops"] / (st32["ms"] * 1e-3) / 1e12, 1),
            "frac_fp32_peak": round(st32["flops"] / (st32["ms"] * 1e-3) / 1e12 / FP32_PEAK_TFLOPS, 4),
            "loss": [round(st32["loss_first"], 4), round(st32["loss_last"], 4)]},
        "step_mfu": round(mfu, 4),
        "loss": [round(st["loss_first"], 4), round(st["loss_last"], 4)],
        "fa_bwd": {"config": "B=4 S=2048 Hq=16 Hkv=8 hd=128 causal bf16 (config 2)",
                   "ms": round(fa["ms"], 4), "tflops": round(fa["tflops"], 1),
                   "frac_bf16_peak": round(fa["tflops"] / BF16_PEAK_TFLOPS, 4)},
        "roofline": {"kernel": "attention backward, config 2: fa_bwd_dq4_k (with the D "
                               "preprocess) + fa_bwd_dkv4_k (one vkh_fa_backward_from_o call)",
                     "bound": "mfma",
                     "achieved": round(fa["tflops"], 1), "peak": BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(fa["tflops"] / BF16_PEAK_TFLOPS, 4),
                     "traffic": measured_traffic("fa_bwd_config2_traffic.md"),
                     "traffic_unit": "bytes per call (rocprofv3 FETCH_SIZE + WRITE_SIZE, "
                                     "calibrated; profiles/fa_bwd_config2_traffic.md)"},
        "cpu_baseline": cpu,
        "bandwidth_kernels": bw,
        "mlp_runner": mlp,
        "configs": cfgs,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
