"""Per-kernel parity of the HIP kernels (through the C ABI) against the C
oracle on identical seeded inputs.

Bars: bit-exact for integer / index work (embedding
scatter targets, token gather), rel-L2 <= 1e-3 for fp32, rel-L2 <= 1e-2 for
bf16-operand contractions (compared with the oracle run on the same
bf16-rounded inputs).  Elementwise kernels that restate the reference formula
with identical fp32 rounding are held to much tighter bounds where that holds.
"""
import math

import numpy as np
import pytest

import oracle as O
from helpers import bf16_dev, dev, grel, host, note, rel_l2, zeros

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-3
BF16_TOL = 1e-2


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    import valkyr_amd as v

    assert v.device_count() > 0, "no GPU visible"
    note(f"[gpu] {v.lib().vkh_build_info().decode()}")


# ── bandwidth kernels ────────────────────────────────────────────────────

def test_rmsnorm_forward_backward_fused_dw():
    from valkyr_amd import kernels as K

    # the wide rows (> 2048: a block per row) at the Qwen3-4B / -8B widths, a
    # ragged last 1024-column chunk, and more rows than the grid's blocks
    for rows, dim in ((128, 256), (2048, 1024), (300, 128), (7, 96), (64, 2560), (1100, 4096),
                      (9, 3000)):
        note(f"rmsnorm rows={rows} dim={dim}")
        x = O.normal(rows * dim, 1)
        w = O.uniform(dim, 2, 0.5, 1.5)
        dy = O.normal(rows * dim, 3)
        res = O.normal(rows * dim, 4)
        y_ref = O.rmsnorm_forward(x, w, 1e-6)
        dx_ref, dw_ref = O.rmsnorm_backward(dy, x, w, 1e-6)
        bx, bw, bdy, bres = dev(x), dev(w), dev(dy), dev(res)
        by, bdx, bdw = zeros(rows * dim), zeros(rows * dim), zeros(dim)
        K.rmsnorm_forward(bx, bw, by, rows, dim, 1e-6)
        K.rmsnorm_backward(bdy, bx, bw, bdx, bdw, rows, dim, 1e-6, residual=bres)
        y, dx, dw = host(by), host(bdx), host(bdw)
        assert grel(y_ref, y) < 1e-6
        assert grel(dx_ref + res, dx) < 1e-5
        assert rel_l2(dw_ref, dw) < 1e-5


def test_rmsnorm_backward_scratch_shared_across_streams():
    """The standalone entry points keep their scratch (gain partials here) per
    stream; calls enqueued back to back on two streams, with no host
    synchronisation between them, must each see their own partials."""
    from valkyr_amd import kernels as K
    from valkyr_amd.device import Stream

    rows, dim = 2048, 1024
    note("rmsnorm backward on two streams sharing the scratch")
    s1, s2 = Stream(), Stream()
    cases = []
    for seed in (11, 21, 31, 41):
        x, w = O.normal(rows * dim, seed), O.uniform(dim, seed + 1, 0.5, 1.5)
        dy = O.normal(rows * dim, seed + 2)
        cases.append((x, w, dy, O.rmsnorm_backward(dy, x, w, 1e-6)))
    bufs = [(dev(x), dev(w), dev(dy), zeros(rows * dim), zeros(dim)) for x, w, dy, _ in cases]
    for i, (bx, bw, bdy, bdx, bdw) in enumerate(bufs):
        K.rmsnorm_backward(bdy, bx, bw, bdx, bdw, rows, dim, 1e-6, stream=(s1 if i % 2 else s2))
    s1.synchronize()
    s2.synchronize()
    for (x, w, dy, (dx_ref, dw_ref)), (_, _, _, bdx, bdw) in zip(cases, bufs):
        assert grel(dx_ref, host(bdx)) < 1e-5
        assert rel_l2(dw_ref, host(bdw)) < 1e-5


def test_swiglu_forward_backward():
    from valkyr_amd import kernels as K

    for n in (2048 * 3072, 1001):
        z, u, dg = O.normal(n, 11, 2.0), O.normal(n, 12), O.normal(n, 13)
        g_ref = O.swiglu_forward(z, u)
        dz_ref, du_ref = O.swiglu_backward(dg, z, u)
        bz, bu, bdg = dev(z), dev(u), dev(dg)
        bg, bdz, bdu = zeros(n), zeros(n), zeros(n)
        K.swiglu_forward(bz, bu, bg, n)
        K.swiglu_backward(bdg, bz, bu, bdz, bdu, n)
        assert grel(g_ref, host(bg)) < 1e-6
        assert grel(dz_ref, host(bdz)) < 1e-6
        assert grel(du_ref, host(bdu)) < 1e-6


@pytest.mark.parametrize("rot", [128, 64, 36])  # 36: the scalar (non-float4) path
def test_qk_rope_forward_backward(rot):
    from valkyr_amd import kernels as K

    S, B, Hq, Hkv, hd, theta = 512, 2, 4, 2, 128, 1e6
    n = S * B
    q, k = O.normal(n * Hq * hd, 21), O.normal(n * Hkv * hd, 22)
    q_ref = O.rope_forward(q, n, Hq, hd, rot, theta, S)
    k_ref = O.rope_forward(k, n, Hkv, hd, rot, theta, S)
    dq_ref = O.rope_backward(q, n, Hq, hd, rot, theta, S)
    dk_ref = O.rope_backward(k, n, Hkv, hd, rot, theta, S)
    p = K.rope_params(n, Hq, Hkv, hd, rot, theta, S)
    bq, bk = dev(q), dev(k)
    oq, ok = zeros(q.size), zeros(k.size)
    K.qk_rope_forward(p, bq, oq, bk, ok)
    assert grel(q_ref, host(oq)) < 1e-6 and grel(k_ref, host(ok)) < 1e-6
    K.qk_rope_backward(p, bq, oq, bk, ok)
    assert grel(dq_ref, host(oq)) < 1e-6 and grel(dk_ref, host(ok)) < 1e-6


def test_embed_lookup_is_exact_gather():
    from valkyr_amd import kernels as K

    V, D, n = 4096, 256, 300
    E = O.normal(V * D, 31)
    ids = O.ids(n, 32, V)
    out = zeros(n * D)
    K.embed_lookup(dev(E), dev(ids), out, n, D)
    assert np.array_equal(host(out), O.embedding_forward(E, ids, D))


@pytest.mark.parametrize("n,V,D", [(6, 16, 5), (2048, 151936, 1024), (8192, 4096, 64),
                                   (1001, 300, 128), (2500, 40, 2560)])
def test_embedding_backward_bit_exact(n, V, D):
    """gpu_train.zig:4845-4930: exact scatter targets and position-order sums."""
    from valkyr_amd import kernels as K

    ids = np.array([3, 7, 3, 11, 7, 3], np.uint32) if n == 6 else O.ids(n, 41, V)
    if n == 8192:
        ids = (ids % 97).astype(np.uint32)  # heavy duplication
    dy = O.normal(n * D, 42)
    base = O.normal(V * D, 43) if n == 6 else np.zeros(V * D, np.float32)
    # embedding_backward.comp:41-46 sums a token's rows in position order and then
    # adds the sum once (dE += acc); the CPU oracle scatter-adds into a zeroed dE,
    # which is the same value when dE starts at zero (as in Runner.step)
    sums = O.embedding_backward(dy, ids, V, D)
    touched = np.zeros(V, bool)
    touched[ids] = True
    ref = base.copy().reshape(V, D)
    ref[touched] = ref[touched] + sums.reshape(V, D)[touched]
    ref = ref.ravel()
    bE = dev(base)
    K.embedding_backward(dev(dy), dev(ids), bE, n, D, V)
    got = host(bE)
    assert np.array_equal(got, ref), "embedding backward is not bit-exact"


def test_adam_matches_shader_formula():
    from valkyr_amd import kernels as K

    n = 1_000_003
    p, g = O.normal(n, 51), O.normal(n, 52, 1e-2)
    m, v = O.normal(n, 53, 1e-3), np.abs(O.normal(n, 54, 1e-5))
    bp, bg, bm, bv = dev(p), dev(g), dev(m), dev(v)
    for t in (1, 2, 7):
        O.adam_step(p, g, m, v, 1e-3, 0.9, 0.999, 1e-8, t)
        K.adam_step(bp, bg, bm, bv, n, 1e-3, 0.9, 0.999, 1e-8, t)
    assert grel(m, host(bm)) < 1e-6
    assert grel(v, host(bv)) < 1e-6
    assert rel_l2(p, host(bp)) < 1e-6


# ── GEMMs ────────────────────────────────────────────────────────────────

GEMM_SHAPES = [(128, 256, 256), (2048, 1024, 1024), (257, 130, 72), (64, 16, 96)]


@pytest.mark.parametrize("prec", [0, 1])
@pytest.mark.parametrize("shape", GEMM_SHAPES)
def test_linear_gemms(prec, shape):
    from valkyr_amd import kernels as K

    M, N, Kd = shape
    note(f"gemm prec={prec} M={M} N={N} K={Kd}")
    x, W, dy = O.normal(M * Kd, 61), O.normal(N * Kd, 62, 0.05), O.normal(M * N, 63)
    if prec == 1:
        x, W, dy = O.round_bf16(x), O.round_bf16(W), O.round_bf16(dy)
    y_ref = (x.astype(np.float64).reshape(M, Kd) @ W.astype(np.float64).reshape(N, Kd).T).ravel()
    dx_ref, dW_ref = O.linear_backward(dy, x, W, M, N, Kd)
    bx, bW, bdy = dev(x), dev(W), dev(dy)
    by, bdx, bdW = zeros(M * N), zeros(M * Kd), zeros(N * Kd)
    K.matmul_nt(bx, bW, by, M, N, Kd, prec)
    K.linear_backward_dx(bdy, bW, bdx, M, N, Kd, prec)
    K.linear_backward_dw(bdy, bx, bdW, M, N, Kd, prec)
    tol = 1e-5  # operands already bf16-exact, accumulation fp32 in both precisions
    assert rel_l2(y_ref, host(by)) < tol
    assert rel_l2(dx_ref, host(bdx)) < tol
    assert rel_l2(dW_ref, host(bdW)) < tol


# fp32 operands on the DMA-staged kernels (precision FP32): shapes that reach
# each tile plan in the forward, dx and dW layouts (256 x 256; 128 x 128 on 8
# waves; 128 x 64 with the in-block split of K; plain 128 x 64), ragged edges
# at multiples of 4, and a shape whose extents are not multiples of 4 (the
# generic kernel).
GEMM32_SHAPES = [(4096, 4096, 256), (2048, 2048, 512), (2048, 512, 4096), (1000, 520, 1000),
                 (2040, 1028, 516), (72, 40, 24), (130, 66, 1001)]


@pytest.mark.parametrize("shape", GEMM32_SHAPES)
def test_linear_gemms_fp32_dma(shape):
    from valkyr_amd import kernels as K

    M, N, Kd = shape
    note(f"gemm fp32 M={M} N={N} K={Kd}")
    rng = np.random.default_rng(M + N + Kd)
    x = rng.standard_normal((M, Kd), dtype=np.float32)
    W = (0.05 * rng.standard_normal((N, Kd))).astype(np.float32)
    dy = rng.standard_normal((M, N), dtype=np.float32)
    x64, W64, dy64 = x.astype(np.float64), W.astype(np.float64), dy.astype(np.float64)
    bx, bW, bdy = dev(x.ravel()), dev(W.ravel()), dev(dy.ravel())
    by, bdx, bdW = zeros(M * N), zeros(M * Kd), zeros(N * Kd)
    K.matmul_nt(bx, bW, by, M, N, Kd, 0)
    K.linear_backward_dx(bdy, bW, bdx, M, N, Kd, 0)
    K.linear_backward_dw(bdy, bx, bdW, M, N, Kd, 0)
    tol = 1e-5  # fp32 products, fp32 accumulation
    assert rel_l2((x64 @ W64.T).ravel(), host(by)) < tol
    assert rel_l2((dy64 @ W64).ravel(), host(bdx)) < tol
    assert rel_l2((dy64.T @ x64).ravel(), host(bdW)) < tol


def test_bf16_gemms_over_2gib_operand():
    """The head's dz at 8192 tokens x 151936 vocabulary (2.49 GB of bf16) is
    past the DMA path's 2 GiB views: dW = dz^T x runs in row chunks that
    accumulate, dx = dz W in independent row chunks.  Sampled output rows
    against float64 products of the same bf16 values."""
    from valkyr_amd import kernels as K
    from valkyr_amd.device import bf16_bits_to_f32

    M, V, D = 8192, 151936, 64
    rng = np.random.default_rng(17)
    note(f"bf16 GEMMs with a [{M}, {V}] operand")
    dz_bits = (rng.integers(0, 1 << 15, (M, V), dtype=np.uint16) & np.uint16(0x3FFF)) | \
        np.uint16(0x3C00)  # |values| in [2^-7, 2^0): no overflow, no denormals
    dz_bits ^= (rng.integers(0, 2, (M, V), dtype=np.uint16) << np.uint16(15))
    x_bits = O.to_bf16_bits(O.normal(M * D, 18).reshape(M, D))
    w_bits = O.to_bf16_bits(O.normal(V * D, 19, 0.05).reshape(V, D))
    bdz, bx, bw = dev(dz_bits), dev(x_bits), dev(w_bits)
    bdw, bdx = zeros(V * D), zeros(M * D)
    K.linear_backward_dw_bf16(bdz, bx, bdw, M, V, D)
    K.linear_backward_dx_bf16(bdz, bw, bdx, M, V, D)
    dw = host(bdw, V * D).reshape(V, D)
    dx = host(bdx, M * D).reshape(M, D)
    xf = bf16_bits_to_f32(x_bits).astype(np.float64)
    wf = bf16_bits_to_f32(w_bits).astype(np.float64)
    for v in rng.integers(0, V, 12):
        ref = bf16_bits_to_f32(dz_bits[:, v]).astype(np.float64) @ xf
        assert rel_l2(ref, dw[v]) < 1e-5, v
    for m in list(rng.integers(0, M, 10)) + [M // 2 - 1, M // 2, M - 1]:
        ref = bf16_bits_to_f32(dz_bits[m]).astype(np.float64) @ wf
        assert rel_l2(ref, dx[m]) < 1e-5, m


def test_gemm_bf16_rounding_within_north_star_tolerance():
    """bf16-operand GEMM on fp32 inputs vs the fp32 oracle: rel-L2 <= 1e-2."""
    from valkyr_amd import kernels as K

    M, N, Kd = 512, 768, 1024
    x, W = O.normal(M * Kd, 64), O.normal(N * Kd, 65, 0.02)
    y_ref = O.matmul_nt(x, W, M, N, Kd)
    by = zeros(M * N)
    K.matmul_nt(dev(x), dev(W), by, M, N, Kd, 1)
    e = rel_l2(y_ref, host(by))
    note(f"bf16 gemm rel-L2 vs fp32 oracle: {e:.2e}")
    assert e < BF16_TOL


# (M, N, K) chosen to reach every plan of the bf16-operand GEMM: 256x256 tiles
# (>= 512 of them), 128x128, 128x128 split-K (long K, few tiles), 128x64,
# ragged edges, and the generic fallback (K not a multiple of 8).
GEMM16_SHAPES = [(2048, 16384, 256), (2048, 3072, 512), (1024, 1024, 8192), (2048, 1024, 1024),
                 (1000, 520, 1000), (72, 40, 24), (130, 66, 1001), (2048, 4096, 256),
                 (2040, 4100, 200), (2048, 1024, 2048), (2000, 1000, 3000), (2048, 3072, 1024)]


@pytest.mark.parametrize("shape", GEMM16_SHAPES)
def test_linear_gemms_bf16_operands(shape):
    """All three contractions on bf16 operands vs the oracle on the same
    bf16 values (products exact in fp32): layout, tiling and split-K errors
    show up far above the 1e-5 accumulation-order noise."""
    from valkyr_amd import kernels as K

    M, N, Kd = shape
    note(f"gemm16 M={M} N={N} K={Kd}")
    bx, x = bf16_dev(O.normal(M * Kd, 71))
    bW, W = bf16_dev(O.normal(N * Kd, 72, 0.05))
    bdy, dy = bf16_dev(O.normal(M * N, 73))
    x64, W64, dy64 = (a.astype(np.float64) for a in (x, W, dy))
    y_ref = (x64.reshape(M, Kd) @ W64.reshape(N, Kd).T).ravel()
    dx_ref = (dy64.reshape(M, N) @ W64.reshape(N, Kd)).ravel()
    dW_ref = (dy64.reshape(M, N).T @ x64.reshape(M, Kd)).ravel()
    by, bdx, bdW = zeros(M * N), zeros(M * Kd), zeros(N * Kd)
    K.matmul_nt_bf16(bx, bW, by, M, N, Kd)
    K.linear_backward_dx_bf16(bdy, bW, bdx, M, N, Kd)
    K.linear_backward_dw_bf16(bdy, bx, bdW, M, N, Kd)
    for name, ref, got in (("y", y_ref, by), ("dx", dx_ref, bdx), ("dW", dW_ref, bdW)):
        e = rel_l2(ref, host(got))
        note(f"  {name} rel-L2 {e:.2e}")
        assert e < 1e-5, name


@pytest.mark.parametrize("shape", [(2048, 3072, 1024), (2000, 3072, 1000), (256, 192, 128),
                                   (130, 100, 72)])
def test_gate_up_swiglu_matches_two_passes(shape):
    """vkh_gate_up_swiglu_bf16 (the step's gate/up projection with the SwiGLU
    in the GEMM's epilogue) bit for bit against the two passes it replaces:
    vkh_matmul_nt_bf16 over the stacked [2F, K] weight, and the SwiGLU of the
    product's halves (vkh_swiglu_forward in fp32, rounded to nearest even as
    the epilogue stores bf16).  The first two shapes take the fused launch
    (config 3's, and a ragged one: M and K off the tile multiples); the last
    two the two-pass form (a plan other than the 128 x 128 tile; F not a
    multiple of 64).  gu is also held to float64 products."""
    from valkyr_amd import kernels as K
    from valkyr_amd.device import f32_to_bf16_bits

    M, F, Kd = shape
    note(f"gate/up + SwiGLU M={M} F={F} K={Kd}")
    bx, x = bf16_dev(O.normal(M * Kd, 81))
    bW, W = bf16_dev(O.normal(2 * F * Kd, 82, 0.05))
    bgu, bg = zeros(M * 2 * F), zeros(M * F, np.uint16)
    K.gate_up_swiglu_bf16(bx, bW, bgu, bg, M, F, Kd)
    gu, gated = host(bgu), host(bg, dtype=np.uint16)
    bref = zeros(M * 2 * F)
    K.matmul_nt_bf16(bx, bW, bref, M, 2 * F, Kd)
    gu_ref = host(bref)
    assert np.array_equal(gu, gu_ref)
    g64 = x.astype(np.float64).reshape(M, Kd) @ W.astype(np.float64).reshape(2 * F, Kd).T
    assert rel_l2(g64.ravel(), gu) < 1e-5
    pg = dev(gu_ref.reshape(M, 2 * F)[:, :F].copy())
    up = dev(gu_ref.reshape(M, 2 * F)[:, F:].copy())
    out = zeros(M * F)
    K.swiglu_forward(pg, up, out, M * F)
    assert np.array_equal(gated, f32_to_bf16_bits(host(out)))


# (rows, q heads, kv heads, K, seq_len, rotary_dim, qk_norm): config 3's layer (the fused
# launch), ragged rows, a partial and no rotation, no Q/K-norm, GQA 4:1, and a shape whose
# plan is not the 128 x 128 tile (the two passes either way)
QKV_PROJ_CASES = [(2048, 16, 8, 1024, 512, 128, 1), (2000, 16, 8, 1000, 500, 128, 1),
                  (2048, 16, 8, 1024, 512, 64, 1), (2048, 16, 8, 1024, 512, 0, 0),
                  (4096, 16, 4, 512, 2048, 128, 1), (256, 4, 2, 256, 128, 128, 1)]


@pytest.mark.parametrize("case", QKV_PROJ_CASES)
def test_qkv_project_fused_matches_two_passes(case):
    """vkh_qkv_project_bf16 with the Q/K-RMSNorm + RoPE in the q|k|v GEMM's
    epilogue against its two passes (the product, then the standalone
    norm-and-rotation pass over it) bit for bit: the fp32 projection and the
    bf16 attention operand; the projection also against float64 products."""
    from valkyr_amd import kernels as K

    M, Hq, Hkv, Kd, S, rot, qkn = case
    hd = 128
    N = (Hq + 2 * Hkv) * hd
    note(f"qkv project rows={M} heads={Hq}/{Hkv} K={Kd} seq={S} rot={rot} qk_norm={qkn}")
    bx, x = bf16_dev(O.normal(M * Kd, 91))
    bW, W = bf16_dev(O.normal(N * Kd, 92, 0.05))
    wq, wk = dev(O.uniform(hd, 93, 0.5, 1.5)), dev(O.uniform(hd, 94, 0.5, 1.5))
    p = K.rope_params(M, Hq, Hkv, hd, rot, 1e6, S)
    outs = []
    for fused in (True, False):
        by, bo = zeros(M * N), zeros(M * N, np.uint16)
        K.qkv_project_bf16(p, Kd, 1e-6, qkn, bx, bW, wq, wk, by, bo, fused=fused)
        outs.append((host(by), host(bo, dtype=np.uint16)))
    (y1, o1), (y0, o0) = outs
    assert np.array_equal(y1, y0)
    assert np.array_equal(o1, o0)
    y64 = x.astype(np.float64).reshape(M, Kd) @ W.astype(np.float64).reshape(N, Kd).T
    assert rel_l2(y64.ravel(), y1) < 1e-5


@pytest.mark.parametrize("case", QKV_PROJ_CASES[:3] + QKV_PROJ_CASES[4:])
def test_qkv_project_fp32_fused_matches_two_passes(case):
    """vkh_qkv_project (fp32 operands, the fp32 step's q|k|v projection with
    the Q/K-RMSNorm + RoPE in the epilogue of the fp32 slab mode) bit for bit
    against its two passes; the projection against float64 products."""
    from valkyr_amd import kernels as K

    M, Hq, Hkv, Kd, S, rot, qkn = case
    hd = 128
    N = (Hq + 2 * Hkv) * hd
    note(f"qkv project fp32 rows={M} heads={Hq}/{Hkv} K={Kd} seq={S} rot={rot}")
    x, W = O.normal(M * Kd, 95), O.normal(N * Kd, 96, 0.05)
    bx, bW = dev(x), dev(W)
    wq, wk = dev(O.uniform(hd, 97, 0.5, 1.5)), dev(O.uniform(hd, 98, 0.5, 1.5))
    p = K.rope_params(M, Hq, Hkv, hd, rot, 1e6, S)
    outs = []
    for fused in (True, False):
        by, bo = zeros(M * N), zeros(M * N)
        K.qkv_project(p, Kd, 1e-6, qkn, bx, bW, wq, wk, by, bo, fused=fused)
        outs.append((host(by), host(bo)))
    (y1, o1), (y0, o0) = outs
    assert np.array_equal(y1, y0) and np.array_equal(o1, o0)
    y64 = x.astype(np.float64).reshape(M, Kd) @ W.astype(np.float64).reshape(N, Kd).T
    assert rel_l2(y64.ravel(), y1) < 1e-5


@pytest.mark.parametrize("shape", [(2048, 3072, 1024), (2000, 3072, 1000), (256, 192, 128)])
def test_gate_up_swiglu_fp32_fused_matches_two_passes(shape):
    """vkh_gate_up_swiglu (fp32: the fp32 step's gate/up projection with the
    SwiGLU in the epilogue) bit for bit against its two passes; gu against
    float64 products.  The last shape's plan is not the 128 x 128 tile (two
    passes either way)."""
    from valkyr_amd import kernels as K

    M, F, Kd = shape
    note(f"gate/up + SwiGLU fp32 M={M} F={F} K={Kd}")
    x, W = O.normal(M * Kd, 99), O.normal(2 * F * Kd, 100, 0.05)
    bx, bW = dev(x), dev(W)
    outs = []
    for fused in (True, False):
        bgu, bg = zeros(M * 2 * F), zeros(M * F)
        K.gate_up_swiglu(bx, bW, bgu, bg, M, F, Kd, fused=fused)
        outs.append((host(bgu), host(bg)))
    (g1, s1), (g0, s0) = outs
    assert np.array_equal(g1, g0) and np.array_equal(s1, s0)
    g64 = x.astype(np.float64).reshape(M, Kd) @ W.astype(np.float64).reshape(2 * F, Kd).T
    assert rel_l2(g64.ravel(), g1) < 1e-5


# (M, N, K, r): the rank-r kernels' shapes (r a multiple of 4 up to 64, N and
# K multiples of 64; ragged M; config 4's k/v projection width at a smaller
# M) and a shape outside them that takes the general GEMMs.
LORA_SHAPES = [(256, 384, 256, 16), (200, 384, 256, 16), (256, 384, 256, 8),
               (256, 384, 256, 32), (96, 128, 192, 48), (130, 192, 320, 64),
               (512, 1024, 2560, 16), (130, 100, 72, 6)]


@pytest.mark.parametrize("n", [1, 3, 4, 1023, 4096 * 1024 + 5, 33 * 1024 * 1024])
def test_scale_add_exact(n):
    """scale / add_in_place / vec_add (the reference's scale and add shaders):
    one fp32 rounding per element, so bit-exact against numpy; sizes cover
    the chunked aligned kernel, its n % 4 tail and the short-vector path."""
    from valkyr_amd import kernels as K

    x = O.normal(n, 31)
    y = O.normal(n, 32)
    bx, by, bo = dev(x), dev(y), zeros(n)
    K.scale(bx, bo, n, 0.37)
    assert np.array_equal(host(bo, n), x * np.float32(0.37))
    K.vec_add(bx, by, bo, n)
    assert np.array_equal(host(bo, n), x + y)
    K.add_in_place(bo, bx, n)
    assert np.array_equal(host(bo, n), (x + y) + x)


@pytest.mark.parametrize("prec", [0, 1])
@pytest.mark.parametrize("shape", LORA_SHAPES)
def test_lora_forward_backward(prec, shape):
    """lora.zig:99-251 against the oracle; at every shape the fp32 factors
    and products of the rank-r kernels (bf16 precision rounds only the base
    GEMM's operands, here pre-rounded) hold 1e-5 in fp32 and the bf16 bar."""
    from valkyr_amd import kernels as K

    M, N, Kd, r = shape
    aor = 2.0
    note(f"lora prec={prec} M={M} N={N} K={Kd} r={r}")
    x, w = O.normal(M * Kd, 71), O.normal(N * Kd, 72, 0.05)
    a, b = O.normal(r * Kd, 73, 0.05), O.normal(N * r, 74, 0.05)
    dy = O.normal(M * N, 75)
    if prec == 1:
        x, w, a, b, dy = (O.round_bf16(t) for t in (x, w, a, b, dy))
    y_ref, inter_ref = O.lora_forward(x, w, a, b, M, N, Kd, r, aor)
    dx_ref, dA_ref, dB_ref = O.lora_backward(dy, x, w, a, b, inter_ref, M, N, Kd, r, aor)
    bx, bw, ba, bb, bdy = dev(x), dev(w), dev(a), dev(b), dev(dy)
    by, binter = zeros(M * N), zeros(M * r)
    K.lora_forward(bx, bw, ba, bb, by, binter, M, N, Kd, r, aor, prec)
    bdx, bdA, bdB = zeros(M * Kd), zeros(r * Kd), zeros(N * r)
    K.lora_backward(bdy, bx, bw, ba, bb, binter, bdx, bdA, bdB, M, N, Kd, r, aor, prec)
    tol = FP32_TOL if prec == 0 else BF16_TOL
    e = {n: rel_l2(ref, host(got)) for n, ref, got in
         (("y", y_ref, by), ("inter", inter_ref, binter), ("dx", dx_ref, bdx),
          ("dA", dA_ref, bdA), ("dB", dB_ref, bdB))}
    note("  " + " ".join(f"{k}={v:.1e}" for k, v in e.items()))
    assert all(v < tol for v in e.values()), e
    if shape[3] % 4 == 0 and shape[1] % 64 == 0 and shape[2] % 64 == 0:
        # the rank-r terms alone are fp32 products of exact inputs
        assert e["inter"] < 1e-5 and e["dA"] < 1e-5 and e["dB"] < 1e-5, e


# The fused projection groups of one decoder layer with adapters on every
# projection (LoraTarget.all): (input width k, output width n of each adapter)
# at dim 256, 4 query / 2 KV heads of 64, FFN 768.
LORA_GROUPS = {"qkv": (256, [256, 128, 128]), "o": (256, [256]), "gate_up": (256, [768, 768]),
               "down": (768, [256])}


@pytest.mark.parametrize("group", list(LORA_GROUPS))
def test_lora_group_bf16_matches_oracle(group):
    """The training step's grouped bf16 LoRA launches (the runner's segment
    lists and kernel instantiations, through vkh_lora_group_*_bf16) against
    the oracle's lora.zig restatement on identical inputs: x and dy are the
    bf16 values the step's kernels read, the factors are non-zero (a step-2
    state), and factors, intermediates and products are fp32 on both sides,
    so the rounding points match and only the summation order differs:
    inter, y, dyb-derived dx, dA and dB within 1e-5."""
    from valkyr_amd import kernels as K

    T, r, aor = 128, 16, 2.0
    k, ns = LORA_GROUPS[group]
    ntot = sum(ns)
    cols = [sum(ns[:i]) for i in range(len(ns))]
    note(f"lora group {group}: k={k} n={ns} T={T} r={r}")
    x16, xr = bf16_dev(O.normal(T * k, 301))
    dy16, dyr = bf16_dev(O.normal(T * ntot, 302, 0.1))
    fa = [O.normal(r * k, 303 + i, 0.05) for i in range(len(ns))]
    fb = [O.normal(n * r, 313 + i, 0.05) for i, n in enumerate(ns)]
    bufs = [dict(col=c, n=n, k=k, a=dev(a), b=dev(b), inter=zeros(T * r), dyb=zeros(T * r),
                 da=zeros(r * k), db=zeros(n * r))
            for c, n, a, b in zip(cols, ns, fa, fb)]
    ad = K.lora_adapters(bufs)
    by, bdx = zeros(T * ntot), zeros(T * k)
    K.lora_group_forward_bf16(x16, k, T, r, aor, ad, by, ntot)
    K.lora_group_backward_bf16(dy16, ntot, x16, k, T, r, aor, ad, bdx, k)
    y = host(by).reshape(T, ntot)
    dx = host(bdx)
    dx_ref = np.zeros(T * k, np.float64)
    dy2 = dyr.reshape(T, ntot)
    errs = {}
    for i, (c, n) in enumerate(zip(cols, ns)):
        dyi = np.ascontiguousarray(dy2[:, c:c + n]).ravel()
        y_ref, inter_ref = O.lora_forward(xr, np.zeros(n * k, np.float32), fa[i], fb[i], T, n, k,
                                          r, aor)
        dxi, da_ref, db_ref = O.lora_backward(dyi, xr, np.zeros(n * k, np.float32), fa[i], fb[i],
                                              inter_ref, T, n, k, r, aor)
        dx_ref += dxi
        b = bufs[i]
        errs[f"inter{i}"] = rel_l2(inter_ref, host(b["inter"]))
        errs[f"y{i}"] = rel_l2(y_ref, y[:, c:c + n])
        errs[f"dA{i}"] = rel_l2(da_ref, host(b["da"]))
        errs[f"dB{i}"] = rel_l2(db_ref, host(b["db"]))
    errs["dx"] = rel_l2(dx_ref, dx)
    note("  " + " ".join(f"{n}={e:.1e}" for n, e in errs.items()))
    assert all(e < 1e-5 for e in errs.values()), errs


def test_lora_b_zero_gives_zero_dA_on_gpu():
    from valkyr_amd import kernels as K

    M, N, Kd, r = 64, 128, 64, 16
    x, w, a = O.normal(M * Kd, 76), O.normal(N * Kd, 77), O.normal(r * Kd, 78)
    b = np.zeros(N * r, np.float32)
    dy = O.normal(M * N, 79)
    bx, bw, ba, bb = dev(x), dev(w), dev(a), dev(b)
    by, bi = zeros(M * N), zeros(M * r)
    K.lora_forward(bx, bw, ba, bb, by, bi, M, N, Kd, r, 2.0)
    bdA, bdB = zeros(r * Kd), zeros(N * r)
    K.lora_backward(dev(dy), bx, bw, ba, bb, bi, None, bdA, bdB, M, N, Kd, r, 2.0)
    assert np.all(host(bdA) == 0)
    assert np.any(host(bdB) != 0)


# ── CCE ──────────────────────────────────────────────────────────────────

@pytest.mark.parametrize("prec", [0, 1])
@pytest.mark.parametrize("n,V,D,zl,ls", [(128, 4096, 256, 0.0, 0.0), (64, 5000, 128, 1e-4, 0.1),
                                         (33, 1000, 64, 0.0, 0.0)])
def test_cce_forward_backward(prec, n, V, D, zl, ls):
    from valkyr_amd import kernels as K

    note(f"cce prec={prec} n={n} V={V} D={D}")
    h, w = O.normal(n * D, 81), O.normal(V * D, 82, 0.05)
    if prec == 1:
        h, w = O.round_bf16(h), O.round_bf16(w)
    t = O.ids(n, 83, V)
    loss_ref, lse_ref, row_ref = O.cce_forward(h, w, t, n, V, D, 1024, zl, ls)
    dh_ref, dW_ref = O.cce_backward(h, w, t, lse_ref, n, V, D, 1024, zl, ls)
    p = K.cce_params(n, V, D, zl, ls, prec)
    bh, bw, bt = dev(h), dev(w), dev(t)
    blse, brow, bmean = zeros(n), zeros(n), zeros(1)
    K.cce_forward(p, bh, bw, bt, blse, brow, bmean)
    assert grel(lse_ref, host(blse)) < 1e-5
    assert grel(row_ref, host(brow)) < 1e-4
    assert abs(host(bmean)[0] - loss_ref) < 1e-4 * abs(loss_ref)
    bdh, bdW = zeros(n * D), zeros(V * D)
    K.cce_backward(p, bh, bw, bt, blse, bdh, bdW)
    tol = FP32_TOL if prec == 0 else BF16_TOL
    assert rel_l2(dh_ref, host(bdh)) < tol
    assert rel_l2(dW_ref, host(bdW)) < tol


# ── FlashAttention ───────────────────────────────────────────────────────

FA_F32_CASES = [  # smoke/cpu.zig:909-916 shapes (n_q, n_kv, H, Hkv, hd, causal) + batch
    (4, 4, 4, 2, 16, True, 1), (16, 16, 16, 8, 128, True, 1), (8, 8, 8, 2, 256, True, 1),
    (10, 12, 4, 2, 16, True, 1), (8, 8, 4, 1, 16, True, 1), (4, 8, 4, 2, 16, False, 1),
    # the fp32 matrix-core kernels (head_dim 64 / 128, whole 64-row tiles): GQA 2:1
    # and 4:1, non-causal with more keys and with more queries, config 3's shape
    (128, 128, 4, 2, 64, True, 3), (256, 256, 16, 8, 128, True, 2),
    (192, 192, 8, 2, 64, True, 1), (128, 256, 4, 2, 128, False, 1),
    (256, 128, 8, 2, 64, False, 2), (512, 512, 16, 8, 128, True, 4),
    # grids of 512 blocks and more (each CU holds two blocks at a time; the
    # zigzag block order of the causal kernels pairs heavy and light ones)
    (64, 64, 64, 32, 64, True, 16), (128, 128, 32, 32, 128, True, 16),
]


def _fa_oracle(Q, K_, V_, dO, B, n_q, n_kv, H, Hkv, hd, causal):
    outs, lses, dqs, dks, dvs = [], [], [], [], []
    for b in range(B):
        q = Q[b * n_q * H * hd:(b + 1) * n_q * H * hd]
        k = K_[b * n_kv * Hkv * hd:(b + 1) * n_kv * Hkv * hd]
        v = V_[b * n_kv * Hkv * hd:(b + 1) * n_kv * Hkv * hd]
        do = dO[b * n_q * H * hd:(b + 1) * n_q * H * hd]
        o, lse = O.flash_forward(q, k, v, n_q, n_kv, H, Hkv, hd, causal)
        dq, dk, dv = O.flash_backward(q, k, v, o, do, lse, n_q, n_kv, H, Hkv, hd, causal)
        outs.append(o); lses.append(lse); dqs.append(dq); dks.append(dk); dvs.append(dv)
    c = np.concatenate
    return c(outs), c(lses), c(dqs), c(dks), c(dvs)


def _run_fa_gpu(p, qb, kb, vb, O_, dO_b, dO_f32, lse, B, n_q, n_kv, H, Hkv, hd, bf16_do=None):
    from valkyr_amd import kernels as K

    nq, nk = B * n_q * H * hd, B * n_kv * Hkv * hd
    bo, blse = zeros(nq), zeros(B * n_q * H)
    K.fa_forward(p, qb, kb, vb, bo, blse)
    bd = zeros(B * n_q * H)
    K.fa_bw_d(p, dev(O_), dO_f32, bd, bf16_do)
    bdq, bdk, bdv = zeros(nq), zeros(nk), zeros(nk)
    lse_b = dev(lse)
    K.fa_bw_dkv(p, qb, kb, vb, dO_b, lse_b, bd, bdk, bdv)
    K.fa_bw_dq(p, qb, kb, vb, dO_b, lse_b, bd, bdq)
    return host(bo), host(blse), host(bd), host(bdq), host(bdk), host(bdv)


@pytest.mark.parametrize("case", FA_F32_CASES)
def test_flash_attention_fp32(case):
    from valkyr_amd import kernels as K

    n_q, n_kv, H, Hkv, hd, causal, B = case
    note(f"fa fp32 {case}")
    Q = O.uniform(B * n_q * H * hd, 91, -0.5, 0.5)
    Kk = O.uniform(B * n_kv * Hkv * hd, 92, -0.5, 0.5)
    Vv = O.uniform(B * n_kv * Hkv * hd, 93, -0.5, 0.5)
    dO = O.uniform(B * n_q * H * hd, 94, -0.5, 0.5)
    o_r, lse_r, dq_r, dk_r, dv_r = _fa_oracle(Q, Kk, Vv, dO, B, n_q, n_kv, H, Hkv, hd, causal)
    p = K.attn_params(n_q, n_kv, H, Hkv, hd, causal, B, K.F32)
    bdo = dev(dO)
    o, lse, d, dq, dk, dv = _run_fa_gpu(p, dev(Q), dev(Kk), dev(Vv), o_r, bdo, bdo, lse_r, B, n_q,
                                        n_kv, H, Hkv, hd)
    assert grel(o_r, o) < 1e-4 and grel(lse_r, lse) < 1e-5
    assert rel_l2(O.fa_bw_d(o_r, dO, B * n_q, H, hd), d) < 1e-6
    assert grel(dq_r, dq) < 1e-4, grel(dq_r, dq)
    assert grel(dk_r, dk) < 1e-4, grel(dk_r, dk)
    assert grel(dv_r, dv) < 1e-4, grel(dv_r, dv)


FA_BF16_CASES = [  # (n, H, Hkv, hd, causal, B)
    (128, 4, 2, 64, True, 1), (256, 16, 8, 128, True, 2), (200, 4, 1, 128, True, 1),
    (192, 8, 2, 64, False, 2), (512, 4, 2, 128, True, 1),
]


@pytest.mark.parametrize("hd,rows", [(128, 4 * 2048 * 16), (64, 3 * 100 * 4)])
def test_fa_bw_d_bf16_inputs(hd, rows):
    """D = rowsum(O dO) from bf16 O and dO (fa_bw_d.comp with bf16 storage) vs
    the oracle's fp64 row dot of the same bf16 values; the first case is
    config 2's full size."""
    from valkyr_amd import kernels as K

    H = 16 if hd == 128 else 4
    n = rows // H
    note(f"fa_bw_d bf16 inputs hd={hd} rows={rows}")
    o16, o_r = bf16_dev(O.normal(n * H * hd, 111))
    d16, d_r = bf16_dev(O.normal(n * H * hd, 112, 0.1))
    p = K.attn_params(n, n, H, H, hd, True, 1, K.BF16)
    bd = zeros(n * H)
    K.fa_bw_d_bf16(p, o16, d16, bd)
    assert rel_l2(O.fa_bw_d(o_r, d_r, n, H, hd), host(bd)) < 1e-6


@pytest.mark.parametrize("case", FA_BF16_CASES)
def test_flash_attention_bf16_mfma(case):
    """MFMA kernels vs the oracle on the same bf16-rounded Q/K/V/dO."""
    from valkyr_amd import kernels as K

    n, H, Hkv, hd, causal, B = case
    note(f"fa bf16 {case}")
    Q = O.normal(B * n * H * hd, 101)
    Kk = O.normal(B * n * Hkv * hd, 102)
    Vv = O.normal(B * n * Hkv * hd, 103)
    dO = O.normal(B * n * H * hd, 104, 0.1)
    qb, Qr = bf16_dev(Q)
    kb, Kr = bf16_dev(Kk)
    vb, Vr = bf16_dev(Vv)
    dob, dOr = bf16_dev(dO)
    o_r, lse_r, dq_r, dk_r, dv_r = _fa_oracle(Qr, Kr, Vr, dOr, B, n, n, H, Hkv, hd, causal)
    p = K.attn_params(n, n, H, Hkv, hd, causal, B, K.BF16)
    dob16 = zeros(dO.size // 2 + 8)
    o, lse, d, dq, dk, dv = _run_fa_gpu(p, qb, kb, vb, o_r, dob, dev(dO), lse_r, B, n, n, H, Hkv,
                                        hd, dob16)
    # fa_bw_d with a bf16 copy: D pairs with the rounded dO, and the copy is exact RNE
    assert rel_l2(O.fa_bw_d(o_r, dOr, B * n, H, hd), d) < 1e-5
    assert np.array_equal(host(dob16, dO.size, np.uint16), O.to_bf16_bits(dO))
    e = [rel_l2(o_r, o), rel_l2(dq_r, dq), rel_l2(dk_r, dk), rel_l2(dv_r, dv)]
    note(f"  rel-L2 O={e[0]:.2e} dQ={e[1]:.2e} dK={e[2]:.2e} dV={e[3]:.2e}")
    assert max(abs(lse_r - lse)) < 2e-2
    assert all(x < BF16_TOL for x in e), e
    # the oracle's bf16-operand model (P and dS rounded where the MFMAs take
    # them) on the same O / lse / D inputs
    m16 = []
    for b in range(B):
        sq = slice(b * n * H * hd, (b + 1) * n * H * hd)
        sk = slice(b * n * Hkv * hd, (b + 1) * n * Hkv * hd)
        m16.append(O.flash_backward(Qr[sq], Kr[sk], Vr[sk], o_r[sq], dOr[sq],
                                    lse_r[b * n * H:(b + 1) * n * H], n, n, H, Hkv, hd, causal,
                                    bf16_ops=True))
    dq16, dk16, dv16 = (np.concatenate([x[i] for x in m16]) for i in range(3))
    e16 = [rel_l2(dq16, dq), rel_l2(dk16, dk), rel_l2(dv16, dv)]
    note(f"  vs the bf16-operand oracle dQ={e16[0]:.2e} dK={e16[1]:.2e} dV={e16[2]:.2e}")
    # same roundings at the same points: only fp32 summation order differs
    assert all(x < 1e-4 for x in e16), e16
    # the fused backward (bf16 dS workspace + dQ GEMM where the shape allows)
    ws_bytes = K.fa_backward_workspace_bytes(p)
    note(f"  fused path: workspace {ws_bytes} bytes")
    bdq, bdk, bdv = zeros(dq.size), zeros(dk.size), zeros(dv.size)
    ws = zeros(ws_bytes // 4 + 1) if ws_bytes else None
    K.fa_backward(p, qb, kb, vb, dob16, dev(lse_r), dev(d), bdq, bdk, bdv, ws)
    f = [rel_l2(dq_r, host(bdq)), rel_l2(dk_r, host(bdk)), rel_l2(dv_r, host(bdv))]
    g = [rel_l2(dq, host(bdq)), rel_l2(dk, host(bdk)), rel_l2(dv, host(bdv))]
    note(f"  fused vs oracle dQ={f[0]:.2e} dK={f[1]:.2e} dV={f[2]:.2e}; "
         f"vs two-kernel dQ={g[0]:.2e} dK={g[1]:.2e} dV={g[2]:.2e}")
    assert all(x < BF16_TOL for x in f), f
    # same dS values and products, only the dQ summation order differs
    assert all(x < 1e-5 for x in g), g
    _check_from_o(p, qb, kb, vb, o, dob16, lse_r, dO.size, ws)


# n_q != n_kv in bf16 (the reference's causal limit k <= q + (n_kv - n_q),
# fa_bw_dq.comp / flash_attn.zig:66-68 causalKeyLimit): more keys than queries
# under the causal mask, and more queries than keys without it; GQA 2:1 and
# 4:1, head_dim 64 and 128, ragged key tiles.  (Causal with n_q > n_kv is not an
# input: the reference's limit is unsigned arithmetic and underflows there, and
# the C ABI refuses it, checked below.)
FA_BF16_SHIFT_CASES = [  # (n_q, n_kv, H, Hkv, hd, causal, B)
    (96, 160, 4, 2, 64, True, 1), (64, 192, 8, 2, 128, True, 2), (40, 100, 8, 2, 64, True, 1),
    (160, 96, 4, 2, 128, False, 1),
]


@pytest.mark.parametrize("case", FA_BF16_SHIFT_CASES)
def test_flash_attention_bf16_unequal_lengths(case):
    """bf16 forward and backward through the C ABI with n_q != n_kv against the
    oracle on the same bf16-rounded Q/K/V/dO (the per-row bf16 kernels take
    these shapes: the MFMA tile kernels need n_q == n_kv under a causal mask)."""
    from valkyr_amd import kernels as K

    n_q, n_kv, H, Hkv, hd, causal, B = case
    note(f"fa bf16 unequal lengths {case}")
    Q = O.normal(B * n_q * H * hd, 121)
    Kk = O.normal(B * n_kv * Hkv * hd, 122)
    Vv = O.normal(B * n_kv * Hkv * hd, 123)
    dO = O.normal(B * n_q * H * hd, 124, 0.1)
    qb, Qr = bf16_dev(Q)
    kb, Kr = bf16_dev(Kk)
    vb, Vr = bf16_dev(Vv)
    dob, dOr = bf16_dev(dO)
    o_r, lse_r, dq_r, dk_r, dv_r = _fa_oracle(Qr, Kr, Vr, dOr, B, n_q, n_kv, H, Hkv, hd, causal)
    p = K.attn_params(n_q, n_kv, H, Hkv, hd, causal, B, K.BF16)
    o, lse, d, dq, dk, dv = _run_fa_gpu(p, qb, kb, vb, o_r, dob, dev(dO), lse_r, B, n_q, n_kv, H,
                                        Hkv, hd)
    assert max(abs(lse_r - lse)) < 2e-2
    e = [rel_l2(o_r, o), rel_l2(dq_r, dq), rel_l2(dk_r, dk), rel_l2(dv_r, dv)]
    note(f"  rel-L2 O={e[0]:.2e} dQ={e[1]:.2e} dK={e[2]:.2e} dV={e[3]:.2e}")
    assert all(x < BF16_TOL for x in e), e
    # the one-call backward takes the same shapes
    ws_bytes = K.fa_backward_workspace_bytes(p)
    bdq, bdk, bdv = zeros(dq.size), zeros(dk.size), zeros(dv.size)
    ws = zeros(ws_bytes // 4 + 1) if ws_bytes else None
    K.fa_backward(p, qb, kb, vb, dob, dev(lse_r), dev(d), bdq, bdk, bdv, ws)
    f = [rel_l2(dq_r, host(bdq)), rel_l2(dk_r, host(bdk)), rel_l2(dv_r, host(bdv))]
    note(f"  one-call backward dQ={f[0]:.2e} dK={f[1]:.2e} dV={f[2]:.2e}")
    assert all(x < BF16_TOL for x in f), f


def test_flash_attention_causal_more_queries_than_keys_refused():
    """Causal attention with n_q > n_kv is refused with InvalidArgument before
    any launch (the reference's key limit q + (n_kv - n_q) is unsigned)."""
    from valkyr_amd import VkhError
    from valkyr_amd import kernels as K

    p = K.attn_params(128, 64, 4, 2, 64, True, 1, K.BF16)
    q, kv = zeros(128 * 4 * 64), zeros(64 * 2 * 64)
    with pytest.raises(VkhError, match="InvalidArgument"):
        K.fa_forward(p, q, kv, kv, zeros(128 * 4 * 64), zeros(128 * 4))


def _check_from_o(p, qb, kb, vb, o, dob16, lse, n_do, ws):
    """vkh_fa_backward_from_o (D formed from the bf16 O inside the backward)
    vs the two calls it replaces, fa_bw_d_bf16 then fa_backward, on the same
    bf16 O: D to fp64-dot accuracy, dQ / dK / dV equal up to summation order."""
    from valkyr_amd import kernels as K

    o16, o_r = bf16_dev(o)
    lse_b = dev(lse)
    n_rows = lse.size
    d_ref = zeros(n_rows)
    K.fa_bw_d_bf16(p, o16, dob16, d_ref)
    dq0, dk0, dv0 = zeros(o.size), zeros(_kv_numel(p)), zeros(_kv_numel(p))
    K.fa_backward(p, qb, kb, vb, dob16, lse_b, d_ref, dq0, dk0, dv0, ws)
    d1 = zeros(n_rows)
    dq1, dk1, dv1 = zeros(o.size), zeros(_kv_numel(p)), zeros(_kv_numel(p))
    K.fa_backward_from_o(p, qb, kb, vb, o16, dob16, lse_b, d1, dq1, dk1, dv1, ws)
    from valkyr_amd.device import bf16_bits_to_f32

    dO_r = bf16_bits_to_f32(host(dob16, n_do, np.uint16))
    d_np = O.fa_bw_d(o_r, dO_r, n_rows // p.n_heads, p.n_heads, p.head_dim)
    e = [rel_l2(d_np, host(d1)), rel_l2(host(dq0), host(dq1)), rel_l2(host(dk0), host(dk1)),
         rel_l2(host(dv0), host(dv1))]
    note(f"  from_o vs two calls: D={e[0]:.1e} dQ={e[1]:.1e} dK={e[2]:.1e} dV={e[3]:.1e}")
    assert e[0] < 1e-6 and rel_l2(d_np, host(d_ref)) < 1e-6
    assert all(x < 1e-5 for x in e[1:]), e


def test_flash_attention_bf16_config3_shape():
    """Config 3's attention shape (B = 4 x S = 512, 16/8 heads, hd 128, causal)
    through the one vkh_fa_backward_from_o call the step makes (the recompute
    kernels: D formed by the dQ kernel from the bf16 O, 128-query dQ blocks,
    no workspace) against the oracle on the same bf16 Q/K/V/dO/O: dQ/dK/dV
    within the bf16 bar of the fp32 oracle, within 1e-4 of its bf16-operand
    model (P and dS rounded where the MFMAs take them), D to fp64-dot
    accuracy."""
    from valkyr_amd import kernels as K
    from valkyr_amd.device import bf16_bits_to_f32

    B, n, H, Hkv, hd = 4, 512, 16, 8, 128
    note("fa bf16 config-3 shape, one-call backward from O")
    Q = O.normal(B * n * H * hd, 131)
    Kk = O.normal(B * n * Hkv * hd, 132)
    Vv = O.normal(B * n * Hkv * hd, 133)
    dO = O.normal(B * n * H * hd, 134, 0.1)
    qb, Qr = bf16_dev(Q)
    kb, Kr = bf16_dev(Kk)
    vb, Vr = bf16_dev(Vv)
    dob16, dOr = bf16_dev(dO)
    p = K.attn_params(n, n, H, Hkv, hd, True, B, K.BF16)
    assert K.fa_backward_workspace_bytes(p) == 0  # the recompute kernels
    o_r, lse_r, dq_r, dk_r, dv_r = _fa_oracle(Qr, Kr, Vr, dOr, B, n, n, H, Hkv, hd, True)
    # the backward reads O in bf16: the oracle's models take the same values
    o16, o16_r = bf16_dev(o_r)
    d_ref = O.fa_bw_d(o16_r, dOr, B * n, H, hd)
    bd, bdq, bdk, bdv = zeros(B * n * H), zeros(Q.size), zeros(Kk.size), zeros(Kk.size)
    K.fa_backward_from_o(p, qb, kb, vb, o16, dob16, dev(lse_r), bd, bdq, bdk, bdv, None)
    d, dq, dk, dv = host(bd), host(bdq), host(bdk), host(bdv)
    assert rel_l2(d_ref, d) < 1e-6, rel_l2(d_ref, d)
    e = [rel_l2(dq_r, dq), rel_l2(dk_r, dk), rel_l2(dv_r, dv)]
    note(f"  vs the fp32 oracle dQ={e[0]:.2e} dK={e[1]:.2e} dV={e[2]:.2e}")
    assert all(x < BF16_TOL for x in e), e
    m16 = []
    for b in range(B):
        sq = slice(b * n * H * hd, (b + 1) * n * H * hd)
        sk = slice(b * n * Hkv * hd, (b + 1) * n * Hkv * hd)
        m16.append(O.flash_backward(Qr[sq], Kr[sk], Vr[sk], o16_r[sq], dOr[sq],
                                    lse_r[b * n * H:(b + 1) * n * H], n, n, H, Hkv, hd, True,
                                    bf16_ops=True))
    dq16, dk16, dv16 = (np.concatenate([x[i] for x in m16]) for i in range(3))
    e16 = [rel_l2(dq16, dq), rel_l2(dk16, dk), rel_l2(dv16, dv)]
    note(f"  vs the bf16-operand oracle dQ={e16[0]:.2e} dK={e16[1]:.2e} dV={e16[2]:.2e}")
    assert all(x < 1e-4 for x in e16), e16


def _kv_numel(p):
    return p.n_batch * p.n_kv * p.n_kv_heads * p.head_dim


def test_flash_attention_bf16_full_size_invariants():
    """Config-2 shape (B=4, S=2048, 16/8 heads, hd 128): size-independent checks.

    sum_k dV[k] = sum_{q, h in group} dO[q]   (rows of P sum to 1)
    sum_k dK[k] = 0                           (rows of dS sum to 0)
    plus closed-form dQ / dK / dV rows in float64 at sampled positions.
    """
    from valkyr_amd import kernels as K

    B, S, H, Hkv, hd = 4, 2048, 16, 8, 128
    note("fa bf16 config-2 invariants")
    Q = O.normal(B * S * H * hd, 111)
    Kk = O.normal(B * S * Hkv * hd, 112)
    Vv = O.normal(B * S * Hkv * hd, 113)
    dO = O.normal(B * S * H * hd, 114, 0.1)
    qb, Qr = bf16_dev(Q)
    kb, Kr = bf16_dev(Kk)
    vb, Vr = bf16_dev(Vv)
    dob, dOr = bf16_dev(dO)
    p = K.attn_params(S, S, H, Hkv, hd, True, B, K.BF16)
    bo, blse, bd = zeros(Q.size), zeros(B * S * H), zeros(B * S * H)
    K.fa_forward(p, qb, kb, vb, bo, blse)
    dob16 = zeros(dO.size // 2 + 8)
    K.fa_bw_d(p, bo, dev(dO), bd, dob16)
    bdq, bdk, bdv = zeros(Q.size), zeros(Kk.size), zeros(Kk.size)
    K.fa_backward(p, qb, kb, vb, dob16, blse, bd, bdq, bdk, bdv)
    o, lse, dq, dk, dv = host(bo), host(blse), host(bdq), host(bdk), host(bdv)
    _check_from_o(p, qb, kb, vb, o, dob16, lse, dO.size, None)
    hpk = H // Hkv
    dv4 = dv.reshape(B, S, Hkv, hd).astype(np.float64)
    dO4 = dOr.reshape(B, S, Hkv, hpk, hd).astype(np.float64)
    lhs, rhs = dv4.sum(1), dO4.sum(axis=(1, 3))
    assert rel_l2(rhs, lhs) < 5e-3
    dk4 = dk.reshape(B, S, Hkv, hd).astype(np.float64)
    # the sum over keys cancels: far below the sum of magnitudes
    assert np.all(np.abs(dk4.sum(1)) <= 2e-2 * np.abs(dk4).sum(1) + 1e-6)
    # closed-form rows (float64 from the bf16-exact operands)
    q5 = Qr.reshape(B, S, H, hd).astype(np.float64)
    k5 = Kr.reshape(B, S, Hkv, hd).astype(np.float64)
    v5 = Vr.reshape(B, S, Hkv, hd).astype(np.float64)
    do5 = dOr.reshape(B, S, H, hd).astype(np.float64)
    sc = 1.0 / math.sqrt(hd)
    rng = np.random.default_rng(5)
    for _ in range(6):
        b, h, qi = rng.integers(B), rng.integers(H), rng.integers(S)
        kv = h // hpk
        s = k5[b, :qi + 1, kv] @ q5[b, qi, h] * sc
        pr = np.exp(s - s.max()); pr /= pr.sum()
        o_ref = pr @ v5[b, :qi + 1, kv]
        assert rel_l2(o_ref, o.reshape(B, S, H, hd)[b, qi, h]) < 1e-2
        dp = v5[b, :qi + 1, kv] @ do5[b, qi, h]
        dd = (pr * dp).sum()
        dq_ref = sc * ((pr * (dp - dd)) @ k5[b, :qi + 1, kv])
        assert rel_l2(dq_ref, dq.reshape(B, S, H, hd)[b, qi, h]) < 1e-2
    # closed-form dK / dV rows at sampled keys (a key-row permutation or a row
    # written to the wrong key would pass the sums above):
    #   dV[j] = sum_{h in group} sum_{q >= j} P[q, j] dO[q, h]
    #   dK[j] = sc sum_{h in group} sum_{q >= j} P[q, j] (dP[q, j] - D[q, h]) Q[q, h]
    dk5 = dk.reshape(B, S, Hkv, hd)
    dv5 = dv.reshape(B, S, Hkv, hd)
    mask = np.tril(np.ones((S, S), bool))
    for _ in range(3):
        b, kv = rng.integers(B), rng.integers(Hkv)
        keys = [0, int(rng.integers(1, S - 1)), int(rng.integers(S // 2, S - 1)), S - 1]
        dv_ref = np.zeros((len(keys), hd))
        dk_ref = np.zeros((len(keys), hd))
        for h in range(kv * hpk, (kv + 1) * hpk):
            s_ = (q5[b, :, h] @ k5[b, :, kv].T) * sc
            s_ = np.where(mask, s_, -np.inf)
            P = np.exp(s_ - s_.max(1, keepdims=True))
            P /= P.sum(1, keepdims=True)
            dP = do5[b, :, h] @ v5[b, :, kv].T
            Dq = (P * dP).sum(1, keepdims=True)
            dS = P * (dP - Dq)
            dv_ref += P[:, keys].T @ do5[b, :, h]
            dk_ref += sc * (dS[:, keys].T @ q5[b, :, h])
        for i, j in enumerate(keys):
            assert rel_l2(dv_ref[i], dv5[b, j, kv]) < 1e-2, ("dV", b, kv, j)
            assert rel_l2(dk_ref[i], dk5[b, j, kv]) < 1e-2, ("dK", b, kv, j)
