"""The tiny-MLP oracle (oracle.c restating src/cpu/train.zig and the
TrainingRunner's batched semantics) pinned on the CPU against published
generator vectors, numpy float64 restatements, finite differences and the
closed forms the reference's own smokes use."""
import numpy as np
import pytest

import oracle as O


# ── Zig std DefaultPrng: xoshiro256++ seeded by SplitMix64 ─────────────────

def test_splitmix64_published_outputs():
    # the first outputs of SplitMix64 from state 0 (Vigna's splitmix64.c)
    assert O.splitmix64_stream(0, 4) == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4,
                                         0x06C45D188009454F, 0xF88BB8A8724C81EC]


def test_xoshiro256pp_reference_vector():
    # xoshiro256plusplus.c from state {1, 2, 3, 4}
    z = O.ZigPrng(state=[1, 2, 3, 4])
    assert [z.next() for _ in range(10)] == [
        41943041, 58720359, 3588806011781223, 3591011842654386, 9228616714210784205,
        9973669472204895162, 14011001112246962877, 12406186145184390807,
        15849039046786891736, 10450023813501588000]


def test_zig_seeding_uses_four_splitmix_outputs():
    a = O.ZigPrng(seed=0xCAFE)
    b = O.ZigPrng(state=O.splitmix64_stream(0xCAFE, 4))
    assert [a.next() for _ in range(8)] == [b.next() for _ in range(8)]


def test_float32_range_and_distribution():
    z = O.ZigPrng(seed=12345)
    u = np.array([z.float32() for _ in range(20000)], np.float64)
    assert u.min() >= 0.0 and u.max() < 1.0
    assert abs(u.mean() - 0.5) < 0.01 and abs(u.var() - 1 / 12) < 0.005
    # the exponent follows the leading zeros of one draw: half the values in [0.5, 1)
    assert abs((u >= 0.5).mean() - 0.5) < 0.02 and abs((u < 0.25).mean() - 0.25) < 0.02


def test_float32_from_draw():
    """One draw r gives 2^-(1 + clz(r)) * (1 + (r mod 2^23) / 2^23)."""
    z1, z2 = O.ZigPrng(seed=99), O.ZigPrng(seed=99)
    for _ in range(200):
        r = z2.next()
        lz = 64 - r.bit_length()
        assert lz < 41
        want = 2.0 ** (-1 - lz) * (1 + (r & 0x7FFFFF) / 2.0 ** 23)
        assert float(z1.float32()) == want


def test_mlp_init_layout():
    I, H, O_ = 5, 7, 3
    m = O.Mlp(I, H, O_, init_scale=0.3, seed=0x70077077)
    z = O.ZigPrng(seed=0x70077077)
    draws = np.array([z.float32() for _ in range(H * I + O_ * H)], np.float32)
    w = (draws * np.float32(2) - np.float32(1)) * np.float32(0.3)
    assert np.array_equal(m.view("w1"), w[:H * I]) and np.array_equal(m.view("w2"), w[H * I:])
    assert not m.view("b1").any() and not m.view("b2").any()
    assert np.abs(m.P).max() <= 0.3
    assert not np.array_equal(O.Mlp(I, H, O_, seed=1).P, m.P)


# ── numpy float64 restatement ─────────────────────────────────────────────

def np_forward(m, X):
    I, H, O_ = m.I, m.H, m.O
    W1 = m.view("w1").astype(np.float64).reshape(H, I)
    W2 = m.view("w2").astype(np.float64).reshape(O_, H)
    hp = X @ W1.T + m.view("b1")
    h = np.maximum(hp, 0)
    return hp, h, h @ W2.T + m.view("b2")


def rand_mlp(I, H, O_, seed):
    m = O.Mlp(I, H, O_, seed=seed)
    m.P[m.spans()["b1"]] = O.normal(H, seed + 1, 0.2)
    m.P[m.spans()["b2"]] = O.normal(O_, seed + 2, 0.2)
    return m


def test_forward_matches_numpy():
    m = rand_mlp(6, 16, 4, 3)
    x = O.normal(6, 7)
    hp, h, y = m.forward(x)
    rhp, rh, ry = np_forward(m, x.astype(np.float64)[None])
    assert np.allclose(hp, rhp[0], rtol=1e-6, atol=1e-6) and np.allclose(h, rh[0], atol=1e-6)
    assert np.allclose(y, ry[0], rtol=1e-5, atol=1e-6)
    assert (hp <= 0).any() and (hp > 0).any()  # both sides of the ReLU exercised


def _loss64(m, P, x, t, ce=False):
    saved = m.P.copy()
    m.P[:] = P
    _, _, y = np_forward(m, np.asarray(x, np.float64)[None])
    m.P[:] = saved
    y = y[0]
    if not ce:
        return 0.5 * np.sum((y - t) ** 2)
    z = y - y.max()
    return -np.sum(t * (z - np.log(np.exp(z).sum())))


def test_backward_matches_finite_differences():
    m = rand_mlp(5, 12, 4, 11)
    x, t = O.normal(5, 12), O.normal(4, 13)
    hp, h, y = m.forward(x)
    dy = np.empty(4, np.float32)
    O.lib().orc_mse_loss_grad(dy, y, O.f32(t), 4)
    G = m.backward(x, hp, h, dy).copy()
    P64 = m.P.astype(np.float64)
    eps = 1e-4
    fd = np.empty(m.n)
    for k in range(m.n):
        e = np.zeros(m.n)
        e[k] = eps
        fd[k] = (_loss64(m, P64 + e, x, t) - _loss64(m, P64 - e, x, t)) / (2 * eps)
    assert np.abs(fd - G).max() <= 2e-4 * max(1.0, np.abs(fd).max())
    # dead ReLU units carry no W1 / b1 gradient
    dead = np.where(hp <= 0)[0]
    assert dead.size and not G[m.spans()["w1"]].reshape(12, 5)[dead].any()


def test_mse_loss_and_grad():
    y, t = O.normal(9, 1), O.normal(9, 2)
    assert abs(O.mse_loss(y, t) - 0.5 * np.sum((y.astype(np.float64) - t) ** 2)) < 1e-5
    d = np.empty(9, np.float32)
    O.lib().orc_mse_loss_grad(d, y, t, 9)
    assert np.array_equal(d, y - t)


def test_ce_grad_row():
    y = O.normal(6, 5, 2.0)
    t = np.abs(O.normal(6, 6))
    t /= t.sum()
    d = O.softmax_ce_grad_row(y, t)
    p = np.exp(y - y.max()) / np.exp(y - y.max()).sum()
    assert np.allclose(d, p - t, atol=1e-6)
    assert abs(d.astype(np.float64).sum()) < 1e-6  # normalised target: rows sum to 0


def test_ce_batch_step_gradient_matches_finite_differences():
    m = rand_mlp(3, 8, 5, 21)
    x = O.normal(3, 22)
    t = np.zeros(5, np.float32)
    t[2] = 1
    P0 = m.P.astype(np.float64)
    m.batch_step(x, t, 1, 0.0, cross_entropy=True)
    eps = 1e-4
    fd = np.array([(_loss64(m, P0 + eps * np.eye(m.n)[k], x, t, True)
                    - _loss64(m, P0 - eps * np.eye(m.n)[k], x, t, True)) / (2 * eps)
                   for k in range(m.n)])
    assert np.abs(fd - m.G).max() <= 2e-4 * max(1.0, np.abs(fd).max())


def test_train_step_is_forward_loss_backward_sgd():
    m = rand_mlp(4, 8, 4, 31)
    x, t = O.normal(4, 32), O.normal(4, 33)
    P0 = m.P.copy()
    _, _, y = m.forward(x)
    loss = m.train_step(x, t, 0.05)
    assert abs(loss - 0.5 * np.sum((y.astype(np.float64) - t) ** 2)) < 1e-5
    assert np.array_equal(m.P, P0 - np.float32(0.05) * m.G)


def test_batch_step_of_one_sample_is_train_step():
    a, b = rand_mlp(4, 8, 3, 41), rand_mlp(4, 8, 3, 41)
    x, t = O.normal(4, 42), O.normal(3, 43)
    a.train_step(x, t, 0.07)
    b.batch_step(x, t, 1, 0.07)
    assert np.array_equal(a.P, b.P) and np.array_equal(a.G, b.G)


@pytest.mark.parametrize("ce", [False, True])
def test_batch_step_gradient_is_the_batch_mean(ce):
    I, H, O_, N = 4, 16, 5, 24
    m = rand_mlp(I, H, O_, 51)
    X = O.normal(N * I, 52).reshape(N, I)
    if ce:
        T = np.abs(O.normal(N * O_, 53)).reshape(N, O_)
        T /= T.sum(1, keepdims=True)
    else:
        T = O.normal(N * O_, 53).reshape(N, O_)
    hp, h, y = np_forward(m, X.astype(np.float64))
    if ce:
        p = np.exp(y - y.max(1, keepdims=True))
        dy = p / p.sum(1, keepdims=True) - T
    else:
        dy = y - T
    W2 = m.view("w2").astype(np.float64).reshape(O_, H)
    dhp = (dy @ W2) * (hp > 0)
    want = np.concatenate([(dhp.T @ X).ravel(), dhp.sum(0), (dy.T @ h).ravel(), dy.sum(0)]) / N
    m.batch_step(X, T, N, 0.0, cross_entropy=ce)
    assert np.abs(m.G - want).max() <= 1e-5 * max(1.0, np.abs(want).max())


@pytest.mark.parametrize("ce", [False, True])
def test_batch_loss(ce):
    I, H, O_, N = 3, 8, 4, 10
    m = rand_mlp(I, H, O_, 61)
    X = O.normal(N * I, 62).reshape(N, I)
    T = np.abs(O.normal(N * O_, 63)).reshape(N, O_)
    T /= T.sum(1, keepdims=True)
    _, _, y = np_forward(m, X.astype(np.float64))
    if ce:
        z = y - y.max(1, keepdims=True)
        want = -np.sum(T * (z - np.log(np.exp(z).sum(1, keepdims=True)))) / N
    else:
        want = 0.5 * np.sum((y - T) ** 2) / N
    assert abs(m.batch_loss(X, T, N, ce) - want) <= 1e-5 * abs(want)


@pytest.mark.parametrize("adam", [False, True])
def test_weight_decay_shrinks_weights_only(adam):
    """smoke/training.zig:1338-1420: zero input and target give zero gradient,
    so K steps scale W by (1 - lr wd)^K and leave the biases at zero."""
    m = O.Mlp(4, 8, 4, seed=0xCDDECA1)
    n0 = {k: np.linalg.norm(m.view(k).astype(np.float64)) for k in ("w1", "w2")}
    lr, wd, K = 0.05, 0.1, 30
    for k in range(K):
        m.batch_step(np.zeros(4), np.zeros(4), 1, lr, adam=adam, weight_decay=wd, t_step=k + 1)
    for k in ("w1", "w2"):
        got = np.linalg.norm(m.view(k).astype(np.float64))
        assert abs(got - n0[k] * (1 - lr * wd) ** K) <= 1e-5 * n0[k]
    assert not m.view("b1").any() and not m.view("b2").any()


def test_adam_first_step_closed_form():
    """t = 1 with zero moments: m_hat = g, v_hat = g^2, so each parameter moves
    by lr * g / (|g| + eps)."""
    m = rand_mlp(3, 8, 2, 71)
    x, t = O.normal(3, 72), O.normal(2, 73)
    P0 = m.P.astype(np.float64)
    ref = rand_mlp(3, 8, 2, 71)
    ref.batch_step(x, t, 1, 0.0)  # gradient only
    g = ref.G.astype(np.float64)
    m.batch_step(x, t, 1, 1e-2, adam=True, t_step=1)
    want = P0 - 1e-2 * g / (np.abs(g) + 1e-8)
    assert np.abs(m.P - want).max() < 1e-6
    # (1 - beta) as the fp32 constants round it
    c1 = float(np.float32(1) - np.float32(0.9))
    c2 = float(np.float32(1) - np.float32(0.999))
    assert np.allclose(m.M, c1 * g, rtol=1e-6, atol=1e-12)
    assert np.allclose(m.V, c2 * g * g, rtol=1e-5, atol=1e-20)
