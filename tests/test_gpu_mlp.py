"""The tiny-MLP TrainingRunner (vkh_mlp_* C ABI, HIP kernels) against the C
oracle of src/cpu/train.zig, on the scenarios of the reference's own smokes
(src/smoke/training.zig:936-2420).

Bars: the reference's tolerances where it states one (batched SGD / Adam
parity 1e-4 absolute after K steps, CE loss gradient 1e-5 absolute,
weight-decay shrink 1e-3 relative); bit-exact where the same kernel computes
both sides (batched vs one-at-a-time prediction) and for the initial weights.
"""
import numpy as np
import pytest

import oracle as O
from helpers import note, rel_l2

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    import valkyr_amd as v

    assert v.device_count() > 0, "no GPU visible"


def make(**kw):
    import valkyr_amd as v

    d = dict(lr=0.05)
    d.update(kw)
    return v.TrainingRunner(**d)


def mirror(r):
    from valkyr_amd import mlp

    return O.Mlp(r.dim_in, r.dim_hidden, r.dim_out, params=r.read_buffer(mlp.BUF_PARAMS))


def params_close(r, m, tol=1e-4):
    from valkyr_amd import mlp

    got = r.read_buffer(mlp.BUF_PARAMS)
    d = float(np.abs(got - m.P).max())
    return d, rel_l2(m.P, got), d <= tol


@pytest.mark.parametrize("dims,seed,scale", [((4, 8, 4), 0xCAFE, 0.3),
                                             ((5, 64, 3), 0x70077077, 0.3),
                                             ((7, 33, 11), 1, 0.5)])
def test_initial_weights_match_oracle_init(dims, seed, scale):
    I, H, O_ = dims
    note(f"mlp init {dims} seed={seed:#x} scale={scale}")
    with make(dim_in=I, dim_hidden=H, dim_out=O_, init_seed=seed, init_scale=scale) as r:
        m = O.Mlp(I, H, O_, init_scale=scale, seed=seed)
        assert np.array_equal(mirror(r).P, m.P)
        w = r.read_weights()
        assert np.array_equal(w["w1"].ravel(), m.view("w1"))
        assert np.array_equal(w["w2"].ravel(), m.view("w2"))
        assert not w["b1"].any() and not w["b2"].any()


def test_tick_step_matches_train_step_and_converges():
    """runTrainingRunnerSmoke (training.zig:950-1026): two alternating pairs,
    200 one-sample SGD steps; every prediction and the final weights against
    cpu/train.zig trainStep."""
    note("mlp tick_step 4-8-4 x200")
    x_a, t_a = np.array([1, 0, 0, 0], np.float32), np.array([1, 0.2, 0, 0], np.float32)
    x_b, t_b = np.array([0, 1, 0, 0], np.float32), np.array([0, 0, 0.7, 0.3], np.float32)
    with make(dim_in=4, dim_hidden=8, dim_out=4, lr=0.05, init_seed=0x70077077) as r:
        m = mirror(r)
        loss0 = O.mse_loss(r.tick_predict(x_a), t_a) + O.mse_loss(r.tick_predict(x_b), t_b)
        worst = 0.0
        for s in range(200):
            x, t = (x_a, t_a) if s % 2 == 0 else (x_b, t_b)
            _, _, y_ref = m.forward(x)
            pred = r.tick_step(x, t)
            m.train_step(x, t, 0.05)
            worst = max(worst, float(np.abs(pred - y_ref).max()))
        d, rl, ok = params_close(r, m, 1e-5)
        loss1 = O.mse_loss(r.tick_predict(x_a), t_a) + O.mse_loss(r.tick_predict(x_b), t_b)
        note(f"  pred max|d|={worst:.2e} params max|d|={d:.2e} loss {loss0:.5f} -> {loss1:.5f}")
        assert worst <= 1e-5 and ok
        assert loss1 < 0.1 * loss0


def test_tick_predict_matches_oracle_forward():
    with make(dim_in=6, dim_hidden=20, dim_out=5, init_seed=7) as r:
        m = mirror(r)
        for k in range(5):
            x = O.normal(6, 100 + k)
            _, _, y = m.forward(x)
            assert np.abs(r.tick_predict(x) - y).max() <= 1e-6 * max(1.0, np.abs(y).max())


# (I, H, O, N, steps): the reference's batched-train smoke (training.zig:1526),
# a batch at the fused kernel's limit, the two-kernel path, the chunk-split
# path, and weights too large for LDS (read from a packed copy in HBM).
BATCH_CASES = [(4, 8, 3, 16, 8), (3, 5, 2, 1024, 3), (50, 64, 40, 200, 3), (6, 64, 10, 3000, 3),
               (200, 64, 100, 8, 2)]


@pytest.mark.parametrize("I,H,O_,N,K", BATCH_CASES)
def test_tick_step_batch_sgd_parity(I, H, O_, N, K):
    from valkyr_amd import mlp

    note(f"mlp tick_step_batch sgd {I}-{H}-{O_} N={N} K={K}")
    X, T = O.uniform(N * I, 0x5EED5, -1, 1), O.uniform(N * O_, 0x5EED6, 0, 1)
    with make(dim_in=I, dim_hidden=H, dim_out=O_, lr=0.05, init_seed=0xBA7C7AA,
              max_batch_size=N) as r:
        m = mirror(r)
        for _ in range(K):
            m.batch_step(X, T, N, 0.05)
            r.tick_step_batch(X, T)
        d, rl, ok = params_close(r, m)
        eg = rel_l2(m.G, r.read_buffer(mlp.BUF_GRADS))
        note(f"  params max|d|={d:.2e} rel-L2={rl:.2e}; last grad rel-L2={eg:.2e}")
        assert ok and rl <= 1e-5 and eg <= 1e-5


@pytest.mark.parametrize("ce,wd", [(False, 0.0), (False, 0.1), (True, 0.01)])
def test_tick_step_batch_adam_parity(ce, wd):
    """runTrainingRunnerAdamSmoke (training.zig:1992-2150), plus AdamW decay
    and the cross-entropy head."""
    from valkyr_amd import mlp

    N, I, H, O_, K = 16, 4, 8, 3, 5
    note(f"mlp adam ce={ce} wd={wd}")
    X = O.uniform(N * I, 0x5EED5, -1, 1)
    if ce:
        T = np.eye(O_, dtype=np.float32)[O.ids(N, 77, O_)].ravel()
    else:
        T = O.uniform(N * O_, 0x5EED6, 0, 1)
    with make(dim_in=I, dim_hidden=H, dim_out=O_, lr=0.01, init_seed=0xADA70A50, max_batch_size=N,
              optimizer="adam", weight_decay=wd, loss="cross_entropy" if ce else "mse") as r:
        m = mirror(r)
        for k in range(K):
            m.batch_step(X, T, N, 0.01, cross_entropy=ce, adam=True, weight_decay=wd,
                         t_step=k + 1)
            r.tick_step_batch(X, T)
        assert r.adam_step == K
        d, rl, ok = params_close(r, m)
        em = rel_l2(m.M, r.read_buffer(mlp.BUF_ADAM_M))
        ev = rel_l2(m.V, r.read_buffer(mlp.BUF_ADAM_V))
        note(f"  params max|d|={d:.2e}; m rel-L2={em:.2e} v rel-L2={ev:.2e}")
        assert ok and em <= 1e-5 and ev <= 1e-5


def test_large_weights_cross_entropy_and_single_sample():
    """Weights beyond LDS: 1000 classes (the reference's CE shader covers up to
    1024, softmax_ce_loss_grad_batched.comp:16) with Adam, and one-sample
    steps of a wide input."""
    from valkyr_amd import mlp

    N, I, H, O_ = 32, 16, 64, 1000
    X = O.uniform(N * I, 81, -1, 1)
    T = np.eye(O_, dtype=np.float32)[O.ids(N, 82, O_)].ravel()
    with make(dim_in=I, dim_hidden=H, dim_out=O_, lr=0.01, init_seed=83, max_batch_size=N,
              optimizer="adam", loss="cross_entropy") as r:
        m = mirror(r)
        for k in range(2):
            m.batch_step(X, T, N, 0.01, cross_entropy=True, adam=True, t_step=k + 1)
            r.tick_step_batch(X, T)
        d, rl, ok = params_close(r, m)
        yb = r.tick_predict_batch(X[: 4 * I]).reshape(4, O_)
        y_ref = np.stack([m.forward(X.reshape(N, I)[n])[2] for n in range(4)])
        note(f"  1000-class adam: params max|d|={d:.2e} rel-L2={rl:.2e}; "
             f"predict max|d|={np.abs(yb - y_ref).max():.2e}")
        assert ok and rl <= 1e-5 and np.abs(yb - y_ref).max() <= 1e-5
    with make(dim_in=300, dim_hidden=64, dim_out=10, lr=0.02, init_seed=84) as r:
        m = mirror(r)
        for k in range(4):
            x, t = O.uniform(300, 90 + k, -1, 1), O.uniform(10, 95 + k, 0, 1)
            _, _, y_ref = m.forward(x)
            pred = r.tick_step(x, t)
            m.train_step(x, t, 0.02)
            assert np.abs(pred - y_ref).max() <= 1e-5
        d, _, ok = params_close(r, m, 1e-5)
        assert ok, d


def test_cross_entropy_loss_gradient():
    """runTrainingRunnerCrossEntropySmoke (training.zig:2158-2262): lr = 0,
    half one-hot and half soft targets; dy = (softmax(y) - t) / N."""
    from valkyr_amd import mlp

    N, O_ = 32, 5
    note("mlp CE dy 4-8-5 N=32")
    X = O.uniform(N * 4, 0xCEED57A, -1, 1)
    T = np.zeros((N, O_), np.float32)
    T[np.arange(N // 2), O.ids(N // 2, 3, O_)] = 1
    soft = O.uniform((N - N // 2) * O_, 4, 0, 1).reshape(-1, O_)
    T[N // 2:] = soft / soft.sum(1, keepdims=True)
    with make(dim_in=4, dim_hidden=8, dim_out=O_, lr=0.0, init_seed=0xC10557E, max_batch_size=N,
              loss="cross_entropy") as r:
        m = mirror(r)
        r.tick_step_batch(X, T)
        y = r.read_buffer(mlp.BUF_Y_TRAIN, N * O_).reshape(N, O_)
        dy = r.read_buffer(mlp.BUF_DY_TRAIN, N * O_).reshape(N, O_)
        want = np.stack([O.softmax_ce_grad_row(y[n], T[n]) for n in range(N)]) / N
        y_ref = np.stack([m.forward(X.reshape(N, 4)[n])[2] for n in range(N)])
        note(f"  dy max|d|={np.abs(dy - want).max():.2e} y max|d|={np.abs(y - y_ref).max():.2e}")
        assert np.abs(dy - want).max() <= 1e-5
        assert np.abs(y - y_ref).max() <= 1e-5
        assert np.array_equal(mirror(r).P, m.P)  # lr = 0: weights untouched


def test_weight_decay_shrinks_w_only():
    """runWeightDecayCosineLrSmoke (training.zig:1338-1420): zero input and
    target, 30 steps: ||W|| = ||W0|| (1 - lr wd)^30, biases stay 0."""
    lr, wd, K = 0.05, 0.1, 30
    with make(dim_in=4, dim_hidden=8, dim_out=4, lr=lr, weight_decay=wd,
              init_seed=0xCDDECA1) as r:
        w0 = r.read_weights()
        for _ in range(K):
            r.tick_step(np.zeros(4), np.zeros(4), want_pred=False)
        w = r.read_weights()
        for k in ("w1", "w2"):
            want = np.linalg.norm(w0[k]) * (1 - lr * wd) ** K
            assert abs(np.linalg.norm(w[k]) - want) <= 1e-3 * want
        assert not w["b1"].any() and not w["b2"].any()


def test_predict_batch_equals_one_at_a_time():
    """runTrainingRunnerBatchedSmoke (training.zig:1443-1512): bit-identical."""
    N = 37
    X = O.uniform(N * 5, 9, -1, 1).reshape(N, 5)
    with make(dim_in=5, dim_hidden=16, dim_out=3, init_seed=0xBA7C4ED, max_batch_size=64) as r:
        yb = r.tick_predict_batch(X).reshape(N, 3)
        ys = np.stack([r.tick_predict(X[n]) for n in range(N)])
        assert np.array_equal(yb, ys)


def test_attach_step_record_matches_tick_step():
    from valkyr_amd.device import Stream
    from valkyr_amd import mlp

    s = Stream()
    # more records than pinned slots, none waited for: every step must train
    # on the values passed to its own call
    xs = [O.uniform(4, 200 + k, -1, 1) for k in range(40)]
    ts = [O.uniform(3, 300 + k, 0, 1) for k in range(40)]
    with make(dim_in=4, dim_hidden=16, dim_out=3, lr=0.1, init_seed=5) as r:
        m = mirror(r)
        for x, t in zip(xs, ts):
            r.tick_step_record(x, t, stream=s)
            m.train_step(x, t, 0.1)
        r.tick_predict_record(xs[0], stream=s)
        s.synchronize()
        d, _, ok = params_close(r, m, 1e-5)
        _, _, y = m.forward(xs[0])
        assert ok and np.abs(r.read_buffer(mlp.BUF_Y) - y).max() <= 1e-5


def test_tick_frame_train_budgets_and_convergence():
    """runTrainingRunnerCoopSmoke (training.zig:1690-1860)."""
    from valkyr_amd.device import Stream
    from valkyr_amd.runner import BUDGET_EITHER, BUDGET_MICROSECONDS

    n = 8
    X = O.uniform(n * 4, 0xCD0CD0, -1, 1).reshape(n, 4)
    T = np.stack([X.sum(1) * 0.5 * (0.7 + 0.1 * o) for o in range(3)], 1).astype(np.float32)
    s = Stream()
    with make(dim_in=4, dim_hidden=16, dim_out=3, lr=0.1, init_seed=0x7177EF00,
              max_batch_size=n) as r:
        m = mirror(r)
        r.upload_train_batch(X, T)
        r.upload_predict_inputs(X)

        def frame(**budget):
            res = r.tick_frame_train(n, stream=s, **budget)
            r.tick_predict_batch_record(n, stream=s)
            r.record_predict_readback(n, stream=s)
            s.synchronize()
            return res

        res = frame(steps=3)
        assert res.steps_completed == 3 and not res.idle
        for k in range(3):
            m.batch_step(X, T, n, 0.1)
        d, _, ok = params_close(r, m)
        assert ok, d
        # the staged prediction is the batched predict of the current weights
        assert np.array_equal(r.read_predict_staging(n * 3), r.tick_predict_batch(X))
        res = frame(mode=BUDGET_MICROSECONDS, microseconds=0)
        assert res.steps_completed == 0 and res.idle
        res = frame(mode=BUDGET_EITHER, steps=1, microseconds=1_000_000)
        assert res.steps_completed == 1
        loss0 = O.mse_loss(r.tick_predict_batch(X), T)
        for _ in range(30):
            frame(steps=2)
        loss1 = O.mse_loss(r.tick_predict_batch(X), T)
        note(f"  coop loss {loss0:.5f} -> {loss1:.5f}")
        assert loss1 < loss0 / 4
        # a time budget records at least one step, then stops at the cap
        res = frame(mode=BUDGET_MICROSECONDS, microseconds=200)
        note(f"  200 us budget: {res.steps_completed} steps in {res.elapsed_us} us")
        assert res.steps_completed >= 1


def test_loss_target_decay_gates_and_resumes():
    """runTrainingRunnerDecaySmoke (training.zig:2271-2420), plus the staged
    loss against the oracle's batch loss of the same weights."""
    from valkyr_amd.device import Stream

    n = 8
    X = O.uniform(n * 4, 0xDECAD0, -1, 1)
    T = O.uniform(n * 3, 0xDECAD1, -2, 2)
    s = Stream()
    with make(dim_in=4, dim_hidden=16, dim_out=3, lr=0.05, init_seed=0xDECA1A77,
              max_batch_size=n, optimizer="adam", decay_target=0.001) as r:
        r.upload_train_batch(X, T)
        idle_at, last = None, None
        for f in range(200):
            res = r.tick_frame_train(n, steps=4, stream=s)
            s.synchronize()
            if f > 0:
                assert res.has_loss and abs(res.last_loss - last) <= 1e-5 * max(abs(last), 1e-3)
            last = mirror(r).batch_loss(X, T, n)  # what this frame's evaluation staged
            if res.idle:
                idle_at = f
                break
        note(f"  idle at frame {idle_at}, last_loss {res.last_loss:.6f}")
        assert idle_at is not None and idle_at >= 3
        assert res.has_loss and res.last_loss <= 0.001 and res.steps_completed == 0
        for _ in range(5):
            res = r.tick_frame_train(n, steps=4, stream=s)
            s.synchronize()
            assert res.idle and res.steps_completed == 0
        r.upload_train_batch(X, np.full(n * 3, 5.0, np.float32))
        resumed = None
        for f in range(3):
            res = r.tick_frame_train(n, steps=4, stream=s)
            s.synchronize()
            if not res.idle:
                resumed = f
                break
        assert resumed is not None and res.steps_completed == 4
        assert r.get_last_loss() > 0.001


def test_error_names():
    import valkyr_amd as v

    def err(fn, *a, **kw):
        with pytest.raises(v.VkhError) as e:
            fn(*a, **kw)
        return e.value.name

    with make(dim_in=4, dim_hidden=8, dim_out=3) as r:
        assert err(r.tick_step, np.zeros(5), np.zeros(3)) == "XDimMismatch"
        assert err(r.tick_step, np.zeros(4), np.zeros(2)) == "TargetDimMismatch"
        assert err(r.tick_step, np.zeros(4), np.zeros(3), out_len=2) == "OutDimMismatch"
        assert err(r.tick_predict, np.zeros(4), out_len=4) == "OutDimMismatch"
        for call in (lambda: r.tick_predict_batch(np.zeros(8)),
                     lambda: r.tick_step_batch(np.zeros(8), np.zeros(6)),
                     lambda: r.upload_train_batch(np.zeros(8), np.zeros(6)),
                     lambda: r.tick_frame_train(2),
                     lambda: r.record_predict_readback(2)):
            assert err(call) == "BatchSizeNotConfigured"
    with make(dim_in=4, dim_hidden=8, dim_out=3, max_batch_size=4) as r:
        assert err(r.tick_predict_batch, np.zeros(7)) == "XBatchDimMismatch"
        assert err(r.tick_predict_batch, np.zeros(20)) == "BatchSizeExceedsMax"
        assert err(r.tick_predict_batch, np.zeros(8), out_len=5) == "OutBatchDimMismatch"
        assert err(r.tick_step_batch, np.zeros(8), np.zeros(5)) == "TargetBatchDimMismatch"
        assert err(r.tick_frame_train, 5) == "BatchSizeExceedsMax"
        assert err(r.read_predict_staging, 13) == "OutputTooLarge"
        r.tick_step_batch(np.zeros(0), np.zeros(7))  # n == 0 returns before the target check
        res = r.tick_frame_train(0)
        assert res.idle and res.steps_completed == 0
