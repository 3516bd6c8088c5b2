"""Python mirror of valkyr's tiny-MLP `TrainingRunner` (src/train/runner.zig)
over the vkh_mlp_* C ABI of libvkhip.

    r = TrainingRunner(dim_in=4, dim_hidden=16, dim_out=3, lr=5e-3,
                       max_batch_size=256, optimizer="adam",
                       decay_target=0.005)                 # Mlp2Config + init
    r.tick_step(x, target)                 # tickStep (runner.zig:598)
    r.tick_step_batch(xb, tb)              # tickStepBatch (:746)
    r.upload_train_batch(xb, tb)           # uploadTrainBatch (:784)
    res = r.tick_frame_train(steps=2, n_samples=len(tb) // 3)   # tickFrameTrain (:904)
    r.tick_predict_batch_record(n); r.record_predict_readback(n)
    y = r.read_predict_staging(n)          # readPredictStaging (:857)

Inputs are fp32 arrays of any shape; their element counts are checked by the
library exactly like the reference's slice lengths (errors XDimMismatch,
XBatchDimMismatch, BatchSizeExceedsMax, ...).
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import MlpConfig, TickResult, TrainBudget, check, lib
from .runner import BUDGET_EITHER, BUDGET_MICROSECONDS, BUDGET_STEPS, TickResultPy

MAX_HIDDEN = 64
SGD, ADAM = 0, 1
MSE, CROSS_ENTROPY = 0, 1
DECAY_NONE, DECAY_LOSS_TARGET = 0, 1
(BUF_PARAMS, BUF_GRADS, BUF_ADAM_M, BUF_ADAM_V, BUF_Y, BUF_X_BATCH, BUF_Y_BATCH, BUF_X_TRAIN,
 BUF_TARGET, BUF_H_PRE_TRAIN, BUF_H_TRAIN, BUF_Y_TRAIN, BUF_DY_TRAIN,
 BUF_DH_PRE_TRAIN) = range(14)

_OPT = {"sgd": SGD, "adam": ADAM, SGD: SGD, ADAM: ADAM}
_LOSS = {"mse": MSE, "cross_entropy": CROSS_ENTROPY, MSE: MSE, CROSS_ENTROPY: CROSS_ENTROPY}


def make_mlp_config(dim_in, dim_hidden, dim_out, lr, decay_target=None, **kw) -> MlpConfig:
    """vkh_mlp_config with the defaults of Mlp2Config (runner.zig:70-123).
    `optimizer` / `loss` take "sgd" | "adam" / "mse" | "cross_entropy";
    `decay_target` set means LossDecay.loss_target."""
    c = MlpConfig()
    lib().vkh_mlp_config_default(C.byref(c), dim_in, dim_hidden, dim_out, lr)
    if decay_target is not None:
        c.decay, c.decay_target = DECAY_LOSS_TARGET, decay_target
    for k, v in kw.items():
        if k == "optimizer":
            v = _OPT[v]
        elif k == "loss":
            v = _LOSS[v]
        setattr(c, k, v)
    return c


def _f32(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    return a, a.ctypes.data_as(C.c_void_p), a.size


def _handle(stream):
    return None if stream is None else stream.handle


class TrainingRunner:
    def __init__(self, dim_in=None, dim_hidden=None, dim_out=None, lr=None, config=None, **kw):
        self.cfg = config if config is not None else make_mlp_config(dim_in, dim_hidden, dim_out,
                                                                     lr, **kw)
        h = C.c_void_p()
        check(lib().vkh_mlp_create(C.byref(self.cfg), C.byref(h)))
        self._h = h
        c = self.cfg
        self.dim_in, self.dim_hidden, self.dim_out = c.dim_in, c.dim_hidden, c.dim_out

    def close(self):
        if getattr(self, "_h", None):
            lib().vkh_mlp_destroy(self._h)
            self._h = None

    __del__ = close

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # ── mutable hyper-parameters ──────────────────────────────────────
    @property
    def lr(self) -> float:
        return lib().vkh_mlp_get_lr(self._h)

    @lr.setter
    def lr(self, v: float):
        check(lib().vkh_mlp_set_lr(self._h, v))

    def set_weight_decay(self, wd: float):
        check(lib().vkh_mlp_set_weight_decay(self._h, wd))

    @property
    def adam_step(self) -> int:
        return lib().vkh_mlp_adam_step(self._h)

    # ── standalone (blocking) ─────────────────────────────────────────
    def tick_step(self, x, target, want_pred=True, out_len=None):
        x, xp, xn = _f32(x)
        t, tp, tn = _f32(target)
        out = np.empty(self.dim_out if out_len is None else out_len, np.float32)
        op = out.ctypes.data_as(C.c_void_p) if want_pred else None
        check(lib().vkh_mlp_tick_step(self._h, xp, xn, tp, tn, op, out.size if want_pred else 0))
        return out if want_pred else None

    def tick_predict(self, x, out_len=None):
        x, xp, xn = _f32(x)
        out = np.empty(self.dim_out if out_len is None else out_len, np.float32)
        check(lib().vkh_mlp_tick_predict(self._h, xp, xn, out.ctypes.data_as(C.c_void_p),
                                         out.size))
        return out

    def tick_predict_batch(self, x_batch, out_len=None):
        x, xp, xn = _f32(x_batch)
        n = out_len if out_len is not None else (xn // self.dim_in) * self.dim_out
        out = np.empty(n, np.float32)
        check(lib().vkh_mlp_tick_predict_batch(self._h, xp, xn, out.ctypes.data_as(C.c_void_p),
                                               out.size))
        return out

    def tick_step_batch(self, x_batch, target_batch):
        x, xp, xn = _f32(x_batch)
        t, tp, tn = _f32(target_batch)
        check(lib().vkh_mlp_tick_step_batch(self._h, xp, xn, tp, tn))

    # ── cooperative (attach) ──────────────────────────────────────────
    def upload_train_batch(self, x_batch, target_batch):
        x, xp, xn = _f32(x_batch)
        t, tp, tn = _f32(target_batch)
        check(lib().vkh_mlp_upload_train_batch(self._h, xp, xn, tp, tn))

    def upload_predict_inputs(self, x_batch):
        x, xp, xn = _f32(x_batch)
        check(lib().vkh_mlp_upload_predict_inputs(self._h, xp, xn))

    def tick_step_record(self, x, target, stream=None):
        x, xp, xn = _f32(x)
        t, tp, tn = _f32(target)
        check(lib().vkh_mlp_tick_step_record(self._h, _handle(stream), xp, xn, tp, tn))

    def tick_predict_record(self, x, stream=None):
        x, xp, xn = _f32(x)
        check(lib().vkh_mlp_tick_predict_record(self._h, _handle(stream), xp, xn))

    def tick_step_batch_record(self, n_samples, stream=None):
        check(lib().vkh_mlp_tick_step_batch_record(self._h, _handle(stream), n_samples))

    def tick_predict_batch_record(self, n_samples, stream=None):
        check(lib().vkh_mlp_tick_predict_batch_record(self._h, _handle(stream), n_samples))

    def record_predict_readback(self, n_samples, stream=None):
        check(lib().vkh_mlp_record_predict_readback(self._h, _handle(stream), n_samples))

    def read_predict_staging(self, n_values):
        out = np.empty(n_values, np.float32)
        check(lib().vkh_mlp_read_predict_staging(self._h, out.ctypes.data_as(C.c_void_p),
                                                 out.size))
        return out

    def tick_frame_train(self, n_samples, steps=1, microseconds=0, mode=BUDGET_STEPS,
                         stream=None) -> TickResultPy:
        """budget: mode BUDGET_STEPS (steps), BUDGET_MICROSECONDS (microseconds)
        or BUDGET_EITHER (both)."""
        res = TickResult()
        check(lib().vkh_mlp_tick_frame_train(self._h, _handle(stream),
                                             TrainBudget(mode, steps, microseconds), n_samples,
                                             C.byref(res)))
        return TickResultPy(res.steps_completed, bool(res.has_loss), res.last_loss,
                            bool(res.idle), res.elapsed_us)

    def get_last_loss(self):
        v, has = C.c_float(0), C.c_uint32(0)
        check(lib().vkh_mlp_get_last_loss(self._h, C.byref(v), C.byref(has)))
        return v.value if has.value else None

    # ── buffers ───────────────────────────────────────────────────────
    def buffer(self, which):
        """(device pointer, element count) of a runner buffer."""
        p, n = C.c_void_p(), C.c_size_t(0)
        check(lib().vkh_mlp_buffer(self._h, which, C.byref(p), C.byref(n)))
        return p.value, n.value

    def read_buffer(self, which, numel=None):
        _, n = self.buffer(which)
        n = n if numel is None else numel
        out = np.empty(n, np.float32)
        check(lib().vkh_mlp_read_buffer(self._h, which, out.ctypes.data_as(C.c_void_p), n))
        return out

    def read_weights(self):
        """readWeights (runner.zig:684-689): dict w1 [H, I], b1, w2 [O, H], b2."""
        I, H, O = self.dim_in, self.dim_hidden, self.dim_out
        w1, b1 = np.empty((H, I), np.float32), np.empty(H, np.float32)
        w2, b2 = np.empty((O, H), np.float32), np.empty(O, np.float32)
        ptr = lambda a: a.ctypes.data_as(C.c_void_p)  # noqa: E731
        check(lib().vkh_mlp_read_weights(self._h, ptr(w1), w1.size, ptr(b1), b1.size, ptr(w2),
                                         w2.size, ptr(b2), b2.size))
        return {"w1": w1, "b1": b1, "w2": w2, "b2": b2}


__all__ = ["TrainingRunner", "make_mlp_config", "MAX_HIDDEN", "BUDGET_STEPS",
           "BUDGET_MICROSECONDS", "BUDGET_EITHER"]
