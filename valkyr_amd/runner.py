"""Python mirror of valkyr's transformer training `Runner`
(src/train/transformer.zig:207-1655) over the C ABI of libvkhip.

    cfg = Config(dim=..., n_heads=..., ...)
    r = Runner(cfg, weights)            # Runner.init (transformer.zig:482)
    r.step(token_ids, target_ids)       # Runner.step (:1257), blocking
    r.forward_logits(token_ids)         # Runner.forwardLogits (:1324)
    r.save_checkpoint(path)             # .vkpt (:1390); .lvkpt (:1479)
    r.tick_frame_train(budget)          # TrainingRunner.tickFrameTrain shape (runner.zig:904)

Weights are passed as a dict of fp32 numpy arrays: `embed`, `final_norm`,
`lm_head` and `layers` (a list of dicts with `w_n1 w_q w_k w_v w_o w_n2 w_gate
w_up w_down [w_q_norm w_k_norm]`), plus optional `lora` =
{proj_index: [{"a": A, "b": B}, ...per layer]}.  Lengths are validated by the
library exactly like the reference (errors EmbedShape, LayerQShape, ...).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from ._lib import (Config, InitWeights, LayerWeights, LoraInit, Tensor, TickResult,
                   TrainBudget, check, lib)

PARAM, GRAD, ADAM_M, ADAM_V = 0, 1, 2, 3
# stack-level "which"
EMBED, FINAL_NORM, LM_HEAD = 0, 1, 2
# per-layer "which" (Layer.paramSlices order, train_decoder.zig:100-102)
N1, Q, K, V, O, N2, GATE, UP, DOWN, Q_NORM, K_NORM = range(11)
LAYER_NAMES = ["w_n1", "w_q", "w_k", "w_v", "w_o", "w_n2", "w_gate", "w_up", "w_down",
               "w_q_norm", "w_k_norm"]
PROJ = {"q": 0, "k": 1, "v": 2, "o": 3, "gate": 4, "up": 5, "down": 6}
LORA_Q, LORA_K, LORA_V, LORA_O = 1, 2, 4, 8
LORA_ALL_ATTN = 0xF


def lora_a(proj: int) -> int:
    return 16 + 2 * proj


def lora_b(proj: int) -> int:
    return 17 + 2 * proj


BUDGET_STEPS, BUDGET_MICROSECONDS, BUDGET_EITHER = 0, 1, 2


@dataclass
class TickResultPy:
    steps_completed: int
    has_loss: bool
    last_loss: float
    idle: bool
    elapsed_us: int


CHECKPOINT_CONFIG_BYTES = 80


def checkpoint_config_bytes(cfg: Config) -> bytes:
    """The 80-byte config block a .vkpt / .lvkpt carries (the reference's
    `Config` bytes, transformer.zig:31-77, :1405-1406)."""
    buf = (C.c_uint8 * CHECKPOINT_CONFIG_BYTES)()
    check(lib().vkh_checkpoint_config_encode(C.byref(cfg), buf, CHECKPOINT_CONFIG_BYTES))
    return bytes(buf)


def checkpoint_config_from_bytes(data: bytes) -> Config:
    cfg = Config()
    buf = (C.c_uint8 * len(data)).from_buffer_copy(data)
    check(lib().vkh_checkpoint_config_decode(buf, len(data), C.byref(cfg)))
    return cfg


def make_config(**kw) -> Config:
    """vkh_config with the reference's defaults (transformer.zig:31-77)."""
    d = dict(rms_eps=1e-5, causal=1, rotary_dim=0, rope_theta=10000.0, qk_norm=0, lr=1e-2,
             beta1=0.9, beta2=0.999, eps_adam=1e-8, lora_targets=0, lora_rank=0, lora_alpha=0.0,
             lora_lr_b_scale=1.0, n_seqs=1, tied_embeddings=0, precision=0, recompute=0)
    d.update(kw)
    return Config(**d)


def _tensor(a, keep):
    if a is None:
        return Tensor(None, 0)
    a = np.ascontiguousarray(a, np.float32).reshape(-1)
    keep.append(a)
    return Tensor(a.ctypes.data_as(C.c_void_p), a.size)


class Runner:
    def __init__(self, cfg: Config, weights: dict | None = None):
        self.cfg = cfg
        self._h = C.c_void_p()
        keep = []
        wp = None
        if weights is not None:
            layers = (LayerWeights * max(1, len(weights["layers"])))()
            for i, lw in enumerate(weights["layers"]):
                for name in LAYER_NAMES:
                    setattr(layers[i], name, _tensor(lw.get(name), keep))
            iw = InitWeights()
            iw.embed = _tensor(weights["embed"], keep)
            iw.final_norm = _tensor(weights["final_norm"], keep)
            iw.lm_head = _tensor(weights.get("lm_head"), keep)
            iw.layers = layers
            iw.n_layers = len(weights["layers"])
            keep.append(layers)
            for p, per_layer in (weights.get("lora") or {}).items():
                arr = (LoraInit * len(per_layer))()
                for i, ab in enumerate(per_layer):
                    arr[i].a = _tensor(ab["a"], keep)
                    arr[i].b = _tensor(ab["b"], keep)
                keep.append(arr)
                iw.lora[p] = C.cast(arr, C.POINTER(LoraInit))
                iw.lora_len[p] = len(per_layer)
            wp = C.byref(iw)
        check(lib().vkh_runner_create(C.byref(cfg), wp, C.byref(self._h)))
        n_seqs = cfg.n_seqs or 1
        self.T = cfg.n_pos * n_seqs

    def close(self):
        if getattr(self, "_h", None) is not None and self._h.value:
            lib().vkh_runner_destroy(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        self.close()

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    @property
    def handle(self):
        return self._h

    # ── steps ────────────────────────────────────────────────────────
    @staticmethod
    def _ids(x):
        x = np.ascontiguousarray(x, np.uint32)
        return x, x.ctypes.data_as(C.c_void_p), x.size

    def init_random(self, seed: int, std: float = 0.02, lora_std: float = 0.02):
        check(lib().vkh_runner_init_random(self._h, seed, std, lora_std))

    def step(self, token_ids, target_ids) -> None:
        t, tp, tn = self._ids(token_ids)
        g, gp, gn = self._ids(target_ids)
        check(lib().vkh_runner_step(self._h, tp, tn, gp, gn))

    def step_async(self, token_ids, target_ids, stream=None) -> None:
        t, tp, tn = self._ids(token_ids)
        g, gp, gn = self._ids(target_ids)
        check(lib().vkh_runner_step_async(self._h, tp, tn, gp, gn,
                                          stream.handle if stream else None))

    def forward_backward(self, token_ids, target_ids) -> float:
        t, tp, tn = self._ids(token_ids)
        g, gp, gn = self._ids(target_ids)
        check(lib().vkh_runner_forward_backward(self._h, tp, tn, gp, gn))
        return self.last_loss()

    def last_loss(self) -> float:
        v = C.c_float()
        check(lib().vkh_runner_last_loss(self._h, C.byref(v)))
        return v.value

    def synchronize(self):
        check(lib().vkh_runner_synchronize(self._h))

    def forward_logits(self, token_ids) -> np.ndarray:
        t, tp, tn = self._ids(token_ids)
        out = np.empty(self.T * self.cfg.vocab_size, np.float32)
        check(lib().vkh_runner_forward_logits(self._h, tp, tn, out.ctypes.data_as(C.c_void_p),
                                              out.size))
        return out.reshape(self.T, self.cfg.vocab_size)

    # ── state ────────────────────────────────────────────────────────
    @property
    def step_t(self) -> int:
        return lib().vkh_runner_step_t(self._h)

    @step_t.setter
    def step_t(self, t: int):
        check(lib().vkh_runner_set_step_t(self._h, t))

    @property
    def lr(self) -> float:
        return lib().vkh_runner_get_lr(self._h)

    @lr.setter
    def lr(self, v: float):
        check(lib().vkh_runner_set_lr(self._h, v))

    def param_count(self) -> int:
        return lib().vkh_runner_param_count(self._h)

    def device_bytes(self) -> int:
        return lib().vkh_runner_device_bytes(self._h)

    def numel(self, kind, layer, which) -> int:
        n = C.c_size_t()
        check(lib().vkh_runner_tensor_numel(self._h, kind, layer, which, C.byref(n)))
        return n.value

    def get(self, kind, layer, which) -> np.ndarray:
        n = self.numel(kind, layer, which)
        out = np.empty(n, np.float32)
        check(lib().vkh_runner_get_tensor(self._h, kind, layer, which,
                                          out.ctypes.data_as(C.c_void_p), n))
        return out

    def set(self, kind, layer, which, values) -> None:
        a = np.ascontiguousarray(values, np.float32).reshape(-1)
        check(lib().vkh_runner_set_tensor(self._h, kind, layer, which,
                                          a.ctypes.data_as(C.c_void_p), a.size))

    def device_ptr(self, kind, layer, which):
        p, n = C.c_void_p(), C.c_size_t()
        check(lib().vkh_runner_tensor_device_ptr(self._h, kind, layer, which, C.byref(p), C.byref(n)))
        return p.value, n.value

    def attention_backward_path(self) -> str:
        """'recompute', 'ds_gemm' or 'rowwise': the step's attention backward."""
        return {0: "rowwise", 1: "ds_gemm", 2: "recompute"}[
            int(lib().vkh_runner_attention_backward_path(self._h))]

    def set_boundary_capture(self, on: bool = True) -> None:
        """Keep the gradient at every layer boundary in later backwards
        (stage-by-stage checks)."""
        check(lib().vkh_runner_set_boundary_capture(self._h, int(bool(on))))

    def boundary(self, l: int, which: int) -> np.ndarray:
        """which = 0: the residual-stream tensor at boundary l (0 the
        embedding output, l the output of layer l - 1); which = 1: the
        captured gradient at it.  fp32 [T, dim] flattened."""
        c = self.cfg
        out = np.empty(c.n_pos * max(1, c.n_seqs) * c.dim, np.float32)
        check(lib().vkh_runner_boundary_read(self._h, l, which,
                                             out.ctypes.data_as(C.c_void_p), out.size))
        return out

    def attention_backward_plan(self) -> dict:
        """The step's attention-backward launch plan: path, query rows per dQ
        block, dQ and dK/dV block counts, and whether RoPE^T and the Q/K-norm
        backward run in the recompute kernels' epilogues."""
        out = (C.c_uint32 * 5)()
        check(lib().vkh_runner_attention_backward_plan(self._h, C.byref(out)))
        return {"path": {0: "rowwise", 1: "ds_gemm", 2: "recompute"}[int(out[0])],
                "dq_block_rows": int(out[1]), "dq_blocks": int(out[2]),
                "dkv_blocks": int(out[3]), "qk_epilogue": bool(out[4])}

    # ── checkpoints ──────────────────────────────────────────────────
    def save_checkpoint(self, path: str):
        check(lib().vkh_runner_save_checkpoint(self._h, path.encode()))

    def load_checkpoint(self, path: str):
        check(lib().vkh_runner_load_checkpoint(self._h, path.encode()))

    def save_lora_checkpoint(self, path: str):
        check(lib().vkh_runner_save_lora_checkpoint(self._h, path.encode()))

    def load_lora_checkpoint(self, path: str):
        check(lib().vkh_runner_load_lora_checkpoint(self._h, path.encode()))

    # ── cooperative per-frame API ────────────────────────────────────
    def upload_train_batch(self, token_ids, target_ids):
        t, tp, tn = self._ids(token_ids)
        g, gp, gn = self._ids(target_ids)
        check(lib().vkh_runner_upload_train_batch(self._h, tp, tn, gp, gn))

    def set_loss_target(self, target: float):
        check(lib().vkh_runner_set_loss_target(self._h, target))

    def tick_frame_train(self, steps=1, microseconds=0, mode=BUDGET_STEPS, stream=None):
        res = TickResult()
        check(lib().vkh_runner_tick_frame_train(self._h, stream.handle if stream else None,
                                                TrainBudget(mode, steps, microseconds),
                                                C.byref(res)))
        return TickResultPy(res.steps_completed, bool(res.has_loss), res.last_loss,
                            bool(res.idle), res.elapsed_us)
