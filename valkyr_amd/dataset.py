"""Host feed of the training step, over libvkhip.so's C ABI.

`Dataset` mirrors train/dataset.zig's `Dataset` (packed token stream with
EOS between examples, sliding n_pos + 1 windows) on token ids; `mean_ce` is
commands/finetune.zig's `computeMeanCe`; `finetune` is that command's
training loop around `Runner.step`.  All of it runs in the library (C++),
not in Python.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import FinetuneResult, check, lib


class Dataset:
    def __init__(self, handle: C.c_void_p, n_pos: int):
        self._h = handle
        self.n_pos = n_pos

    @classmethod
    def from_examples(cls, examples, n_pos: int, eos_id: int) -> "Dataset":
        """buildFromExamples (dataset.zig:76-96) on token-id sequences."""
        arrs = [np.ascontiguousarray(e, np.uint32) for e in examples]
        ptrs = (C.c_void_p * max(1, len(arrs)))(*[a.ctypes.data_as(C.c_void_p) for a in arrs])
        lens = (C.c_size_t * max(1, len(arrs)))(*[a.size for a in arrs])
        h = C.c_void_p()
        check(lib().vkh_dataset_from_examples(ptrs, lens, len(arrs), n_pos, eos_id, C.byref(h)))
        return cls(h, n_pos)

    @classmethod
    def from_jsonl(cls, path: str, n_pos: int, eos_id: int) -> "Dataset":
        """buildFromJsonl (dataset.zig:98-148) with an "ids" array per line."""
        h = C.c_void_p()
        check(lib().vkh_dataset_from_jsonl(str(path).encode(), n_pos, eos_id, C.byref(h)))
        return cls(h, n_pos)

    def close(self):
        if getattr(self, "_h", None) is not None and self._h.value:
            lib().vkh_dataset_destroy(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        self.close()

    @property
    def handle(self):
        return self._h

    def num_batches(self) -> int:
        return lib().vkh_dataset_num_batches(self._h)

    def packed(self) -> np.ndarray:
        n = lib().vkh_dataset_packed_len(self._h)
        out = np.empty(n, np.uint32)
        check(lib().vkh_dataset_packed(self._h, out.ctypes.data_as(C.c_void_p), n))
        return out

    def batch(self, idx: int, n_input: int | None = None, n_target: int | None = None):
        """(input_ids, target_ids) of window idx (dataset.zig:50-66)."""
        ni = self.n_pos if n_input is None else n_input
        nt = self.n_pos if n_target is None else n_target
        a, b = np.zeros(max(ni, 1), np.uint32), np.zeros(max(nt, 1), np.uint32)
        check(lib().vkh_dataset_batch(self._h, idx, a.ctypes.data_as(C.c_void_p), ni,
                                      b.ctypes.data_as(C.c_void_p), nt))
        return a[:ni], b[:nt]

    def batch_seqs(self, idx: int, stride: int, n_seqs: int):
        a = np.zeros(n_seqs * self.n_pos, np.uint32)
        b = np.zeros(n_seqs * self.n_pos, np.uint32)
        check(lib().vkh_dataset_batch_seqs(self._h, idx, stride, n_seqs, a.ctypes.data_as(C.c_void_p),
                                           b.ctypes.data_as(C.c_void_p)))
        return a, b


def mean_ce(logits, target_ids, vocab: int) -> float:
    """computeMeanCe (commands/finetune.zig:256-268), fp64 accumulation."""
    lg = np.ascontiguousarray(logits, np.float32)
    tg = np.ascontiguousarray(target_ids, np.uint32)
    return lib().vkh_mean_ce(lg.ctypes.data_as(C.c_void_p), tg.ctypes.data_as(C.c_void_p), tg.size,
                             vocab)


def finetune(runner, dataset: Dataset, batch_idx: int, n_steps: int, rotate: bool = False) -> dict:
    """The training loop of commands/finetune.zig:155-196 on the library's Runner."""
    res = FinetuneResult()
    check(lib().vkh_runner_finetune(runner.handle, dataset.handle, batch_idx, n_steps,
                                    1 if rotate else 0, C.byref(res)))
    return {"ce_initial": res.ce_initial, "ce_final": res.ce_final, "total_ms": res.total_ms,
            "mean_step_ms": res.mean_step_ms}
