"""Shared helpers for the GPU parity tests (comparison metrics, uploads)."""
from __future__ import annotations

import sys

import numpy as np


def rel_l2(ref, got) -> float:
    ref = np.asarray(ref, np.float64).ravel()
    got = np.asarray(got, np.float64).ravel()
    n = np.linalg.norm(ref)
    return float(np.linalg.norm(ref - got) / (n if n > 0 else 1.0))


def grel(ref, got) -> float:
    """max|a-b| / max|a| (the reference smokes' metric, cce.zig:358-368)."""
    ref = np.asarray(ref, np.float64).ravel()
    got = np.asarray(got, np.float64).ravel()
    m = np.abs(ref).max()
    d = np.abs(ref - got).max()
    return float(d / m if m > 1e-30 else d)


def dev(a):
    from valkyr_amd.device import DeviceBuffer

    return DeviceBuffer.from_numpy(np.ascontiguousarray(a))


def zeros(n, dtype=np.float32):
    from valkyr_amd.device import DeviceBuffer

    return DeviceBuffer.zeros(int(n) * np.dtype(dtype).itemsize)


def host(buf, n=None, dtype=np.float32):
    from valkyr_amd.device import synchronize

    synchronize()
    return buf.to_numpy(dtype, n)


def bf16_dev(a):
    """Upload fp32 values as bf16 (RNE) and return (buffer, widened fp32 values)."""
    from valkyr_amd.device import bf16_bits_to_f32, f32_to_bf16_bits

    bits = f32_to_bf16_bits(np.asarray(a, np.float32))
    return dev(bits), bf16_bits_to_f32(bits)


def note(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()
