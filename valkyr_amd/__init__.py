"""valkyr_amd — MI355X (gfx950) training backward path of valkyr.

The compute is libvkhip.so (hand-written HIP kernels behind the C ABI in
include/vkhip.h); this package is its Python host mirror.  There is no CPU
fallback: without the built library, `lib()` raises MissingLibraryError.
"""
from ._lib import (Config, MissingLibraryError, VkhError, check, device_count, lib)  # noqa: F401
from .runner import Runner, make_config  # noqa: F401
from .dataset import Dataset, finetune, mean_ce  # noqa: F401
from .mlp import TrainingRunner, make_mlp_config  # noqa: F401

__all__ = ["Config", "MissingLibraryError", "VkhError", "Runner", "make_config", "lib", "check",
           "device_count", "build", "Dataset", "finetune", "mean_ce", "TrainingRunner",
           "make_mlp_config"]


def build(jobs: int = 8) -> str:
    """Compile libvkhip.so for gfx950 in-tree (hipcc, no network)."""
    from .build import build_library

    return build_library(jobs)
