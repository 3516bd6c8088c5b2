"""ctypes binding of libvkhip.so (the C ABI declared in include/vkhip.h).

The HIP library is the product: there is no Python or CPU fallback.  If the
shared library has not been built, importing anything that needs it raises
`MissingLibraryError` with the build command.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libvkhip.so")


class MissingLibraryError(RuntimeError):
    pass


class VkhError(RuntimeError):
    def __init__(self, status: int, name: str, message: str):
        super().__init__(f"{name} ({status}): {message}")
        self.status = status
        self.name = name
        self.message = message


# vkh_status codes (include/vkhip.h)
STATUS = {
    0: "Ok", 1: "InvalidArgument", 2: "HipError", 3: "OutOfMemory", 4: "Unsupported",
    5: "NoDevice", 10: "TokenIdsLen", 11: "TargetLen", 12: "OutLogitsLen",
    13: "TokenOutOfRange", 20: "EmbedShape", 21: "FinalNormShape", 22: "LmHeadShape",
    23: "LayerCount", 24: "LayerN1Shape", 25: "LayerQShape", 26: "LayerKShape",
    27: "LayerVShape", 28: "LayerOShape", 29: "LayerN2Shape", 30: "LayerGateShape",
    31: "LayerUpShape", 32: "LayerDownShape", 33: "LayerQNormShape", 34: "LayerKNormShape",
    35: "LoraRankZero", 36: "LoraInitLen", 40: "InvalidCheckpointMagic",
    41: "UnsupportedCheckpointVersion", 42: "CheckpointConfigSizeMismatch",
    43: "CheckpointConfigMismatch", 44: "EndOfStream", 45: "InvalidLoraCheckpointMagic",
    46: "UnsupportedLoraCheckpointVersion", 47: "LoraCheckpointConfigSizeMismatch",
    48: "LoraCheckpointConfigMismatch", 49: "LoraCheckpointEmpty", 50: "IoError",
    60: "InputIdsLen", 61: "TargetIdsLen", 62: "BatchIndexOutOfRange", 63: "EmptyDataset",
    64: "DatasetTooShort", 65: "BatchIdxOutOfRange", 70: "HiddenDimExceedsMax",
    71: "XDimMismatch", 72: "TargetDimMismatch", 73: "OutDimMismatch",
    74: "BatchSizeNotConfigured", 75: "BatchSizeExceedsMax", 76: "XBatchDimMismatch",
    77: "TargetBatchDimMismatch", 78: "OutBatchDimMismatch", 79: "OutputTooLarge",
}


class Config(C.Structure):
    """vkh_config: transformer.zig:31-77 plus n_seqs / tied_embeddings / precision."""

    _fields_ = [
        ("dim", C.c_uint32), ("n_heads", C.c_uint32), ("n_kv_heads", C.c_uint32),
        ("head_dim", C.c_uint32), ("ff_dim", C.c_uint32), ("n_pos", C.c_uint32),
        ("n_layers", C.c_uint32), ("vocab_size", C.c_uint32), ("rms_eps", C.c_float),
        ("causal", C.c_uint32), ("rotary_dim", C.c_uint32), ("rope_theta", C.c_float),
        ("qk_norm", C.c_uint32), ("lr", C.c_float), ("beta1", C.c_float),
        ("beta2", C.c_float), ("eps_adam", C.c_float), ("lora_targets", C.c_uint32),
        ("lora_rank", C.c_uint32), ("lora_alpha", C.c_float), ("lora_lr_b_scale", C.c_float),
        ("n_seqs", C.c_uint32), ("tied_embeddings", C.c_uint32), ("precision", C.c_uint32),
        ("recompute", C.c_uint32),
    ]


class Tensor(C.Structure):
    _fields_ = [("data", C.c_void_p), ("len", C.c_size_t)]


class LayerWeights(C.Structure):
    _fields_ = [(n, Tensor) for n in ("w_n1", "w_q", "w_k", "w_v", "w_o", "w_n2", "w_gate",
                                      "w_up", "w_down", "w_q_norm", "w_k_norm")]


class LoraInit(C.Structure):
    _fields_ = [("a", Tensor), ("b", Tensor)]


class InitWeights(C.Structure):
    _fields_ = [("embed", Tensor), ("final_norm", Tensor), ("lm_head", Tensor),
                ("layers", C.POINTER(LayerWeights)), ("n_layers", C.c_size_t),
                ("lora", C.POINTER(LoraInit) * 7), ("lora_len", C.c_size_t * 7)]


class AttnParams(C.Structure):
    _fields_ = [("n_batch", C.c_uint32), ("n_q", C.c_uint32), ("n_kv", C.c_uint32),
                ("n_heads", C.c_uint32), ("n_kv_heads", C.c_uint32), ("head_dim", C.c_uint32),
                ("causal", C.c_uint32), ("inv_sqrt_dim", C.c_float), ("dtype", C.c_uint32)]


class LoraAdapter(C.Structure):
    _fields_ = [("col", C.c_uint32), ("n", C.c_uint32), ("k", C.c_uint32),
                ("a", C.c_void_p), ("b", C.c_void_p), ("inter", C.c_void_p), ("dyb", C.c_void_p),
                ("da", C.c_void_p), ("db", C.c_void_p)]


class CceParams(C.Structure):
    _fields_ = [("n", C.c_uint32), ("vocab", C.c_uint32), ("dim", C.c_uint32),
                ("z_loss_scale", C.c_float), ("label_smoothing", C.c_float),
                ("precision", C.c_uint32)]


class RopeParams(C.Structure):
    _fields_ = [("n_pos", C.c_uint32), ("n_q_heads", C.c_uint32), ("n_kv_heads", C.c_uint32),
                ("head_dim", C.c_uint32), ("rotary_dim", C.c_uint32), ("theta_base", C.c_float),
                ("seq_len", C.c_uint32)]


class TrainBudget(C.Structure):
    _fields_ = [("mode", C.c_uint32), ("steps", C.c_uint32), ("microseconds", C.c_uint64)]


class TickResult(C.Structure):
    _fields_ = [("steps_completed", C.c_uint32), ("has_loss", C.c_uint32),
                ("last_loss", C.c_float), ("idle", C.c_uint32), ("elapsed_us", C.c_uint64)]


class FinetuneResult(C.Structure):
    _fields_ = [("ce_initial", C.c_float), ("ce_final", C.c_float), ("total_ms", C.c_double),
                ("mean_step_ms", C.c_double)]


class MlpConfig(C.Structure):
    """vkh_mlp_config: Mlp2Config (runner.zig:70-123)."""

    _fields_ = [
        ("dim_in", C.c_uint32), ("dim_hidden", C.c_uint32), ("dim_out", C.c_uint32),
        ("lr", C.c_float), ("init_scale", C.c_float), ("max_batch_size", C.c_uint32),
        ("init_seed", C.c_uint64), ("optimizer", C.c_uint32), ("adam_beta1", C.c_float),
        ("adam_beta2", C.c_float), ("adam_eps", C.c_float), ("loss", C.c_uint32),
        ("decay", C.c_uint32), ("decay_target", C.c_float), ("weight_decay", C.c_float),
    ]


P = C.c_void_p
U32 = C.c_uint32
SZ = C.c_size_t
F = C.c_float
ST = C.c_int

# (name, restype, argtypes) for every function include/vkhip.h declares.
SIGNATURES = [
    ("vkh_runner_create", ST, [C.POINTER(Config), C.POINTER(InitWeights), C.POINTER(P)]),
    ("vkh_runner_destroy", None, [P]),
    ("vkh_runner_init_random", ST, [P, C.c_uint64, F, F]),
    ("vkh_runner_step", ST, [P, P, SZ, P, SZ]),
    ("vkh_runner_step_async", ST, [P, P, SZ, P, SZ, P]),
    ("vkh_runner_last_loss", ST, [P, C.POINTER(F)]),
    ("vkh_runner_forward_logits", ST, [P, P, SZ, P, SZ]),
    ("vkh_runner_forward_backward", ST, [P, P, SZ, P, SZ]),
    ("vkh_runner_synchronize", ST, [P]),
    ("vkh_runner_step_t", U32, [P]),
    ("vkh_runner_set_step_t", ST, [P, U32]),
    ("vkh_runner_get_lr", F, [P]),
    ("vkh_runner_set_lr", ST, [P, F]),
    ("vkh_runner_get_config", ST, [P, C.POINTER(Config)]),
    ("vkh_runner_param_count", SZ, [P]),
    ("vkh_runner_device_bytes", SZ, [P]),
    ("vkh_runner_tensor_numel", ST, [P, C.c_int, C.c_int, C.c_int, C.POINTER(SZ)]),
    ("vkh_runner_get_tensor", ST, [P, C.c_int, C.c_int, C.c_int, P, SZ]),
    ("vkh_runner_set_tensor", ST, [P, C.c_int, C.c_int, C.c_int, P, SZ]),
    ("vkh_runner_tensor_device_ptr", ST, [P, C.c_int, C.c_int, C.c_int, C.POINTER(P), C.POINTER(SZ)]),
    ("vkh_runner_save_checkpoint", ST, [P, C.c_char_p]),
    ("vkh_runner_load_checkpoint", ST, [P, C.c_char_p]),
    ("vkh_runner_save_lora_checkpoint", ST, [P, C.c_char_p]),
    ("vkh_runner_load_lora_checkpoint", ST, [P, C.c_char_p]),
    ("vkh_runner_attention_backward_path", U32, [P]),
    ("vkh_runner_attention_backward_plan", ST, [P, C.POINTER(C.c_uint32 * 5)]),
    ("vkh_runner_set_boundary_capture", ST, [P, U32]),
    ("vkh_runner_boundary_read", ST, [P, U32, U32, P, SZ]),
    ("vkh_checkpoint_config_encode", ST, [C.POINTER(Config), P, SZ]),
    ("vkh_checkpoint_config_decode", ST, [P, SZ, C.POINTER(Config)]),
    ("vkh_runner_upload_train_batch", ST, [P, P, SZ, P, SZ]),
    ("vkh_runner_set_loss_target", ST, [P, F]),
    ("vkh_runner_tick_frame_train", ST, [P, P, TrainBudget, C.POINTER(TickResult)]),
    ("vkh_dataset_from_examples", ST, [P, P, SZ, U32, U32, C.POINTER(P)]),
    ("vkh_dataset_from_jsonl", ST, [C.c_char_p, U32, U32, C.POINTER(P)]),
    ("vkh_dataset_destroy", None, [P]),
    ("vkh_dataset_num_batches", SZ, [P]),
    ("vkh_dataset_packed_len", SZ, [P]),
    ("vkh_dataset_packed", ST, [P, P, SZ]),
    ("vkh_dataset_batch", ST, [P, SZ, P, SZ, P, SZ]),
    ("vkh_dataset_batch_seqs", ST, [P, SZ, SZ, U32, P, P]),
    ("vkh_mean_ce", F, [P, P, SZ, SZ]),
    ("vkh_runner_finetune", ST, [P, P, U32, U32, U32, C.POINTER(FinetuneResult)]),
    ("vkh_mlp_config_default", None, [C.POINTER(MlpConfig), U32, U32, U32, F]),
    ("vkh_mlp_create", ST, [C.POINTER(MlpConfig), C.POINTER(P)]),
    ("vkh_mlp_destroy", None, [P]),
    ("vkh_mlp_get_config", ST, [P, C.POINTER(MlpConfig)]),
    ("vkh_mlp_set_lr", ST, [P, F]),
    ("vkh_mlp_get_lr", F, [P]),
    ("vkh_mlp_set_weight_decay", ST, [P, F]),
    ("vkh_mlp_adam_step", U32, [P]),
    ("vkh_mlp_tick_step", ST, [P, P, SZ, P, SZ, P, SZ]),
    ("vkh_mlp_tick_predict", ST, [P, P, SZ, P, SZ]),
    ("vkh_mlp_tick_predict_batch", ST, [P, P, SZ, P, SZ]),
    ("vkh_mlp_tick_step_batch", ST, [P, P, SZ, P, SZ]),
    ("vkh_mlp_upload_train_batch", ST, [P, P, SZ, P, SZ]),
    ("vkh_mlp_upload_predict_inputs", ST, [P, P, SZ]),
    ("vkh_mlp_tick_step_record", ST, [P, P, P, SZ, P, SZ]),
    ("vkh_mlp_tick_predict_record", ST, [P, P, P, SZ]),
    ("vkh_mlp_tick_step_batch_record", ST, [P, P, U32]),
    ("vkh_mlp_tick_predict_batch_record", ST, [P, P, U32]),
    ("vkh_mlp_record_predict_readback", ST, [P, P, U32]),
    ("vkh_mlp_read_predict_staging", ST, [P, P, SZ]),
    ("vkh_mlp_tick_frame_train", ST, [P, P, TrainBudget, U32, C.POINTER(TickResult)]),
    ("vkh_mlp_get_last_loss", ST, [P, C.POINTER(F), C.POINTER(U32)]),
    ("vkh_mlp_buffer", ST, [P, U32, C.POINTER(P), C.POINTER(SZ)]),
    ("vkh_mlp_read_buffer", ST, [P, U32, P, SZ]),
    ("vkh_mlp_read_weights", ST, [P, P, SZ, P, SZ, P, SZ, P, SZ]),
    ("vkh_fa_forward", ST, [C.POINTER(AttnParams), P, P, P, P, P, P]),
    ("vkh_fa_bw_d", ST, [C.POINTER(AttnParams), P, P, P, P, P]),
    ("vkh_fa_bw_d_bf16", ST, [C.POINTER(AttnParams), P, P, P, P]),
    ("vkh_fa_bw_dq", ST, [C.POINTER(AttnParams), P, P, P, P, P, P, P, P]),
    ("vkh_fa_bw_dkv", ST, [C.POINTER(AttnParams), P, P, P, P, P, P, P, P, P]),
    ("vkh_fa_backward_workspace_bytes", SZ, [C.POINTER(AttnParams)]),
    ("vkh_fa_backward", ST, [C.POINTER(AttnParams), P, P, P, P, P, P, P, P, P, P, P]),
    ("vkh_fa_backward_from_o", ST, [C.POINTER(AttnParams), P, P, P, P, P, P, P, P, P, P, P, P]),
    ("vkh_matmul_nt", ST, [P, P, P, U32, U32, U32, U32, P]),
    ("vkh_linear_backward_dx", ST, [P, P, P, U32, U32, U32, U32, P]),
    ("vkh_linear_backward_dw", ST, [P, P, P, U32, U32, U32, U32, P]),
    ("vkh_matmul_nt_bf16", ST, [P, P, P, U32, U32, U32, P]),
    ("vkh_gate_up_swiglu_bf16", ST, [P, P, P, P, U32, U32, U32, P]),
    ("vkh_qkv_project_bf16", ST, [P, U32, C.c_float, C.c_int, P, P, P, P, P, P, C.c_int, P]),
    ("vkh_qkv_project", ST, [P, U32, C.c_float, C.c_int, P, P, P, P, P, P, C.c_int, P]),
    ("vkh_gate_up_swiglu", ST, [P, P, P, P, U32, U32, U32, C.c_int, P]),
    ("vkh_linear_backward_dx_bf16", ST, [P, P, P, U32, U32, U32, P]),
    ("vkh_linear_backward_dw_bf16", ST, [P, P, P, U32, U32, U32, P]),
    ("vkh_lora_forward", ST, [P, P, P, P, P, P, U32, U32, U32, U32, F, U32, P]),
    ("vkh_lora_backward", ST, [P, P, P, P, P, P, P, P, P, U32, U32, U32, U32, F, U32, P]),
    ("vkh_lora_group_forward_bf16", ST, [P, U32, U32, U32, F, C.POINTER(LoraAdapter), U32, P, U32, P]),
    ("vkh_lora_group_backward_bf16", ST, [P, U32, P, U32, U32, U32, F, C.POINTER(LoraAdapter), U32, P, U32, P]),
    ("vkh_cce_forward", ST, [C.POINTER(CceParams), P, P, P, P, P, P, P]),
    ("vkh_cce_backward", ST, [C.POINTER(CceParams), P, P, P, P, P, P, U32, P]),
    ("vkh_rmsnorm_forward", ST, [P, P, P, U32, U32, F, U32, P]),
    ("vkh_rmsnorm_backward", ST, [P, P, P, P, P, P, U32, U32, F, U32, P]),
    ("vkh_rmsnorm_backward_noalloc", ST, [P, P, P, P, P, P, U32, U32, F, U32, P]),
    ("vkh_allocation_count", C.c_uint64, []),
    ("vkh_swiglu_forward", ST, [P, P, P, SZ, P]),
    ("vkh_swiglu_backward", ST, [P, P, P, P, P, SZ, P]),
    ("vkh_qk_rope_forward", ST, [C.POINTER(RopeParams), P, P, P, P, P]),
    ("vkh_qk_rope_backward", ST, [C.POINTER(RopeParams), P, P, P, P, P]),
    ("vkh_embed_lookup", ST, [P, P, P, U32, U32, F, P]),
    ("vkh_embedding_backward", ST, [P, P, P, U32, U32, U32, P]),
    ("vkh_adam_step", ST, [P, P, P, P, SZ, F, F, F, F, U32, F, P]),
    ("vkh_add_in_place", ST, [P, P, SZ, P]),
    ("vkh_vec_add", ST, [P, P, P, SZ, P]),
    ("vkh_scale", ST, [P, P, SZ, F, P]),
    ("vkh_cast_f32_to_bf16", ST, [P, P, SZ, P]),
    ("vkh_device_count", ST, [C.POINTER(C.c_int)]),
    ("vkh_set_device", ST, [C.c_int]),
    ("vkh_malloc", ST, [C.POINTER(P), SZ]),
    ("vkh_free", ST, [P]),
    ("vkh_memcpy_h2d", ST, [P, P, SZ]),
    ("vkh_memcpy_d2h", ST, [P, P, SZ]),
    ("vkh_memset", ST, [P, C.c_int, SZ]),
    ("vkh_device_synchronize", ST, []),
    ("vkh_stream_create", ST, [C.POINTER(P)]),
    ("vkh_stream_destroy", ST, [P]),
    ("vkh_stream_synchronize", ST, [P]),
    ("vkh_event_create", ST, [C.POINTER(P)]),
    ("vkh_event_destroy", ST, [P]),
    ("vkh_event_record", ST, [P, P]),
    ("vkh_event_synchronize", ST, [P]),
    ("vkh_event_elapsed_ms", ST, [P, P, C.POINTER(F)]),
    ("vkh_last_error", C.c_char_p, []),
    ("vkh_status_name", C.c_char_p, [C.c_int]),
    ("vkh_build_info", C.c_char_p, []),
]

_lib = None


def lib():
    """The loaded libvkhip.so (raises MissingLibraryError if it is not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise MissingLibraryError(
                f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; "
                f"g.build()'` (or `make -C valkyr_amd/csrc`)")
        L = C.CDLL(LIB_PATH)
        for name, res, args in SIGNATURES:
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def check(status: int) -> None:
    if status != 0:
        msg = lib().vkh_last_error().decode(errors="replace")
        raise VkhError(status, STATUS.get(status, "Unknown"), msg)


def device_count() -> int:
    n = C.c_int(0)
    st = lib().vkh_device_count(C.byref(n))
    return n.value if st == 0 else 0
