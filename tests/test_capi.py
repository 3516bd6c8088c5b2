"""CPU-side checks of the C ABI: the library loads, exports every symbol
include/vkhip.h declares, the Python binding covers them all, and host-side
argument validation works without a GPU."""
import ctypes as C
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "vkhip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(vkh_[a-z0-9_]+)\s*\(", text)))


def test_header_compiles_as_c_and_cpp(tmp_path):
    src = tmp_path / "t.c"
    src.write_text('#include "vkhip.h"\nint main(void){ vkh_config c = {0}; (void)c; return 0; }\n')
    for cc, flag in (("gcc", "-std=c99"), ("g++", "-std=c++17")):
        out = tmp_path / f"t_{cc}"
        r = subprocess.run([cc, flag, "-Wall", "-Werror", "-I", os.path.dirname(HEADER),
                            "-x", "c" if cc == "gcc" else "c++", str(src), "-o", str(out)],
                           capture_output=True, text=True)
        assert r.returncode == 0, r.stderr


def test_library_exports_every_declared_symbol():
    from valkyr_amd._lib import LIB_PATH, lib

    lib()  # loads
    out = subprocess.run(["nm", "-D", "--defined-only", LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (vkh_[a-z0-9_]+)", out))
    missing = [f for f in declared_functions() if f not in exported]
    assert not missing, missing


def test_binding_covers_every_declared_symbol():
    from valkyr_amd._lib import SIGNATURES

    bound = {name for name, _, _ in SIGNATURES}
    assert set(declared_functions()) == bound


def test_config_struct_layout_matches_header(tmp_path):
    """sizeof/offsets of the ABI structs agree between C and ctypes."""
    from valkyr_amd import _lib as L

    structs = {"vkh_config": L.Config, "vkh_attn_params": L.AttnParams,
               "vkh_cce_params": L.CceParams, "vkh_rope_params": L.RopeParams,
               "vkh_train_budget": L.TrainBudget, "vkh_tick_result": L.TickResult,
               "vkh_init_weights": L.InitWeights, "vkh_layer_weights": L.LayerWeights,
               "vkh_mlp_config": L.MlpConfig}
    body = "\n".join(f'printf("%s %zu\\n", "{n}", sizeof({n}));' for n in structs)
    src = tmp_path / "s.c"
    src.write_text(f'#include <stdio.h>\n#include "vkhip.h"\nint main(void){{ {body} return 0; }}\n')
    exe = tmp_path / "s"
    subprocess.run(["gcc", "-I", os.path.dirname(HEADER), str(src), "-o", str(exe)], check=True)
    sizes = dict(line.split() for line in subprocess.run([str(exe)], capture_output=True,
                                                          text=True, check=True).stdout.split("\n") if line)
    for n, cls in structs.items():
        assert int(sizes[n]) == C.sizeof(cls), n


def test_status_names_match():
    from valkyr_amd._lib import STATUS, lib

    for code, name in STATUS.items():
        assert lib().vkh_status_name(code).decode() == name


def test_invalid_arguments_rejected_on_host():
    """Argument validation happens before any device work."""
    from valkyr_amd import kernels as K
    from valkyr_amd._lib import VkhError

    with pytest.raises(VkhError) as e:
        K.fa_forward(K.attn_params(4, 4, 3, 2, 16), None, None, None, None)  # 3 % 2 != 0
    assert e.value.name == "InvalidArgument"
    with pytest.raises(VkhError) as e:
        K.fa_forward(K.attn_params(8, 4, 4, 2, 16, causal=True), 1, 1, 1, 1)  # n_q > n_kv
    assert e.value.name == "InvalidArgument"
    with pytest.raises(VkhError) as e:
        K.fa_forward(K.attn_params(8, 8, 4, 2, 96, dtype=K.BF16), 1, 1, 1, 1)
    assert e.value.name == "Unsupported"


def test_runner_without_device_reports_no_device():
    import valkyr_amd as v

    if v.device_count() > 0:
        pytest.skip("a GPU is present")
    cfg = v.make_config(dim=16, n_heads=2, n_kv_heads=1, head_dim=8, ff_dim=32, n_pos=4,
                        n_layers=1, vocab_size=8)
    with pytest.raises(v.VkhError) as e:
        v.Runner(cfg)
    assert e.value.name == "NoDevice"


def test_mlp_config_checks_before_device():
    """runner.zig:329: HiddenDimExceedsMax comes before any device work."""
    import valkyr_amd as v

    with pytest.raises(v.VkhError) as e:
        v.TrainingRunner(4, 65, 3, 0.1)
    assert e.value.name == "HiddenDimExceedsMax"
    with pytest.raises(v.VkhError) as e:
        v.TrainingRunner(0, 8, 3, 0.1)
    assert e.value.name == "InvalidArgument"
    c = v.make_mlp_config(4, 8, 3, 0.05)
    # Mlp2Config defaults (runner.zig:70-123)
    assert (c.init_seed, c.max_batch_size, c.optimizer, c.loss, c.decay) == (0xCAFE, 0, 0, 0, 0)
    assert abs(c.init_scale - 0.3) < 1e-7 and abs(c.adam_beta1 - 0.9) < 1e-7
    assert abs(c.adam_beta2 - 0.999) < 1e-7 and abs(c.adam_eps - 1e-8) < 1e-15
    assert c.weight_decay == 0.0


def test_checkpoint_config_block_layout():
    """The .vkpt / .lvkpt config block is the reference's `Config` as bytes
    (transformer.zig:31-77, :1405-1406): an auto-layout Zig struct, so its
    nineteen 4-byte fields in declaration order, then causal and qk_norm as
    one byte each, then two bytes of padding (80 bytes).  Checked against a
    block packed here field by field, both ways."""
    import struct

    import valkyr_amd as v
    from valkyr_amd.runner import checkpoint_config_bytes, checkpoint_config_from_bytes

    cfg = v.make_config(dim=1024, n_heads=16, n_kv_heads=8, head_dim=128, ff_dim=3072, n_pos=512,
                        n_layers=28, vocab_size=151936, rms_eps=1e-6, causal=1, rotary_dim=96,
                        rope_theta=1e6, qk_norm=1, lr=3e-4, beta1=0.85, beta2=0.995,
                        eps_adam=1e-7, lora_targets=0x15, lora_rank=8, lora_alpha=16.0,
                        lora_lr_b_scale=4.0, n_seqs=4, tied_embeddings=1, precision=1)
    fields = (1024, 16, 8, 128, 3072, 512, 28, 151936, 1e-6, 96, 1e6, 3e-4, 0.85, 0.995, 1e-7,
              0x15, 8, 16.0, 4.0, 1, 1)
    want = struct.pack("<8If If 4f 2I 2f 2B 2x", *fields)
    assert len(want) == 80
    assert checkpoint_config_bytes(cfg) == want
    back = checkpoint_config_from_bytes(want)
    for name in ("dim", "n_heads", "n_kv_heads", "head_dim", "ff_dim", "n_pos", "n_layers",
                 "vocab_size", "rotary_dim", "lora_targets", "lora_rank", "causal", "qk_norm"):
        assert getattr(back, name) == getattr(cfg, name), name
    for name in ("rms_eps", "rope_theta", "lr", "beta1", "beta2", "eps_adam", "lora_alpha",
                 "lora_lr_b_scale"):
        assert getattr(back, name) == getattr(cfg, name), name
    # the extensions are not in the reference's block
    assert (back.n_seqs, back.tied_embeddings, back.precision) == (1, 0, 0)
    # bool bytes: causal off, qk_norm off
    off = struct.pack("<8If If 4f 2I 2f 2B 2x", *(fields[:19] + (0, 0)))
    c2 = checkpoint_config_from_bytes(off)
    assert c2.causal == 0 and c2.qk_norm == 0
    with pytest.raises(v.VkhError) as e:
        checkpoint_config_from_bytes(want + b"\0\0\0\0")
    assert e.value.name == "CheckpointConfigSizeMismatch"
