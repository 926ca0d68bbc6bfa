"""The C-ABI library builds for gfx950, loads, and exports every symbol include/sid_hip.h
declares; argument validation runs before any device work (no GPU needed)."""

from __future__ import annotations

import ctypes
import re

import pytest

from conftest import ROOT


def _declared() -> list[str]:
    text = (ROOT / "include" / "sid_hip.h").read_text()
    return sorted(set(re.findall(r"^\w[\w\s\*]*?\b(sid_\w+)\(", text, flags=re.M)))


@pytest.fixture(scope="module")
def ext():
    from sid.kernels.jit import load_ext
    return load_ext()


def test_header_declares_the_path():
    names = _declared()
    for must in ("sid_flash_decode_fwd", "sid_reshape_and_cache", "sid_extend_attention_fwd",
                 "sid_rmsnorm", "sid_fused_add_rmsnorm", "sid_rope_apply", "sid_linear"):
        assert must in names


def test_library_exports_every_declared_symbol(ext):
    for name in _declared():
        assert hasattr(ext.lib, name), f"{name} declared in sid_hip.h but not exported"


def test_python_binding_matches_header(ext):
    from sid.kernels._native import EXPORTED
    assert sorted(EXPORTED) == _declared()


def test_abi_version(ext):
    from sid.kernels._native import ABI_VERSION
    assert ext.lib.sid_abi_version() == ABI_VERSION == 22


def test_validation_errors_without_device_work(ext):
    lib = ext.lib
    f = ctypes.c_float(0.1)
    # head_dim 64 is rejected before anything touches the device
    rc = lib.sid_flash_decode_fwd(1, 1, 1, 1, 1, 1, 1, 16, 8, 64, 10, 1, 0, f, None, None, 1, 1,
                                  1, None)
    assert rc == 1 and b"head_dim" in lib.sid_last_error()
    rc = lib.sid_flash_decode_fwd(1, 1, 1, 1, 1, 1, 1, 12, 8, 128, 10, 1, 0, f, None, None, 1, 1,
                                  1, None)
    assert rc == 1 and b"q heads" in lib.sid_last_error()
    rc = lib.sid_flash_decode_fwd(1, 1, 1, 1, 1, 1, 2, 16, 8, 128, 10, 4, 0, f, 1, 1, 1, 2, 1,
                                  None)
    assert rc == 1 and b"workspace" in lib.sid_last_error()
    rc = lib.sid_linear(16, 1000, 16, None, 16, 4, 64, 1000, 0, None)
    assert rc == 1 and b"multiple of 256" in lib.sid_last_error()
    rc = lib.sid_linear(16, 1024, 16, None, 16, 4, 60, 1024, 0, None)
    assert rc == 1 and b"multiple of 64" in lib.sid_last_error()
    rc = lib.sid_reshape_and_cache(1, 1, 1, 1, 1, 4, 1, 3, 10, None)
    assert rc == 1 and b"16-byte" in lib.sid_last_error()
    # gate_up + SwiGLU: K fixed at 1024, I a multiple of 8, 16-byte aligned operands
    rc = lib.sid_linear_silu_mul(16, 16, 16, 4, 2048, 3072, None)
    assert rc == 1 and b"K must be 1024" in lib.sid_last_error()
    rc = lib.sid_linear_silu_mul(16, 16, 16, 4, 1024, 3074, None)
    assert rc == 1 and b"multiple of 8" in lib.sid_last_error()
    rc = lib.sid_linear_silu_mul(8, 16, 16, 4, 1024, 3072, None)
    assert rc == 1 and b"misaligned" in lib.sid_last_error()
    assert lib.sid_linear_silu_mul(None, None, None, 0, 1024, 3072, None) == 0
    # empty work is a successful no-op
    assert lib.sid_reshape_and_cache(None, None, None, None, None, 0, 8, 128, 10, None) == 0
    assert lib.sid_flash_decode_fwd(None, None, None, None, None, None, 0, 16, 8, 128, 10, 1, 0, f,
                                    None, None, 0, 0, None, None) == 0


def test_ops_reject_cpu_tensors(ext):
    import torch
    q = torch.zeros(1, 16, 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU tensor"):
        ext.reshape_and_cache(q[:, :8], q[:, :8], q[:, :8], q[:, :8], torch.zeros(1, dtype=torch.int64))
