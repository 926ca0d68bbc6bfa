"""Build and load the native HIP library (`libsid_hip.so`, the C-ABI in include/sid_hip.h).

Mirrors the role of sid/kernels/jit.py:17-35 in the reference (`load_ext()` returns the
module that carries `flash_decode_fwd` and `reshape_and_cache`), but the library is an
ahead-of-time `hipcc --offload-arch=gfx950` build into the source tree, loaded with ctypes:
no JIT cache, no pybind, no torch types across the boundary.

`build_library()` always recompiles; `load_ext()` loads what is built and compiles only
when no library exists yet. There is no fallback: without the library every op raises.
"""

from __future__ import annotations

import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent.parent            # .../sid
CSRC_DIR = PKG_DIR.parent / "csrc"                         # .../deterministic-inference_amd/csrc
INCLUDE_DIR = PKG_DIR.parent.parent / "include"            # repo/include
BUILD_DIR = PKG_DIR.parent / "_build"
LIB_PATH = PKG_DIR / "libsid_hip.so"

ARCH = "gfx950"
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-mcode-object-version=5",
    # No packed-fp32 VALU instructions anywhere in this library.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]

_ext = None


# Per-source extra flags. extend_attention: the MFMA accumulators live in VGPRs (the
# softmax rescales them with VALU ops, which cannot read AGPRs).
SOURCE_FLAGS = {
    "extend_attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
}


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: cannot build libsid_hip.so")


def sources() -> list[Path]:
    return sorted(CSRC_DIR.glob("*.hip"))


def build_library(verbose: bool = False) -> Path:
    """Compile every csrc/*.hip for gfx950 and link libsid_hip.so (always rebuilds)."""
    hipcc = _hipcc()
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC_DIR}")

    def compile_one(src: Path) -> Path:
        obj = BUILD_DIR / (src.stem + ".o")
        cmd = [hipcc, *HIPCC_FLAGS, *SOURCE_FLAGS.get(src.name, []), f"-I{INCLUDE_DIR}", "-c",
               str(src), "-o", str(obj)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stderr[-4000:]}")
        if verbose:
            print(f"[sid build] {src.name}")
        return obj

    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as pool:
        objs = list(pool.map(compile_one, srcs))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link of libsid_hip.so failed:\n{res.stderr[-4000:]}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def load_ext():
    """Return the native op module (a `sid.kernels._native.NativeLib`), building it if absent."""
    global _ext
    if _ext is not None:
        return _ext
    import torch  # noqa: F401  (torch's HIP runtime must be loaded before the library binds it)

    from sid.kernels._native import NativeLib

    if not LIB_PATH.exists():
        build_library()
    _ext = NativeLib(LIB_PATH)
    return _ext


def build_all() -> None:
    """Compile the library, load it and check one decode-attention call on the GPU against a
    closed form (the build-and-verify entry point that sid/kernels/jit.py:38 provides).

    The case has an exact answer: every key of the request is the same row, so the softmax
    is uniform and each query head's output is the mean of its KV head's value rows."""
    import torch

    build_library()
    global _ext
    _ext = None
    ext = load_ext()
    assert torch.cuda.is_available(), "build_all() checks the kernels on a GPU"
    dev = torch.device("cuda", torch.cuda.current_device())
    hq, hkv, d, n = 16, 8, 128, 37
    g = torch.Generator().manual_seed(7)
    keys = torch.randn(1, hkv, d, generator=g).expand(n + 3, hkv, d).contiguous()
    vals = torch.randn(n + 3, hkv, d, generator=g)
    k_pool = keys.to(torch.bfloat16).to(dev)
    v_pool = vals.to(torch.bfloat16).to(dev)
    q = torch.randn(1, hq, d, generator=g).to(torch.bfloat16).to(dev)
    slots = torch.arange(3, n + 3, dtype=torch.int32)  # the request's positions -> slots 3..
    out = torch.empty_like(q)
    part_o = torch.empty(1, hq, 2, d, dtype=torch.float32, device=dev)
    part_lse = torch.empty(1, hq, 2, dtype=torch.float32, device=dev)
    ext.flash_decode_fwd(q, k_pool, v_pool, torch.tensor([0, n], dtype=torch.int32, device=dev),
                         slots.to(dev), torch.full((1,), 2, dtype=torch.int32, device=dev), 2, 0,
                         d ** -0.5, part_o, part_lse, out)
    want = v_pool[3:].float().mean(0).repeat_interleave(hq // hkv, 0).cpu()
    err = (out[0].float().cpu() - want).abs().max().item()
    assert err < 2e-2, f"decode attention check failed: max |error| {err:.3g}"
    print(f"{LIB_PATH.name}: built for {ARCH}, decode attention within {err:.1e} of the closed form")


if __name__ == "__main__":
    build_library(verbose=True)
    print(LIB_PATH)
