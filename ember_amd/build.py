"""Builds libember_hip.so (gfx950 kernels + host C++ + the C ABI) in-tree.

Every HIP source is compiled with hipcc for gfx950 only; the host-only C++
(block manager, step planner, C ABI) goes through hipcc too so that one
toolchain links everything. Objects land in ember_amd/_build/, the library
next to this file, where ember_amd._lib loads it.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libember_hip.so"

SOURCES = [
    CSRC / "capi.hip",
    CSRC / "kv_append.hip",
    CSRC / "paged_decode.hip",
    CSRC / "prefill_attn.hip",
    CSRC / "copy_pages.hip",
    CSRC / "linear.hip",
    CSRC / "static_scratch.hip",
    CSRC / "sampling.hip",
    CSRC / "host" / "kvcache" / "block_manager.cpp",
    CSRC / "host" / "common" / "json.cpp",
    CSRC / "host" / "common" / "mmap_file.cpp",
    CSRC / "host" / "model" / "config.cpp",
    CSRC / "host" / "model" / "safetensors.cpp",
    CSRC / "host" / "backend" / "hip_paged_kv.cpp",
    CSRC / "host" / "backend" / "hip_backend.cpp",
    CSRC / "host" / "backend" / "backend.cpp",
    CSRC / "host" / "capi_host.cpp",
]

ARCH = "gfx950"


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found: the ROCm toolchain is required to build ember_amd")
    return path


def common_flags() -> list[str]:
    return [
        "-O3",
        "-std=c++20",
        "-fPIC",
        "-Wall",
        f"--offload-arch={ARCH}",
        # No contraction: every multiply-add the kernels fuse is written as fmaf,
        # so rounding is fixed by the source (decode == verify bit-exactly).
        "-ffp-contract=off",
        # Packed FP32 instructions stay off (they have produced wrong results on this pool).
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        f"-I{ROOT / 'include'}",
        f"-I{CSRC}",
        f"-I{CSRC / 'host'}",
    ]


# Per-source additions. The decode kernel rescales its MFMA accumulators on the
# VALU every page: they stay in VGPRs (the VGPR form of v_mfma) instead of
# being copied out of and back into AGPRs around each rescale. Its first seven
# kernel arguments (the work descriptors' address, n_kv, the pools, the block
# tables, qkv and the rotary frequencies) are preloaded into scalar registers at
# launch, so a work-group's descriptor load does not wait for a kernel-argument
# load first (gfx950 supports the preload; the code object carries a prologue
# that loads them itself where the firmware does not).
# The linear layers' kernels take plain arguments: their first nine (the
# GEMV's operands, shapes and staging constant; all of RMSNorm's) are
# preloaded, so their first loads issue at once.
EXTRA_FLAGS = {
    "paged_decode.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form", "-mllvm", "-amdgpu-kernarg-preload-count=7"],
    "linear.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=9"],
    "kv_append.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=8"],
    "prefill_attn.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=9"],
}


def _compile(src: Path) -> Path:
    obj = BUILD / (src.relative_to(CSRC).as_posix().replace("/", "__") + ".o")
    cmd = [hipcc(), *common_flags(), *EXTRA_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    if src.suffix == ".cpp":
        cmd[1:1] = ["-x", "hip"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compiling {src.name} failed:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    # The host pass does not know the packed-fp32 feature: that warning is expected.
    noise = [ln for ln in res.stderr.splitlines() if ln.strip() and "packed-fp32-ops" not in ln]
    if noise:
        sys.stderr.write(f"[ember_amd build] {src.name}:\n" + "\n".join(noise) + "\n")
    return obj


def build(verbose: bool = True) -> Path:
    """Compiles every source and links ember_amd/libember_hip.so. Always rebuilds."""
    BUILD.mkdir(exist_ok=True)
    workers = min(len(SOURCES), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(workers) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"linking libember_hip.so failed:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"[ember_amd build] {LIB} ({LIB.stat().st_size // 1024} KiB, {ARCH})")
    return LIB


if __name__ == "__main__":
    build()
