"""Build of the HIP library behind modelcore_amd: every ``csrc/*.hip`` file is compiled for gfx950
with hipcc and linked into ``modelcore_amd/_lib/libmodelcore_amd.so`` (a C-ABI shared library,
declared in ``include/modelcore_amd.h``, loaded with ctypes by ``modelcore_amd._ext``).

Run ``python -m modelcore_amd.build`` (or call :func:`build`). The library is built in-tree so it
travels with the source tree to the machine that runs it.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC_DIR = PKG_DIR / "csrc"
BUILD_DIR = PKG_DIR / "_build"
LIB_DIR = PKG_DIR / "_lib"
LIB_NAME = "libmodelcore_amd.so"
LIB_PATH = LIB_DIR / LIB_NAME

ARCH = "gfx950"

# -mcode-object-version=5: loadable by the HIP runtime bundled with PyTorch-ROCm as well as by
# the system one. The packed-fp32 feature is switched off for device code: hipcc would otherwise
# fuse pairs of fp32 FMAs into v_pk_fma_f32.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-mcode-object-version=5",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-command-line-argument",
    "-I", str(REPO_DIR / "include"),
    # Kernel arguments: LLVM preloads up to the first 16 kernel *arguments* (the count is of
    # arguments, not dwords) into SGPRs at dispatch instead of loading them from the
    # kernel-argument buffer. It stops at the first aggregate (struct) argument or when the free
    # user SGPRs run out, so on gfx950 at most 14 dwords of leading scalar arguments arrive this
    # way; the kernels that care put the fields they need first as leading scalar arguments.
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
]


# Per-source extra flags. The chunked-prefill kernel keeps its score accumulators in VGPRs, where
# the softmax reads them; without this the allocator parks them in AGPRs and copies them back and
# forth on every key tile (measured: ~500 v_accvgpr moves per tile).
SOURCE_FLAGS = {
    "prefill_mfma.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
    "decode_fused.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],  # its shared-prefix jobs
}


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found (expected on PATH or at /opt/rocm/bin/hipcc)")
    return path


def sources() -> list[Path]:
    return sorted(CSRC_DIR.glob("*.hip"))


def _compile(src: Path, verbose: bool) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, *SOURCE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass reports the device-only feature flag as unknown; drop that line.
    noise = "packed-fp32-ops' is not a recognized feature"
    err = "\n".join(line for line in res.stderr.splitlines() if noise not in line)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{err}")
    if err.strip() and verbose:
        print(err, file=sys.stderr)
    return obj


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every HIP source and link the shared library. Always rebuilds."""
    BUILD_DIR.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    srcs = sources()
    jobs = jobs or min(8, len(srcs), os.cpu_count() or 1)
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(lambda s: _compile(s, verbose), srcs))
    tmp = LIB_DIR / (LIB_NAME + ".tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
