"""Build libnvdsa.so (gfx950) in-tree with hipcc.

Each .hip translation unit is compiled separately (in parallel) into
``_build/`` at the repository root, then linked into
``nanovllm-dsa-offload_amd/nanovllm_amd/libnvdsa.so``.  Run as a script or
call :func:`build`.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

CSRC = Path(__file__).resolve().parent
PKG_ROOT = CSRC.parent
REPO = PKG_ROOT.parent
BUILD_DIR = REPO / "_build" / "nvdsa"
OUTPUT = PKG_ROOT / "nanovllm_amd" / "libnvdsa.so"
SOURCES = ("scatter_copy.hip", "lim.hip", "sfa.hip", "indexer.hip", "persist.hip", "nvdsa_abi.hip")
ARCH = os.environ.get("NVDSA_OFFLOAD_ARCH", "gfx950")

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-mcode-object-version=5",
    # Packed fp32 ops have produced silent wrong results on this pool; keep
    # the compiler from forming them.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    f"-I{REPO / 'include'}",
    f"-I{CSRC}",
]


# Per-unit additions.  lim.hip: MFMA results in VGPRs (the score epilogue reads
# every accumulator; in AGPRs each one costs an extra v_accvgpr_read).
EXTRA_FLAGS = {"lim.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=true"]}


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the nvdsa HIP library cannot be built")


def _compile(hipcc: str, src: Path, obj: Path) -> None:
    cmd = [hipcc, *COMMON_FLAGS, *EXTRA_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stdout}\n{proc.stderr}")


def build(verbose: bool = False) -> Path:
    """Compile every HIP source and link libnvdsa.so; returns its path."""
    hipcc = _hipcc()
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    objs = []
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(len(SOURCES), 8)) as pool:
        futs = []
        for name in SOURCES:
            src = CSRC / name
            obj = BUILD_DIR / (src.stem + ".o")
            objs.append(obj)
            futs.append(pool.submit(_compile, hipcc, src, obj))
        for f in futs:
            f.result()
    tmp = OUTPUT.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, OUTPUT)
    if verbose:
        print(f"built {OUTPUT}")
    return OUTPUT


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
