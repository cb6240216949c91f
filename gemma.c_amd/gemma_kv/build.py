"""Builds libgemma4_kv.so (the gfx950 HIP kernels + C-ABI) in-tree with hipcc.

Every HIP source is compiled for gfx950 only, with packed-FP32 instruction
selection disabled, and linked into one shared library next to this file.
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC_DIR = PKG_DIR.parent / "csrc"
REPO_ROOT = PKG_DIR.parent.parent
INCLUDE_DIR = REPO_ROOT / "include"
LIB_NAME = "libgemma4_kv.so"
LIB_PATH = PKG_DIR / LIB_NAME
OBJ_DIR = PKG_DIR / "_build"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE_DIR}",
    f"-I{CSRC_DIR}",
]


# Per-source additions. The prefill kernels rescale their MFMA accumulators with
# VALU multiplies on a rarely taken path; in the AGPR form the register
# allocator copies all 128 accumulators between AGPRs and VGPRs on every tile
# to serve that path, so their MFMAs are selected in the VGPR form.
EXTRA_FLAGS = {
    "prefill_attention": ["-mllvm", "-amdgpu-mfma-vgpr-form=true"],
    "prefill_norm_rope": ["-mllvm", "-amdgpu-mfma-vgpr-form=true"],
}


def sources() -> list[Path]:
    return sorted(list(CSRC_DIR.glob("*.hip")) + list(CSRC_DIR.glob("*.cpp")))


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature.
    noise = ("packed-fp32-ops", "not a recognized feature")
    err = "\n".join(l for l in proc.stderr.splitlines() if not any(n in l for n in noise))
    if proc.returncode != 0:
        raise RuntimeError(f"command failed: {' '.join(cmd)}\n{err}")
    if err.strip():
        print(err, file=sys.stderr)


def build(jobs: int = 8) -> Path:
    """Compile every source and link the shared library; returns its path."""
    OBJ_DIR.mkdir(exist_ok=True)
    objs = []
    procs = []
    for src in sources():
        obj = OBJ_DIR / (src.stem + ".o")
        objs.append(obj)
        cmd = [HIPCC, *HIP_FLAGS, *EXTRA_FLAGS.get(src.stem, []), "-c", str(src), "-o", str(obj)]
        procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE,
                                            stderr=subprocess.PIPE, text=True)))
        if len(procs) >= jobs:
            _drain(procs)
    _drain(procs)
    tmp = LIB_PATH.with_suffix(".so.tmp")
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp),
          *map(str, objs)])
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def _drain(procs) -> None:
    noise = ("packed-fp32-ops", "not a recognized feature")
    while procs:
        cmd, p = procs.pop(0)
        _, err = p.communicate()
        err = "\n".join(l for l in err.splitlines() if not any(n in l for n in noise))
        if p.returncode != 0:
            raise RuntimeError(f"command failed: {' '.join(cmd)}\n{err}")
        if err.strip():
            print(err, file=sys.stderr)


if __name__ == "__main__":
    print(build())
