"""Build libtinytron_amd.so in-tree with hipcc for gfx950.

Usage: python -m tinytron_amd.build  (or tinytron_amd.build.build()).
The library is written next to this file so that it travels with the source
tree; nothing is installed.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
LIB_PATH = PKG_DIR / "libtinytron_amd.so"
OBJ_DIR = PKG_DIR / "_build"  # per-source objects (git-ignored)
SOURCES = ["abi.hip", "rope_append.hip", "decode_attn.hip", "prefill_attn.hip", "layer_ops.hip", "sampler.hip"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fno-gpu-flush-denormals-to-zero",
    # no packed-fp32 VALU ops anywhere in the device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-command-line-argument",
]

# Per-source additions. prefill_attn: MFMA accumulators in the VGPR form, with
# AGPRs left to the register allocator as spill room. The head_dim-128 bf16
# prefill kernel (4 column blocks at up to 512 registers a wave) otherwise keeps
# its loop-carried O accumulators in VGPRs and copies them to AGPRs and back
# around every PV: about 290 v_accvgpr moves per 32-key tile, a third of the
# tile's VALU instructions. The other kernels of the file compile the same.
SOURCE_FLAGS = {"prefill_attn.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the gfx950 library cannot be built")


def _run(cmd, verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed with exit code {res.returncode}")


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every HIP source into LIB_PATH (always recompiles): one object
    per source, compiled concurrently, then one link."""
    OBJ_DIR.mkdir(exist_ok=True)
    inc = ["-I", str(PKG_DIR.parent / "include")]
    objs = [OBJ_DIR / (Path(s).stem + ".o") for s in SOURCES]
    cmds = [[hipcc(), *HIPCC_FLAGS, *SOURCE_FLAGS.get(s, []), *inc, "-c", str(CSRC / s), "-o", str(o)]
            for s, o in zip(SOURCES, objs)]
    jobs = jobs or min(len(cmds), max(1, min(os.cpu_count() or 1, 16)))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        for f in [pool.submit(_run, c, verbose) for c in cmds]:
            f.result()
    tmp = LIB_PATH.with_suffix(".so.tmp")
    _run([hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", *[str(o) for o in objs], "-o", str(tmp)], verbose)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
