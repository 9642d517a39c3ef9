"""In-tree build of libfemtochat_attn.so with hipcc for gfx950.

Each HIP source is compiled to an object in femtochat_amd/_build/ (in
parallel), then linked into femtochat_amd/libfemtochat_attn.so, which the
ctypes binding loads.  Always recompiles: this is the build check.
"""
from __future__ import annotations

import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
SOURCES = ["attn_api.hip", "attn_fwd.hip", "attn_bwd.hip", "attn_fwd_fast.hip", "attn_bwd_fast.hip", "attn_bwd_dkdv_vgpr.hip", "rope_norm.hip", "loss.hip", "xla_bridge.hip", "optim.hip", "embed_sort.hip", "convert.hip"]
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    # Packed fp32 VALU ops are disabled for every HIP translation unit.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]

# Per-source additions.  The dK/dV kernel at head dims up to 64 selects the
# vector-register form of every MFMA, so that S and dP are not copied out of
# the accumulation registers element by element (at D = 128 the compiler's
# default, accumulation-register form stays: that kernel needs both files).
EXTRA_FLAGS = {"attn_bwd_dkdv_vgpr.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build the attention library)")


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the GPU-only feature.
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{err}")
    return err


def build(verbose: bool = False) -> Path:
    cc = hipcc()
    BUILD.mkdir(exist_ok=True)
    objs = [BUILD / (Path(s).stem + ".o") for s in SOURCES]
    cmds = [[cc, *HIPCC_FLAGS, *EXTRA_FLAGS.get(s, []), "-c", str(CSRC / s), "-o", str(o)]
            for s, o in zip(SOURCES, objs)]
    with ThreadPoolExecutor(max_workers=len(cmds)) as ex:
        for err in ex.map(_run, cmds):
            if verbose and err.strip():
                print(err)
    out = PKG / "libfemtochat_attn.so"
    tmp = out.with_suffix(".so.tmp")
    rocm_lib = Path(cc).resolve().parent.parent / "lib"
    # rocBLAS: the batched GEMMs of Polar Express (optim.hip)
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs), f"-L{rocm_lib}",
          f"-Wl,-rpath,{rocm_lib}", "-lrocblas"])
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build(verbose=True))
