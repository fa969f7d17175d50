"""Build libh3attn.so (HIP, gfx950) in-tree: h3-hrx_amd/libh3attn.so.

Every translation unit is compiled with hipcc for gfx950 only, with
  -ffp-contract=off             each float operation is one IEEE operation, as the bit-exact
                                quantizer requires (no fused multiply-add unless written);
  -packed-fp32-ops disabled     no v_pk_{add,mul,fma}_f32 (hipcc's host pass warns that it does
                                not know the feature; that warning is harmless).
Usage: python h3-hrx_amd/build.py  (or __graft_entry__.build()).
"""
from __future__ import annotations

import concurrent.futures as futures
import os
import pathlib
import shutil
import subprocess
import sys

HERE = pathlib.Path(__file__).resolve().parent
CSRC = HERE / "csrc"
INCLUDE = HERE.parent / "include"
OUT = HERE / "libh3attn.so"
OBJ = HERE / "_build"
SOURCES = ["prepare.hip", "plain.hip", "attention.hip", "attention_hm.hip", "noalloc.hip", "gemm.hip",
           "abi.cpp", "stack.cpp",
           "tables.cpp", "vsa.hip", "vsa_host.cpp", "fp6.hip"]
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and pathlib.Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the HIP library cannot be built")


FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


# Per-file extras. The attention kernel is checked to a tolerance (never bit-exact) and never
# sees NaN operands, so it may drop the NaN-quieting canonicalisations IEEE mode otherwise adds
# to every max; infinities stay honoured (masked keys are -inf). The quantizer files keep full
# IEEE semantics.
EXTRA = {"attention.hip": ["-fno-honor-nans"], "attention_hm.hip": ["-fno-honor-nans"]}


def _compile(src: pathlib.Path, obj: pathlib.Path) -> None:
    cmd = [hipcc(), "-x", "hip", *FLAGS, *EXTRA.get(src.name, []), f"-I{INCLUDE}", "-c",
           str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")


def build(verbose: bool = False) -> pathlib.Path:
    """Compile every source and link libh3attn.so. Always rebuilds."""
    OBJ.mkdir(exist_ok=True)
    objs = [OBJ / (pathlib.Path(s).stem + ".o") for s in SOURCES]
    with futures.ThreadPoolExecutor(max_workers=len(SOURCES)) as pool:
        list(pool.map(lambda so: _compile(CSRC / so[0], so[1]), zip(SOURCES, objs)))
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT}")
    return OUT


if __name__ == "__main__":
    build(verbose=True)
