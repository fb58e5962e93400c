"""Builds libdecisive_rocm.so for gfx950 in-tree (decisive_amd/lib/).

hipcc cross-compiles without a GPU. Each .hip translation unit is compiled in
parallel, then linked. DZ_SOURCE_HASH (SHA-256 of the kernel sources) feeds
the tuner's cache key, so a kernel change invalidates cached selections.
"""
from __future__ import annotations

import concurrent.futures as cf
import hashlib
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
INCLUDE = PKG.parent / "include"
OUT_DIR = PKG / "lib"
LIB = OUT_DIR / "libdecisive_rocm.so"
BUILD = PKG / "_build"

ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    # no packed FP32 instructions anywhere in device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in VGPRs: in the AGPR form the compiler copied every int32
    # group dot of the bit-exact products back with v_accvgpr_read before the
    # fold (4 of about 18 VALU instructions per MFMA in those VALU-bound loops)
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wno-unused-result",
    "-Wno-unused-value",
]


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def source_hash() -> str:
    h = hashlib.sha256()
    for p in sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.hpp")) + [INCLUDE / "decisive_rocm.h"]):
        h.update(p.name.encode())
        h.update(p.read_bytes())
    return h.hexdigest()[:32]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found")


def build(verbose: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    OUT_DIR.mkdir(exist_ok=True)
    cc = hipcc()
    define = f"-DDZ_SOURCE_HASH=\"{source_hash()}\""

    def compile_one(src: Path) -> Path:
        obj = BUILD / (src.stem + ".o")
        cmd = [cc, *FLAGS, define, f"-I{INCLUDE}", "-c", str(src), "-o", str(obj)]
        r = subprocess.run(cmd, capture_output=True, text=True)
        noise = "is not a recognized feature for this target"
        err = "\n".join(l for l in r.stderr.splitlines() if noise not in l)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
        if verbose and err.strip():
            print(err, file=sys.stderr)
        return obj

    with cf.ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
        objs = list(ex.map(compile_one, sources()))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
