"""Build libg5moe.so (gfx950) in-tree with hipcc.

    python -m genet5_amd.build        # compiles csrc/*.hip -> genet5_amd/libg5moe.so

Every HIP source is compiled for gfx950 only, with packed-fp32 VALU forms
disabled, then linked into one shared library exposing the C ABI of
include/g5moe.h.  Objects go to genet5_amd/_build/.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
BUILD_DIR = PKG_DIR / "_build"
LIB_PATH = PKG_DIR / "libg5moe.so"
INCLUDE_DIR = PKG_DIR.parent / "include"

HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-command-line-argument",
    # no packed fp32 VALU forms (v_pk_fma_f32 and friends) in device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE_DIR}",
]
SOURCES = ["api.hip", "router.hip", "dispatch.hip", "grouped_gemm.hip", "combine.hip",
           "backward.hip", "attention.hip", "wgrad.hip", "xcd_balance.hip"]


def _compile(src: Path, obj: Path, verbose: bool) -> None:
    cmd = [HIPCC, *FLAGS, "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature and says so; drop that line.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in r.stderr.splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def build(verbose: bool = False) -> Path:
    """Compile every HIP source and link libg5moe.so; returns the library path."""
    BUILD_DIR.mkdir(exist_ok=True)
    objs = []
    with cf.ThreadPoolExecutor(max_workers=min(len(SOURCES), 8)) as ex:
        futs = []
        for s in SOURCES:
            obj = BUILD_DIR / (Path(s).stem + ".o")
            objs.append(obj)
            futs.append(ex.submit(_compile, CSRC / s, obj, verbose))
        for f in futs:
            f.result()
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    # A kernel whose host stub was dropped (e.g. a device builtin the host pass
    # rejected) links fine and only fails at dlopen; catch it here.
    nm = subprocess.run(["nm", "-D", "--undefined-only", str(tmp)], capture_output=True, text=True)
    missing = [l.split()[-1] for l in nm.stdout.splitlines() if "__device_stub__" in l]
    if missing:
        raise RuntimeError(f"undefined kernel host stubs in {tmp.name}: {missing}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
