"""Compile libgsdft.so for gfx950 in-tree (``gs-dft_amd/lib/libgsdft.so``).

The library is plain hipcc output with no library dependency beyond the HIP runtime; the
translation units are compiled in parallel and linked into one shared object. FP contraction is off so every fused
multiply-add in the kernels is an explicit ``fma``; packed-FP32 instruction selection is disabled.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import pathlib
import shutil
import subprocess
import sys

HERE = pathlib.Path(__file__).resolve().parent
CSRC = HERE / "csrc"
OUT_DIR = HERE / "lib"
LIB = OUT_DIR / "libgsdft.so"
ROCM = pathlib.Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
ARCH = os.environ.get("GSDFT_ARCH", "gfx950")

SOURCES = ["abi.hip", "screen.hip", "dfj.hip", "solve.hip", "order.hip", "grid.hip",
           "exchange.hip", "gemm.hip"]

CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-ffp-contract=off",
    "-mcode-object-version=5",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-command-line-argument",
    "-I", str(HERE.parent / "include"),
]


def _hipcc() -> str:
    exe = shutil.which("hipcc") or str(ROCM / "bin" / "hipcc")
    if not pathlib.Path(exe).exists():
        raise RuntimeError("hipcc not found: the DF-J library needs ROCm's hipcc to build")
    return exe


def _compile(src: pathlib.Path, obj: pathlib.Path, extra: list[str]) -> None:
    cmd = [_hipcc(), *CFLAGS, *extra, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{r.stdout}\n{r.stderr}")
    if r.stderr.strip():
        noise = [l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l and l.strip()]
        if noise:
            sys.stderr.write("\n".join(noise) + "\n")


def build(verbose: bool = False, extra: list[str] | None = None) -> pathlib.Path:
    """Compile every translation unit and link ``libgsdft.so``; returns its path."""
    extra = list(extra or [])
    obj_dir = OUT_DIR / "obj"
    obj_dir.mkdir(parents=True, exist_ok=True)
    jobs = []
    with cf.ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        for name in SOURCES:
            src = CSRC / name
            obj = obj_dir / (src.stem + ".o")
            jobs.append(ex.submit(_compile, src, obj, extra))
        for j in jobs:
            j.result()
    tmp = LIB.with_suffix(".so.tmp")
    link = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
            *[str(obj_dir / (pathlib.Path(s).stem + ".o")) for s in SOURCES],
            f"-Wl,-rpath,{ROCM / 'lib'}"]
    r = subprocess.run(link, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
