"""Build the gfx950 C-ABI library ``libtasft_amd.so`` in-tree with hipcc.

Each source is compiled to an object in parallel, then linked into
``tasft_amd/_lib/libtasft_amd.so``. Run as ``python -m tasft_amd.csrc.build``.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
OUT_DIR = HERE.parent / "_lib"
LIB_NAME = "libtasft_amd.so"
SOURCES = ["capi.cpp", "prefill.hip", "decode.hip", "gate.hip", "gate_target.hip", "mask.hip"]
ARCH = "gfx950"


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm under /opt/rocm)")


def _flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-Wall",
        "-Wno-unused-function",
        # Packed fp32 VALU ops are disabled for all device code.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        # fmaxf() need not quiet its inputs first (without this flag every max over MFMA
        # results costs an extra v_max_f32 x, x per input). A NaN score may then be dropped
        # from a running maximum, but it still reaches the output through exp2 and the PV
        # product, so NaN in Q, K or V gives NaN output rows as in the reference
        # (tests/test_gpu_nan.py); infinities stay honoured.
        "-fno-honor-nans",
    ]


def _compile(hipcc: str, src: Path, obj: Path) -> None:
    lang = ["-x", "hip"] if src.suffix in (".hip", ".cpp") else []
    cmd = [hipcc, *_flags(), *lang, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in res.stderr.splitlines() if noise not in line)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")


def build(verbose: bool = True) -> Path:
    """Compile every source for gfx950 and link the shared library; returns its path."""
    hipcc = _hipcc()
    obj_dir = HERE / "_build"
    obj_dir.mkdir(exist_ok=True)
    OUT_DIR.mkdir(exist_ok=True)
    objs = [obj_dir / (Path(s).stem + ".o") for s in SOURCES]
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        futs = [ex.submit(_compile, hipcc, HERE / s, o) for s, o in zip(SOURCES, objs)]
        for f in futs:
            f.result()
    out = OUT_DIR / LIB_NAME
    tmp = OUT_DIR / (LIB_NAME + ".tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}")
    return out


if __name__ == "__main__":
    build()
