"""Build the MI355X C-ABI library ``librxmet.so`` from ``csrc/`` with hipcc (gfx950).

Usage: ``python rx-met_amd/build.py`` (also called by ``__graft_entry__.build()``).
Objects go to ``rx-met_amd/_build/``; the shared library lands next to this file so it
travels with the source tree.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "librxmet.so"

ARCH = os.environ.get("RXMET_OFFLOAD_ARCH", "gfx950")

COMMON_FLAGS = [
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-ffp-contract=off",  # kernels and the C oracle share one rounding sequence
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
    "-Wall",
    "-Wno-unused-function",
]
# Device-code flags: no packed-FP32 instructions (v_pk_*_f32) in generated code.
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found; the MI355X library cannot be built")


def _compile(src: Path) -> Path:
    obj = BUILD / (src.name + ".o")
    cmd = [_hipcc(), *COMMON_FLAGS]
    if src.suffix == ".hip":
        cmd += ["-x", "hip", *DEVICE_FLAGS]
    cmd += ["-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    warn = (proc.stderr or "").strip()
    if warn:
        # hipcc's host pass does not know the packed-fp32 feature name; drop that note.
        lines = [l for l in warn.splitlines() if "packed-fp32-ops" not in l and l.strip()]
        if lines:
            print("\n".join(lines), file=sys.stderr)
    return obj


# ONNX Runtime headers for the QcQuantizeOp plugin (librxmet_ort_ops.so): $RXMET_ORT_INCLUDE, or
# the copy vendored in the reference checkout.  The plugin is built only where they exist.
ORT_INCLUDE_DEFAULT = "/root/reference/docker/environment/third_party/onnxruntime/include"
ORT_LIB = PKG / "librxmet_ort_ops.so"


def ort_include() -> Path | None:
    cand = Path(os.environ.get("RXMET_ORT_INCLUDE", ORT_INCLUDE_DEFAULT))
    return cand if (cand / "onnxruntime_lite_custom_op.h").is_file() else None


def build_ort_ops(verbose: bool = True) -> Path | None:
    """The ONNX Runtime plugin over librxmet.so (host code only, g++), when ORT's headers are
    available; returns its path or None."""
    inc = ort_include()
    if inc is None:
        if verbose:
            print("ONNX Runtime headers not found; librxmet_ort_ops.so not rebuilt")
        return None
    tmp = ORT_LIB.with_suffix(".so.tmp")
    cmd = [shutil.which("g++") or "g++", "-std=c++17", "-O2", "-fPIC", "-shared", "-Wall",
           f"-I{inc}", f"-I{ROOT / 'include'}", "-o", str(tmp),
           str(PKG / "ort" / "qc_quantize_op.cpp"), f"-L{PKG}", "-lrxmet",
           "-Wl,-rpath,$ORIGIN", "-Wl,--no-undefined"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"ORT plugin build failed: {' '.join(cmd)}\n{proc.stdout}\n"
                           f"{proc.stderr}")
    os.replace(tmp, ORT_LIB)
    if verbose:
        print(f"built {ORT_LIB}")
    return ORT_LIB


def build(verbose: bool = True) -> Path:
    BUILD.mkdir(exist_ok=True)
    sources = sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))
    if not sources:
        raise RuntimeError(f"no sources in {CSRC}")
    jobs = min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs),
           "-Wl,--no-undefined"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(sources)} sources")
    build_ort_ops(verbose)
    return LIB


if __name__ == "__main__":
    build()
