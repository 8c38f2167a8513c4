"""Builds libcastforge_hip.so in-tree with hipcc for gfx950.

Every HIP source under csrc/ is compiled to an object in castforge_amd/_build/ and linked
into castforge_amd/libcastforge_hip.so.  Kernels are written for gfx950 only.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libcastforge_hip.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

COMMON = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    # packed-FP32 VALU forms are kept out of every kernel
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
# Sources whose arithmetic must round exactly like the CPU reference (no a*b+c contraction).
EXACT = {"quantize.hip", "quantize_ref.hip", "elementwise.hip", "rotate.hip"}


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile(src: Path) -> tuple[Path, str]:
    obj = BUILD / (src.stem + ".o")
    flags = list(COMMON)
    if src.name in EXACT:
        flags.append("-ffp-contract=off")
    cmd = [HIPCC, *flags, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj, r.stderr


def build(verbose: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    srcs = sources()
    workers = min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=workers) as ex:
        results = list(ex.map(_compile, srcs))
    if verbose:
        for obj, err in results:
            warn = "\n".join(l for l in err.splitlines() if "packed-fp32-ops" not in l and l.strip())
            if warn:
                print(f"[{obj.name}] {warn}", file=sys.stderr)
    tmp = LIB.with_suffix(".so.tmp")
    # --no-undefined: a kernel whose host stub the compiler failed to emit fails here, not at load
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,--no-undefined", "-o", str(tmp),
           *[str(o) for o, _ in results]]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
