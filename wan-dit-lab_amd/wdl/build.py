"""Builds the C-ABI library lib/libwdl.so from csrc/*.hip with hipcc for gfx950 only.

Each source compiles to its own object in parallel (`hipcc -c`), then one `hipcc -shared` link. Flags:
- `-ffp-contract=off`: no implicit fused multiply-adds, so every kernel rounds exactly as its source is written
  (fmaf where a fused multiply-add is meant);
- `-Xclang -target-feature -Xclang -packed-fp32-ops`: no packed FP32 VALU instructions are generated;
- `-munsafe-fp-atomics` is NOT used: the library has no floating-point atomics.

Run as `python -m wdl.build` from the package root, or call build().
"""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]  # wan-dit-lab_amd/
CSRC = ROOT / "csrc"
OBJ = ROOT / "_build"
LIB = ROOT / "lib" / "libwdl.so"
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form",  # MFMA results in VGPRs: no accvgpr read-backs before VALU use
    "-Wno-unused-command-line-argument",
]


def _hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if candidate and (Path(candidate).exists() or candidate == "hipcc"):
            return candidate
    raise FileNotFoundError("hipcc not found")


def _compile(src: Path) -> Path:
    obj = OBJ / (src.stem + ".o")
    deps = [src, *CSRC.glob("*.h")]
    if obj.exists() and all(obj.stat().st_mtime >= d.stat().st_mtime for d in deps):
        return obj
    cmd = [_hipcc(), *FLAGS, "-I", str(CSRC), "-c", str(src), "-o", str(obj)]
    run = subprocess.run(cmd, capture_output=True, text=True)
    if run.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{run.stdout}\n{run.stderr}")
    return obj


def build(force: bool = False, jobs: int | None = None) -> Path:
    """Compiles every csrc/*.hip and links lib/libwdl.so; returns its path."""
    OBJ.mkdir(exist_ok=True)
    LIB.parent.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if force:
        for o in OBJ.glob("*.o"):
            o.unlink()
    jobs = jobs or min(8, len(sources)) or 1
    with ThreadPoolExecutor(jobs) as pool:
        objs = list(pool.map(_compile, sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    run = subprocess.run(cmd, capture_output=True, text=True)
    if run.returncode != 0:
        raise RuntimeError(f"link failed:\n{run.stdout}\n{run.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(force="--force" in sys.argv))
