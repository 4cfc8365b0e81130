"""Builds newch_amd/libnc.so: the nc.h engine plus the nc_hip.h kernel layer, for gfx950.

    python -m newch_amd.build          # compile everything (always recompiles)

The .hip files go through hipcc and carry device code for gfx950 only; the
engine's .cpp files are host code against the HIP runtime, compiled by g++.  Device code is compiled with
-ffp-contract=off (fused multiply-adds only where written) and with packed-fp32 instructions
disabled.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = ROOT / "_build" / "newch_amd"
LIB = PKG / "libnc.so"
ARCH = "gfx950"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm 7.x is required to build newch_amd)")


COMMON = ["-O3", "-std=c++17", "-fPIC", "-fvisibility=hidden", "-Wall", "-Wno-unused-function",
          f"-I{ROOT / 'include'}", f"-I{CSRC / 'kernels'}", f"-I{CSRC / 'engine'}"]
DEVICE = [f"--offload-arch={ARCH}", "-ffp-contract=off", "-Xclang", "-target-feature", "-Xclang",
          "-packed-fp32-ops"]


def sources() -> list[Path]:
    return sorted(CSRC.glob("kernels/*.hip")) + sorted(CSRC.glob("engine/*.cpp"))


def _compile(src: Path) -> Path:
    obj = BUILD / (src.parent.name + "_" + src.stem + ".o")
    if src.suffix == ".hip":
        cmd = [hipcc(), *COMMON, *DEVICE, "-x", "hip"]
    else:  # host-only engine code against the HIP runtime API
        cmd = ["g++", *COMMON, "-D__HIP_PLATFORM_AMD__", f"-I{ROCM / 'include'}"]
    cmd += ["-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(line for line in (res.stdout + res.stderr).splitlines()
                    if "packed-fp32-ops" not in line and line.strip())
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {src.name}\n{' '.join(cmd)}\n{out}")
    if out:
        print(out, file=sys.stderr)
    return obj


def build(verbose: bool = True) -> Path:
    BUILD.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    jobs = min(len(srcs), max(1, min(os.cpu_count() or 4, 16)))
    with ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs),
           "-Wl,-soname,libnc.so"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed\n{' '.join(cmd)}\n{res.stdout}{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} ({LIB.stat().st_size // 1024} KiB, {len(objs)} objects)")
    return LIB


if __name__ == "__main__":
    build()
