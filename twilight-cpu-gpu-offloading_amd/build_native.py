"""Build the native libraries of the package in-tree.

* ``headinfer/_lib/libtwilight_hip.so`` -- every ``csrc/*.hip`` kernel plus the
  C ABI helpers, compiled by hipcc for gfx950 only.
* ``headinfer/_lib/libtwilight_host.so`` -- the host-side natives (OpenMP row
  gather, token union), compiled by g++.

Run ``python build_native.py`` (or ``__graft_entry__.build()``).  Objects go to
``_build/`` next to this file; the libraries are renamed into place only after
a successful link.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent
CSRC = ROOT / "csrc"
LIB_DIR = ROOT / "headinfer" / "_lib"
OBJ_DIR = ROOT / "_build"
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
HIP_FLAGS = [
    "-std=c++17",
    "-O3",
    f"--offload-arch={ARCH}",
    "-fPIC",
    "-ffp-contract=off",
    "-fno-gpu-flush-denormals-to-zero",
    # Packed FP32 VALU ops are disabled for the whole library.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    lines = [ln for ln in proc.stdout.splitlines() if "packed-fp32-ops" not in ln and ln.strip()]
    if proc.returncode != 0:
        raise RuntimeError("command failed: " + " ".join(cmd) + "\n" + "\n".join(lines))
    if lines:
        sys.stderr.write("\n".join(lines) + "\n")


def build(verbose: bool = False) -> dict[str, Path]:
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    OBJ_DIR.mkdir(parents=True, exist_ok=True)
    hip_sources = sorted(CSRC.glob("*.hip"))
    jobs = []
    for src in hip_sources:
        obj = OBJ_DIR / (src.stem + ".o")
        jobs.append([HIPCC, *HIP_FLAGS, "-c", str(src), "-o", str(obj)])
    capi_obj = OBJ_DIR / "capi.o"
    jobs.append([HIPCC, "-std=c++17", "-O3", "-fPIC", "-Wall", "-c", str(CSRC / "capi.cpp"), "-o", str(capi_obj)])
    workers = min(len(jobs), max(1, (os.cpu_count() or 4)))
    with cf.ThreadPoolExecutor(max_workers=workers) as ex:
        for fut in [ex.submit(_run, j) for j in jobs]:
            fut.result()
    objs = [str(OBJ_DIR / (s.stem + ".o")) for s in hip_sources] + [str(capi_obj)]
    hip_lib = LIB_DIR / "libtwilight_hip.so"
    tmp = hip_lib.with_suffix(".so.tmp")
    _run([HIPCC, "-shared", f"--offload-arch={ARCH}", "-o", str(tmp), *objs])
    os.replace(tmp, hip_lib)

    host_lib = LIB_DIR / "libtwilight_host.so"
    tmp = host_lib.with_suffix(".so.tmp")
    _run(["g++", "-std=c++17", "-O3", "-fopenmp", "-fPIC", "-shared", "-Wall", str(CSRC / "host_gather.cpp"), "-o",
          str(tmp)])
    os.replace(tmp, host_lib)
    if verbose:
        print(f"built {hip_lib} and {host_lib}")
    return {"hip": hip_lib, "host": host_lib}


def clean() -> None:
    shutil.rmtree(OBJ_DIR, ignore_errors=True)


if __name__ == "__main__":
    build(verbose=True)
