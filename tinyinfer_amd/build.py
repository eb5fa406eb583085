"""In-tree build of the MI355X (gfx950) MXFP4 library and its torch wrapper.

Two artefacts, both inside the package directory so they travel with the
source tree:

* ``libtinyinfer_mxfp4.so``: every ``csrc/*.hip`` file compiled by hipcc
  for gfx950 and linked as a shared library exporting the C ABI declared in
  ``include/tinyinfer_mxfp4.h``.
* ``_C.<abi>.so``: the pybind11/torch extension (``csrc/bind.cpp``) that
  links the library above (rpath ``$ORIGIN``); built by ``setup.py``.

``python -m tinyinfer_amd.build`` builds both.
"""

from __future__ import annotations

import glob
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
LIB_NAME = "libtinyinfer_mxfp4.so"
LIB_PATH = os.path.join(PKG, LIB_NAME)
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # Packed FP32 (v_pk_*_f32) code generation off for all device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found; a ROCm toolchain is required to build tinyinfer_amd")


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in proc.stdout.splitlines()
                    if "packed-fp32-ops' is not a recognized feature" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


def build_hip_library(verbose: bool = True) -> str:
    """Compile csrc/*.hip with hipcc for gfx950 and link the C-ABI library."""
    os.makedirs(BUILD, exist_ok=True)
    sources = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    if not sources:
        raise RuntimeError("no HIP sources found")
    cc = hipcc()
    objs = [os.path.join(BUILD, os.path.basename(s) + ".o") for s in sources]

    def compile_one(pair):
        src, obj = pair
        _run([cc, *HIPCC_FLAGS, "-I", os.path.join(ROOT, "include"), "-c", src, "-o", obj])
        return obj

    jobs = min(len(sources), int(os.environ.get("MAX_JOBS", "8")))
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        list(ex.map(compile_one, zip(sources, objs)))
    tmp = LIB_PATH + ".tmp"
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}", file=sys.stderr)
    return LIB_PATH


def build_torch_extension() -> None:
    """Build tinyinfer_amd._C in place via setup.py (links the HIP library)."""
    env = dict(os.environ, TINYINFER_SKIP_HIP_LIB="1")
    proc = subprocess.run([sys.executable, os.path.join(ROOT, "setup.py"), "build_ext", "--inplace"],
                          cwd=ROOT, env=env, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"torch extension build failed:\n{proc.stdout[-4000:]}")


def build_all() -> None:
    build_hip_library()
    build_torch_extension()


if __name__ == "__main__":
    build_all()
