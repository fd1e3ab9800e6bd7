"""Build recipe of the HIP backend: ``lucid_amd/_lib/liblucid_amd.so`` for gfx950.

Run ``python -m lucid_amd.build``.  Every ``csrc/*.hip`` file is compiled with
hipcc for gfx950 and linked into one shared library exporting the C ABI of
``include/lq_api.h``.

Flags that carry numerics:

* ``-ffp-contract=off``: no FMA contraction, so every float expression is the single
  IEEE operation it spells (Lucid's CPU path runs one op per pass; a fused multiply-add
  would round differently).
* ``-fhip-fp32-correctly-rounded-divide-sqrt``: ``1.0f / s`` is the IEEE division
  Lucid's tensor reciprocal performs.
* ``-Xclang -target-feature -Xclang -packed-fp32-ops``: keep packed fp32 instructions out
  of every kernel (the host pass warns that it does not know the feature; harmless).
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
OUT_DIR = os.path.join(HERE, "_lib")
LIB_NAME = "liblucid_amd.so"
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def lib_path() -> str:
    return os.path.join(OUT_DIR, LIB_NAME)


def _compile(src: str, obj_dir: str) -> str:
    obj = os.path.join(obj_dir, os.path.basename(src)[:-4] + ".o")
    cmd = [HIPCC, *COMMON_FLAGS, "-c", src, "-o", obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # The host pass warns about the packed-fp32 feature it does not know; keep the rest.
    noise = "is not a recognized feature for this target"
    errs = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{errs}")
    if errs.strip():
        sys.stderr.write(errs + "\n")
    return obj


def build(verbose: bool = True) -> str:
    """Compile every HIP source and link the shared library; returns its path."""
    if not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    obj_dir = os.path.join(HERE, "_build")
    os.makedirs(obj_dir, exist_ok=True)
    os.makedirs(OUT_DIR, exist_ok=True)
    srcs = sources()
    workers = min(len(srcs), 8)
    with cf.ThreadPoolExecutor(max_workers=workers) as ex:
        objs = list(ex.map(lambda s: _compile(s, obj_dir), srcs))
    tmp = lib_path() + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    shutil.move(tmp, lib_path())
    if verbose:
        print(f"built {lib_path()} from {len(srcs)} sources")
    return lib_path()


if __name__ == "__main__":
    build()
