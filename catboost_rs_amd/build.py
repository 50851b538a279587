"""Build the gfx950 training library ``catboost_rs_amd/libcbhip.so`` with hipcc.

Every source under ``csrc/`` is compiled for gfx950 only (no other target, no CUDA path)
and linked into one shared library exporting the C-ABI of ``include/cbhip.h`` and
``include/cbtrain.h``.

    python -m catboost_rs_amd.build          # or: python catboost_rs_amd/build.py
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
OUT = os.path.join(HERE, "libcbhip.so")
OBJ_DIR = os.path.join(HERE, "_build")

SOURCES = ["session.hip", "entry.hip", "apply.hip", "borders.hip", "categorical.hip", "driver.cpp"]

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

# -ffp-contract=off: keep every rounding step of the reference's arithmetic (no fused
# multiply-add); the packed-fp32 feature is disabled for all device code.
COMMON = ["-O3", "-fPIC", "-std=c++17", "-ffp-contract=off", "-Wall", "-Wno-unused-function",
          "-I", os.path.join(ROOT, "include")]
DEVICE = ["--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _compile(src: str) -> str:
    obj = os.path.join(OBJ_DIR, os.path.basename(src) + ".o")
    cmd = [HIPCC, "-x", "hip"] + DEVICE + COMMON + ["-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    if r.stderr.strip():
        msgs = [l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l and "not a recognized feature" not in l]
        if any(m.strip() for m in msgs):
            sys.stderr.write("\n".join(msgs) + "\n")
    return obj


RATE_SRC = os.path.join(CSRC, "lds_atomic_rate.hip")
RATE_BIN = os.path.join(HERE, "lds_atomic_rate")


def build_rate_probe() -> str:
    """The LDS atomic-rate probe bench.py runs to report the fill's LDS-atomic roofline."""
    cmd = [HIPCC, "-x", "hip"] + DEVICE + ["-O3", "-std=c++17", RATE_SRC, "-o", RATE_BIN + ".tmp"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for lds_atomic_rate.hip:\n{r.stdout}\n{r.stderr}")
    os.replace(RATE_BIN + ".tmp", RATE_BIN)
    return RATE_BIN


def build(verbose: bool = True) -> str:
    os.makedirs(OBJ_DIR, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(len(SOURCES), 8)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = OUT + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, OUT)
    build_rate_probe()
    if verbose:
        print(f"built {OUT}")
    return OUT


if __name__ == "__main__":
    build()
