"""Build recipe for the HIP codec library (gfx950).

The library keeps the reference's file name, ``libunchain_kv_splitzip_cuda.so``,
so the ``UNCHAIN_KV_SPLITZIP_LIB`` override and the loader search path work the
same way (src/unchain_kv/splitzip_cuda.py:34-43). It is built in-tree, into
``unchainkv_amd/lib/``.
"""

from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
CSRC = PACKAGE / "csrc"
LIB_DIR = PACKAGE / "lib"
LIB_NAME = "libunchain_kv_splitzip_cuda.so"
LIB_PATH = LIB_DIR / LIB_NAME
SOURCES = ("splitzip_top16.hip", "splitzip_fixed6.hip", "splitzip_histogram.hip",
           "splitzip_attention.hip", "splitzip_writeback.hip", "splitzip_torchop.hip")

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # no packed fp32 instructions are generated (v_pk_{add,mul,fma}_f32)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    return found


def sources() -> list[Path]:
    return [CSRC / name for name in SOURCES if (CSRC / name).exists()]


def build_library(verbose: bool = False) -> Path:
    """Compile every HIP source into the shared library (always recompiles)."""
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIPCC_FLAGS, "-o", str(tmp), *map(str, sources())]
    env = dict(os.environ)
    result = subprocess.run(cmd, capture_output=True, text=True, env=env)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed ({result.returncode}):\n{result.stderr[-4000:]}")
    if verbose and result.stderr.strip():
        print(result.stderr)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH
