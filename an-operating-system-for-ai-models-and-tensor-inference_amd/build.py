"""Build libmyos_hip.so (gfx950) in-tree with hipcc.

Each source compiles to an object in parallel, then one shared library is
linked into <package>/_build/. Packed-FP32 instructions are disabled for the
device code (-target-feature -packed-fp32-ops).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG, "csrc")
OUT = os.path.join(PKG, "_build")
LIB = os.path.join(OUT, "libmyos_hip.so")
ARCH = os.environ.get("MYOS_OFFLOAD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

SOURCES = ["myos_kernels.hip", "myos_persistent.hip", "myos_noalloc.hip", "myos_ops.cpp", "myos_model.cpp",
           "myos_safetensors.cpp",
           "myos_gen.cpp", "myos_sha256.cpp"]
CLI_SOURCES = ["myos_cli.cpp", "myos_arena.cpp"]

COMMON = ["-O3", "-std=c++17", "-fPIC", "-Wall", f"--offload-arch={ARCH}",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _compile(src: str) -> str:
    obj = os.path.join(OUT, os.path.basename(src) + ".o")
    cmd = [HIPCC, *COMMON, "-c", os.path.join(CSRC, src), "-o", obj + ".tmp"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")
    os.replace(obj + ".tmp", obj)
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(OUT, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
        objs = list(ex.map(_compile, SOURCES))
        cli_objs = list(ex.map(_compile, CLI_SOURCES)) if all(
            os.path.exists(os.path.join(CSRC, s)) for s in CLI_SOURCES) else []
    tmp = LIB + ".tmp"
    subprocess.run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-o", tmp, *objs, "-lpthread"],
                   check=True)
    os.replace(tmp, LIB)
    if cli_objs:
        exe = os.path.join(OUT, "myos")
        subprocess.run([HIPCC, f"--offload-arch={ARCH}", "-o", exe + ".tmp", *cli_objs, *objs,
                        "-lpthread"], check=True)
        os.replace(exe + ".tmp", exe)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
