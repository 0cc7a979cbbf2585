"""Build recipe for libanelm_hip.so (gfx950) and the C++ drop-in test driver.

Run as ``python ane-lm_amd/build.py`` or through ``__graft_entry__.build()``.
Every HIP source is compiled for gfx950 only, with hipcc's correctly rounded
fp32 divide/sqrt (the default), IEEE subnormals, no fast-math, and packed
fp32 instructions disabled in device code.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
INCLUDE = os.path.join(ROOT, "include")
CSRC = os.path.join(PKG, "csrc")
HOST = os.path.join(PKG, "host")
BUILD = os.path.join(PKG, "_build")
LIBDIR = os.path.join(PKG, "lib")
LIB = os.path.join(LIBDIR, "libanelm_hip.so")

SOURCES = [
    os.path.join(CSRC, "status.hip"),
    os.path.join(CSRC, "norm.hip"),
    os.path.join(CSRC, "layer.hip"),
    os.path.join(CSRC, "elementwise.hip"),
    os.path.join(CSRC, "sampling.hip"),
    os.path.join(CSRC, "attention.hip"),
    os.path.join(CSRC, "deltanet.hip"),
    os.path.join(CSRC, "projection.hip"),
    os.path.join(HOST, "dropin.hip"),
    os.path.join(HOST, "safetensors.hip"),
    os.path.join(HOST, "qwen3.hip"),
]

ARCH = "gfx950"


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = os.path.join(rocm, "bin", "hipcc")
    if not os.path.exists(path):
        path = shutil.which("hipcc") or path
    return path


COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    # packed fp32 (v_pk_*_f32) off in device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", INCLUDE,
    "-I", CSRC,
    "-I", HOST,
]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass warns about the device-only target feature: harmless
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l and "not a recognized feature" not in l)
    if r.returncode != 0:
        sys.stderr.write(out + "\n")
        raise RuntimeError("command failed: " + " ".join(cmd))
    if out.strip():
        sys.stderr.write(out + "\n")


def build_lib(jobs: int = 8) -> str:
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    cc = hipcc()
    objs = []
    cmds = []
    for src in SOURCES:
        obj = os.path.join(BUILD, os.path.basename(src) + ".o")
        objs.append(obj)
        cmds.append([cc, *COMMON_FLAGS, "-c", src, "-o", obj])
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_run, cmds))
    tmp = LIB + ".tmp"
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, LIB)
    return LIB


def build_oracle() -> str:
    """Compile the CPU oracle (test infrastructure) with its own Makefile."""
    oracle = os.path.join(ROOT, "oracle")
    _run(["make", "-s", "-C", oracle])
    if os.path.isdir("/root/reference"):
        _run(["make", "-s", "-C", oracle, "ref"])
    return os.path.join(oracle, "liboracle.so")


def build_dropin_check() -> str:
    """C++ driver that calls the ane_lm:: drop-in functions against the oracle."""
    src = os.path.join(ROOT, "tests", "cpp", "dropin_check.cpp")
    out = os.path.join(ROOT, "tests", "cpp", "dropin_check")
    oracle = os.path.join(ROOT, "oracle")
    tmp = out + ".tmp"
    _run([hipcc(), "-O2", "-std=c++17", "-I", INCLUDE, "-I", HOST, "-I", oracle, src, "-o", tmp,
          "-L", LIBDIR, "-lanelm_hip", "-L", oracle, "-loracle",
          "-Wl,-rpath,$ORIGIN/../../ane-lm_amd/lib", "-Wl,-rpath,$ORIGIN/../../oracle"])
    os.replace(tmp, out)
    return out


def check_integration_doc() -> None:
    """Compile every call INTEGRATION.md documents against the headers."""
    cpp = os.path.join(ROOT, "tests", "cpp")
    if not os.path.exists(os.path.join(cpp, "integration_doc.py")):
        return
    sys.path.insert(0, cpp)
    try:
        import integration_doc
    finally:
        sys.path.remove(cpp)
    integration_doc.check()


def build_all() -> None:
    build_oracle()
    build_lib()
    if os.path.exists(os.path.join(ROOT, "tests", "cpp", "dropin_check.cpp")):
        build_dropin_check()
    check_integration_doc()


if __name__ == "__main__":
    build_all()
    print("built", LIB)
