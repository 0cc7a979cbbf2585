"""Build recipe for libanelm_hip.so (gfx950) and the C++ drop-in test driver.

Run as ``python ane-lm_amd/build.py`` or through ``__graft_entry__.build()``;
``python ane-lm_amd/build.py --sanitize [pytest args]`` builds the oracle and
the library's host code with AddressSanitizer + UBSan and runs the CPU tests
against that build.
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


def build_dropin_check(name: str = "dropin_check") -> str:
    """C++ driver that calls the ane_lm:: drop-in functions beside the oracle:
    dropin_check compares them, dropin_timing times them."""
    src = os.path.join(ROOT, "tests", "cpp", name + ".cpp")
    out = os.path.join(ROOT, "tests", "cpp", name)
    oracle = os.path.join(ROOT, "oracle")
    tmp = out + ".tmp"
    _run([hipcc(), "-O2", "-std=c++17", "-I", INCLUDE, "-I", HOST, "-I", oracle, src, "-o", tmp,
          "-L", LIBDIR, "-lanelm_hip", "-L", oracle, "-loracle",
          "-Wl,-rpath,$ORIGIN/../../ane-lm_amd/lib", "-Wl,-rpath,$ORIGIN/../../oracle"])
    os.replace(tmp, out)
    return out


def check_integration_doc() -> None:
    """Compile every call the integration guide documents against the headers."""
    cpp = os.path.join(ROOT, "tests", "cpp")
    if not os.path.exists(os.path.join(cpp, "integration_doc.py")):
        return
    sys.path.insert(0, cpp)
    try:
        import integration_doc
    finally:
        sys.path.remove(cpp)
    integration_doc.check()


SAN_DIR = os.path.join(BUILD, "san")
# Host code only: each -fsanitize= follows -Xarch_host, so the device code of
# the sanitizer build is the same as the product's.
SAN_HOST_FLAGS = "-Xarch_host -fsanitize=address -Xarch_host -fsanitize=undefined -Xarch_host -fno-sanitize-recover=undefined".split()


def _rocm_llvm(*parts: str) -> str:
    return os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "llvm", *parts)


def asan_runtime() -> str:
    """clang's shared AddressSanitizer runtime (it carries UBSan's too)."""
    import glob

    found = sorted(glob.glob(_rocm_llvm("lib", "clang", "*", "lib", "*", "libclang_rt.asan-x86_64.so")))
    if not found:
        raise RuntimeError("clang's libclang_rt.asan-x86_64.so not found under " + _rocm_llvm("lib", "clang"))
    return found[-1]


def build_sanitized(jobs: int = 8) -> dict:
    """CPU sanitizer build: the oracle and the library's host code (the
    drop-in staging, the safetensors parser and blob writer, argument
    checks of every entry point) with AddressSanitizer and UBSan, both
    against clang's shared runtime so one process can load the two.
    Outputs go to ane-lm_amd/_build/san/ and are never the product."""
    os.makedirs(SAN_DIR, exist_ok=True)
    oracle_src = os.path.join(ROOT, "oracle", "anelm_oracle.cpp")
    oracle_so = os.path.join(SAN_DIR, "liboracle.so")
    clangxx = _rocm_llvm("bin", "clang++")
    san = ["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined", "-shared-libsan"]
    _run([clangxx, "-O1", "-g", "-fno-omit-frame-pointer", "-ffp-contract=off", "-fopenmp", "-fPIC", "-std=c++17",
          *san, "-shared", "-o", oracle_so, oracle_src, "-Wl,-rpath," + _rocm_llvm("lib")])
    cc = hipcc()
    objs, cmds = [], []
    for src in SOURCES:
        obj = os.path.join(SAN_DIR, os.path.basename(src) + ".o")
        objs.append(obj)
        cmds.append([cc, *COMMON_FLAGS, "-g", "-fno-omit-frame-pointer", *SAN_HOST_FLAGS, "-c", src, "-o", obj])
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_run, cmds))
    lib = os.path.join(SAN_DIR, "libanelm_hip.so")
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-shared-libsan", *SAN_HOST_FLAGS, "-o", lib, *objs])
    return dict(oracle=oracle_so, lib=lib, runtime=asan_runtime())


def run_sanitized_tests(extra: list[str] | None = None) -> int:
    """The CPU test suite (-m "not gpu") against the sanitizer build: the
    runtime preloaded into the interpreter, the two libraries swapped in by
    ANELM_LIB / ANELM_ORACLE_LIB.  Any AddressSanitizer or UBSan report
    aborts the run.  Returns pytest's exit status."""
    b = build_sanitized()
    env = dict(os.environ, LD_PRELOAD=b["runtime"], ANELM_LIB=b["lib"], ANELM_ORACLE_LIB=b["oracle"],
               # leaks of the HIP runtime and torch at exit are not this library's; everything else aborts
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=1:halt_on_error=1:detect_odr_violation=0",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    cmd = [sys.executable, "-m", "pytest", os.path.join(ROOT, "tests"), "-q", "-m", "not gpu", "-p", "no:cacheprovider",
           *(extra or [])]
    return subprocess.run(cmd, env=env, cwd=ROOT).returncode


def build_all() -> None:
    build_oracle()
    build_lib()
    for name in ("dropin_check", "dropin_timing"):
        if os.path.exists(os.path.join(ROOT, "tests", "cpp", name + ".cpp")):
            build_dropin_check(name)
    check_integration_doc()


if __name__ == "__main__":
    if "--sanitize" in sys.argv:
        sys.exit(run_sanitized_tests(sys.argv[sys.argv.index("--sanitize") + 1:]))
    build_all()
    print("built", LIB)
