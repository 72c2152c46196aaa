"""CPU-only AddressSanitizer + UndefinedBehaviorSanitizer build of the host code.

Builds, with g++/gcc and -fsanitize=address,undefined (host code only: no
device code is built here, the gfx950 code objects are not involved):
  _build/san/liblucattn.so      luc_attn.cpp (argument checks, workspace and
                                split policy, RoPE table) + luc_blocks.cpp
                                (the page allocator), linked against the HIP
                                runtime like the product library
  _build/san/libluc_oracle.so   the oracle (oracle/luc_oracle.c)
and then runs the CPU test suite against them:

  python lucciola-rs_amd/sanitize.py [pytest args]   # default: tests -m "not gpu"

The Python interpreter is not instrumented, so the ASan runtime is preloaded
(LD_PRELOAD) and leak checking is off (the interpreter's own allocations are
never freed).  UBSan findings abort the run (-fno-sanitize-recover).  The
libraries are picked up through LUC_LIB_PATH and LUC_ORACLE_LIB.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(ROOT, "_build", "san")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined",
       "-fno-omit-frame-pointer", "-g", "-O1"]


def _run(cmd):
    print("+", " ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)


def build():
    """Build both sanitized libraries into _build/san/."""
    os.makedirs(OUT, exist_ok=True)
    # luc_scratch.o (the device scratch and its set-up) is the product build's
    # own object, by hipcc, linked in uninstrumented
    sys.path.insert(0, HERE)
    import build as product_build
    scratch = product_build.build_scratch_object()
    _run(["g++", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wextra", *SAN,
          "-D__HIP_PLATFORM_AMD__",
          "-I", os.path.join(ROCM, "include"), "-I", os.path.join(ROOT, "include"),
          os.path.join(CSRC, "luc_attn.cpp"), os.path.join(CSRC, "luc_blocks.cpp"), scratch,
          "-L", os.path.join(ROCM, "lib"), "-lamdhip64", f"-Wl,-rpath,{ROCM}/lib",
          "-o", os.path.join(OUT, "liblucattn.so")])
    _run(["gcc", "-std=c11", "-fPIC", "-shared", "-fopenmp", "-ffp-contract=off",
          "-fno-fast-math", "-Wall", "-Wextra", *SAN,
          os.path.join(ROOT, "oracle", "luc_oracle.c"), "-lm",
          "-o", os.path.join(OUT, "libluc_oracle.so")])


def runtime(name):
    return subprocess.run(["gcc", f"-print-file-name={name}"], capture_output=True, text=True,
                          check=True).stdout.strip()


def run_tests(args):
    env = dict(os.environ)
    env["LD_PRELOAD"] = runtime("libasan.so")
    env["ASAN_OPTIONS"] = "detect_leaks=0:abort_on_error=1:halt_on_error=1"
    env["UBSAN_OPTIONS"] = "print_stacktrace=1:halt_on_error=1"
    env["LUC_LIB_PATH"] = os.path.join(OUT, "liblucattn.so")
    env["LUC_ORACLE_LIB"] = os.path.join(OUT, "libluc_oracle.so")
    cmd = [sys.executable, "-m", "pytest", *(args or ["tests", "-q", "-m", "not gpu"])]
    print("+", " ".join(cmd), flush=True)
    return subprocess.run(cmd, cwd=ROOT, env=env).returncode


if __name__ == "__main__":
    build()
    sys.exit(run_tests(sys.argv[1:]))
