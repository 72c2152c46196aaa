"""Build recipe for the gfx950 paged-attention library.

Outputs (next to this file, in lib/):
  lib/*.hsaco        gfx950 code objects, one per csrc/kernels/*.hip
                     (hipcc --genco), loaded at run time with hipModuleLoad
  lib/liblucattn.so  the C-ABI host library (include/luc_attn.h), g++ against
                     the HIP runtime; it launches the kernels above

Run `python lucciola-rs_amd/build.py` or call build().  hipcc cross-compiles
for gfx950 without a GPU.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
KDIR = os.path.join(CSRC, "kernels")
LIB = os.path.join(HERE, "lib")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
ARCH = "gfx950"

KERNELS = ["rope_append", "paged_decode", "paged_decode_w8", "paged_prefill", "model_ops", "sampling",
           "probe_gather"]
# code objects built from another object's source with extra flags
KERNEL_SOURCES = {"paged_decode_w8": ("paged_decode", ["-DLUC_DECODE_WIDE"])}

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "--genco", "--no-gpu-bundle-output",
    "-mcode-object-version=5", "-std=c++17",
    # no packed-FP32 instructions (v_pk_{add,mul,fma}_f32)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
# per code object: the prefill kernels keep their MFMA results in ordinary
# VGPRs (the scores go straight to the VALU; the two-heads-per-wave kernels
# hold their K and V operands in AGPRs, read by the MFMAs directly)
KERNEL_FLAGS = {"paged_prefill": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _run(cmd, verbose):
    if verbose:
        print("+", " ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"build step failed ({res.returncode}): {' '.join(cmd)}")
    return res


def build_kernel(name, verbose=False):
    base, defs = KERNEL_SOURCES.get(name, (name, []))
    src = os.path.join(KDIR, base + ".hip")
    out = os.path.join(LIB, name + ".hsaco")
    tmp = out + ".tmp"
    _run([os.path.join(ROCM, "bin", "hipcc"), *HIPCC_FLAGS, *KERNEL_FLAGS.get(name, []), *defs, "-I", KDIR,
          src, "-o", tmp], verbose)
    os.replace(tmp, out)
    return out


def build_scratch_object(verbose=False):
    """luc_scratch.hip: the library's fixed device scratch (a __device__ array
    registered with the HIP runtime) and its set-up, as a relocatable object."""
    out = os.path.join(LIB, "luc_scratch.o")
    tmp = out + ".tmp"
    _run([os.path.join(ROCM, "bin", "hipcc"), f"--offload-arch={ARCH}", "-O2", "-std=c++17",
          "-fPIC", "-c", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-I", os.path.join(ROOT, "include"), os.path.join(CSRC, "luc_scratch.hip"), "-o", tmp],
         verbose)
    os.replace(tmp, out)
    return out


def build_host(verbose=False):
    scratch = build_scratch_object(verbose)
    out = os.path.join(LIB, "liblucattn.so")
    tmp = out + ".tmp"
    _run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wextra",
          "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(ROCM, "include"),
          "-I", os.path.join(ROOT, "include"), os.path.join(CSRC, "luc_attn.cpp"),
          os.path.join(CSRC, "luc_blocks.cpp"), scratch,
          "-L", os.path.join(ROCM, "lib"), "-lamdhip64", f"-Wl,-rpath,{ROCM}/lib",
          "-o", tmp], verbose)
    os.replace(tmp, out)
    return out


def build(verbose=False):
    os.makedirs(LIB, exist_ok=True)
    with ThreadPoolExecutor(max_workers=len(KERNELS) + 1) as ex:
        futs = [ex.submit(build_kernel, k, verbose) for k in KERNELS]
        futs.append(ex.submit(build_host, verbose))
        return [f.result() for f in futs]


if __name__ == "__main__":
    for p in build(verbose=True):
        print(p)
