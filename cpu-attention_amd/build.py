"""Builds the gfx950 kernel library the Python package loads through ctypes.

    python cpu-attention_amd/build.py [--jobs N] [--verbose]

Each ``csrc/*.hip`` file is compiled by hipcc for gfx950 only, in parallel, and the
objects are linked into ``cpu_attention/libcpu_attention_hip.so`` next to the
Python package, so the library travels with the source tree.  Objects go to
``_build/`` beside this file.  Packed-fp32 instructions are disabled for every
device compile.

Beside it, ``csrc/ca_binding.cpp`` (host code only: the decode/store/flash
argument handling, against torch's C++ headers) becomes the CPython extension
``cpu_attention/_binding<EXT_SUFFIX>``, built by the host compiler.
"""

import argparse
import concurrent.futures
import os
import shutil
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "cpu_attention", "libcpu_attention_hip.so")
ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature flag; that warning is noise.
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{err}")
    if err.strip() and verbose:
        print(err, file=sys.stderr)


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def binding_command(out):
    """The host-compiler line that builds the ``_binding`` extension into ``out``."""
    import torch
    from torch.utils import cpp_extension

    cxx = os.environ.get("CXX", shutil.which("g++") or "g++")
    incs = [*cpp_extension.include_paths(), sysconfig.get_paths()["include"],
            os.path.join(os.path.dirname(HERE), "include")]
    libdir = cpp_extension.library_paths()[0]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    return [cxx, "-O2", "-std=c++17", "-shared", "-fPIC", "-Wall", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
            *[f"-I{i}" for i in incs], os.path.join(CSRC, "ca_binding.cpp"), "-o", out,
            f"-L{libdir}", "-lc10", "-ltorch_cpu", "-ltorch_python", f"-Wl,-rpath,{libdir}"]


def binding_path():
    return os.path.join(HERE, "cpu_attention", "_binding" + sysconfig.get_config_var("EXT_SUFFIX"))


def build(jobs=None, verbose=False):
    """Compile every kernel source and link the shared library, and build the
    ``_binding`` extension; returns the library's path."""
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    objs = [os.path.join(BUILD, os.path.basename(s)[:-4] + ".o") for s in srcs]
    jobs = jobs or min(len(srcs) + 1, max(1, (os.cpu_count() or 1)))
    ext = binding_path()
    with concurrent.futures.ThreadPoolExecutor(jobs) as pool:
        futs = [pool.submit(_run, [HIPCC, *FLAGS, "-c", s, "-o", o], verbose)
                for s, o in zip(srcs, objs)]
        futs.append(pool.submit(_run, binding_command(ext + ".tmp"), verbose))
        for f in futs:
            f.result()
    os.replace(ext + ".tmp", ext)
    tmp = LIB + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp], verbose)
    os.replace(tmp, LIB)
    return LIB


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--verbose", action="store_true")
    args = ap.parse_args()
    print(build(args.jobs, args.verbose))


if __name__ == "__main__":
    main()
