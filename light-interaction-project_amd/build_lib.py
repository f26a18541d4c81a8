"""Build libli_sparse_attn.so (gfx950) in-tree with hipcc.

Usage: python light-interaction-project_amd/build_lib.py [--jobs N]

Compiles every ``csrc/*.hip`` to an object under ``_build/`` and links the
shared library into ``li_sparse/libli_sparse_attn.so`` next to the Python
package that loads it, then builds the torch operator layer
``li_sparse/libli_torch_ops.so`` from ``csrc/li_torch_ops.cpp`` (host-only
C++, linked against the HIP library and torch).
"""
import argparse
import concurrent.futures
import hashlib
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
OUT = os.path.join(HERE, "li_sparse", "libli_sparse_attn.so")
# Hash of the sources and flags the library was built from, written next to it.
STAMP = OUT + ".stamp"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    "-I", os.path.join(REPO, "include"), "-I", CSRC,
    # code object v5 loads in every ROCm 7.x runtime, including the one torch ships
    "-mcode-object-version=5",
    # packed fp32 VALU ops stay disabled for all device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def source_hash():
    """sha256 over the HIP and C++ sources, the C header and the compile flags."""
    h = hashlib.sha256(" ".join(CFLAGS).encode())
    inc = os.path.join(REPO, "include")
    files = [os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith((".hip", ".hpp", ".h", ".cpp"))]
    files += [os.path.join(inc, f) for f in os.listdir(inc) if f.endswith(".h")]
    for path in sorted(files):
        h.update(os.path.relpath(path, REPO).encode())
        with open(path, "rb") as f:
            h.update(f.read())
    return h.hexdigest()


def is_current():
    """Whether both built libraries exist and were built from the current sources."""
    try:
        with open(STAMP) as f:
            return os.path.exists(OUT) and os.path.exists(OPS_OUT) and f.read().strip() == source_hash()
    except OSError:
        return False


def _compile(src):
    obj = os.path.join(BUILD, os.path.splitext(os.path.basename(src))[0] + ".o")
    cmd = [HIPCC] + CFLAGS + ["-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    return obj


OPS_SRC = os.path.join(CSRC, "li_torch_ops.cpp")
OPS_OUT = os.path.join(HERE, "li_sparse", "libli_torch_ops.so")


def build_ops(verbose=True):
    """The torch.ops.li operator library: host-only C++ (g++) over the C ABI, linked against the HIP library."""
    import torch
    from torch.utils import cpp_extension

    inc = sum((["-I", p] for p in cpp_extension.include_paths()), [])
    libdir = cpp_extension.library_paths()[0]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    tmp = OPS_OUT + ".tmp"
    cmd = [os.environ.get("CXX", "g++"), "-O2", "-fPIC", "-shared", "-std=c++17", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           "-DUSE_ROCM=1", "-D__HIP_PLATFORM_AMD__=1", "-I", os.path.join(REPO, "include"), *inc,
           "-I", "/opt/rocm/include", OPS_SRC, "-o", tmp,
           "-L", os.path.dirname(OUT), "-lli_sparse_attn", "-L", libdir, "-lc10", "-lc10_hip", "-ltorch",
           "-ltorch_cpu", "-ltorch_hip", "-Wl,-rpath,$ORIGIN"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"g++ failed for {OPS_SRC}:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, OPS_OUT)
    if verbose:
        print(f"built {OPS_OUT}")
    return OPS_OUT


def build(jobs=4, verbose=True):
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = OUT + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT}")
    build_ops(verbose)
    with open(STAMP, "w") as f:
        f.write(source_hash() + "\n")
    return OUT


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=4)
    args = ap.parse_args()
    try:
        build(args.jobs)
    except RuntimeError as e:
        print(e, file=sys.stderr)
        sys.exit(1)
