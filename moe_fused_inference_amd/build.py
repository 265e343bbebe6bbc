"""Builds the gfx950 HIP library ``lib/libmxfp4_hip.so`` in-tree with hipcc,
and the compiled torch binding ``lib/mxfp4_ext.so`` on top of it with g++.

Every ``csrc/*.hip`` file is compiled for gfx950 only and linked into one
shared library that exports the C ABI declared in ``include/mxfp4_hip.h``.
Objects are compiled in parallel and cached by source/flag hash under
``csrc/_build``; the link always runs.  ``csrc/torch_binding.cpp`` is host
code only (the pybind module with the reference extensions' surface); it is
linked against the HIP library and torch's libraries.
"""
import hashlib
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
OBJ = os.path.join(CSRC, "_build")
LIBDIR = os.path.join(PKG, "lib")
LIB = os.path.join(LIBDIR, "libmxfp4_hip.so")
EXT = os.path.join(LIBDIR, "mxfp4_ext.so")
INCLUDE = os.path.join(ROOT, "include")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-fno-gpu-flush-denormals-to-zero",
    # packed fp32 (v_pk_*_f32) code generation is disabled for all device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-command-line-argument",
    f"-I{INCLUDE}", f"-I{CSRC}",
]


def _sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _headers_digest():
    h = hashlib.sha1()
    for d in (CSRC, INCLUDE):
        for f in sorted(os.listdir(d)):
            if f.endswith(".h"):
                with open(os.path.join(d, f), "rb") as fh:
                    h.update(fh.read())
    return h.hexdigest()


def _compile(src, hdr, extra, verbose):
    with open(src, "rb") as fh:
        key = hashlib.sha1(fh.read() + hdr.encode() + " ".join(CFLAGS + extra).encode()).hexdigest()[:16]
    obj = os.path.join(OBJ, os.path.basename(src)[:-4] + "." + key + ".o")
    if not os.path.exists(obj):
        cmd = [HIPCC, *CFLAGS, *extra, "-c", src, "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
        warn = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l and l.strip())
        if warn and verbose:
            print(warn, file=sys.stderr)
    return obj


def build(verbose=False, extra=()):
    """Compile and link the library; returns its path."""
    os.makedirs(OBJ, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    hdr = _headers_digest()
    srcs = _sources()
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(lambda s: _compile(s, hdr, list(extra), verbose), srcs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    build_binding(verbose)
    return LIB


def _binding_cmd(out):
    import sysconfig
    import torch
    from torch.utils import cpp_extension
    libs = cpp_extension.library_paths()
    return ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-D__HIP_PLATFORM_AMD__",
            "-DTORCH_API_INCLUDE_EXTENSION_H", "-DTORCH_EXTENSION_NAME=mxfp4_ext",
            f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
            f"-I{INCLUDE}", *[f"-I{p}" for p in cpp_extension.include_paths()],
            f"-I{sysconfig.get_paths()['include']}", "-I/opt/rocm/include",
            os.path.join(CSRC, "torch_binding.cpp"), "-o", out,
            f"-L{LIBDIR}", "-lmxfp4_hip", *[f"-L{p}" for p in libs],
            "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_python",
            "-Wl,-rpath,$ORIGIN", *[f"-Wl,-rpath,{p}" for p in libs]]


def build_binding(verbose=False):
    """Compile the torch binding (cached by source, header and command hash
    under ``csrc/_build``) and place it at ``lib/mxfp4_ext.so``."""
    import shutil
    cmd = _binding_cmd("@OUT@")
    h = hashlib.sha1(" ".join(cmd).encode())
    for f in (os.path.join(CSRC, "torch_binding.cpp"), os.path.join(INCLUDE, "mxfp4_hip.h")):
        with open(f, "rb") as fh:
            h.update(fh.read())
    obj = os.path.join(OBJ, f"mxfp4_ext.{h.hexdigest()[:16]}.so")
    if not os.path.exists(obj):
        cmd = [obj + ".tmp" if c == "@OUT@" else c for c in cmd]
        if verbose:
            print(" ".join(cmd), flush=True)
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"g++ failed for the torch binding:\n{r.stdout}\n{r.stderr}")
        os.replace(obj + ".tmp", obj)
    shutil.copyfile(obj, EXT + ".tmp")
    os.replace(EXT + ".tmp", EXT)
    return EXT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
