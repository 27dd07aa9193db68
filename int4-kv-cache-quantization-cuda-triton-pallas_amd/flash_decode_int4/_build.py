"""In-tree build of the native parts of flash_decode_int4.

Two artefacts are written next to this file:

  libfdi4.so   the HIP kernels for gfx950 and the C ABI of include/fdi4.h
               (hipcc, -O3, no fast-math, -ffp-contract=off so the quantizer
               and dequantizer arithmetic is one IEEE float32 operation per
               source operation)
  _C.so        the thin PyTorch binding (csrc/binding.cpp): host code only,
               linked against libfdi4.so with an $ORIGIN runpath

Run ``python -m flash_decode_int4._build`` (or ``__graft_entry__.build()``).
Nothing is compiled at import time; the package raises if the libraries are
missing.
"""

import os
import subprocess
import sys
import sysconfig

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(ROOT_DIR, "csrc")
INCLUDE = os.path.join(os.path.dirname(ROOT_DIR), "include")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

HIP_SOURCES = ("quantize.hip", "decode.hip", "decode_gqa.hip", "decode_mfma.hip", "fake_quant.hip",
               "capi.hip")
LIB_PATH = os.path.join(PKG_DIR, "libfdi4.so")
EXT_PATH = os.path.join(PKG_DIR, "_C.so")

HIPCC_FLAGS = [
    "-O3",
    "--offload-arch=gfx950",
    "-mcode-object-version=5",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    # Packed fp32 instructions are not emitted (they are not used on purpose).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-result",
]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(line for line in res.stdout.splitlines()
                    if "packed-fp32-ops" not in line)
    if res.returncode != 0:
        raise RuntimeError(f"build step failed ({res.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out, flush=True)


def build_library(verbose=False):
    """One hipcc per source in parallel (each object carries its own gfx950
    code object), then one link."""
    import tempfile
    from concurrent.futures import ThreadPoolExecutor
    hipcc = os.path.join(ROCM, "bin", "hipcc")
    with tempfile.TemporaryDirectory(prefix="fdi4_build_") as tmpdir:
        objs = []
        cmds = []
        for src in HIP_SOURCES:
            obj = os.path.join(tmpdir, src + ".o")
            objs.append(obj)
            cmds.append([hipcc, *HIPCC_FLAGS, "-I", INCLUDE, "-c", os.path.join(CSRC, src),
                         "-o", obj])
        workers = max(1, min(len(cmds), os.cpu_count() or 1))
        with ThreadPoolExecutor(max_workers=workers) as pool:
            for fut in [pool.submit(_run, c, verbose) for c in cmds]:
                fut.result()
        tmp = LIB_PATH + ".tmp"
        _run([hipcc, "-shared", "-fPIC", "--offload-arch=gfx950", *objs, "-o", tmp], verbose)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def build_binding(verbose=False):
    import torch
    import torch.utils.cpp_extension as ce

    incs = list(ce.include_paths()) + [sysconfig.get_paths()["include"],
                                        os.path.join(ROCM, "include"), INCLUDE]
    libdirs = list(ce.library_paths())
    abi = int(bool(torch._C._GLIBCXX_USE_CXX11_ABI))
    tmp = EXT_PATH + ".tmp"
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-w",
           "-DTORCH_EXTENSION_NAME=_C", "-DTORCH_API_INCLUDE_EXTENSION_H",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           *[f"-I{p}" for p in incs],
           os.path.join(CSRC, "binding.cpp"), "-o", tmp,
           *[f"-L{p}" for p in libdirs],
           f"-L{PKG_DIR}", "-lfdi4",
           "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-ltorch_python",
           "-Wl,-rpath,$ORIGIN"]
    _run(cmd, verbose)
    os.replace(tmp, EXT_PATH)
    return EXT_PATH


def build(verbose=False):
    """Compile libfdi4.so then _C.so (always recompiles)."""
    build_library(verbose)
    build_binding(verbose)


if __name__ == "__main__":
    build(verbose="-q" not in sys.argv)
