"""Build the gfx950 decode library and its PyTorch extension in-tree.

Two artefacts, both next to this package (``mega-kernel_amd/``):
  ``libmegakernel_amd.so``   the HIP kernels (decode, prefill) and their C ABI (``include/megakernel_amd.h``), no torch
  ``megakernel_extension*.so``  the PyTorch operator ``decode`` (reference name, reference signature)
                                linked against the library with an $ORIGIN rpath.
Run ``python -m megakernel.build`` from ``mega-kernel_amd/`` or call ``build()``.
"""

import os
import shutil
import subprocess
import sys
import sysconfig

PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))   # mega-kernel_amd/
REPO = os.path.dirname(PKG_ROOT)
CSRC = os.path.join(PKG_ROOT, "csrc")
INCLUDE = os.path.join(REPO, "include")
LIB = os.path.join(PKG_ROOT, "libmegakernel_amd.so")
EXT_NAME = "megakernel_extension"
ARCH = "gfx950"
# packed-fp32 VALU forms are disabled for every HIP translation unit
HIP_FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _hipcc():
    return shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


def ext_path():
    suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    return os.path.join(PKG_ROOT, EXT_NAME + suffix)


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)


def build_library(verbose=True):
    srcs = [os.path.join(CSRC, f) for f in ("decode_kernel.hip", "layers_kernel.hip", "batch_kernel.hip")]
    tmp = LIB + ".tmp"
    _run([_hipcc(), *HIP_FLAGS, "-shared", f"-I{INCLUDE}", *srcs, "-o", tmp], verbose)
    os.replace(tmp, LIB)
    return LIB


def build_extension(verbose=True):
    import torch
    from torch.utils import cpp_extension
    tdir = os.path.dirname(torch.__file__)
    incs = cpp_extension.include_paths(device_type="cuda")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    out = ext_path()
    tmp = out + ".tmp"
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-w",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           f"-DTORCH_EXTENSION_NAME={EXT_NAME}", "-DTORCH_API_INCLUDE_EXTENSION_H",
           *[f"-I{p}" for p in incs], f"-I{sysconfig.get_paths()['include']}", f"-I{INCLUDE}",
           os.path.join(CSRC, "torch_binding.cpp"),
           f"-L{os.path.join(tdir, 'lib')}", "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python",
           "-lc10_hip", "-ltorch_hip", f"-L{PKG_ROOT}", "-lmegakernel_amd",
           "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{os.path.join(tdir, 'lib')}", "-o", tmp]
    _run(cmd, verbose)
    os.replace(tmp, out)
    return out


def build_bench(verbose=True):
    """``mk_bench``: the C-ABI-only driver (profiling and phase traces)."""
    out = os.path.join(PKG_ROOT, "mk_bench")
    _run([_hipcc(), *HIP_FLAGS, f"-I{INCLUDE}", os.path.join(CSRC, "mk_bench.cpp"), f"-L{PKG_ROOT}",
          "-lmegakernel_amd", "-Wl,-rpath,$ORIGIN", "-o", out + ".tmp"], verbose)
    os.replace(out + ".tmp", out)
    return out


def build(verbose=True):
    """Compile every artefact (always; this is the build check)."""
    build_library(verbose)
    build_extension(verbose)
    build_bench(verbose)


if __name__ == "__main__":
    build(verbose="-q" not in sys.argv)
