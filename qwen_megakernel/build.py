"""Build and load the gfx950 decode library and its torch operator library.

Replaces the reference's JIT build (qwen_megakernel/build.py:47-63), which ran
``torch.utils.cpp_extension.load`` with nvcc ``-arch=sm_120a``.  Here two
shared objects are built in-tree, next to this file:

* ``libqwen_megakernel_amd.so`` -- the HIP kernels and the C ABI
  (include/qwen_megakernel.h), compiled by ``hipcc --offload-arch=gfx950``;
  no torch dependency.
* ``qwen_megakernel_C.so`` -- ``TORCH_LIBRARY(qwen_megakernel_C)`` with the
  reference's operator schemas, host-only C++ compiled by g++ against torch's
  headers and linked to the library above.

``get_extension()`` loads them (building first if they are missing or older
than their sources) and registers ``torch.ops.qwen_megakernel_C``.  There is
no fallback: without the built library the ops do not exist and callers fail.
"""

from __future__ import annotations

import os
import subprocess
import sys
import sysconfig

_DIR = os.path.dirname(os.path.abspath(__file__))
_CSRC = os.path.join(_DIR, "csrc")
_ROOT = os.path.dirname(_DIR)
_INCLUDE = os.path.join(_ROOT, "include")

LIB = os.path.join(_DIR, "libqwen_megakernel_amd.so")
OPS = os.path.join(_DIR, "qwen_megakernel_C.so")

ARCH = os.environ.get("QMK_OFFLOAD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

HIP_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    f"--offload-arch={ARCH}",
    # packed-fp32 VALU forms are disabled for all device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{_INCLUDE}",
]

_LIB_SOURCES = ["qmk_api.hip", "qmk_batch.hip", "qmk_sample.hip", "qmk_decode_kernel.h", "qmk_batch_decode.h",
                "qmk_device.h", "qmk_state.h", "qmk_phase_bench.h", "qmk_sample.h"]
_LIB_UNITS = ["qmk_api.hip", "qmk_batch.hip", "qmk_sample.hip"]
_OPS_SOURCES = ["torch_bindings.cpp"]

_module = None


def _sources(names):
    return [os.path.join(_CSRC, n) for n in names] + [os.path.join(_INCLUDE, "qwen_megakernel.h")]


def _stale(target, sources):
    if not os.path.exists(target):
        return True
    t = os.path.getmtime(target)
    return any(os.path.getmtime(s) > t for s in sources)


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"build failed ({res.returncode}):\n{' '.join(cmd)}\n{res.stdout}")
    return res.stdout


def build_library(verbose: bool = False) -> str:
    """Compile libqwen_megakernel_amd.so (HIP kernels + C ABI)."""
    tmp = LIB + ".tmp"
    _run([HIPCC, *HIP_FLAGS, *[os.path.join(_CSRC, n) for n in _LIB_UNITS], "-o", tmp], verbose)
    os.replace(tmp, LIB)
    return LIB


def build_ops(verbose: bool = False) -> str:
    """Compile qwen_megakernel_C.so (torch operator registration)."""
    import torch
    from torch.utils import cpp_extension

    torch_lib = os.path.join(os.path.dirname(torch.__file__), "lib")
    incs = cpp_extension.include_paths(device_type="cuda") + [
        sysconfig.get_paths()["include"], os.path.join(ROCM, "include"), _INCLUDE]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    tmp = OPS + ".tmp"
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-w",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           "-DTORCH_EXTENSION_NAME=qwen_megakernel_C", "-DTORCH_API_INCLUDE_EXTENSION_H",
           *[f"-I{p}" for p in incs],
           os.path.join(_CSRC, "torch_bindings.cpp"), "-o", tmp,
           f"-L{_DIR}", "-lqwen_megakernel_amd", f"-L{torch_lib}",
           "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip",
           f"-L{os.path.join(ROCM, 'lib')}", "-lamdhip64",
           "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{torch_lib}", f"-Wl,-rpath,{os.path.join(ROCM, 'lib')}"]
    _run(cmd, verbose)
    os.replace(tmp, OPS)
    return OPS


def build(force: bool = True, verbose: bool = False) -> None:
    """Build both shared objects (always when ``force``, else only if stale)."""
    if force or _stale(LIB, _sources(_LIB_SOURCES)):
        build_library(verbose)
    if force or _stale(OPS, _sources(_OPS_SOURCES)) or _stale(OPS, [LIB]):
        build_ops(verbose)


def is_built() -> bool:
    return os.path.exists(LIB) and os.path.exists(OPS)


def get_extension(build_if_missing: bool = True):
    """Load the operator library (building it if needed); returns torch.ops.qwen_megakernel_C.

    Same entry name as the reference (qwen_megakernel/build.py:47).
    """
    global _module
    if _module is not None:
        return _module
    import torch

    if build_if_missing and (not is_built() or _stale(LIB, _sources(_LIB_SOURCES))
                             or _stale(OPS, _sources(_OPS_SOURCES))):
        build(force=False)
    if not is_built():
        raise RuntimeError("qwen_megakernel: the HIP library is not built; run "
                           "QMK_NO_IMPORT_LOAD=1 python -m qwen_megakernel.build")
    torch.ops.load_library(OPS)
    _module = torch.ops.qwen_megakernel_C
    return _module


def load_c_library():
    """ctypes handle on libqwen_megakernel_amd.so (the C ABI, no torch)."""
    import ctypes

    if not os.path.exists(LIB):
        raise RuntimeError("libqwen_megakernel_amd.so is not built")
    return ctypes.CDLL(LIB)


if __name__ == "__main__":
    build(force=True, verbose="-v" in sys.argv)
    print(LIB)
    print(OPS)
