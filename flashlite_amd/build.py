"""In-tree build of the HIP library and the torch binding.

    python flashlite_amd/build.py

(run as a script: importing the package needs the extension it builds)

1. ``hipcc --offload-arch=gfx950`` compiles the kernels and the C ABI
   (``csrc/*.hip``, one object per source, in parallel) and links them
   into ``flashlite_amd/libflashlite_attn.so``.  The diagnostic kernels
   (``csrc/diag.hip``, not part of the attention path) become
   ``flashlite_amd/libflashlite_diag.so``.
2. The host C++ compiler compiles the binding (``csrc/flash_attn.cpp``)
   against the torch headers into
   ``flashlite_amd/flash_attn_wmma<EXT_SUFFIX>``, linked to the library
   with an ``$ORIGIN`` rpath.

No hipify step, no JIT cache: both files are written next to this script so
they travel with the source tree.  Every call rebuilds.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import sysconfig
import tempfile
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
INCLUDE = os.path.join(REPO_DIR, "include")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
ARCH = "gfx950"

LIB_NAME = "libflashlite_attn.so"
DIAG_LIB_NAME = "libflashlite_diag.so"
EXT_NAME = "flash_attn_wmma"

HIP_SOURCES = ["fa2_fwd.hip", "fa2_pipe.hip", "fa2_slot.hip", "fa2_stream.hip", "fa2_short.hip",
               "fa2_d128.hip",
               "naive_fwd.hip", "capi.hip"]
DIAG_SOURCES = ["diag.hip", "diag_timeline.hip"]

# -packed-fp32-ops: keep the compiler from emitting v_pk_{add,mul,fma}_f32.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-command-line-argument",
]


def _run(cmd):
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass does not know the packed-fp32 target feature; that
    # warning is expected and dropped from the log.
    out = "\n".join(line for line in proc.stdout.splitlines()
                    if "is not a recognized feature for this target" not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    return out


def lib_path() -> str:
    return os.path.join(PKG_DIR, LIB_NAME)


def ext_path() -> str:
    return os.path.join(PKG_DIR, EXT_NAME + sysconfig.get_config_var("EXT_SUFFIX"))


def _build_shared(sources, out: str, verbose: bool, exports: str) -> str:
    """Compiles each source to an object in parallel, then links them,
    exporting only the C symbols that match `exports` (the internal C++
    launchers stay local, so two of these libraries in one process never
    resolve each other's)."""
    hipcc = os.path.join(ROCM, "bin", "hipcc")
    with tempfile.TemporaryDirectory(prefix="flashlite_build_") as tmpdir:
        objs = [os.path.join(tmpdir, os.path.splitext(s)[0] + ".o") for s in sources]
        cmds = [[hipcc, *HIP_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-c",
                 os.path.join(CSRC, s), "-o", o] for s, o in zip(sources, objs)]
        workers = max(1, min(len(cmds), os.cpu_count() or 1, 16))
        with ThreadPoolExecutor(max_workers=workers) as pool:
            logs = list(pool.map(_run, cmds))
        tmp = out + ".tmp"
        script = os.path.join(tmpdir, "exports.map")
        with open(script, "w") as f:
            f.write("{ global: %s; local: *; };\n" % exports)
        logs.append(_run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs,
                          f"-Wl,--version-script={script}", "-o", tmp]))
    if verbose:
        for log in logs:
            if log.strip():
                print(log)
    os.replace(tmp, out)
    return out


def build_library(verbose: bool = False) -> str:
    return _build_shared(HIP_SOURCES, lib_path(), verbose, "fl_attn_*")


def build_diag_library(verbose: bool = False) -> str:
    return _build_shared(DIAG_SOURCES, os.path.join(PKG_DIR, DIAG_LIB_NAME), verbose, "fl_diag_*")


def build_extension(verbose: bool = False) -> str:
    import torch.utils.cpp_extension as ce

    cxx = shutil.which(os.environ.get("CXX", "g++")) or "g++"
    torch_inc = ce.include_paths(device_type="cuda")
    torch_lib = ce.library_paths(device_type="cuda")
    py_inc = sysconfig.get_paths()["include"]
    abi = int(__import__("torch")._C._GLIBCXX_USE_CXX11_ABI)
    out = ext_path()
    tmp = out + ".tmp"
    cmd = [cxx, "-O2", "-std=c++17", "-fPIC", "-shared", "-fvisibility=hidden",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", "-DHIPBLAS_V2",
           f"-D_GLIBCXX_USE_CXX11_ABI={abi}", f"-DTORCH_EXTENSION_NAME={EXT_NAME}",
           "-DTORCH_API_INCLUDE_EXTENSION_H",
           *[f"-I{p}" for p in torch_inc], f"-I{py_inc}", f"-I{INCLUDE}",
           os.path.join(CSRC, "flash_attn.cpp"),
           f"-L{PKG_DIR}", "-lflashlite_attn",
           *[f"-L{p}" for p in torch_lib],
           "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python", "-lc10_hip", "-ltorch_hip",
           f"-L{ROCM}/lib", "-lamdhip64",
           "-Wl,-rpath,$ORIGIN", *[f"-Wl,-rpath,{p}" for p in torch_lib], f"-Wl,-rpath,{ROCM}/lib",
           "-o", tmp]
    log = _run(cmd)
    if verbose and log.strip():
        print(log)
    os.replace(tmp, out)
    return out


def build(verbose: bool = False):
    # The diagnostic library compiles its own copy of the slot kernels:
    # build it beside the product library instead of after it.
    with ThreadPoolExecutor(max_workers=2) as pool:
        diag = pool.submit(build_diag_library, verbose)
        lib = build_library(verbose)
        ext = build_extension(verbose)
        diag.result()
    return lib, ext


if __name__ == "__main__":
    for path in build(verbose="-v" in sys.argv):
        print("built", os.path.relpath(path, REPO_DIR))
