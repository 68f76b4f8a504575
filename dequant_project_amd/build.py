"""In-tree build of the engine's native code (gfx950 only).

Produces, next to this file:
  libdequant_hip.so    HIP kernels + the C ABI of include/dequant_hip.h
                       (hipcc --offload-arch=gfx950)
  dequant_cuda<ext>    the PyTorch-ROCm extension module with the reference's
                       `dequant_cuda` surface (kernels/bindings.cpp:5-17); a thin
                       C++ layer over libdequant_hip.so, built with g++ against
                       torch's headers and linked with rpath $ORIGIN.

Run:  python -m dequant_project_amd.build      (or __graft_entry__.build())
Both steps always recompile. hipcc cross-compiles for gfx950 without a GPU.
"""

import os
import shutil
import subprocess
import sys
import sysconfig
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))

LIB_NAME = "libdequant_hip.so"
EXT_NAME = "dequant_cuda"

# -packed-fp32-ops: never emit v_pk_{add,mul,fma}_f32 (hipcc warns on the host
# pass that it does not know the feature; that is harmless).
HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def _run(cmd):
    print("+", " ".join(str(c) for c in cmd), flush=True)
    proc = subprocess.run([str(c) for c in cmd], capture_output=True, text=True)
    out = "\n".join(line for line in (proc.stdout + proc.stderr).splitlines()
                    if "is not a recognized feature for this target" not in line)
    if out.strip():
        print(out, flush=True)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {cmd[0]}")


def build_hip_lib():
    hipcc = shutil.which("hipcc") or str(ROCM / "bin" / "hipcc")
    out = PKG / LIB_NAME
    tmp = out.with_suffix(".so.tmp")
    _run([hipcc, *HIPCC_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}",
          CSRC / "dq_kernels.hip", CSRC / "dq_capi.cpp", "-o", tmp])
    os.replace(tmp, out)
    return out


def ext_filename():
    return EXT_NAME + sysconfig.get_config_var("EXT_SUFFIX")


def build_torch_ext():
    import torch
    from torch.utils import cpp_extension as ce

    incs = ce.include_paths(device_type="cuda")
    libdirs = ce.library_paths(device_type="cuda")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    # the check torch's own extension builder makes of the host compiler
    compatible, version = ce.get_compiler_abi_compatibility_and_version("g++")
    if not compatible:
        raise RuntimeError(f"g++ {version} is not ABI-compatible with this torch build")
    out = PKG / ext_filename()
    tmp = out.with_suffix(".tmp")
    cmd = [
        "g++", "-O2", "-std=c++17", "-fPIC", "-shared",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-DUSE_ROCM=1", "-D__HIP_PLATFORM_AMD__=1",
        f"-DTORCH_EXTENSION_NAME={EXT_NAME}", "-DTORCH_API_INCLUDE_EXTENSION_H",
        f"-I{INCLUDE}", *[f"-I{p}" for p in incs],
        f"-I{sysconfig.get_paths()['include']}",
        CSRC / "dq_torch.cpp",
        "-o", tmp,
        f"-L{PKG}", "-ldequant_hip", "-Wl,-rpath,$ORIGIN",
        *[f"-L{p}" for p in libdirs],
        "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python", "-lc10_hip", "-ltorch_hip",
        "-lamdhip64",
    ]
    _run(cmd)
    os.replace(tmp, out)
    return out


def build_all():
    lib = build_hip_lib()
    ext = build_torch_ext()
    return lib, ext


if __name__ == "__main__":
    sys.exit(0 if build_all() else 1)
