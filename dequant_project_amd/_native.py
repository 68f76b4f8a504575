"""Loading of the engine's native libraries (built in-tree by build.py).

  ext()   the torch extension module `dequant_project_amd.dequant_cuda`
          (the reference's `dequant_cuda` surface: add_one, gemv, dequantize,
          plus unpack). Imported lazily, as the reference's
          dequant/quant_linear.py:49-69 does, and an ImportError with the build
          command is raised if it is missing -- there is no fallback path.
  capi()  ctypes handle on libdequant_hip.so with argtypes for every entry
          point of include/dequant_hip.h, for FFI-level use and tests.
"""

import ctypes
import importlib
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
LIB_PATH = PKG / "libdequant_hip.so"

_ext = None
_capi = None

BUILD_HINT = (
    "Build it once with:\n"
    f"    cd {ROOT}\n"
    "    python -m dequant_project_amd.build\n"
    "Re-run that after any change under dequant_project_amd/csrc/."
)


def ext():
    """The torch extension module (gemv / dequantize / unpack / add_one)."""
    global _ext
    if _ext is not None:
        return _ext
    import torch  # noqa: F401  (loads libc10/libtorch before the extension)
    try:
        _ext = importlib.import_module("dequant_project_amd.dequant_cuda")
    except ImportError as exc:
        raise ImportError("dequant_cuda extension is not built. " + BUILD_HINT) from exc
    return _ext


class DqTensor(ctypes.Structure):
    """struct dq_tensor of include/dequant_hip.h."""

    _fields_ = [
        ("data", ctypes.c_void_p),
        ("is_device", ctypes.c_int32),
        ("device", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("contiguous", ctypes.c_int32),
        ("ndim", ctypes.c_int32),
        ("sizes", ctypes.c_int64 * 4),
    ]


class DqGemvProblem(ctypes.Structure):
    """struct dq_gemv_problem of include/dequant_hip.h."""

    _fields_ = [
        ("x", ctypes.c_void_p),
        ("qweight", ctypes.c_void_p),
        ("scales", ctypes.c_void_p),
        ("zeros", ctypes.c_void_p),
        ("y", ctypes.c_void_p),
        ("N", ctypes.c_int64),
        ("K", ctypes.c_int64),
        ("group_size", ctypes.c_int64),
    ]


DQ_MAX_BATCH = 16
DQ_DTYPE_OTHER, DQ_DTYPE_INT32, DQ_DTYPE_FLOAT16, DQ_DTYPE_FLOAT32 = 0, 1, 2, 3
DQ_OK, DQ_ERR_INVALID_ARGUMENT, DQ_ERR_UNSUPPORTED, DQ_ERR_LAUNCH, DQ_ERR_HIP = 0, 1, 2, 3, 4

# name -> (restype, argtypes); keep in sync with include/dequant_hip.h
_P, _I, _I64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
_T = ctypes.POINTER(DqTensor)
SIGNATURES = {
    "dq_last_error": (ctypes.c_char_p, []),
    "dq_status_name": (ctypes.c_char_p, [_I]),
    "dq_version": (_I, []),
    "dq_check_gemv": (_I, [_T, _T, _T, _T, _I64, _I64, _I]),
    "dq_check_gemm_small": (_I, [_T, _T, _T, _T, _I64, _I64, _I]),
    "dq_check_dequantize": (_I, [_T, _T, _T, _I64, _I64, _I, _I64]),
    "dq_check_unpack": (_I, [_T, _I64, _I64]),
    "dq_gemv": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I, _I, _P]),
    "dq_gemv_batched": (_I, [ctypes.POINTER(DqGemvProblem), _I, _I64, _I64, _I, _I, _P]),
    "dq_gemm_small": (_I, [ctypes.POINTER(DqGemvProblem), _I, _I64, _I64, _I, _I, _P]),
    "dq_gemm_small_noalloc": (_I, [ctypes.POINTER(DqGemvProblem), _I, _I64, _I64, _I, _I, _P]),
    "dq_gemm_small_plan": (_I, [ctypes.POINTER(DqGemvProblem), _I, _I64, _I64, ctypes.POINTER(ctypes.c_int)]),
    "dq_gemv_prologue_batched": (_I, [ctypes.POINTER(DqGemvProblem), ctypes.POINTER(_P), _I, _I64, _I64, _I, _I,
                                      _I, ctypes.c_float, _P]),
    "dq_gemv_plan": (_I, [ctypes.POINTER(DqGemvProblem), _I, _I64, _I64, ctypes.POINTER(ctypes.c_int),
                          ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int)]),
    "dq_set_launch_events": (_I, [_P, _P]),
    "dq_dequantize": (_I, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I, _I, _P]),
    "dq_unpack": (_I, [_P, _P, _I64, _I64, _I64, _I, _P]),
    "dq_add_one": (_I, [_P, _P, _I64, _P]),
    "dq_stream_read": (_I, [_P, _I64, _P, _P]),
    "dq_empty_kernel": (_I, [_P]),
}


def capi():
    """ctypes.CDLL of libdequant_hip.so with typed entry points."""
    global _capi
    if _capi is not None:
        return _capi
    if not LIB_PATH.exists():
        raise ImportError(f"{LIB_PATH.name} is not built. " + BUILD_HINT)
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _capi = lib
    return lib


def describe(t):
    """DqTensor for a torch tensor (what the C++ binding builds internally)."""
    import torch

    d = DqTensor()
    d.data = t.data_ptr()
    d.is_device = 1 if t.is_cuda else 0
    d.device = t.get_device() if t.is_cuda else -1
    d.dtype = {torch.int32: DQ_DTYPE_INT32, torch.float16: DQ_DTYPE_FLOAT16,
               torch.float32: DQ_DTYPE_FLOAT32}.get(t.dtype, DQ_DTYPE_OTHER)
    d.contiguous = 1 if t.is_contiguous() else 0
    d.ndim = t.dim()
    for i in range(min(t.dim(), 4)):
        d.sizes[i] = t.size(i)
    return d


def check(status):
    """Raise RuntimeError(dq_last_error()) for a non-OK status."""
    if status != DQ_OK:
        raise RuntimeError(capi().dq_last_error().decode())
