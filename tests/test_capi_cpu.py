"""The C ABI on a machine without a GPU: it loads, exports what the header
declares, and validates arguments in the reference's order with the
reference's messages (kernels/dequant_gemv.cu:230-283, 310-317, 342-361).
No compute call is made here."""

import ctypes
import re

import pytest
import torch

from dequant_project_amd import _native
from dequant_project_amd._native import DQ_DTYPE_FLOAT16, DQ_DTYPE_FLOAT32, DQ_DTYPE_INT32, DqTensor
from tests._helpers import ROOT

HEADER = ROOT / "include" / "dequant_hip.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\**(dq_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_boundary():
    names = declared_functions()
    for required in ("dq_gemv", "dq_dequantize", "dq_unpack", "dq_add_one", "dq_check_gemv",
                     "dq_check_dequantize", "dq_check_unpack", "dq_last_error", "dq_status_name",
                     "dq_version"):
        assert required in names


def test_library_exports_every_declared_symbol():
    lib = _native.capi()
    for name in declared_functions():
        assert hasattr(lib, name), name
        assert name in _native.SIGNATURES, f"{name} missing from _native.SIGNATURES"
    assert lib.dq_version() == 100
    assert lib.dq_status_name(0) == b"DQ_OK"


def dev(t):
    """Describe a CPU tensor as if it lived on GPU 0 (validation only)."""
    d = _native.describe(t)
    d.is_device, d.device = 1, 0
    return d


def gemv_args(m=1, n=64, k=256, bits=4, gs=128, sym=False):
    per = 32 // bits
    x = torch.zeros(m, k, dtype=torch.float16)
    qw = torch.zeros(n, k // per, dtype=torch.int32)
    sc = torch.zeros(n, k // gs, dtype=torch.float16)
    ze = None if sym else torch.zeros(n, k // gs, dtype=torch.float16)
    return x, qw, sc, ze


def check_gemv(x, qw, sc, ze, bits=4, gs=128, sym=False):
    lib = _native.capi()
    st = lib.dq_check_gemv(x, qw, sc, ze, bits, gs, int(sym))
    return st, lib.dq_last_error().decode()


def test_check_gemv_accepts_valid():
    x, qw, sc, ze = gemv_args()
    assert check_gemv(dev(x), dev(qw), dev(sc), dev(ze)) == (0, "")
    x, qw, sc, ze = gemv_args(m=8, bits=2, gs=64, sym=True)
    assert check_gemv(dev(x), dev(qw), dev(sc), None, bits=2, gs=64, sym=True) == (0, "")


@pytest.mark.parametrize("mutate,status,msg", [
    (lambda a: a.__setitem__("x", _native.describe(a["x_t"])), 1, "x must be a CUDA tensor"),
    (lambda a: setattr(a["x"], "dtype", DQ_DTYPE_FLOAT32), 1, "x must be float16"),
    (lambda a: setattr(a["x"], "contiguous", 0), 1, "x must be contiguous"),
    (lambda a: setattr(a["x"], "ndim", 3), 1, "x must be 2-D [M, K], got 3-D"),
    (lambda a: a["x"].sizes.__setitem__(0, 9), 2,
     "gemv handles 1 <= M <= 8, got M=9; use the dequantize + F.linear fallback"),
    (lambda a: a["x"].sizes.__setitem__(0, 0), 2,
     "gemv handles 1 <= M <= 8, got M=0; use the dequantize + F.linear fallback"),
    (lambda a: setattr(a["x"], "data", a["x"].data + 2), 1, "x must be 16-byte aligned"),
    (lambda a: a.__setitem__("bits", 3), 1, "bits must be 2, 4 or 8, got 3"),
    (lambda a: a.__setitem__("gs", 0), 1, "group_size must be positive, got 0"),
    (lambda a: a.__setitem__("gs", 96), 1, "K=256 is not divisible by group_size=96"),
    (lambda a: setattr(a["qw"], "is_device", 0), 1, "qweight must be a CUDA tensor"),
    (lambda a: setattr(a["qw"], "dtype", DQ_DTYPE_FLOAT16), 1, "qweight must be int32"),
    (lambda a: setattr(a["qw"], "contiguous", 0), 1, "qweight must be contiguous"),
    (lambda a: setattr(a["qw"], "ndim", 1), 1, "qweight must be 2-D, got 1-D"),
    (lambda a: a["qw"].sizes.__setitem__(1, 31), 1,
     "qweight has 31 words per row, which is 248 codes, but K=256"),
    (lambda a: setattr(a["sc"], "is_device", 0), 1, "scales must be a CUDA tensor"),
    (lambda a: setattr(a["sc"], "dtype", DQ_DTYPE_FLOAT32), 1, "scales must be float16"),
    (lambda a: setattr(a["sc"], "contiguous", 0), 1, "scales must be contiguous"),
    (lambda a: a["sc"].sizes.__setitem__(1, 3), 1, "scales must be [64, 2], got [64, 3]"),
    (lambda a: setattr(a["sc"], "device", 1), 1, "scales and qweight must be on the same device"),
    (lambda a: a.__setitem__("ze", None), 1, "symmetric=false requires zeros"),
    (lambda a: a.__setitem__("sym", True), 1, "symmetric=true takes no zeros"),
    (lambda a: setattr(a["ze"], "is_device", 0), 1, "zeros must be a CUDA tensor"),
    (lambda a: setattr(a["ze"], "dtype", DQ_DTYPE_INT32), 1, "zeros must be float16"),
    (lambda a: setattr(a["ze"], "contiguous", 0), 1, "zeros must be contiguous"),
    (lambda a: a["ze"].sizes.__setitem__(0, 63), 1, "zeros must have the same shape as scales, got [63, 2]"),
    (lambda a: setattr(a["ze"], "device", 1), 1, "zeros and qweight must be on the same device"),
    (lambda a: setattr(a["x"], "device", 1), 1, "x and qweight must be on the same device"),
])
def test_check_gemv_messages(mutate, status, msg):
    x_t, qw_t, sc_t, ze_t = gemv_args()
    a = {"x_t": x_t, "x": dev(x_t), "qw": dev(qw_t), "sc": dev(sc_t), "ze": dev(ze_t),
         "bits": 4, "gs": 128, "sym": False}
    mutate(a)
    st, text = check_gemv(a["x"], a["qw"], a["sc"], a["ze"], a["bits"], a["gs"], a["sym"])
    assert (st, text) == (status, msg)


def test_check_gemv_int2_group32_rejected():
    x, qw, sc, _ = gemv_args(bits=2, gs=32, sym=True)
    st, text = check_gemv(dev(x), dev(qw), dev(sc), None, bits=2, gs=32, sym=True)
    assert st == 1
    assert text == ("group_size=32 must be a multiple of 64 (the codes one lane loads per uint4) at 2 bits; "
                    "this excludes INT2 with group_size 32")


def test_check_order_follows_reference():
    # x is checked before the weight (dequant_gemv.cu:342-354): a bad M wins over bad bits
    x, qw, sc, ze = gemv_args(m=9)
    assert check_gemv(dev(x), dev(qw), dev(sc), dev(ze), bits=5)[1].startswith("gemv handles")
    # bits before group_size before K divisibility (:233-238)
    assert check_gemv(dev(x[:1]), dev(qw), dev(sc), dev(ze), bits=5, gs=0)[1].startswith("bits must")
    assert check_gemv(dev(x[:1]), dev(qw), dev(sc), dev(ze), gs=0)[1].startswith("group_size must")


def test_check_dequantize_messages():
    lib = _native.capi()
    qw = torch.zeros(4, 8, dtype=torch.int32)     # INT4, K = 64
    sc = torch.zeros(4, 4, dtype=torch.float16)   # g16
    st = lib.dq_check_dequantize(dev(qw), dev(sc), None, 4, 16, 1, 64)
    assert (st, lib.dq_last_error()) == (0, b"")
    sc2 = torch.zeros(4, 16, dtype=torch.float16)  # g4: not a multiple of 8 values per word
    st = lib.dq_check_dequantize(dev(qw), dev(sc2), None, 4, 4, 1, 64)
    assert st == 1
    assert lib.dq_last_error() == b"group_size=4 must be a multiple of 8 values per uint32 word at 4 bits"
    st = lib.dq_check_dequantize(dev(qw), dev(sc), None, 4, 16, 1, 80)
    assert lib.dq_last_error() == b"qweight has 8 words per row, which is 64 codes, but K=80"


def test_check_unpack_messages():
    lib = _native.capi()
    qw = torch.zeros(4, 8, dtype=torch.int32)
    assert lib.dq_check_unpack(dev(qw), 4, 64) == 0
    assert lib.dq_check_unpack(dev(qw), 6, 64) == 1
    assert lib.dq_last_error() == b"bits must be 2, 4 or 8, got 6"
    assert lib.dq_check_unpack(dev(qw), 2, 64) == 1
    assert lib.dq_last_error() == b"qweight has 8 words per row, which is 128 codes, but K=64"


def test_raw_entry_points_validate_before_any_launch():
    lib = _native.capi()
    P = ctypes.c_void_p
    fake = P(0x1000)  # never dereferenced: every call below fails validation first
    assert lib.dq_gemv(fake, fake, fake, None, fake, 9, 4, 256, 4, 128, 1, 0, None) == 2
    assert lib.dq_last_error().startswith(b"gemv handles 1 <= M <= 8, got M=9")
    assert lib.dq_gemv(P(0x1002), fake, fake, None, fake, 1, 4, 256, 4, 128, 1, 0, None) == 1
    assert lib.dq_last_error() == b"x must be 16-byte aligned"
    assert lib.dq_gemv(fake, fake, fake, fake, fake, 1, 4, 256, 4, 128, 1, 0, None) == 1
    assert lib.dq_last_error() == b"symmetric=true takes no zeros"
    assert lib.dq_gemv(fake, fake, fake, None, fake, 1, 4, 256, 2, 32, 1, 0, None) == 1
    assert lib.dq_last_error().startswith(b"group_size=32 must be a multiple of 64")
    assert lib.dq_gemv(fake, P(0x1004), fake, None, fake, 1, 4, 256, 4, 128, 1, 0, None) == 1
    assert lib.dq_last_error() == b"qweight must be 16-byte aligned"
    assert lib.dq_gemv(None, fake, fake, None, fake, 1, 4, 256, 4, 128, 1, 0, None) == 1
    assert lib.dq_dequantize(fake, fake, None, fake, 4, 256, 8, 2, 1, 0, None) == 1
    assert lib.dq_last_error() == b"group_size=2 must be a multiple of 4 values per uint32 word at 8 bits"
    assert lib.dq_unpack(fake, P(0x1008), 4, 256, 4, 0, None) == 1
    assert lib.dq_last_error() == b"out must be 16-byte aligned"
    assert lib.dq_add_one(fake, fake, -1, None) == 1
    # empty problems are a no-op success without touching the GPU
    assert lib.dq_gemv(fake, fake, fake, None, fake, 1, 0, 256, 4, 128, 1, 0, None) == 0
    assert lib.dq_add_one(None, None, 0, None) == 0


def test_torch_binding_rejects_cpu_tensors_with_reference_messages():
    ext = _native.ext()
    x, qw, sc, ze = gemv_args()
    with pytest.raises(RuntimeError, match="^x must be a CUDA tensor$"):
        ext.gemv(x, qw, sc, ze, 4, 128, False, False)
    with pytest.raises(RuntimeError, match="^qweight must be a CUDA tensor$"):
        ext.dequantize(qw, sc, ze, 4, 128, False, False, 256)
    with pytest.raises(RuntimeError, match="^x must be a CUDA tensor$"):
        ext.add_one(torch.ones(4))
    # keyword names of kernels/bindings.cpp:6-16
    with pytest.raises(RuntimeError, match="CUDA tensor"):
        ext.gemv(x=x, qweight=qw, scales=sc, zeros=ze, bits=4, group_size=128, symmetric=False,
                 interleaved=False)
    with pytest.raises(RuntimeError, match="CUDA tensor"):
        ext.dequantize(qweight=qw, scales=sc, zeros=ze, bits=4, group_size=128, symmetric=False,
                       interleaved=False, K=256)
    with pytest.raises(RuntimeError, match="CUDA tensor"):
        ext.unpack(qweight=qw, bits=4, interleaved=False, K=256)


def test_gemm_small_plan_splits():
    """dq_gemm_small_plan (host logic): launches with 16 < M split K across
    blocks while the column groups (64 columns each) give fewer than 160
    blocks, at least one 4-iteration trip per split; M <= 16 never splits."""
    lib = _native.capi()

    def plan(m, shapes, bits=4):
        arr = (_native.DqGemvProblem * len(shapes))()
        for i, (n, k) in enumerate(shapes):
            arr[i].N, arr[i].K, arr[i].group_size = n, k, 128
        sp = (ctypes.c_int * len(shapes))()
        assert lib.dq_gemm_small_plan(arr, len(shapes), m, bits, sp) == 0, lib.dq_last_error()
        return list(sp)

    q, kv, gate, down = (4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)
    for m in (9, 16):
        assert plan(m, [q, kv, gate, down]) == [1, 1, 1, 1]
    for m in (17, 64):
        # 64 groups: 4 splits (256 blocks); 16 groups: 8 (32 iterations, 4 each); 224 groups: none
        assert plan(m, [q]) == [4] and plan(m, [kv]) == [8] and plan(m, [gate]) == [1] and plan(m, [down]) == [4]
    assert plan(64, [q, kv]) == [2, 2]       # 80 groups together: 2 splits
    assert plan(64, [(1000, 96)]) == [1]     # one iteration: nothing to split
    assert plan(64, [q], bits=8) == [4] and plan(64, [q], bits=2) == [4]
    arr = (_native.DqGemvProblem * 1)()
    arr[0].N, arr[0].K, arr[0].group_size = 64, 256, 128
    sp = (ctypes.c_int * 1)()
    assert lib.dq_gemm_small_plan(arr, 1, 65, 4, sp) == 2
    assert lib.dq_last_error().startswith(b"gemm_small handles 1 <= M <= 64, got M=65")
    assert lib.dq_gemm_small_plan(arr, 1, 64, 3, sp) == 1
    assert lib.dq_gemm_small_plan(arr, 1, 64, 4, None) == 1


def test_gemv_plan_geometry():
    """dq_gemv_plan (host logic): launch geometry chosen per launch from the problems' shapes."""
    lib = _native.capi()

    def plan(shapes, m=1, bits=4, gs=128):
        arr = (_native.DqGemvProblem * len(shapes))()
        for i, (n, k) in enumerate(shapes):
            arr[i].N, arr[i].K, arr[i].group_size = n, k, gs or k
        wk, rows, kind = (ctypes.c_int * len(shapes))(), ctypes.c_int(), ctypes.c_int()
        st = lib.dq_gemv_plan(arr, len(shapes), m, bits, wk, ctypes.byref(rows), ctypes.byref(kind))
        assert st == 0, lib.dq_last_error()
        return list(wk), rows.value, kind.value

    # M = 1: gemv_m1_kernel (kind 2; kind 3, its MFMA-dot variant, is not chosen),
    # or gemv_m1_pipe_kernel (kind 4) when every problem's tiles are one wave wide
    # (INT4 and INT8). INT4: 32 codes per 16-byte column. Rows per tile: 8 for
    # launches with >= 6144 tiles of 8 rows, else 4. wk: smallest of 1, 2, 4 giving
    # the launch 6144 waves (INT4), capped so each wave keeps >= 40 columns; but
    # one-wave tiles for INT2 launches and for launches of 512 to 1024 tiles.
    assert plan([(14336, 4096)]) == ([2], 4, 2)
    assert plan([(14336, 4096)] * 2) == ([1, 1], 4, 4)          # gate | up: 7168 waves already
    assert plan([(4096, 14336)]) == ([1], 4, 4)                 # 1024 tiles: one wave each
    assert plan([(4096, 4096)]) == ([1], 4, 4)
    assert plan([(1024, 4096)]) == ([2], 4, 8)                  # 256 tiles: under 512, the split stays
    assert plan([(1024, 8192)]) == ([4], 4, 8)                  # (pipelined split walk: kind 8)
    assert plan([(2048, 4096)]) == ([1], 4, 4)                  # 512 tiles: one wave each
    assert plan([(4096, 4096), (1024, 4096), (1024, 4096)]) == ([2, 2, 2], 4, 8)  # 1536 tiles: split
    assert plan([(4096, 4096), (1024, 4096), (1024, 4096)], bits=8, gs=128) == ([4, 4, 4], 4, 2)  # 1536 block-tiles
    assert plan([(8192, 8192)]) == ([4], 8, 2)                  # K >= 8192, 1024 tiles of 8 rows: 8-row split
    assert plan([(8192, 8192), (1024, 8192), (1024, 8192)]) == ([4, 4, 4], 8, 2)
    assert plan([(4096, 8192)]) == ([1], 4, 4)                  # 512 tiles of 8 rows: the 4-row rule
    assert plan([(14336, 4096)] * 16) == ([1] * 16, 8, 4)       # a stack of projections: 8-row tiles
    assert plan([(4096, 14336)] * 16) == ([1] * 16, 8, 4)
    assert plan([(4096, 14336)] * 16, bits=8, gs=None) == ([1] * 16, 8, 4)
    assert plan([(14336, 4096)] * 16, bits=2, gs=64) == ([1] * 16, 8, 6)  # INT2: activations kept across tiles
    assert plan([(14336, 8192)] * 16, bits=2, gs=64) == ([1] * 16, 8, 4)  # INT2 K = 8192: pipelined
    assert plan([(14336, 4096)] * 2, bits=2, gs=64) == ([1, 1], 4, 4)     # INT2 decode gate | up: pipelined
    assert plan([(4096, 11008)], bits=2, gs=64) == ([1], 4, 4)  # INT2: one-wave tiles, pipelined
    assert plan([(8192, 28672)], bits=2, gs=64) == ([1], 8, 4)
    assert plan([(11008, 4096)], bits=8, gs=None) == ([4], 4, 2)  # INT8 wants 8192 waves
    # M = 2, launches whose M = 1 plan has one-wave tiles: gemv_mx_pipe_kernel
    # (kind 7) with the M = 1 rows per tile.
    assert plan([(14336, 4096)] * 16, m=2) == ([1] * 16, 8, 7)
    assert plan([(14336, 4096)] * 2, m=2) == ([1, 1], 4, 7)
    assert plan([(14336, 4096)] * 16, m=2, bits=2, gs=64) == ([1] * 16, 8, 7)
    # the others, and 3 <= M <= 8: gemv_quad_kernel (kind 1) for every format and
    # group size; 8-row tiles (two quads), wk by the M = 1 rule for 8-row tiles.
    assert plan([(14336, 4096)] * 16, m=4) == ([1] * 16, 8, 1)
    assert plan([(14336, 4096)] * 2, m=3) == ([2, 2], 8, 1)
    assert plan([(4096, 4096)], m=4) == ([2], 8, 1)
    assert plan([(14336, 4096)] * 2, m=8) == ([2, 2], 8, 1)
    assert plan([(11008, 4096)], m=4, bits=8, gs=None) == ([2], 8, 1)  # INT8 quad launches: 2048 waves
    assert plan([(4096, 11008)], m=4, bits=2, gs=64) == ([4], 8, 1)
    assert plan([(4096, 4096)], m=2, gs=64) == ([2], 8, 1)
    assert plan([(14336, 4096)] * 16, m=8) == ([1] * 16, 8, 1)
    arr = (_native.DqGemvProblem * 1)()
    arr[0].N, arr[0].K, arr[0].group_size = 8, 100, 100
    wk, rows, kind = (ctypes.c_int * 1)(), ctypes.c_int(), ctypes.c_int()
    assert lib.dq_gemv_plan(arr, 1, 1, 4, wk, ctypes.byref(rows), ctypes.byref(kind)) == 1
    assert b"must be a positive multiple of 32" in lib.dq_last_error()
    arr[0].K, arr[0].group_size = 128, 48
    assert lib.dq_gemv_plan(arr, 1, 1, 4, wk, ctypes.byref(rows), ctypes.byref(kind)) == 1
    assert b"group_size=48 must divide K" in lib.dq_last_error()
    assert lib.dq_gemv_plan(arr, 1, 1, 4, wk, ctypes.byref(rows), None) == 1


def test_gemv_batched_validation():
    lib = _native.capi()
    arr = (_native.DqGemvProblem * 2)()
    assert lib.dq_gemv_batched(arr, 0, 1, 4, 1, 0, None) == 1
    assert lib.dq_last_error() == b"count must be in [1, 16], got 0"
    assert lib.dq_gemv_batched(arr, 2, 9, 4, 1, 0, None) == 2
    for i in range(2):
        arr[i].x = arr[i].qweight = arr[i].scales = arr[i].y = 0x1000
        arr[i].N, arr[i].K, arr[i].group_size = 4, 256, 128
    arr[1].K = 250
    assert lib.dq_gemv_batched(arr, 2, 1, 4, 1, 0, None) == 1
    assert lib.dq_last_error() == b"problem 1: K=250 is not divisible by group_size=128"
    assert lib.dq_set_launch_events(ctypes.c_void_p(0x10), None) == 1
    assert lib.dq_set_launch_events(None, None) == 0


def test_gemv_prologue_validation():
    """dq_gemv_prologue_batched rejects bad arguments before any launch."""
    lib = _native.capi()
    arr = (_native.DqGemvProblem * 2)()
    aux = (ctypes.c_void_p * 2)(0x2000, 0x2000)
    for i in range(2):
        arr[i].x = arr[i].qweight = arr[i].scales = arr[i].zeros = arr[i].y = 0x1000
        arr[i].N, arr[i].K, arr[i].group_size = 4, 256, 128
    call = lib.dq_gemv_prologue_batched
    assert call(arr, aux, 0, 1, 4, 0, 0, 1, 1e-5, None) == 1
    assert lib.dq_last_error() == b"count must be in [1, 16], got 0"
    assert call(arr, None, 2, 1, 4, 0, 0, 1, 1e-5, None) == 1
    assert lib.dq_last_error() == b"problems and aux must not be NULL"
    assert call(arr, aux, 2, 1, 4, 0, 0, 3, 1e-5, None) == 1
    assert lib.dq_last_error() == b"unknown prologue 3"
    assert call(arr, aux, 2, 1, 4, 0, 0, 1, -1.0, None) == 1
    assert b"eps must be finite and non-negative" in lib.dq_last_error()
    assert call(arr, aux, 2, 1, 4, 0, 0, 1, float("nan"), None) == 1
    assert call(arr, aux, 2, 2, 4, 0, 0, 2, 0.0, None) == 2
    assert lib.dq_last_error() == b"fused prologues handle M = 1, got M=2"
    aux[1] = 0x2008
    assert call(arr, aux, 2, 1, 4, 0, 0, 2, 0.0, None) == 1
    assert lib.dq_last_error() == b"problem 1: aux must be 16-byte aligned"
    aux[1] = None
    assert call(arr, aux, 2, 1, 4, 0, 0, 2, 0.0, None) == 1
    assert lib.dq_last_error() == b"problem 1: aux must not be NULL"
    aux[1] = 0x2000
    arr[0].K = 250
    assert call(arr, aux, 2, 1, 4, 0, 0, 1, 1e-5, None) == 1
    assert lib.dq_last_error() == b"problem 0: K=250 is not divisible by group_size=128"
