"""Parity of the HIP kernels with the CPU oracle (MI355X only).

Restates scripts/test_dequant_kernel.py of the reference (tests 1-5, :56-252)
and extends it to the benchmark configurations and edge shapes:

  unpack       bit-exact with oracle.packer_ref.unpack and the reference's
               golden codes
  dequantize   bit-exact (torch.equal) with the oracle and the golden fp16
               weights, every bits x layout x symmetry x group, gauss + skew
  gemv         two tolerances, both written here:
                 * the reference's elementwise fp32-accumulation criterion
                   |y - ref| <= 2^-11 |ref| + 2^-20 |W|@|x| against the fp64
                   product of exact_weight (test_dequant_kernel.py:112-122);
                 * the north star's rel-L2 <= 1e-3 against fp32
                   dequantize-then-matmul.
Weights come from seeded numpy generators; the packed tensors are made by the
product packer on the GPU and read back, so the oracle and the kernel consume
the same bytes.
"""

import numpy as np
import pytest

from oracle import packer_ref as P
from tests._helpers import (GOLDEN_CASES, activations, gauss_weight, golden, golden_tag,
                            outlier_weight, skew_weight)

pytestmark = pytest.mark.gpu

REL_L2_TOL = 1e-3   # north star: GEMV within rel-L2 <= 1e-3 of fp32 dequantize-then-matmul


# ------------------------------------------------------------------ helpers
def ext():
    from dequant_project_amd import _native
    return _native.ext()


def to_gpu(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def pack_on_gpu(torch, w16, bits, gs, sym, layout):
    """Product packer on the GPU; returns (pw, numpy copies for the oracle)."""
    from dequant_project_amd.packer import QuantConfig, quantize_tensor

    pw = quantize_tensor(to_gpu(torch, w16), QuantConfig(bits, gs, sym, layout))
    qw = pw.qweight.cpu().numpy()
    sc = pw.scales.cpu().numpy()
    ze = None if pw.zeros is None else pw.zeros.cpu().numpy()
    return pw, qw, sc, ze


def ext_args(pw):
    k = pw.shape[1]
    cfg = pw.config
    return (pw.qweight, pw.scales, pw.zeros, cfg.bits, cfg.effective_group_size(k), cfg.symmetric,
            cfg.layout == "interleaved")


class OracleCase:
    """Oracle-side view of one packed weight. rows: optional sample of output rows.

    Tolerances (both from the reference's own tests and north star):
      * elementwise |y - ref| <= 2^-11 |ref| + 2^-20 |W|@|x| with ref the fp64
        product of exact_weight (fp32 dequantize, no fp16 store);
      * rel-L2 <= 1e-3 against fp32 dequantize-then-matmul: against the
        exact_weight product always, and, when deq_ref is set, also against
        F.linear over packer.dequantize's fp16 weight. The latter is skipped
        for all-positive (skewed) weights: their outputs cancel, and the
        reference weight's own fp16 rounding then exceeds 1e-3 by itself.
    """

    def __init__(self, pw, qw, sc, ze, rows=None, deq_ref=True):
        n, k = pw.shape
        self.cfg = P.Config(pw.config.bits, pw.config.group_size, pw.config.symmetric, pw.config.layout)
        if rows is not None:
            qw, sc = qw[rows], sc[rows]
            ze = None if ze is None else ze[rows]
            n = len(rows)
        self.rows = rows
        self.w64 = P.exact_weight(qw, sc, ze, self.cfg, (n, k)).astype(np.float64)
        self.absw64 = np.abs(self.w64)
        self.deq32 = P.dequantize(qw, sc, ze, self.cfg, (n, k)).astype(np.float32) if deq_ref else None

    def check(self, y, x16, label):
        if self.rows is not None:
            y = y[:, self.rows]
        x64 = x16.astype(np.float64)
        ref = x64 @ self.w64.T
        absref = np.abs(x64) @ self.absw64.T
        ok, worst = P.gemv_criterion(y, ref, absref)
        rl2 = P.rel_l2(y, ref)
        rl2_deq = P.rel_l2(y, x16.astype(np.float32) @ self.deq32.T) if self.deq32 is not None else 0.0
        print(f"{label}: worst={worst:.3f}x tol rel_l2={rl2:.2e} rel_l2_vs_fp16_deq={rl2_deq:.2e}", flush=True)
        assert ok, f"{label}: elementwise criterion violated, worst {worst:.3f}x tol"
        assert rl2 <= REL_L2_TOL, f"{label}: rel-L2 {rl2:.3e} > {REL_L2_TOL}"
        assert rl2_deq <= REL_L2_TOL, f"{label}: rel-L2 vs fp16 dequantize {rl2_deq:.3e} > {REL_L2_TOL}"


def run_gemv(torch, pw, x16):
    return ext().gemv(to_gpu(torch, x16), *ext_args(pw)).cpu().numpy()


def check_gemv(torch, pw, qw, sc, ze, x16s, label, rows=None, deq_ref=True):
    """Run the fused GEMV for each x in x16s and apply both tolerances."""
    case = OracleCase(pw, qw, sc, ze, rows, deq_ref)
    for x16 in x16s:
        case.check(run_gemv(torch, pw, x16), x16, f"{label} M={x16.shape[0]}")


# --------------------------------------------------------- 1. extension loads
def test_extension_loads(torch_gpu):
    torch = torch_gpu
    out = ext().add_one(torch.ones(4, device="cuda"))
    assert torch.equal(out, torch.full((4,), 2.0, device="cuda"))
    big = torch.arange(1 << 20, dtype=torch.float32, device="cuda")
    assert torch.equal(ext().add_one(big), big + 1)


# ------------------------------------------------------------------- unpack
@pytest.mark.parametrize("bits", (2, 4, 8))
@pytest.mark.parametrize("layout", ("sequential", "interleaved"))
def test_unpack_bit_exact(torch_gpu, bits, layout):
    torch = torch_gpu
    cfg = P.Config(bits, None, True, layout)
    for n, k in [(1, 32 // bits), (37, 256), (1024, 3072)]:
        words = np.random.Generator(np.random.PCG64(n * k + bits)).integers(
            0, 2 ** 32, (n, k // cfg.per_pack), dtype=np.uint64).astype(np.uint32).view(np.int32)
        got = ext().unpack(to_gpu(torch, words), bits, layout == "interleaved", k).cpu().numpy()
        assert np.array_equal(got, P.unpack(words, cfg, k)), (n, k)


@pytest.mark.parametrize("bits,gs,sym,layout", GOLDEN_CASES, ids=[golden_tag(*c) for c in GOLDEN_CASES])
def test_unpack_and_dequantize_match_reference_golden(torch_gpu, bits, gs, sym, layout):
    torch = torch_gpu
    g = golden()
    t = golden_tag(bits, gs, sym, layout)
    n, k = g["w16"].shape
    qw = to_gpu(torch, g[t + "/qweight"])
    codes = ext().unpack(qw, bits, layout == "interleaved", k).cpu().numpy()
    assert np.array_equal(codes, g[t + "/codes"])
    sc = to_gpu(torch, g[t + "/scales"].view(np.float16))
    ze = None if sym else to_gpu(torch, g[t + "/zeros"].view(np.float16))
    deq = ext().dequantize(qw, sc, ze, bits, k if gs is None else gs, sym, layout == "interleaved", k)
    assert np.array_equal(deq.cpu().numpy().view(np.uint16), g[t + "/deq"])


# --------------------------------------------------------------- dequantize
@pytest.mark.parametrize("bits", (2, 4, 8))
@pytest.mark.parametrize("layout", ("sequential", "interleaved"))
def test_dequantize_bit_exact(torch_gpu, bits, layout):
    """scripts/test_dequant_kernel.py:63-89: torch.equal over sym x group x data."""
    torch = torch_gpu
    n, k = 1024, 3072
    gauss = gauss_weight(n, k, seed=100)
    skew = skew_weight(n, k, seed=101)
    for sym in (True, False):
        for gs in (32, 64, 128, 256, None):
            for tag, w in ([("gauss", gauss)] if sym else [("gauss", gauss), ("skew", skew)]):
                pw, qw, sc, ze = pack_on_gpu(torch, w, bits, gs, sym, layout)
                got = ext().dequantize(*ext_args(pw), k).cpu().numpy()
                want = P.dequantize(qw, sc, ze, P.Config(bits, gs, sym, layout), (n, k))
                bad = int((got.view(np.uint16) != want.view(np.uint16)).sum())
                assert bad == 0, f"{bits}-bit {layout} sym={sym} g{gs} {tag}: {bad} values differ"


def test_gpu_packer_matches_cpu_packer(torch_gpu):
    """The product packer gives the same bytes on the GPU as on the CPU."""
    torch = torch_gpu
    from dequant_project_amd.packer import QuantConfig, quantize_tensor

    w = torch.from_numpy(outlier_weight(512, 4096, seed=7))
    for args in [(4, 128, False, "sequential"), (2, 64, False, "interleaved"), (8, None, True, "sequential"),
                 (4, 32, True, "interleaved")]:
        a = quantize_tensor(w, QuantConfig(*args))
        b = quantize_tensor(w.cuda(), QuantConfig(*args))
        assert torch.equal(a.qweight, b.qweight.cpu()), args
        assert torch.equal(a.scales, b.scales.cpu()), args
        assert (a.zeros is None) == (b.zeros is None)
        if a.zeros is not None:
            assert torch.equal(a.zeros, b.zeros.cpu()), args


# --------------------------------------------------------------------- gemv
GEMV_FORMATS = [  # scripts/test_dequant_kernel.py:137-145, plus INT2 and asym INT8
    (4, 128, True, "sequential"), (4, 128, False, "sequential"),
    (4, 128, True, "interleaved"), (4, 128, False, "interleaved"),
    (8, 128, True, "sequential"), (8, 128, True, "interleaved"),
    (4, None, True, "sequential"),
    (2, 64, True, "sequential"), (2, 64, False, "interleaved"), (2, 128, False, "sequential"),
    (8, None, False, "interleaved"), (8, 16, False, "sequential"), (4, 32, False, "interleaved"),
]
GEMV_SHAPES = [(3072, 3072), (1024, 3072), (8192, 3072), (3072, 8192)]


@pytest.mark.parametrize("n,k", GEMV_SHAPES)
def test_gemv_reference_suite(torch_gpu, n, k):
    """scripts/test_dequant_kernel.py:149-172 (M in {1,2,3,8}) over more formats."""
    torch = torch_gpu
    w16 = gauss_weight(n, k, seed=n + k)
    for fmt in GEMV_FORMATS:
        pw, qw, sc, ze = pack_on_gpu(torch, w16, *fmt)
        check_gemv(torch, pw, qw, sc, ze, [activations(m, k, seed=m) for m in (1, 2, 3, 8)], f"[{n},{k}] {fmt}")


@pytest.mark.parametrize("m", range(1, 9))
def test_gemv_every_m(torch_gpu, m):
    torch = torch_gpu
    n, k = 777, 2048
    for fmt in [(4, 128, False, "sequential"), (2, 64, False, "sequential"), (8, None, True, "interleaved")]:
        pw, qw, sc, ze = pack_on_gpu(torch, gauss_weight(n, k, seed=5), *fmt)
        check_gemv(torch, pw, qw, sc, ze, [activations(m, k, seed=10 + m)], f"{fmt}")


@pytest.mark.parametrize("n,k,fmt", [
    (1, 128, (4, 128, False, "sequential")),      # a single row
    (3, 64, (2, 64, True, "interleaved")),        # one chunk per row
    (17, 16, (8, 16, False, "sequential")),       # K = one 16-byte chunk at INT8
    (5, 4160, (2, 64, False, "sequential")),      # 65 chunks: one lane takes two
    (19, 4096 + 64 * 32, (4, 64, True, "interleaved")),
    (65, 11008, (2, 64, False, "sequential")),    # 172 chunks (config C3's K)
    (130, 28672, (2, 64, False, "interleaved")),  # C5 down_proj K
    (31, 8192, (8, None, True, "sequential")),    # C5 lm_head K
])
def test_gemv_edge_shapes(torch_gpu, n, k, fmt):
    torch = torch_gpu
    pw, qw, sc, ze = pack_on_gpu(torch, gauss_weight(n, k, seed=n * 3 + k), *fmt)
    check_gemv(torch, pw, qw, sc, ze, [activations(m, k, seed=m + 1) for m in (1, 4, 8)], f"[{n},{k}] {fmt}")


def test_gemv_skewed_weights_negative_zero_points(torch_gpu):
    torch = torch_gpu
    n, k = 512, 4096
    for fmt in [(4, 128, False, "sequential"), (2, 64, False, "interleaved"), (8, 128, False, "sequential"),
                (8, None, False, "sequential")]:
        pw, qw, sc, ze = pack_on_gpu(torch, skew_weight(n, k, seed=21), *fmt)
        assert (ze.astype(np.float32) < 0).any()
        check_gemv(torch, pw, qw, sc, ze, [activations(m, k, seed=22) for m in (1, 8)], f"skew {fmt}",
                   deq_ref=False)


def test_gemv_zero_points_beyond_fp16_exact_range(torch_gpu):
    """Zero points outside [-1024, 1024] (unclamped, packer.py:136-137): (q - z)
    is then not exact in fp16 and the kernels take their separate path (q
    exactly, minus z * sum(x) in fp32) for the tiles that hold one. Bands of 8
    rows of far-offset weights alternate with N(0, 0.02) rows, so tiles mix
    both kinds; every M = 1 kernel variant (VALU and MFMA dots) and both
    batch-row groupings of the 2 <= M <= 8 kernel (M <= 4, M > 4) are
    covered."""
    torch = torch_gpu
    n, k = 256, 4096
    # offset per format such that zero = round(-min / scale) lands past -1024
    for fmt, base in [((4, 128, False, "sequential"), 50.0), ((4, 128, False, "interleaved"), 50.0),
                      ((2, 64, False, "sequential"), 200.0), ((2, 64, False, "interleaved"), 200.0),
                      ((8, 128, False, "sequential"), 3.0), ((8, None, False, "sequential"), 3.0)]:
        w = gauss_weight(n, k, seed=31).astype(np.float32)
        band = (np.arange(n) // 8) % 2 == 1
        u = np.random.Generator(np.random.PCG64(32)).random((n, k), dtype=np.float32)
        w[band] = base + 0.5 * u[band]
        pw, qw, sc, ze = pack_on_gpu(torch, w.astype(np.float16), *fmt)
        zf = ze.astype(np.float32)
        assert (np.abs(zf[band]) > 1024).all() and (np.abs(zf[~band]) <= 1024).all(), fmt
        check_gemv(torch, pw, qw, sc, ze, [activations(m, k, seed=33) for m in (1, 3, 8)], f"wide zeros {fmt}",
                   deq_ref=False)


# ------------------------------------------------- fused small GEMM (M <= 64)
def check_gemm_small(torch, pw, qw, sc, ze, ms, label):
    """gemm_small against fp64 x @ W16^T, W16 = the oracle's packer.dequantize
    (the reference's M > 8 product): the reference's elementwise fp32
    criterion on that weight and rel-L2 <= 1e-3."""
    n, k = pw.shape
    cfg = P.Config(pw.config.bits, pw.config.group_size, pw.config.symmetric, pw.config.layout)
    w16 = P.dequantize(qw, sc, ze, cfg, (n, k)).astype(np.float64)
    for m in ms:
        x16 = activations(m, k, seed=100 + m)
        y = ext().gemm_small(to_gpu(torch, x16), *ext_args(pw)).cpu().numpy()
        ref = x16.astype(np.float64) @ w16.T
        absref = np.abs(x16.astype(np.float64)) @ np.abs(w16).T
        ok, worst = P.gemv_criterion(y, ref, absref)
        rl2 = P.rel_l2(y, ref)
        print(f"{label} M={m}: worst={worst:.3f}x tol rel_l2={rl2:.2e}", flush=True)
        assert ok, f"{label} M={m}: elementwise criterion violated, worst {worst:.3f}x tol"
        assert rl2 <= REL_L2_TOL, f"{label} M={m}: rel-L2 {rl2:.3e}"


@pytest.mark.parametrize("fmt", [(4, 128, False, "sequential"), (4, 64, True, "interleaved"),
                                 (8, None, True, "sequential")])
def test_gemm_small_shared_activation_kernel(torch_gpu, fmt):
    """gemm_small on a gate_proj shape (14336 x 4096) at M <= 32: M <= 16 runs
    the variant that shares each K-share's activations across the block's 4
    tiles (896 tiles of 16 rows split 4 ways along K, 224 blocks of 16
    waves), 16 < M <= 32 the column walk (224 groups of 64 columns, unsplit),
    against the dequantized product on a sample of rows including the last
    tile."""
    torch = torch_gpu
    from dequant_project_amd.packer import QuantConfig, quantize_tensor

    n, k = 14336, 4096
    gen = torch.Generator(device="cuda").manual_seed(77)
    pw = quantize_tensor(torch.randn(n, k, generator=gen, device="cuda", dtype=torch.float16) * 0.02,
                         QuantConfig(*fmt))
    rows = np.unique(np.concatenate([np.random.Generator(np.random.PCG64(5)).choice(n - 16, 300, replace=False),
                                     np.arange(n - 16, n)]))
    qw, sc = pw.qweight[rows].cpu().numpy(), pw.scales[rows].cpu().numpy()
    ze = None if pw.zeros is None else pw.zeros[rows].cpu().numpy()
    cfg = P.Config(*fmt)
    w16 = P.dequantize(qw, sc, ze, cfg, (len(rows), k)).astype(np.float64)
    for m in (3, 9, 16, 24, 32):
        x16 = activations(m, k, seed=200 + m)
        y = ext().gemm_small(to_gpu(torch, x16), *ext_args(pw)).cpu().numpy()[:, rows]
        ref = x16.astype(np.float64) @ w16.T
        absref = np.abs(x16.astype(np.float64)) @ np.abs(w16).T
        ok, worst = P.gemv_criterion(y, ref, absref)
        rl2 = P.rel_l2(y, ref)
        print(f"shared-activation gemm {fmt} M={m}: worst={worst:.3f}x tol rel_l2={rl2:.2e}", flush=True)
        assert ok, f"{fmt} M={m}: elementwise criterion violated, worst {worst:.3f}x tol"
        assert rl2 <= REL_L2_TOL, f"{fmt} M={m}: rel-L2 {rl2:.3e}"


def test_random_formats_and_shapes_sweep(torch_gpu):
    """A seeded sweep over the operand space the C ABI accepts: 36 cases of
    random bits, layout, symmetry, group size (a multiple of one 16-byte
    chunk's codes, or per-channel), ragged N up to 2500, K up to ~6000 and
    M in 1..8, each GEMV against the oracle's two tolerances; every third
    case also runs the small GEMM at an M in 9..64 against the dequantized
    product. Shapes no fixed test names (odd N, K of a few chunks, groups
    that straddle a batch of 64 chunks) land here."""
    torch = torch_gpu
    rng = np.random.Generator(np.random.PCG64(2026))
    for case in range(36):
        bits = int(rng.choice([2, 4, 8]))
        cpl = 128 // bits
        layout = str(rng.choice(["sequential", "interleaved"]))
        sym = bool(rng.integers(2))
        groups = [g for g in (16, 32, 64, 128, 256) if g % cpl == 0] + [None]
        gs = groups[int(rng.integers(len(groups)))]
        unit = cpl if gs is None else gs
        k = unit * int(rng.integers(1, max(2, 6144 // unit)))
        n = int(rng.integers(1, 2501))
        m = int(rng.choice([1, 1, 2, 3, 5, 8]))
        label = f"sweep {case}: INT{bits} g{gs} {'sym' if sym else 'asym'} {layout} [{n},{k}]"
        pw, qw, sc, ze = pack_on_gpu(torch, gauss_weight(n, k, seed=3000 + case), bits, gs, sym, layout)
        check_gemv(torch, pw, qw, sc, ze, [activations(m, k, seed=4000 + case)], label)
        if case % 3 == 0:
            check_gemm_small(torch, pw, qw, sc, ze, (int(rng.integers(9, 65)),), label)


GEMM_SMALL_CASES = [
    ((4, 128, False, "sequential"), 1000, 4096),
    ((4, 32, True, "interleaved"), 256, 96),       # 3 chunks: a partial iteration of 4
    ((2, 64, False, "sequential"), 512, 3072),     # 4 groups per MFMA iteration
    ((2, 128, True, "interleaved"), 384, 1024),
    ((8, None, True, "sequential"), 1100, 4096),   # per-channel
    ((8, 64, False, "interleaved"), 640, 2048),
]


@pytest.mark.parametrize("fmt,n,k", GEMM_SMALL_CASES, ids=[f"{c[0]}-{c[1]}x{c[2]}" for c in GEMM_SMALL_CASES])
def test_gemm_small_matches_dequantized_product(torch_gpu, fmt, n, k):
    torch = torch_gpu
    pw, qw, sc, ze = pack_on_gpu(torch, gauss_weight(n, k, seed=n + k), *fmt)
    check_gemm_small(torch, pw, qw, sc, ze, (1, 9, 16, 17, 33, 64), f"gemm_small {fmt} [{n},{k}]")


def test_gemm_small_zero_points_beyond_fp16_exact_range(torch_gpu):
    """Bands of far-offset rows (zero points past -1024) take W16 from fp32
    arithmetic; the result must still be the dequantized weight's product."""
    torch = torch_gpu
    n, k = 256, 2048
    for fmt, base in [((4, 128, False, "sequential"), 50.0), ((2, 64, False, "interleaved"), 200.0),
                      ((8, 128, False, "sequential"), 3.0)]:
        w = gauss_weight(n, k, seed=41).astype(np.float32)
        band = (np.arange(n) // 16) % 2 == 1
        u = np.random.Generator(np.random.PCG64(42)).random((n, k), dtype=np.float32)
        w[band] = base + 0.5 * u[band]
        pw, qw, sc, ze = pack_on_gpu(torch, w.astype(np.float16), *fmt)
        assert (np.abs(ze.astype(np.float32)[band]) > 1024).all()
        check_gemm_small(torch, pw, qw, sc, ze, (12, 40), f"gemm_small wide zeros {fmt}")


def test_gemm_small_split_along_k_in_graph_replays(torch_gpu):
    """16 < M <= 64 launches with few column groups split K across blocks:
    partial tiles in a per-stream scratch, summed in split order by a second
    launch. Captured in a CUDA graph on a stream that never ran a small GEMM
    (its scratch is allocated inside the capture), every replay, with eager
    work and synchronizations between them, must equal the eager result
    bit for bit; the eager result passes the dequantized-product check."""
    torch = torch_gpu
    n, k = 1000, 4096  # 16 column groups: 8 splits of 4 iterations
    pw, qw, sc, ze = pack_on_gpu(torch, gauss_weight(n, k, seed=91), 4, 128, False, "sequential")
    for m in (40, 64):
        check_gemm_small(torch, pw, qw, sc, ze, (m,), f"split gemm_small [{n},{k}]")
        x = to_gpu(torch, activations(m, k, seed=100 + m))
        eager = ext().gemm_small(x, *ext_args(pw))
        y = torch.empty_like(eager)
        side = torch.cuda.Stream()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=side):
            y.copy_(ext().gemm_small(x, *ext_args(pw)))
        for rep in range(3):
            y.zero_()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(y, eager), f"M={m} replay {rep} differs from the eager result"
            ext().gemm_small(x * 2, *ext_args(pw))  # eager work on the default stream between replays
            torch.cuda.synchronize()


def test_gemm_small_rejects_batches_past_its_range(torch_gpu):
    torch = torch_gpu
    pw, _, _, _ = pack_on_gpu(torch, gauss_weight(64, 256, seed=5), 4, 128, False, "sequential")
    x = torch.zeros(65, 256, dtype=torch.float16, device="cuda")
    with pytest.raises(RuntimeError, match="gemm_small handles 1 <= M <= 64, got M=65"):
        ext().gemm_small(x, *ext_args(pw))


# ------------------------------------------------------- benchmark configs
def test_config_c1_int4_asym_g128(torch_gpu):
    torch = torch_gpu
    pw, qw, sc, ze = pack_on_gpu(torch, gauss_weight(4096, 4096, seed=1), 4, 128, False, "sequential")
    check_gemv(torch, pw, qw, sc, ze, [activations(1, 4096, seed=1)], "C1")


def test_config_c2_int8_per_channel(torch_gpu):
    torch = torch_gpu
    pw, qw, sc, ze = pack_on_gpu(torch, gauss_weight(11008, 4096, seed=2), 8, None, True, "sequential")
    check_gemv(torch, pw, qw, sc, ze, [activations(m, 4096, seed=2 + m) for m in (1, 4)], "C2")


def test_config_c3_int2_asym_g64_outliers(torch_gpu):
    torch = torch_gpu
    pw, qw, sc, ze = pack_on_gpu(torch, outlier_weight(4096, 11008, seed=3), 2, 64, False, "sequential")
    check_gemv(torch, pw, qw, sc, ze, [activations(1, 11008, seed=3)], "C3")


@pytest.mark.parametrize("name,n,k,fmt", [
    ("C4 q/o", 4096, 4096, (4, 128, False, "sequential")),
    ("C4 k/v", 1024, 4096, (4, 128, False, "sequential")),
    ("C4 gate/up", 14336, 4096, (4, 128, False, "sequential")),
    ("C4 down", 4096, 14336, (4, 128, False, "sequential")),
    ("C5 q/o", 8192, 8192, (4, 128, False, "sequential")),
    ("C5 k/v", 1024, 8192, (4, 128, False, "sequential")),
    ("C5 gate/up", 28672, 8192, (2, 64, False, "sequential")),
    ("C5 down", 8192, 28672, (2, 64, False, "sequential")),
])
def test_config_layer_shapes(torch_gpu, name, n, k, fmt):
    """Llama-3-8B / 70B projection shapes; M sweep of C4; rows sampled for the fp64 reference."""
    torch = torch_gpu
    pw, qw, sc, ze = pack_on_gpu(torch, gauss_weight(n, k, seed=n ^ k), *fmt)
    rows = np.sort(np.random.Generator(np.random.PCG64(n)).choice(n, min(n, 1024), replace=False))
    check_gemv(torch, pw, qw, sc, ze, [activations(m, k, seed=m) for m in (1, 2, 4, 8)], name, rows=rows)


def test_config_c5_lm_head_int8(torch_gpu):
    """The 70B lm_head (128256 x 8192, INT8 per channel): 512 sampled rows
    against the oracle, then every row against the same criterion."""
    torch = torch_gpu
    n, k = 128256, 8192
    from dequant_project_amd.packer import QuantConfig, quantize_tensor

    w = torch.randn(n, k, generator=torch.Generator(device="cuda").manual_seed(5), device="cuda",
                    dtype=torch.float16) * 0.02
    pw = quantize_tensor(w, QuantConfig(8, None, True))
    del w
    rows = np.sort(np.random.Generator(np.random.PCG64(9)).choice(n, 512, replace=False))
    qw = pw.qweight[torch.from_numpy(rows).cuda()].cpu().numpy()
    sc = pw.scales[torch.from_numpy(rows).cuda()].cpu().numpy()
    x16 = activations(1, k, seed=12)
    y = ext().gemv(to_gpu(torch, x16), *ext_args(pw)).cpu().numpy()
    cfg = P.Config(8, None, True)
    ew = P.exact_weight(qw, sc, None, cfg, (len(rows), k))
    ref, absref = P.gemv_reference(x16, ew)
    ok, worst = P.gemv_criterion(y[:, rows], ref, absref)
    assert ok, worst
    assert P.rel_l2(y[:, rows], x16.astype(np.float32) @ P.dequantize(qw, sc, None, cfg, (len(rows), k))
                    .astype(np.float32).T) <= REL_L2_TOL
    # Every row, against the same criterion in float64 on the GPU. INT8
    # sequential words hold codes 4j..4j+3 in bytes 0..3, so the uint8 view of
    # a row is its codes in order; the exact weight is (q - 128) * s, checked
    # bit for bit against the oracle's on the sampled rows.
    xd = torch.from_numpy(x16.astype(np.float64)).cuda()
    codes = pw.qweight.view(torch.uint8).view(n, k)
    sd = pw.scales.double()
    assert torch.equal((codes[torch.from_numpy(rows).cuda()].double() - 128) * sd[torch.from_numpy(rows).cuda()],
                       torch.from_numpy(ew.astype(np.float64)).cuda())
    yd = torch.from_numpy(y.astype(np.float64)).cuda()
    worst_all = 0.0
    for r0 in range(0, n, 16384):
        w = (codes[r0:r0 + 16384].double() - 128) * sd[r0:r0 + 16384]
        ref_c, abs_c = xd @ w.T, xd.abs() @ w.abs().T
        tol = 2.0 ** -11 * ref_c.abs() + 2.0 ** -20 * abs_c
        err = (yd[:, r0:r0 + 16384] - ref_c).abs()
        worst_all = max(worst_all, float((err / (tol + 1e-30)).max()))
        assert bool((err <= tol).all()), (r0, worst_all)
        del w


# ----------------------------------------------------------- errors (3b)
def test_excluded_formats_raise(torch_gpu):
    """scripts/test_dequant_kernel.py:174-191."""
    torch = torch_gpu
    from dequant_project_amd.packer import QuantConfig, quantize_tensor

    pw = quantize_tensor(torch.randn(64, 256, device="cuda", dtype=torch.float16), QuantConfig(2, 32, True))
    with pytest.raises(RuntimeError, match="this excludes INT2 with group_size 32"):
        ext().gemv(torch.randn(1, 256, device="cuda", dtype=torch.float16), *ext_args(pw))
    pw = quantize_tensor(torch.randn(64, 256, device="cuda", dtype=torch.float16), QuantConfig(4, 128, True))
    with pytest.raises(RuntimeError, match=r"^gemv handles 1 <= M <= 8, got M=9"):
        ext().gemv(torch.randn(9, 256, device="cuda", dtype=torch.float16), *ext_args(pw))
    buf = torch.randn(258, device="cuda", dtype=torch.float16)
    x_misaligned = buf[1:257].view(1, 256)          # contiguous, 2 bytes past an aligned address
    with pytest.raises(RuntimeError, match="^x must be 16-byte aligned$"):
        ext().gemv(x_misaligned, *ext_args(pw))


# -------------------------------------------------- 4. negative control
def test_negative_control(torch_gpu):
    """scripts/test_dequant_kernel.py:194-217: one flipped bit fails only [0, 0]."""
    torch = torch_gpu
    n, k = 3072, 3072
    pw, qw, sc, ze = pack_on_gpu(torch, gauss_weight(n, k, seed=0), 4, 128, True, "sequential")
    x16 = activations(1, k, seed=1000)   # a seed unrelated to the weight's, so y[0, 0] ~ N(0, 1)
    x16[0, 0] = np.float16(1.0)
    cfg = P.Config(4, 128, True, "sequential")
    ref, absref = P.gemv_reference(x16, P.exact_weight(qw, sc, ze, cfg, (n, k)))
    bad = pw.qweight.clone()
    bad[0, 0] ^= 1
    y = ext().gemv(to_gpu(torch, x16), bad, pw.scales, None, 4, 128, True, False).cpu().numpy()
    tol = 2.0 ** -11 * np.abs(ref) + 2.0 ** -20 * absref
    over = np.abs(y.astype(np.float64) - ref) > tol
    y_clean = ext().gemv(to_gpu(torch, x16), *ext_args(pw)).cpu().numpy()
    detail = (f"y_bad={float(y[0, 0])!r} y_clean={float(y_clean[0, 0])!r} ref={ref[0, 0]!r} tol={tol[0, 0]!r} "
              f"scale={float(sc[0, 0])!r} word={int(qw[0, 0]) & 0xFFFFFFFF:#010x} "
              f"bad_word={int(bad[0, 0].item()) & 0xFFFFFFFF:#010x}")
    print(detail, flush=True)
    assert over[0, 0], "flipped bit not detected: " + detail
    assert int(over.sum()) == 1, f"{int(over.sum())} elements over tolerance"


# ---------------------------------------------------- 5. graph capture
def test_graph_capture_replays_live_input(torch_gpu):
    """scripts/test_dequant_kernel.py:220-252."""
    torch = torch_gpu
    n, k = 3072, 3072
    pw, *_ = pack_on_gpu(torch, gauss_weight(n, k, seed=0), 4, 128, False, "sequential")
    args = ext_args(pw)
    x = to_gpu(torch, activations(1, k, seed=1))
    x2 = to_gpu(torch, activations(1, k, seed=2))
    eager1 = ext().gemv(x, *args).clone()
    eager2 = ext().gemv(x2, *args).clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            ext().gemv(x, *args)
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y = ext().gemv(x, *args)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager1)
    x.copy_(x2)
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(y, eager2)


def test_results_are_deterministic(torch_gpu):
    torch = torch_gpu
    pw, *_ = pack_on_gpu(torch, gauss_weight(4096, 4096, seed=8), 2, 64, False, "sequential")
    x = to_gpu(torch, activations(4, 4096, seed=8))
    y0 = ext().gemv(x, *ext_args(pw))
    for _ in range(5):
        assert torch.equal(ext().gemv(x, *ext_args(pw)), y0)


# ------------------------------------------------------- direct C ABI
def test_c_abi_matches_extension(torch_gpu):
    """Calls through include/dequant_hip.h with raw device pointers (ctypes)."""
    torch = torch_gpu
    from dequant_project_amd import _native

    lib = _native.capi()
    stream = torch.cuda.current_stream().cuda_stream
    n, k = 2048, 4096
    for fmt in [(4, 128, False, "sequential"), (2, 64, True, "interleaved"), (8, None, True, "sequential")]:
        pw, *_ = pack_on_gpu(torch, gauss_weight(n, k, seed=31), *fmt)
        bits, gs, sym, inter = fmt[0], fmt[1] or k, fmt[2], fmt[3] == "interleaved"
        for m in (1, 5):
            x = to_gpu(torch, activations(m, k, seed=m))
            y = torch.empty(m, n, dtype=torch.float16, device="cuda")
            st = lib.dq_gemv(x.data_ptr(), pw.qweight.data_ptr(), pw.scales.data_ptr(),
                             None if sym else pw.zeros.data_ptr(), y.data_ptr(), m, n, k, bits, gs,
                             int(sym), int(inter), stream)
            assert st == 0, lib.dq_last_error()
            assert torch.equal(y, ext().gemv(x, *ext_args(pw)))
        out = torch.empty(n, k, dtype=torch.float16, device="cuda")
        st = lib.dq_dequantize(pw.qweight.data_ptr(), pw.scales.data_ptr(),
                               None if sym else pw.zeros.data_ptr(), out.data_ptr(), n, k, bits, gs, int(sym),
                               int(inter), stream)
        assert st == 0 and torch.equal(out, ext().dequantize(*ext_args(pw), k))
        codes = torch.empty(n, k, dtype=torch.int32, device="cuda")
        st = lib.dq_unpack(pw.qweight.data_ptr(), codes.data_ptr(), n, k, bits, int(inter), stream)
        assert st == 0 and torch.equal(codes, ext().unpack(pw.qweight, bits, inter, k))
    a = torch.arange(1000, dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    assert lib.dq_add_one(a.data_ptr(), b.data_ptr(), 1000, stream) == 0
    torch.cuda.synchronize()
    assert torch.equal(b, a + 1)


# ------------------------------------------------------- grouped launch
GROUPED_VS_SINGLE_REL_L2 = 1e-4


@pytest.mark.parametrize("m", (1, 3, 8))
def test_grouped_launch_matches_oracle_and_single_calls(torch_gpu, m):
    """dq_gemv_batched: one launch; every problem within the oracle tolerances,
    deterministic, and equal to its single call up to split-K fp32 rounding.

    GROUPED_VS_SINGLE_REL_L2: a grouped launch may split a tile's K over a
    different number of waves than the single call, which changes the fp32
    summation order; the M = 1 kernel sums (bias + q) x products, with a
    bias of 64 (INT4), 4 (INT2) or 1024 (INT8) that cancels only
    at the end, so about 0.3% of the fp16 outputs round to the neighbouring
    value (rel-L2 ~2e-5). 1e-4 still sits 10x below the oracle's 1e-3."""
    torch = torch_gpu
    specs = [(4096, 4096, 128), (1024, 4096, 128), (1024, 4096, 128),   # q | k | v
             (14336, 4096, 128), (4096, 14336, 128),                    # mixed K in one launch
             (37, 256, 64), (3, 4096, None)]                             # ragged N, group 64, per-channel
    pws, xs, cases, x16s = [], [], [], []
    for i, (n, k, gs) in enumerate(specs):
        pw, qw, sc, ze = pack_on_gpu(torch, gauss_weight(n, k, seed=40 + i), 4, gs, False, "sequential")
        rows = None if n <= 1024 else np.sort(np.random.Generator(np.random.PCG64(i)).choice(n, 512, replace=False))
        pws.append(pw)
        cases.append(OracleCase(pw, qw, sc, ze, rows))
        x16s.append(activations(m, k, seed=50 + i))
        xs.append(to_gpu(torch, x16s[-1]))
    args = ([p.qweight for p in pws], [p.scales for p in pws], [p.zeros for p in pws], 4,
            [p.config.effective_group_size(p.shape[1]) for p in pws], False, False)
    ys = ext().gemv_batched(xs, *args)
    again = ext().gemv_batched(xs, *args)
    for i, (x, pw) in enumerate(zip(xs, pws)):
        assert torch.equal(ys[i], again[i]), f"problem {i}: grouped launch not deterministic"
        cases[i].check(ys[i].cpu().numpy(), x16s[i], f"grouped problem {i} M={m}")
        single = ext().gemv(x, *ext_args(pw)).float()
        diff = (ys[i].float() - single).norm() / single.norm().clamp_min(1e-30)
        assert diff <= GROUPED_VS_SINGLE_REL_L2, f"problem {i}: grouped vs single rel-L2 {float(diff):.2e}"


def test_grouped_launch_sixteen_problems_and_python_api(torch_gpu):
    torch = torch_gpu
    from dequant_project_amd.quant_linear import gemv, gemv_grouped

    pws = [pack_on_gpu(torch, gauss_weight(512 + 64 * i, 2048, seed=60 + i), 2, 64, True, "interleaved")[0]
           for i in range(16)]
    xs = [to_gpu(torch, activations(1, 2048, seed=70 + i)).view(1, 1, 2048) for i in range(16)]
    ys = gemv_grouped(xs, pws)
    for y, x, pw in zip(ys, xs, pws):
        assert y.shape == (1, 1, pw.shape[0])
        single = gemv(x, pw).float()
        assert (y.float() - single).norm() <= GROUPED_VS_SINGLE_REL_L2 * single.norm()
    with pytest.raises(RuntimeError, match="1..16 problems"):
        ext().gemv_batched(xs * 2, [p.qweight for p in pws] * 2, [p.scales for p in pws] * 2, [None] * 32, 2,
                           [64] * 32, True, True)


@pytest.mark.parametrize("bits,gs,sym,n,k,count", [
    (4, 128, False, 12000, 4096, 8),   # R = 8 tiles
    (2, 64, False, 8000, 14336, 6),    # R = 4 tiles, 224 chunks per row (3.5 batches)
    (8, None, True, 8000, 4096, 10),   # per-channel INT8
    (2, 64, False, 4093, 4096, 16),    # INT2 rows under 8192 codes, last 8-row tile partial
    (2, 64, False, 28672, 8192, 2),    # INT2 pipelined at under two rounds (the C5
                                       # gate | up launch: 1792 block-tiles)
    (2, 64, False, 8165, 8192, 16),    # INT2 pipelined over 4084 block-tiles of two
                                       # batches, ~4 rounds; each problem's last
                                       # block-tile holds one 5-row tile and three
                                       # waves that only stage activations
])
def test_grouped_launch_over_several_rounds(torch_gpu, bits, gs, sym, n, k, count):
    """M = 1 launches with more block-tiles than the persistent grid holds
    (1792-4096 block-tiles against at most ~2000 resident blocks), so blocks
    walk several rounds and cross problem boundaries mid-walk; the INT2 cases
    of K = 8192 (every tile one wave wide, two batches per tile) run the
    pipelined walk over up to about four rounds of its grid. Every problem
    against the oracle on a sample of rows that includes each problem's last
    40 rows, and against its single call (a launch of its own geometry)."""
    torch = torch_gpu
    from dequant_project_amd.packer import QuantConfig, quantize_tensor

    gen = torch.Generator(device="cuda").manual_seed(bits * 1000 + count)
    cfg = QuantConfig(bits, gs, sym, "sequential")
    pws, cases, xs, x16s = [], [], [], []
    for i in range(count):
        pw = quantize_tensor(torch.randn(n, k, generator=gen, device="cuda", dtype=torch.float16) * 0.02, cfg)
        rng = np.random.Generator(np.random.PCG64(i))
        rows = np.unique(np.concatenate([rng.choice(n - 40, 200, replace=False), np.arange(n - 40, n)]))
        qw, sc = pw.qweight.cpu().numpy(), pw.scales.cpu().numpy()
        ze = None if pw.zeros is None else pw.zeros.cpu().numpy()
        cases.append(OracleCase(pw, qw, sc, ze, rows, deq_ref=False))
        x16s.append(activations(1, k, seed=90 + i))
        xs.append(to_gpu(torch, x16s[-1]))
        pws.append(pw)
    ys = ext().gemv_batched(xs, [p.qweight for p in pws], [p.scales for p in pws], [p.zeros for p in pws], bits,
                            [p.config.effective_group_size(k) for p in pws], sym, False)
    for i, (x, pw) in enumerate(zip(xs, pws)):
        cases[i].check(ys[i].cpu().numpy(), x16s[i], f"INT{bits} [{n},{k}] x{count} problem {i}")
        single = ext().gemv(x, *ext_args(pw)).float()
        diff = (ys[i].float() - single).norm() / single.norm().clamp_min(1e-30)
        assert diff <= GROUPED_VS_SINGLE_REL_L2, f"problem {i}: grouped vs single rel-L2 {float(diff):.2e}"


def _plan(shapes, bits, gs, m=1):
    import ctypes

    from dequant_project_amd import _native
    arr = (_native.DqGemvProblem * len(shapes))()
    for i, (n, k) in enumerate(shapes):
        arr[i].N, arr[i].K, arr[i].group_size = n, k, gs or k
    wk, rows, kind = (ctypes.c_int * len(shapes))(), ctypes.c_int(), ctypes.c_int()
    assert _native.capi().dq_gemv_plan(arr, len(shapes), m, bits, wk, ctypes.byref(rows), ctypes.byref(kind)) == 0
    return list(wk), rows.value, kind.value


@pytest.mark.parametrize("bits,gs,sym,layout,shapes,rows_per_tile", [
    # INT4 g32 sym interleaved, 8-row tiles: ragged row counts (each problem's
    # last block-tile has empty wave slots), K of 160 / 96 / 33 chunks (partial
    # last batches), a one-row problem, and different x per problem
    (4, 32, True, "interleaved", [(5003, 5120), (7001, 3072), (9999, 5120), (30005, 1056), (1, 5120),
                                  (20000, 4096)], 8),
    # INT4 g128 asym sequential, 4-row tiles (the decode gate | up launch)
    (4, 128, False, "sequential", [(14336, 4096), (14336, 4096)], 4),
    # INT8 per-channel sym interleaved, 4-row tiles, plus a five-row problem
    (8, None, True, "interleaved", [(11008, 4096), (11008, 4096), (11008, 4096), (5, 4096)], 4),
    # INT8 g64 asym sequential, 8-row tiles over K = 14336 (seven batches per tile)
    (8, 64, False, "sequential", [(4100, 14336)] * 16, 8),
    # INT2 g64 asym, 4-row tiles: the C4 decode gate | up launch
    (2, 64, False, "sequential", [(14336, 4096), (14336, 4096)], 4),
    # INT2 g128 sym interleaved, 4-row tiles, K of 120 / 64 / 2 chunks, ragged rows
    (2, 128, True, "interleaved", [(9001, 7680), (5003, 4096), (777, 128), (2, 7680), (3000, 4096)], 4),
])
def test_pipelined_m1_kernel_walk(torch_gpu, bits, gs, sym, layout, shapes, rows_per_tile):
    """gemv_m1_pipe_kernel (kind 4 of dq_gemv_plan): the walk that issues the
    next batch's rows while the current batch is computed, crossing tiles and
    problems, with the activations staged per block in pair order. Every
    problem against the oracle on a sample of rows that includes its last 40,
    and against its single call."""
    torch = torch_gpu
    from dequant_project_amd.packer import QuantConfig, quantize_tensor

    wk, r, kind = _plan(shapes, bits, gs)
    assert (wk, r, kind) == ([1] * len(shapes), rows_per_tile, 4)
    gen = torch.Generator(device="cuda").manual_seed(bits * 7 + len(shapes))
    cfg = QuantConfig(bits, gs, sym, layout)
    pws, cases, xs, x16s = [], [], [], []
    for i, (n, k) in enumerate(shapes):
        pw = quantize_tensor(torch.randn(n, k, generator=gen, device="cuda", dtype=torch.float16) * 0.02, cfg)
        rng = np.random.Generator(np.random.PCG64(500 + i))
        rows = np.unique(np.concatenate([rng.choice(n, min(n, 160), replace=False), np.arange(max(0, n - 40), n)]))
        qw, sc = pw.qweight.cpu().numpy(), pw.scales.cpu().numpy()
        ze = None if pw.zeros is None else pw.zeros.cpu().numpy()
        cases.append(OracleCase(pw, qw, sc, ze, rows, deq_ref=False))
        x16s.append(activations(1, k, seed=600 + i))
        xs.append(to_gpu(torch, x16s[-1]))
        pws.append(pw)
    args = ([p.qweight for p in pws], [p.scales for p in pws], [p.zeros for p in pws], bits,
            [p.config.effective_group_size(p.shape[1]) for p in pws], sym, layout == "interleaved")
    ys = ext().gemv_batched(xs, *args)
    again = ext().gemv_batched(xs, *args)
    for i, (x, pw) in enumerate(zip(xs, pws)):
        assert torch.equal(ys[i], again[i]), f"problem {i}: not deterministic"
        cases[i].check(ys[i].cpu().numpy(), x16s[i], f"pipelined INT{bits} {shapes[i]} problem {i}")
        single = ext().gemv(x, *ext_args(pw)).float()
        diff = (ys[i].float() - single).norm() / single.norm().clamp_min(1e-30)
        assert diff <= GROUPED_VS_SINGLE_REL_L2, f"problem {i}: grouped vs single rel-L2 {float(diff):.2e}"


@pytest.mark.parametrize("bits,gs,sym,layout,shapes,wk", [
    # INT4 g128 asym: two K shares of one batch each, three problems
    (4, 128, False, "sequential", [(600, 4096), (500, 4096), (300, 4096)], 2),
    # INT4 g128 asym: four shares of 112 columns (a full and a 48-column
    # batch each), ragged row counts
    (4, 128, False, "sequential", [(500, 14336), (262, 14336)], 4),
    # INT4 g32 sym interleaved: four shares of 40 columns (one partial
    # batch), a one-row problem
    (4, 32, True, "interleaved", [(600, 5120), (333, 5120), (1, 5120)], 4),
    # INT8 g128 sym interleaved and per-channel sym: four shares of 48 columns
    (8, 128, True, "interleaved", [(700, 3072), (333, 3072)], 4),
    (8, None, True, "sequential", [(700, 3072), (333, 3072)], 4),
])
def test_pipelined_split_walk(torch_gpu, bits, gs, sym, layout, shapes, wk):
    """gemv_m1_pipe_split_kernel (kind 8 of dq_gemv_plan): the pipelined walk
    over K shares, the block staging every share's activations, the shares'
    sums meeting in LDS at each tile's end, crossing problems. Every problem
    against the oracle on a sample of rows that includes its last 40, against
    a second launch (bit-equal) and against its single call."""
    torch = torch_gpu
    from dequant_project_amd.packer import QuantConfig, quantize_tensor

    assert _plan(shapes, bits, gs) == ([wk] * len(shapes), 4, 8)
    gen = torch.Generator(device="cuda").manual_seed(bits * 13 + len(shapes) + wk)
    cfg = QuantConfig(bits, gs, sym, layout)
    pws, cases, xs, x16s = [], [], [], []
    for i, (n, k) in enumerate(shapes):
        pw = quantize_tensor(torch.randn(n, k, generator=gen, device="cuda", dtype=torch.float16) * 0.02, cfg)
        rng = np.random.Generator(np.random.PCG64(900 + i))
        rows = np.unique(np.concatenate([rng.choice(n, min(n, 160), replace=False), np.arange(max(0, n - 40), n)]))
        qw, sc = pw.qweight.cpu().numpy(), pw.scales.cpu().numpy()
        ze = None if pw.zeros is None else pw.zeros.cpu().numpy()
        cases.append(OracleCase(pw, qw, sc, ze, rows, deq_ref=False))
        x16s.append(activations(1, k, seed=950 + i))
        xs.append(to_gpu(torch, x16s[-1]))
        pws.append(pw)
    args = ([p.qweight for p in pws], [p.scales for p in pws], [p.zeros for p in pws], bits,
            [p.config.effective_group_size(p.shape[1]) for p in pws], sym, layout == "interleaved")
    ys = ext().gemv_batched(xs, *args)
    again = ext().gemv_batched(xs, *args)
    for i, (x, pw) in enumerate(zip(xs, pws)):
        assert torch.equal(ys[i], again[i]), f"problem {i}: not deterministic"
        cases[i].check(ys[i].cpu().numpy(), x16s[i], f"split walk INT{bits} {shapes[i]} problem {i}")
        single = ext().gemv(x, *ext_args(pw)).float()
        diff = (ys[i].float() - single).norm() / single.norm().clamp_min(1e-30)
        assert diff <= GROUPED_VS_SINGLE_REL_L2, f"problem {i}: grouped vs single rel-L2 {float(diff):.2e}"


@pytest.mark.parametrize("bits,gs,sym,layout,shapes,rows_per_tile,m", [
    # the pipelined M = 1 walk's launches (one-wave tiles) at 2 batch rows:
    # ragged rows, partial last batches, a one-row problem (INT4 g32, 8-row tiles)
    (4, 32, True, "interleaved", [(5003, 5120), (7001, 3072), (9999, 5120), (30005, 1056), (1, 5120),
                                  (20000, 4096)], 8, 2),
    (4, 128, False, "sequential", [(14336, 4096), (14336, 4096)], 4, 2),
    (8, None, True, "interleaved", [(11008, 4096), (11008, 4096), (11008, 4096), (5, 4096)], 4, 2),
    (8, 64, False, "sequential", [(4100, 14336)] * 16, 8, 2),
    (2, 64, False, "sequential", [(14336, 4096), (14336, 4096)], 4, 2),
    # INT2 symmetric with a K = 128 problem (two chunks per row: rows whose
    # codes sit mostly at the zero point have the smallest tolerance)
    (2, 128, True, "interleaved", [(9001, 7680), (5003, 4096), (777, 128), (2, 7680), (3000, 4096)], 4, 2),
])
def test_pipelined_batch_rows_walk(torch_gpu, bits, gs, sym, layout, shapes, rows_per_tile, m):
    """gemv_mx_pipe_kernel (kind 7 of dq_gemv_plan): the pipelined walk with
    two batch rows, each weight chunk dotted with both. Every problem against
    the oracle on a sample of rows that includes its last 40, both batch
    rows, and deterministic."""
    torch = torch_gpu
    from dequant_project_amd.packer import QuantConfig, quantize_tensor

    wk, r, kind = _plan(shapes, bits, gs, m)
    assert (wk, r, kind) == ([1] * len(shapes), rows_per_tile, 7)
    gen = torch.Generator(device="cuda").manual_seed(bits * 11 + len(shapes) + m)
    cfg = QuantConfig(bits, gs, sym, layout)
    pws, cases, xs, x16s = [], [], [], []
    for i, (n, k) in enumerate(shapes):
        pw = quantize_tensor(torch.randn(n, k, generator=gen, device="cuda", dtype=torch.float16) * 0.02, cfg)
        rng = np.random.Generator(np.random.PCG64(700 + i))
        rows = np.unique(np.concatenate([rng.choice(n, min(n, 160), replace=False), np.arange(max(0, n - 40), n)]))
        qw, sc = pw.qweight.cpu().numpy(), pw.scales.cpu().numpy()
        ze = None if pw.zeros is None else pw.zeros.cpu().numpy()
        cases.append(OracleCase(pw, qw, sc, ze, rows, deq_ref=False))
        x16s.append(activations(m, k, seed=800 + i))
        xs.append(to_gpu(torch, x16s[-1]))
        pws.append(pw)
    args = ([p.qweight for p in pws], [p.scales for p in pws], [p.zeros for p in pws], bits,
            [p.config.effective_group_size(p.shape[1]) for p in pws], sym, layout == "interleaved")
    ys = ext().gemv_batched(xs, *args)
    again = ext().gemv_batched(xs, *args)
    for i in range(len(pws)):
        assert torch.equal(ys[i], again[i]), f"problem {i}: not deterministic"
        cases[i].check(ys[i].cpu().numpy(), x16s[i], f"pipelined M={m} INT{bits} {shapes[i]} problem {i}")


def test_int2_shared_and_mixed_activations_across_tiles(torch_gpu):
    """An INT2 launch of one-batch 8-row tiles over more than two rounds of
    the grid, the case where each wave runs a contiguous range of tiles and
    reuses the activations of its previous tile when the next one reads the
    same columns of the same x: problems share one x tensor (consecutive and
    not), one reads only the first half of that tensor as a K = 2048 problem
    (same pointer, other columns: must load again), others have their own x,
    and row counts are ragged. Every problem against the oracle (sampled rows
    including its last 40) and against its single call."""
    torch = torch_gpu
    from dequant_project_amd.packer import QuantConfig, quantize_tensor

    gen = torch.Generator(device="cuda").manual_seed(2024)
    cfg = QuantConfig(2, 64, False, "sequential")
    x_a16, x_b16, x_c16 = (activations(1, 4096, seed=s) for s in (301, 302, 303))
    x_a, x_b, x_c = (to_gpu(torch, v) for v in (x_a16, x_b16, x_c16))
    # (rows, x source, K): 'a2' = the first 2048 columns of x_a (a view, same data pointer)
    plan = [(6000, "a", 4096), (5003, "a", 4096), (4000, "a2", 2048), (7001, "b", 4096), (6003, "a", 4096),
            (2000, "a2", 2048), (8000, "c", 4096), (7999, "c", 4096), (5000, "b", 4096), (6000, "a", 4096),
            (3005, "a2", 2048), (12000, "b", 4096), (7000, "c", 4096)]
    srcs = {"a": (x_a, x_a16), "b": (x_b, x_b16), "c": (x_c, x_c16),
            "a2": (x_a[:, :2048], x_a16[:, :2048].copy())}
    pws, cases, xs, x16s = [], [], [], []
    for i, (n, src, k) in enumerate(plan):
        pw = quantize_tensor(torch.randn(n, k, generator=gen, device="cuda", dtype=torch.float16) * 0.02, cfg)
        rng = np.random.Generator(np.random.PCG64(400 + i))
        rows = np.unique(np.concatenate([rng.choice(n - 40, 160, replace=False), np.arange(n - 40, n)]))
        qw, sc, ze = pw.qweight.cpu().numpy(), pw.scales.cpu().numpy(), pw.zeros.cpu().numpy()
        cases.append(OracleCase(pw, qw, sc, ze, rows, deq_ref=False))
        xs.append(srcs[src][0])
        x16s.append(srcs[src][1])
        pws.append(pw)
    assert xs[2].data_ptr() == x_a.data_ptr() and xs[2].is_contiguous()
    # the variant's preconditions: 8-row tiles, one wave per tile; 2469 block-tiles
    # against a grid of 4 blocks per CU (two rounds on a 256-CU device)
    import ctypes

    from dequant_project_amd import _native
    arr = (_native.DqGemvProblem * len(plan))()
    for i, (n, _, k) in enumerate(plan):
        arr[i].N, arr[i].K, arr[i].group_size = n, k, 64
    wk, rows_per_tile, kind = (ctypes.c_int * len(plan))(), ctypes.c_int(), ctypes.c_int()
    assert _native.capi().dq_gemv_plan(arr, len(plan), 1, 2, wk, ctypes.byref(rows_per_tile), ctypes.byref(kind)) == 0
    assert (list(wk), rows_per_tile.value, kind.value) == ([1] * len(plan), 8, 6)
    assert sum((n + 7) // 8 for n, _, _ in plan) // 4 >= 2 * 4 * 256
    ys = ext().gemv_batched(xs, [p.qweight for p in pws], [p.scales for p in pws], [p.zeros for p in pws], 2,
                            [p.config.effective_group_size(p.shape[1]) for p in pws], False, False)
    for i, (x, pw) in enumerate(zip(xs, pws)):
        cases[i].check(ys[i].cpu().numpy(), x16s[i], f"INT2 {plan[i]} problem {i}")
        single = ext().gemv(x, *ext_args(pw)).float()
        diff = (ys[i].float() - single).norm() / single.norm().clamp_min(1e-30)
        assert diff <= GROUPED_VS_SINGLE_REL_L2, f"problem {i}: grouped vs single rel-L2 {float(diff):.2e}"


def test_launch_event_hook_times_the_kernel(torch_gpu):
    torch = torch_gpu
    from dequant_project_amd import _native

    lib = _native.capi()
    pw, *_ = pack_on_gpu(torch, gauss_weight(8192, 4096, seed=3), 4, 128, False, "sequential")
    x = to_gpu(torch, activations(1, 4096, seed=3))
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    e1.record()
    assert lib.dq_set_launch_events(e0.cuda_event, e1.cuda_event) == 0
    y = ext().gemv(x, *ext_args(pw))
    e1.synchronize()
    ms = e0.elapsed_time(e1)
    assert 0.0 < ms < 50.0
    assert torch.equal(y, ext().gemv(x, *ext_args(pw)))  # the hook changes timing only


def test_measurement_kernels(torch_gpu):
    """dq_stream_read reads its buffer and leaves the sink alone for real
    data; dq_empty_kernel launches; both validate their arguments."""
    torch = torch_gpu
    from dequant_project_amd import _native

    lib = _native.capi()
    stream = torch.cuda.current_stream().cuda_stream
    buf = torch.randint(-2**31, 2**31 - 1, (1 << 24,), dtype=torch.int32, device="cuda")
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    assert lib.dq_stream_read(buf.data_ptr(), buf.numel() * 4, sink.data_ptr(), stream) == 0
    assert lib.dq_stream_read(buf.data_ptr(), 4096 + 16, sink.data_ptr(), stream) == 0  # a short tail
    assert lib.dq_empty_kernel(stream) == 0
    torch.cuda.synchronize()
    assert int(sink.abs().sum()) == 0
    assert lib.dq_stream_read(buf.data_ptr(), 24, sink.data_ptr(), stream) == 1
    assert b"multiple of 16" in lib.dq_last_error()
    assert lib.dq_stream_read(buf.data_ptr() + 4, 32, sink.data_ptr(), stream) == 1
    assert b"16-byte aligned" in lib.dq_last_error()


@pytest.mark.parametrize("m", (1, 4, 16))
def test_weights_past_two_gib_run_as_row_slices(torch_gpu, m):
    """An INT8 per-channel weight of 140000 x 16384 (2.29 GB of qweight, past
    the kernels' 32-bit buffer offsets; a 140k-token vocabulary's lm_head):
    the C ABI launches it as two row slices (131008 rows, then the rest),
    each writing its own columns of y with the whole y's row stride. Rows on both sides of the cut and the last
    rows against the oracle, for the M = 1 kernel, the 2 <= M <= 8 kernel and
    the small GEMM."""
    torch = torch_gpu
    from dequant_project_amd.packer import QuantConfig, quantize_tensor

    n, k = 140000, 16384
    gen = torch.Generator(device="cuda").manual_seed(77)
    w = torch.randn(n, k, generator=gen, device="cuda", dtype=torch.float16) * 0.02
    pw = quantize_tensor(w, QuantConfig(8, None, True))
    del w
    assert pw.qweight.numel() * 4 >= 2 ** 31
    rows = np.unique(np.concatenate([np.arange(0, 24), np.arange(131000, 131016), np.arange(n - 40, n),
                                     np.random.Generator(np.random.PCG64(78)).choice(n, 64, replace=False)]))
    ridx = torch.from_numpy(rows).cuda()
    qw = pw.qweight[ridx].cpu().numpy()
    sc = pw.scales[ridx].cpu().numpy()
    cfg = P.Config(8, None, True, "sequential")
    # the GEMV multiplies by exact (q - z) * s; the small GEMM, like the
    # reference's M > 8 path, by packer.dequantize's fp16 weight
    if m <= 8:
        w64 = P.exact_weight(qw, sc, None, cfg, (len(rows), k)).astype(np.float64)
    else:
        w64 = P.dequantize(qw, sc, None, cfg, (len(rows), k)).astype(np.float64)
    x16 = activations(m, k, seed=79)
    x = to_gpu(torch, x16)
    if m <= 8:
        y = ext().gemv(x, *ext_args(pw))
    else:
        y = ext().gemm_small(x, *ext_args(pw))
    assert tuple(y.shape) == (m, n)
    y = y[:, ridx].cpu().numpy()
    x64 = x16.astype(np.float64)
    ref, absref = x64 @ w64.T, np.abs(x64) @ np.abs(w64).T
    ok, worst = P.gemv_criterion(y, ref, absref)
    print(f"2.29 GB INT8 weight M={m}: worst={worst:.3f}x tol rel_l2={P.rel_l2(y, ref):.2e}", flush=True)
    assert ok, f"elementwise criterion violated, worst {worst:.3f}x"
    assert P.rel_l2(y, ref) <= REL_L2_TOL


@pytest.mark.parametrize("bits,gs,sym,n,k,plan", [
    (4, 128, False, 2044, 4096, ([2], 4, 8)),   # 511 four-row tiles: the K split stays (pipelined)
    (4, 128, False, 2048, 4096, ([1], 4, 4)),   # 512: one-wave tiles, pipelined
    (4, 128, False, 4096, 4096, ([1], 4, 4)),   # 1024: the last one-wave size
    (4, 128, False, 4100, 4096, ([2], 4, 8)),   # 1025: the K split again (513 block-tiles)
    (4, 128, False, 8200, 4096, ([2], 4, 2)),   # 2050 tiles x 2 waves: gemv_m1_kernel's split
    (4, 128, False, 8184, 8192, ([4], 4, 2)),   # K = 8192, 1023 eight-row tiles: four-row split
    (4, 128, False, 8192, 8192, ([4], 8, 2)),   # 1024 eight-row tiles: eight-row split
    (2, 64, False, 2044, 14336, ([4], 4, 2)),   # INT2 under 512 tiles: split
    (2, 64, False, 2048, 14336, ([1], 4, 4)),   # INT2 from 512 tiles: pipelined
    (8, None, True, 4096, 4096, ([1], 4, 4)),   # INT8 per-channel, 1024 tiles
    (8, None, True, 4100, 4096, ([4], 4, 2)),
])
def test_launch_geometry_thresholds(torch_gpu, bits, gs, sym, n, k, plan):
    """M = 1 launches on both sides of each geometry threshold (one-wave tiles
    for 512..1024 four-row tiles and for INT2 from 512 tiles, eight-row
    tiles for 1024+ of them at K >= 8192): the plan the launch takes, and its
    output against the oracle on a sample of rows that includes the last 40."""
    torch = torch_gpu
    from dequant_project_amd.packer import QuantConfig, quantize_tensor

    assert _plan([(n, k)], bits, gs) == plan
    gen = torch.Generator(device="cuda").manual_seed(n + k + bits)
    pw = quantize_tensor(torch.randn(n, k, generator=gen, device="cuda", dtype=torch.float16) * 0.02,
                         QuantConfig(bits, gs, sym, "sequential"))
    rng = np.random.Generator(np.random.PCG64(n))
    rows = np.unique(np.concatenate([rng.choice(n - 40, 160, replace=False), np.arange(n - 40, n)]))
    qw, sc = pw.qweight.cpu().numpy(), pw.scales.cpu().numpy()
    ze = None if pw.zeros is None else pw.zeros.cpu().numpy()
    case = OracleCase(pw, qw, sc, ze, rows, deq_ref=False)
    x16 = activations(1, k, seed=n + 3)
    y = ext().gemv(to_gpu(torch, x16), *ext_args(pw))
    case.check(y.cpu().numpy(), x16, f"INT{bits} [{n},{k}] plan {plan}")
