"""Fused activation prologues on MI355X (dequant_project_amd.fused, the C ABI's
dq_gemv_prologue_batched) against the CPU oracle.

  gemv_rmsnorm  y_i = W_i (rmsnorm(x) * gamma) for one row; reference: the
                fp64 product of exact_weight with oracle.prologue_ref.rmsnorm64
                (and with the unfused fp16 module's output, rmsnorm_fp16)
  gemv_swiglu   y = W (silu(gate) * up); reference: exact_weight times
                swiglu64 (and times the unfused fp16 composition, swiglu_fp16)
Tolerance: the north star's GEMV bound, rel-L2 <= 1e-3, against both. The
fused path differs from the unfused one only in where the activations are
rounded to fp16, which bounds it near 2^-11 relative.
"""

import numpy as np
import pytest

from oracle import packer_ref as P
from oracle import prologue_ref as R
from tests._helpers import activations, gauss_weight, rng
from tests.test_kernels_gpu import pack_on_gpu, to_gpu

pytestmark = pytest.mark.gpu

REL_L2_TOL = 1e-3
EPS = 1e-5
FORMATS = [(4, 128, False, "sequential"), (2, 64, False, "interleaved"), (8, None, True, "sequential"),
           (4, 32, True, "interleaved")]


def exact64(pw, qw, sc, ze):
    cfg = P.Config(pw.config.bits, pw.config.group_size, pw.config.symmetric, pw.config.layout)
    return P.exact_weight(qw, sc, ze, cfg, pw.shape).astype(np.float64)


def check(y, refs, label):
    y = y.astype(np.float64)
    errs = [P.rel_l2(y, r) for r in refs]
    print(f"{label}: rel-L2 " + " / ".join(f"{e:.2e}" for e in errs), flush=True)
    assert np.isfinite(y).all(), label
    for e in errs:
        assert e <= REL_L2_TOL, f"{label}: rel-L2 {e:.3e} > {REL_L2_TOL}"


def packed_group(torch, n, k, count, fmt, seed):
    out = []
    for i in range(count):
        pw, qw, sc, ze = pack_on_gpu(torch, gauss_weight(n, k, seed=seed + i), *fmt)
        out.append((pw, exact64(pw, qw, sc, ze)))
    return out


# (N, K, problems): split-K tiles (one small problem) and full-K tiles (a
# 16-problem launch), K = 11008 (172 INT2 chunks: a ragged last column), two
# problems of one-wave 4-row tiles (the decode step's gate | up shape class:
# RMSNorm on the pipelined kernel, the prologue staged per block), and three
# problems of 1536 four-row tiles (the q|k|v class: RMSNorm launches of up to
# 2048 tiles take one-wave tiles too)
SHAPES = [(256, 4096, 1), (1000, 2048, 3), (4096, 4096, 16), (300, 11008, 2), (12288, 1024, 2), (2048, 4096, 3)]


@pytest.mark.parametrize("n,k,count", SHAPES)
def test_gemv_rmsnorm_matches_oracle(torch_gpu, n, k, count):
    torch = torch_gpu
    from dequant_project_amd.fused import gemv_rmsnorm

    x = activations(1, k, seed=k + count)
    gamma = (1.0 + 0.2 * rng(k + 7).standard_normal(k)).astype(np.float16)
    h64 = R.rmsnorm64(x, gamma, EPS)
    h16 = R.rmsnorm_fp16(x, gamma, EPS).astype(np.float64)
    for fmt in FORMATS:
        if fmt[1] and k % fmt[1]:
            continue
        group = packed_group(torch, n, k, count, fmt, seed=n + k)
        ys = gemv_rmsnorm(to_gpu(torch, x), to_gpu(torch, gamma), EPS, [pw for pw, _ in group])
        for i, ((pw, w64), y) in enumerate(zip(group, ys)):
            assert tuple(y.shape) == (1, n)
            check(y.cpu().numpy(), [h64 @ w64.T, h16 @ w64.T], f"rmsnorm {fmt} [{n},{k}] problem {i}/{count}")


@pytest.mark.parametrize("n,k,count", SHAPES)
def test_gemv_swiglu_matches_oracle(torch_gpu, n, k, count):
    torch = torch_gpu
    from dequant_project_amd import fused

    gate = (rng(k).standard_normal((1, k)) * 2.5).astype(np.float16)
    up = activations(1, k, seed=k + 1)
    h64 = R.swiglu64(gate, up)
    h16 = R.swiglu_fp16(gate, up).astype(np.float64)
    for fmt in FORMATS:
        if fmt[1] and k % fmt[1]:
            continue
        group = packed_group(torch, n, k, count, fmt, seed=3 * n + k)
        for i, (pw, w64) in enumerate(group):
            y = fused.gemv_swiglu(to_gpu(torch, gate), to_gpu(torch, up), pw)
            check(y.cpu().numpy(), [h64 @ w64.T, h16 @ w64.T], f"swiglu {fmt} [{n},{k}] problem {i}")


@pytest.mark.parametrize("scale", ["residual", "tiny"])
def test_gemv_rmsnorm_at_residual_stream_scales(torch_gpu, scale):
    """RMSNorm prologue on inputs shaped like a decoder's residual stream: a
    few outlier features in the thousands over N(0, 1) entries ("residual"),
    and a row of magnitude ~1e-3 ("tiny"). The fused form rounds x * gamma to
    fp16 before dividing by rms(x); both cases stay far inside fp16's range
    (|x * gamma| <= 65504), so it must match the unfused module."""
    torch = torch_gpu
    from dequant_project_amd.fused import gemv_rmsnorm

    n, k = 2048, 4096
    g = rng(41 if scale == "residual" else 42)
    x = g.standard_normal((1, k)).astype(np.float32)
    if scale == "residual":
        idx = g.choice(k, 8, replace=False)
        x[0, idx] = np.sign(g.standard_normal(8)) * g.uniform(1000.0, 6000.0, 8)
    else:
        x *= 1e-3
    x = x.astype(np.float16)
    gamma = (1.0 + 0.2 * g.standard_normal(k)).astype(np.float16)
    assert np.isfinite(x.astype(np.float32) * gamma.astype(np.float32)).all()
    h64 = R.rmsnorm64(x, gamma, EPS)
    h16 = R.rmsnorm_fp16(x, gamma, EPS).astype(np.float64)
    for fmt in FORMATS:
        (pw, w64), = packed_group(torch, n, k, 1, fmt, seed=43)
        (y,) = gemv_rmsnorm(to_gpu(torch, x), to_gpu(torch, gamma), EPS, [pw])
        check(y.cpu().numpy(), [h64 @ w64.T, h16 @ w64.T], f"rmsnorm {scale} {fmt}")


def test_prologues_with_zero_points_beyond_fp16_exact_range(torch_gpu):
    """The kernels' separate path for zero points outside [-1024, 1024]
    re-reads the activations: it must apply the prologue too."""
    torch = torch_gpu
    from dequant_project_amd import fused

    n, k = 256, 4096
    w = gauss_weight(n, k, seed=31).astype(np.float32)
    band = (np.arange(n) // 8) % 2 == 1
    w[band] = 50.0 + 0.5 * rng(32).random((int(band.sum()), k), dtype=np.float32)
    fmt = (4, 128, False, "sequential")
    pw, qw, sc, ze = pack_on_gpu(torch, w.astype(np.float16), *fmt)
    assert (np.abs(ze.astype(np.float32)[band]) > 1024).all()
    w64 = exact64(pw, qw, sc, ze)
    x = activations(1, k, seed=33)
    gamma = (1.0 + 0.2 * rng(34).standard_normal(k)).astype(np.float16)
    (y,) = fused.gemv_rmsnorm(to_gpu(torch, x), to_gpu(torch, gamma), EPS, [pw])
    check(y.cpu().numpy(), [R.rmsnorm64(x, gamma, EPS) @ w64.T], "rmsnorm wide zeros")
    gate = (rng(35).standard_normal((1, k)) * 2.5).astype(np.float16)
    y = fused.gemv_swiglu(to_gpu(torch, gate), to_gpu(torch, x), pw)
    check(y.cpu().numpy(), [R.swiglu64(gate, x) @ w64.T], "swiglu wide zeros")


def test_prologue_rejects_unsupported_calls(torch_gpu):
    torch = torch_gpu
    from dequant_project_amd import fused
    from dequant_project_amd.packer import QuantConfig, quantize_tensor

    pw = quantize_tensor(torch.randn(64, 256, device="cuda", dtype=torch.float16) * 0.02, QuantConfig(4, 128, False))
    x2 = torch.randn(2, 256, device="cuda", dtype=torch.float16)
    g = torch.ones(256, device="cuda", dtype=torch.float16)
    with pytest.raises(RuntimeError, match="fused prologues handle M = 1, got M=2"):
        fused.gemv_rmsnorm(x2, g, EPS, [pw])
    with pytest.raises(RuntimeError, match="aux must be a contiguous float16 tensor"):
        fused.gemv_rmsnorm(x2[:1], g[:128], EPS, [pw])
    with pytest.raises(RuntimeError, match="shaped like x"):
        fused.gemv_swiglu(x2[:1], x2, pw)


def test_fused_llama_decode_matches_unfused(torch_gpu):
    """fuse_llama on a small Llama: the decode step's logits match the same
    quantized model without fusion, graph replays match the eager step, and
    prefill (more than one row) runs the model's own modules."""
    torch = torch_gpu
    pytest.importorskip("transformers")
    import copy

    from dequant_project_amd import decode
    from dequant_project_amd.fused import fuse_llama
    from dequant_project_amd.packer import QuantConfig
    from dequant_project_amd.quant_linear import quantize_model

    for cfg in (QuantConfig(4, 128, False), QuantConfig(8, None, True)):
        model = decode.build_llama("tiny", seed=21)
        quantize_model(model, cfg)
        fused_model = copy.deepcopy(model)
        stats = fuse_llama(fused_model)
        assert stats == {"attention": 2, "mlp": 2}
        for seq_len in (8, 40):
            step, _, out = decode.decode_step_fn(model, seq_len)
            step()
            want = out["logits"].float()
            fstep, frestore, fout = decode.decode_step_fn(fused_model, seq_len)
            fstep()
            got = fout["logits"].float().clone()
            err = float((got.double() - want.double()).norm() / want.double().norm())
            print(f"fused {cfg} seq {seq_len}: logits rel-L2 {err:.2e}", flush=True)
            assert torch.isfinite(got).all() and err <= 2e-3
        frestore()
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            fstep()
            frestore()
        torch.cuda.current_stream().wait_stream(side)
        with torch.cuda.graph(graph):
            fstep()
        for _ in range(3):
            frestore()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(fout["logits"].float(), got)
            fstep()  # eager work between replays
            torch.cuda.synchronize()
