"""The M = 1 kernels' accumulation with biased codes, modelled on the CPU.

dq_kernels.hip (biased_pairs / bias_sums / biased_dot_m1 /
tile_math_m1_sums) multiplies each activation pair by fp16 (bias + q) codes,
exactly, and sums in fp32 with v_dot2_f32_f16 (one rounding per pair step);
per lane and batch it takes S = sum(x) and C = sum(bias * x) over the same
pairs, subtracts C + z S (one fma, one subtraction), folds the group scale
in with an fma per batch, and reduces the 64 lanes in fp32. The bias terms
cancel only in that subtraction, so the sums' rounding error grows with the
bias; the kernels place the codes high in the fp16 mantissa (INT4 bias 64,
INT2 16 / 4 by pair, INT8 1024).

This model follows that order in numpy (float64 arithmetic, rounded to fp32
where the kernel rounds) and checks the accumulation error against the fp32
part of the reference kernel test's criterion, 2^-20 * sum |w||x|
(scripts/test_dequant_kernel.py:112-122), before the fp16 output rounding,
and, at small K, against the whole criterion (that term plus the fp16
output's 2^-11 |ref|, of which half is left after the output rounding).
Rejected placements show the model separates them: INT4's low nibble at
bit 0 (bias 1024), and INT2's codes at bits 4 / 6 / 8 (bias 64 / 16 / 4),
which fails the whole criterion at K <= 256.
"""
import numpy as np
import pytest

from oracle import packer_ref as P

F32 = np.float32


def _f32(v):
    return np.asarray(v, dtype=np.float64).astype(F32).astype(np.float64)


def _model(q, zk, sk, x, bits, bias_of_pair):
    """fp32 result per row of the biased-code summation (rows vectorized).
    q: codes [n, k] (logical order), zk / sk: zero / scale per chunk [n, nch],
    x: activations [k] (fp16 values), bias_of_pair: bias of pair i's slots."""
    n, k = q.shape
    per, cpl = 32 // bits, 128 // bits
    half = per // 2
    nch = k // cpl
    bias_slot = np.array([bias_of_pair(s % half) for s in range(per)], dtype=np.float64)
    qb = (q.astype(np.float64) + np.tile(bias_slot, k // per)[None, :]).reshape(n, nch, 4, per)
    xv = x.reshape(nch, 4, per)
    classes = sorted({bias_of_pair(i) for i in range(half)}, reverse=True)
    dot = np.zeros((n, nch))
    sc = {b: np.zeros(nch) for b in classes}
    for j in range(4):
        for i in range(half):
            dot = _f32(dot + qb[:, :, j, i] * xv[None, :, j, i] + qb[:, :, j, i + half] * xv[None, :, j, i + half])
            b = bias_of_pair(i)
            sc[b] = _f32(sc[b] + xv[:, j, i] + xv[:, j, i + half])
    S = sc[classes[0]]
    C = _f32(classes[0] * sc[classes[0]])
    for b in classes[1:]:
        S = _f32(S + sc[b])
        C = _f32(b * sc[b] + C)
    v = _f32(dot - _f32(zk * S[None, :] + C[None, :]))
    lanes = np.zeros((n, 64))
    for c0 in range(0, nch, 64):  # lane l holds chunk column c0 + l of each batch
        c1 = min(nch, c0 + 64)
        lanes[:, :c1 - c0] = _f32(sk[:, c0:c1] * v[:, c0:c1] + lanes[:, :c1 - c0])
    while lanes.shape[1] > 1:
        h = lanes.shape[1] // 2
        lanes = _f32(lanes[:, :h] + lanes[:, h:])
    return lanes[:, 0]


def _case(n, k, bits, gs, sym, bias_of_pair, seed, full=False):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float16)
    cfg = P.Config(bits, gs, sym, "sequential")
    q, sc, ze = P.quantize(w, cfg)
    g = cfg.effective_group_size(k)
    s = sc.astype(np.float64)
    z = np.full_like(s, 1 << (bits - 1)) if sym else ze.astype(np.float64)
    x = rng.standard_normal(k).astype(np.float16).astype(np.float64)
    zfull, sfull = np.repeat(z, g, axis=1), np.repeat(s, g, axis=1)
    ref = ((q - zfull) * sfull) @ x
    budget = 2.0 ** -20 * ((np.abs(q - zfull) * sfull) @ np.abs(x))
    if full:
        budget = budget + 2.0 ** -12 * np.abs(ref)
    cpl = 128 // bits
    y = _model(q, np.repeat(z, g // cpl, axis=1), np.repeat(s, g // cpl, axis=1), x, bits, bias_of_pair)
    return float(np.max(np.abs(y - ref) / budget))


INT2_BIAS = [4.0, 16.0, 4.0, 16.0, 4.0, 16.0, 4.0, 4.0]  # Biased<2>::cls per pair: bits 8 / 6
INT2_BIAS_REJECTED = [64, 16, 64, 16, 4, 64, 16, 4]     # the earlier placement, bits 4 / 6 / 8 by pair


@pytest.mark.parametrize("n,k", [(512, 4096), (256, 14336)])
def test_biased_accumulation_within_the_fp32_budget(n, k):
    int4 = _case(n, k, 4, 128, False, lambda i: 64.0, seed=k + 1)
    int2 = _case(n, k, 2, 64, False, lambda i: INT2_BIAS[i], seed=k + 2)
    int8 = _case(n, k, 8, None, True, lambda i: 1024.0, seed=k + 3)
    exact = _case(n, k, 4, 128, False, lambda i: 0.0, seed=k + 1)
    # measured: INT4 0.12 / 0.05, INT2 0.05 / 0.02, INT8 0.13 / 0.07 of the budget (K = 4096 / 14336)
    assert int4 < 0.25 and int2 < 0.1 and int8 < 0.25, (int4, int2, int8)
    assert exact < int4  # the biases cost accuracy, none of it past the budget
    # the placement that was rejected: INT4 low nibble at bit 0 (bias 1024)
    low = _case(n, k, 4, 128, False, lambda i: 1024.0 if i % 2 == 0 else 64.0, seed=k + 1)
    assert low > 3 * int4, (low, int4)


@pytest.mark.parametrize("k", [128, 256])
def test_int2_small_k_within_the_whole_criterion(k):
    """INT2 at K of 2-4 chunks, symmetric (z = 2, most |q - z| <= 1) and
    asymmetric, against the reference kernel test's whole criterion: every
    element within a half of it (measured: at most 0.43), where the earlier
    placement exceeded it (measured: 4.4x at K = 128, 3.3x at K = 256)."""
    worst = max(_case(777, k, 2, gs, sym, lambda i: INT2_BIAS[i], seed=s, full=True)
                for gs, sym in ((64, False), (128, True)) for s in range(4))
    assert worst < 0.5, worst
    old = max(_case(777, k, 2, 128, True, lambda i: float(INT2_BIAS_REJECTED[i]), seed=s, full=True)
              for s in range(4))
    assert old > 1.0, old
