"""Pins oracle/prologue_ref.py (CPU): closed forms, then the transformers
modules it restates run on CPU fp16 tensors."""

import numpy as np
import pytest
import torch

from oracle import prologue_ref as R
from tests._helpers import activations, rng


def test_rmsnorm_closed_forms():
    gamma = (1.0 + 0.1 * rng(1).standard_normal(64)).astype(np.float16)
    for c in (3.0, -0.25):
        h = R.rmsnorm64(np.full(64, c, dtype=np.float16), gamma, 0.0)
        np.testing.assert_allclose(h, np.sign(c) * gamma.astype(np.float64), rtol=1e-12)
    x = activations(1, 256, seed=2)[0]
    g = np.ones(256, dtype=np.float16)
    np.testing.assert_allclose(R.rmsnorm64(x.astype(np.float64) * 7.5, g, 0.0), R.rmsnorm64(x, g, 0.0), rtol=1e-12)
    h = R.rmsnorm64(x, g, 0.0)
    assert abs(np.mean(h * h) - 1.0) < 1e-12           # unit mean square
    # eps enters under the root: a zero vector stays zero, a tiny one is damped
    assert np.all(R.rmsnorm64(np.zeros(8, np.float16), np.ones(8, np.float16), 1e-5) == 0.0)


def test_silu_closed_forms():
    from scipy.special import expit

    g = np.linspace(-30, 30, 1001)
    np.testing.assert_allclose(R.silu64(g), g * expit(g), rtol=1e-13, atol=1e-300)
    assert R.silu64(np.array([0.0]))[0] == 0.0
    u = rng(3).standard_normal(1001)
    np.testing.assert_allclose(R.swiglu64(g, u), g * expit(g) * u, rtol=1e-13, atol=1e-300)


def ulps16(a, b):
    ia = a.view(np.int16).astype(np.int32)
    ib = b.view(np.int16).astype(np.int32)
    ia = np.where(ia < 0, -32768 - ia, ia)
    ib = np.where(ib < 0, -32768 - ib, ib)
    return np.abs(ia - ib)


@pytest.mark.parametrize("k", [64, 4096, 14336])
def test_rmsnorm_fp16_matches_transformers(k):
    transformers = pytest.importorskip("transformers")
    from transformers.models.llama.modeling_llama import LlamaRMSNorm

    x = activations(4, k, seed=k)
    gamma = (1.0 + 0.1 * rng(k + 1).standard_normal(k)).astype(np.float16)
    norm = LlamaRMSNorm(k, eps=1e-5)
    with torch.no_grad():
        norm.weight.copy_(torch.from_numpy(gamma))
        want = norm.half()(torch.from_numpy(x)).numpy()
    got = R.rmsnorm_fp16(x, gamma, 1e-5)
    d = ulps16(got, want)
    assert d.max() <= 1 and (d == 0).mean() > 0.99, (d.max(), (d == 0).mean())


def test_swiglu_fp16_matches_torch():
    g = (rng(5).standard_normal((4, 4096)) * 3).astype(np.float16)
    u = activations(4, 4096, seed=6)
    g[0, :4] = [-70000 / 7, 12.0, -12.0, 0.0]  # saturating ends
    want = (torch.nn.functional.silu(torch.from_numpy(g)) * torch.from_numpy(u)).numpy()
    got = R.swiglu_fp16(g, u)
    d = ulps16(got, want)
    # silu values that fall within an fp32 ulp of an fp16 rounding tie may round
    # the other way (torch's exp differs from numpy's in the last fp32 bit); the
    # product with up can then move by two ulps
    assert d.max() <= 2 and (d == 0).mean() > 0.99, (d.max(), (d == 0).mean())
