"""Pins oracle/cpu_path.py (the timed CPU baseline) to the reference's golden
vectors and to the numpy oracle."""

import numpy as np
import pytest
import torch

from oracle import cpu_path
from oracle import packer_ref as P
from tests._helpers import GOLDEN_CASES, activations, gauss_weight, golden, golden_tag


@pytest.mark.parametrize("bits,gs,sym,layout", GOLDEN_CASES, ids=[golden_tag(*c) for c in GOLDEN_CASES])
def test_cpu_path_matches_reference_golden(bits, gs, sym, layout):
    g = golden()
    t = golden_tag(bits, gs, sym, layout)
    n, k = g["w16"].shape
    qw = torch.from_numpy(g[t + "/qweight"].copy())
    sc = torch.from_numpy(g[t + "/scales"].view(np.float16).copy())
    ze = None if sym else torch.from_numpy(g[t + "/zeros"].view(np.float16).copy())
    inter = layout == "interleaved"
    assert np.array_equal(cpu_path.unpack(qw, bits, inter, k).numpy(), g[t + "/codes"])
    deq = cpu_path.dequantize(qw, sc, ze, bits, k if gs is None else gs, sym, inter, k)
    assert np.array_equal(deq.numpy().view(np.uint16), g[t + "/deq"])


def test_cpu_path_gemv_matches_numpy_oracle():
    n, k = 96, 1024
    for args in [(4, 128, False, "sequential"), (2, 64, True, "interleaved"), (8, None, True, "sequential")]:
        cfg = P.Config(*args)
        qw, sc, ze = P.quantize_tensor(gauss_weight(n, k, seed=4), cfg)
        x = activations(3, k, seed=5)
        y = cpu_path.gemv(torch.from_numpy(x), torch.from_numpy(qw), torch.from_numpy(sc),
                          None if ze is None else torch.from_numpy(ze), args[0], args[1] or k, args[2],
                          args[3] == "interleaved").numpy()
        want = x.astype(np.float32) @ P.dequantize(qw, sc, ze, cfg, (n, k)).astype(np.float32).T
        assert np.allclose(y, want, rtol=1e-5, atol=1e-5)
