"""The product packer (dequant_project_amd.packer) on the CPU.

Restates the reference's scripts/test_packer.py (checks 1-7, :47-155) and adds
bit-exact equality with the reference's own outputs (tests/golden vectors) and
with the numpy oracle, so packed weights are interchangeable with the
reference's.
"""

import numpy as np
import pytest
import torch

from dequant_project_amd.packer import (QuantConfig, dequantize, pack, quantize, quantize_tensor,
                                        unpack)
from oracle import packer_ref as P
from tests._helpers import GOLDEN_CASES, gauss_weight, golden, golden_tag

BITS = (2, 4, 8)
LAYOUTS = ("sequential", "interleaved")
GROUPS = (32, 64, 128, 256, None)


@pytest.mark.parametrize("bits,gs,sym,layout", GOLDEN_CASES,
                         ids=[golden_tag(*c) for c in GOLDEN_CASES])
def test_bit_exact_with_reference_golden(bits, gs, sym, layout):
    g = golden()
    t = golden_tag(bits, gs, sym, layout)
    w = torch.from_numpy(g["w16"].view(np.float16).copy())
    cfg = QuantConfig(bits, gs, sym, layout)
    pw = quantize_tensor(w, cfg)
    assert np.array_equal(pw.qweight.numpy(), g[t + "/qweight"])
    assert np.array_equal(pw.scales.numpy().view(np.uint16), g[t + "/scales"])
    if sym:
        assert pw.zeros is None
    else:
        assert np.array_equal(pw.zeros.numpy().view(np.uint16), g[t + "/zeros"])
    assert np.array_equal(unpack(pw.qweight, cfg, w.shape[1]).numpy(), g[t + "/codes"])
    assert np.array_equal(dequantize(pw).numpy().view(np.uint16), g[t + "/deq"])
    assert pw.nbytes == P.packed_nbytes(*w.shape, P.Config(bits, gs, sym, layout))


def test_matches_numpy_oracle_on_llama_rows():
    w16 = gauss_weight(64, 4096, seed=11)
    for cfg_args in [(4, 128, False, "sequential"), (2, 64, False, "interleaved"), (8, None, True, "sequential")]:
        pw = quantize_tensor(torch.from_numpy(w16), QuantConfig(*cfg_args))
        qw, s, z = P.quantize_tensor(w16, P.Config(*cfg_args))
        assert np.array_equal(pw.qweight.numpy(), qw)
        assert np.array_equal(pw.scales.numpy().view(np.uint16), s.view(np.uint16))
        if z is not None:
            assert np.array_equal(pw.zeros.numpy().view(np.uint16), z.view(np.uint16))


# ---- scripts/test_packer.py restated ------------------------------------------

def test_pack_roundtrip():                                   # :47-55
    torch.manual_seed(0)
    for bits in BITS:
        for layout in LAYOUTS:
            cfg = QuantConfig(bits=bits, layout=layout)
            q = torch.randint(0, cfg.qmax + 1, (8, 512), dtype=torch.int32)
            assert torch.equal(unpack(pack(q, cfg), cfg, 512), q)


def test_error_bound():                                      # :58-76
    torch.manual_seed(0)
    w = torch.randn(64, 512, dtype=torch.float16)
    for bits in BITS:
        for sym in (True, False):
            for gs in GROUPS:
                cfg = QuantConfig(bits=bits, group_size=gs, symmetric=sym)
                pw = quantize_tensor(w, cfg)
                err = (dequantize(pw).float() - w.float()).abs()
                step = pw.scales.float().repeat_interleave(cfg.effective_group_size(512), dim=1)
                bound = step * (0.5 if sym else 1.0) + 1e-3
                assert (err / bound).max().item() <= 1.0, (bits, gs, sym)


def test_monotonic_in_bits():                                # :79-89
    torch.manual_seed(0)
    w = torch.randn(64, 512, dtype=torch.float16)
    errs = [(dequantize(quantize_tensor(w, QuantConfig(bits=b, group_size=128))).float() - w.float())
            .abs().mean().item() for b in BITS]
    assert all(a > b for a, b in zip(errs, errs[1:]))


def test_monotonic_in_group_size():                          # :92-103
    torch.manual_seed(0)
    w = torch.randn(64, 512, dtype=torch.float16)
    errs = [(dequantize(quantize_tensor(w, QuantConfig(bits=4, group_size=g))).float() - w.float())
            .abs().mean().item() for g in (32, 64, 128, 256, None)]
    assert all(a < b for a, b in zip(errs, errs[1:]))


def test_asymmetric_beats_symmetric_on_skew():               # :106-118
    torch.manual_seed(0)
    w = (torch.rand(64, 512) * 0.5 + 2.0).to(torch.float16)
    e_sym = (dequantize(quantize_tensor(w, QuantConfig(4, 128, True))).float() - w.float()).abs().mean()
    e_asym = (dequantize(quantize_tensor(w, QuantConfig(4, 128, False))).float() - w.float()).abs().mean()
    assert e_asym < e_sym


def test_layout_is_storage_only():                          # :121-128
    torch.manual_seed(0)
    w = torch.randn(64, 512, dtype=torch.float16)
    for bits in BITS:
        a = dequantize(quantize_tensor(w, QuantConfig(bits, 128, True, "sequential")))
        b = dequantize(quantize_tensor(w, QuantConfig(bits, 128, True, "interleaved")))
        assert torch.equal(a, b)


@pytest.mark.parametrize("n,k", [(3072, 3072), (1024, 3072), (8192, 3072), (3072, 8192)])
def test_error_matches_prediction(n, k):                     # :131-155
    torch.manual_seed(0)
    w = torch.randn(n, k, dtype=torch.float16) * 0.02
    pw = quantize_tensor(w, QuantConfig(4, 128, True))
    err = (dequantize(pw).float() - w.float()).abs().mean().item()
    ratio = err / (pw.scales.float().mean().item() / 4)
    assert 0.85 <= ratio <= 1.15


def test_config_validation():                                # packer.py:51-57
    with pytest.raises(ValueError, match="bits must be 2, 4 or 8"):
        QuantConfig(bits=3)
    with pytest.raises(ValueError, match="unknown layout"):
        QuantConfig(layout="zigzag")
    with pytest.raises(ValueError, match="group_size must be positive"):
        QuantConfig(group_size=0)
    with pytest.raises(ValueError, match="expected a 2-D weight"):
        quantize(torch.zeros(4), QuantConfig())
    with pytest.raises(ValueError, match="not divisible by group_size"):
        quantize(torch.zeros(2, 100, dtype=torch.float16), QuantConfig(group_size=64))
    with pytest.raises(ValueError, match="values per word"):
        pack(torch.zeros(2, 6, dtype=torch.int32), QuantConfig(bits=4))
    cfg = QuantConfig(8, None, True)
    assert (cfg.per_pack, cfg.qmax, cfg.bias, cfg.groups_for(4096), cfg.effective_group_size(4096)) == \
        (4, 255, 128, 1, 4096)
