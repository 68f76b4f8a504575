"""Pins the CPU oracle (oracle/packer_ref.py and oracle/dq_oracle.c).

Each check is chosen so that a plausible mistake in the oracle -- a wrong
interleave entry, a swapped slot/logical index, a missing bias, truncation
instead of round-to-nearest-even, a dropped zero point -- fails it:

  * known-answer words derived by hand from the interleave tables
    (dequant/packer.py:37-41) for codes i & qmax in logical order;
  * golden vectors written by the reference's own packer.py
    (tests/golden/make_golden.py): quantize, pack, unpack, dequantize, 48
    configurations over edge-case rows;
  * brute force: every code value in every slot, alone;
  * the C oracle's fp32 -> fp16 conversion against numpy at every fp16
    rounding midpoint (and one float32 ulp either side);
  * closed forms for dequantize and the GEMV reference on hand-picked values;
  * the reference's negative control: one flipped weight bit must break the
    GEMV criterion at exactly one output (test_dequant_kernel.py:194-217),
    planted in the oracle on the CPU.
"""

import numpy as np
import pytest

from oracle import packer_ref as P
from tests._helpers import (GOLDEN_CASES, activations, gauss_weight, golden, golden_tag, oracle_lib,
                            ptr)

# Known-answer words: codes (i & qmax) for i = 0..per-1 in LOGICAL order.
KAT = {
    (4, "sequential"): 0x76543210,
    (4, "interleaved"): 0x75316420,
    (8, "sequential"): 0x03020100,
    (8, "interleaved"): 0x03010200,
    (2, "sequential"): 0xE4E4E4E4,
    (2, "interleaved"): 0xFFAA5500,
}


@pytest.mark.parametrize("bits,layout", sorted(KAT))
def test_known_answer_words(bits, layout):
    cfg = P.Config(bits, 128, True, layout)
    codes = (np.arange(cfg.per_pack, dtype=np.int32) & cfg.qmax)[None, :]
    word = P.pack(codes, cfg)
    assert word.shape == (1, 1)
    assert int(word.view(np.uint32)[0, 0]) == KAT[(bits, layout)]
    assert np.array_equal(P.unpack(word, cfg, cfg.per_pack), codes)
    lib = oracle_lib()
    out = np.zeros((1, cfg.per_pack), dtype=np.int32)
    lib.dqo_unpack(ptr(word.view(np.uint32)), ptr(out), 1, cfg.per_pack, bits, layout == "interleaved")
    assert np.array_equal(out, codes)


def test_all_fifteen_int4_is_minus_one():
    cfg = P.Config(4, 128, True, "sequential")
    assert int(P.pack(np.full((1, 8), 15, dtype=np.int32), cfg)[0, 0]) == -1


@pytest.mark.parametrize("bits", (2, 4, 8))
@pytest.mark.parametrize("layout", ("sequential", "interleaved"))
def test_every_code_in_every_slot(bits, layout):
    cfg = P.Config(bits, 128, True, layout)
    per, order = cfg.per_pack, cfg.order()
    lib = oracle_lib()
    for logical in range(per):
        slot = order.index(logical)
        for code in range(cfg.qmax + 1):
            q = np.zeros((1, per), dtype=np.int32)
            q[0, logical] = code
            w = int(P.pack(q, cfg).view(np.uint32)[0, 0])
            assert w == code << (bits * slot)
            out = np.zeros((1, per), dtype=np.int32)
            lib.dqo_unpack(ptr(np.array([w], dtype=np.uint32)), ptr(out), 1, per, bits,
                           layout == "interleaved")
            assert np.array_equal(out, q)


@pytest.mark.parametrize("bits,gs,sym,layout", GOLDEN_CASES,
                         ids=[golden_tag(*c) for c in GOLDEN_CASES])
def test_numpy_oracle_matches_reference_golden(bits, gs, sym, layout):
    g = golden()
    t = golden_tag(bits, gs, sym, layout)
    w16 = g["w16"].view(np.float16)
    cfg = P.Config(bits, gs, sym, layout)
    qw, s, z = P.quantize_tensor(w16, cfg)
    assert np.array_equal(qw, g[t + "/qweight"])
    assert np.array_equal(s.view(np.uint16), g[t + "/scales"])
    if not sym:
        assert np.array_equal(z.view(np.uint16), g[t + "/zeros"])
    assert np.array_equal(P.unpack(g[t + "/qweight"], cfg, w16.shape[1]), g[t + "/codes"])
    deq = P.dequantize(g[t + "/qweight"], g[t + "/scales"].view(np.float16),
                       None if sym else g[t + "/zeros"].view(np.float16), cfg, w16.shape)
    assert np.array_equal(deq.view(np.uint16), g[t + "/deq"])


@pytest.mark.parametrize("bits,gs,sym,layout", GOLDEN_CASES,
                         ids=[golden_tag(*c) for c in GOLDEN_CASES])
def test_c_oracle_matches_reference_golden(bits, gs, sym, layout):
    g = golden()
    t = golden_tag(bits, gs, sym, layout)
    n, k = g["w16"].shape
    gsz = k if gs is None else gs
    qw = np.ascontiguousarray(g[t + "/qweight"].view(np.uint32))
    sc = np.ascontiguousarray(g[t + "/scales"])
    ze = None if sym else np.ascontiguousarray(g[t + "/zeros"])
    lib = oracle_lib()
    codes = np.zeros((n, k), dtype=np.int32)
    lib.dqo_unpack(ptr(qw), ptr(codes), n, k, bits, layout == "interleaved")
    assert np.array_equal(codes, g[t + "/codes"])
    deq = np.zeros((n, k), dtype=np.uint16)
    lib.dqo_dequantize(ptr(qw), ptr(sc), ptr(ze), ptr(deq), n, k, bits, gsz, sym, layout == "interleaved")
    assert np.array_equal(deq, g[t + "/deq"])
    # exact_weight rounds to the same fp16 values as dequantize
    ew = np.zeros((n, k), dtype=np.float32)
    lib.dqo_exact_weight(ptr(qw), ptr(sc), ptr(ze), ptr(ew), n, k, bits, gsz, sym, layout == "interleaved")
    with np.errstate(over="ignore", invalid="ignore"):
        assert np.array_equal(ew.astype(np.float16).view(np.uint16), g[t + "/deq"])
    np_ew = P.exact_weight(qw.view(np.int32), sc.view(np.float16), None if sym else ze.view(np.float16),
                           P.Config(bits, gs, sym, layout), (n, k))
    assert np.array_equal(ew.view(np.uint32), np_ew.view(np.uint32))


def test_c_oracle_fp16_rounding_at_every_midpoint():
    lib = oracle_lib()
    h = np.arange(0x7C00, dtype=np.uint32).astype(np.uint16)  # finite non-negative fp16
    lo = h.view(np.float16).astype(np.float64)
    hi = (h + 1).view(np.float16).astype(np.float64)
    mids = ((lo + hi) / 2).astype(np.float32)                   # exact in float32
    cand = [mids, np.nextafter(mids, np.float32(np.inf)), np.nextafter(mids, np.float32(0)),
            lo.astype(np.float32), np.float32(65520.0) * np.ones(1, np.float32),
            np.array([1e-9, 2.0 ** -25, 2.0 ** -25 * 1.0000001, 3.0 * 2.0 ** -26, np.inf, 1e30], np.float32)]
    f = np.concatenate([c.astype(np.float32) for c in cand])
    f = np.concatenate([f, -f])
    out = np.zeros(f.shape, dtype=np.uint16)
    lib.dqo_f32_to_f16_array(ptr(f), ptr(out), f.size)
    assert np.array_equal(out, f.astype(np.float16).view(np.uint16))
    back = np.array([lib.dqo_f16_to_f32(int(u)) for u in h[::97]], dtype=np.float32)
    assert np.array_equal(back, h[::97].view(np.float16).astype(np.float32))


def test_dequantize_closed_form():
    # INT4 asym, one group of 8: codes 0..7 (sequential), zero 3, scale 0.5 -> (q - 3) * 0.5
    cfg = P.Config(4, 8, False, "sequential")
    q = np.arange(8, dtype=np.int32)[None, :]
    w = np.float16(0.5) * (q.astype(np.float32) - 3)
    deq = P.dequantize(P.pack(q, cfg), np.array([[0.5]], np.float16), np.array([[3.0]], np.float16),
                       cfg, (1, 8))
    assert np.array_equal(deq.astype(np.float32), w)
    # INT8 sym per-channel: code 0 -> -128 * s, code 255 -> 127 * s
    cfg8 = P.Config(8, None, True, "interleaved")
    q8 = np.array([[0, 255, 128, 1]], dtype=np.int32)
    deq8 = P.dequantize(P.pack(q8, cfg8), np.array([[0.25]], np.float16), None, cfg8, (1, 4))
    assert deq8.astype(np.float32).tolist() == [[-32.0, 31.75, 0.0, -31.75]]
    # fp16 rounding of the fp32 product: 3 * (1 + 2^-10) = 3.0029296875 lies exactly halfway
    # between fp16 3.001953125 (odd mantissa) and 3.00390625 (even): RNE picks the even one.
    cfg2 = P.Config(2, 16, False, "sequential")
    q2 = np.full((1, 16), 3, dtype=np.int32)
    s2 = np.array([[1 + 2 ** -10]], np.float16)
    deq2 = P.dequantize(P.pack(q2, cfg2), s2, np.array([[0.0]], np.float16), cfg2, (1, 16))
    assert float(deq2[0, 0]) == float(np.float16(3 * (1 + 2 ** -10)))
    assert float(deq2[0, 0]) == 3.00390625  # 3.0029296875 is a tie -> even mantissa


def test_gemv_reference_brute_force():
    # tiny shape, pure-Python loops in exact rational-free float64
    cfg = P.Config(4, 16, False, "interleaved")
    w16 = gauss_weight(3, 32, seed=1)
    qw, s, z = P.quantize_tensor(w16, cfg)
    ew = P.exact_weight(qw, s, z, cfg, (3, 32))
    x = activations(2, 32, seed=2)
    ref, absref = P.gemv_reference(x, ew)
    codes = P.unpack(qw, cfg, 32)
    for mi in range(2):
        for r in range(3):
            acc = 0.0
            aacc = 0.0
            for c in range(32):
                g = c // 16
                wv = float(np.float32((np.float32(codes[r, c]) - np.float32(z[r, g])) * np.float32(s[r, g])))
                acc += float(x[mi, c]) * wv
                aacc += abs(float(x[mi, c])) * abs(wv)
            assert ref[mi, r] == pytest.approx(acc, rel=1e-15, abs=1e-300)
            assert absref[mi, r] == pytest.approx(aacc, rel=1e-15)
    # the C oracle's reference agrees
    lib = oracle_lib()
    cref = np.zeros((2, 3)); cabs = np.zeros((2, 3))
    lib.dqo_gemv_ref(ptr(x.view(np.uint16)), ptr(ew), ptr(cref), ptr(cabs), 2, 3, 32)
    assert np.allclose(cref, ref, rtol=1e-14, atol=0) and np.allclose(cabs, absref, rtol=1e-14)


def test_gemv_criterion_has_teeth():
    """Negative control (scripts/test_dequant_kernel.py:194-217), planted in the oracle."""
    n, k = 256, 1024
    cfg = P.Config(4, 128, True, "sequential")
    qw, s, z = P.quantize_tensor(gauss_weight(n, k, seed=3), cfg)
    x = activations(1, k, seed=4)
    x[0, 0] = np.float16(1.0)
    ew = P.exact_weight(qw, s, z, cfg, (n, k))
    ref, absref = P.gemv_reference(x, ew)
    # a faithful fp32 computation passes
    y_ok = (x.astype(np.float32) @ ew.T).astype(np.float16)
    assert P.gemv_criterion(y_ok, ref, absref)[0]
    assert P.rel_l2(y_ok, ref) <= 1e-3
    # one flipped bit of the first word fails at exactly [0, 0]
    bad = qw.copy()
    bad[0, 0] ^= 1
    y_bad = (x.astype(np.float32) @ P.exact_weight(bad, s, z, cfg, (n, k)).T).astype(np.float16)
    tol = 2.0 ** -11 * np.abs(ref) + 2.0 ** -20 * absref
    over = np.abs(y_bad.astype(np.float64) - ref) > tol
    assert over[0, 0] and int(over.sum()) == 1


def test_packed_nbytes_closed_form():
    # per-call bytes of the benchmark configs C1, C2 (M=1), C3: PackedWeight.nbytes + x + y
    assert P.packed_nbytes(4096, 4096, P.Config(4, 128, False)) + 4096 * 2 * 2 == 8_929_280
    assert P.packed_nbytes(11008, 4096, P.Config(8, None, True)) + 4096 * 2 + 11008 * 2 == 45_140_992
    assert P.packed_nbytes(4096, 11008, P.Config(2, 64, False)) + 11008 * 2 + 4096 * 2 == 14_120_448
