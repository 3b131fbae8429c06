"""Pins the oracle's fp32 -> fp16 conversion (GGML_FP32_TO_FP16, used for the
Q4_0 scale) against two independent implementations: the host's F16C
instruction over all 2^32 inputs, and numpy's float16 cast."""
import numpy as np
import pytest

import oracle


@pytest.mark.slow
def test_fp16_exhaustive_vs_f16c():
    bad = oracle.selftest_fp16_exhaustive()
    if bad == -1:
        pytest.skip("host has no F16C")
    assert bad == 0


def _special_values():
    vals = [0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, -65520.0, 1e-8, 5.960464477539063e-08,
            2.980232238769531e-08, 2.9802326e-08, 8.940697e-08, 6.103515625e-05, 6.1035153e-05,
            np.inf, -np.inf, 3.4028235e38, 1.4e-45, -1.4e-45]
    # every fp16 value and the midpoints between neighbours (ties to even)
    h = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float32)
    mids = ((h[:-1].astype(np.float64) + h[1:].astype(np.float64)) / 2).astype(np.float32)
    return np.concatenate([np.array(vals, np.float32), h, -h, mids, -mids])


def test_fp16_vs_numpy_specials_and_ties():
    x = _special_values()
    ours = np.array([oracle.fp32_to_fp16_bits(float(v)) for v in x], dtype=np.uint16)
    ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(ours, ref)


def test_fp16_vs_numpy_random_bits():
    rng = np.random.default_rng(0xB0A0)
    bits = rng.integers(0, 2**32, size=200_000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[np.isfinite(x)]
    ours = np.array([oracle.fp32_to_fp16_bits(float(v)) for v in x[:50_000]], dtype=np.uint16)
    ref = x[:50_000].astype(np.float16).view(np.uint16)
    assert np.array_equal(ours, ref)


def test_fp16_to_fp32_all_codes():
    codes = np.arange(0, 65536, dtype=np.uint32)
    ref = codes.astype(np.uint16).view(np.float16).astype(np.float32)
    ours = np.array([oracle.fp16_bits_to_fp32(int(c)) for c in codes], dtype=np.float32)
    finite = np.isfinite(ref)
    assert np.array_equal(ours[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.all(np.isnan(ours[np.isnan(ref)]))
    assert np.array_equal(ours[np.isinf(ref)], ref[np.isinf(ref)])
