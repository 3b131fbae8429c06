"""Pins the oracle's Q4_0 quantizer/dequantizer (restatement of ggml
quantize_row_q4_0_ref / dequantize_row_q4_0; format of
src/bmo_cuda_kernels.cu:496-499, dequant (q-8)*d of src/bmo_kernel_bench.cu:92-93,
nibble order of src/bmo_cuda_kernels.cu:626-629).

Pins, chosen so a plausible slip fails one of them:
  * hand-derived known answers (tests/golden/q4_0_kat.json): sign of d, the
    -8 divisor, tie-breaking, rounding points, the clamp, nibble order, fp16
    rounding/underflow/overflow of the scale;
  * an independent brute-force formulation: each code is the c in 0..15
    minimizing |(c - 8) - x*id| with halves rounding up (a search, not the
    closed formula), the max element always codes to 0;
  * error bounds of the dequantized block against the input;
  * dequantization against numpy on the raw bytes.
"""
import json
import os

import numpy as np
import pytest

import oracle

KAT = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "q4_0_kat.json")))


@pytest.mark.parametrize("case", KAT["cases"], ids=[c["name"] for c in KAT["cases"]])
def test_known_answers(case):
    b = oracle.quantize_q4_0(np.array(case["x"], dtype=np.float32))
    assert int(b["d"][0]) == case["d"], case["why"]
    assert [int(v) for v in b["qs"][0]] == case["qs"], case["why"]


def _codes(blocks):
    qs = blocks["qs"].astype(np.int32)
    return np.concatenate([qs & 0xF, qs >> 4], axis=-1)  # element order 0..31


def _blocks_random(seed, n, outlier_p=0.0):
    x = oracle.normal(seed, n * 32).reshape(n, 32)
    if outlier_p:
        u = oracle.words(seed + 1, n * 32).reshape(n, 32)
        x = np.where((u % 10000) < outlier_p * 10000, x * 8.0, x).astype(np.float32)
    return x


def test_brute_force_nearest_code():
    x = _blocks_random(11, 4000, outlier_p=0.01)
    b = oracle.quantize_q4_0(x)
    codes = _codes(b)
    amax_idx = np.argmax(np.abs(x), axis=1)  # first occurrence, like the scan
    m = x[np.arange(len(x)), amax_idx]
    d = (m / np.float32(-8.0)).astype(np.float32)
    idv = (np.float32(1.0) / d).astype(np.float32)
    t = (x * idv[:, None]).astype(np.float32)  # x*id in fp32
    # search: the code whose (c-8) is nearest to t, halves going up, clamped
    cand = np.arange(16, dtype=np.float64)[None, None, :] - 8.0
    dist = np.abs(cand - t.astype(np.float64)[..., None])
    best = np.argmin(dist + 1e-12 * (15 - np.arange(16))[None, None, :], axis=-1)
    # exact halves: the formula rounds up (trunc(t + 8.5)); the search's tiny
    # bias picks the upper candidate on exact ties
    assert np.array_equal(codes, best)
    assert np.all(codes[np.arange(len(x)), amax_idx] == 0)
    assert codes.min() >= 0 and codes.max() <= 15


def test_scale_is_fp16_of_max_over_minus_8():
    x = _blocks_random(12, 2000)
    b = oracle.quantize_q4_0(x)
    m = x[np.arange(len(x)), np.argmax(np.abs(x), axis=1)]
    ref = (m / np.float32(-8.0)).astype(np.float32).astype(np.float16).view(np.uint16)
    assert np.array_equal(b["d"], ref)


def test_dequant_matches_numpy_on_bytes():
    x = _blocks_random(13, 500, outlier_p=0.01)
    b = oracle.quantize_q4_0(x)
    y = oracle.dequantize_q4_0(b).reshape(-1, 32)
    d = b["d"].view(np.float16).astype(np.float32)
    ref = ((_codes(b) - 8).astype(np.float32) * d[:, None]).astype(np.float32)
    assert np.array_equal(y, ref)


def test_error_bounds():
    x = _blocks_random(14, 3000, outlier_p=0.01)
    b = oracle.quantize_q4_0(x)
    y = oracle.dequantize_q4_0(b).reshape(-1, 32)
    m = x[np.arange(len(x)), np.argmax(np.abs(x), axis=1)]
    d = np.abs(m / 8.0)
    d16 = np.abs(b["d"].view(np.float16).astype(np.float64))
    err = np.abs(x.astype(np.float64) - y)
    codes = _codes(b)
    bound = d[:, None] / 2 + 8 * np.abs(d - d16)[:, None] + 1e-6 * d[:, None]
    # the clamped side (x near -m) may be off by up to a whole step
    clamped = codes == 15
    assert np.all(err[~clamped] <= np.broadcast_to(bound, err.shape)[~clamped])
    assert np.all(err[clamped] <= (d[:, None] + 8 * np.abs(d - d16)[:, None] + 1e-6 * d[:, None])
                  .repeat(32, 1)[clamped])


def test_planted_mistake_is_caught():
    """A quantizer with the wrong tie rule (last occurrence wins) must fail the
    tie KATs: the KATs are sensitive to this class of slip."""
    x = np.array(KAT["cases"][3]["x"], np.float32)
    amax = np.max(np.abs(x))
    last = np.where(np.abs(x) == amax)[0][-1]
    d_wrong = np.float32(x[last] / np.float32(-8.0)).astype(np.float16).view(np.uint16)
    assert int(d_wrong) != KAT["cases"][3]["d"]
