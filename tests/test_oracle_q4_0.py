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


# ---- the checks above must catch plausible slips -----------------------------
#
# quantize_numpy is a vectorized restatement of the same published steps with
# switches for the slips a restatement could make.  With no switch set it
# must pass every check; each mutant must fail at least one.  The checks are
# functions of the quantizer, so they are exactly the ones the oracle passes.

def quantize_numpy(x, tie_last=False, divisor=-8.0, fused=False, swap_nibbles=False,
                   clamp=True, id_from_fp16=False, round_even=False):
    """x: (n, 32) float32 -> (d bits uint16 [n], qs uint8 [n, 16])."""
    x = np.ascontiguousarray(x, np.float32)
    n = x.shape[0]
    ax = np.abs(x)
    idx = 31 - np.argmax(ax[:, ::-1], axis=1) if tie_last else np.argmax(ax, axis=1)
    m = x[np.arange(n), idx]
    d = (m / np.float32(divisor)).astype(np.float32)
    d16 = d.astype(np.float16)
    dd = d16.astype(np.float32) if id_from_fp16 else d
    with np.errstate(divide="ignore"):
        idv = np.where(dd != 0, (np.float32(1.0) / dd).astype(np.float32), np.float32(0.0))
    if round_even:
        q = np.rint((x * idv[:, None]).astype(np.float32)).astype(np.int64) + 8
    elif fused:
        q = np.trunc(x.astype(np.float64) * idv[:, None].astype(np.float64) + 8.5).astype(np.int64)
    else:
        t = (x * idv[:, None]).astype(np.float32)
        q = np.trunc((t + np.float32(8.5)).astype(np.float32)).astype(np.int64)
    if clamp:
        q = np.minimum(q, 15)
    lo, hi = q[:, :16], q[:, 16:]
    qs = (hi | (lo << 4)) if swap_nibbles else (lo | (hi << 4))
    return d16.view(np.uint16), (qs & 0xFF).astype(np.uint8)


def _oracle_quant(x):
    b = oracle.quantize_q4_0(x)
    return b["d"].copy(), b["qs"].copy()


def check_kats(quant):
    for c in KAT["cases"]:
        d, qs = quant(np.array(c["x"], np.float32).reshape(1, 32))
        if int(d[0]) != c["d"] or [int(v) for v in qs[0]] != c["qs"]:
            return False
    return True


def check_brute_force(quant):
    x = _blocks_random(11, 4000, outlier_p=0.01)
    d, qs = quant(x)
    qs = qs.astype(np.int32)
    codes = np.concatenate([qs & 0xF, qs >> 4], axis=-1)
    amax_idx = np.argmax(np.abs(x), axis=1)
    m = x[np.arange(len(x)), amax_idx]
    dm = (m / np.float32(-8.0)).astype(np.float32)
    t = (x * (np.float32(1.0) / dm).astype(np.float32)[:, None]).astype(np.float32)
    cand = np.arange(16, dtype=np.float64)[None, None, :] - 8.0
    dist = np.abs(cand - t.astype(np.float64)[..., None])
    best = np.argmin(dist + 1e-12 * (15 - np.arange(16))[None, None, :], axis=-1)
    return bool(np.array_equal(codes, best) and np.all(codes[np.arange(len(x)), amax_idx] == 0))


def check_scale(quant):
    x = _blocks_random(12, 2000)
    d, _ = quant(x)
    m = x[np.arange(len(x)), np.argmax(np.abs(x), axis=1)]
    ref = (m / np.float32(-8.0)).astype(np.float32).astype(np.float16).view(np.uint16)
    return bool(np.array_equal(d, ref))


CHECKS = (check_kats, check_brute_force, check_scale)


def test_checks_pass_oracle_and_numpy_restatement():
    for check in CHECKS:
        assert check(_oracle_quant), check.__name__
        assert check(quantize_numpy), check.__name__


MUTANTS = {
    "tie_last": dict(tie_last=True),            # >= in the max scan: last occurrence wins
    "divisor_plus_8": dict(divisor=8.0),        # sign of d flipped
    "divisor_minus_7": dict(divisor=-7.0),      # a symmetric 7-level scale
    "swap_nibbles": dict(swap_nibbles=True),    # element j in the high nibble
    "no_clamp": dict(clamp=False),              # min(15, .) dropped
    "id_from_fp16": dict(id_from_fp16=True),    # 1/d taken from the rounded scale
    "round_even": dict(round_even=True),        # rint instead of trunc(x*id + 8.5)
    "fused": dict(fused=True),                  # x*id + 8.5 contracted into one rounding
}


@pytest.mark.parametrize("name", sorted(MUTANTS))
def test_planted_mistake_is_caught(name):
    """Each plausible slip in a restatement of the quantizer fails at least one
    of the checks the oracle passes."""
    quant = lambda x: quantize_numpy(x, **MUTANTS[name])
    failed = [c.__name__ for c in CHECKS if not c(quant)]
    assert failed, f"mutant {name} passes every check"
