"""Pins the GEMV oracle (orc_quantize_row_q8_1_bmo / orc_gemv_q4_0_q8_1_f64,
restating src/bmo_cuda_kernels.cu:529-711): hand-derived Q8_1 known answers,
nearest-code invariants, and an independent numpy evaluation of the dot
formula from the raw block bytes."""
import numpy as np
import pytest

import oracle


def _f16(bits):
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float64)


def test_q8_1_known_answers():
    z = oracle.quantize_q8_1(np.zeros(32, np.float32))[0]
    assert z["d"] == 0 and z["s"] == 0 and not z["qs"].any()
    # amax 127 -> d = 1, id = 1: codes are roundf(x), halves away from zero
    x = np.zeros(32, np.float32)
    x[:8] = [127.0, -63.5, 0.5, -0.5, 2.5, -2.5, 1.4999999, 3.0]
    b = oracle.quantize_q8_1(x)[0]
    assert _f16(b["d"]) == 1.0
    assert list(b["qs"][:8]) == [127, -64, 1, -1, 3, -3, 1, 3]
    assert _f16(b["s"]) == np.float16(np.float32(127.0 - 63.5 + 0.5 - 0.5 + 2.5 - 2.5 + 1.4999999 + 3.0))
    # amax 254 -> d = 2: codes are roundf(x / 2)
    y = np.zeros(32, np.float32)
    y[:4] = [-254.0, 5.0, 3.0, -1.0]
    b = oracle.quantize_q8_1(y)[0]
    assert _f16(b["d"]) == 2.0 and list(b["qs"][:4]) == [-127, 3, 2, -1]
    # the s field is fp16 of the fp32 sum of the values (not d * sum(q))
    w = np.full(32, 0.1, np.float32)
    b = oracle.quantize_q8_1(w)[0]
    assert _f16(b["s"]) == np.float64(np.float16(np.float32(np.sum(w, dtype=np.float32))))
    assert _f16(b["s"]) != pytest.approx(_f16(b["d"]) * int(b["qs"].astype(np.int64).sum()), rel=1e-6)


def test_q8_1_nearest_code_invariants():
    x = (oracle.normal(77, 64 * 32) * np.float32(3.0)).astype(np.float32)
    blocks = oracle.quantize_q8_1(x)
    xb = x.reshape(-1, 32).astype(np.float64)
    d = _f16(blocks["d"])[:, None]
    # d is fp16(amax / 127): the largest magnitude quantizes to +-127
    amax = np.abs(xb).max(axis=1)
    assert np.all(np.abs(blocks["qs"]).max(axis=1) == 127)
    assert np.allclose(d[:, 0], amax / 127.0, rtol=2.0**-10)
    # each code is the nearest integer to x * id (id = 1/d in fp32)
    dd = (amax / 127.0).astype(np.float32)
    idd = (np.float32(1.0) / dd)[:, None]
    p = (x.reshape(-1, 32) * idd).astype(np.float64)
    assert np.all(np.abs(p - blocks["qs"]) <= 0.5)


def _numpy_gemv(w_blocks, xq, rows, cols):
    nb = cols // 32
    w = w_blocks.reshape(rows, nb)
    codes = np.concatenate([w["qs"] & 0x0F, w["qs"] >> 4], axis=-1).astype(np.int64)  # [rows, nb, 32]
    q8 = xq["qs"].astype(np.int64)                                                     # [nb, 32]
    sumi = np.einsum("rbj,bj->rb", codes, q8)
    d4 = _f16(w["d"])
    d8 = _f16(xq["d"])[None, :]
    s8 = _f16(xq["s"])[None, :]
    return np.sum(d4 * (sumi * d8 - 8.0 * s8), axis=1)


@pytest.mark.parametrize("rows,cols", [(7, 64), (33, 4096), (5, 5632)])
def test_gemv_oracle_matches_numpy(rows, cols):
    wf = oracle.normal(5 + rows, rows * cols)
    w = oracle.quantize_q4_0(wf)
    x = oracle.normal(6 + cols, cols)
    xq = oracle.quantize_q8_1(x)
    y, tabs = oracle.gemv_q4_0_q8_1_f64(w, xq, rows, cols)
    ref = _numpy_gemv(w, xq, rows, cols)
    assert np.allclose(y, ref, rtol=1e-12, atol=1e-12 * tabs.max())
    # and it approximates the fp32 product of the dequantized operands
    exact = oracle.dequantize_q4_0(w).reshape(rows, cols).astype(np.float64) @ x.astype(np.float64)
    assert np.all(np.abs(y - exact) <= 0.02 * tabs + 1e-3)


def test_planted_q8_1_sum_mistake_is_caught():
    """ggml's own Q8_1 stores s = d * sum(q); the reference stores the sum of
    x.  The numpy evaluation with the reference's field tells them apart."""
    rows, cols = 16, 1024
    w = oracle.quantize_q4_0(oracle.normal(8, rows * cols))
    x = oracle.normal(9, cols)
    xq = oracle.quantize_q8_1(x)
    y, tabs = oracle.gemv_q4_0_q8_1_f64(w, xq, rows, cols)
    wrong = xq.copy()
    wrong["s"] = (_f16(xq["d"]) * xq["qs"].astype(np.int64).sum(axis=1)).astype(np.float16).view(np.uint16)
    y_wrong = _numpy_gemv(w, wrong, rows, cols)
    assert np.abs(y - y_wrong).max() > 1e-4 * tabs.max()
