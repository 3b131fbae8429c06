"""Pins the RoPE oracle (orc_rope_interleaved, restating the reference's
interleaved rotation, src/bmo_cuda_kernels.cu:317-354) against mathematics:
a complex-exponential evaluation in numpy, the pos = 0 identity, norm
preservation, composition of rotations, the relative-position property of
rotated dot products, and a planted pairing mistake that must be caught."""
import numpy as np
import pytest

import oracle

THETA = 10000.0  # src/bmo.cpp:301-303 default


def _complex_rope(x, pos, theta=THETA):
    """Independent formulation: pair i as the complex number x[2i] + j x[2i+1]
    times exp(j * pos * theta^(-2i/d)), in complex128."""
    d = x.shape[-1]
    i = np.arange(d // 2, dtype=np.float64)
    ang = float(pos) * np.power(theta, -2.0 * i / d)
    z = x[..., 0::2].astype(np.float64) + 1j * x[..., 1::2].astype(np.float64)
    w = z * np.exp(1j * ang)
    y = np.empty(x.shape, dtype=np.float64)
    y[..., 0::2] = w.real
    y[..., 1::2] = w.imag
    return y


@pytest.mark.parametrize("d", [128, 64])
@pytest.mark.parametrize("pos", [0, 1, 7, 700, 4095, 100_000, 2**31 - 1])
def test_rope_matches_complex_exponential(d, pos):
    x = oracle.normal(900 + pos % 97, 4 * d).reshape(4, d)
    y = oracle.rope_interleaved(x, pos)
    ref = _complex_rope(x, pos)
    # fp32 cos/sin and fp32 products: a few ulp of the pair's magnitude; the
    # angle itself is exact to double precision at every position
    scale = np.abs(x).max()
    assert np.abs(y - ref).max() <= 4 * 2.0**-23 * scale * 2


def test_rope_identity_at_zero_and_frequencies():
    x = oracle.normal(5, 3 * 128).reshape(3, 128)
    assert np.array_equal(oracle.rope_interleaved(x, 0), x)
    for d in (64, 128):
        r = THETA ** (-2.0 / d)
        for i in range(d // 2):
            assert oracle.rope_freq(r, i) == pytest.approx(THETA ** (-2.0 * i / d), rel=1e-14)
    cs, sn = oracle.rope_cos_sin(128, 700)
    # pair 0 turns by exactly pos radians
    assert cs[0] == np.float32(np.cos(700.0)) and sn[0] == np.float32(np.sin(700.0))


def test_rope_preserves_pair_norms_and_composes():
    x = oracle.normal(11, 8 * 128).reshape(8, 128)
    y = oracle.rope_interleaved(x, 1234)
    nx = np.hypot(x[:, 0::2], x[:, 1::2])
    ny = np.hypot(y[:, 0::2], y[:, 1::2])
    assert np.allclose(nx, ny, rtol=1e-6, atol=1e-6)
    # R(a) R(b) = R(a + b)
    two = oracle.rope_interleaved(oracle.rope_interleaved(x, 300), 934)
    assert np.abs(two - y).max() < 1e-5


def test_rope_scores_depend_on_relative_position_only():
    q = oracle.normal(21, 4 * 128).reshape(4, 128)
    k = oracle.normal(22, 4 * 128).reshape(4, 128)
    base = np.sum(oracle.rope_interleaved(q, 40).astype(np.float64)
                  * oracle.rope_interleaved(k, 17), axis=1)
    for shift in (1, 500, 3000):
        s = np.sum(oracle.rope_interleaved(q, 40 + shift).astype(np.float64)
                   * oracle.rope_interleaved(k, 17 + shift), axis=1)
        assert np.allclose(s, base, atol=2e-4)


def test_planted_pairing_mistake_is_caught():
    """A half-split (NeoX) pairing would pass the norm and relative-position
    checks; the complex evaluation with interleaved pairs rejects it."""
    x = oracle.normal(31, 2 * 128).reshape(2, 128)
    pos = 700
    d = 128
    perm = np.concatenate([np.arange(0, d, 2), np.arange(1, d, 2)])  # interleaved -> halves
    wrong = np.empty_like(x)
    wrong[:, perm] = oracle.rope_interleaved(x[:, perm], pos)
    ref = _complex_rope(x, pos)
    assert np.abs(oracle.rope_interleaved(x, pos) - ref).max() < 1e-5
    assert np.abs(wrong - ref).max() > 0.1
