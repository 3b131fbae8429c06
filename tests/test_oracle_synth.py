"""The synthetic input stream of the benchmark configurations (oracle
orc_fill_normal / orc_fill_kv): splitmix64 words and Box-Muller normals with
ln and cos(2 pi .) evaluated from basic IEEE operations, so that the device
twin (libbmo_synth.so) can reproduce it bit for bit.

Pinned here, on the CPU:
  * synth_ln against math.log and synth_cos2pi against math.cos(2 pi t) at
    random points and at the edges of their reductions (the ln split at
    sqrt(2), exact powers of two, the quadrant and octant boundaries of t);
  * every normal equal, to the float32 rounding, to a numpy Box-Muller of the
    same splitmix64 words with numpy's own log and cos;
  * the stream's moments (mean 0, variance 1, skewness 0, kurtosis 3) and
    tail mass, and the kv variant's x8 rate (1%) and values."""
import math

import numpy as np

import oracle

L = oracle.lib()


def test_synth_ln_matches_libm():
    rng = np.random.default_rng(1)
    xs = list(rng.random(20000))
    xs += [2.0 ** -54, 2.0 ** -53, 0.5, 1.0, math.sqrt(0.5), math.sqrt(2.0) / 2, 0.75]
    xs += [math.nextafter(math.sqrt(0.5), 0), math.nextafter(math.sqrt(0.5), 1)]
    xs += [2.0 ** -k * f for k in range(1, 54) for f in (1.0, 1.41421356, 1.41421357, 1.9999999)]
    for x in xs:
        if not 2.0 ** -54 <= x <= 1.0:
            continue
        got = L.orc_synth_ln(x)
        ref = math.log(x)
        assert abs(got - ref) <= 4e-16 * max(1.0, abs(ref)), (x, got, ref)
    assert L.orc_synth_ln(1.0) == 0.0


def test_synth_cos2pi_matches_libm():
    rng = np.random.default_rng(2)
    ts = list(rng.random(20000)) + [k / 16 for k in range(16)]
    ts += [math.nextafter(k / 8, 0) for k in range(1, 8)] + [math.nextafter(k / 8, 1) for k in range(8)]
    for t in ts:
        got = L.orc_synth_cos2pi(t)
        ref = math.cos(2 * math.pi * t)   # (its argument 2 pi t is itself rounded)
        assert abs(got - ref) <= 2e-15, (t, got, ref)
    # exact at the quadrant starts
    assert [L.orc_synth_cos2pi(t) for t in (0.0, 0.25, 0.5, 0.75)] == [1.0, 0.0, -1.0, 0.0]


def test_normals_are_box_muller_of_the_words():
    n, seed, off = 200000, 0xB0A00003, 12345
    z = oracle.normal(seed, n, offset=off)
    w = oracle.words(seed, 2 * n, offset=2 * off)   # mix64(seed ^ mix64(2c)), mix64(seed ^ mix64(2c+1))
    u1 = ((w[0::2] >> np.uint64(11)).astype(np.float64) + 0.5) * 2.0 ** -53
    u2 = (w[1::2] >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
    ref = (np.sqrt(-2.0 * np.log(u1)) * np.cos(2 * np.pi * u2)).astype(np.float32)
    ulp = np.spacing(np.abs(ref))
    assert np.all(np.abs(z.astype(np.float64) - ref) <= ulp), "normals differ from Box-Muller beyond 1 ulp"


def test_normal_moments():
    z = oracle.normal(0xB0A00004, 1 << 22).astype(np.float64)
    assert abs(z.mean()) < 3e-3
    assert abs(z.var() - 1.0) < 4e-3
    assert abs(np.mean(z ** 3)) < 1e-2
    assert abs(np.mean(z ** 4) - 3.0) < 3e-2
    assert abs(np.mean(np.abs(z) > 3.0) - 0.0026998) < 3e-4


def test_kv_outliers():
    n, seed = 1 << 21, 0xB0A00003
    z = oracle.normal(seed, n)
    kv = oracle.kv_normal(seed, n)
    big = kv != z
    assert np.all(kv[big] == z[big] * np.float32(8.0))
    assert abs(big.mean() - 0.01) < 6e-4
    # the decision is a pure function of (seed, c): an offset window agrees
    assert np.array_equal(oracle.kv_normal(seed, 1000, offset=5000), kv[5000:6000])
