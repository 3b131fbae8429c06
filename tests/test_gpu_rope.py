"""GPU parity of the RoPE-fused append + decode (bmo_kv_ring_append_decode_rope)
against the oracle: q and k rotated by orc_rope_interleaved (the reference's
interleaved RoPE, src/bmo_cuda_kernels.cu:317-354) at each entry's absolute
position, then the oracle append (the ring must match bit-exactly: the kernel
rotates with the same fp32-rounded cosines and sines and the same fp32
operations) and the float64 decode (|gpu - ref| <= 2e-3 + 1e-3 |ref|)."""
import numpy as np
import pytest

import oracle
from _ringsim import Mirror, check_close

pytestmark = pytest.mark.gpu


def _i32(torch, vals):
    return torch.tensor(list(vals), dtype=torch.int32, device="cuda")


def _step(gpu, m, layer, entries, n_heads, theta, seed):
    """entries: list of (session, pos); one fused RoPE call for all of them."""
    n = len(entries)
    d, n_kv = m.d, m.n_kv
    q = oracle.normal(seed, n * n_heads * d).reshape(n, n_heads, d)
    k = oracle.normal(seed + 1, n * n_kv * d).reshape(n, n_kv, d)
    v = oracle.normal(seed + 2, n * n_kv * d).reshape(n, n_kv, d)
    out = gpu.full((n, n_heads, d), float("nan"), dtype=gpu.float32, device="cuda")
    sids = [s for s, _ in entries]
    pos = [p for _, p in entries]
    m.ring.append_decode(layer, _i32(gpu, pos), m.dev(q), m.dev(k), m.dev(v), out, n_heads,
                         session_ids=_i32(gpu, sids), stream=m.stream, rope_theta=theta)
    refs = []
    for b, (s, p) in enumerate(entries):
        m.oracle_append(layer, s, p, oracle.rope_interleaved(k[b], p, theta), v[b])
        refs.append(m.oracle_decode(layer, s, p, oracle.rope_interleaved(q[b], p, theta), n_heads))
    gpu.cuda.synchronize()
    got = out.cpu().numpy()
    for b, (s, p) in enumerate(entries):
        check_close(got[b], refs[b], f"rope decode entry {b} pos {p}")
        m.assert_ring_equal(layer, s)


def test_rope_b1_cfg1(gpu):
    """BASELINE config 1 shape (H=32, d=128, W=512, pos 700) with RoPE fused."""
    m = Mirror(gpu, 1, 1, 32, 128, 512)
    m.fill_range(0, 0, 0, 700, seed=1000)
    _step(gpu, m, 0, [(0, 700)], 32, 10000.0, seed=1)


@pytest.mark.parametrize("pos", [0, 1, 511, 4095, 100_000, 2**31 - 2])
def test_rope_positions(gpu, pos):
    """Positions where fp32 angles would lose precision (up to 2^31 - 2)."""
    m = Mirror(gpu, 1, 1, 4, 128, 64)
    m.fill_range(0, 0, 0, pos, seed=2000 + pos % 1000)
    _step(gpu, m, 0, [(0, pos)], 4, 10000.0, seed=2 + pos % 97)


def test_rope_batched_gqa_and_head_dim_64(gpu):
    m = Mirror(gpu, 2, 5, 2, 128, 96)
    pos = {0: 0, 1: 95, 2: 96, 3: 1234, 4: 77}
    for s, p in pos.items():
        m.fill_range(1, s, 0, p, seed=3000 + s)
    _step(gpu, m, 1, [(3, 1234), (0, 0), (4, 77), (1, 95), (2, 96)], 8, 10000.0, seed=3)
    m2 = Mirror(gpu, 1, 2, 4, 64, 8)
    for s in range(2):
        m2.fill_range(0, s, 0, 5 + s, seed=4000 + s)
    _step(gpu, m2, 0, [(1, 6), (0, 5)], 4, 500000.0, seed=4)


def test_rope_autoregressive_steps(gpu):
    """36 consecutive steps wrap a 16-slot ring; each step's ring state and
    output must keep matching."""
    m = Mirror(gpu, 1, 2, 4, 128, 16)
    for p in range(36):
        _step(gpu, m, 0, [(0, p), (1, 3 * p + 1)], 8, 10000.0, seed=100 + p)


def test_rope_argument_errors(gpu):
    from bmo_jetson_amd import KVRing, RingError
    ring = KVRing(1, 1, 2, 128, 16)
    x = gpu.zeros(2 * 128, dtype=gpu.float32, device="cuda")
    pos = _i32(gpu, [3])
    for theta in (0.0, -1.0, float("inf"), float("nan")):
        with pytest.raises(RingError) as e:
            ring.append_decode(0, pos, x, x, x, x, 2, rope_theta=theta)
        assert e.value.rc == 2
    ring.append_decode(0, pos, x, x, x, x, 2, rope_theta=10000.0)
    gpu.cuda.synchronize()
    assert ring.last_error() is None
    ring.close()
