"""Seeded random shapes for batched decode and fused append + decode against
the float64 oracle (same bar as tests/test_gpu_parity.py): head_dim 64 or
128, ring sizes on and off the 32-slot grid (8 to 1024 slots), 1, 2 or 4 kv
heads with 1, 2 or 4 query heads each, 1 to 4 sessions in a permuted order
(a batch names each at most once, at most n_sessions entries), positions
from the first token to many wraps, and sometimes an entry whose session id
is out of range (its output must be zeroed).  After a fused call every named
session's ring must match the oracle bit for bit."""
import numpy as np
import pytest

import oracle
from _ringsim import Mirror, check_close

pytestmark = pytest.mark.gpu

SEEDS = list(range(24))


def _i32(torch, vals):
    return torch.tensor(list(vals), dtype=torch.int32, device="cuda")


def _case(seed):
    r = np.random.default_rng(0xD0C0D000 + seed)
    d = int(r.choice([64, 128]))
    n_ctx = int(r.choice([8, 24, 32, 40, 64, 100, 256, 512, 1024]))
    n_kv = int(r.choice([1, 2, 4]))
    n_heads = n_kv * int(r.choice([1, 2, 4]))
    n_sess = int(r.integers(1, 5))
    sids = [int(s) for s in r.permutation(n_sess)]
    if n_sess >= 2 and r.random() < 0.4:
        sids[int(r.integers(0, n_sess))] = n_sess   # out of range: skipped
    pos = [int(r.choice([0, int(r.integers(1, n_ctx)), int(r.integers(n_ctx, 6 * n_ctx))]))
           for _ in sids]
    fused = bool(r.integers(0, 2))
    return d, n_ctx, n_kv, n_heads, n_sess, sids, pos, fused


@pytest.mark.parametrize("seed", SEEDS)
def test_decode_random_batch(gpu, seed):
    d, n_ctx, n_kv, n_heads, n_sess, sids, pos, fused = _case(seed)
    m = Mirror(gpu, 1, n_sess, n_kv, d, n_ctx)
    n_batch = len(sids)
    for b, (s, p) in enumerate(zip(sids, pos)):
        if s < n_sess:
            # decode reads the window ending at p; a fused call writes p itself
            m.fill_range(0, s, 0, p if fused else p + 1, seed=700 + 31 * seed + b)
    q = oracle.normal(800 + seed, n_batch * n_heads * d).reshape(n_batch, n_heads, d)
    k = oracle.normal(900 + seed, n_batch * n_kv * d).reshape(n_batch, n_kv, d)
    v = oracle.normal(1000 + seed, n_batch * n_kv * d).reshape(n_batch, n_kv, d)
    out = gpu.full((n_batch, n_heads, d), 7.0, dtype=gpu.float32, device="cuda")
    if fused:
        m.ring.append_decode(0, _i32(gpu, pos), m.dev(q), m.dev(k), m.dev(v), out, n_heads,
                             session_ids=_i32(gpu, sids), stream=m.stream)
    else:
        m.ring.decode(0, _i32(gpu, pos), m.dev(q), out, n_heads, session_ids=_i32(gpu, sids),
                      stream=m.stream)
    gpu.cuda.synchronize()
    got = out.cpu().numpy()
    for b, (s, p) in enumerate(zip(sids, pos)):
        what = f"seed {seed} entry {b} session {s} pos {p} d {d} n_ctx {n_ctx} " \
               f"heads {n_heads}/{n_kv} fused {fused}"
        if s >= n_sess:
            assert np.all(got[b] == 0.0), what + ": skipped entry must be zeroed"
            continue
        if fused:
            m.oracle_append(0, s, p, k[b], v[b])
        check_close(got[b], m.oracle_decode(0, s, p, q[b], n_heads), what)
        m.assert_ring_equal(0, s)
