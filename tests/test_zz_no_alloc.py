"""The allocation-free prefill entry point (bmo_kv_ring_prefill_noalloc)
against bmo_kv_ring_prefill, both called through the C ABI with ctypes.

Two rings are filled alike and receive the same calls, one through each entry
point: a staged chunk (4 query heads per kv head), then a smaller staged
chunk, then a direct one (one query head per kv head).  Outputs must be
identical (the same kernels run on the same inputs, only the staging memory
differs), the rings byte-identical, and one entry per call is also checked
against the float64 oracle at |gpu - ref| <= 2e-3 + 1e-3 |ref|.  A staged
chunk larger than the fixed scratch is rejected without launching."""
import numpy as np
import pytest

import oracle
from _ringsim import Mirror, check_close
from bmo_jetson_amd import KVRing, lib

pytestmark = pytest.mark.gpu

N_KV, D, N_CTX = 2, 128, 128


def _bf16(seed, shape):
    return oracle.round_bf16(oracle.normal(seed, int(np.prod(shape)))).reshape(shape)


def _call(gpu, fn, ring, pos0, n_tok, n_heads, q, k, v, out):
    pos_dev = gpu.tensor(pos0, dtype=gpu.int32, device="cuda")
    gpu.cuda.synchronize()
    rc = getattr(lib(), fn)(ring.handle, 0, len(pos0), None, pos_dev.data_ptr(), n_tok, n_heads,
                            q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), 0.0,
                            gpu.cuda.current_stream().cuda_stream)
    gpu.cuda.synchronize()
    return rc


def _mirrors(gpu, pos0):
    ms = [Mirror(gpu, 1, 3, N_KV, D, N_CTX) for _ in range(2)]
    for m in ms:
        for s, p in enumerate(pos0):
            m.fill_range(0, s, 0, p, seed=4000 + s)
    return ms


def _step(gpu, ms, pos0, n_tok, n_heads, seed):
    q = _bf16(seed, (len(pos0), n_tok, n_heads, D))
    k = _bf16(seed + 1, (len(pos0), n_tok, N_KV, D))
    v = _bf16(seed + 2, (len(pos0), n_tok, N_KV, D))
    outs = []
    for m, fn in zip(ms, ("bmo_kv_ring_prefill", "bmo_kv_ring_prefill_noalloc")):
        out = gpu.full((len(pos0), n_tok, n_heads, D), float("nan"), dtype=gpu.float32, device="cuda")
        rc = _call(gpu, fn, m.ring, pos0, n_tok, n_heads, m.dev(q, gpu.bfloat16),
                   m.dev(k, gpu.bfloat16), m.dev(v, gpu.bfloat16), out)
        assert rc == 0, (fn, rc, m.ring.last_error())
        outs.append(out.cpu().numpy())
    assert np.array_equal(outs[0], outs[1]), f"outputs differ (n_tok {n_tok}, n_heads {n_heads})"
    # the oracle on entry 0, and both rings after the commit
    kc, vc = ms[0].orc[(0, 0)]
    ref = oracle.ring_prefill_f64(kc, vc, pos0[0], q[0], k[0], v[0], n_heads)
    check_close(outs[1][0], ref, f"noalloc prefill n_tok {n_tok} n_heads {n_heads}")
    for b, p in enumerate(pos0):
        for m in ms:
            for i in range(n_tok):
                m.oracle_append(0, b, p + i, k[b, i], v[b, i])
    for s in range(3):
        for m in ms:
            m.assert_ring_equal(0, s)


def test_noalloc_matches_prefill_twice_then_smaller(gpu):
    pos0 = [200, 150, 300]
    ms = _mirrors(gpu, pos0)
    _step(gpu, ms, pos0, 100, 8, seed=11)                  # staged, 3 entries
    pos1 = [300, 250]
    _step(gpu, ms, pos1, 40, 8, seed=21)                   # staged, smaller
    pos2 = [340, 290, 400]
    _step(gpu, ms, pos2, 64, N_KV, seed=31)                # direct path
    for m in ms:
        m.ring.close()


def test_noalloc_rejects_oversized_staging(gpu):
    # 2 entries x 64 kv heads x 256 groups x 2304 B = 75.5 MB of staging > 32 MiB
    ring = KVRing(1, 2, 64, 128, 4096)
    x = gpu.zeros(16, dtype=gpu.float32, device="cuda")
    pos_dev = gpu.tensor([0, 0], dtype=gpu.int32, device="cuda")
    gpu.cuda.synchronize()
    rc = lib().bmo_kv_ring_prefill_noalloc(ring.handle, 0, 2, None, pos_dev.data_ptr(), 4096, 128,
                                           x.data_ptr(), x.data_ptr(), x.data_ptr(), x.data_ptr(),
                                           0.0, None)
    assert rc == 2
    assert "scratch" in ring.last_error()
    gpu.cuda.synchronize()
    assert not ring.export_q4_0(0, 1, 0, 0, 64).any()  # nothing launched
    ring.close()
