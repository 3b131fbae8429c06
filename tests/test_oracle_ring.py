"""Pins the oracle's ring geometry and attention (src/bmo_cuda_kernels.cu:739-847,
src/bmo_compute.cpp:927-970) with closed forms, brute-force enumeration,
invariants and an identity between prefill and decode."""
import numpy as np
import pytest

import oracle


def test_window_closed_forms():
    # W=512, write head at absolute position 700
    assert oracle.ring_window(700, 512) == (512, 189, 188)
    assert oracle.ring_window(0, 512) == (1, 0, 0)
    assert oracle.ring_window(510, 512) == (511, 0, 510)
    assert oracle.ring_window(511, 512) == (512, 0, 511)
    assert oracle.ring_window(512, 512) == (512, 1, 0)
    assert oracle.ring_window(3, 8) == (4, 0, 3)  # depformer step 3


@pytest.mark.parametrize("n_ctx", [1, 3, 4, 8])
def test_window_brute_force(n_ctx):
    """Enumerate which slots hold the window; they are always {0..window-1}
    (the property the GPU kernel relies on to walk slots in order)."""
    for p in range(0, 5 * n_ctx):
        hist = {}
        for t in range(p + 1):          # write positions 0..p into the ring
            hist[t % n_ctx] = t
        newest = sorted(hist.values())[-min(p + 1, n_ctx):]
        w, start, cur = oracle.ring_window(p, n_ctx)
        assert newest == list(range(start, p + 1))
        assert w == len(newest) and cur == p % n_ctx
        assert sorted(t % n_ctx for t in newest) == list(range(w))


def _fill(kc, vc, positions, seed, n_kv, d):
    rows = {}
    for t in positions:
        k = oracle.normal(seed, n_kv * d, offset=2 * t * n_kv * d)
        v = oracle.normal(seed, n_kv * d, offset=(2 * t + 1) * n_kv * d)
        oracle.ring_append(kc, vc, t, k, v)
        rows[t] = (k, v)
    return rows


def _deq_rows(c, slots):
    return oracle.dequantize_q4_0(c[:, slots, :]).reshape(c.shape[0], len(slots), -1)


def _np_decode(kc, vc, pos, q, n_heads, scale):
    n_kv, n_ctx, nblk = kc.shape
    d = nblk * 32
    w, start, _ = oracle.ring_window(pos, n_ctx)
    slots = [(start + i) % n_ctx for i in range(w)]
    K = _deq_rows(kc, slots).astype(np.float64)
    V = _deq_rows(vc, slots).astype(np.float64)
    qf = q.reshape(n_heads, d).astype(np.float64)
    out = np.zeros((n_heads, d))
    for h in range(n_heads):
        kv = h // (n_heads // n_kv)
        s = K[kv] @ qf[h] * scale
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ V[kv]
    return out


@pytest.mark.parametrize("pos", [0, 1, 7, 63, 64, 100, 191])
def test_decode_vs_numpy(pos):
    n_kv, n_heads, d, n_ctx = 2, 4, 64, 64
    kc, vc = oracle.new_ring(n_kv, n_ctx, d)
    _fill(kc, vc, range(max(0, pos - 2 * n_ctx), pos + 1), 0xB0A00001, n_kv, d)
    q = oracle.normal(7, n_heads * d)
    ref = _np_decode(kc, vc, pos, q, n_heads, 1 / np.sqrt(np.float32(d), dtype=np.float32))
    got = oracle.ring_decode_f64(kc, vc, pos, q, n_heads)
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-13)


def test_window_one_returns_cached_v():
    n_kv, d, n_ctx = 3, 128, 16
    kc, vc = oracle.new_ring(n_kv, n_ctx, d)
    rows = _fill(kc, vc, [0], 5, n_kv, d)
    q = oracle.normal(9, n_kv * d)
    got = oracle.ring_decode_f64(kc, vc, 0, q, n_kv)
    vhat = oracle.dequantize_q4_0(oracle.quantize_q4_0(rows[0][1])).reshape(n_kv, d)
    assert np.array_equal(got, vhat.astype(np.float64))


def test_equal_keys_and_zero_query_give_mean_v():
    n_kv, d, n_ctx, pos = 1, 64, 32, 45
    kc, vc = oracle.new_ring(n_kv, n_ctx, d)
    _fill(kc, vc, range(pos + 1), 21, n_kv, d)
    vmean = _deq_rows(vc, list(range(n_ctx))).astype(np.float64).mean(axis=1)
    # q = 0: every score is 0
    got = oracle.ring_decode_f64(kc, vc, pos, np.zeros(d, np.float32), 1)
    np.testing.assert_allclose(got, vmean, rtol=0, atol=1e-12)
    # all keys equal: same scores whatever q
    kc[:] = kc[:, :1, :]
    got = oracle.ring_decode_f64(kc, vc, pos, oracle.normal(3, d), 1)
    np.testing.assert_allclose(got, vmean, rtol=0, atol=1e-12)


def test_dominant_key():
    n_kv, d, n_ctx, pos = 1, 128, 64, 200
    kc, vc = oracle.new_ring(n_kv, n_ctx, d)
    _fill(kc, vc, range(pos - n_ctx + 1, pos + 1), 31, n_kv, d)
    slot = 17
    khat = _deq_rows(kc, [slot])[0, 0]
    q = (khat * 400.0).astype(np.float32)  # score gap of thousands
    got = oracle.ring_decode_f64(kc, vc, pos, q, 1)
    np.testing.assert_allclose(got[0], _deq_rows(vc, [slot])[0, 0], rtol=0, atol=1e-9)


def test_slot_permutation_invariance():
    n_kv, d, n_ctx, pos = 2, 64, 32, 90
    kc, vc = oracle.new_ring(n_kv, n_ctx, d)
    _fill(kc, vc, range(pos - n_ctx + 1, pos + 1), 41, n_kv, d)
    q = oracle.normal(4, 2 * d)
    a = oracle.ring_decode_f64(kc, vc, pos, q, 2)
    perm = np.random.default_rng(0).permutation(n_ctx)
    b = oracle.ring_decode_f64(np.ascontiguousarray(kc[:, perm]), np.ascontiguousarray(vc[:, perm]),
                               pos, q, 2)
    np.testing.assert_allclose(a, b, rtol=1e-12, atol=1e-14)


def test_gqa_maps_query_heads_to_kv_heads():
    n_kv, n_heads, d, n_ctx, pos = 2, 8, 64, 16, 20
    kc, vc = oracle.new_ring(n_kv, n_ctx, d)
    _fill(kc, vc, range(pos + 1), 51, n_kv, d)
    q = oracle.normal(6, n_heads * d).reshape(n_heads, d)
    got = oracle.ring_decode_f64(kc, vc, pos, q, n_heads)
    for h in range(n_heads):
        kv = h // 4
        one = oracle.ring_decode_f64(np.ascontiguousarray(kc[kv:kv + 1]),
                                     np.ascontiguousarray(vc[kv:kv + 1]), pos, q[h], 1)
        np.testing.assert_allclose(got[h], one[0], rtol=1e-13, atol=1e-15)


def test_planted_window_slip_is_caught():
    """An oracle that dropped the oldest key (start+1) must disagree."""
    n_kv, d, n_ctx, pos = 1, 64, 16, 40
    kc, vc = oracle.new_ring(n_kv, n_ctx, d)
    _fill(kc, vc, range(pos - n_ctx + 1, pos + 1), 61, n_kv, d)
    q = oracle.normal(8, d)
    good = oracle.ring_decode_f64(kc, vc, pos, q, 1)
    w, start, _ = oracle.ring_window(pos, n_ctx)
    slots = [(start + 1 + i) % n_ctx for i in range(w - 1)]
    K = _deq_rows(kc, slots)[0].astype(np.float64)
    V = _deq_rows(vc, slots)[0].astype(np.float64)
    s = K @ q.astype(np.float64) / np.sqrt(d)
    p = np.exp(s - s.max())
    slipped = (p / p.sum()) @ V
    assert np.max(np.abs(slipped - good[0])) > 1e-4


@pytest.mark.parametrize("pos0,n_tok", [(0, 5), (3, 8), (20, 16), (29, 16)])
def test_prefill_equals_successive_decodes(pos0, n_tok):
    n_kv, n_heads, d, n_ctx = 2, 4, 64, 16
    kc, vc = oracle.new_ring(n_kv, n_ctx, d)
    _fill(kc, vc, range(max(0, pos0 - n_ctx), pos0), 71, n_kv, d)
    kc2, vc2 = kc.copy(), vc.copy()
    q = oracle.round_bf16(oracle.normal(1, n_tok * n_heads * d)).reshape(n_tok, n_heads, d)
    k = oracle.round_bf16(oracle.normal(2, n_tok * n_kv * d)).reshape(n_tok, n_kv, d)
    v = oracle.round_bf16(oracle.normal(3, n_tok * n_kv * d)).reshape(n_tok, n_kv, d)
    got = oracle.ring_prefill_f64(kc, vc, pos0, q, k, v, n_heads)
    for i in range(n_tok):
        oracle.ring_append(kc2, vc2, pos0 + i, k[i], v[i])
        ref = oracle.ring_decode_f64(kc2, vc2, pos0 + i, q[i], n_heads)
        np.testing.assert_allclose(got[i], ref, rtol=1e-12, atol=1e-14)
    assert np.array_equal(kc, kc2) and np.array_equal(vc, vc2)


def test_copy_k_layout():
    n_kv, d, n_ctx = 3, 128, 8
    kc, vc = oracle.new_ring(n_kv, n_ctx, d)
    _fill(kc, vc, range(11), 81, n_kv, d)
    out = oracle.ring_copy_k_f32(kc, 2, 5)
    for ti in range(5):
        for h in range(n_kv):
            np.testing.assert_array_equal(out[ti, h], oracle.dequantize_q4_0(kc[h, 2 + ti]))


def test_cpu_baseline_matches_oracle():
    n_kv, d, n_ctx, pos = 4, 128, 64, 150
    kc, vc = oracle.new_ring(n_kv, n_ctx, d)
    _fill(kc, vc, range(pos - n_ctx + 1, pos + 1), 91, n_kv, d)
    q = oracle.normal(10, n_kv * d)
    ref = oracle.ring_decode_f64(kc, vc, pos, q, n_kv)
    got = oracle.cpu_decode_f32(kc, vc, pos, q, n_kv)
    assert np.all(np.abs(got - ref) <= 2e-3 + 1e-3 * np.abs(ref))
    secs, out = oracle.cpu_baseline_run(kc[None], vc[None], np.array([pos]), q[None], n_kv, 2, 1)
    assert secs > 0
    np.testing.assert_array_equal(out[0], got)
